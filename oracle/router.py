"""Router oracle (test infrastructure only).

Restates expert selection as the hot path defines it:
  * gate: logits = x . Wg^T, exact (float64) accumulation rounded to f32
    then bf16 — the gate matmul of ops/fused_moe/moe_router_op.py:228-231;
  * logit bias (the gate's linear bias): added to the logits before scoring;
  * softmax top-k: f32 softmax over E, k best probabilities (plus the
    correction bias, for the selection only), ties to the
    lower expert id, renorm w / max(sum w, eps) (patch_fused_moe.py:597-632),
    times routed_scaling_factor, cast to bf16 (moe_router_op.py:128-162
    fixes the bf16 weight / int32 id ABI);
  * grouped sigmoid: s = sigmoid(l); selection score s + bias; group score =
    sum of the two best selection scores of each contiguous group; keep the
    topk_group best groups (ties to the lower group id); k best selection
    scores inside them; weights s renormalised, then scaled.

The f32 arithmetic is written out operation by operation in the same order
as the gfx950 kernel (csrc/router.hip): exp by Cody-Waite reduction and a
degree-7 Taylor polynomial, sum of exponentials as a per-lane sum over
j = 0..7 of experts j*64 + lane followed by a butterfly over lane distances
32, 16, 8, 4, 2, 1, so selection and weights can be compared bit for bit.

Pinning (tests/test_oracle_core.py): exp_nonpos against float64 np.exp
(<= 2 ulp); softmax against a float64 softmax; selection against brute-force
Python loops on tiny E with planted ties; renorm against the reference
golden vector weights [1, 3] -> [0.25, 0.75] (tests/test_patch_fused_moe.py:560);
grouped selection against a brute-force enumeration; gate against an exact
integer-scaled product.
"""

from __future__ import annotations

import numpy as np

from .bf16 import bf16_to_f32, f32_to_bf16

F32 = np.float32
_LOG2E = np.uint32(0x3FB8AA3B).view(np.float32)
_LN2_HI = np.uint32(0x3F318000).view(np.float32)
_LN2_LO = np.uint32(0xB95E8083).view(np.float32)
_C = [np.uint32(b).view(np.float32) for b in (0x39500D01, 0x3AB60B61, 0x3C088889, 0x3D2AAAAB, 0x3E2AAAAB)]
_HALF = F32(0.5)
_ONE = F32(1.0)
_EPS = np.finfo(np.float32).eps
_LANES = 64
_EPL = 8


def exp_nonpos(x: np.ndarray) -> np.ndarray:
    """exp(x) for x <= 0 in float32, rounding-for-rounding the device routine."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        n = np.rint(x * _LOG2E).astype(np.float32)
        r = (x - n * _LN2_HI).astype(np.float32)
        r = (r - n * _LN2_LO).astype(np.float32)
        p = _C[0]
        for c in _C[1:]:
            p = (p * r + c).astype(np.float32)
        p = (p * r + _HALF).astype(np.float32)
        p = (p * r + _ONE).astype(np.float32)
        p = (p * r + _ONE).astype(np.float32)
        out = np.ldexp(p, np.where(np.isfinite(n), n, 0).astype(np.int32)).astype(np.float32)
    return np.where(x >= F32(-86.0), out, F32(0.0)).astype(np.float32)


def sigmoid(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    pos = x >= 0
    e = exp_nonpos(np.where(pos, -x, x))
    with np.errstate(invalid="ignore", divide="ignore"):
        a = (_ONE / (_ONE + e)).astype(np.float32)
        b = (e / (_ONE + e)).astype(np.float32)
    return np.where(pos, a, b).astype(np.float32)


def _lane_layout(v: np.ndarray, fill) -> np.ndarray:
    """[T, E] -> [T, 8, 64] with expert j*64 + lane at [:, j, lane]."""
    T, E = v.shape
    if E > _EPL * _LANES:
        raise ValueError("E > 512 is not supported")
    pad = np.full((T, _EPL * _LANES), fill, dtype=np.float32)
    pad[:, :E] = v
    return pad.reshape(T, _EPL, _LANES)


def _butterfly_sum(v: np.ndarray) -> np.ndarray:
    """Butterfly sum over the last axis (64 lanes); returns lane 0's value."""
    lanes = np.arange(_LANES)
    for o in (32, 16, 8, 4, 2, 1):
        v = (v + v[..., lanes ^ o]).astype(np.float32)
    return v[..., 0]


def softmax_probs(logits: np.ndarray) -> np.ndarray:
    """f32 softmax over the last axis with the kernel's reduction order."""
    lg = np.asarray(logits, dtype=np.float32)
    T, E = lg.shape
    m = lg.max(axis=1, keepdims=True).astype(np.float32)
    ex = exp_nonpos((lg - m).astype(np.float32))
    lay = _lane_layout(ex, 0.0)
    local = lay[:, 0, :].copy()
    for j in range(1, _EPL):
        local = (local + lay[:, j, :]).astype(np.float32)
    s = _butterfly_sum(local)
    return (ex / s[:, None]).astype(np.float32)


def _order(score: np.ndarray, eligible: np.ndarray) -> np.ndarray:
    """Indices sorted by (score desc, index asc) among eligible entries."""
    idx = np.nonzero(eligible)[0]
    key = score[idx]
    o = np.lexsort((idx, -key.astype(np.float64)))
    return idx[o]


def _finish(sel_w: np.ndarray, renorm: bool, scale: float) -> tuple[np.ndarray, np.ndarray]:
    """Renormalise in selection order, scale, round: returns (w_f32, w_bf16 bits)."""
    w = sel_w.astype(np.float32)
    if renorm:
        s = w[:, 0].copy()
        for j in range(1, w.shape[1]):
            s = (s + w[:, j]).astype(np.float32)
        d = np.maximum(s, F32(_EPS)).astype(np.float32)
        w = (w / d[:, None]).astype(np.float32)
    w = (w * F32(scale)).astype(np.float32)
    return w, f32_to_bf16(w)


def _with_logit_bias(logits: np.ndarray, logit_bias: np.ndarray | None) -> np.ndarray:
    """logits + logit_bias in f32 (the router gate's linear bias, one rounding)."""
    lg = np.asarray(logits, dtype=np.float32)
    if logit_bias is None:
        return lg
    return (lg + np.asarray(logit_bias, dtype=np.float32)[None, :]).astype(np.float32)


def softmax_topk(
    logits: np.ndarray,
    k: int,
    *,
    renorm: bool = True,
    scale: float = 1.0,
    bias: np.ndarray | None = None,
    logit_bias: np.ndarray | None = None,
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Returns (ids int32 [T,k], w_f32 [T,k], w_bf16 bits [T,k]).

    logit_bias is added to the logits (one f32 rounding) before the softmax;
    bias (e_score_correction_bias) is added to the probabilities for the
    selection only, the weights stay the unbiased probabilities."""
    p = softmax_probs(_with_logit_bias(logits, logit_bias))
    T, E = p.shape
    ps = (p + np.asarray(bias, dtype=np.float32)[None, :]).astype(np.float32) if bias is not None else p
    ids = np.empty((T, k), dtype=np.int32)
    sel = np.empty((T, k), dtype=np.float32)
    for t in range(T):
        o = _order(ps[t], np.ones(E, dtype=bool))[:k]
        ids[t] = o
        sel[t] = p[t, o]
    w, wb = _finish(sel, renorm, scale)
    return ids, w, wb


def grouped_sigmoid_topk(
    logits: np.ndarray,
    k: int,
    *,
    bias: np.ndarray | None,
    n_group: int,
    topk_group: int,
    renorm: bool = True,
    scale: float = 1.0,
    logit_bias: np.ndarray | None = None,
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """DeepSeek-V3-style selection.  Returns (ids, w_f32, w_bf16 bits)."""
    lg = _with_logit_bias(logits, logit_bias)
    T, E = lg.shape
    sg = sigmoid(lg)
    sb = (sg + np.asarray(bias, dtype=np.float32)[None, :]).astype(np.float32) if bias is not None else sg
    ids = np.empty((T, k), dtype=np.int32)
    sel = np.empty((T, k), dtype=np.float32)
    gs = E // n_group if n_group > 1 else E
    for t in range(T):
        if n_group > 1:
            g = sb[t].reshape(n_group, gs)
            top2 = -np.sort(-g, axis=1)[:, :2]
            gscore = (top2[:, 0] + top2[:, 1]).astype(np.float32)
            kept = _order(gscore, np.ones(n_group, dtype=bool))[:topk_group]
            elig = np.zeros(E, dtype=bool)
            for gi in kept:
                elig[gi * gs:(gi + 1) * gs] = True
        else:
            elig = np.ones(E, dtype=bool)
        o = _order(sb[t], elig)[:k]
        ids[t] = o
        sel[t] = sg[t, o]
    w, wb = _finish(sel, renorm, scale)
    return ids, w, wb


def gate_logits(x_bf16: np.ndarray, wg_bf16: np.ndarray, *, out_f32: bool = False) -> np.ndarray:
    """Exact gate product rounded to f32 (then bf16 unless out_f32); float32 out."""
    x = bf16_to_f32(x_bf16).astype(np.float64)
    w = bf16_to_f32(wg_bf16).astype(np.float64)
    l32 = (x @ w.T).astype(np.float32)
    return l32 if out_f32 else bf16_to_f32(f32_to_bf16(l32))
