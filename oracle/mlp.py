"""Grouped expert MLP and combine oracle (test infrastructure only).

Restates the reference's per-wave arithmetic with f32 accumulation and the
bf16 rounding points of its device ops:
  GMM1   h = x . W13_s^T           f32 accumulate, bf16 out
  swiglu act = silu(h[:I]) * h[I:]  f32 math, bf16 out
  GMM2   y = act . W2_s^T           f32 accumulate, bf16 out
  unpermute / single combine: out[t] = sum_j w[t,j] * y[t*k+j]   f32, bf16 out
(patches/patch_fused_moe.py:3772-3774 GMM1+swiglu+GMM2, :3342-3379 one
combine with the original top-k weights; phase_split.py:1649-1656 gives the
unpermute index semantics).  A resident shared expert (the DeepSeek-style
layer) is added to the routed output before the final rounding.

Pinning (tests/test_oracle_core.py): expert_mlp against a float64
brute-force triple loop on tiny H/I; the reference combine golden vectors
(tests/test_phase_split_b2.py:863-1016 weighted gathers and
scatter-adds); wave-split invariance (outputs of any split of the pairs into
waves followed by one combine equal the unsplit layer bit for bit,
docs/evidence/issue-13-multi-wave-prefill.md:53-56).
"""

from __future__ import annotations

import numpy as np

from .bf16 import bf16_to_f32, f32_to_bf16, round_bf16


def silu(g: np.ndarray) -> np.ndarray:
    g = np.asarray(g, dtype=np.float32)
    with np.errstate(over="ignore"):
        return (g / (np.float32(1.0) + np.exp(-g))).astype(np.float32)


def expert_mlp(x_rows: np.ndarray, w13: np.ndarray, w2: np.ndarray) -> np.ndarray:
    """One expert over its rows.  x_rows f32 [n, H] (bf16 values), w13 f32
    [2I, H], w2 f32 [H, I].  Returns y as f32 holding bf16 values [n, H]."""
    I = w13.shape[0] // 2
    h = round_bf16((x_rows @ w13.T).astype(np.float32))
    act = round_bf16((silu(h[:, :I]) * h[:, I:]).astype(np.float32))
    return round_bf16((act @ w2.T).astype(np.float32))


def grouped_mlp(
    x_bf16: np.ndarray,
    slot_of_pair: np.ndarray,
    top_k: int,
    w13_slots_bf16: np.ndarray,
    w2_slots_bf16: np.ndarray,
) -> np.ndarray:
    """y[p] for every flat pair p with slot_of_pair[p] >= 0 (others zero).

    Weights are passed as bf16 bits [P, 2I, H] / [P, H, I] (only slots
    referenced are converted).
    """
    x = bf16_to_f32(x_bf16)
    slot_of_pair = np.asarray(slot_of_pair).reshape(-1)  # flat pair order
    N = slot_of_pair.size
    H = x.shape[1]
    y = np.zeros((N, H), dtype=np.float32)
    for s in np.unique(slot_of_pair[slot_of_pair >= 0]):
        pairs = np.nonzero(slot_of_pair == s)[0]
        rows = x[pairs // top_k]
        y[pairs] = expert_mlp(rows, bf16_to_f32(w13_slots_bf16[s]), bf16_to_f32(w2_slots_bf16[s]))
    return y


def combine(y: np.ndarray, w_bf16: np.ndarray, *, mask: np.ndarray | None = None,
            add: np.ndarray | None = None, round_output: bool = True) -> np.ndarray:
    """out[t] = add[t] + sum_j w[t,j] * y[t*k+j] in f32 (j order).

    round_output=True returns the bf16-rounded layer output (as f32);
    False returns the f32-accumulated value before the final cast, the
    quantity the bf16 output tolerance is measured against."""
    w = bf16_to_f32(w_bf16)
    T, k = w.shape
    H = y.shape[1]
    acc = np.zeros((T, H), dtype=np.float32)
    for j in range(k):
        rows = y[np.arange(T) * k + j]
        term = (w[:, j:j + 1] * rows).astype(np.float32)
        if mask is not None:
            term = np.where((mask.reshape(T, k)[:, j] >= 0)[:, None], term, np.float32(0.0))
        acc = (acc + term).astype(np.float32)
    if add is not None:
        acc = (acc + np.asarray(add, dtype=np.float32)).astype(np.float32)
    return round_bf16(acc) if round_output else acc


def moe_layer(
    x_bf16: np.ndarray,
    ids: np.ndarray,
    w_bf16: np.ndarray,
    log2phy: np.ndarray | None,
    w13_slots_bf16: np.ndarray,
    w2_slots_bf16: np.ndarray,
    *,
    shared: tuple[np.ndarray, np.ndarray] | None = None,
    round_output: bool = False,
) -> np.ndarray:
    """Full routed layer through the slot bank, [T, H] f32: the f32-accumulated
    result before the final bf16 cast (round_output=False) or after it.

    shared = (w13 [2I_s, H], w2 [H, I_s]) bf16 bits of a resident shared
    expert applied to every token and added before the final rounding.
    """
    from .permute import remap

    T, k = ids.shape
    P = w13_slots_bf16.shape[0]
    slot = remap(ids, log2phy, P)
    if np.any(slot < 0):
        raise RuntimeError("topk_ids contain experts without ready slots")
    y = grouped_mlp(x_bf16, slot, k, w13_slots_bf16, w2_slots_bf16)
    add = None
    if shared is not None:
        add = expert_mlp(bf16_to_f32(x_bf16), bf16_to_f32(shared[0]), bf16_to_f32(shared[1]))
    return combine(y, w_bf16, add=add, round_output=round_output)


def to_bf16_bits(a: np.ndarray) -> np.ndarray:
    return f32_to_bf16(np.asarray(a, dtype=np.float32))
