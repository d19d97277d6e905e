"""GPU parity of the router kernels against the oracle.

Selection (ids) and weights (bf16 and f32) are bit-exact against
oracle.router on the same logits tensor; the gate GEMV/GEMM is within one
bf16 ulp of the exact product (its f32 accumulation order differs).
"""

import numpy as np
import pytest
import torch

from oracle import router as orc
from oracle.bf16 import bf16_to_f32, f32_to_bf16, normal_bf16
from tests._util import bf16_ulp, from_dev_bf16, to_dev_bf16, ulp_mismatch_stats

pytestmark = pytest.mark.gpu


def _native():
    from vllm_moe_offload_amd import native

    return native


def _tied_logits(rng, T, E, step=0.25):
    """bf16 logits on a coarse grid so equal values (ties) are common."""
    v = np.round(rng.standard_normal((T, E)) / step) * step
    return f32_to_bf16(v.astype(np.float32))


@pytest.mark.parametrize("T,E,k,dtype", [
    (1, 128, 8, "bf16"),
    (16, 128, 8, "bf16"),
    (257, 128, 8, "bf16"),
    (64, 60, 4, "bf16"),
    (33, 256, 8, "f32"),
    (8, 512, 16, "bf16"),
    (5, 8, 2, "f32"),
])
def test_softmax_topk_bit_exact(T, E, k, dtype):
    native = _native()
    print(f"case softmax T={T} E={E} k={k} {dtype}", flush=True)
    rng = np.random.default_rng(1000 + T * 7 + E)
    bits = _tied_logits(rng, T, E)
    lg32 = bf16_to_f32(bits)
    if dtype == "bf16":
        dev = to_dev_bf16(bits)
    else:
        lg32 = (lg32 + rng.standard_normal(lg32.shape).astype(np.float32) * 1e-3).astype(np.float32)
        dev = torch.from_numpy(lg32).cuda()
    w_f32 = torch.empty((T, k), dtype=torch.float32, device="cuda")
    w, ids, _ = native.router_topk(dev, k, w_f32=w_f32)
    torch.cuda.synchronize()
    r_ids, r_w, r_wb = orc.softmax_topk(lg32, k)
    np.testing.assert_array_equal(ids.cpu().numpy(), r_ids)
    np.testing.assert_array_equal(from_dev_bf16(w), r_wb)
    np.testing.assert_array_equal(w_f32.cpu().numpy().view(np.uint32), r_w.view(np.uint32))


def test_softmax_with_logit_bias_bit_exact():
    native = _native()
    rng = np.random.default_rng(21)
    T, E, k = 64, 128, 8
    bits = _tied_logits(rng, T, E)
    bias = (rng.standard_normal(E) * 0.7).astype(np.float32)
    w_f32 = torch.empty((T, k), dtype=torch.float32, device="cuda")
    w, ids, _ = native.router_topk(to_dev_bf16(bits), k, logit_bias=torch.from_numpy(bias).cuda(), w_f32=w_f32)
    torch.cuda.synchronize()
    r_ids, r_w, r_wb = orc.softmax_topk(bf16_to_f32(bits), k, logit_bias=bias)
    np.testing.assert_array_equal(ids.cpu().numpy(), r_ids)
    np.testing.assert_array_equal(from_dev_bf16(w), r_wb)
    np.testing.assert_array_equal(w_f32.cpu().numpy().view(np.uint32), r_w.view(np.uint32))


@pytest.mark.parametrize("E", [64, 128, 256])
def test_softmax_with_correction_bias_selects_only(E):
    """e_score_correction_bias with softmax scoring: selection by p + bias,
    weights the unbiased probabilities (renormalised), bit for bit."""
    native = _native()
    print(f"case softmax correction bias E={E}", flush=True)
    rng = np.random.default_rng(22 + E)
    T, k = 48, 8
    bits = _tied_logits(rng, T, E)
    cb = (rng.standard_normal(E) * 0.01).astype(np.float32)
    lb = (rng.standard_normal(E) * 0.5).astype(np.float32)
    for logit_bias in (None, lb):
        w_f32 = torch.empty((T, k), dtype=torch.float32, device="cuda")
        w, ids, _ = native.router_topk(
            to_dev_bf16(bits), k, bias=torch.from_numpy(cb).cuda(),
            logit_bias=None if logit_bias is None else torch.from_numpy(logit_bias).cuda(), w_f32=w_f32)
        torch.cuda.synchronize()
        r_ids, r_w, r_wb = orc.softmax_topk(bf16_to_f32(bits), k, bias=cb, logit_bias=logit_bias)
        np.testing.assert_array_equal(ids.cpu().numpy(), r_ids)
        np.testing.assert_array_equal(from_dev_bf16(w), r_wb)
        np.testing.assert_array_equal(w_f32.cpu().numpy().view(np.uint32), r_w.view(np.uint32))
    # the bias changed the choice somewhere (else the test pins nothing)
    plain, _, _ = orc.softmax_topk(bf16_to_f32(bits), k)
    assert not np.array_equal(plain, orc.softmax_topk(bf16_to_f32(bits), k, bias=cb)[0])


def test_softmax_ties_break_to_lower_id():
    native = _native()
    T, E, k = 4, 128, 8
    lg = np.zeros((T, E), dtype=np.float32)
    lg[1, [100, 3, 77, 5]] = 1.0          # 4 tied winners, then 124 tied zeros
    lg[2, ::2] = 0.5                      # every even expert tied
    lg[3] = -np.arange(E, dtype=np.float32) * 0  # all equal
    dev = to_dev_bf16(f32_to_bf16(lg))
    _, ids, _ = native.router_topk(dev, k)
    got = ids.cpu().numpy()
    np.testing.assert_array_equal(got[0], np.arange(8))
    np.testing.assert_array_equal(got[1], [3, 5, 77, 100, 0, 1, 2, 4])
    np.testing.assert_array_equal(got[2], [0, 2, 4, 6, 8, 10, 12, 14])
    np.testing.assert_array_equal(got[3], np.arange(8))


@pytest.mark.parametrize("T,E,G,TG,k,scale", [
    (1, 256, 8, 4, 8, 2.5),
    (32, 256, 8, 4, 8, 2.5),
    (2048, 256, 8, 4, 8, 2.5),
    (7, 64, 4, 2, 6, 1.0),
    (9, 160, 1, 1, 8, 1.0),
])
def test_grouped_sigmoid_bit_exact(T, E, G, TG, k, scale):
    native = _native()
    print(f"case sigmoid T={T} E={E} G={G}", flush=True)
    rng = np.random.default_rng(77 + T)
    bits = _tied_logits(rng, T, E, step=0.125)
    lg32 = bf16_to_f32(bits)
    bias = (rng.standard_normal(E) * 0.01).astype(np.float32)
    w_f32 = torch.empty((T, k), dtype=torch.float32, device="cuda")
    w, ids, _ = native.router_topk(
        to_dev_bf16(bits), k, scoring="sigmoid", bias=torch.from_numpy(bias).cuda(),
        num_expert_group=G, topk_group=TG, renormalize=True, routed_scaling_factor=scale, w_f32=w_f32,
    )
    torch.cuda.synchronize()
    r_ids, r_w, r_wb = orc.grouped_sigmoid_topk(lg32, k, bias=bias, n_group=G, topk_group=TG, scale=scale)
    np.testing.assert_array_equal(ids.cpu().numpy(), r_ids)
    np.testing.assert_array_equal(from_dev_bf16(w), r_wb)
    np.testing.assert_array_equal(w_f32.cpu().numpy().view(np.uint32), r_w.view(np.uint32))


@pytest.mark.parametrize("T,H,E", [(1, 2048, 128), (7, 2048, 128), (16, 2048, 128), (64, 7168, 256), (300, 2048, 128), (1000, 7168, 256)])
def test_gate_within_one_bf16_ulp(T, H, E):
    native = _native()
    print(f"case gate T={T} H={H} E={E}", flush=True)
    rng = np.random.default_rng(5 + T)
    x = normal_bf16(rng, (T, H), 1.0)
    wg = normal_bf16(rng, (E, H), 0.02)
    logits = torch.empty((T, E), dtype=torch.bfloat16, device="cuda")
    native.router_gate(to_dev_bf16(x), to_dev_bf16(wg), logits)
    torch.cuda.synchronize()
    got = bf16_to_f32(from_dev_bf16(logits))
    ref = orc.gate_logits(x, wg)
    # bound: one bf16 ulp of rounding plus the f32 accumulation error of a
    # K-term sum, |err| <= 4 sqrt(K) 2^-24 sum_h |x_h w_h| (cancellation aware)
    absdot = np.abs(bf16_to_f32(x)).astype(np.float64) @ np.abs(bf16_to_f32(wg)).astype(np.float64).T
    bound = bf16_ulp(ref) + 4.0 * np.sqrt(H) * 2.0 ** -24 * absdot
    assert np.all(np.abs(got - ref) <= bound)
    frac, _ = ulp_mismatch_stats(got, ref)
    assert frac < 1e-3


@pytest.mark.parametrize("T,H,E", [(77, 2048, 200), (333, 1024, 64), (130, 2048, 60), (2048, 7168, 256)])
def test_large_t_gate_f32_bound_and_bf16_is_its_rounding(T, H, E):
    """Past 64 tokens the gate is one dense MFMA GEMM (64 x 128 tiles over a
    4-stage ring when H % 64 == 0 and E % 8 == 0, else 128 x 128 tiles).
    Ragged row and expert tiles included: the f32 logits stay within the
    f32 accumulation bound of the exact product, and the bf16 logits are
    exactly those f32 values rounded to nearest even."""
    native = _native()
    print(f"case large-T gate T={T} H={H} E={E}", flush=True)
    rng = np.random.default_rng(11 + T + E)
    x = normal_bf16(rng, (T, H), 1.0)
    wg = normal_bf16(rng, (E, H), 0.02)
    d_x, d_wg = to_dev_bf16(x), to_dev_bf16(wg)
    lf = torch.empty((T, E), dtype=torch.float32, device="cuda")
    lb = torch.empty((T, E), dtype=torch.bfloat16, device="cuda")
    native.router_gate(d_x, d_wg, lf)
    native.router_gate(d_x, d_wg, lb)
    torch.cuda.synchronize()
    got = lf.cpu().numpy()
    exact = bf16_to_f32(x).astype(np.float64) @ bf16_to_f32(wg).astype(np.float64).T
    absdot = np.abs(bf16_to_f32(x)).astype(np.float64) @ np.abs(bf16_to_f32(wg)).astype(np.float64).T
    assert np.all(np.abs(got - exact) <= 4.0 * np.sqrt(H) * 2.0 ** -24 * absdot + 1e-30)
    np.testing.assert_array_equal(from_dev_bf16(lb), f32_to_bf16(got))


def test_large_t_gate_ring_tiles_equal_register_tiles_bitwise():
    """The two dense kernels of the large-T gate sum every logit's K/16 MFMA
    steps in the same order: 60 experts (E % 8 != 0: 128 x 128
    register-staged tiles) give the same f32 bits as the first 60 of 64
    experts with the same rows (the 64 x 128 ring tiles)."""
    native = _native()
    T, H = 200, 2048
    rng = np.random.default_rng(77)
    x = to_dev_bf16(normal_bf16(rng, (T, H), 1.0))
    wg64 = normal_bf16(rng, (64, H), 0.02)
    a = torch.empty((T, 60), dtype=torch.float32, device="cuda")
    b = torch.empty((T, 64), dtype=torch.float32, device="cuda")
    native.router_gate(x, to_dev_bf16(np.ascontiguousarray(wg64[:60])), a)
    native.router_gate(x, to_dev_bf16(wg64), b)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b[:, :60].contiguous().view(torch.int32))


@pytest.mark.parametrize("T,H", [(7, 2048), (13, 7168)])
def test_gate_grouped_tokens_equal_one_at_a_time(T, H):
    """The GEMV path reduces several tokens at once; each token's f32
    logits must be bit-identical to a call with that token alone."""
    native = _native()
    E = 128
    rng = np.random.default_rng(31 + T)
    x = to_dev_bf16(normal_bf16(rng, (T, H), 1.0))
    wg = to_dev_bf16(normal_bf16(rng, (E, H), 0.02))
    all_t = torch.empty((T, E), dtype=torch.float32, device="cuda")
    native.router_gate(x, wg, all_t)
    for t in range(T):
        one = torch.empty((1, E), dtype=torch.float32, device="cuda")
        native.router_gate(x[t:t + 1].contiguous(), wg, one)
        torch.cuda.synchronize()
        assert torch.equal(one[0].view(torch.int32), all_t[t].view(torch.int32)), t


def test_gate_f32_output():
    native = _native()
    rng = np.random.default_rng(9)
    x = normal_bf16(rng, (4, 2048), 1.0)
    wg = normal_bf16(rng, (128, 2048), 0.02)
    logits = torch.empty((4, 128), dtype=torch.float32, device="cuda")
    native.router_gate(to_dev_bf16(x), to_dev_bf16(wg), logits)
    exact = orc.gate_logits(x, wg, out_f32=True)
    np.testing.assert_allclose(logits.cpu().numpy(), exact, rtol=1e-5, atol=1e-5)
