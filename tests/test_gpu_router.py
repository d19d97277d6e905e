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
    w, ids, _ = native.router_topk(to_dev_bf16(bits), k, bias=torch.from_numpy(bias).cuda(), w_f32=w_f32)
    torch.cuda.synchronize()
    r_ids, r_w, r_wb = orc.softmax_topk(bf16_to_f32(bits), k, bias=bias)
    np.testing.assert_array_equal(ids.cpu().numpy(), r_ids)
    np.testing.assert_array_equal(from_dev_bf16(w), r_wb)
    np.testing.assert_array_equal(w_f32.cpu().numpy().view(np.uint32), r_w.view(np.uint32))


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


@pytest.mark.parametrize("T,H,E", [(1, 2048, 128), (16, 2048, 128), (64, 7168, 256), (300, 2048, 128), (1000, 7168, 256)])
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


def test_gate_f32_output():
    native = _native()
    rng = np.random.default_rng(9)
    x = normal_bf16(rng, (4, 2048), 1.0)
    wg = normal_bf16(rng, (128, 2048), 0.02)
    logits = torch.empty((4, 128), dtype=torch.float32, device="cuda")
    native.router_gate(to_dev_bf16(x), to_dev_bf16(wg), logits)
    exact = orc.gate_logits(x, wg, out_f32=True)
    np.testing.assert_allclose(logits.cpu().numpy(), exact, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("T,H,E,k,scoring,G,TG", [
    (1, 2048, 128, 8, "softmax", 1, 1),
    (4, 2048, 128, 8, "softmax", 1, 1),
    (16, 2048, 128, 8, "softmax", 1, 1),
    (3, 1024, 60, 4, "softmax", 1, 1),
    (1, 7168, 256, 8, "sigmoid", 8, 4),
    (16, 7168, 256, 8, "sigmoid", 8, 4),
    (5, 4096, 512, 16, "softmax", 1, 1),
])
def test_router_decode_equals_gate_plus_topk_and_oracle(T, H, E, k, scoring, G, TG):
    """One-launch decode router: logits bit-identical to lmoe_router_gate,
    selection bit-exact against the oracle on those logits; the counter is
    left at zero so repeated calls agree."""
    native = _native()
    print(f"case router-decode T={T} H={H} E={E} k={k} {scoring}", flush=True)
    rng = np.random.default_rng(31 + T + E)
    x = normal_bf16(rng, (T, H), 1.0)
    wg = normal_bf16(rng, (E, H), 0.02)
    bias = (rng.standard_normal(E) * (0.01 if scoring == "sigmoid" else 0.5)).astype(np.float32)
    dx, dwg, dbias = to_dev_bf16(x), to_dev_bf16(wg), torch.from_numpy(bias).cuda()
    kw = dict(scoring=scoring, bias=dbias, num_expert_group=G, topk_group=TG,
              routed_scaling_factor=2.5 if scoring == "sigmoid" else 1.0)
    sync = torch.zeros(1, dtype=torch.int32, device="cuda")
    w_f32 = torch.empty((T, k), dtype=torch.float32, device="cuda")
    w, ids, logits = native.router_decode(dx, dwg, k, sync, w_f32=w_f32, **kw)
    ref_logits = torch.empty((T, E), dtype=torch.bfloat16, device="cuda")
    native.router_gate(dx, dwg, ref_logits)
    w2_, ids2, _ = native.router_topk(ref_logits, k, **kw)
    w3, ids3, _ = native.router_decode(dx, dwg, k, sync, **kw)
    torch.cuda.synchronize()
    assert int(sync.item()) == 0
    assert torch.equal(logits.view(torch.int16), ref_logits.view(torch.int16))
    lg32 = bf16_to_f32(from_dev_bf16(logits))
    if scoring == "softmax":
        r_ids, r_w, r_wb = orc.softmax_topk(lg32, k, bias=bias)
    else:
        r_ids, r_w, r_wb = orc.grouped_sigmoid_topk(lg32, k, bias=bias, n_group=G, topk_group=TG, scale=2.5)
    np.testing.assert_array_equal(ids.cpu().numpy(), r_ids)
    np.testing.assert_array_equal(from_dev_bf16(w), r_wb)
    np.testing.assert_array_equal(w_f32.cpu().numpy().view(np.uint32), r_w.view(np.uint32))
    for a, b in ((ids2, ids), (ids3, ids)):
        assert torch.equal(a, b)
    for a, b in ((w2_, w), (w3, w)):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_router_decode_graph_replays():
    native = _native()
    rng = np.random.default_rng(5150)
    T, H, E, k = 4, 2048, 128, 8
    wg = to_dev_bf16(normal_bf16(rng, (E, H), 0.02))
    sync = torch.zeros(1, dtype=torch.int32, device="cuda")
    x = torch.zeros((T, H), dtype=torch.bfloat16, device="cuda")
    w = torch.empty((T, k), dtype=torch.bfloat16, device="cuda")
    ids = torch.empty((T, k), dtype=torch.int32, device="cuda")
    logits = torch.empty((T, E), dtype=torch.bfloat16, device="cuda")
    x.copy_(to_dev_bf16(normal_bf16(rng, (T, H), 1.0)))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        native.router_decode(x, wg, k, sync, logits=logits, w_bf16=w, ids=ids)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        native.router_decode(x, wg, k, sync, logits=logits, w_bf16=w, ids=ids)
    for rep in range(4):
        xs = normal_bf16(rng, (T, H), 1.0)
        x.copy_(to_dev_bf16(xs))
        g.replay()
        torch.cuda.synchronize()
        got_lg = bf16_to_f32(from_dev_bf16(logits))
        wgb = from_dev_bf16(wg)
        exact = orc.gate_logits(xs, wgb)
        absdot = np.abs(bf16_to_f32(xs)).astype(np.float64) @ np.abs(bf16_to_f32(wgb)).astype(np.float64).T
        assert np.all(np.abs(got_lg - exact) <= bf16_ulp(exact) + 4.0 * np.sqrt(H) * 2.0 ** -24 * absdot)
        ref_ids, _, ref_wb = orc.softmax_topk(got_lg, k)
        np.testing.assert_array_equal(ids.cpu().numpy(), ref_ids)
        np.testing.assert_array_equal(from_dev_bf16(w), ref_wb)
        # eager work between replays
        e_w, e_ids, _ = native.router_decode(x, wg, k, sync)
        torch.cuda.synchronize()
        assert torch.equal(e_ids, ids) and int(sync.item()) == 0
