"""GPU parity of the one-launch selection + permutation (lmoe_router_topk_permute)
and of the decode layer built on it.

Everything here is integer or bit-exact: the ids, bf16 and f32 weights
against oracle.router, the permutation against oracle.permute, and the
decode layer against route() + fused_experts() on the same GPU.
"""

import numpy as np
import pytest
import torch

from oracle import permute as operm
from oracle import router as orc
from oracle.bf16 import bf16_to_f32, f32_to_bf16, normal_bf16
from tests._util import from_dev_bf16, to_dev_bf16, to_dev_i32

pytestmark = pytest.mark.gpu


def _native():
    from vllm_moe_offload_amd import native

    return native


def _tied_logits(rng, T, E, step=0.25):
    v = np.round(rng.standard_normal((T, E)) / step) * step
    return f32_to_bf16(v.astype(np.float32))


def _check_perm(native, perm, ref, n_pairs):
    np.testing.assert_array_equal(perm.counts.cpu().numpy(), ref.counts)
    np.testing.assert_array_equal(perm.offsets.cpu().numpy(), ref.offsets)
    np.testing.assert_array_equal(perm.sorted_pairs.cpu().numpy()[: ref.placed], ref.sorted_pairs)
    np.testing.assert_array_equal(perm.row_idx.cpu().numpy()[:n_pairs], ref.row_idx)
    np.testing.assert_array_equal(perm.active.cpu().numpy()[: ref.active.size], ref.active)
    np.testing.assert_array_equal(perm.tile_off.cpu().numpy(), ref.tile_off)
    meta = perm.meta.cpu().numpy()
    assert list(meta[:4]) == [ref.active.size, ref.placed, ref.errors, ref.tile_off[-1]]
    assert meta[native.META_GEN] == perm.builds  # one per build


@pytest.mark.parametrize("T,E,k,P,skip,skew", [
    (1, 128, 8, 64, False, False),
    (4, 128, 8, 64, False, False),
    (16, 128, 8, 64, False, False),
    (16, 128, 8, 32, True, False),    # a wave table: ids outside it are left to another pass
    (17, 128, 8, 128, False, False),  # past the one-block limit: the two-launch path
    (3, 60, 4, 16, False, False),
    # skewed gate bias: heavy slots lead the active list (one wave, one
    # block of 512 and of 1024 pairs)
    (16, 128, 8, 128, False, True),
    (64, 128, 8, 128, False, True),
    (128, 128, 8, 128, False, True),
])
def test_softmax_select_and_permute_bit_exact(T, E, k, P, skip, skew):
    native = _native()
    print(f"case topk-permute softmax T={T} E={E} k={k} P={P} skip={skip} skew={skew}", flush=True)
    rng = np.random.default_rng(500 + T * 13 + P)
    bits = _tied_logits(rng, T, E)
    lbias = (rng.standard_normal(E) * 0.7).astype(np.float32)
    if skew:  # Zipf-like: expert of rank r gets -1.5 log r
        lbias = (-1.5 * np.log(rng.permutation(E) + 1.0)).astype(np.float32)
    cbias = (rng.standard_normal(E) * 0.004).astype(np.float32)
    r_ids, r_w, r_wb = orc.softmax_topk(bf16_to_f32(bits), k, bias=cbias, logit_bias=lbias)
    # slot table: every selected expert mapped (skip: only a subset)
    used = np.unique(r_ids)
    l2p = np.full(E, -1, dtype=np.int32)
    chosen = used[: P] if not skip else used[: min(P, max(1, used.size // 2))]
    l2p[chosen] = rng.permutation(P)[: chosen.size]
    perm = native.Permutation.allocate(T * k, P, "cuda")
    w_f32 = torch.empty((T, k), dtype=torch.float32, device="cuda")
    w, ids, _ = native.router_topk_permute(
        to_dev_bf16(bits), k, perm, log2phy=to_dev_i32(l2p), skip_unmapped=skip,
        bias=torch.from_numpy(cbias).cuda(), logit_bias=torch.from_numpy(lbias).cuda(), w_f32=w_f32,
    )
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ids.cpu().numpy(), r_ids)
    np.testing.assert_array_equal(from_dev_bf16(w), r_wb)
    np.testing.assert_array_equal(w_f32.cpu().numpy().view(np.uint32), r_w.view(np.uint32))
    ref = operm.init_routing(r_ids, P, log2phy=l2p, skip_unmapped=skip, block_m=native.MFMA_BLOCK_M)
    if skew:  # the case exercises the heavy-first order
        assert ((ref.counts >= operm.HEAVY_MIN_PAIRS) & (16 * ref.counts >= ref.placed)).sum() >= 2
    _check_perm(native, perm, ref, T * k)
    assert perm.block_m == native.MFMA_BLOCK_M


@pytest.mark.parametrize("T", [1, 8, 16])
def test_grouped_sigmoid_select_and_permute_bit_exact(T):
    native = _native()
    E, G, TG, k, P, scale = 256, 8, 4, 8, 128, 2.5  # P covers the <= 128 selected experts
    print(f"case topk-permute sigmoid T={T}", flush=True)
    rng = np.random.default_rng(900 + T)
    bits = _tied_logits(rng, T, E, step=0.125)
    bias = (rng.standard_normal(E) * 0.01).astype(np.float32)
    r_ids, r_w, r_wb = orc.grouped_sigmoid_topk(bf16_to_f32(bits), k, bias=bias, n_group=G, topk_group=TG,
                                                scale=scale)
    used = np.unique(r_ids)
    l2p = np.full(E, -1, dtype=np.int32)
    l2p[used] = rng.permutation(P)[: used.size]
    perm = native.Permutation.allocate(T * k, P, "cuda")
    w, ids, _ = native.router_topk_permute(
        to_dev_bf16(bits), k, perm, log2phy=to_dev_i32(l2p), scoring="sigmoid",
        bias=torch.from_numpy(bias).cuda(), num_expert_group=G, topk_group=TG,
        routed_scaling_factor=scale,
    )
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ids.cpu().numpy(), r_ids)
    np.testing.assert_array_equal(from_dev_bf16(w), r_wb)
    _check_perm(native, perm, operm.init_routing(r_ids, P, log2phy=l2p, block_m=native.MFMA_BLOCK_M), T * k)


def test_unmapped_selection_counts_as_error():
    """An id the table does not map (outside wave mode) is an error pair."""
    native = _native()
    T, E, k, P = 2, 64, 4, 8
    rng = np.random.default_rng(3)
    bits = _tied_logits(rng, T, E)
    r_ids, _, _ = orc.softmax_topk(bf16_to_f32(bits), k)
    l2p = np.full(E, -1, dtype=np.int32)
    l2p[np.unique(r_ids)[:-1]] = np.arange(np.unique(r_ids).size - 1) % P
    perm = native.Permutation.allocate(T * k, P, "cuda")
    native.router_topk_permute(to_dev_bf16(bits), k, perm, log2phy=to_dev_i32(l2p))
    torch.cuda.synchronize()
    ref = operm.init_routing(r_ids, P, log2phy=l2p, block_m=native.MFMA_BLOCK_M)
    assert ref.errors > 0
    _check_perm(native, perm, ref, T * k)


@pytest.mark.parametrize("T", [1, 4, 16])
def test_decode_layer_equals_route_then_fused_experts(T):
    from vllm_moe_offload_amd import fused_moe
    from vllm_moe_offload_amd.fused_moe import RouterSpec

    native = _native()
    H, I, E, k = 2048, 768, 128, 8
    P = 64 if T <= 4 else 128  # enough slots for every selected expert
    print(f"case decode-layer T={T}", flush=True)
    rng = np.random.default_rng(40 + T)
    x = to_dev_bf16(normal_bf16(rng, (T, H), 1.0))
    gate = to_dev_bf16(normal_bf16(rng, (E, H), 0.02))
    lbias = torch.from_numpy((rng.standard_normal(E) * 0.5).astype(np.float32)).cuda()
    cbias = torch.from_numpy((rng.standard_normal(E) * 0.004).astype(np.float32)).cuda()
    spec = RouterSpec(top_k=k, e_score_correction_bias=cbias, logit_bias=lbias)
    w13 = to_dev_bf16(normal_bf16(rng, (P, 2 * I, H), 0.02))
    w2 = to_dev_bf16(normal_bf16(rng, (P, H, I), 0.02))
    # the table: route once to learn the experts, map them to slots
    w0, ids0, _ = fused_moe.route(x, gate, spec)
    torch.cuda.synchronize()
    used = np.unique(ids0.cpu().numpy())
    l2p = np.full(E, -1, dtype=np.int32)
    l2p[used] = rng.permutation(P)[: used.size]
    d_l2p = to_dev_i32(l2p)
    ws_a = fused_moe.get_workspace(T, k, P, H, I, "cuda", tag="t-sep")
    ws_b = fused_moe.get_workspace(T, k, P, H, I, "cuda", tag="t-fused")
    w1, ids1, _ = fused_moe.route(x, gate, spec)
    out1 = fused_moe.fused_experts(x, w1, ids1, w13, w2, d_l2p, workspace=ws_a).clone()
    out2, w2_, ids2 = fused_moe.decode_layer(x, gate, spec, w13, w2, d_l2p, workspace=ws_b)
    torch.cuda.synchronize()
    assert torch.equal(ids1, ids2)
    assert torch.equal(w1.view(torch.int16), w2_.view(torch.int16))
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16))
    if T == 1:  # one token: the layer's router leaves the pairs in pair order
        _check_pair_order(native, ws_b.perm, ids2.cpu().numpy(), l2p, P, False)
        return
    for name in ("counts", "offsets", "sorted_pairs", "row_idx", "active", "tile_off", "meta"):
        a, b = getattr(ws_a.perm, name), getattr(ws_b.perm, name)
        # meta: the four counts (past them, build count and decode hand-off state)
        n = T * k if name in ("sorted_pairs", "row_idx") else 4 if name == "meta" else a.numel()
        assert torch.equal(a[:n], b[:n]), name


@pytest.mark.parametrize("T,E,k,P,H,scoring,f32", [
    (1, 128, 8, 64, 2048, "softmax", False),
    (4, 128, 8, 64, 2048, "softmax", True),
    (16, 128, 8, 128, 2048, "softmax", False),   # 1024-thread blocks, block permutation
    (3, 60, 4, 16, 512, "softmax", False),       # E not a multiple of the waves per block
    (1, 256, 8, 128, 7168, "sigmoid", False),    # grouped sigmoid, long rows (one token only)
    (8, 256, 8, 128, 2048, "sigmoid", False),    # grouped sigmoid, several tokens
])
def test_gate_select_permute_one_launch_equals_separate_calls(T, E, k, P, H, scoring, f32):
    """lmoe_router_gate_topk_permute == lmoe_router_gate then
    lmoe_router_topk_permute, bit for bit, over three calls in a row (the
    arrival counter must be back at zero after each)."""
    native = _native()
    print(f"case gate-topk-permute T={T} E={E} k={k} P={P} H={H} {scoring} f32={f32}", flush=True)
    rng = np.random.default_rng(70 + T + E)
    grouped = scoring == "sigmoid"
    kw = dict(scoring=scoring, num_expert_group=8 if grouped else 1, topk_group=4 if grouped else 1,
              routed_scaling_factor=2.5 if grouped else 1.0)
    bias = torch.from_numpy((rng.standard_normal(E) * 0.01).astype(np.float32)).cuda()
    if not grouped:  # softmax: a gate bias as well as the correction bias
        kw["logit_bias"] = torch.from_numpy((rng.standard_normal(E) * 0.5).astype(np.float32)).cuda()
    dt = torch.float32 if f32 else torch.bfloat16
    wg = to_dev_bf16(normal_bf16(rng, (E, H), 0.02))
    perm_a = native.Permutation.allocate(T * k, P, "cuda")
    perm_b = native.Permutation.allocate(T * k, P, "cuda")
    for it in range(3):
        x = to_dev_bf16(normal_bf16(rng, (T, H), 1.0))
        # slot table covering whatever this step selects
        lg0 = torch.empty((T, E), dtype=dt, device="cuda")
        native.router_gate(x, wg, lg0)
        _, ids0, _ = native.router_topk(lg0, k, bias=bias, **kw)
        used = np.unique(ids0.cpu().numpy())
        l2p = np.full(E, -1, dtype=np.int32)
        l2p[used] = rng.permutation(P)[: used.size]
        d_l2p = to_dev_i32(l2p)
        lg_a = torch.empty((T, E), dtype=dt, device="cuda")
        native.router_gate(x, wg, lg_a)
        wa, ida, wfa = native.router_topk_permute(lg_a, k, perm_a, log2phy=d_l2p, bias=bias,
                                                  w_f32=torch.empty((T, k), device="cuda"), **kw)
        lg_b = torch.empty((T, E), dtype=dt, device="cuda")
        wb, idb, wfb = native.router_gate_topk_permute(x, wg, lg_b, k, perm_b, log2phy=d_l2p, bias=bias,
                                                       w_f32=torch.empty((T, k), device="cuda"), **kw)
        torch.cuda.synchronize()
        view = torch.int32 if f32 else torch.int16
        assert torch.equal(lg_a.view(view), lg_b.view(view)), it
        assert torch.equal(ida, idb), it
        assert torch.equal(wa.view(torch.int16), wb.view(torch.int16)), it
        assert torch.equal(wfa.view(torch.int32), wfb.view(torch.int32)), it
        for name in ("counts", "offsets", "sorted_pairs", "row_idx", "active", "tile_off", "meta"):
            assert torch.equal(getattr(perm_a, name), getattr(perm_b, name)), (it, name)
        assert perm_b.sync[0].item() == 0
        assert perm_b.meta[native.META_ROUTER_TIMEOUT].item() == 0


@pytest.mark.parametrize("T,E,k,S,scoring,H", [
    (1, 128, 8, 1, "softmax", 2048),
    (16, 128, 8, 2, "softmax", 2048),
    (1, 256, 8, 1, "sigmoid", 7168),   # the DeepSeek-style decode layer with its shared expert
    (3, 256, 8, 1, "sigmoid", 7168),
])
def test_shared_suffix_in_all_three_routers(T, E, k, S, scoring, H):
    """n_shared = S appends ids E..E+S-1 with weight 1 after the k routed
    columns (the mix-placement suffix), in the plain selection, the
    selection + permutation, and the gate + selection + permutation
    launches; the permutation covers the suffix pairs through the slot
    table like any other."""
    native = _native()
    print(f"case shared-suffix T={T} E={E} k={k} S={S} {scoring}", flush=True)
    rng = np.random.default_rng(4100 + T * 7 + S)
    grouped = scoring == "sigmoid"
    G, TG, scale = (8, 4, 2.5) if grouped else (1, 1, 1.0)
    kw = dict(scoring=scoring, num_expert_group=G, topk_group=TG, routed_scaling_factor=scale, n_shared=S)
    bias_np = (rng.standard_normal(E) * 0.01).astype(np.float32)
    bias = torch.from_numpy(bias_np).cuda()
    x = to_dev_bf16(normal_bf16(rng, (T, H), 1.0))
    wg = to_dev_bf16(normal_bf16(rng, (E, H), 0.02))
    logits = torch.empty((T, E), dtype=torch.bfloat16, device="cuda")
    native.router_gate(x, wg, logits)
    lg = bf16_to_f32(from_dev_bf16(logits))
    if grouped:
        r_ids, r_w, r_wb = orc.grouped_sigmoid_topk(lg, k, bias=bias_np, n_group=G, topk_group=TG, scale=scale)
    else:
        r_ids, r_w, r_wb = orc.softmax_topk(lg, k, bias=bias_np)
    # expected rows: the routed columns, then the suffix with weight 1
    suffix = np.broadcast_to(np.arange(E, E + S, dtype=np.int32), (T, S))
    e_ids = np.concatenate([r_ids, suffix], axis=1)
    e_w = np.concatenate([r_w, np.ones((T, S), np.float32)], axis=1)
    e_wb = np.concatenate([r_wb, np.full((T, S), 0x3F80, np.uint16)], axis=1)
    # slot table over E + S ids: the suffix pinned at the last S slots
    used = np.unique(r_ids)
    P = max(64, used.size + S)
    l2p = np.full(E + S, -1, dtype=np.int32)
    l2p[used] = rng.permutation(P - S)[: used.size]
    l2p[E:] = np.arange(P - S, P, dtype=np.int32)
    d_l2p = to_dev_i32(l2p)
    ref = operm.init_routing(e_ids, P, log2phy=l2p, block_m=native.MFMA_BLOCK_M)

    def check(w, ids, w_f32):
        np.testing.assert_array_equal(ids.cpu().numpy(), e_ids)
        np.testing.assert_array_equal(from_dev_bf16(w), e_wb)
        np.testing.assert_array_equal(w_f32.cpu().numpy().view(np.uint32), e_w.view(np.uint32))

    wf = torch.empty((T, k + S), dtype=torch.float32, device="cuda")
    w, ids, _ = native.router_topk(logits, k, bias=bias, w_f32=wf, **kw)
    torch.cuda.synchronize()
    check(w, ids, wf)
    for fused_gate in (False, True):
        perm = native.Permutation.allocate(T * (k + S), P, "cuda")
        wf = torch.empty((T, k + S), dtype=torch.float32, device="cuda")
        if fused_gate:
            lg2 = torch.empty((T, E), dtype=torch.bfloat16, device="cuda")
            w, ids, _ = native.router_gate_topk_permute(x, wg, lg2, k, perm, log2phy=d_l2p, bias=bias, w_f32=wf, **kw)
        else:
            w, ids, _ = native.router_topk_permute(logits, k, perm, log2phy=d_l2p, bias=bias, w_f32=wf, **kw)
        torch.cuda.synchronize()
        check(w, ids, wf)
        _check_perm(native, perm, ref, T * (k + S))


@pytest.mark.parametrize("E,k,P,H,tie_rows", [
    (128, 8, 64, 2048, 6),   # the Qwen3-shaped decode router, six experts tied with a seventh
    (256, 8, 128, 1024, 9),  # four experts per lane
    (60, 4, 16, 512, 5),     # E not a multiple of 64: lanes past E hold no expert
    (16, 2, 8, 512, 0),
])
def test_one_token_one_launch_router_with_ties_equals_separate_calls_and_oracle(E, k, P, H, tie_rows):
    """The one-token one-launch router (gate, selection and permutation in
    one kernel, the decode replay's router) against the separate calls and
    the oracle, bit for bit, ties included: tie_rows gate rows are copies of
    one row, so their logits are equal and the lower ids must be taken
    first; every other step steers the token onto the tied rows."""
    native = _native()
    print(f"case one-token-router-ties E={E} k={k} P={P} H={H} ties={tie_rows}", flush=True)
    rng = np.random.default_rng(900 + E + tie_rows)
    wg_h = normal_bf16(rng, (E, H), 0.02)
    if tie_rows:
        src = int(rng.integers(E))
        for r in rng.permutation(E)[:tie_rows]:
            wg_h[r] = wg_h[src]
    wg = to_dev_bf16(wg_h)
    perm_a = native.Permutation.allocate(k, P, "cuda")
    perm_b = native.Permutation.allocate(k, P, "cuda")
    for it in range(4):
        x_h = normal_bf16(rng, (1, H), 1.0)
        x = to_dev_bf16(x_h)
        if tie_rows and it % 2 == 1:
            # steer the tied experts to the top: x along their shared row
            x_h = f32_to_bf16(bf16_to_f32(wg_h[src])[None, :] * np.float32(40.0))
            x = to_dev_bf16(x_h)
        lg0 = torch.empty((1, E), dtype=torch.bfloat16, device="cuda")
        native.router_gate(x, wg, lg0)
        _, ids0, _ = native.router_topk(lg0, k)
        used = np.unique(ids0.cpu().numpy())
        l2p = np.full(E, -1, dtype=np.int32)
        l2p[used] = rng.permutation(P)[: used.size]
        d_l2p = to_dev_i32(l2p)
        lg_a = torch.empty((1, E), dtype=torch.bfloat16, device="cuda")
        native.router_gate(x, wg, lg_a)
        wa, ida, wfa = native.router_topk_permute(lg_a, k, perm_a, log2phy=d_l2p,
                                                  w_f32=torch.empty((1, k), device="cuda"))
        lg_b = torch.empty((1, E), dtype=torch.bfloat16, device="cuda")
        wb, idb, wfb = native.router_gate_topk_permute(x, wg, lg_b, k, perm_b, log2phy=d_l2p,
                                                       w_f32=torch.empty((1, k), device="cuda"))
        torch.cuda.synchronize()
        assert torch.equal(lg_a.view(torch.int16), lg_b.view(torch.int16)), it
        assert torch.equal(ida, idb), it
        assert torch.equal(wa.view(torch.int16), wb.view(torch.int16)), it
        assert torch.equal(wfa.view(torch.int32), wfb.view(torch.int32)), it
        for name in ("counts", "offsets", "sorted_pairs", "row_idx", "active", "tile_off"):
            assert torch.equal(getattr(perm_a, name), getattr(perm_b, name)), (it, name)
        lg = bf16_to_f32(from_dev_bf16(lg_b))
        r_ids, _, r_wb = orc.softmax_topk(lg, k)
        assert np.array_equal(idb.cpu().numpy(), r_ids), it
        assert np.array_equal(wb.view(torch.int16).cpu().numpy().view(np.uint16), r_wb), it
        if tie_rows and it % 2 == 1:
            # the steered step really selects tied experts
            vals = lg[0, r_ids[0]]
            assert np.unique(vals).size < k, "no tie among the selected experts"


def _check_pair_order(native, perm, ids, l2p, P, skip, n_shared_ids=()):
    """The one-token pair-order outputs against the oracle's remap: the
    placed pairs at positions 0, 1, ... in pair order."""
    flat = ids.reshape(-1)
    slot = operm.remap(flat, l2p, P, skip_unmapped=skip)
    placed = np.flatnonzero(slot >= 0)
    n = placed.size
    row_idx = perm.row_idx.cpu().numpy()[: flat.size]
    want_rows = np.full(flat.size, -1)
    want_rows[placed] = np.arange(n)
    np.testing.assert_array_equal(row_idx, want_rows)
    np.testing.assert_array_equal(perm.sorted_pairs.cpu().numpy()[:n], placed)
    active = perm.active.cpu().numpy()
    np.testing.assert_array_equal(active[:n], slot[placed])
    assert (active[n:P] == -1).all()
    meta = perm.meta.cpu().numpy()
    assert list(meta[:3]) == [n, n, int((slot == -2).sum())]
    assert meta[native.META_GEN] == perm.builds
    return n


@pytest.mark.parametrize("E,k,S,P,H,scoring,table", [
    (128, 8, 0, 64, 2048, "softmax", "map"),      # the Qwen3-shaped decode replay
    (128, 8, 0, 128, 2048, "softmax", "none"),    # no table: ids are slots
    (128, 8, 0, 64, 1536, "softmax", "skip"),     # guarded gate rows; two pairs left to another pass
    (128, 8, 0, 64, 2048, "softmax", "error"),    # a selected expert in no slot: an error
    (256, 8, 1, 300, 7168, "sigmoid", "map"),     # grouped sigmoid, long rows, a shared expert
])
def test_pair_order_router_equals_one_launch_router(E, k, S, P, H, scoring, table):
    """lmoe_router_gate_topk_pairs gives lmoe_router_gate_topk_permute's
    logits, ids and weights bit for bit (three calls in a row: the arrival
    counter is back at zero after each), and the pairs in pair order against
    the oracle's remap."""
    native = _native()
    print(f"case pair-order router E={E} k={k} S={S} P={P} H={H} {scoring} table={table}", flush=True)
    rng = np.random.default_rng(300 + E + H)
    grouped = scoring == "sigmoid"
    kw = dict(scoring=scoring, num_expert_group=8 if grouped else 1, topk_group=4 if grouped else 1,
              routed_scaling_factor=2.5 if grouped else 1.0, n_shared=S)
    bias = torch.from_numpy((rng.standard_normal(E) * 0.01).astype(np.float32)).cuda()
    wg = to_dev_bf16(normal_bf16(rng, (E, H), 0.02))
    kwp = k + S
    perm_a = native.Permutation.allocate(kwp, P, "cuda")
    perm_b = native.Permutation.allocate(kwp, P, "cuda")
    perm_b.active.fill_(77)  # stale entries the call must overwrite
    for it in range(3):
        x = to_dev_bf16(normal_bf16(rng, (1, H), 1.0))
        lg0 = torch.empty((1, E), dtype=torch.bfloat16, device="cuda")
        native.router_gate(x, wg, lg0)
        _, ids0, _ = native.router_topk(lg0, k, bias=bias, **kw)
        used = np.unique(ids0.cpu().numpy())
        skip = table == "skip"
        if table == "none":
            l2p, d_l2p = None, None
        else:
            l2p = np.full(E + S, -1, dtype=np.int32)
            l2p[used] = rng.permutation(P)[: used.size]
            if table in ("skip", "error"):
                l2p[used[:2]] = -1  # in no slot of this table
            d_l2p = to_dev_i32(l2p)
        lg_a = torch.empty((1, E), dtype=torch.bfloat16, device="cuda")
        wa, ida, wfa = native.router_gate_topk_permute(x, wg, lg_a, k, perm_a, log2phy=d_l2p, bias=bias,
                                                       skip_unmapped=skip, w_f32=torch.empty((1, kwp), device="cuda"),
                                                       **kw)
        lg_b = torch.empty((1, E), dtype=torch.bfloat16, device="cuda")
        wb, idb, wfb = native.router_gate_topk_pairs(x, wg, lg_b, k, perm_b, log2phy=d_l2p, bias=bias,
                                                     skip_unmapped=skip, w_f32=torch.empty((1, kwp), device="cuda"),
                                                     **kw)
        torch.cuda.synchronize()
        assert torch.equal(lg_a.view(torch.int16), lg_b.view(torch.int16)), it
        assert torch.equal(ida, idb), it
        assert torch.equal(wa.view(torch.int16), wb.view(torch.int16)), it
        assert torch.equal(wfa.view(torch.int32), wfb.view(torch.int32)), it
        ids_np = idb.cpu().numpy()
        n = _check_pair_order(native, perm_b, ids_np, l2p, P, skip)
        assert n == (kwp - 2 if table in ("skip", "error") else kwp)
        assert perm_b.sync[0].item() == 0
        assert perm_b.meta[native.META_ROUTER_TIMEOUT].item() == 0


@pytest.mark.parametrize("E,k,S,P,H,I,scoring", [
    (128, 8, 0, 64, 2048, 768, "softmax"),
    (256, 8, 1, 64, 7168, 2048, "sigmoid"),   # nine pairs: a half wave takes two slots
])
def test_one_token_body_from_pair_order_equals_sorted(E, k, S, P, H, I, scoring):
    """fused_moe_decode(distinct_slots=True) from the pair-order router's
    outputs gives the bits it gives from the sorted permutation (with an add
    term), and decode_layer at one token (which takes the pair order) equals
    route() + fused_experts()."""
    native = _native()
    from vllm_moe_offload_amd import fused_moe

    print(f"case one-token body pair order E={E} H={H} I={I}", flush=True)
    rng = np.random.default_rng(900 + E)
    grouped = scoring == "sigmoid"
    kw = dict(scoring=scoring, num_expert_group=8 if grouped else 1, topk_group=4 if grouped else 1,
              routed_scaling_factor=2.5 if grouped else 1.0, n_shared=S)
    kwp = k + S
    wg = to_dev_bf16(normal_bf16(rng, (E, H), 0.02))
    w13 = to_dev_bf16(normal_bf16(rng, (P, 2 * I, H), 0.02))
    w2 = to_dev_bf16(normal_bf16(rng, (P, H, I), 0.02))
    x = to_dev_bf16(normal_bf16(rng, (1, H), 1.0))
    add = to_dev_bf16(normal_bf16(rng, (1, H), 0.5))
    l2p = np.full(E + S, -1, dtype=np.int32)
    l2p[rng.permutation(E + S)[:P]] = rng.permutation(P)
    # make sure the selected experts are in slots: route once, then map them
    lg0 = torch.empty((1, E), dtype=torch.bfloat16, device="cuda")
    native.router_gate(x, wg, lg0)
    _, ids0, _ = native.router_topk(lg0, k, **kw)
    used = np.unique(ids0.cpu().numpy())
    l2p[:] = -1
    l2p[used] = rng.permutation(P)[: used.size]
    d_l2p = to_dev_i32(l2p)
    outs = []
    for form in ("sorted", "pairs"):
        perm = native.Permutation.allocate(kwp, P, "cuda")
        lg = torch.empty((1, E), dtype=torch.bfloat16, device="cuda")
        router = native.router_gate_topk_permute if form == "sorted" else native.router_gate_topk_pairs
        w, ids, _ = router(x, wg, lg, k, perm, log2phy=d_l2p, **kw)
        act = torch.empty((kwp, I), dtype=torch.bfloat16, device="cuda")
        y = torch.empty((kwp, H), dtype=torch.bfloat16, device="cuda")
        out = torch.empty((1, H), dtype=torch.bfloat16, device="cuda")
        native.fused_moe_decode(x, w, w13, w2, perm, act, out, add=add, y=y, distinct_slots=True)
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
