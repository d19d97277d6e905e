"""An empty batch (no tokens) through every stage of the path on the GPU.

Empty device tensors have no address, so each C-ABI entry checks its sizes
and returns before it reads a token-sized operand; the entries that build a
permutation still write it, empty, so nothing of the previous batch is read
afterwards (counts are what the fused-experts result reports as
expert_tokens)."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _stale(perm):
    """Fill a permutation's outputs with values no empty build writes."""
    perm.counts.fill_(7)
    perm.offsets.fill_(7)
    perm.tile_off.fill_(7)
    perm.active.fill_(3)
    perm.meta[:4].fill_(7)


def _assert_empty(native, perm, P):
    torch.cuda.synchronize()
    assert int(perm.counts.abs().sum().item()) == 0
    assert int(perm.offsets.abs().sum().item()) == 0
    assert int(perm.tile_off.abs().sum().item()) == 0
    assert bool((perm.active == -1).all().item())
    for slot in (native.META_ACTIVE, native.META_PAIRS, native.META_TILES, native.META_ERRORS):
        assert int(perm.meta[slot].item()) == 0


@pytest.mark.parametrize("H,E,I,k,P", [(512, 16, 128, 4, 16), (2048, 128, 768, 8, 64)])
def test_empty_batch_through_router_permutation_mlp_and_combine(H, E, I, k, P):
    from vllm_moe_offload_amd import fused_moe, native
    from vllm_moe_offload_amd.fused_moe import RouterSpec

    print(f"case empty batch H={H} E={E} I={I} k={k} P={P}", flush=True)
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(H + E)
    gate = (0.05 * torch.randn((E, H), generator=g, device=dev)).to(torch.bfloat16)
    w13 = (0.02 * torch.randn((P, 2 * I, H), generator=g, device=dev)).to(torch.bfloat16)
    w2 = (0.02 * torch.randn((P, H, I), generator=g, device=dev)).to(torch.bfloat16)
    l2p = torch.full((E,), -1, dtype=torch.int32, device=dev)
    l2p[:P] = torch.arange(P, dtype=torch.int32, device=dev)
    spec = RouterSpec(top_k=k)

    x0 = torch.empty((0, H), dtype=torch.bfloat16, device=dev)
    w0, ids0, logits0 = fused_moe.route(x0, gate, spec)
    assert tuple(w0.shape) == (0, k) and tuple(ids0.shape) == (0, k) and tuple(logits0.shape) == (0, E)

    # the permutation, alone and fused after the selection (with and without the gate)
    perm = native.Permutation.allocate(0, P, dev)
    _stale(perm)
    native.permute(ids0, perm, log2phy=l2p)
    _assert_empty(native, perm, P)
    _stale(perm)
    native.router_topk_permute(logits0, k, perm, log2phy=l2p)
    _assert_empty(native, perm, P)
    _stale(perm)
    native.router_gate_topk_permute(x0, gate, logits0, k, perm, log2phy=l2p)
    _assert_empty(native, perm, P)

    # a decode overflow layer's two tables in one build, and both passes'
    # GEMVs in shared launches
    perm2 = native.Permutation.allocate(0, P, dev)
    _stale(perm)
    _stale(perm2)
    native.permute_two_tables(ids0, perm, l2p, perm2, l2p)
    _assert_empty(native, perm, P)
    _assert_empty(native, perm2, P)
    act0 = torch.empty((0, I), dtype=torch.bfloat16, device=dev)
    y2 = torch.empty((0, H), dtype=torch.bfloat16, device=dev)
    native.decode_mlp_two_passes(x0, k, w13, w2, perm, w13, w2, perm2, act0, y2)

    # the layer body on both paths, and the combine alone
    for path in (native.LMOE_PATH_AUTO, native.LMOE_PATH_MFMA):
        out = fused_moe.fused_experts(x0, w0, ids0, w13, w2, l2p, path=path)
        assert tuple(out.shape) == (0, H)
    y0 = torch.empty((0, H), dtype=torch.bfloat16, device=dev)
    out0 = torch.empty((0, H), dtype=torch.bfloat16, device=dev)
    native.combine(y0, w0, out0)

    # and a batch after the empty one still computes (nothing was left behind)
    x1 = torch.randn((3, H), generator=g, device=dev).to(torch.bfloat16)
    l2p_all = torch.arange(E, dtype=torch.int32, device=dev) % P
    w1, ids1, _ = fused_moe.route(x1, gate, spec)
    out1 = fused_moe.fused_experts(x1, w1, ids1, w13, w2, l2p_all)
    torch.cuda.synchronize()
    assert tuple(out1.shape) == (3, H)
    assert bool(torch.isfinite(out1.float()).all().item())
