"""lmoe_fused_moe_decode_noalloc (act / y in the library's per-GPU scratch
array) against lmoe_fused_moe_decode with caller workspaces, through the
C-ABI: bit for bit, on calls in a row whose later inputs are smaller, so a
stale row of an earlier call would show.  Sizes past the scratch array are
refused on the host before any device work."""

import numpy as np
import pytest
import torch

from oracle.bf16 import f32_to_bf16, normal_bf16
from tests._util import to_dev_bf16, to_dev_i32

pytestmark = pytest.mark.gpu


def _case(native, seed, T, k, E, P, H, I):
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    used = np.unique(ids)
    l2p = np.full(E, -1, dtype=np.int32)
    l2p[used] = rng.permutation(P)[: used.size]
    w = rng.random((T, k)).astype(np.float32)
    w = f32_to_bf16(w / w.sum(1, keepdims=True))
    x = to_dev_bf16(normal_bf16(rng, (T, H), 1.0))
    perm = native.Permutation.allocate(T * k, P, "cuda")
    native.permute(to_dev_i32(ids), perm, log2phy=to_dev_i32(l2p))
    return x, to_dev_bf16(w), perm


@pytest.mark.parametrize("H,I,E,P,k,sizes", [
    (2048, 768, 128, 128, 8, (16, 1, 4)),    # Qwen3 shape: y body, then one-token kernels
    (7168, 2048, 256, 64, 9, (4, 2, 1)),     # DeepSeek-V3 expert shape, nine pairs a token
])
def test_noalloc_decode_equals_workspace_decode(H, I, E, P, k, sizes):
    from vllm_moe_offload_amd import native

    g = torch.Generator(device="cuda").manual_seed(H + k)
    w13 = (torch.randn((P, 2 * I, H), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    w2 = (torch.randn((P, H, I), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    for call, T in enumerate(sizes):
        for distinct in (False, True):
            print(f"case noalloc H={H} T={T} call={call} distinct={distinct}", flush=True)
            x, w, perm = _case(native, 100 * call + T, T, k, E, P, H, I)
            act = torch.empty((T * k, I), dtype=torch.bfloat16, device="cuda")
            y = torch.empty((T * k, H), dtype=torch.bfloat16, device="cuda")
            ref = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
            native.fused_moe_decode(x, w, w13, w2, perm, act, ref, y=y, distinct_slots=distinct)
            out = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device="cuda")
            native.fused_moe_decode_noalloc(x, w, w13, w2, perm, out, distinct_slots=distinct)
            torch.cuda.synchronize()
            assert torch.equal(ref.view(torch.int16), out.view(torch.int16)), (call, T, distinct)


def test_noalloc_refuses_sizes_past_the_scratch_array():
    from vllm_moe_offload_amd import native

    H, I, k, P = 7168, 2048, 8, 8
    T = 100  # 800 pairs (within the 1024-pair limit): 3.3 MB of act + 11.5 MB of y > 8 MiB
    x = torch.zeros((T, H), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((T, k), dtype=torch.bfloat16, device="cuda")
    w13 = torch.zeros((P, 2 * I, H), dtype=torch.bfloat16, device="cuda")
    w2 = torch.zeros((P, H, I), dtype=torch.bfloat16, device="cuda")
    perm = native.Permutation.allocate(T * k, P, "cuda")
    out = torch.zeros((T, H), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="workspace too small"):
        native.fused_moe_decode_noalloc(x, w, w13, w2, perm, out)
    torch.cuda.synchronize()


@pytest.mark.parametrize("H,I,k,t_max,err", [
    (2048, 768, 8, 128, "unsupported shape"),      # Qwen3 shape: the 1024-pair limit binds
    (7168, 2048, 9, 50, "workspace too small"),    # DeepSeek-V3 expert shape + shared pair: the array binds
])
def test_noalloc_limit_boundary(H, I, k, t_max, err):
    """The largest batch the entry point takes runs (bit for bit equal to
    the workspace form); one token more is refused before any device work."""
    from vllm_moe_offload_amd import native

    E = P = 64
    g = torch.Generator(device="cuda").manual_seed(H + 3 * k)
    w13 = (torch.randn((P, 2 * I, H), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    w2 = (torch.randn((P, H, I), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    print(f"case noalloc boundary H={H} T={t_max}", flush=True)
    x, w, perm = _case(native, 900 + k, t_max, k, E, P, H, I)
    act = torch.empty((t_max * k, I), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((t_max * k, H), dtype=torch.bfloat16, device="cuda")
    ref = torch.empty((t_max, H), dtype=torch.bfloat16, device="cuda")
    native.fused_moe_decode(x, w, w13, w2, perm, act, ref, y=y)
    out = torch.full((t_max, H), float("nan"), dtype=torch.bfloat16, device="cuda")
    native.fused_moe_decode_noalloc(x, w, w13, w2, perm, out)
    torch.cuda.synchronize()
    assert torch.equal(ref.view(torch.int16), out.view(torch.int16))
    print(f"case noalloc boundary H={H} T={t_max + 1} (refused)", flush=True)
    x, w, perm = _case(native, 901 + k, t_max + 1, k, E, P, H, I)
    out = torch.zeros((t_max + 1, H), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match=err):
        native.fused_moe_decode_noalloc(x, w, w13, w2, perm, out)
    torch.cuda.synchronize()
