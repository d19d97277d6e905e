"""The C-ABI library loads on the CPU host and exports exactly what
include/latchmoe.h declares; host-side argument checks fail before any
device work (no GPU needed)."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _declared():
    text = (ROOT / "include" / "latchmoe.h").read_text()
    return sorted(set(re.findall(r"\b(lmoe_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    from vllm_moe_offload_amd import native

    assert sorted(native.EXPORTED_SYMBOLS) == _declared()


def test_library_exports_every_declared_symbol():
    from vllm_moe_offload_amd import native

    lib = native.load_library()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.lmoe_abi_version() == 8
    assert lib.lmoe_status_string(1001) == b"unsupported shape"


def test_argument_errors_are_reported_without_a_gpu():
    from vllm_moe_offload_amd import native

    lib = native.load_library()
    # null outputs / bad sizes are rejected on the host
    assert lib.lmoe_router_topk(None, 0, 1, 128, 8, 0, 0, None, None, 1, 1, 1, 1.0, None, None, None, None) == 1000
    assert lib.lmoe_router_topk(ctypes.c_void_p(16), 0, 1, 1024, 8, 0, 0, None, None, 1, 1, 1, 1.0, None,
                                ctypes.c_void_p(16), ctypes.c_void_p(16), None) == 1001
    # shared suffix: a negative count is an argument error, k + n_shared > 16 a shape error
    p16 = ctypes.c_void_p(16)
    assert lib.lmoe_router_topk(p16, 0, 1, 128, 8, -1, 0, None, None, 1, 1, 1, 1.0, None, p16, p16, None) == 1000
    assert lib.lmoe_router_topk(p16, 0, 1, 128, 8, 9, 0, None, None, 1, 1, 1, 1.0, None, p16, p16, None) == 1001
    assert lib.lmoe_permute(None, 4, None, 0, 0, 0, 128, *([None] * 7), None, 0, None) == 1000
    assert lib.lmoe_grouped_mlp(*([ctypes.c_void_p(16)] * 1), 1, 2048, 100, 8, *([ctypes.c_void_p(16)] * 2), 4,
                                *([ctypes.c_void_p(16)] * 5), 8, 128, 0, ctypes.c_void_p(16), ctypes.c_void_p(16), None) == 1001
    assert lib.lmoe_permute_workspace_bytes(1024, 64) == 0
    assert lib.lmoe_permute_workspace_bytes(32768, 48) > 0
    assert lib.lmoe_stage_copy(None, None, None, 0, None, None, None) == 0
    # slot-table update: indices must be distinct and inside the table
    i3 = (ctypes.c_int32 * 3)
    tbl = ctypes.c_void_p(16)
    assert lib.lmoe_table_update(tbl, 8, i3(1, 5, 1), i3(0, 1, 2), 3, None) == 1000
    assert lib.lmoe_table_update(tbl, 8, i3(1, 8, 2), i3(0, 1, 2), 3, None) == 1000
    assert lib.lmoe_table_update(tbl, 8, i3(-1, 3, 2), i3(0, 1, 2), 3, None) == 1000
    assert lib.lmoe_table_update(None, 8, i3(1, 3, 2), i3(0, 1, 2), 3, None) == 1000
    assert lib.lmoe_table_update(None, 8, None, None, 0, None) == 0
    # the one-launch router's sync buffer holds 64-bit words: 8-byte alignment
    p = ctypes.c_void_p(4096)
    args = [p, p, 1, 2048, 128, p, 0, 8, 0, 0, None, None, 1, 1, 1, 1.0, None, p, p, p, 128, 64, 0, 128,
            p, p, p, p, p, p, p]
    assert lib.lmoe_router_gate_topk_permute(*args, ctypes.c_void_p(4100), None) == 1001


def test_empty_batch_is_legal_with_null_operands():
    """T == 0 (or n_pairs == 0): the sizes are still checked, then the call
    returns 0 without touching its token-sized operands, which are null for
    an empty device tensor.  These entries queue nothing for an empty batch,
    so no GPU is needed; the permutation-building ones are covered on the GPU."""
    from vllm_moe_offload_amd import native

    lib = native.load_library()
    N = None
    H, E, I, k, P = 2048, 128, 768, 8, 64
    assert lib.lmoe_router_gate(N, N, 0, H, E, N, 0, N) == 0
    assert lib.lmoe_router_gate(N, N, -1, H, E, N, 0, N) == 1000
    assert lib.lmoe_router_gate(N, N, 0, H + 4, E, N, 0, N) == 1001
    assert lib.lmoe_router_topk(N, 0, 0, E, k, 0, 0, N, N, 1, 1, 1, 1.0, N, N, N, N) == 0
    assert lib.lmoe_router_topk(N, 0, 0, E, E + 1, 0, 0, N, N, 1, 1, 1, 1.0, N, N, N, N) == 1001
    assert lib.lmoe_gateup_silu(N, 0, H, I, k, N, P, N, N, N, N, N, 0, 320, 0, N, N) == 0
    assert lib.lmoe_down(N, H, I, N, P, N, N, N, N, N, 0, 320, 0, N, N) == 0
    assert lib.lmoe_grouped_mlp(N, 0, H, I, k, N, N, P, N, N, N, N, N, 0, 320, 0, N, N, N) == 0
    assert lib.lmoe_grouped_mlp(N, 0, H, 100, k, N, N, P, N, N, N, N, N, 0, 320, 0, N, N, N) == 1001
    assert lib.lmoe_fused_moe_decode(N, 0, H, I, k, N, N, P, *([N] * 10), 0, N) == 0
    assert lib.lmoe_fused_moe_decode_noalloc(N, 0, H, I, k, N, N, P, *([N] * 8), 0, N) == 0
    assert lib.lmoe_down_combine(N, 0, H, I, k, N, P, *([N] * 8)) == 0
    assert lib.lmoe_combine(N, N, N, 0, k, H, N, N, N) == 0
    assert lib.lmoe_combine(N, N, N, 0, k, H - 4, N, N, N) == 1001
    assert lib.lmoe_gather_rows(N, H, k, N, N, 0, N, N) == 0
    # a non-empty batch still needs its operands
    assert lib.lmoe_combine(N, N, N, 1, k, H, N, N, N) == 1000
    assert lib.lmoe_router_gate(N, N, 1, H, E, N, 0, N) == 1000


def test_block_range_gemm_refuses_operands_past_32_bit_offsets():
    """The 320-row block-range prefill kernel forms activation offsets in 32
    bits; an activation operand of 2^31 elements or more is refused on the
    host (LMOE_ERR_SHAPE) before any launch, and prefill_block_m then picks
    the 256-row kernel, whose offsets are 64-bit."""
    import torch

    from vllm_moe_offload_amd import native

    if torch.cuda.is_available():
        pytest.skip("host-only check: the pointers below are placeholders")
    lib = native.load_library()
    p = ctypes.c_void_p(4096)
    H, I, k = 2048, 768, 8
    # down: n_pairs * I = 2.3e9 elements of act
    n = 3_000_000
    assert lib.lmoe_down(p, H, I, p, 64, p, p, p, p, p, n, 320, native.LMOE_PATH_MFMA, p, None) == 1001
    # gate-up: T * H = 2.25e9 elements of x
    T = 1_100_000
    assert lib.lmoe_gateup_silu(p, T, H, I, k, p, 64, p, p, p, p, p, T * k, 320, native.LMOE_PATH_MFMA,
                                p, None) == 1001
    assert native.prefill_block_m(128, H, I, cu_count=256, n_pairs=n) == native.MFMA_BLOCK_M
    assert native.prefill_block_m(128, H, I, cu_count=256, n_pairs=32768) == native.PART_BLOCK_M


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from vllm_moe_offload_amd import native

    monkeypatch.setattr(native, "_LIB", None)
    monkeypatch.setenv("LATCHMOE_HIP_LIB", str(tmp_path / "absent.so"))
    with pytest.raises(native.NativeLibraryMissing, match="no CPU or PyTorch fallback"):
        native.load_library()


def test_prefill_block_m_policy():
    """Row-tile height per prefill pass (no GPU: the CU count is given).
    One round of 320-row units (6 per slot at I = 768) or many rounds -> 320;
    just past one round on 256 CUs (258..320 units) -> the 256-row grid."""
    from vllm_moe_offload_amd import native

    H, I = 2048, 768
    pick = lambda n, cus=256, h=H, i=I: native.prefill_block_m(n, h, i, cu_count=cus)
    assert pick(42) == 320    # 252 units: one round
    assert pick(43) == 256    # 258 units: two would run alone
    assert pick(53) == 256    # 318 units
    assert pick(54) == 320    # 324 units: balanced rounds
    assert pick(128) == 320   # the full layer: 3 units per CU
    assert pick(1) == 320
    assert pick(43, cus=304) == 320          # fits one round on a larger part
    assert pick(42, h=1000) == 256           # K = H not a multiple of 64
    assert pick(64, i=2048) == 320           # 16 units per slot: 1024 units, 4 rounds
