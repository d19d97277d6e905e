"""ctypes binding of liblatchmoe_hip.so (the gfx950 hot-path kernels).

Every wrapper takes torch tensors that already live on the GPU, checks shape,
dtype and contiguity on the host, and launches on the current torch stream
(or the stream given).  Nothing here falls back to a CPU or PyTorch
implementation: if the library is missing the import of a wrapper raises.

The C declarations live in include/latchmoe.h; `EXPORTED_SYMBOLS` lists them.
"""

from __future__ import annotations

import atexit
import ctypes
import os
from dataclasses import dataclass
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "liblatchmoe_hip.so"

LMOE_SCORING_SOFTMAX = 0
LMOE_SCORING_SIGMOID = 1
LMOE_PATH_AUTO = 0
LMOE_PATH_GEMV = 1
LMOE_PATH_MFMA = 2
LMOE_ERR_ARG = 1000
LMOE_ERR_SHAPE = 1001
META_ACTIVE, META_PAIRS, META_ERRORS, META_TILES = 0, 1, 2, 3
META_GEN, META_ROUTER_TIMEOUT = 4, 6
ROUTER_SYNC_WORDS = 64 + 2 * 16 * 256  # LMOE_ROUTER_SYNC_WORDS: arrival count, then the tagged logit words
META_COUNT = 64  # LMOE_META_COUNT
FLAG_UNPLACED, FLAG_ROUTER_TIMEOUT, FLAG_COUNT = 0, 1, 4  # lmoe_device_flags words
MFMA_BLOCK_M = 256  # row-tile height of the prefill MFMA GEMM (tile table of lmoe_permute)
PART_BLOCK_M = 320  # row tiles of the one-workgroup-per-CU prefill GEMM (lmoe_grouped_mlp)
FUSED_DECODE_MAX_PAIRS = 1024
SKIP_KEEP_ROWS = 2  # LMOE_SKIP_KEEP_ROWS: lmoe_permute mode of the later passes of a multi-pass layer
GEMV_MAX_I = 4096  # the decode GEMV kernels hold at most 16 chunks of 256 act columns
TWO_PASS_MAX_COLS = 4096  # lmoe_decode_mlp_two_passes: the row-per-wave GEMVs only
PERMUTE_TWO_MAX_PAIRS = 1024  # lmoe_permute_two_tables: one workgroup per table

EXPORTED_SYMBOLS = (
    "lmoe_status_string",
    "lmoe_abi_version",
    "lmoe_device_flags",
    "lmoe_router_gate",
    "lmoe_router_topk",
    "lmoe_router_topk_permute",
    "lmoe_router_gate_topk_permute",
    "lmoe_router_gate_topk_pairs",
    "lmoe_permute_workspace_bytes",
    "lmoe_permute",
    "lmoe_permute_two_tables",
    "lmoe_gather_rows",
    "lmoe_grouped_mlp",
    "lmoe_gateup_silu",
    "lmoe_down",
    "lmoe_decode_mlp_two_passes",
    "lmoe_combine",
    "lmoe_fused_moe_decode",
    "lmoe_fused_moe_decode_noalloc",
    "lmoe_down_combine",
    "lmoe_stage_copy",
    "lmoe_stage_gather",
    "lmoe_table_update",
    "lmoe_slot_plan",
    "lmoe_wave_plan_bytes",
    "lmoe_wave_plan",
    "lmoe_wave_stage",
)

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t

_SIGNATURES = {
    "lmoe_status_string": (ctypes.c_char_p, [_i]),
    "lmoe_abi_version": (_i, []),
    "lmoe_device_flags": (_i, [_vp, _i, _vp]),
    "lmoe_router_gate": (_i, [_vp, _vp, _i, _i, _i, _vp, _i, _vp]),
    "lmoe_router_topk": (
        _i,
        [_vp, _i, _i, _i, _i, _i, _i, _vp, _vp, _i, _i, _i, _f, _vp, _vp, _vp, _vp],
    ),
    "lmoe_router_topk_permute": (
        _i,
        [_vp, _i, _i, _i, _i, _i, _i, _vp, _vp, _i, _i, _i, _f, _vp, _vp, _vp,
         _vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    ),
    "lmoe_router_gate_topk_permute": (
        _i,
        [_vp, _vp, _i, _i, _i, _vp, _i, _i, _i, _i, _vp, _vp, _i, _i, _i, _f, _vp, _vp, _vp,
         _vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    ),
    "lmoe_router_gate_topk_pairs": (
        _i,
        [_vp, _vp, _i, _i, _vp, _i, _i, _i, _i, _vp, _vp, _i, _i, _i, _f, _vp, _vp, _vp, _vp, _i, _i, _i,
         _vp, _vp, _vp, _vp, _vp, _vp],
    ),
    "lmoe_permute_workspace_bytes": (_sz, [_i, _i]),
    "lmoe_permute": (
        _i,
        [_vp, _i, _vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    ),
    "lmoe_permute_two_tables": (
        _i,
        [_vp, _i, _i, _vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp,
         _vp, _vp],
    ),
    "lmoe_gather_rows": (_i, [_vp, _i, _i, _vp, _vp, _i, _vp, _vp]),
    "lmoe_grouped_mlp": (
        _i,
        [_vp, _i, _i, _i, _i, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp, _vp, _vp],
    ),
    "lmoe_gateup_silu": (
        _i,
        [_vp, _i, _i, _i, _i, _vp, _i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp, _vp],
    ),
    "lmoe_down": (_i, [_vp, _i, _i, _vp, _i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp, _vp]),
    "lmoe_decode_mlp_two_passes": (
        _i,
        [_vp, _i, _i, _i, _i, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp, _i, _vp,
         _vp, _vp],
    ),
    "lmoe_combine": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp, _vp, _vp]),
    "lmoe_fused_moe_decode": (
        _i,
        [_vp, _i, _i, _i, _i, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
         _i, _vp],
    ),
    "lmoe_fused_moe_decode_noalloc": (
        _i,
        [_vp, _i, _i, _i, _i, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp],
    ),
    "lmoe_down_combine": (_i, [_vp, _i, _i, _i, _i, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "lmoe_stage_copy": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _vp]),
    "lmoe_stage_gather": (_i, [_vp, _vp, _vp, _i, _vp, _i, _vp, _vp, _i, _i, _vp, _vp, _vp]),
    "lmoe_slot_plan": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _i, _vp, _i, ctypes.c_int64, _vp, _vp]),
    "lmoe_table_update": (_i, [_vp, _i, _vp, _vp, _i, _vp]),
    "lmoe_wave_plan_bytes": (ctypes.c_longlong, [_i, _i, _i]),
    "lmoe_wave_plan": (_i, [_vp, _i, _i, _i, _i, _i, _vp, _vp]),
    "lmoe_wave_stage": (
        _i,
        [_vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, ctypes.c_longlong, ctypes.c_longlong,
         _vp, _i, _i, _i, _vp],
    ),
}

_LIB: ctypes.CDLL | None = None


class NativeLibraryMissing(RuntimeError):
    """liblatchmoe_hip.so is not built; there is no fallback path."""


def library_path() -> Path:
    override = os.environ.get("LATCHMOE_HIP_LIB")
    return Path(override) if override else LIB_PATH


def load_library() -> ctypes.CDLL:
    """Load (once) and return the HIP kernel library, raising if absent."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = library_path()
    if not path.exists():
        raise NativeLibraryMissing(
            f"{path} is missing: build it with "
            "`python vllm-ascend-hust-latchmoe_amd/build_native.py` "
            "(the slot-indexed MoE path has no CPU or PyTorch fallback)"
        )
    lib = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _LIB = lib
    atexit.register(release_device_resources)
    return lib


def release_device_resources() -> dict:
    """Drop every device and page-locked buffer this package holds and
    return them to the HIP runtime while it is fully up: the workspace and
    constant caches, the runtime singleton (slot banks, stage banks, host
    store, events), then torch's device cache and its page-locked host cache.
    Registered with atexit when the library loads, so it runs at the start of
    interpreter shutdown: a page-locked block still cached there would be
    freed only by torch's allocator destructor during C++ static teardown,
    after tools attached to the runtime (a profiler's memory-copy tracing) may
    already have shut down.  Returns torch's host-allocator statistics after
    the release (empty when unavailable).  Safe to call more than once."""
    import gc

    from vllm_moe_offload_amd import fused_moe, layer
    from vllm_moe_offload_amd.moe_offload import runtime

    fused_moe.clear_workspaces()
    layer.clear_constants()
    runtime.reset_moe_offload_runtime()
    gc.collect()
    stats: dict = {}
    try:
        if torch.cuda.is_available() and torch.cuda.is_initialized():
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
            empty_host = getattr(torch._C, "_host_emptyCache", None)
            if empty_host is not None:
                empty_host()
            host_stats = getattr(torch.cuda, "host_memory_stats", None)
            if host_stats is not None:
                stats = dict(host_stats())
    except RuntimeError:
        pass  # a device that already failed has nothing left to return
    return stats


def _check(status: int, fn: str) -> None:
    if status != 0:
        msg = load_library().lmoe_status_string(int(status))
        raise RuntimeError(f"{fn} failed with status {status}: {msg.decode()}")


def device_flags(*, clear: bool = True, stream=None) -> list[int]:
    """The current device's status words (lmoe_device_flags: pairs a masked
    combine dropped, one-launch router waits that gave up), summed over the
    library's kernels since the last clear.  Synchronizes the stream."""
    lib = load_library()
    buf = (ctypes.c_int32 * FLAG_COUNT)()
    _check(lib.lmoe_device_flags(ctypes.cast(buf, ctypes.c_void_p), int(bool(clear)), _stream(stream)),
           "lmoe_device_flags")
    return [int(v) for v in buf]


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else int(t.data_ptr())


def _stream(stream: torch.cuda.Stream | None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def _need(t: torch.Tensor, name: str, dtype: torch.dtype, shape: tuple | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a device tensor, got {t.device}")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")


# ---------------------------------------------------------------------------
# router
# ---------------------------------------------------------------------------
def _check_biases(bias: torch.Tensor | None, logit_bias: torch.Tensor | None, E: int) -> None:
    if bias is not None:
        _need(bias, "e_score_correction_bias", torch.float32, (E,))
    if logit_bias is not None:
        _need(logit_bias, "logit_bias", torch.float32, (E,))


def router_gate(x: torch.Tensor, wg: torch.Tensor, logits: torch.Tensor, *, stream=None) -> torch.Tensor:
    """logits = x . wg^T with f32 accumulation (bf16 or f32 output)."""
    lib = load_library()
    T, H = x.shape
    E = wg.shape[0]
    _need(x, "x", torch.bfloat16)
    _need(wg, "wg", torch.bfloat16, (E, H))
    if logits.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("logits must be bf16 or f32")
    _need(logits, "logits", logits.dtype, (T, E))
    _check(
        lib.lmoe_router_gate(_ptr(x), _ptr(wg), T, H, E, _ptr(logits),
                             int(logits.dtype == torch.float32), _stream(stream)),
        "lmoe_router_gate",
    )
    return logits


def router_topk(
    logits: torch.Tensor,
    top_k: int,
    *,
    scoring: str = "softmax",
    bias: torch.Tensor | None = None,
    logit_bias: torch.Tensor | None = None,
    num_expert_group: int = 1,
    topk_group: int = 1,
    renormalize: bool = True,
    routed_scaling_factor: float = 1.0,
    n_shared: int = 0,
    w_bf16: torch.Tensor | None = None,
    ids: torch.Tensor | None = None,
    w_f32: torch.Tensor | None = None,
    stream=None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """Select top_k experts per token (bias: e_score_correction_bias, for
    selection only; logit_bias: added to the logits before scoring).
    Returns (w_bf16 [T,k+S], ids int32 [T,k+S], w_f32) with S = n_shared
    columns of the pinned shared-expert suffix (ids E, E+1, ..., weight 1)
    after the routed ones."""
    lib = load_library()
    if logits.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("logits must be bf16 or f32")
    _need(logits, "logits", logits.dtype)
    T, E = logits.shape
    if scoring == "softmax":
        mode = LMOE_SCORING_SOFTMAX
    elif scoring == "sigmoid":
        mode = LMOE_SCORING_SIGMOID
    else:
        raise ValueError(f"unsupported scoring function {scoring!r}")
    _check_biases(bias, logit_bias, E)
    dev = logits.device
    kw = int(top_k) + int(n_shared)
    if w_bf16 is None:
        w_bf16 = torch.empty((T, kw), dtype=torch.bfloat16, device=dev)
    if ids is None:
        ids = torch.empty((T, kw), dtype=torch.int32, device=dev)
    _need(w_bf16, "topk_weights", torch.bfloat16, (T, kw))
    _need(ids, "topk_ids", torch.int32, (T, kw))
    if w_f32 is not None:
        _need(w_f32, "w_f32", torch.float32, (T, kw))
    _check(
        lib.lmoe_router_topk(
            _ptr(logits), int(logits.dtype == torch.float32), T, E, int(top_k), int(n_shared), mode,
            _ptr(bias), _ptr(logit_bias), int(num_expert_group or 1), int(topk_group or 1),
            int(bool(renormalize)), float(routed_scaling_factor),
            _ptr(w_f32), _ptr(w_bf16), _ptr(ids), _stream(stream),
        ),
        "lmoe_router_topk",
    )
    return w_bf16, ids, w_f32


def router_topk_permute(
    logits: torch.Tensor,
    top_k: int,
    perm: "Permutation",
    *,
    log2phy: torch.Tensor | None = None,
    skip_unmapped: bool = False,
    block_m: int | None = None,
    scoring: str = "softmax",
    bias: torch.Tensor | None = None,
    logit_bias: torch.Tensor | None = None,
    num_expert_group: int = 1,
    topk_group: int = 1,
    renormalize: bool = True,
    routed_scaling_factor: float = 1.0,
    n_shared: int = 0,
    w_bf16: torch.Tensor | None = None,
    ids: torch.Tensor | None = None,
    w_f32: torch.Tensor | None = None,
    second: "tuple[Permutation, torch.Tensor] | None" = None,
    stream=None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """router_topk then permute into perm, in one launch when the shape allows
    it (T <= 16, E <= 256); otherwise the two launches.  For a slot table
    (log2phy) that is final before the router runs.  second = (permutation,
    table) of a later pass over the same ids (the decode overflow stage
    buffer; perm is then built with skip_unmapped): built after perm in skip
    mode 2 on perm.row_idx, in the same launch as perm when the selection
    runs on its own (permute_two_tables)."""
    lib = load_library()
    if logits.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("logits must be bf16 or f32")
    _need(logits, "logits", logits.dtype)
    T, E = logits.shape
    mode = {"softmax": LMOE_SCORING_SOFTMAX, "sigmoid": LMOE_SCORING_SIGMOID}.get(scoring)
    if mode is None:
        raise ValueError(f"unsupported scoring function {scoring!r}")
    _check_biases(bias, logit_bias, E)
    dev = logits.device
    kw = int(top_k) + int(n_shared)
    if w_bf16 is None:
        w_bf16 = torch.empty((T, kw), dtype=torch.bfloat16, device=dev)
    if ids is None:
        ids = torch.empty((T, kw), dtype=torch.int32, device=dev)
    _need(w_bf16, "topk_weights", torch.bfloat16, (T, kw))
    _need(ids, "topk_ids", torch.int32, (T, kw))
    if w_f32 is not None:
        _need(w_f32, "w_f32", torch.float32, (T, kw))
    if T * kw != perm.n_pairs:
        raise ValueError(f"permutation buffers sized for {perm.n_pairs} pairs, got {T * kw}")
    n_table = 0
    if log2phy is not None:
        _need(log2phy, "log2phy", torch.int32)
        n_table = int(log2phy.numel())
    if second is not None and (log2phy is None or not skip_unmapped):
        raise ValueError("a second pass needs the first pass's table with skip_unmapped")
    bm = MFMA_BLOCK_M if block_m is None else int(block_m)
    status = lib.lmoe_router_topk_permute(
        _ptr(logits), int(logits.dtype == torch.float32), T, E, int(top_k), int(n_shared), mode,
        _ptr(bias), _ptr(logit_bias), int(num_expert_group or 1), int(topk_group or 1),
        int(bool(renormalize)), float(routed_scaling_factor),
        _ptr(w_f32), _ptr(w_bf16), _ptr(ids),
        _ptr(log2phy), n_table, perm.n_slots, int(bool(skip_unmapped)), bm,
        _ptr(perm.counts), _ptr(perm.offsets), _ptr(perm.sorted_pairs), _ptr(perm.row_idx),
        _ptr(perm.active), _ptr(perm.tile_off), _ptr(perm.meta), _stream(stream),
    )
    if status == LMOE_ERR_SHAPE:
        router_topk(logits, top_k, scoring=scoring, bias=bias, logit_bias=logit_bias,
                    num_expert_group=num_expert_group,
                    topk_group=topk_group, renormalize=renormalize,
                    routed_scaling_factor=routed_scaling_factor, n_shared=n_shared, w_bf16=w_bf16, ids=ids,
                    w_f32=w_f32, stream=stream)
        if second is not None:
            permute_two_tables(ids, perm, log2phy, second[0], second[1], block_m=bm, stream=stream)
        else:
            permute(ids, perm, log2phy=log2phy, skip_unmapped=skip_unmapped, block_m=bm, stream=stream)
        return w_bf16, ids, w_f32
    _check(status, "lmoe_router_topk_permute")
    perm.builds += 1
    perm.block_m = bm
    if second is not None:
        permute(ids, second[0], log2phy=second[1], keep_rows=True, row_idx=perm.row_idx, block_m=bm,
                stream=stream)
    return w_bf16, ids, w_f32


def router_gate_topk_permute(
    x: torch.Tensor,
    wg: torch.Tensor,
    logits: torch.Tensor,
    top_k: int,
    perm: "Permutation",
    *,
    log2phy: torch.Tensor | None = None,
    skip_unmapped: bool = False,
    block_m: int | None = None,
    scoring: str = "softmax",
    bias: torch.Tensor | None = None,
    logit_bias: torch.Tensor | None = None,
    num_expert_group: int = 1,
    topk_group: int = 1,
    renormalize: bool = True,
    routed_scaling_factor: float = 1.0,
    n_shared: int = 0,
    w_bf16: torch.Tensor | None = None,
    ids: torch.Tensor | None = None,
    w_f32: torch.Tensor | None = None,
    stream=None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """router_gate, router_topk and permute into perm in one launch when the
    shape allows it (T <= 16, E <= 256, H <= 8192); otherwise router_gate and
    router_topk_permute.  Same outputs bit for bit; logits is written too.
    Uses perm.sync (arrival count and tagged logit words): calls that may run concurrently
    need separate Permutation buffers."""
    lib = load_library()
    T, H = x.shape
    E = wg.shape[0]
    _need(x, "x", torch.bfloat16)
    _need(wg, "wg", torch.bfloat16, (E, H))
    if logits.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("logits must be bf16 or f32")
    _need(logits, "logits", logits.dtype, (T, E))
    mode = {"softmax": LMOE_SCORING_SOFTMAX, "sigmoid": LMOE_SCORING_SIGMOID}.get(scoring)
    if mode is None:
        raise ValueError(f"unsupported scoring function {scoring!r}")
    _check_biases(bias, logit_bias, E)
    dev = x.device
    kw = int(top_k) + int(n_shared)
    if w_bf16 is None:
        w_bf16 = torch.empty((T, kw), dtype=torch.bfloat16, device=dev)
    if ids is None:
        ids = torch.empty((T, kw), dtype=torch.int32, device=dev)
    _need(w_bf16, "topk_weights", torch.bfloat16, (T, kw))
    _need(ids, "topk_ids", torch.int32, (T, kw))
    if w_f32 is not None:
        _need(w_f32, "w_f32", torch.float32, (T, kw))
    if T * kw != perm.n_pairs:
        raise ValueError(f"permutation buffers sized for {perm.n_pairs} pairs, got {T * kw}")
    n_table = 0
    if log2phy is not None:
        _need(log2phy, "log2phy", torch.int32)
        n_table = int(log2phy.numel())
    bm = MFMA_BLOCK_M if block_m is None else int(block_m)
    status = lib.lmoe_router_gate_topk_permute(
        _ptr(x), _ptr(wg), T, H, E, _ptr(logits), int(logits.dtype == torch.float32), int(top_k),
        int(n_shared), mode, _ptr(bias), _ptr(logit_bias), int(num_expert_group or 1),
        int(topk_group or 1),
        int(bool(renormalize)), float(routed_scaling_factor),
        _ptr(w_f32), _ptr(w_bf16), _ptr(ids),
        _ptr(log2phy), n_table, perm.n_slots, int(bool(skip_unmapped)), bm,
        _ptr(perm.counts), _ptr(perm.offsets), _ptr(perm.sorted_pairs), _ptr(perm.row_idx),
        _ptr(perm.active), _ptr(perm.tile_off), _ptr(perm.meta), _ptr(perm.sync), _stream(stream),
    )
    if status == LMOE_ERR_SHAPE:
        router_gate(x, wg, logits, stream=stream)
        return router_topk_permute(
            logits, top_k, perm, log2phy=log2phy, skip_unmapped=skip_unmapped, block_m=bm,
            scoring=scoring, bias=bias, logit_bias=logit_bias, num_expert_group=num_expert_group,
            topk_group=topk_group,
            renormalize=renormalize, routed_scaling_factor=routed_scaling_factor, n_shared=n_shared,
            w_bf16=w_bf16, ids=ids, w_f32=w_f32, stream=stream,
        )
    _check(status, "lmoe_router_gate_topk_permute")
    perm.builds += 1
    perm.block_m = bm
    return w_bf16, ids, w_f32


def router_gate_topk_pairs(
    x: torch.Tensor,
    wg: torch.Tensor,
    logits: torch.Tensor,
    top_k: int,
    perm: "Permutation",
    *,
    log2phy: torch.Tensor | None = None,
    skip_unmapped: bool = False,
    scoring: str = "softmax",
    bias: torch.Tensor | None = None,
    logit_bias: torch.Tensor | None = None,
    num_expert_group: int = 1,
    topk_group: int = 1,
    renormalize: bool = True,
    routed_scaling_factor: float = 1.0,
    n_shared: int = 0,
    w_bf16: torch.Tensor | None = None,
    ids: torch.Tensor | None = None,
    w_f32: torch.Tensor | None = None,
    stream=None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """One token: router_gate_topk_permute's gate and selection (the same
    bits) with perm in the one-token pair order (lmoe_router_gate_topk_pairs:
    the placed pairs at positions 0, 1, ... in pair order, active[pos] their
    slots; counts, offsets and tile_off are not written), the form
    fused_moe_decode(distinct_slots=True) reads.  Falls back to
    router_gate_topk_permute (the sorted permutation, which that call reads
    the same way) where the one launch does not take the shape."""
    lib = load_library()
    T, H = x.shape
    E = wg.shape[0]
    if T != 1:
        raise ValueError("the pair-order router serves one token")
    _need(x, "x", torch.bfloat16)
    _need(wg, "wg", torch.bfloat16, (E, H))
    if logits.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("logits must be bf16 or f32")
    _need(logits, "logits", logits.dtype, (T, E))
    mode = {"softmax": LMOE_SCORING_SOFTMAX, "sigmoid": LMOE_SCORING_SIGMOID}.get(scoring)
    if mode is None:
        raise ValueError(f"unsupported scoring function {scoring!r}")
    _check_biases(bias, logit_bias, E)
    dev = x.device
    kw = int(top_k) + int(n_shared)
    if w_bf16 is None:
        w_bf16 = torch.empty((T, kw), dtype=torch.bfloat16, device=dev)
    if ids is None:
        ids = torch.empty((T, kw), dtype=torch.int32, device=dev)
    _need(w_bf16, "topk_weights", torch.bfloat16, (T, kw))
    _need(ids, "topk_ids", torch.int32, (T, kw))
    if w_f32 is not None:
        _need(w_f32, "w_f32", torch.float32, (T, kw))
    if kw != perm.n_pairs:
        raise ValueError(f"permutation buffers sized for {perm.n_pairs} pairs, got {kw}")
    n_table = 0
    if log2phy is not None:
        _need(log2phy, "log2phy", torch.int32)
        n_table = int(log2phy.numel())
    status = lib.lmoe_router_gate_topk_pairs(
        _ptr(x), _ptr(wg), H, E, _ptr(logits), int(logits.dtype == torch.float32), int(top_k),
        int(n_shared), mode, _ptr(bias), _ptr(logit_bias), int(num_expert_group or 1), int(topk_group or 1),
        int(bool(renormalize)), float(routed_scaling_factor), _ptr(w_f32), _ptr(w_bf16), _ptr(ids),
        _ptr(log2phy), n_table, perm.n_slots, int(bool(skip_unmapped)),
        _ptr(perm.sorted_pairs), _ptr(perm.row_idx), _ptr(perm.active), _ptr(perm.meta), _ptr(perm.sync),
        _stream(stream),
    )
    if status == LMOE_ERR_SHAPE:
        return router_gate_topk_permute(
            x, wg, logits, top_k, perm, log2phy=log2phy, skip_unmapped=skip_unmapped, scoring=scoring,
            bias=bias, logit_bias=logit_bias, num_expert_group=num_expert_group, topk_group=topk_group,
            renormalize=renormalize, routed_scaling_factor=routed_scaling_factor, n_shared=n_shared,
            w_bf16=w_bf16, ids=ids, w_f32=w_f32, stream=stream,
        )
    _check(status, "lmoe_router_gate_topk_pairs")
    perm.builds += 1
    return w_bf16, ids, w_f32


# ---------------------------------------------------------------------------
# permutation
# ---------------------------------------------------------------------------
_CU_COUNT: dict[int, int] = {}


def _cu_count(device) -> int:
    idx = torch.device(device).index
    idx = torch.cuda.current_device() if idx is None else idx
    if idx not in _CU_COUNT:
        _CU_COUNT[idx] = int(torch.cuda.get_device_properties(idx).multi_processor_count)
    return _CU_COUNT[idx]


_OFFSET32_LIMIT = 2**31 - 1


def prefill_block_m(n_experts: int, hidden: int, intermediate: int, device="cuda",
                    cu_count: int | None = None, n_pairs: int | None = None) -> int:
    """Row-tile height for the prefill GEMMs of one pass over n_experts slots
    (the block_m to build the permutation with).

    320 selects the kernel with one workgroup per CU: a slot of up to 320
    pairs is one row tile, and each CU runs an equal number of units (a row
    tile's 128 gate-up columns).  With n_experts * ceil(I / 128) units it
    takes one round when they fit on the CUs, and balanced rounds when there
    are many.  Just past one round (a 43-slot wave on 256 CUs: 258 units) the
    last units would run alone, and the 256-row tile grid finishes first
    (measured 136 + 64 us against 166 + 74 us for gate_up + down); there 256
    is returned.  Needs hidden % 64 == 0 (else 256), and activation operands
    below 2^31 elements (the 320-row kernel's offsets are 32-bit: n_pairs
    rows of max(hidden, intermediate) bounds both GEMMs; else 256, whose
    offsets are 64-bit).  cu_count defaults to the device's."""
    if hidden % 64 != 0:
        return MFMA_BLOCK_M
    if n_pairs is not None and int(n_pairs) * max(int(hidden), int(intermediate)) > _OFFSET32_LIMIT:
        return MFMA_BLOCK_M
    cus = int(cu_count) if cu_count is not None else _cu_count(device)
    units = int(n_experts) * ((int(intermediate) + 127) // 128)
    if cus < units <= cus + cus // 4:
        return MFMA_BLOCK_M
    return PART_BLOCK_M


@dataclass
class Permutation:
    """Device outputs of lmoe_permute for one (n_pairs, n_slots) shape.

    Buffers are allocated once and reused (fixed addresses, graph safe).
    """

    n_pairs: int
    n_slots: int
    counts: torch.Tensor        # [P] i32 histogram (expert_tokens, count type)
    offsets: torch.Tensor       # [P+1] i32
    sorted_pairs: torch.Tensor  # [N] i32 flat pair at each sorted position
    row_idx: torch.Tensor       # [N] i32 sorted position of each pair (expanded_row_idx) or -1
    active: torch.Tensor        # [P] i32 slots with count > 0: heavy slots first (by count), then ascending
    tile_off: torch.Tensor      # [P+1] i32 MFMA tile prefix
    meta: torch.Tensor          # [4] i32
    workspace: torch.Tensor     # int8 scratch for the multi-block path
    sync: torch.Tensor          # [ROUTER_SYNC_WORDS] i32: the one-launch router's arrival count (kept at 0) and tagged logit words
    block_m: int = MFMA_BLOCK_M  # tile height tile_off was last built with
    builds: int = 0  # lmoe_permute builds issued on these buffers

    @classmethod
    def allocate(cls, n_pairs: int, n_slots: int, device) -> "Permutation":
        lib = load_library()
        ws = int(lib.lmoe_permute_workspace_bytes(int(n_pairs), int(n_slots)))
        i32 = dict(dtype=torch.int32, device=device)
        return cls(
            n_pairs=int(n_pairs),
            n_slots=int(n_slots),
            counts=torch.zeros(n_slots, **i32),
            offsets=torch.zeros(n_slots + 1, **i32),
            sorted_pairs=torch.zeros(max(1, n_pairs), **i32),
            row_idx=torch.zeros(max(1, n_pairs), **i32),
            active=torch.zeros(n_slots, **i32),
            tile_off=torch.zeros(n_slots + 1, **i32),
            meta=torch.zeros(META_COUNT, **i32),
            workspace=torch.empty(max(ws, 1), dtype=torch.int8, device=device),
            sync=torch.zeros(ROUTER_SYNC_WORDS, **i32),
        )


def permute(
    ids: torch.Tensor,
    perm: Permutation,
    *,
    log2phy: torch.Tensor | None = None,
    skip_unmapped: bool = False,
    keep_rows: bool = False,
    row_idx: torch.Tensor | None = None,
    table_len: int | None = None,
    block_m: int = MFMA_BLOCK_M,
    stream=None,
) -> Permutation:
    """Remap ids through log2phy and stable-sort the flat pairs by slot.

    table_len (<= log2phy.numel()) limits the ids the table covers; with
    skip_unmapped, ids past it are left to another pass.  keep_rows (a later
    pass of a multi-pass layer; implies skip_unmapped) leaves the row_idx of
    the pairs this pass does not place as an earlier pass wrote it, so the
    layer's single combine masks exactly the pairs no pass placed.  row_idx
    replaces perm.row_idx as the output (the first pass's permutation when
    the passes build separate permutations)."""
    lib = load_library()
    _need(ids, "topk_ids", torch.int32)
    n = int(ids.numel())
    if n != perm.n_pairs:
        raise ValueError(f"permutation buffers sized for {perm.n_pairs} pairs, got {n}")
    rows = perm.row_idx if row_idx is None else row_idx
    if row_idx is not None:
        _need(row_idx, "row_idx", torch.int32)
        if int(row_idx.numel()) < max(1, n):
            raise ValueError("row_idx has fewer entries than pairs")
    mode = SKIP_KEEP_ROWS if keep_rows else int(bool(skip_unmapped))
    n_table = 0
    if log2phy is not None:
        _need(log2phy, "log2phy", torch.int32)
        n_table = int(log2phy.numel()) if table_len is None else min(int(table_len), int(log2phy.numel()))
    _check(
        lib.lmoe_permute(
            _ptr(ids), n, _ptr(log2phy), n_table,
            perm.n_slots, mode, int(block_m),
            _ptr(perm.counts), _ptr(perm.offsets), _ptr(perm.sorted_pairs),
            _ptr(rows), _ptr(perm.active), _ptr(perm.tile_off), _ptr(perm.meta),
            _ptr(perm.workspace), int(perm.workspace.numel()), _stream(stream),
        ),
        "lmoe_permute",
    )
    perm.block_m = int(block_m)
    perm.builds += 1
    return perm


def permute_two_tables(
    ids: torch.Tensor,
    perm: Permutation,
    log2phy: torch.Tensor,
    second: Permutation,
    second_log2phy: torch.Tensor,
    *,
    block_m: int = MFMA_BLOCK_M,
    stream=None,
) -> tuple[Permutation, Permutation]:
    """permute(ids, perm, log2phy, skip_unmapped=True) followed by
    permute(ids, second, second_log2phy, keep_rows=True, row_idx=perm.row_idx)
    (the bank and overflow-table builds of a decode overflow layer), in one
    launch up to PERMUTE_TWO_MAX_PAIRS pairs, as the two calls past that."""
    lib = load_library()
    _need(ids, "topk_ids", torch.int32)
    _need(log2phy, "log2phy", torch.int32)
    _need(second_log2phy, "second_log2phy", torch.int32)
    n = int(ids.numel())
    if n != perm.n_pairs or n != second.n_pairs:
        raise ValueError(f"permutation buffers sized for {perm.n_pairs} / {second.n_pairs} pairs, got {n}")
    if n > PERMUTE_TWO_MAX_PAIRS:
        permute(ids, perm, log2phy=log2phy, skip_unmapped=True, block_m=block_m, stream=stream)
        permute(ids, second, log2phy=second_log2phy, keep_rows=True, row_idx=perm.row_idx, block_m=block_m,
                stream=stream)
        return perm, second
    _check(
        lib.lmoe_permute_two_tables(
            _ptr(ids), n, int(block_m), _ptr(perm.row_idx),
            _ptr(log2phy), int(log2phy.numel()), perm.n_slots, _ptr(perm.counts), _ptr(perm.offsets),
            _ptr(perm.sorted_pairs), _ptr(perm.active), _ptr(perm.tile_off), _ptr(perm.meta),
            _ptr(second_log2phy), int(second_log2phy.numel()), second.n_slots, _ptr(second.counts),
            _ptr(second.offsets), _ptr(second.sorted_pairs), _ptr(second.active), _ptr(second.tile_off),
            _ptr(second.meta), _stream(stream),
        ),
        "lmoe_permute_two_tables",
    )
    for p in (perm, second):
        p.block_m = int(block_m)
        p.builds += 1
    return perm, second


def gather_rows(x: torch.Tensor, top_k: int, perm: Permutation, out: torch.Tensor | None = None,
                *, stream=None) -> torch.Tensor:
    """expanded_x: out[pos] = x[sorted_pairs[pos] // top_k]."""
    lib = load_library()
    _need(x, "x", torch.bfloat16)
    H = x.shape[1]
    if out is None:
        out = torch.empty((perm.n_pairs, H), dtype=torch.bfloat16, device=x.device)
    _need(out, "x_sorted", torch.bfloat16, (perm.n_pairs, H))
    _check(
        lib.lmoe_gather_rows(_ptr(x), H, int(top_k), _ptr(perm.sorted_pairs), _ptr(perm.meta),
                             perm.n_pairs, _ptr(out), _stream(stream)),
        "lmoe_gather_rows",
    )
    return out


# ---------------------------------------------------------------------------
# expert MLP and combine
# ---------------------------------------------------------------------------
def _check_bank(w13: torch.Tensor, w2: torch.Tensor, H: int) -> tuple[int, int]:
    _need(w13, "w13_slots", torch.bfloat16)
    _need(w2, "w2_slots", torch.bfloat16)
    if w13.dim() != 3 or w2.dim() != 3:
        raise ValueError("slot banks must be [P, 2I, H] and [P, H, I]")
    P, two_i, h = w13.shape
    if h != H or two_i % 2 != 0:
        raise ValueError(f"w13_slots shape {tuple(w13.shape)} does not match H={H}")
    I = two_i // 2
    if tuple(w2.shape) != (P, H, I):
        raise ValueError(f"w2_slots shape {tuple(w2.shape)} != {(P, H, I)}")
    return P, I


def grouped_mlp(
    x: torch.Tensor,
    top_k: int,
    w13_slots: torch.Tensor,
    w2_slots: torch.Tensor,
    perm: Permutation,
    act: torch.Tensor,
    y: torch.Tensor,
    *,
    path: int = LMOE_PATH_AUTO,
    stream=None,
) -> torch.Tensor:
    """y[pair] = W2_s . (silu(W13_s[:I] x) * W13_s[I:] x) for the placed pairs."""
    lib = load_library()
    _need(x, "x", torch.bfloat16)
    T, H = x.shape
    P, I = _check_bank(w13_slots, w2_slots, H)
    if P != perm.n_slots:
        raise ValueError(f"slot bank has {P} slots, permutation {perm.n_slots}")
    if perm.n_pairs != T * top_k:
        raise ValueError("permutation does not match T * top_k pairs")
    _need(act, "act", torch.bfloat16, (perm.n_pairs, I))
    _need(y, "y", torch.bfloat16, (perm.n_pairs, H))
    _check(
        lib.lmoe_grouped_mlp(
            _ptr(x), T, H, I, int(top_k), _ptr(w13_slots), _ptr(w2_slots), P,
            _ptr(perm.offsets), _ptr(perm.sorted_pairs), _ptr(perm.active), _ptr(perm.tile_off),
            _ptr(perm.meta), perm.n_pairs, perm.block_m, int(path), _ptr(act), _ptr(y),
            _stream(stream),
        ),
        "lmoe_grouped_mlp",
    )
    return y


def gateup_silu(x: torch.Tensor, top_k: int, w13_slots: torch.Tensor, perm: Permutation, act: torch.Tensor,
                *, path: int = LMOE_PATH_AUTO, stream=None) -> torch.Tensor:
    """act[pos] = silu(W13_s[:I] x) * (W13_s[I:] x) for the placed pairs (GMM1 + SwiGLU)."""
    lib = load_library()
    _need(x, "x", torch.bfloat16)
    _need(w13_slots, "w13_slots", torch.bfloat16)
    T, H = x.shape
    P, two_i, h = w13_slots.shape
    if h != H or P != perm.n_slots:
        raise ValueError("w13_slots does not match x or the permutation")
    I = two_i // 2
    _need(act, "act", torch.bfloat16, (perm.n_pairs, I))
    _check(
        lib.lmoe_gateup_silu(
            _ptr(x), T, H, I, int(top_k), _ptr(w13_slots), P, _ptr(perm.offsets), _ptr(perm.sorted_pairs),
            _ptr(perm.active), _ptr(perm.tile_off), _ptr(perm.meta), perm.n_pairs, perm.block_m, int(path),
            _ptr(act), _stream(stream),
        ),
        "lmoe_gateup_silu",
    )
    return act


def down(act: torch.Tensor, w2_slots: torch.Tensor, perm: Permutation, y: torch.Tensor,
         *, path: int = LMOE_PATH_AUTO, stream=None) -> torch.Tensor:
    """y[pair] = W2_s act[pos] for the placed pairs (GMM2)."""
    lib = load_library()
    _need(w2_slots, "w2_slots", torch.bfloat16)
    P, H, I = w2_slots.shape
    if P != perm.n_slots:
        raise ValueError("w2_slots does not match the permutation")
    _need(act, "act", torch.bfloat16, (perm.n_pairs, I))
    _need(y, "y", torch.bfloat16, (perm.n_pairs, H))
    _check(
        lib.lmoe_down(
            _ptr(act), H, I, _ptr(w2_slots), P, _ptr(perm.offsets), _ptr(perm.sorted_pairs), _ptr(perm.active),
            _ptr(perm.tile_off), _ptr(perm.meta), perm.n_pairs, perm.block_m, int(path), _ptr(y), _stream(stream),
        ),
        "lmoe_down",
    )
    return y


def decode_mlp_two_passes(
    x: torch.Tensor,
    top_k: int,
    w13_a: torch.Tensor,
    w2_a: torch.Tensor,
    perm_a: Permutation,
    w13_b: torch.Tensor,
    w2_b: torch.Tensor,
    perm_b: Permutation,
    act: torch.Tensor,
    y: torch.Tensor,
    *,
    stream=None,
) -> torch.Tensor:
    """The decode GEMVs of both passes of an overflow layer (bank a, overflow
    stage buffer b, each with its own permutation over the same ids) in one
    gate_up and one down launch; y[pair] as grouped_mlp(path=GEMV) writes it
    for either pass.  The tables must map disjoint experts.  Rows up to
    TWO_PASS_MAX_COLS columns (H and I): past that, run the passes one by
    one (grouped_mlp)."""
    lib = load_library()
    _need(x, "x", torch.bfloat16)
    T, H = x.shape
    Pa, I = _check_bank(w13_a, w2_a, H)
    Pb, Ib = _check_bank(w13_b, w2_b, H)
    if Ib != I:
        raise ValueError("the two passes' banks have different intermediate sizes")
    if H > TWO_PASS_MAX_COLS or I > TWO_PASS_MAX_COLS:
        raise ValueError(f"rows past {TWO_PASS_MAX_COLS} columns: run the passes one by one")
    if Pa != perm_a.n_slots or Pb != perm_b.n_slots:
        raise ValueError("a slot bank does not match its permutation")
    if perm_a.n_pairs != T * top_k or perm_b.n_pairs != T * top_k:
        raise ValueError("permutations do not match T * top_k pairs")
    _need(act, "act", torch.bfloat16, (perm_a.n_pairs, I))
    _need(y, "y", torch.bfloat16, (perm_a.n_pairs, H))
    _check(
        lib.lmoe_decode_mlp_two_passes(
            _ptr(x), T, H, I, int(top_k), _ptr(w13_a), _ptr(w2_a), Pa, _ptr(perm_a.offsets),
            _ptr(perm_a.sorted_pairs), _ptr(perm_a.active), _ptr(perm_a.meta), _ptr(w13_b), _ptr(w2_b), Pb,
            _ptr(perm_b.offsets), _ptr(perm_b.sorted_pairs), _ptr(perm_b.active), perm_a.n_pairs, _ptr(act),
            _ptr(y), _stream(stream),
        ),
        "lmoe_decode_mlp_two_passes",
    )
    return y


def combine(
    y: torch.Tensor,
    topk_weights: torch.Tensor,
    out: torch.Tensor,
    *,
    row_mask: torch.Tensor | None = None,
    add: torch.Tensor | None = None,
    stream=None,
) -> torch.Tensor:
    """out[t] = add[t] + sum_j w[t,j] * y[t*k+j] (pairs with row_mask < 0 skipped)."""
    lib = load_library()
    _need(topk_weights, "topk_weights", torch.bfloat16)
    T, k = topk_weights.shape
    _need(y, "y", torch.bfloat16)
    H = y.shape[1]
    if y.shape[0] < T * k:
        raise ValueError("y has fewer rows than pairs")
    _need(out, "out", torch.bfloat16, (T, H))
    if row_mask is not None:
        _need(row_mask, "row_mask", torch.int32)
    if add is not None:
        _need(add, "add", torch.bfloat16, (T, H))
    _check(
        lib.lmoe_combine(_ptr(y), _ptr(row_mask), _ptr(topk_weights), T, k, H, _ptr(add),
                         _ptr(out), _stream(stream)),
        "lmoe_combine",
    )
    return out


def fused_moe_decode(
    x: torch.Tensor,
    topk_weights: torch.Tensor,
    w13_slots: torch.Tensor,
    w2_slots: torch.Tensor,
    perm: Permutation,
    act: torch.Tensor,
    out: torch.Tensor,
    *,
    add: torch.Tensor | None = None,
    y: torch.Tensor | None = None,
    distinct_slots: bool = False,
    stream=None,
) -> torch.Tensor:
    """Decode layer body: gate_up GEMV, then down GEMV fused with the combine
    (up to 16 pairs, or no y), or with a [T*k, H] bf16 workspace y and more
    pairs the down GEMV per (row block, slot) into y and the combine; same out
    either way.  distinct_slots: the caller promises that no slot serves two
    pairs of one token (router-fed ids through a slot table); with one token
    it selects the faster one-pair-per-slot kernels."""
    lib = load_library()
    _need(x, "x", torch.bfloat16)
    T, H = x.shape
    _need(topk_weights, "topk_weights", torch.bfloat16)
    k = topk_weights.shape[1]
    P, I = _check_bank(w13_slots, w2_slots, H)
    if perm.n_pairs != T * k or perm.n_slots != P:
        raise ValueError("permutation does not match the batch or the slot bank")
    if T * k > FUSED_DECODE_MAX_PAIRS:
        raise ValueError(f"fused decode supports at most {FUSED_DECODE_MAX_PAIRS} pairs")
    _need(act, "act", torch.bfloat16, (perm.n_pairs, I))
    _need(out, "out", torch.bfloat16, (T, H))
    if add is not None:
        _need(add, "add", torch.bfloat16, (T, H))
    if y is not None:
        _need(y, "y", torch.bfloat16, (perm.n_pairs, H))
    _check(
        lib.lmoe_fused_moe_decode(
            _ptr(x), T, H, I, k, _ptr(w13_slots), _ptr(w2_slots), P, _ptr(topk_weights),
            _ptr(perm.offsets), _ptr(perm.sorted_pairs), _ptr(perm.row_idx), _ptr(perm.active),
            _ptr(perm.meta), _ptr(add), _ptr(act), _ptr(y), _ptr(out), int(bool(distinct_slots)),
            _stream(stream),
        ),
        "lmoe_fused_moe_decode",
    )
    return out


NOALLOC_SCRATCH_BYTES = 8 << 20  # LMOE_NOALLOC_SCRATCH_BYTES


def fused_moe_decode_noalloc(
    x: torch.Tensor,
    topk_weights: torch.Tensor,
    w13_slots: torch.Tensor,
    w2_slots: torch.Tensor,
    perm: Permutation,
    out: torch.Tensor,
    *,
    add: torch.Tensor | None = None,
    distinct_slots: bool = False,
    stream=None,
) -> torch.Tensor:
    """fused_moe_decode with act / y in the library's per-GPU scratch array
    (nothing is allocated; calls that overlap on one GPU race)."""
    lib = load_library()
    _need(x, "x", torch.bfloat16)
    T, H = x.shape
    _need(topk_weights, "topk_weights", torch.bfloat16)
    k = topk_weights.shape[1]
    P, I = _check_bank(w13_slots, w2_slots, H)
    if perm.n_pairs != T * k or perm.n_slots != P:
        raise ValueError("permutation does not match the batch or the slot bank")
    _need(out, "out", torch.bfloat16, (T, H))
    if add is not None:
        _need(add, "add", torch.bfloat16, (T, H))
    _check(
        lib.lmoe_fused_moe_decode_noalloc(
            _ptr(x), T, H, I, k, _ptr(w13_slots), _ptr(w2_slots), P, _ptr(topk_weights),
            _ptr(perm.offsets), _ptr(perm.sorted_pairs), _ptr(perm.row_idx), _ptr(perm.active),
            _ptr(perm.meta), _ptr(add), _ptr(out), int(bool(distinct_slots)), _stream(stream),
        ),
        "lmoe_fused_moe_decode_noalloc",
    )
    return out


def down_combine(
    act: torch.Tensor,
    topk_weights: torch.Tensor,
    w2_slots: torch.Tensor,
    perm: Permutation,
    out: torch.Tensor,
    *,
    add: torch.Tensor | None = None,
    stream=None,
) -> torch.Tensor:
    """Second half of fused_moe_decode: down GEMV fused with the combine."""
    lib = load_library()
    _need(topk_weights, "topk_weights", torch.bfloat16)
    T, k = topk_weights.shape
    _need(w2_slots, "w2_slots", torch.bfloat16)
    P, H, I = w2_slots.shape
    if perm.n_pairs != T * k or perm.n_slots != P:
        raise ValueError("permutation does not match the batch or the slot bank")
    _need(act, "act", torch.bfloat16, (perm.n_pairs, I))
    _need(out, "out", torch.bfloat16, (T, H))
    if add is not None:
        _need(add, "add", torch.bfloat16, (T, H))
    _check(
        lib.lmoe_down_combine(
            _ptr(act), T, H, I, k, _ptr(w2_slots), P, _ptr(topk_weights), _ptr(perm.offsets),
            _ptr(perm.row_idx), _ptr(perm.active), _ptr(perm.meta), _ptr(add), _ptr(out), _stream(stream),
        ),
        "lmoe_down_combine",
    )
    return out


# ---------------------------------------------------------------------------
# staging
# ---------------------------------------------------------------------------
def _table_pairs(table_update):
    """(table, idx tuple, val tuple, fill) of a table_update argument."""
    table, idx, val = table_update[:3]
    fill = bool(table_update[3]) if len(table_update) > 3 else False
    return table, tuple(int(i) for i in idx), tuple(int(v) for v in val), fill


def stage_copy(
    copies: list[tuple[int, int, int]],
    transfer_stream: torch.cuda.Stream,
    *,
    wait_event: torch.cuda.Event | None = None,
    done_event: torch.cuda.Event | None = None,
    table_update: tuple | None = None,
) -> None:
    """Queue (dst_ptr, src_ptr, nbytes) copies on transfer_stream with one
    hipMemcpyAsync each (any host memory, pageable included).

    The stream first waits for wait_event (slot release) and done_event is
    recorded after the batch; both are torch events, ordered through torch so
    their lazily created handles stay valid.  table_update = (table,
    indices, values[, fill]) writes those int32 entries after the copies
    (fill: every other entry becomes -1), inside the same done_event."""
    lib = load_library()
    if wait_event is not None:
        transfer_stream.wait_event(wait_event)
    n = len(copies)
    dst = (ctypes.c_void_p * max(n, 1))(*[c[0] for c in copies])
    src = (ctypes.c_void_p * max(n, 1))(*[c[1] for c in copies])
    nbytes = (ctypes.c_size_t * max(n, 1))(*[c[2] for c in copies])
    _check(
        lib.lmoe_stage_copy(dst, src, nbytes, n, int(transfer_stream.cuda_stream), None, None),
        "lmoe_stage_copy",
    )
    if table_update is not None:
        table, idx, val, fill = _table_pairs(table_update)
        if fill:
            full = dict.fromkeys(range(int(table.numel())), -1)
            full.update(zip(idx, val))
            idx, val = tuple(full), tuple(full.values())
        table_update_entries(table, idx, val, stream=transfer_stream)
    if done_event is not None:
        done_event.record(transfer_stream)


def stage_gather(
    copies: list[tuple[int, int, int]],
    transfer_stream: torch.cuda.Stream,
    *,
    table_update: tuple | None = None,
) -> bool:
    """Queue (dst_ptr, src_ptr, nbytes) copies as gather-copy kernel launches
    on transfer_stream, with the table_update = (table, indices, values[,
    fill]) entries written by the same launch.  Sources must be page-locked
    host memory or device memory; the library checks every range and refuses
    (returns False, nothing queued) what the device cannot read or what is
    not 16-byte aligned, so the caller can take stage_copy."""
    lib = load_library()
    n = len(copies)
    dst = (ctypes.c_void_p * max(n, 1))(*[c[0] for c in copies])
    src = (ctypes.c_void_p * max(n, 1))(*[c[1] for c in copies])
    nbytes = (ctypes.c_size_t * max(n, 1))(*[c[2] for c in copies])
    table = None
    n_table = n_tab = fill = 0
    ia = va = None
    if table_update is not None:
        table, idx, val, fill_b = _table_pairs(table_update)
        _need(table, "table", torch.int32)
        n_table, n_tab, fill = int(table.numel()), len(idx), int(fill_b)
        ia = (ctypes.c_int32 * max(n_tab, 1))(*idx)
        va = (ctypes.c_int32 * max(n_tab, 1))(*val)
    status = lib.lmoe_stage_gather(dst, src, nbytes, n, _ptr(table), n_table, ia, va, n_tab, fill,
                                   int(transfer_stream.cuda_stream), None, None)
    if status in (LMOE_ERR_ARG, LMOE_ERR_SHAPE):
        return False
    _check(status, "lmoe_stage_gather")
    return True


def table_update_entries(table: torch.Tensor, idx, val, *, stream=None) -> None:
    """table[idx[i]] = val[i] (distinct int indices) with one small kernel
    whose arguments carry the pairs: no staging tensor, no copy."""
    lib = load_library()
    _need(table, "table", torch.int32)
    n = len(idx)
    if n != len(val):
        raise ValueError(f"indices and values differ in length: {n} != {len(val)}")
    if n == 0:
        return
    ia = (ctypes.c_int32 * n)(*[int(i) for i in idx])
    va = (ctypes.c_int32 * n)(*[int(v) for v in val])
    _check(lib.lmoe_table_update(_ptr(table), int(table.numel()), ia, va, n, _stream(stream)),
           "lmoe_table_update")


# ---------------------------------------------------------------------------
# device-side capacity waves (lmoe_wave_plan / lmoe_wave_stage)
# ---------------------------------------------------------------------------
WAVE_PLAN_MAX_EXPERTS = 1024
WAVE_PLAN_MAX_SLOTS = 1024
WAVE_PLAN_MAX_WAVES = 256


class WavePlan:
    """Device buffer of one layer shape's wave plan (fixed address, graph safe)."""

    HEADER = 4

    def __init__(self, n_routed: int, n_slots: int, max_waves: int, device) -> None:
        n = int(load_library().lmoe_wave_plan_bytes(int(n_routed), int(n_slots), int(max_waves)))
        if n < 0:
            raise ValueError(f"device wave plan supports <= {WAVE_PLAN_MAX_EXPERTS} experts, "
                             f"<= {WAVE_PLAN_MAX_SLOTS} slots and <= {WAVE_PLAN_MAX_WAVES} waves; got "
                             f"{n_routed}, {n_slots}, {max_waves}")
        self.n_routed, self.n_slots, self.max_waves = int(n_routed), int(n_slots), int(max_waves)
        self.buf = torch.zeros(n // 4, dtype=torch.int32, device=device)

    # host views (tests and evidence; each reads the device buffer)
    def to_host(self) -> dict:
        b = self.buf.cpu().tolist()
        E, W, P, h = self.n_routed, self.max_waves, self.n_slots, self.HEADER
        counts = b[h:h + E]
        wave_of = b[h + E:h + 2 * E]
        slot_of = b[h + 2 * E:h + 3 * E]
        size = b[h + 3 * E:h + 3 * E + W]
        members = b[h + 3 * E + W:]
        n_waves = b[0]
        waves = tuple(tuple(members[w * P:w * P + size[w]]) for w in range(max(n_waves, 0)))
        return {"n_waves": n_waves, "n_active": b[1], "invalid": b[2], "counts": counts, "wave_of": wave_of,
                "slot_of": slot_of, "size": size, "waves": waves}


def wave_plan(ids: torch.Tensor, plan: WavePlan, *, n_total: int | None = None, stream=None) -> WavePlan:
    lib = load_library()
    _need(ids, "topk_ids", torch.int32)
    n_total = plan.n_routed if n_total is None else int(n_total)
    _check(lib.lmoe_wave_plan(_ptr(ids), int(ids.numel()), plan.n_routed, n_total, plan.n_slots, plan.max_waves,
                              _ptr(plan.buf), _stream(stream)), "lmoe_wave_plan")
    return plan


def wave_stage(plan: WavePlan, wave: int, *, main_table: torch.Tensor, main_owner: torch.Tensor,
               main_w13: torch.Tensor,
               main_w2: torch.Tensor, main_slots: int, host_w13: torch.Tensor, host_w2: torch.Tensor,
               stage_w13: torch.Tensor, stage_w2: torch.Tensor, stage_table: torch.Tensor,
               n_pinned: int = 0, stream=None) -> None:
    """Copy wave `wave`'s experts into the stage buffer and write its table.
    host_w13 / host_w2 must be page-locked [n_routed, ...] blocks."""
    lib = load_library()
    for name, t in (("main_w13", main_w13), ("main_w2", main_w2), ("stage_w13", stage_w13),
                    ("stage_w2", stage_w2), ("host_w13", host_w13), ("host_w2", host_w2)):
        if t.dtype != torch.bfloat16 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous bf16 tensor")
    if not (host_w13.is_pinned() and host_w2.is_pinned()):
        raise ValueError("device wave staging reads the host store directly: it must be page-locked")
    if int(host_w13.shape[0]) < plan.n_routed or int(main_table.numel()) < plan.n_routed:
        raise ValueError("host store or main table does not cover the routed experts")
    if int(stage_w13.shape[0]) < plan.n_slots + int(n_pinned) or int(main_w13.shape[0]) < int(main_slots):
        raise ValueError("stage buffer or main bank is smaller than its slot count")
    _need(main_table, "main_table", torch.int32)
    _need(main_owner, "main_owner", torch.int32)
    if int(main_owner.numel()) < int(main_slots):
        raise ValueError("main_owner must hold one entry per main slot")
    _need(stage_table, "stage_table", torch.int32)
    b13 = int(host_w13[0].numel()) * 2
    b2 = int(host_w2[0].numel()) * 2
    if int(stage_w13[0].numel()) * 2 != b13 or int(stage_w2[0].numel()) * 2 != b2 or \
            int(main_w13[0].numel()) * 2 != b13 or int(main_w2[0].numel()) * 2 != b2:
        raise ValueError("expert row sizes differ between host store, main bank and stage buffer")
    _check(lib.lmoe_wave_stage(
        _ptr(plan.buf), plan.n_routed, plan.n_slots, plan.max_waves, int(wave), _ptr(main_table),
        _ptr(main_owner), _ptr(main_w13), _ptr(main_w2), int(main_slots), _ptr(host_w13), _ptr(host_w2), _ptr(stage_w13),
        _ptr(stage_w2), b13, b2, _ptr(stage_table), int(stage_table.numel()), int(n_pinned), plan.n_slots,
        _stream(stream)), "lmoe_wave_stage")
