"""CPU-first loading: offloaded layers' expert weights never occupy HBM whole.

For a layer that runs on fixed slots, the expert parameters are created in
host memory (page-locked when the host store pins) in the checkpoint layout
the slot kernels read, w13 [E, 2I, H] (rows 0..I-1 gate, I..2I-1 up) and w2
[E, H, I].  The checkpoint loads straight into them, one expert tensor at a
time; registration then adopts the two blocks as the layer's host store
without a copy, and only the P-slot bank is allocated on the device.  No
format conversion is needed on this device: the layout of the checkpoint is
the layout of the kernels, so processing is at most a pinning copy.

Two entry points mirror the reference's quant-method hooks
(create_weights, process_weights_after_loading); load_expert_checkpoint is
the loader for callers without vLLM's weight loader: it reads per-expert
tensors from safetensors files (gate_proj/up_proj/down_proj, or w1/w3/w2,
or already stacked w13_weight/w2_weight) into the host blocks.

Reference: moe_offload/cpu_first_loader.py:30-177 (the predicates, the two
hooks, the markers and the registration/release order) and :286-320
(recovering the layer index).
"""

from __future__ import annotations

import re
from typing import Any

import torch

from vllm_moe_offload_amd.moe_offload.host_store import to_host_block

CPU_FIRST_MARKER = "_moe_offload_cpu_first_load"
CPU_FIRST_PROCESSED_MARKER = "_moe_offload_cpu_first_processed"

# checkpoint tensor names of one expert's three projections, by family
EXPERT_NAME_SETS = (
    ("gate_proj", "up_proj", "down_proj"),  # Qwen2/3-MoE, DeepSeek-V2/V3
    ("w1", "w3", "w2"),  # Mixtral
)


def _layer_id(layer: torch.nn.Module) -> int:
    try:
        return int(getattr(layer, "layer_id", -1))
    except (TypeError, ValueError):
        return -1


def layer_index_from_name(name: str) -> int:
    """The layer index in a dotted module path ("model.layers.12.mlp.experts"
    -> 12): the one integer component; -1 when there is none or several."""
    ints = [p for p in str(name).split(".") if p.isdigit()]
    return int(ints[0]) if len(ints) == 1 else -1


def ensure_moe_layer_id(layer: torch.nn.Module) -> int:
    """layer.layer_id, recovered from layer_name or moe_layer_id when the
    container does not carry it yet (and cached on the layer)."""
    layer_id = _layer_id(layer)
    if layer_id >= 0:
        return layer_id
    layer_id = layer_index_from_name(getattr(layer, "layer_name", "") or "")
    if layer_id < 0:
        try:
            layer_id = int(getattr(layer, "moe_layer_id", -1))
        except (TypeError, ValueError):
            layer_id = -1
    if layer_id >= 0:
        setattr(layer, "layer_id", layer_id)
    return layer_id


def should_cpu_first_load_layer(layer: torch.nn.Module, runtime: Any) -> bool:
    config = getattr(runtime, "config", None)
    if not bool(getattr(config, "cpu_first_load", False)):
        return False
    layer_id = ensure_moe_layer_id(layer)
    if layer_id < 0:
        return False
    return bool(runtime.should_use_fixed_slot_plan_for_layer(layer_id))


def is_cpu_first_layer(layer: torch.nn.Module) -> bool:
    return bool(getattr(layer, CPU_FIRST_MARKER, False))


def _empty_host(shape: tuple[int, ...], dtype: torch.dtype, pin: bool) -> torch.Tensor:
    if pin:
        try:
            return torch.empty(shape, dtype=dtype, device="cpu", pin_memory=True)
        except Exception:  # no device runtime, or out of page-locked memory
            pass
    return torch.empty(shape, dtype=dtype, device="cpu")


def _set_weight_attrs(param: torch.Tensor, attrs: dict[str, Any] | None) -> None:
    for key, value in (attrs or {}).items():
        if hasattr(param, key):
            raise AttributeError(f"weight attribute {key} is already set")
        setattr(param, key, value)


def create_cpu_first_expert_weights(
    layer: torch.nn.Module,
    *,
    num_experts: int,
    hidden_size: int,
    intermediate_size: int,
    dtype: torch.dtype,
    pin_memory: bool,
    gated: bool = True,
    extra_weight_attrs: dict[str, Any] | None = None,
) -> None:
    """Register host w13_weight [E, 2I (I if not gated), H] and w2_weight
    [E, H, I] parameters on the layer and mark it CPU-first."""
    E, H, I = int(num_experts), int(hidden_size), int(intermediate_size)
    if E <= 0 or H <= 0 or I <= 0:
        raise ValueError(f"expert shape must be positive: E={E}, H={H}, I={I}")
    up = 2 * I if gated else I
    for name, shape in (("w13_weight", (E, up, H)), ("w2_weight", (E, H, I))):
        param = torch.nn.Parameter(_empty_host(shape, dtype, pin_memory), requires_grad=False)
        layer.register_parameter(name, param)
        _set_weight_attrs(param, extra_weight_attrs)
    setattr(layer, CPU_FIRST_MARKER, True)


def maybe_create_unquantized_cpu_first_weights(
    method: Any,
    layer: torch.nn.Module,
    *,
    runtime: Any,
    num_experts: int,
    hidden_size: int,
    intermediate_size_per_partition: int,
    params_dtype: torch.dtype,
    extra_weight_attrs: dict[str, Any],
) -> bool:
    """create_weights hook: host expert parameters for offloaded layers.
    Returns False (the caller creates device weights) for resident or
    disabled layers and for experts with biases."""
    if not should_cpu_first_load_layer(layer, runtime):
        return False
    moe = getattr(method, "moe", None)
    if bool(getattr(moe, "has_bias", False)):
        return False
    create_cpu_first_expert_weights(
        layer,
        num_experts=num_experts,
        hidden_size=hidden_size,
        intermediate_size=intermediate_size_per_partition,
        dtype=params_dtype,
        pin_memory=bool(getattr(getattr(runtime, "config", None), "should_pin_host_memory", False)),
        gated=bool(getattr(moe, "is_act_and_mul", True)),
        extra_weight_attrs=extra_weight_attrs,
    )
    return True


def _can_process_cpu_first_weight_pair(w13_weight, w2_weight) -> bool:
    """Both on the host, or both on the device (vLLM may move parameters to
    the target device around process_weights_after_loading; they return to
    the host before registration, one layer at a time)."""
    a, b = w13_weight.device.type, w2_weight.device.type
    return a == b and a in {"cpu", "cuda"}


def _current_device_or_cpu() -> torch.device:
    if torch.cuda.is_available():
        return torch.device("cuda", torch.cuda.current_device())
    return torch.device("cpu")


def maybe_process_unquantized_cpu_first_weights(method: Any, layer: torch.nn.Module, *, runtime: Any) -> bool:
    """process_weights_after_loading hook: bring the loaded expert blocks to
    (page-locked) host memory if needed and register the layer's host store
    and slot bank.  Idempotent."""
    if not is_cpu_first_layer(layer):
        return False
    if bool(getattr(layer, CPU_FIRST_PROCESSED_MARKER, False)):
        return True
    if not should_cpu_first_load_layer(layer, runtime):
        return False
    w13, w2 = layer.w13_weight, layer.w2_weight
    if not _can_process_cpu_first_weight_pair(w13, w2):
        return False
    pin = bool(getattr(getattr(runtime, "config", None), "should_pin_host_memory", False))
    blocks = []
    for t in (w13.data, w2.data):
        block, _ = to_host_block(t, pin=pin, copy=False)
        blocks.append(block)
    layer.w13_weight = torch.nn.Parameter(blocks[0], requires_grad=False)
    layer.w2_weight = torch.nn.Parameter(blocks[1], requires_grad=False)
    setattr(layer, CPU_FIRST_PROCESSED_MARKER, True)
    maybe_register_unquantized_fixed_slot_weights(layer, runtime=runtime, slot_device=_current_device_or_cpu())
    return True


def maybe_register_unquantized_fixed_slot_weights(layer: torch.nn.Module, *, runtime: Any,
                                                  slot_device: torch.device | None = None) -> bool:
    """Register a loaded layer for fixed-slot execution (once), then release
    its original expert tensors when the configuration asks for it.  Both
    loading paths (CPU-first and device weights) end here."""
    layer_id = ensure_moe_layer_id(layer)
    if layer_id < 0 or not runtime.should_use_fixed_slot_plan_for_layer(layer_id):
        return False
    if not hasattr(layer, "w13_weight") or not hasattr(layer, "w2_weight"):
        return False
    if not runtime.is_layer_registered(layer_id):
        if slot_device is None:
            slot_device = layer.w13_weight.device
        runtime.register_layer_for_fixed_slots(layer, slot_device=slot_device)
    if bool(getattr(getattr(runtime, "config", None), "release_original_expert_weights", False)):
        runtime.release_original_expert_weights_if_ready(layer)
    return True


# ------------------------------------------------------------------ loading
def _expert_key_pattern(prefix: str, names: tuple[str, str, str]) -> re.Pattern:
    alt = "|".join(re.escape(n) for n in names)
    return re.compile(rf"^{re.escape(prefix)}\.experts\.(\d+)\.({alt})\.weight$")


def load_expert_checkpoint(layer: torch.nn.Module, files, *, prefix: str,
                           names: tuple[str, str, str] | None = None) -> int:
    """Stream the experts of one MoE block from safetensors files into the
    layer's w13_weight / w2_weight (host or device blocks, any dtype: values
    are cast on copy).  prefix is the block's module path, e.g.
    "model.layers.3.mlp"; per-expert names are {prefix}.experts.{e}.{gate,
    up, down}.weight (or the names given), stacked names are
    {prefix}.experts.w13_weight / w2_weight.  Every expert must be found
    exactly once; returns the bytes written."""
    from safetensors import safe_open

    w13, w2 = layer.w13_weight, layer.w2_weight
    E, two_i, H = (int(d) for d in w13.shape)
    I = int(w2.shape[2])
    if two_i != 2 * I or tuple(w2.shape) != (E, H, I):
        raise ValueError(f"layer expert blocks must be [E, 2I, H] / [E, H, I], got "
                         f"{tuple(w13.shape)} / {tuple(w2.shape)}")
    name_sets = (names,) if names is not None else EXPERT_NAME_SETS
    patterns = [(_expert_key_pattern(prefix, ns), ns) for ns in name_sets]
    stacked = {f"{prefix}.experts.w13_weight": (w13, (E, 2 * I, H)),
               f"{prefix}.experts.w2_weight": (w2, (E, H, I))}
    seen: set[tuple[int, int]] = set()
    written = 0
    if isinstance(files, (str, bytes)) or hasattr(files, "__fspath__"):
        files = [files]
    with torch.no_grad():
        for path in files:
            with safe_open(str(path), framework="pt", device="cpu") as fh:
                for key in fh.keys():
                    if key in stacked:
                        dst, shape = stacked[key]
                        src = fh.get_tensor(key)
                        if tuple(src.shape) != shape:
                            raise ValueError(f"{key}: shape {tuple(src.shape)} != {shape}")
                        part = 0 if dst is w13 else 2
                        parts = (0, 1) if part == 0 else (2,)
                        for e in range(E):
                            for p in parts:
                                if (e, p) in seen:
                                    raise ValueError(f"{key}: expert {e} loaded twice")
                                seen.add((e, p))
                        dst.copy_(src)
                        written += tensor_bytes(dst)
                        continue
                    for pat, ns in patterns:
                        m = pat.match(key)
                        if m is None:
                            continue
                        e, part = int(m.group(1)), ns.index(m.group(2))
                        if e >= E:
                            raise ValueError(f"{key}: expert {e} outside the layer's {E} experts")
                        if (e, part) in seen:
                            raise ValueError(f"{key}: expert {e} {m.group(2)} loaded twice")
                        src = fh.get_tensor(key)
                        want = (I, H) if part < 2 else (H, I)
                        if tuple(src.shape) != want:
                            raise ValueError(f"{key}: shape {tuple(src.shape)} != {want}")
                        dst = w13[e, part * I:(part + 1) * I] if part < 2 else w2[e]
                        dst.copy_(src)
                        written += tensor_bytes(dst)
                        seen.add((e, part))
                        break
    missing = [(e, p) for e in range(E) for p in range(3) if (e, p) not in seen]
    if missing:
        e, p = missing[0]
        raise ValueError(f"checkpoint misses {len(missing)} expert tensors under {prefix}; "
                         f"first: expert {e} {('gate', 'up', 'down')[p]}")
    return written


def tensor_bytes(t: torch.Tensor) -> int:
    return int(t.numel()) * int(t.element_size())
