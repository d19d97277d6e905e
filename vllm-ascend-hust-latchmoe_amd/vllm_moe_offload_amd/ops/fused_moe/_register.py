"""Custom-op registration: vLLM's direct_register_custom_op when vLLM is
importable, else torch.library in the same `vllm` namespace.  Device
implementations are registered for the CUDA dispatch key, which is the HIP
device key of PyTorch-ROCm (the reference registers PrivateUse1 on Ascend,
moe_router_op.py:165-171)."""

from __future__ import annotations

import torch

_LIB: torch.library.Library | None = None
_REGISTERED: set[str] = set()


def register_custom_op(op_name: str, op_func, fake_impl, mutates_args: list[str]) -> None:
    if op_name in _REGISTERED:
        return
    try:
        from vllm.utils.torch_utils import direct_register_custom_op  # type: ignore
    except Exception:
        direct_register_custom_op = None
    if direct_register_custom_op is not None:
        direct_register_custom_op(
            op_name=op_name, op_func=op_func, fake_impl=fake_impl, mutates_args=mutates_args,
            dispatch_key="CUDA",
        )
    else:
        global _LIB
        if _LIB is None:
            _LIB = torch.library.Library("vllm", "FRAGMENT")
        schema = torch.library.infer_schema(op_func, mutates_args=mutates_args)
        _LIB.define(op_name + schema)
        _LIB.impl(op_name, op_func, "CUDA")
        torch.library.register_fake(f"vllm::{op_name}", fake_impl, lib=_LIB)
    _REGISTERED.add(op_name)


# layer registry for the layer-name-indirect ops (vLLM's get_layer_from_name
# when vLLM is present)
_LAYERS: dict[str, object] = {}


def register_moe_layer(layer_name: str, layer) -> None:
    _LAYERS[str(layer_name)] = layer


def get_layer_from_name(layer_name: str):
    layer = _LAYERS.get(str(layer_name))
    if layer is not None:
        return layer
    try:
        from vllm.model_executor.layers.fused_moe.runner.moe_runner import get_layer_from_name as _g  # type: ignore
    except Exception as exc:
        raise KeyError(f"unknown MoE layer {layer_name!r}") from exc
    return _g(layer_name)
