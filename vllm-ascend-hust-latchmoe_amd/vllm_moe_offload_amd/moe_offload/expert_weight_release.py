"""Dropping a layer's original expert tensors once the slot path owns them.

After registration the host store holds every routed expert row (a copy, or
the very host tensors of a CPU-first layer), so the layer's own w13_weight /
w2_weight are no longer read on the offloaded path.  Releasing them replaces
both parameters with empty tensors of the same device and dtype; the device
memory goes back to torch's caching allocator as soon as nothing else holds
the old tensors.  A CPU-first layer's host tensors stay alive through the
host store.

Reference: moe_offload/expert_weight_release.py:29-44 (the replacement with
empty parameters and the freed-byte count).
"""

from __future__ import annotations

import torch


def tensor_nbytes(t: torch.Tensor | None) -> int:
    if t is None:
        return 0
    return int(t.numel()) * int(t.element_size())


def release_layer_original_expert_weights(layer: torch.nn.Module) -> int:
    """Replace layer.w13_weight / layer.w2_weight with empty parameters;
    returns the bytes the layer no longer references."""
    w13 = getattr(layer, "w13_weight")
    w2 = getattr(layer, "w2_weight")
    freed = tensor_nbytes(w13) + tensor_nbytes(w2)
    for name, t in (("w13_weight", w13), ("w2_weight", w2)):
        empty = torch.nn.Parameter(torch.empty(0, device=t.device, dtype=t.dtype), requires_grad=False)
        if name in getattr(layer, "_parameters", {}):
            layer._parameters[name] = empty
        else:
            setattr(layer, name, empty)
    return freed
