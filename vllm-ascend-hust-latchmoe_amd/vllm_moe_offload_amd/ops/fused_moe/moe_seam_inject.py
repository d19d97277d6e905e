"""Per-layer hand-off of the router's top-k into the MLP piece (single-threaded
forward).  Reference: ops/fused_moe/moe_seam_inject.py:44-65."""

from __future__ import annotations

import torch

_INJECTED: dict[int, tuple[torch.Tensor, torch.Tensor]] = {}


def set_injected_topk(layer_id: int, topk_weights: torch.Tensor, topk_ids: torch.Tensor) -> None:
    _INJECTED[int(layer_id)] = (topk_weights, topk_ids)


def has_injected_topk(layer_id: int) -> bool:
    return int(layer_id) in _INJECTED


def peek_injected_topk(layer_id: int):
    return _INJECTED.get(int(layer_id))


def clear_injected_topk(layer_id: int) -> None:
    _INJECTED.pop(int(layer_id), None)
