"""vllm::moe_mlp / vllm::moe_mlp_shared — captured piece 2 of the seam.

Runs the routed experts with the router's precomputed top-k (handed over
through moe_seam_inject) on the slot bank: lmoe_permute through the layer's
persistent log2phy, then the decode kernels or the MFMA grouped GEMM, then
the combine.  An overflow the stage op deferred runs as capacity-bounded
waves with one combine.

Reference: ops/fused_moe/moe_mlp_op.py — _moe_mlp_impl :69-130 (inject,
then the layer's forward), fakes :133-150 / :204-229, _moe_mlp_shared_impl
:152-201, registration :232-247 (mutates_args=["hidden_states"]).
"""

from __future__ import annotations

from typing import Optional

import torch

from vllm_moe_offload_amd.ops.fused_moe import moe_seam_inject
from vllm_moe_offload_amd.ops.fused_moe._register import get_layer_from_name, register_custom_op


def _moe_mlp_impl(
    hidden_states: torch.Tensor,
    router_logits: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    shared_experts_input: Optional[torch.Tensor],
    input_ids: Optional[torch.Tensor],
    layer_name: str,
    hidden_dim_unpadded: int = -1,
) -> torch.Tensor:
    layer = get_layer_from_name(layer_name)
    layer_id = int(getattr(layer, "layer_id", -1))
    if bool(getattr(layer, "has_separate_shared_expert", False)):
        # the reference's single-tensor op covers only layers without a
        # separate shared expert (moe_mlp_op.py:124-127); those take
        # moe_mlp_shared and its (shared_out, routed_out) tuple
        raise RuntimeError("moe_mlp seam supports only the _shared_experts is None path; use moe_mlp_shared")
    moe_seam_inject.set_injected_topk(layer_id, topk_weights, topk_ids)
    try:
        out = layer.forward_experts(hidden_states, shared_experts_input=shared_experts_input)
    finally:
        moe_seam_inject.clear_injected_topk(layer_id)
    if isinstance(out, tuple):
        raise RuntimeError("moe_mlp seam supports only the routed-output path")
    if hidden_dim_unpadded > 0 and out.shape[-1] != hidden_dim_unpadded:
        out = out[..., :hidden_dim_unpadded]
    return out.clone()


def _moe_mlp_fake(
    hidden_states: torch.Tensor,
    router_logits: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    shared_experts_input: Optional[torch.Tensor],
    input_ids: Optional[torch.Tensor],
    layer_name: str,
    hidden_dim_unpadded: int = -1,
) -> torch.Tensor:
    if hidden_dim_unpadded > 0:
        return hidden_states.new_empty((*hidden_states.shape[:-1], hidden_dim_unpadded))
    return torch.empty_like(hidden_states)


def _moe_mlp_shared_impl(
    hidden_states: torch.Tensor,
    router_logits: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    shared_experts_input: Optional[torch.Tensor],
    input_ids: Optional[torch.Tensor],
    layer_name: str,
    hidden_dim_unpadded: int = -1,
) -> tuple[torch.Tensor, torch.Tensor]:
    layer = get_layer_from_name(layer_name)
    layer_id = int(getattr(layer, "layer_id", -1))
    if layer_id < 0:
        raise RuntimeError(f"moe_mlp_shared requires a stable non-negative layer_id; layer={layer_name!r}")
    moe_seam_inject.set_injected_topk(layer_id, topk_weights, topk_ids)
    try:
        # routed_out excludes the shared expert: the runner adds the two
        # (moe_mlp_op.py:152-201)
        routed = layer.forward_experts(hidden_states, shared_experts_input=None, include_shared=False)
        routed = routed.clone()  # the shared pass below may reuse the output workspace
        src = shared_experts_input if shared_experts_input is not None else hidden_states
        shared = layer.shared_expert_forward(src).clone()
    finally:
        moe_seam_inject.clear_injected_topk(layer_id)
    return shared, routed


def _moe_mlp_shared_fake(
    hidden_states: torch.Tensor,
    router_logits: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    shared_experts_input: Optional[torch.Tensor],
    input_ids: Optional[torch.Tensor],
    layer_name: str,
    hidden_dim_unpadded: int = -1,
) -> tuple[torch.Tensor, torch.Tensor]:
    routed = _moe_mlp_fake(hidden_states, router_logits, topk_weights, topk_ids, shared_experts_input,
                           input_ids, layer_name, hidden_dim_unpadded)
    shared = torch.empty_like(shared_experts_input if shared_experts_input is not None else hidden_states)
    return shared, routed


def register() -> None:
    register_custom_op("moe_mlp", _moe_mlp_impl, _moe_mlp_fake, ["hidden_states"])
    register_custom_op("moe_mlp_shared", _moe_mlp_shared_impl, _moe_mlp_shared_fake, ["hidden_states"])
