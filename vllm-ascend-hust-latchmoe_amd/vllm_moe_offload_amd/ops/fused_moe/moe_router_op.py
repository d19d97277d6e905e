"""vllm::moe_router / vllm::moe_router_indirect — captured piece 1 of the seam.

Expert selection runs in lmoe_router_topk (one wave64 per token, ties to the
lower expert id); the indirect op first applies the layer's gate with
lmoe_router_gate.  Output ABI as the reference: topk_weights in the hidden
dtype, topk_ids int32, [T, k (+ shared suffix)].

Reference: ops/fused_moe/moe_router_op.py — _moe_router_impl :72-125,
_moe_router_fake :128-162, _moe_router_indirect_impl :191-278 (gate at
:228-231, preserved routed scaling :246-250).
"""

from __future__ import annotations

from typing import Optional

import torch

from vllm_moe_offload_amd.ops.fused_moe._register import get_layer_from_name, register_custom_op


def _moe_router_impl(
    hidden_states: torch.Tensor,
    router_logits: torch.Tensor,
    top_k: int,
    use_grouped_topk: bool,
    renormalize: bool,
    topk_group: Optional[int],
    num_expert_group: Optional[int],
    scoring_func: str,
    routed_scaling_factor: float,
    e_score_correction_bias: Optional[torch.Tensor],
    num_experts: int,
    mix_placement: bool = False,
    num_shared_experts: int = 0,
) -> tuple[torch.Tensor, torch.Tensor]:
    from vllm_moe_offload_amd.fused_moe import RouterSpec, route

    logits = router_logits
    if logits.dtype not in (torch.bfloat16, torch.float32):
        logits = logits.float()
    logits = logits.contiguous()
    if int(logits.shape[-1]) != int(num_experts):
        logits = logits[..., : int(num_experts)].contiguous()
    bias = e_score_correction_bias.float().contiguous() if e_score_correction_bias is not None else None
    spec = RouterSpec(
        top_k=int(top_k), scoring_func=str(scoring_func), renormalize=bool(renormalize),
        use_grouped_topk=bool(use_grouped_topk), num_expert_group=int(num_expert_group or 1),
        topk_group=int(topk_group or 1), routed_scaling_factor=float(routed_scaling_factor),
        e_score_correction_bias=bias,
        # the selection kernel appends the shared suffix (ids num_experts..,
        # weight 1) itself
        n_shared=int(num_shared_experts) if mix_placement else 0,
    )
    w, ids, _ = route(hidden_states, None, spec, router_logits=logits)
    if w.dtype != hidden_states.dtype:
        w = w.to(hidden_states.dtype)
    return w, ids


def _moe_router_fake(
    hidden_states: torch.Tensor,
    router_logits: torch.Tensor,
    top_k: int,
    use_grouped_topk: bool,
    renormalize: bool,
    topk_group: Optional[int],
    num_expert_group: Optional[int],
    scoring_func: str,
    routed_scaling_factor: float,
    e_score_correction_bias: Optional[torch.Tensor],
    num_experts: int,
    mix_placement: bool = False,
    num_shared_experts: int = 0,
) -> tuple[torch.Tensor, torch.Tensor]:
    T = hidden_states.shape[0]
    k = int(top_k) + (int(num_shared_experts) if mix_placement else 0)
    return (
        torch.empty((T, k), dtype=hidden_states.dtype, device=hidden_states.device),
        torch.empty((T, k), dtype=torch.int32, device=hidden_states.device),
    )


def _moe_router_indirect_impl(
    hidden_states: torch.Tensor, router_logits: torch.Tensor, layer_name: str
) -> tuple[torch.Tensor, torch.Tensor]:
    layer = get_layer_from_name(layer_name)
    gate = getattr(layer, "gate_weight", None)
    if gate is not None:
        from vllm_moe_offload_amd import native

        T = hidden_states.shape[0]
        router_logits = native.router_gate(
            hidden_states, gate, torch.empty((T, gate.shape[0]), dtype=hidden_states.dtype, device=hidden_states.device)
        )
        if getattr(layer, "gate_bias", None) is not None:
            # a gate with a linear bias: the selection adds it to the logits
            from vllm_moe_offload_amd.fused_moe import route

            w, ids, _ = route(hidden_states, None, layer.router_spec, router_logits=router_logits)
            return w, ids
    return _moe_router_impl(
        hidden_states, router_logits, layer.top_k, layer.use_grouped_topk, layer.renormalize,
        layer.topk_group, layer.num_expert_group, layer.scoring_func,
        float(getattr(layer, "_original_routed_scaling_factor", getattr(layer, "routed_scaling_factor", 1.0))),
        layer.e_score_correction_bias, layer.num_routed_experts,
        bool(getattr(layer, "mix_placement", False)), int(getattr(layer, "n_shared_experts", 0) or 0),
    )


def _moe_router_indirect_fake(
    hidden_states: torch.Tensor, router_logits: torch.Tensor, layer_name: str
) -> tuple[torch.Tensor, torch.Tensor]:
    layer = get_layer_from_name(layer_name)
    k = int(layer.top_k) + (int(getattr(layer, "n_shared_experts", 0) or 0) if getattr(layer, "mix_placement", False) else 0)
    T = hidden_states.shape[0]
    return (
        torch.empty((T, k), dtype=hidden_states.dtype, device=hidden_states.device),
        torch.empty((T, k), dtype=torch.int32, device=hidden_states.device),
    )


def register() -> None:
    register_custom_op("moe_router", _moe_router_impl, _moe_router_fake, [])
    register_custom_op("moe_router_indirect", _moe_router_indirect_impl, _moe_router_indirect_fake, [])
