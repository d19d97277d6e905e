"""vllm::moe_offload_stage — the eager splitting op between the captured
router piece and the captured MLP piece.

Reads the routed ids to the host (the one unavoidable D2H of the seam),
counts the active experts, and either stages them into the fixed slots
(runtime.stage_fixed_slot_plan: H2D on the transfer stream, consumer wait,
in-place log2phy), or, for a decode-sized batch whose union exceeds the slots
by at most the slot count (with decode_overflow on), stages the bank plus one
overflow pass; a decode-sized union past that goes to the device-planned
waves when the layer has them; when the union exceeds the slot capacity
otherwise in a known phase, it defers to the wave executor and caches the
histogram for it.  It
returns nothing and declares topk_ids mutated so the MLP piece reads the
router's tensor at its captured address.

Reference: ops/fused_moe/moe_offload_stage_op.py — phases :77-80, profile /
graph-warm-up context :88-135, _moe_offload_stage_impl :160-471,
_count_active_experts_from_cpu_topk :474-508, registration :523-529.
"""

from __future__ import annotations

import os
from contextvars import ContextVar

import torch

from vllm_moe_offload_amd.ops.fused_moe._register import register_custom_op

PHASE_DECODE: int = 0
PHASE_PREFILL: int = 1
PHASE_MIXED: int = 2
PHASE_UNKNOWN: int = -1

_PROFILE_RUN_ACTIVE: ContextVar[bool] = ContextVar("latchmoe_profile_run_active", default=False)
_GRAPH_WARMUP_ACTIVE: ContextVar[bool] = ContextVar("latchmoe_graph_warmup_active", default=False)


def set_moe_offload_profile_run_active(active: bool):
    return _PROFILE_RUN_ACTIVE.set(bool(active))


def reset_moe_offload_profile_run_active(token) -> None:
    _PROFILE_RUN_ACTIVE.reset(token)


def is_moe_offload_profile_run_active() -> bool:
    return bool(_PROFILE_RUN_ACTIVE.get())


def set_moe_offload_graph_warmup_active(active: bool):
    return _GRAPH_WARMUP_ACTIVE.set(bool(active))


def reset_moe_offload_graph_warmup_active(token) -> None:
    _GRAPH_WARMUP_ACTIVE.reset(token)


def is_moe_offload_graph_warmup_active() -> bool:
    return bool(_GRAPH_WARMUP_ACTIVE.get())


def is_moe_offload_adaptive_wave_context() -> bool:
    return is_moe_offload_profile_run_active() or is_moe_offload_graph_warmup_active()


def count_active_experts_from_cpu_topk(flat_topk_ids: torch.Tensor, *, num_logical_experts: int,
                                       small_threshold: int = 64) -> tuple[dict[int, int], list[int] | None]:
    """Histogram of valid ids in [0, num_logical_experts) of a host tensor."""
    if flat_topk_ids.numel() == 0:
        return {}, []
    flat = flat_topk_ids.reshape(-1)
    if int(flat.numel()) <= int(small_threshold):
        ids = [int(e) for e in flat.tolist()]
        counts: dict[int, int] = {}
        for e in ids:
            if 0 <= e < int(num_logical_experts):
                counts[e] = counts.get(e, 0) + 1
        return counts, ids
    u, c = flat.unique(return_counts=True)
    return {int(e): int(n) for e, n in zip(u.tolist(), c.tolist()) if 0 <= int(e) < int(num_logical_experts) and int(n) > 0}, None


def _moe_offload_stage_impl(topk_ids: torch.Tensor, layer_id: int, num_logical_experts: int, phase: int) -> None:
    from vllm_moe_offload_amd.moe_offload.runtime import get_moe_offload_runtime

    stage_topk_for_layer(get_moe_offload_runtime(), topk_ids, layer_id, num_logical_experts, phase)


def stage_topk_for_layer(runtime, topk_ids: torch.Tensor, layer_id: int, num_logical_experts: int, phase: int) -> None:
    """The seam's staging decision for one layer of the given runtime."""
    from vllm_moe_offload_amd.moe_offload import runtime as runtime_mod

    _is_current_graph_capturing = runtime_mod._is_current_graph_capturing
    layer_id = int(layer_id)
    routed = runtime.routed_expert_count_for_layer(layer_id=layer_id, fallback=int(num_logical_experts))
    total = runtime.total_logical_expert_count_for_layer(layer_id=layer_id, fallback=int(num_logical_experts))
    if _is_current_graph_capturing():
        if runtime.should_use_fixed_slot_plan_for_layer(layer_id) and not runtime.is_layer_registered(layer_id):
            raise RuntimeError(
                f"graph capture reached an unregistered fixed-slot MoE layer {layer_id}; refusing native-weight fallback"
            )
        return
    if runtime.is_static_residency_regime_for_layer(layer_id=layer_id, fallback_routed_expert_count=routed) and (
            runtime.is_full_residency_staged(layer_id) or not runtime.is_layer_registered(layer_id)):
        # every expert is staged and the table static; a registered layer
        # whose full residency was not staged (no graph mode) stages per step
        return
    if not runtime.should_use_fixed_slot_plan_for_layer(layer_id):
        return
    if not runtime.is_layer_registered(layer_id):
        raise RuntimeError(f"fixed-slot MoE layer {layer_id} is not registered; refusing native-weight fallback")
    phase = int(phase)
    hint = int(runtime.config.max_num_seqs_hint or 0)
    tokens = int(topk_ids.shape[0]) if topk_ids.ndim > 0 else 0
    prefill_sized = phase == PHASE_PREFILL or (phase == PHASE_UNKNOWN and hint > 0 and tokens > hint)
    if prefill_sized and runtime.can_run_device_waves(layer_id):
        # the waves are planned and staged on the device: no D2H here
        runtime.mark_device_waves(layer_id=layer_id, topk_ids=topk_ids)
        if os.environ.get("LATCHMOE_SEAM_PROBE"):
            print(f"LATCHMOE_SEAM branch=device_waves layer={layer_id}", flush=True)
        return
    flat = topk_ids.detach().reshape(-1).to("cpu", non_blocking=False)  # the seam's D2H
    bad = int(((flat < 0) | (flat >= total)).sum()) if flat.numel() else 0
    if bad:
        # no slot, stage buffer or wave serves such a pair: fail closed here,
        # as the reference's remap does (slot_mapping.py:116-140), rather than
        # let a pass skip it
        raise RuntimeError(f"layer {layer_id}: topk_ids hold {bad} pairs with expert ids outside [0, {total})")
    runtime.check_device_flags(layer_id=layer_id)
    counts, _ = count_active_experts_from_cpu_topk(flat, num_logical_experts=routed)
    active = tuple(sorted(counts))
    n_active = len(active)
    over = n_active > int(runtime.config.num_slots)
    known = phase in (PHASE_PREFILL, PHASE_DECODE, PHASE_MIXED)
    decode_sized = phase == PHASE_DECODE or (phase == PHASE_UNKNOWN and 0 < tokens <= hint)
    if over and decode_sized and not is_moe_offload_adaptive_wave_context() and \
            runtime.can_stage_decode_overflow(layer_id=layer_id, active_expert_count=n_active):
        # bank + one overflow pass, both inside the captured MLP piece
        runtime.stage_fixed_slot_plan(layer_id=layer_id, active_experts=active, num_logical_experts=total,
                                      token_counts=counts)
        if os.environ.get("LATCHMOE_SEAM_PROBE"):
            print(f"LATCHMOE_SEAM branch=decode_overflow layer={layer_id} n_active={n_active}", flush=True)
        return
    if over and decode_sized and not is_moe_offload_adaptive_wave_context() and runtime.can_run_device_waves(layer_id):
        # past what one overflow pass holds: the device-planned waves, a
        # fixed number of launches with no host step, so the decode MLP piece
        # stays capturable
        runtime.mark_device_waves(layer_id=layer_id, topk_ids=topk_ids)
        if os.environ.get("LATCHMOE_SEAM_PROBE"):
            print(f"LATCHMOE_SEAM branch=decode_device_waves layer={layer_id} n_active={n_active}", flush=True)
        return
    defer = (known and runtime.should_use_b2_pair_waves(layer_id=layer_id, active_expert_count=n_active)) or (
        runtime.config.b2_wave_prefill and phase == PHASE_UNKNOWN and hint > 0 and tokens > hint and over
    ) or (is_moe_offload_adaptive_wave_context() and over)
    if defer:
        runtime.cache_prefill_route_stats(layer_id=layer_id, topk_ids=topk_ids, token_counts_by_expert=counts)
        if os.environ.get("LATCHMOE_SEAM_PROBE"):
            print(f"LATCHMOE_SEAM branch=wave_defer layer={layer_id} n_active={n_active}", flush=True)
        return
    runtime.stage_fixed_slot_plan(layer_id=layer_id, active_experts=active, num_logical_experts=total)


def _moe_offload_stage_fake(topk_ids: torch.Tensor, layer_id: int, num_logical_experts: int, phase: int) -> None:
    return None


def register() -> None:
    register_custom_op("moe_offload_stage", _moe_offload_stage_impl, _moe_offload_stage_fake, ["topk_ids"])
