"""A slot-bank MoE layer: the model-side object the seam ops drive.

Holds the router (gate weight + routing scalars), the routed expert weights
it registers into the runtime's host store / slot bank, and an optional
shared expert.  A shared expert whose shape equals a routed expert is placed
as a pinned suffix row of the slot bank and appended to every token's top-k
with weight 1 (one combine covers routed + shared); any other shared expert
runs as a dense 1-slot pass whose output enters the routed combine as `add`.

The three pieces map onto the reference's seam: router() is captured piece
1 (moe_router_indirect), stage() the eager splitting op
(moe_offload_stage), forward_experts() captured piece 2 (moe_mlp -> the
fused-experts hook).  Reference: patches/patch_fused_moe.py:4873-5283
(AscendMoERunner seam entry), :4509-4870 (quant-method create/apply),
:2300-2441 (fused shared lane).
"""

from __future__ import annotations

import torch

from vllm_moe_offload_amd import native
from vllm_moe_offload_amd.fused_moe import (
    MoECommMethod,
    MoEFusedExpertsInput,
    MoEOffloadParams,
    MoEWeights,
    RouterSpec,
    fused_experts,
    get_workspace,
    route,
    run_overflow_prefill,
)
from vllm_moe_offload_amd.moe_offload.cpu_first_loader import (
    CPU_FIRST_MARKER,
    create_cpu_first_expert_weights,
    load_expert_checkpoint,
)
from vllm_moe_offload_amd.moe_offload.runtime import MoeOffloadRuntime, _is_current_graph_capturing
from vllm_moe_offload_amd.ops.fused_moe import moe_seam_inject
from vllm_moe_offload_amd.ops.fused_moe.moe_offload_stage_op import PHASE_DECODE


class SlotMoELayer(torch.nn.Module):
    def __init__(
        self,
        *,
        layer_id: int,
        runtime: MoeOffloadRuntime,
        gate_weight: torch.Tensor,
        w13_weight: torch.Tensor,
        w2_weight: torch.Tensor,
        top_k: int,
        scoring_func: str = "softmax",
        renormalize: bool = True,
        use_grouped_topk: bool = False,
        num_expert_group: int = 1,
        topk_group: int = 1,
        routed_scaling_factor: float = 1.0,
        e_score_correction_bias: torch.Tensor | None = None,
        gate_bias: torch.Tensor | None = None,
        shared_w13: torch.Tensor | None = None,
        shared_w2: torch.Tensor | None = None,
        layer_name: str | None = None,
        device: torch.device | str = "cuda",
    ) -> None:
        super().__init__()
        self.layer_id = int(layer_id)
        self.layer_name = layer_name or f"model.layers.{layer_id}.mlp.experts"
        self.runtime = runtime
        self.device = torch.device(device)
        self.top_k = int(top_k)
        self.scoring_func = scoring_func
        self.renormalize = bool(renormalize)
        self.use_grouped_topk = bool(use_grouped_topk)
        self.num_expert_group = int(num_expert_group)
        self.topk_group = int(topk_group)
        self.routed_scaling_factor = float(routed_scaling_factor)
        self.e_score_correction_bias = e_score_correction_bias
        self.gate_weight = gate_weight
        # the gate's linear bias (f32 [E]), added to the logits before scoring
        self.gate_bias = gate_bias
        self.num_routed_experts = int(w13_weight.shape[0])
        self.hidden_size = int(w13_weight.shape[2])
        self.intermediate_size = int(w13_weight.shape[1]) // 2
        self.mix_placement = False
        self.n_shared_experts = 0
        self.shared_w13 = None
        self.shared_w2 = None
        if shared_w13 is not None:
            if tuple(shared_w13.shape) == tuple(w13_weight.shape[1:]) and tuple(shared_w2.shape) == tuple(w2_weight.shape[1:]):
                self.mix_placement = True
                self.n_shared_experts = 1
                w13_weight = torch.cat([w13_weight, shared_w13.unsqueeze(0).to(w13_weight.device)])
                w2_weight = torch.cat([w2_weight, shared_w2.unsqueeze(0).to(w2_weight.device)])
            else:
                self.shared_w13 = shared_w13.unsqueeze(0).contiguous()
                self.shared_w2 = shared_w2.unsqueeze(0).contiguous()
        # registration copies these to the host store (or adopts them, for a
        # CPU-first layer); release_original_expert_weights drops them after
        self.w13_weight = w13_weight
        self.w2_weight = w2_weight

    @classmethod
    def from_checkpoint(cls, files, *, prefix: str, layer_id: int, runtime: MoeOffloadRuntime,
                        num_experts: int, hidden_size: int, intermediate_size: int,
                        dtype: torch.dtype = torch.bfloat16, names: tuple[str, str, str] | None = None,
                        **kwargs) -> "SlotMoELayer":
        """CPU-first construction: the routed experts under `prefix` stream
        from safetensors `files` into host blocks (page-locked when the
        runtime pins), which registration then adopts as the host store; the
        device only ever holds the slot bank.  kwargs are the constructor's
        (gate_weight, top_k, routing options, shared expert, device)."""
        holder = torch.nn.Module()
        create_cpu_first_expert_weights(
            holder, num_experts=num_experts, hidden_size=hidden_size, intermediate_size=intermediate_size,
            dtype=dtype, pin_memory=runtime.config.should_pin_host_memory)
        load_expert_checkpoint(holder, files, prefix=prefix, names=names)
        layer = cls(layer_id=layer_id, runtime=runtime, w13_weight=holder.w13_weight.data,
                    w2_weight=holder.w2_weight.data, **kwargs)
        setattr(layer, CPU_FIRST_MARKER, True)
        return layer

    # -------------------------------------------------------------- setup
    @property
    def num_logical_experts(self) -> int:
        return self.num_routed_experts + self.n_shared_experts

    def register(self) -> None:
        rt = self.runtime
        rt.register_layer_for_fixed_slots(self, slot_device=self.device)
        rt.stage_full_residency_slot_plan(layer_id=self.layer_id)
        # the host store owns the routed rows now; the originals go when the
        # configuration asks for it (the ledger counts them until then)
        if rt.config.release_original_expert_weights:
            rt.release_original_expert_weights_if_ready(self)
        from vllm_moe_offload_amd.ops.fused_moe._register import register_moe_layer

        register_moe_layer(self.layer_name, self)

    @property
    def router_spec(self) -> RouterSpec:
        return RouterSpec(
            top_k=self.top_k, scoring_func=self.scoring_func, renormalize=self.renormalize,
            use_grouped_topk=self.use_grouped_topk, num_expert_group=self.num_expert_group,
            topk_group=self.topk_group, routed_scaling_factor=self.routed_scaling_factor,
            e_score_correction_bias=self.e_score_correction_bias,
            logit_bias=self.gate_bias,
            n_shared=self.n_shared_experts if self.mix_placement else 0,
        )

    # ------------------------------------------------------------ pieces
    def router(self, hidden: torch.Tensor):
        """Captured piece 1: (topk_weights, topk_ids) incl. the shared suffix."""
        w, ids, _ = route(hidden, self.gate_weight, self.router_spec)
        return w, ids

    def stage(self, topk_ids: torch.Tensor, phase: int = PHASE_DECODE) -> None:
        """Eager seam between the pieces."""
        from vllm_moe_offload_amd.ops.fused_moe.moe_offload_stage_op import stage_topk_for_layer

        stage_topk_for_layer(self.runtime, topk_ids, self.layer_id, self.num_logical_experts, int(phase))

    def shared_expert_forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.shared_w13 is None:
            raise RuntimeError("layer has no separate shared expert")
        T, H = x.shape
        ones = _ones_bf16(T, x.device)
        zeros = _zeros_i32(T, x.device)
        ws = get_workspace(T, 1, 1, H, int(self.shared_w13.shape[1]) // 2, x.device, tag=f"shared{self.layer_id}")
        return fused_experts(x, ones, zeros, self.shared_w13, self.shared_w2, None, workspace=ws)

    @property
    def has_separate_shared_expert(self) -> bool:
        return self.shared_w13 is not None

    def forward_experts(self, hidden: torch.Tensor, shared_experts_input: torch.Tensor | None = None, *,
                        include_shared: bool = True) -> torch.Tensor:
        """Captured piece 2, with the injected router output.  A separate
        shared expert is added to the routed output unless include_shared is
        False (the tuple ABI of moe_mlp_shared returns the two apart); a
        pinned-suffix shared expert is one of the routed pairs."""
        injected = moe_seam_inject.peek_injected_topk(self.layer_id)
        if injected is None:
            raise RuntimeError(f"layer {self.layer_id}: forward_experts needs the injected top-k")
        w, ids = injected
        add = None
        if include_shared and self.shared_w13 is not None:
            add = self.shared_expert_forward(shared_experts_input if shared_experts_input is not None else hidden)
        rt = self.runtime
        if rt.consume_device_waves(layer_id=self.layer_id, topk_ids=ids):
            return run_overflow_prefill(rt, layer_id=self.layer_id, hidden=hidden, topk_weights=w, topk_ids=ids,
                                        num_logical_experts=self.num_logical_experts, device_planned=True, add=add)
        if not _is_current_graph_capturing():
            stats = rt.consume_prefill_route_stats_record(layer_id=self.layer_id, topk_ids=ids)
            if stats is not None:
                return run_overflow_prefill(
                    rt, layer_id=self.layer_id, hidden=hidden, topk_weights=w, topk_ids=ids,
                    num_logical_experts=self.num_logical_experts, device_planned=False, add=add,
                    token_counts_by_expert=_with_shared(stats.token_counts_by_expert, self),
                )
        comm = MoECommMethod(rt)
        res = comm.fused_experts(
            MoEFusedExpertsInput(
                hidden_states=hidden, topk_weights=w, topk_ids=ids, weights=MoEWeights(None, None),
                offload=MoEOffloadParams(enabled=True, layer_id=self.layer_id,
                                         num_logical_experts=self.num_logical_experts,
                                         expected_device_type=self.device.type),
                shared_output=add,
            )
        )
        return res.routed_out

    def forward(self, hidden: torch.Tensor, phase: int = PHASE_DECODE) -> torch.Tensor:
        """Eager router -> stage -> experts (what the three ops do in turn)."""
        w, ids = self.router(hidden)
        self.stage(ids, phase)
        moe_seam_inject.set_injected_topk(self.layer_id, w, ids)
        try:
            return self.forward_experts(hidden)
        finally:
            moe_seam_inject.clear_injected_topk(self.layer_id)


def _with_shared(counts: dict[int, int], layer: SlotMoELayer) -> dict[int, int]:
    # the shared suffix is pinned, never a wave member
    return {e: c for e, c in counts.items() if e < layer.num_routed_experts}


_CONST: dict[tuple, torch.Tensor] = {}


def clear_constants() -> None:
    """Drop the cached constant tensors (ones / zeros of the separate shared
    expert pass)."""
    _CONST.clear()


def _ones_bf16(T: int, device) -> torch.Tensor:
    key = ("ones", T, str(device))
    if key not in _CONST:
        _CONST[key] = torch.ones((T, 1), dtype=torch.bfloat16, device=device)
    return _CONST[key]


def _zeros_i32(T: int, device) -> torch.Tensor:
    key = ("zeros", T, str(device))
    if key not in _CONST:
        _CONST[key] = torch.zeros((T, 1), dtype=torch.int32, device=device)
    return _CONST[key]
