"""Slot-indexed fused-MoE execution on the gfx950 kernels.

fused_experts() is the body of the reference's fused-experts call with the
slot bank in place of the expert weights: lmoe_permute remaps the top-k ids
through log2phy and sorts the pairs by slot, then either

  * lmoe_fused_moe_decode (<= 1024 pairs): gate_up GEMV + SiLU*mul, then the
    down GEMV fused with the weighted combine (one token), or the down GEMV
    per (row block, slot) into y and the combine (several tokens); or
  * lmoe_grouped_mlp (GEMV or bf16 MFMA) into a flat-pair buffer y, then
    lmoe_combine.

Every buffer comes from a shape-keyed workspace cache, so repeated calls (and
hipGraph replays) see the same addresses and allocate nothing.

run_wave_prefill() executes an active expert union larger than the slot
capacity as canonical waves staged through the runtime's double-buffered
stage banks, and finishes with ONE combine over the original top-k weights
(the result is identical, bit for bit, to the unsplit layer).
run_full_layer() is the blocking reference fallback.

Reference: patches/patch_fused_moe.py — fused_experts hook :3946-4009,
_maybe_apply_moe_offload_plan :2101-2128, _with_prepared_slot_weights
:2039-2099, _run_b2_wave_prefill :2443-3470 (one native combine :3342-3379),
_run_b2_full_layer_reference :3472-3650; MoEFusedExpertsInput fields
:2051-2099 and result fields :3462-3470.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field
from time import perf_counter

import torch

from vllm_moe_offload_amd import native
from vllm_moe_offload_amd.moe_offload import phase_split
from vllm_moe_offload_amd.moe_offload.runtime import MoeOffloadRuntime, _is_current_graph_capturing
from vllm_moe_offload_amd.moe_offload.slot_mapping import PreparedSlotWeights


# ---------------------------------------------------------------------------
# workspaces (fixed addresses per shape)
# ---------------------------------------------------------------------------
@dataclass
class MoEWorkspace:
    perm: native.Permutation
    act: torch.Tensor   # [N, I] bf16, sorted order
    y: torch.Tensor     # [N, H] bf16, flat pair order
    out: torch.Tensor   # [T, H] bf16
    perm_overflow: native.Permutation | None = None  # the decode overflow pass's permutation

    def overflow_perm(self, n_pairs: int, n_slots: int, device) -> native.Permutation:
        p = self.perm_overflow
        if p is None or p.n_pairs != int(n_pairs) or p.n_slots != int(n_slots):
            p = self.perm_overflow = native.Permutation.allocate(int(n_pairs), int(n_slots), device)
        return p


_WORKSPACES: dict[tuple, MoEWorkspace] = {}


def get_workspace(T: int, k: int, P: int, H: int, I: int, device, *, tag: str = "") -> MoEWorkspace:
    key = (int(T), int(k), int(P), int(H), int(I), str(device), tag)
    ws = _WORKSPACES.get(key)
    if ws is None:
        N = T * k
        ws = MoEWorkspace(
            perm=native.Permutation.allocate(N, P, device),
            act=torch.empty((max(N, 1), I), dtype=torch.bfloat16, device=device),
            y=torch.empty((max(N, 1), H), dtype=torch.bfloat16, device=device),
            out=torch.empty((max(T, 1), H), dtype=torch.bfloat16, device=device),
        )
        _WORKSPACES[key] = ws
    return ws


def clear_workspaces() -> None:
    _WORKSPACES.clear()


# ---------------------------------------------------------------------------
# router
# ---------------------------------------------------------------------------
@dataclass
class RouterSpec:
    """Routing scalars of one MoE layer (moe_router_op.py:72-86 arguments)."""

    top_k: int
    scoring_func: str = "softmax"
    renormalize: bool = True
    use_grouped_topk: bool = False
    num_expert_group: int = 1
    topk_group: int = 1
    routed_scaling_factor: float = 1.0
    # selection-only bias of the scores (vLLM's e_score_correction_bias)
    e_score_correction_bias: torch.Tensor | None = None
    # the router gate's linear bias, added to the logits before scoring
    logit_bias: torch.Tensor | None = None
    # pinned shared experts appended to every token by the router (ids
    # E, E+1, ..., weight 1): select_experts' mix-placement suffix
    # (patch_fused_moe.py:4697-4727)
    n_shared: int = 0


def route(hidden: torch.Tensor, gate_weight: torch.Tensor | None, spec: RouterSpec, *,
          router_logits: torch.Tensor | None = None, logits_out: torch.Tensor | None = None,
          w_out: torch.Tensor | None = None, ids_out: torch.Tensor | None = None):
    """Gate (if gate_weight is given) then expert selection on the GPU.
    Returns (topk_weights bf16 [T,k+S], topk_ids int32 [T,k+S], logits), S =
    spec.n_shared suffix columns."""
    if gate_weight is not None:
        T = hidden.shape[0]
        E = gate_weight.shape[0]
        if logits_out is None:
            logits_out = torch.empty((T, E), dtype=hidden.dtype, device=hidden.device)
        router_logits = native.router_gate(hidden, gate_weight, logits_out)
    if router_logits is None:
        raise ValueError("route() needs router_logits or a gate weight")
    grouped = bool(spec.use_grouped_topk)
    w, ids, _ = native.router_topk(
        router_logits, int(spec.top_k), scoring=spec.scoring_func,
        bias=spec.e_score_correction_bias, logit_bias=spec.logit_bias,
        num_expert_group=int(spec.num_expert_group or 1) if grouped else 1,
        topk_group=int(spec.topk_group or 1) if grouped else 1,
        renormalize=bool(spec.renormalize), routed_scaling_factor=float(spec.routed_scaling_factor),
        n_shared=int(spec.n_shared), w_bf16=w_out, ids=ids_out,
    )
    return w, ids, router_logits


# ---------------------------------------------------------------------------
# one pass over the slot bank
# ---------------------------------------------------------------------------
def fused_experts(
    hidden: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    w13_slots: torch.Tensor,
    w2_slots: torch.Tensor,
    log2phy: torch.Tensor | None,
    *,
    add: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    path: int = native.LMOE_PATH_AUTO,
    workspace: MoEWorkspace | None = None,
) -> torch.Tensor:
    """out[t] = add[t] + sum_j w[t,j] * MLP_{slot(ids[t,j])}(x_t).

    Permute, then: up to 1024 pairs (unless path is MFMA) and I <= 4096 the
    decode body (gate_up GEMV, down GEMV fused with the combine); otherwise
    the grouped GEMM (MFMA unless path is GEMV; always MFMA past the GEMV's
    I <= 4096) and the combine.  topk_ids come from the caller, so a token
    may name one expert twice: the decode body takes its general form,
    which holds no one-pair-per-slot assumption."""
    return _fused_experts_ws(hidden, topk_weights, topk_ids, w13_slots, w2_slots, log2phy, add=add, out=out,
                             path=path, workspace=workspace)[0]


def _pass_path(n_pairs: int, I: int, path: int) -> int:
    """The MLP path of one pass of a multi-pass layer, by the rule the
    single-pass layer uses (fused_experts): the decode GEMVs up to
    FUSED_DECODE_MAX_PAIRS pairs (and I <= GEMV_MAX_I), MFMA tiles past
    that, so a split layer gives the unsplit layer's bits."""
    if path != native.LMOE_PATH_AUTO:
        return path
    return native.LMOE_PATH_GEMV if n_pairs <= native.FUSED_DECODE_MAX_PAIRS and I <= native.GEMV_MAX_I \
        else native.LMOE_PATH_MFMA


def _overflow_perm(hidden, k: int, overflow: PreparedSlotWeights, ws: MoEWorkspace) -> native.Permutation:
    """The workspace's permutation buffers of the overflow table."""
    return ws.overflow_perm(hidden.shape[0] * k, int(overflow.physical_expert_count), hidden.device)


def _overflow_permute(hidden, topk_ids, k: int, overflow: PreparedSlotWeights, ws: MoEWorkspace, *,
                      decode: bool) -> native.Permutation:
    """The second pass's permutation: the pairs the overflow table maps
    (every other pair is skipped).  The bank pass's row_idx then marks the
    pairs placed by either pass: the combine's row mask."""
    T, H = hidden.shape
    P2 = int(overflow.physical_expert_count)
    I = int(overflow.w1.shape[1]) // 2
    perm = _overflow_perm(hidden, k, overflow, ws)
    bm = native.MFMA_BLOCK_M if decode else native.prefill_block_m(P2, H, I, hidden.device, n_pairs=T * k)
    native.permute(topk_ids, perm, log2phy=overflow.log2phy, keep_rows=True, row_idx=ws.perm.row_idx,
                   block_m=bm)
    return perm


def _overflow_pass(hidden, topk_ids, k: int, overflow: PreparedSlotWeights, ws: MoEWorkspace, *, decode: bool):
    """Second pass of a decode step whose routed experts exceed the bank:
    the pairs the overflow table maps run from the stage buffer into their
    rows of y."""
    T = hidden.shape[0]
    perm = _overflow_permute(hidden, topk_ids, k, overflow, ws, decode=decode)
    native.grouped_mlp(hidden, k, overflow.w1, overflow.w2, perm, ws.act[: T * k], ws.y[: T * k],
                       path=native.LMOE_PATH_GEMV if decode else native.LMOE_PATH_MFMA)


def _merged_passes(hidden, I: int, decode: bool) -> bool:
    """Whether a decode overflow layer runs both passes' GEMVs in shared
    launches (decode_mlp_two_passes): the decode GEMV path with rows of at
    most TWO_PASS_MAX_COLS columns.  In the 48-layer B=64 decode graph
    (Qwen3-30B-A3B shapes, ~33 of 48 layers with an overflow pass) shared
    launches took the layer from 186.0 to 180.2 us, and both tables' builds
    in one permutation launch on top of them to 176.0 us (same box)."""
    return decode and hidden.shape[1] <= native.TWO_PASS_MAX_COLS and I <= native.TWO_PASS_MAX_COLS


def _two_passes(hidden, topk_ids, k: int, w13_slots, w2_slots, overflow: PreparedSlotWeights,
                ws: MoEWorkspace, perm: native.Permutation | None = None) -> None:
    """Both passes of a decode overflow layer after the bank permutation
    (skip_unmapped): the overflow permutation (unless perm already holds
    it), then one gate_up and one down launch serve both; y[pair] has the
    bits of the passes run one by one."""
    T = hidden.shape[0]
    if perm is None:
        perm = _overflow_permute(hidden, topk_ids, k, overflow, ws, decode=True)
    native.decode_mlp_two_passes(hidden, k, w13_slots, w2_slots, ws.perm, overflow.w1, overflow.w2, perm,
                                 ws.act[: T * k], ws.y[: T * k])


def _fused_experts_ws(hidden, topk_weights, topk_ids, w13_slots, w2_slots, log2phy, *, add=None, out=None,
                      path=native.LMOE_PATH_AUTO, workspace=None, events=None, overflow=None):
    """fused_experts returning (out, workspace); events = three torch events
    recorded before the permutation, before GMM2 and before the combine.
    overflow: the decode overflow pass (the bank pass then skips the pairs
    its table leaves unmapped, the combine sums both passes' rows)."""
    T, H = hidden.shape
    k = int(topk_ids.shape[1])
    P = int(w13_slots.shape[0])
    I = int(w13_slots.shape[1]) // 2
    ws = workspace or get_workspace(T, k, P, H, I, hidden.device)
    dst = out if out is not None else ws.out[:T]
    if I > native.GEMV_MAX_I and path == native.LMOE_PATH_AUTO:
        path = native.LMOE_PATH_MFMA
    decode = T * k <= native.FUSED_DECODE_MAX_PAIRS and path != native.LMOE_PATH_MFMA
    bm = native.MFMA_BLOCK_M if decode else native.prefill_block_m(P, H, I, hidden.device, n_pairs=T * k)
    merged = overflow is not None and log2phy is not None and _merged_passes(hidden, I, decode) and not events
    if events:
        events[0].record()
    perm_b = None
    if merged:  # both tables' builds in one launch
        perm_b = _overflow_perm(hidden, k, overflow, ws)
        native.permute_two_tables(topk_ids, ws.perm, log2phy, perm_b, overflow.log2phy, block_m=bm)
    else:
        native.permute(topk_ids, ws.perm, log2phy=log2phy, skip_unmapped=overflow is not None, block_m=bm)
    if overflow is not None:
        if merged:
            _two_passes(hidden, topk_ids, k, w13_slots, w2_slots, overflow, ws, perm_b)
        else:
            mlp_path = native.LMOE_PATH_GEMV if decode else native.LMOE_PATH_MFMA
            native.gateup_silu(hidden, k, w13_slots, ws.perm, ws.act[: T * k], path=mlp_path)
            if events:
                events[1].record()
            native.down(ws.act[: T * k], w2_slots, ws.perm, ws.y[: T * k], path=mlp_path)
            _overflow_pass(hidden, topk_ids, k, overflow, ws, decode=decode)
            if events:
                events[2].record()
        native.combine(ws.y[: T * k], topk_weights, dst, row_mask=ws.perm.row_idx[: T * k], add=add)
        return dst, ws
    if decode:
        if events:  # the decode body fuses GMM2 with the combine
            events[1].record()
            events[2].record()
        native.fused_moe_decode(hidden, topk_weights, w13_slots, w2_slots, ws.perm, ws.act[: T * k], dst, add=add,
                                y=ws.y[: T * k], distinct_slots=False)
    else:
        native.gateup_silu(hidden, k, w13_slots, ws.perm, ws.act[: T * k], path=path)
        if events:
            events[1].record()
        native.down(ws.act[: T * k], w2_slots, ws.perm, ws.y[: T * k], path=path)
        if events:
            events[2].record()
        native.combine(ws.y[: T * k], topk_weights, dst, row_mask=ws.perm.row_idx[: T * k], add=add)
    return dst, ws


# Up to this many tokens the decode router runs as one launch (gate,
# selection, permutation); with more, the separate gate launch and the
# selection + permutation launch are faster.  Measured in the 48-layer decode
# graph: one token 23.6 against 23.8 us per layer; with the one launch's gate
# split over token groups and its fence-free logit hand-off, four tokens
# 43.6 against 43.4 us and sixteen 81.5 against 80.4 us per layer (same box).
ONE_LAUNCH_ROUTER_MAX_TOKENS = 1


def decode_layer(
    hidden: torch.Tensor,
    gate_weight: torch.Tensor,
    spec: RouterSpec,
    w13_slots: torch.Tensor,
    w2_slots: torch.Tensor,
    log2phy: torch.Tensor | None,
    *,
    workspace: MoEWorkspace,
    add: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    logits_out: torch.Tensor | None = None,
    w_out: torch.Tensor | None = None,
    ids_out: torch.Tensor | None = None,
    overflow: PreparedSlotWeights | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """route() followed by fused_experts(), for a slot table that is final
    before the router runs (the decode replay after staging): gate, expert
    selection and permutation (one launch for up to
    ONE_LAUNCH_ROUTER_MAX_TOKENS tokens; one token on the fused body takes
    its pairs in pair order, router_gate_topk_pairs, which leaves the sort
    off the router's dependent chain: B=1 23.42 -> 22.69 us per layer in the
    48-layer graph, same box), then the decode MLP body.  Returns
    (out, topk_weights, topk_ids), equal bit for bit to the separate calls.
    overflow: the layer's second pass (stage buffer + overflow table) for a
    working set past the bank; both passes and the combine are fixed-shape
    launches, so a graph captured with them replays any split."""
    T = hidden.shape[0]
    k = int(spec.top_k)
    kw = k + int(spec.n_shared)  # pairs per token, shared suffix included
    P = int(w13_slots.shape[0])
    ws = workspace
    if ws.perm.n_slots != P or ws.perm.n_pairs != T * kw:
        raise ValueError("workspace permutation does not match the slot bank or the batch")
    if logits_out is None:
        logits_out = torch.empty((T, gate_weight.shape[0]), dtype=hidden.dtype, device=hidden.device)
    grouped = bool(spec.use_grouped_topk)
    sel = dict(
        log2phy=log2phy, scoring=spec.scoring_func, bias=spec.e_score_correction_bias,
        logit_bias=spec.logit_bias,
        num_expert_group=int(spec.num_expert_group or 1) if grouped else 1,
        topk_group=int(spec.topk_group or 1) if grouped else 1,
        renormalize=bool(spec.renormalize), routed_scaling_factor=float(spec.routed_scaling_factor),
        n_shared=int(spec.n_shared), w_bf16=w_out, ids=ids_out, skip_unmapped=overflow is not None,
    )
    I = int(w13_slots.shape[1]) // 2
    decode = T * kw <= native.FUSED_DECODE_MAX_PAIRS and I <= native.GEMV_MAX_I
    merged = overflow is not None and log2phy is not None and _merged_passes(hidden, I, decode)
    perm_b = None
    fused_body = overflow is None and decode
    if T == 1 and fused_body:
        # the one-token body reads the pairs in pair order: no sort at the
        # end of the router's chain (the same bits as the sorted form)
        w, ids, _ = native.router_gate_topk_pairs(hidden, gate_weight, logits_out, k, ws.perm, **sel)
    elif T <= ONE_LAUNCH_ROUTER_MAX_TOKENS:
        w, ids, _ = native.router_gate_topk_permute(hidden, gate_weight, logits_out, k, ws.perm, **sel)
    else:
        logits = native.router_gate(hidden, gate_weight, logits_out)
        if merged:  # the overflow table's build rides with the bank's
            perm_b = _overflow_perm(hidden, kw, overflow, ws)
            sel["second"] = (perm_b, overflow.log2phy)
        w, ids, _ = native.router_topk_permute(logits, k, ws.perm, **sel)
    dst = out if out is not None else ws.out[:T]
    if overflow is not None:
        if merged:
            _two_passes(hidden, ids, kw, w13_slots, w2_slots, overflow, ws, perm_b)
        else:
            native.grouped_mlp(hidden, kw, w13_slots, w2_slots, ws.perm, ws.act[: T * kw], ws.y[: T * kw],
                               path=native.LMOE_PATH_GEMV if decode else native.LMOE_PATH_MFMA)
            _overflow_pass(hidden, ids, kw, overflow, ws, decode=decode)
        native.combine(ws.y[: T * kw], w, dst, row_mask=ws.perm.row_idx[: T * kw], add=add)
        return dst, w, ids
    if fused_body:
        # router-fed ids: distinct experts per token, in distinct slots
        native.fused_moe_decode(hidden, w, w13_slots, w2_slots, ws.perm, ws.act[: T * kw], dst, add=add,
                                y=ws.y[: T * kw], distinct_slots=True)
    else:
        path = native.LMOE_PATH_MFMA if I > native.GEMV_MAX_I else native.LMOE_PATH_AUTO
        native.grouped_mlp(hidden, kw, w13_slots, w2_slots, ws.perm, ws.act[: T * kw], ws.y[: T * kw], path=path)
        native.combine(ws.y[: T * kw], w, dst, row_mask=ws.perm.row_idx[: T * kw], add=add)
    return dst, w, ids


def check_placed(ws: MoEWorkspace) -> None:
    """Host validation (synchronising): fail if a pair mapped to no slot."""
    meta = ws.perm.meta.cpu().tolist()
    if meta[native.META_ERRORS]:
        raise RuntimeError(f"topk_ids contain experts without ready slots: {meta[native.META_ERRORS]} pairs")


# ---------------------------------------------------------------------------
# the fused-experts extension hook
# ---------------------------------------------------------------------------
# The contract types of the hook, with every field the reference threads
# through it (patch_fused_moe.py:2051-2099 input, :3462-3470 result).  When
# vLLM provides its own classes the installer in patches/patch_fused_moe.py
# uses those; these stand in for them otherwise.
@dataclass
class MoEWeights:
    w1: torch.Tensor | None = None
    w2: torch.Tensor | None = None
    w1_bias: torch.Tensor | None = None
    w2_bias: torch.Tensor | None = None
    w1_scale: torch.Tensor | None = None
    w2_scale: torch.Tensor | None = None
    w1_scale_bias: torch.Tensor | None = None
    w2_scale_bias: torch.Tensor | None = None
    w1_offset: torch.Tensor | None = None
    w2_offset: torch.Tensor | None = None


@dataclass
class MoERoutingParams:
    expert_map: torch.Tensor | None = None
    global_redundant_expert_num: int = 0
    mc2_mask: torch.Tensor | None = None
    apply_router_weight_on_input: bool = False
    log2phy: torch.Tensor | None = None
    physical_expert_count: int | None = None
    pertoken_scale: torch.Tensor | None = None


@dataclass
class MoEOffloadParams:
    enabled: bool = False
    profile_only: bool = False
    layer_id: int = -1
    num_logical_experts: int = 0
    expected_device_type: str = "cuda"
    step_id: int = -1


@dataclass
class MoEFusedExpertsInput:
    hidden_states: torch.Tensor
    topk_weights: torch.Tensor
    topk_ids: torch.Tensor
    weights: MoEWeights = field(default_factory=MoEWeights)
    routing: MoERoutingParams = field(default_factory=MoERoutingParams)
    quant: object | None = None
    activation: str | None = "silu"
    need_trans: bool = False
    dynamic_eplb: bool = False
    swiglu_limit: float | None = None
    offload: MoEOffloadParams = field(default_factory=MoEOffloadParams)
    # resident shared-expert output added before the final rounding (this
    # build's seam; vLLM's runner adds it itself)
    shared_output: torch.Tensor | None = None


@dataclass
class FusedExpertsResult:
    routed_out: torch.Tensor
    before_dispatch_evt: object | None = None
    before_gmm2_evt: object | None = None
    before_combine_evt: object | None = None
    group_list_type: int = 1
    expert_tokens: torch.Tensor | None = None
    swiglu_limit: float | None = None


def check_supported_input(inp) -> None:
    """Fail closed on the parts of the contract the gfx950 kernels do not
    implement (bf16 SwiGLU experts on one GPU)."""
    if getattr(inp, "quant", None) not in (None, False):
        raise RuntimeError("slot-bank fused experts run bf16 weights only; quantized experts are not supported")
    act = getattr(inp, "activation", None)
    if act not in (None, "silu", "swiglu", "SiluAndMul"):
        raise RuntimeError(f"slot-bank fused experts implement SwiGLU only, got activation={act!r}")
    if getattr(inp, "swiglu_limit", None) is not None:
        raise RuntimeError("slot-bank fused experts do not clamp SwiGLU (swiglu_limit must be None)")
    if bool(getattr(inp, "need_trans", False)):
        raise RuntimeError("slot banks hold checkpoint layout ([P, 2I, H] / [P, H, I]); need_trans must be False")
    routing = getattr(inp, "routing", None)
    if routing is not None:
        if bool(getattr(routing, "apply_router_weight_on_input", False)):
            raise RuntimeError("apply_router_weight_on_input is not supported by the slot-bank combine")
        if getattr(routing, "expert_map", None) is not None:
            raise RuntimeError("expert_map (expert parallelism) is not supported on one GPU")


def run_fused_experts_contract(inp, *, result_cls=FusedExpertsResult, record_events: bool = False,
                               overflow: PreparedSlotWeights | None = None):
    """The hook's body: experts over the input's weights (a slot bank with
    its log2phy when prepared), returning the result contract with the
    per-slot token counts (group_list_type 1) and, if asked for, the events
    before dispatch (permutation), before GMM2 and before the combine."""
    check_supported_input(inp)
    hidden, w, ids = inp.hidden_states, inp.topk_weights, inp.topk_ids
    routing = getattr(inp, "routing", None)
    log2phy = getattr(routing, "log2phy", None) if routing is not None else None
    w1, w2 = inp.weights.w1, inp.weights.w2
    if w.dtype != torch.bfloat16:
        w = w.to(torch.bfloat16)
    if ids.dtype != torch.int32:
        ids = ids.to(torch.int32)
    evts = [torch.cuda.Event() for _ in range(3)] if record_events else None
    out, ws = _fused_experts_ws(hidden, w, ids.contiguous(), w1, w2, log2phy,
                                add=getattr(inp, "shared_output", None), events=evts, overflow=overflow)
    P = int(w1.shape[0])
    return result_cls(
        routed_out=out,
        before_dispatch_evt=evts[0] if evts else None,
        before_gmm2_evt=evts[1] if evts else None,
        before_combine_evt=evts[2] if evts else None,
        group_list_type=1,
        expert_tokens=ws.perm.counts[:P],
        swiglu_limit=getattr(inp, "swiglu_limit", None),
    )


class MoECommMethod:
    """World-size-1 fused-experts method over the slot bank (the contract the
    vLLM seam calls: fused_experts, _maybe_apply_moe_offload_plan)."""

    def __init__(self, runtime: MoeOffloadRuntime) -> None:
        self.runtime = runtime
        self._slot_compute_handle = None

    def _with_prepared_slot_weights(self, inp, prepared: PreparedSlotWeights, *, offload_enabled=None,
                                    use_log2phy: bool = True):
        self._slot_compute_handle = self.runtime.begin_slot_compute(prepared)
        return with_slot_weights(inp, prepared, offload_enabled=offload_enabled, use_log2phy=use_log2phy)

    def _maybe_apply_moe_offload_plan(self, inp):
        off = getattr(inp, "offload", None)
        if off is None or not off.enabled:
            return inp
        prepared = self.runtime.capture_safe_slot_weights(layer_id=int(off.layer_id))
        if prepared is None:
            raise RuntimeError(f"fixed-slot MoE layer {off.layer_id} is not registered")
        prepared.validate_backend_ready(expected_device_type=off.expected_device_type)
        return self._with_prepared_slot_weights(inp, prepared)

    def fused_experts(self, inp) -> FusedExpertsResult:
        off = getattr(inp, "offload", None)
        overflow = None
        if off is not None and off.enabled:
            overflow = self.runtime.decode_overflow_slot_weights(layer_id=int(off.layer_id),
                                                                 n_pairs=int(inp.topk_ids.numel()))
        inp = self._maybe_apply_moe_offload_plan(inp)
        try:
            return run_fused_experts_contract(inp, overflow=overflow)
        finally:
            self.runtime.end_slot_compute(self._slot_compute_handle)
            self._slot_compute_handle = None
            if overflow is not None:
                self.runtime.end_overflow_compute(int(off.layer_id))


def with_slot_weights(inp, prepared: PreparedSlotWeights, *, offload_enabled=None, use_log2phy: bool = True,
                      contracts=None):
    """A copy of a fused-experts input whose weights are the slot bank and
    whose routing carries its log2phy and physical expert count; every other
    field is carried over unchanged (patch_fused_moe.py:2039-2099).
    contracts = (input, weights, routing, offload) classes to build with
    (vLLM's own when the seam provides them)."""
    in_cls, w_cls, r_cls, o_cls = contracts or (MoEFusedExpertsInput, MoEWeights, MoERoutingParams,
                                                MoEOffloadParams)
    src_w, src_r, src_o = inp.weights, getattr(inp, "routing", None), inp.offload
    g = lambda obj, name, default=None: getattr(obj, name, default) if obj is not None else default
    weights = w_cls(w1=prepared.w1, w2=prepared.w2, **{
        k: g(src_w, k) for k in ("w1_bias", "w2_bias", "w1_scale", "w2_scale", "w1_scale_bias",
                                 "w2_scale_bias", "w1_offset", "w2_offset")})
    routing = r_cls(
        expert_map=g(src_r, "expert_map"),
        global_redundant_expert_num=g(src_r, "global_redundant_expert_num", 0),
        mc2_mask=g(src_r, "mc2_mask"),
        apply_router_weight_on_input=g(src_r, "apply_router_weight_on_input", False),
        log2phy=prepared.log2phy if use_log2phy else None,
        physical_expert_count=prepared.physical_expert_count,
        pertoken_scale=g(src_r, "pertoken_scale"),
    )
    offload = o_cls(
        enabled=g(src_o, "enabled", False) if offload_enabled is None else bool(offload_enabled),
        profile_only=g(src_o, "profile_only", False),
        layer_id=g(src_o, "layer_id", -1),
        num_logical_experts=g(src_o, "num_logical_experts", 0),
        expected_device_type=g(src_o, "expected_device_type", "cuda"),
        step_id=g(src_o, "step_id", -1),
    )
    fields = dict(
        hidden_states=inp.hidden_states, topk_weights=inp.topk_weights, topk_ids=inp.topk_ids,
        weights=weights, routing=routing, quant=getattr(inp, "quant", None),
        activation=getattr(inp, "activation", "silu"), need_trans=getattr(inp, "need_trans", False),
        dynamic_eplb=getattr(inp, "dynamic_eplb", False), swiglu_limit=getattr(inp, "swiglu_limit", None),
        offload=offload,
    )
    if hasattr(inp, "shared_output"):
        fields["shared_output"] = inp.shared_output
    return in_cls(**fields)


# ---------------------------------------------------------------------------
# capacity-bounded waves with one combine
# ---------------------------------------------------------------------------
@dataclass
class WaveRunReport:
    waves: tuple[tuple[int, ...], ...]
    compute_order: tuple[int, ...]
    h2d_bytes: int = 0
    d2d_bytes: int = 0
    issue_log: list = field(default_factory=list)
    seconds: float = 0.0


def run_wave_prefill(
    runtime: MoeOffloadRuntime,
    *,
    layer_id: int,
    hidden: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    num_logical_experts: int,
    add: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    token_counts_by_expert: dict[int, int] | None = None,
    path: int = native.LMOE_PATH_AUTO,
) -> tuple[torch.Tensor, WaveRunReport]:
    """Overflow execution: plan waves, stage each into a stage buffer (or run
    it from the main bank when all its experts are resident), compute every
    wave's pairs into one flat-pair y, then ONE combine."""
    t0 = perf_counter()
    cfg = runtime.config
    T, H = hidden.shape
    k = int(topk_ids.shape[1])
    bank = runtime.slot_bank(layer_id)
    if bank is None:
        raise RuntimeError(f"layer {layer_id} is not registered for fixed-slot execution")
    P = bank.physical_expert_count
    I = int(bank.w13_slots.shape[1]) // 2
    cache_hit = token_counts_by_expert is not None
    if token_counts_by_expert is None:
        token_counts_by_expert = runtime.consume_prefill_route_stats(layer_id=layer_id, topk_ids=topk_ids)
        cache_hit = token_counts_by_expert is not None
    if token_counts_by_expert is None:
        token_counts_by_expert = phase_split.count_routed_tokens_by_expert(topk_ids)  # D2H
    t_count = perf_counter()
    routed = runtime.routed_expert_count_for_layer(layer_id=layer_id, fallback=num_logical_experts)
    counts = {e: c for e, c in token_counts_by_expert.items() if 0 <= e < routed}
    readiness = runtime.slot_readiness_for_experts(layer_id=layer_id, expert_ids=tuple(counts))
    t_ready = perf_counter()
    plan = phase_split.plan_balanced_b2_waves(counts, int(cfg.num_slots))
    if not plan.waves:
        raise phase_split.B2WaveFallback("no routed pairs to execute")
    t_plan = perf_counter()
    per_expert = runtime.cached_layer_expert_weight_bytes(layer_id=layer_id)
    h2d = {i: per_expert * sum(1 for e in w if not readiness.get(e, False)) for i, w in enumerate(plan.waves)}
    cost = {i: float(plan.wave_tokens(w)) for i, w in enumerate(plan.waves)}
    sched = phase_split.plan_b2_prefill_async_schedule(
        plan.waves, slot_readiness=readiness,
        prefetch_depth=cfg.effective_prefill_prefetch_depth, buffer_count=cfg.effective_prefill_buffer_count,
        h2d_bytes_by_wave=h2d, compute_cost_by_wave=cost, transfer_aware=cfg.transfer_aware_wave_schedule,
    )
    t_sched = perf_counter()
    profiling = bool(runtime.profile_path)
    wave_profiles: dict[int, dict] = {}
    ws = get_workspace(T, k, P, H, I, hidden.device, tag="waves")
    report = WaveRunReport(plan.waves, sched.compute_order)
    staged: dict[int, tuple] = {}
    total_logical = runtime.total_logical_expert_count_for_layer(layer_id=layer_id, fallback=num_logical_experts)
    # pairs of a pinned shared suffix (ids in [routed, total)) run with the
    # first computed wave only; later waves' tables stop at the routed ids
    shared_pairs = phase_split.count_shared_suffix_pairs(topk_ids, routed, total_logical)
    # fail closed before any wave runs: the waves must cover every pair
    # exactly once (phase_split.py:1808-1812); an id outside [0, total) is
    # in no wave, and the caller falls back to the full layer
    if plan.total_pairs + shared_pairs != T * k:
        raise phase_split.B2WaveFallback(
            "B2 wave pair coverage does not match the original top-k routing: "
            f"covered={plan.total_pairs + shared_pairs} expected={T * k}"
        )
    first = True
    t_loop = perf_counter()
    computed: set[int] = set()
    for kind, w, buf in phase_split.iterate_b2_schedule(sched):
        report.issue_log.append((kind, w))
        t_step = perf_counter()
        if kind == "issue_stage":
            prepared, ready, payload = runtime.prepare_prefill_stage_plan(
                layer_id=layer_id, active_experts=plan.waves[w], num_logical_experts=total_logical,
                device=hidden.device, buffer_index=buf, async_load=True,
            )
            report.h2d_bytes += int(payload["h2d_bytes"])
            report.d2d_bytes += int(payload["d2d_bytes"])
            staged[w] = (prepared, ready, buf)
            if profiling:
                wave_profiles[w] = _wave_profile(plan, w, "async_stage", len(payload["hit_experts"]),
                                                 len(payload["miss_experts"]), payload["h2d_bytes"],
                                                 payload["d2d_bytes"], computed, t_step, buf)
        elif kind == "issue_hit":
            prepared = runtime.prepare_ready_slot_plan(
                layer_id=layer_id, active_experts=plan.waves[w], num_logical_experts=total_logical,
                device=hidden.device,
            )
            staged[w] = (prepared, None, None)
            if profiling:
                wave_profiles[w] = _wave_profile(plan, w, "main_slot_hit", len(plan.waves[w]), 0, 0, 0,
                                                 computed, t_step, None)
        else:
            prepared, ready, buf = staged.pop(w)
            t_wait = perf_counter()
            runtime.wait_prefill_stage_plan(ready)
            t_mlp = perf_counter()
            handle = runtime.begin_slot_compute(prepared)
            try:
                native.permute(topk_ids, ws.perm, log2phy=prepared.log2phy, skip_unmapped=True, keep_rows=not first,
                               table_len=total_logical if first else routed,
                               block_m=native.prefill_block_m(len(plan.waves[w]), H, I, hidden.device, n_pairs=T * k))
                first = False
                native.grouped_mlp(hidden, k, prepared.w1, prepared.w2, ws.perm, ws.act[: T * k], ws.y[: T * k],
                                   path=_pass_path(T * k, I, path))
            finally:
                runtime.end_slot_compute(handle)
            if buf is not None:
                ev = torch.cuda.Event()
                ev.record(torch.cuda.current_stream())
                runtime.remember_prefill_stage_buffer_release(layer_id=layer_id, buffer_index=buf, event=ev)
            computed.add(w)
            if profiling and w in wave_profiles:
                wp = wave_profiles[w]
                wp["stage_wait_ms"] = round((t_mlp - t_wait) * 1000.0, 3)
                wp["mlp_ms"] = round((perf_counter() - t_mlp) * 1000.0, 3)  # host issue time
                wp["issue_end_to_compute_ms"] = round((t_wait - wp.pop("_issue_end")) * 1000.0, 3)
    t_scatter = perf_counter()
    dst = out if out is not None else ws.out[:T]
    native.combine(ws.y[: T * k], topk_weights, dst, row_mask=ws.perm.row_idx[: T * k], add=add)
    t_end = perf_counter()
    report.seconds = t_end - t0
    if profiling:
        _record_b2_prefill_event(
            runtime, layer_id=layer_id, plan=plan, sched=sched, T=T, k=k, shared_pairs=shared_pairs,
            waves=[wave_profiles[w] for w in sched.compute_order if w in wave_profiles],
            cache_hit=cache_hit, start=t0,
            control_ms={"token_count": t_count - t0, "readiness": t_ready - t_count, "wave_plan": t_plan - t_ready,
                        "schedule": t_sched - t_plan, "loop": t_scatter - t_loop,
                        "scatter_total": t_end - t_scatter, "end_to_end": t_end - t0},
        )
    return dst, report


def _wave_profile(plan, w: int, mode: str, hits: int, misses: int, h2d: int, d2d: int, computed: set,
                  t_issue: float, buf) -> dict:
    """Per-wave evidence at issue time; a stage issued after its own wave's
    compute would count in prefetch_after_compute_count."""
    experts = plan.waves[w]
    tokens = plan.wave_tokens(experts)
    return {"wave_index": int(w), "experts": [int(e) for e in experts], "tokens": tokens, "pairs": tokens,
            "hits": int(hits), "misses": int(misses), "h2d_bytes": int(h2d), "d2d_bytes": int(d2d),
            "stage_mode": mode, "buffer_index": buf, "issued_before_compute": w not in computed,
            "prefetch_before_compute_count": int(w not in computed and mode != "main_slot_hit"),
            "prefetch_after_compute_count": int(w in computed),
            "stage_issue_ms": round((perf_counter() - t_issue) * 1000.0, 3), "_issue_end": perf_counter()}


def _record_b2_prefill_event(runtime, *, layer_id, plan, sched, T, k, shared_pairs, waves, cache_hit, start,
                             control_ms) -> None:
    """The b2_work_conserving_prefill evidence line, with the reference's
    payload keys (patches/patch_fused_moe.py:3386-3461, 1826-1930)."""
    tokens = [int(wp["tokens"]) for wp in waves] or [0]
    mean = sum(tokens) / len(tokens)
    summary = {"wave_count": len(waves), "hit_only_waves": 0, "miss_only_waves": 0, "mixed_waves": 0,
               "main_slot_hit_waves": 0, "staged_waves": 0, "sync_slot_cache_waves": 0,
               "issued_before_compute_waves": 0, "prefetch_before_compute_issues": 0,
               "prefetch_after_compute_issues": 0}
    for key in ("tokens", "pairs", "hits", "misses", "h2d_bytes", "d2d_bytes"):
        summary[key] = sum(int(wp[key]) for wp in waves)
    for wp in waves:
        h, m = int(wp["hits"]), int(wp["misses"])
        kind = "hit_only_waves" if m == 0 and h > 0 else "miss_only_waves" if h == 0 and m > 0 else \
            "mixed_waves" if h and m else None
        if kind:
            summary[kind] += 1
        summary["main_slot_hit_waves" if wp["stage_mode"] == "main_slot_hit" else "staged_waves"] += 1
        summary["issued_before_compute_waves"] += int(bool(wp["issued_before_compute"]))
        summary["prefetch_before_compute_issues"] += int(wp["prefetch_before_compute_count"])
        summary["prefetch_after_compute_issues"] += int(wp["prefetch_after_compute_count"])
    for key in ("stage_issue_ms", "stage_wait_ms", "mlp_ms", "issue_end_to_compute_ms"):
        summary[key] = round(sum(float(wp.get(key, 0.0)) for wp in waves), 3)
    summary["max_issue_end_to_compute_ms"] = max((float(wp.get("issue_end_to_compute_ms", 0.0)) for wp in waves),
                                                 default=0.0)
    summary["max_stage_wait_ms"] = max((float(wp.get("stage_wait_ms", 0.0)) for wp in waves), default=0.0)
    summary["layer_scatter_ms"] = round(control_ms["scatter_total"] * 1000.0, 3)
    payload = {
        "n_tokens": int(T),
        "n_active": int(plan.active_expert_count),
        "n_pairs": int(plan.total_pairs),
        "logical_pairs": int(plan.total_pairs),
        "shared_pairs": int(shared_pairs),
        "num_slots": int(runtime.config.num_slots),
        "n_waves": len(plan.waves),
        "masked_full_prompt_pairs": int(T) * len(plan.waves) * int(k),
        "work_conserving_saved_pairs": int(T) * len(plan.waves) * int(k) - int(plan.total_pairs),
        "execution_mode": "pair_microbatch",
        "wave_membership_uses_slot_readiness": False,
        "wave_accumulation_dtype": "bfloat16_pairs_one_combine",
        "wave_token_summary": {"min": min(tokens), "max": max(tokens), "mean": round(mean, 3),
                               "imbalance": round(max(tokens) / mean, 3) if mean else 0.0},
        "control_ms": {key: round(v * 1000.0, 3) for key, v in control_ms.items()},
        "route_stats_cache_hit": bool(cache_hit),
        "pair_index_cache_hit": False,
        "pair_planner_mode": "device_permute",
        "forward_phase": "prefill",
        "wave_summary": summary,
    }
    if os.environ.get("VLLM_ASCEND_MOE_B2_PROFILE_DETAILS", "0").strip().lower() in {"1", "true", "yes", "on"}:
        payload.update({"wave_plan": plan.to_jsonable(), "async_schedule": sched.to_jsonable(), "waves": waves})
    else:
        payload["profile_details"] = "omitted"
    runtime._record_profile_event("b2_work_conserving_prefill", layer_id=int(layer_id), start=start,
                                  payload=payload)


def run_device_waves(
    runtime: MoeOffloadRuntime,
    *,
    layer_id: int,
    hidden: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    num_logical_experts: int,
    add: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    path: int = native.LMOE_PATH_AUTO,
) -> torch.Tensor:
    """Overflow prefill with no host step: the waves are planned on the device
    from the routed ids (lmoe_wave_plan), each wave's experts are copied into
    a stage buffer on the transfer stream (main-bank slot or host row,
    lmoe_wave_stage) while the previous wave computes, and every wave's pairs
    land in one flat-pair y; then ONE combine.  The number of launched waves
    is fixed by the shapes (ceil(min(routed, T k) / slots)); waves the plan
    does not need copy and compute nothing, so the whole call can be
    captured.  Same bits as the host-planned waves and the full layer: each
    pair's row is computed alone."""
    T, H = hidden.shape
    k = int(topk_ids.shape[1])
    bank = runtime.slot_bank(layer_id)
    if bank is None:
        raise RuntimeError(f"layer {layer_id} is not registered for fixed-slot execution")
    if not runtime.can_run_device_waves(layer_id):
        raise RuntimeError(f"device wave planning is not available for layer {layer_id}")
    dev = hidden.device
    P = int(bank.num_dynamic_slots)
    I = int(bank.w13_slots.shape[1]) // 2
    routed = runtime.routed_expert_count_for_layer(layer_id=layer_id, fallback=num_logical_experts)
    total = runtime.total_logical_expert_count_for_layer(layer_id=layer_id, fallback=num_logical_experts)
    n_pinned = total - routed
    n_waves = max(1, -(-min(routed, T * k) // P))
    plan = runtime.device_wave_plan_buffer(n_routed=routed, n_slots=P, max_waves=n_waves, device=dev)
    host = runtime.host_store.get_layer_buffer(layer_id)
    main_table = runtime.log2phy_buffer(layer_id)
    main_owner = runtime.slot_owner_buffer(layer_id)
    n_buf = runtime.config.effective_prefill_buffer_count
    stages = [runtime._get_prefill_stage_bank(layer_id=layer_id, buffer_index=b, template_bank=bank)
              for b in range(min(n_buf, n_waves))]
    tables = [runtime._get_prefill_stage_log2phy_buffer(template_bank=bank, buffer_index=b, num_logical_experts=total,
                                                        device=dev) for b in range(len(stages))]
    ws = get_workspace(T, k, int(stages[0].physical_expert_count), H, I, dev, tag="device_waves")
    capturing = _is_current_graph_capturing()
    compute = torch.cuda.current_stream(dev)
    tx = runtime.transfer_engine._transfer_stream(dev)
    native.wave_plan(topk_ids, plan, n_total=total)
    if not capturing:
        # fail closed before any copy: a pair whose id lies outside
        # [0, total) is in no wave (phase_split.py:1808-1812).  Under capture
        # nothing is read back: the plan header's invalid count (word 2)
        # stays on the device, and the combine's row mask drops such pairs
        invalid = int(plan.buf[2].item())
        if invalid:
            raise phase_split.B2WaveFallback(
                f"device wave plan left {invalid} pairs with ids outside [0, {total}) in no wave")
    planned = torch.cuda.Event()
    planned.record(compute)
    tx.wait_event(planned)
    if not capturing:
        # earlier users of the stage buffers (host-planned waves, decode
        # overflow passes) release them with events of their own
        for b in range(len(stages)):
            ev = runtime.prefill_stage_buffer_release_event(layer_id=layer_id, buffer_index=b)
            ev = getattr(ev, "event", ev)
            if isinstance(ev, torch.cuda.Event):
                tx.wait_event(ev)
    released: list = [None] * len(stages)
    bm = native.prefill_block_m(P, H, I, dev, n_pairs=-(-(T * k) // n_waves))
    for w in range(n_waves):
        b = w % len(stages)
        stage, table = stages[b], tables[b]
        if released[b] is not None:
            tx.wait_event(released[b])
        native.wave_stage(plan, w, main_table=main_table, main_owner=main_owner, main_w13=bank.w13_slots,
                          main_w2=bank.w2_slots, main_slots=P, host_w13=host.w13, host_w2=host.w2,
                          stage_w13=stage.w13_slots, stage_w2=stage.w2_slots, stage_table=table,
                          n_pinned=n_pinned, stream=tx)
        ready = torch.cuda.Event()
        ready.record(tx)
        compute.wait_event(ready)
        native.permute(topk_ids, ws.perm, log2phy=table, skip_unmapped=True, keep_rows=w > 0, block_m=bm)
        native.grouped_mlp(hidden, k, stage.w13_slots, stage.w2_slots, ws.perm, ws.act[: T * k], ws.y[: T * k],
                           path=_pass_path(T * k, I, path))
        done = torch.cuda.Event()
        done.record(compute)
        released[b] = done
    if not capturing:
        for b, ev in enumerate(released):
            if ev is not None:
                runtime.remember_prefill_stage_buffer_release(layer_id=layer_id, buffer_index=b, event=ev)
                # the host copy of the stage buffer's contents is void now
                for sid in range(stages[b].num_dynamic_slots):
                    stages[b].clear_slot(sid, force=True)
    else:
        compute.wait_stream(tx)  # the forked transfer stream rejoins the capture
    dst = out if out is not None else ws.out[:T]
    native.combine(ws.y[: T * k], topk_weights, dst, row_mask=ws.perm.row_idx[: T * k], add=add)
    return dst


def run_full_layer(
    runtime: MoeOffloadRuntime,
    *,
    layer_id: int,
    hidden: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    num_logical_experts: int,
    add: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    path: int = native.LMOE_PATH_AUTO,
) -> torch.Tensor:
    """Blocking fallback: stage the whole layer, one pass, one combine.
    Eager calls fail closed (RuntimeError) when a pair maps to no slot of
    the full layer, as the reference's remap does (slot_mapping.py:116-140)."""
    prepared, _ = runtime.prepare_full_layer_prefill_plan(
        layer_id=layer_id, num_logical_experts=num_logical_experts, device=hidden.device,
    )
    T, H = hidden.shape
    k = int(topk_ids.shape[1])
    ws = get_workspace(T, k, prepared.physical_expert_count, H, int(prepared.w1.shape[1]) // 2, hidden.device, tag="full")
    dst = fused_experts(hidden, topk_weights, topk_ids, prepared.w1, prepared.w2, prepared.log2phy,
                        add=add, out=out, path=path, workspace=ws)
    if not _is_current_graph_capturing():
        check_placed(ws)
    return dst


def run_overflow_prefill(
    runtime: MoeOffloadRuntime,
    *,
    layer_id: int,
    hidden: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    num_logical_experts: int,
    device_planned: bool,
    add: torch.Tensor | None = None,
    token_counts_by_expert: dict[int, int] | None = None,
) -> torch.Tensor:
    """Capacity waves (device- or host-planned) with the reference's one
    recoverable error: a B2WaveFallback runs the blocking full layer instead
    (patches/patch_fused_moe.py:2281-2298 -> _run_b2_full_layer_reference
    :3472-3650), and the reason goes to the profile evidence."""
    t0 = perf_counter()
    try:
        if device_planned:
            return run_device_waves(runtime, layer_id=layer_id, hidden=hidden, topk_weights=topk_weights,
                                    topk_ids=topk_ids, num_logical_experts=num_logical_experts, add=add)
        out, _ = run_wave_prefill(runtime, layer_id=layer_id, hidden=hidden, topk_weights=topk_weights,
                                  topk_ids=topk_ids, num_logical_experts=num_logical_experts, add=add,
                                  token_counts_by_expert=token_counts_by_expert)
        return out
    except phase_split.B2WaveFallback as exc:
        reason = f"{type(exc).__name__}: {exc}"
        if os.environ.get("SEW_B2_PROBE") or os.environ.get("SEW_OFFLOAD_PROBE"):
            print(f"SEW_B2 branch=FALLBACK_FULL_LAYER layer={layer_id} reason={reason}", flush=True)
        total = runtime.total_logical_expert_count_for_layer(layer_id=layer_id, fallback=num_logical_experts)
        out = run_full_layer(runtime, layer_id=layer_id, hidden=hidden, topk_weights=topk_weights,
                             topk_ids=topk_ids, num_logical_experts=total, add=add)
        if runtime.profile_path:
            runtime._record_profile_event("b2_full_layer_fallback", layer_id=int(layer_id), start=t0,
                                          payload={"fallback_reason": reason, "n_tokens": int(hidden.shape[0]),
                                                   "device_planned": bool(device_planned)})
        return out
