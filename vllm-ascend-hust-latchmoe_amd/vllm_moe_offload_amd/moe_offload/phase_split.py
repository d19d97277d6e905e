"""Capacity-bounded wave planning for an active expert union larger than the
slot capacity, plus the pair-level index builders and combine helpers of the
wave path.

Plan: experts are packed into the fewest waves of at most num_slots experts
by longest-processing-time on routed-pair counts (canonical: residency never
changes membership, so equivalent requests run identical expert groups), each
wave sorted ascending.  Schedule: waves with any miss are staged (double
buffered, largest transfer first when transfer-aware), hit-only waves run from
the main bank.  Execution (fused_moe.run_wave_prefill) permutes every wave
with its own log2phy on the GPU (lmoe_permute, skip_unmapped) and writes the
MLP output of each pair into one flat-pair buffer, so ONE combine over the
original top-k weights finishes the layer: the result does not depend on the
wave split.

The torch builders here (pair microbatches, device wave plans, native combine
inputs, f32 scatter-adds) restate the reference's index bookkeeping for
callers that drive waves themselves; the hot path uses the kernels instead.

Reference: moe_offload/phase_split.py — count_routed_tokens_by_expert
:479-492; plan_balanced_b2_waves :495-554; plan_b2_prefill_async_schedule
:557-640; simulate_b2_prefill_issue_log :681-766; pair builders :769-1582;
scatter-adds :1585-1762; build_b2_native_combine_inputs :1765-1855;
B2WaveFallback :292-299.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field

import torch


class B2WaveFallback(RuntimeError):
    """A recoverable wave-qualification failure detected before any wave
    result is published; the caller may fall back to the full-layer path."""


@dataclass(frozen=True)
class B2WavePlan:
    waves: tuple[tuple[int, ...], ...]
    token_counts_by_expert: dict[int, int]

    @property
    def active_expert_count(self) -> int:
        return len(self.token_counts_by_expert)

    @property
    def total_pairs(self) -> int:
        return int(sum(self.token_counts_by_expert.values()))

    def wave_tokens(self, wave: tuple[int, ...]) -> int:
        return int(sum(self.token_counts_by_expert.get(int(e), 0) for e in wave))

    def to_jsonable(self) -> dict[str, object]:
        """Evidence form read by the reference's verifiers
        (phase_split.py:151-167 there)."""
        return {
            "n_active": self.active_expert_count,
            "n_pairs": self.total_pairs,
            "n_waves": len(self.waves),
            "waves": [
                {"experts": [int(e) for e in w], "tokens": self.wave_tokens(w),
                 "per_expert_tokens": {str(int(e)): int(self.token_counts_by_expert.get(int(e), 0)) for e in w}}
                for w in self.waves
            ],
        }


@dataclass(frozen=True)
class B2PrefillAsyncSchedule:
    compute_order: tuple[int, ...]
    hit_wave_indices: tuple[int, ...]
    staged_wave_indices: tuple[int, ...]
    staged_issue_order: tuple[int, ...]
    prefetch_depth: int = 1
    buffer_count: int = 2
    initial_stage_count: int = 0
    transfer_aware: bool = False
    estimated_h2d_bytes_by_wave: tuple[int, ...] = ()
    estimated_compute_cost_by_wave: tuple[float, ...] = ()

    def to_jsonable(self) -> dict[str, object]:
        return {k: (list(v) if isinstance(v, tuple) else v) for k, v in self.__dict__.items()}


@dataclass(frozen=True)
class B2PairMicrobatch:
    hidden_states: torch.Tensor
    topk_ids: torch.Tensor
    topk_weights: torch.Tensor
    restore_token_indices: torch.Tensor
    logical_expert_ids: torch.Tensor

    @property
    def num_pairs(self) -> int:
        return int(self.topk_ids.shape[0])


@dataclass(frozen=True)
class B2RoutedPairIndex:
    topk_ids: torch.Tensor
    topk_weights: torch.Tensor
    num_tokens: int
    top_k: int
    pair_offsets_by_expert: dict[int, tuple[int, ...]]

    @property
    def total_pairs(self) -> int:
        return int(sum(len(v) for v in self.pair_offsets_by_expert.values()))


@dataclass(frozen=True)
class B2WaveMicrobatchPlan:
    wave_experts: tuple[int, ...]
    token_indices: torch.Tensor
    topk_positions: torch.Tensor
    logical_expert_ids: torch.Tensor
    physical_slot_ids: torch.Tensor
    flat_pair_offsets: torch.Tensor | None = None
    top_k: int = 1
    layer_pair_start: int = 0
    layer_pair_end: int = 0

    @property
    def num_pairs(self) -> int:
        return int(self.token_indices.numel())

    @property
    def pair_offsets(self) -> torch.Tensor:
        if self.flat_pair_offsets is not None:
            return self.flat_pair_offsets
        return self.token_indices * int(self.top_k) + self.topk_positions


@dataclass(frozen=True)
class B2DirectScatterPayload:
    permuted_tokens: torch.Tensor
    expanded_row_idx: torch.Tensor
    topk_weights: torch.Tensor
    restore_token_indices: torch.Tensor
    wave_index: int = 0
    pair_offsets: torch.Tensor | None = None
    combine_metadata: object | None = None


# ---------------------------------------------------------------------------
# planning
# ---------------------------------------------------------------------------
def count_routed_tokens_by_expert(topk_ids: torch.Tensor) -> dict[int, int]:
    """Routed (token, k) pairs per logical expert (negative ids dropped)."""
    if topk_ids.numel() == 0:
        return {}
    flat = topk_ids.detach().reshape(-1)
    if flat.device.type != "cpu":
        flat = flat.cpu()
    ids, counts = flat.unique(return_counts=True)
    return {int(e): int(c) for e, c in zip(ids.tolist(), counts.tolist()) if int(e) >= 0 and int(c) > 0}


def count_shared_suffix_pairs(topk_ids: torch.Tensor, routed: int, total: int) -> int:
    """Pairs of a pinned shared suffix: ids in [routed, total).  An id at or
    past total belongs to no expert, so it is not counted and the layer's
    coverage check (waves + shared pairs == T * k) fails closed on it."""
    if int(total) <= int(routed) or topk_ids.numel() == 0:
        return 0
    return int(((topk_ids >= int(routed)) & (topk_ids < int(total))).sum().item())


def plan_balanced_b2_waves(
    token_counts_by_expert: dict[int, int],
    num_slots: int,
    *,
    slot_readiness: dict[int, bool] | None = None,
    fold_partial_hits_into_miss: bool = True,
) -> B2WavePlan:
    """Canonical LPT packing of the active experts into <= num_slots waves.

    Experts in (-count, id) order go to the least-loaded wave that still has
    room (lowest index on ties); a new wave opens only when all are full.
    Readiness arguments are accepted for interface compatibility and do not
    influence membership.
    """
    if num_slots <= 0:
        raise ValueError(f"num_slots must be greater than 0, got {num_slots}")
    del slot_readiness, fold_partial_hits_into_miss
    counts = {int(e): int(c) for e, c in token_counts_by_expert.items() if int(c) > 0}
    if not counts:
        return B2WavePlan(waves=(), token_counts_by_expert={})
    order = sorted(counts, key=lambda e: (-counts[e], e))
    n_bins = -(-len(order) // num_slots)
    bins: list[list[int]] = [[] for _ in range(n_bins)]
    loads = [0] * n_bins
    for e in order:
        best = None
        for i in range(len(bins)):
            if len(bins[i]) < num_slots and (best is None or loads[i] < loads[best]):
                best = i
        if best is None:
            bins.append([e])
            loads.append(counts[e])
        else:
            bins[best].append(e)
            loads[best] += counts[e]
    return B2WavePlan(waves=tuple(tuple(sorted(b)) for b in bins), token_counts_by_expert=counts)


def _per_wave(estimates, n: int, cast):
    if estimates is None:
        return tuple(cast(0) for _ in range(n))
    if isinstance(estimates, dict):
        return tuple(max(cast(0), cast(estimates.get(i, 0))) for i in range(n))
    vals = tuple(cast(v) for v in estimates)
    return tuple(max(cast(0), vals[i]) if i < len(vals) else cast(0) for i in range(n))


def plan_b2_prefill_async_schedule(
    waves: tuple[tuple[int, ...], ...],
    *,
    slot_readiness: dict[int, bool] | None = None,
    prefetch_depth: int = 1,
    buffer_count: int = 2,
    h2d_bytes_by_wave=None,
    compute_cost_by_wave=None,
    transfer_aware: bool = False,
) -> B2PrefillAsyncSchedule:
    """Staging order for the waves.  Hit-only waves read the main bank;
    waves with any miss go through stage buffers and may be primed early.
    Transfer-aware: biggest transfers issued first, costliest hit waves
    computed first to cover them."""
    ready = slot_readiness or {}
    hit = [i for i, w in enumerate(waves) if all(ready.get(int(e), False) for e in w)]
    staged = [i for i, w in enumerate(waves) if i not in set(hit)]
    depth = max(0, int(prefetch_depth))
    nbuf = max(1, int(buffer_count))
    h2d = _per_wave(h2d_bytes_by_wave, len(waves), int)
    cost = _per_wave(compute_cost_by_wave, len(waves), float)
    aware = bool(transfer_aware) and bool(waves) and depth > 0 and nbuf > 1
    if aware:
        hit_order = tuple(sorted(hit, key=lambda i: (-cost[i], i)))
        issue = tuple(sorted(staged, key=lambda i: (-h2d[i], -cost[i], i)))
        compute = hit_order + issue
    else:
        issue = tuple(staged)
        compute = tuple(range(len(waves)))
    return B2PrefillAsyncSchedule(
        compute_order=compute,
        hit_wave_indices=tuple(hit),
        staged_wave_indices=tuple(staged),
        staged_issue_order=issue,
        prefetch_depth=depth,
        buffer_count=nbuf,
        initial_stage_count=min(depth, nbuf, len(staged)),
        transfer_aware=aware,
        estimated_h2d_bytes_by_wave=h2d,
        estimated_compute_cost_by_wave=cost,
    )


class _StageIssuer:
    """Buffer bookkeeping of the staged-wave pipeline (shared by the
    simulator and the executor): which staged wave is in which buffer."""

    def __init__(self, issue_order, buffer_count: int) -> None:
        self.order = list(issue_order)
        self.cursor = 0
        self.buffers = max(1, int(buffer_count))
        self.in_flight: dict[int, int] = {}  # wave -> buffer

    def free_buffer(self, busy_extra: int | None = None) -> int | None:
        busy = set(self.in_flight.values())
        if busy_extra is not None:
            busy.add(int(busy_extra))
        return next((b for b in range(self.buffers) if b not in busy), None)

    def next_wave(self, busy_extra: int | None = None) -> tuple[int, int] | None:
        if self.cursor >= len(self.order):
            return None
        buf = self.free_buffer(busy_extra)
        if buf is None:
            return None
        w = int(self.order[self.cursor])
        self.cursor += 1
        self.in_flight[w] = buf
        return w, buf


def iterate_b2_schedule(schedule: B2PrefillAsyncSchedule, *, prefetch_depth: int | None = None,
                        buffer_count: int | None = None):
    """Yield ("issue_stage", wave, buffer), ("issue_hit", wave, None) and
    ("compute", wave, buffer or None) in execution order."""
    depth = int(schedule.prefetch_depth if prefetch_depth is None else prefetch_depth)
    nbuf = int(schedule.buffer_count if buffer_count is None else buffer_count)
    st = _StageIssuer(schedule.staged_issue_order, nbuf)
    issued: set[int] = set()
    initial = min(max(depth, 0), max(nbuf, 1), len(st.order))
    while st.cursor < initial:
        nxt = st.next_wave()
        if nxt is None:
            break
        issued.add(nxt[0])
        yield ("issue_stage", nxt[0], nxt[1])

    def prefetch(current: int | None):
        out = []
        if depth <= 0:
            return out
        target = min(max(depth, 0), max(nbuf, 1) - (1 if current is not None else 0))
        while len(st.in_flight) < target:
            nxt = st.next_wave(current)
            if nxt is None:
                break
            issued.add(nxt[0])
            out.append(("issue_stage", nxt[0], nxt[1]))
        return out

    staged = set(int(i) for i in schedule.staged_wave_indices)
    for w in schedule.compute_order:
        w = int(w)
        if w not in issued:
            if w in staged:
                nxt = st.next_wave()
                if nxt is None:
                    raise RuntimeError(f"unable to issue staged wave {w}; no buffer available")
                issued.add(nxt[0])
                yield ("issue_stage", nxt[0], nxt[1])
            else:
                issued.add(w)
                yield ("issue_hit", w, None)
        current = st.in_flight.pop(w, None)
        yield from prefetch(current)
        yield ("compute", w, current)
        yield from prefetch(None)


def simulate_b2_prefill_issue_log(schedule: B2PrefillAsyncSchedule, *, prefetch_depth: int | None = None,
                                  buffer_count: int | None = None) -> tuple[tuple[str, int], ...]:
    """Issue/compute order of the pipeline, without tensors or streams."""
    return tuple((kind, w) for kind, w, _ in iterate_b2_schedule(
        schedule, prefetch_depth=prefetch_depth, buffer_count=buffer_count))


# ---------------------------------------------------------------------------
# pair-level builders (torch, any device)
# ---------------------------------------------------------------------------
def _empty_microbatch(hidden: torch.Tensor, ids: torch.Tensor, w: torch.Tensor) -> B2PairMicrobatch:
    e = torch.empty(0, dtype=torch.long, device=hidden.device)
    return B2PairMicrobatch(
        hidden_states=hidden.index_select(0, e),
        topk_ids=torch.empty(0, 1, dtype=ids.dtype, device=ids.device),
        topk_weights=torch.empty(0, 1, dtype=w.dtype, device=w.device),
        restore_token_indices=e,
        logical_expert_ids=torch.empty(0, dtype=ids.dtype, device=ids.device),
    )


def _validate_staged(physical: torch.Tensor, logical: torch.Tensor) -> None:
    if os.environ.get("LATCHMOE_B2_VALIDATE") or os.environ.get("SEW_B2_VALIDATE"):
        if bool((physical < 0).any().item()):
            missing = logical[physical < 0].detach().cpu().unique().tolist()
            raise RuntimeError(f"B2 wave has unstaged experts in logical_to_physical: {missing}")


def build_b2_pair_microbatch(hidden_states, topk_ids, topk_weights, logical_to_physical, wave_experts) -> B2PairMicrobatch:
    """top_k=1 microbatch of the pairs whose expert is in the wave, in flat
    pair order, ids remapped to physical slots."""
    if topk_ids.shape != topk_weights.shape:
        raise ValueError(
            f"topk_ids and topk_weights must have identical shape, got {tuple(topk_ids.shape)} vs {tuple(topk_weights.shape)}"
        )
    if hidden_states.shape[0] != topk_ids.shape[0]:
        raise ValueError(f"hidden_states and topk_ids disagree on token count, got {hidden_states.shape[0]} vs {topk_ids.shape[0]}")
    if not wave_experts:
        return _empty_microbatch(hidden_states, topk_ids, topk_weights)
    members = torch.tensor([int(e) for e in wave_experts], dtype=topk_ids.dtype, device=topk_ids.device)
    mask = torch.isin(topk_ids, members)
    tok, pos = torch.nonzero(mask, as_tuple=True)
    if tok.numel() == 0:
        return _empty_microbatch(hidden_states, topk_ids, topk_weights)
    logical = topk_ids[tok, pos]
    physical = logical_to_physical[logical.long()]
    _validate_staged(physical, logical)
    restore = tok.to(device=hidden_states.device, dtype=torch.long)
    return B2PairMicrobatch(
        hidden_states=hidden_states.index_select(0, restore).contiguous(),
        topk_ids=physical.reshape(-1, 1).contiguous(),
        topk_weights=topk_weights[tok, pos].reshape(-1, 1).contiguous(),
        restore_token_indices=restore,
        logical_expert_ids=logical.contiguous(),
    )


def build_b2_routed_pair_index(topk_ids, topk_weights, *, pair_offsets_by_expert=None,
                               validate_pair_offsets: bool = True) -> B2RoutedPairIndex:
    """expert -> flat pair offsets, built once per layer."""
    if topk_ids.shape != topk_weights.shape:
        raise ValueError(
            f"topk_ids and topk_weights must have identical shape, got {tuple(topk_ids.shape)} vs {tuple(topk_weights.shape)}"
        )
    if topk_ids.ndim == 0:
        raise ValueError("topk_ids must have at least one dimension")
    top_k = int(topk_ids.shape[1]) if topk_ids.ndim > 1 else 1
    if pair_offsets_by_expert is None:
        flat = topk_ids.detach().reshape(-1).cpu().tolist()
        buckets: dict[int, list[int]] = {}
        for off, e in enumerate(flat):
            if int(e) >= 0:
                buckets.setdefault(int(e), []).append(off)
        offsets = {e: tuple(v) for e, v in buckets.items()}
    else:
        offsets = {int(e): tuple(int(o) for o in v) for e, v in pair_offsets_by_expert.items() if v}
    if validate_pair_offsets:
        n = int(topk_ids.numel())
        for e, v in offsets.items():
            for o in v:
                if o < 0 or o >= n:
                    raise ValueError(f"pair offset {o} for expert {e} outside topk_ids flat size {n}")
    return B2RoutedPairIndex(topk_ids, topk_weights, int(topk_ids.shape[0]), top_k, offsets)


def build_b2_pair_microbatch_from_index(hidden_states, pair_index: B2RoutedPairIndex, logical_to_physical,
                                        wave_experts) -> B2PairMicrobatch:
    if hidden_states.shape[0] != pair_index.num_tokens:
        raise ValueError(
            f"hidden_states and routed-pair index disagree on token count, got {hidden_states.shape[0]} vs {pair_index.num_tokens}"
        )
    offs = sorted(o for e in wave_experts for o in pair_index.pair_offsets_by_expert.get(int(e), ()))
    if not offs:
        return _empty_microbatch(hidden_states, pair_index.topk_ids, pair_index.topk_weights)
    po = torch.tensor(offs, dtype=torch.long, device=pair_index.topk_ids.device)
    tok = po // pair_index.top_k
    pos = po % pair_index.top_k
    logical = pair_index.topk_ids.reshape(-1).index_select(0, po)
    physical = logical_to_physical[logical.long()]
    _validate_staged(physical, logical)
    restore = tok.to(device=hidden_states.device)
    return B2PairMicrobatch(
        hidden_states=hidden_states.index_select(0, restore).contiguous(),
        topk_ids=physical.reshape(-1, 1).contiguous(),
        topk_weights=pair_index.topk_weights[tok, pos].reshape(-1, 1).contiguous(),
        restore_token_indices=restore,
        logical_expert_ids=logical.contiguous(),
    )


def _wave_slot_table(waves, physical_slot_by_expert) -> dict[int, int]:
    """expert -> slot used by its wave: the main-bank slot when the whole wave
    is resident there, else its position inside the sorted wave (stage bank)."""
    ready = physical_slot_by_expert or {}
    table: dict[int, int] = {}
    for wave in waves:
        pure_hit = bool(ready) and all(int(e) in ready for e in wave)
        for i, e in enumerate(wave):
            table[int(e)] = int(ready[int(e)]) if pure_hit else i
    return table


def build_b2_wave_microbatch_plans(pair_index: B2RoutedPairIndex, waves, *, physical_slot_by_expert=None,
                                   **_: object) -> tuple[B2WaveMicrobatchPlan, ...]:
    """Per-wave pair lists (flat order) with their physical slots."""
    waves = tuple(tuple(int(e) for e in w) for w in waves)
    slot_of = _wave_slot_table(waves, physical_slot_by_expert)
    dev = pair_index.topk_ids.device
    plans = []
    start = 0
    for w in waves:
        offs = sorted(o for e in w for o in pair_index.pair_offsets_by_expert.get(e, ()))
        po = torch.tensor(offs, dtype=torch.long, device=dev)
        logical = pair_index.topk_ids.reshape(-1).index_select(0, po)
        slots = torch.tensor([slot_of[int(e)] for e in logical.tolist()], dtype=pair_index.topk_ids.dtype, device=dev)
        plans.append(B2WaveMicrobatchPlan(
            wave_experts=w, token_indices=po // pair_index.top_k, topk_positions=po % pair_index.top_k,
            logical_expert_ids=logical, physical_slot_ids=slots, flat_pair_offsets=po, top_k=pair_index.top_k,
            layer_pair_start=start, layer_pair_end=start + len(offs),
        ))
        start += len(offs)
    return tuple(plans)


def build_b2_pair_microbatch_from_plan(hidden_states, topk_weights, logical_to_physical, plan: B2WaveMicrobatchPlan) -> B2PairMicrobatch:
    """Materialise one wave microbatch from its plan; slots come from the plan
    (logical_to_physical is ignored when the plan carries physical ids)."""
    po = plan.pair_offsets.to(torch.long)
    tok = plan.token_indices.to(torch.long)
    slots = plan.physical_slot_ids
    if slots.numel() != po.numel() and logical_to_physical is not None:
        slots = logical_to_physical[plan.logical_expert_ids.long()]
    return B2PairMicrobatch(
        hidden_states=hidden_states.index_select(0, tok.to(hidden_states.device)).contiguous(),
        topk_ids=slots.reshape(-1, 1).contiguous(),
        topk_weights=topk_weights.reshape(-1).index_select(0, po.to(topk_weights.device)).reshape(-1, 1).contiguous(),
        restore_token_indices=tok,
        logical_expert_ids=plan.logical_expert_ids,
    )


def materialize_b2_pair_microbatches_from_plans(hidden_states, topk_weights, plans) -> tuple[B2PairMicrobatch, ...]:
    """One layer-level gather per wave plan (hidden rows, weights, slot ids)."""
    return tuple(build_b2_pair_microbatch_from_plan(hidden_states, topk_weights, None, p) for p in plans)


def build_b2_device_wave_microbatch_plans(topk_ids, waves, *, num_logical_experts: int, active_experts,
                                          physical_slot_by_expert=None, wave_pair_counts=None,
                                          include_logical_expert_ids: bool = False) -> tuple[B2WaveMicrobatchPlan, ...]:
    """Wave membership, flat offsets, tokens and slots with device tensor ops;
    only the expert->wave and expert->slot tables come from the host."""
    waves = tuple(tuple(int(e) for e in w) for w in waves)
    if not waves:
        if active_experts or int(topk_ids.numel()) != 0:
            raise ValueError("B2 waves are empty but routed experts are present")
        return ()
    E = int(num_logical_experts)
    if E <= 0:
        raise ValueError("num_logical_experts must be greater than 0")
    active = tuple(sorted({int(e) for e in active_experts}))
    bad = tuple(e for e in active if e < 0 or e >= E)
    if bad:
        raise ValueError(f"routed experts are outside the logical expert range: invalid={bad} num_logical_experts={E}")
    flat_w = tuple(e for w in waves for e in w)
    bad = tuple(e for e in flat_w if e < 0 or e >= E)
    if bad:
        raise ValueError(f"wave experts are outside the logical expert range: invalid={bad} num_logical_experts={E}")
    if len(set(flat_w)) != len(flat_w):
        raise ValueError("each active expert must appear in exactly one B2 wave")
    if set(flat_w) != set(active):
        raise ValueError(
            "B2 waves do not match the routed expert set: "
            f"missing={tuple(sorted(set(active) - set(flat_w)))} extra={tuple(sorted(set(flat_w) - set(active)))}"
        )
    sizes = tuple(int(v) for v in wave_pair_counts) if wave_pair_counts is not None else None
    if sizes is not None and len(sizes) != len(waves):
        raise ValueError("wave_pair_counts must align with waves")
    if sizes is not None and sum(sizes) != int(topk_ids.numel()):
        raise ValueError(
            f"device pair planner requires waves to cover every routed pair: planned={sum(sizes)} routed={int(topk_ids.numel())}"
        )
    top_k = int(topk_ids.shape[1]) if topk_ids.ndim > 1 else 1
    dev = topk_ids.device
    wave_of = [-1] * (E + 1)  # last entry: sentinel for invalid ids
    slot_tab = [-1] * (E + 1)
    for e, s in _wave_slot_table(waves, physical_slot_by_expert).items():
        slot_tab[e] = s
    for i, w in enumerate(waves):
        for e in w:
            wave_of[e] = i
    wave_map = torch.tensor(wave_of, dtype=torch.long, device=dev)
    slot_map = torch.tensor(slot_tab, dtype=topk_ids.dtype, device=dev)
    flat = topk_ids.reshape(-1)
    fl = flat.long()
    safe = torch.where((fl >= 0) & (fl < E), fl, torch.full_like(fl, E))
    pw = wave_map.index_select(0, safe)
    offs = tuple(torch.nonzero(pw == i, as_tuple=False).reshape(-1) for i in range(len(waves)))
    all_off = torch.cat(offs)
    actual = tuple(int(o.numel()) for o in offs)
    if int(all_off.numel()) != int(topk_ids.numel()):
        raise ValueError(
            f"device pair planner found invalid or uncovered top-k IDs: covered={int(all_off.numel())} "
            f"routed={int(topk_ids.numel())} active_experts={active}"
        )
    if sizes is not None and actual != sizes:
        raise ValueError(f"wave_pair_counts do not match current top-k contents: expected={sizes} actual={actual}")
    tokens = torch.div(all_off, top_k, rounding_mode="floor")
    slots = slot_map.index_select(0, safe.index_select(0, all_off))
    logical = flat.index_select(0, all_off) if include_logical_expert_ids else torch.empty(0, dtype=flat.dtype, device=dev)
    empty = torch.empty(0, dtype=torch.long, device=dev)
    plans = []
    cur = 0
    for w, n in zip(waves, actual):
        end = cur + n
        plans.append(B2WaveMicrobatchPlan(
            wave_experts=w, token_indices=tokens[cur:end], topk_positions=empty,
            logical_expert_ids=logical[cur:end] if include_logical_expert_ids else logical,
            physical_slot_ids=slots[cur:end], flat_pair_offsets=all_off[cur:end], top_k=top_k,
            layer_pair_start=cur, layer_pair_end=end,
        ))
        cur = end
    return tuple(plans)


# ---------------------------------------------------------------------------
# combine helpers
# ---------------------------------------------------------------------------
def scatter_add_b2_pair_output(full_output, pair_output, restore_token_indices):
    if pair_output.numel() == 0:
        return full_output
    full_output.index_add_(0, restore_token_indices.to(full_output.device),
                           pair_output.to(device=full_output.device, dtype=full_output.dtype))
    return full_output


def scatter_add_b2_pair_outputs(full_output, pair_outputs, restore_token_indices):
    if len(pair_outputs) != len(restore_token_indices):
        raise ValueError(
            f"pair_outputs and restore_token_indices must have the same length, got {len(pair_outputs)} vs {len(restore_token_indices)}"
        )
    live = [(o, i) for o, i in zip(pair_outputs, restore_token_indices) if o.numel() > 0]
    if not live:
        return full_output
    out = torch.cat([o.to(device=full_output.device, dtype=full_output.dtype) for o, _ in live])
    idx = torch.cat([i.to(full_output.device) for _, i in live])
    full_output.index_add_(0, idx, out)
    return full_output


def _weighted_rows(payload: B2DirectScatterPayload, dtype) -> torch.Tensor:
    rows = payload.expanded_row_idx.reshape(-1).abs().to(device=payload.permuted_tokens.device, dtype=torch.long)
    w = payload.topk_weights.reshape(-1).to(device=payload.permuted_tokens.device, dtype=dtype)
    return payload.permuted_tokens.index_select(0, rows).to(dtype) * w.unsqueeze(-1)


def direct_scatter_add_b2_permuted_output(full_output, *, permuted_tokens, expanded_row_idx, topk_weights,
                                          restore_token_indices, device_descriptor=None):
    """f32 alternative combine of one wave: gather by |expanded_row_idx|,
    weight, index_add into the token rows."""
    if permuted_tokens.numel() == 0:
        return full_output
    p = B2DirectScatterPayload(permuted_tokens, expanded_row_idx, topk_weights, restore_token_indices)
    full_output.index_add_(0, restore_token_indices.to(full_output.device),
                           _weighted_rows(p, full_output.dtype).to(full_output.device))
    return full_output


def direct_scatter_add_b2_permuted_outputs(full_output, payloads):
    """All waves in canonical wave order, one index_add."""
    live = sorted((p for p in payloads if p.permuted_tokens.numel() > 0), key=lambda p: int(p.wave_index))
    if not live:
        return full_output
    w = torch.cat([_weighted_rows(p, full_output.dtype).to(full_output.device) for p in live])
    idx = torch.cat([p.restore_token_indices.to(full_output.device) for p in live])
    full_output.index_add_(0, idx, w)
    return full_output


def build_b2_native_combine_inputs(payloads, *, total_pairs: int):
    """Concatenate wave outputs (wave order) and build the global unpermute
    index in original flat pair order for ONE native combine; fails closed
    unless the waves cover every pair exactly once."""
    total = int(total_pairs)
    if total < 0:
        raise ValueError("total_pairs must be non-negative")
    live = sorted((p for p in payloads if p.permuted_tokens.numel() > 0), key=lambda p: int(p.wave_index))
    if not live:
        raise ValueError("native B2 combine requires at least one non-empty wave")
    if any(p.pair_offsets is None for p in live):
        raise B2WaveFallback("native B2 combine requires original flat pair offsets for every wave")
    meta = live[0].combine_metadata
    if meta is None:
        raise B2WaveFallback("native B2 combine requires a combine metadata template")
    covered = sum(int(p.pair_offsets.numel()) for p in live)
    if covered != total:
        raise B2WaveFallback(f"B2 wave pair coverage does not match the original top-k routing: covered={covered} expected={total}")
    dev = live[0].permuted_tokens.device
    g = torch.empty(total, dtype=live[0].expanded_row_idx.dtype, device=dev)
    base = 0
    for p in live:
        po = p.pair_offsets.to(device=dev, dtype=torch.long)
        rows = p.expanded_row_idx.reshape(-1).abs().to(device=dev, dtype=g.dtype)
        if int(rows.numel()) != int(po.numel()):
            raise B2WaveFallback(f"B2 wave unpermute index does not match its routed-pair count: indices={int(rows.numel())} pairs={int(po.numel())}")
        g.index_copy_(0, po, rows + base)
        base += int(p.permuted_tokens.shape[0])
    if os.environ.get("LATCHMOE_B2_VALIDATE") or os.environ.get("SEW_B2_VALIDATE"):
        allp = torch.sort(torch.cat([p.pair_offsets.to(device=dev, dtype=torch.long) for p in live])).values
        if not torch.equal(allp, torch.arange(total, dtype=torch.long, device=dev)):
            raise B2WaveFallback("B2 waves must cover every original top-k pair exactly once")
    return torch.cat([p.permuted_tokens for p in live]), g, meta
