"""Staging controller: fixed-slot decode staging, prefill stage banks and the
compute-protected slot lifecycle, on HIP streams and events.

Decode (per offloaded layer, eager, between the captured router piece and the
captured MLP piece): de-duplicate the routed experts, let a placement-plan
provider reorder them, drain in-flight work if any slot is LOADING or
COMPUTING, then in order: a READY resident expert is a hit (touched); a miss
reserves a slot (first EMPTY, else LRU READY) and joins one async batch on the
transfer stream; the compute stream waits on the batch's event BEFORE the
persistent log2phy is updated (only changed entries are written; inactive
entries are kept).  The log2phy tensor and the slot banks never move, so a
hipGraph captured against them stays valid; their addresses are fingerprinted
at capture and re-checked before every staging.

Prefill overflow waves stage into layout-scoped double-buffered stage banks
(slot i = i-th expert of the wave), D2D from the main bank for hits and H2D
from the host store for misses, each buffer reused only after the compute
stream's release event for it.

Reference: moe_offload/runtime.py — MoeOffloadRuntime :262; register
:591-693; drain/leases :863-1108; prepare_fixed_slot_plan_into_log2phy
:1636-1936; prepare_ready_slot_plan :1938-2033; prepare_prefill_stage_plan
:2035-2258; full-layer plan :2260-2370; waits :2372-2398; stage pool
:2400-2575; stage_fixed_slot_plan / capture_safe_slot_weights / address
lock :2652-2790; full residency :2792-2862; log2phy update :3068-3101.
"""

from __future__ import annotations

import itertools
import os
import threading
from contextlib import contextmanager
from dataclasses import dataclass
from time import perf_counter

import numpy as np
import torch

from vllm_moe_offload_amd.moe_offload.config import MoeOffloadConfig
from vllm_moe_offload_amd.moe_offload.cpu_first_loader import CPU_FIRST_MARKER, is_cpu_first_layer
from vllm_moe_offload_amd.moe_offload.expert_weight_release import release_layer_original_expert_weights
from vllm_moe_offload_amd.moe_offload.expert_key import ExpertKey
from vllm_moe_offload_amd.moe_offload.host_store import HostExpertStore
from vllm_moe_offload_amd.moe_offload.placement_plan import PlacementPlanProvider, resolve_placement_plan
from vllm_moe_offload_amd.moe_offload.profile_io import append_jsonl, profile_path_from_env
from vllm_moe_offload_amd.moe_offload.slot_bank import ExpertSlotBank, SlotLease, SlotState
from vllm_moe_offload_amd.moe_offload.slot_mapping import (
    ExpertSlotMapping,
    PreparedSlotWeights,
    dedupe_preserve_order,
)
from vllm_moe_offload_amd.moe_offload.transfer_engine import TransferEngine


def _nbytes(t: torch.Tensor) -> int:
    return int(t.numel()) * int(t.element_size())


_CUDA_AVAILABLE: bool | None = None


def _cuda_available() -> bool:
    """torch.cuda.is_available(), asked once (it costs microseconds per call
    on the per-layer staging path)."""
    global _CUDA_AVAILABLE
    if _CUDA_AVAILABLE is None:
        _CUDA_AVAILABLE = bool(torch.cuda.is_available())
    return _CUDA_AVAILABLE


def _is_current_graph_capturing() -> bool:
    try:
        return bool(_cuda_available() and torch.cuda.is_current_stream_capturing())
    except Exception:
        return False


@dataclass(frozen=True)
class MoeOffloadMemoryLedger:
    registered_layers: int
    host_experts: int
    original_expert_weight_bytes: int
    host_store_bytes: int
    slot_bank_bytes: int
    prefill_stage_bank_count: int = 0
    prefill_stage_bank_bytes: int = 0
    prefill_stage_mapping_bytes: int = 0
    full_layer_prefill_bank_count: int = 0
    full_layer_prefill_bank_bytes: int = 0
    full_layer_prefill_mapping_bytes: int = 0
    pinned_shared_lane_bytes: int = 0

    @property
    def total_device_slot_bytes(self) -> int:
        return (
            self.slot_bank_bytes
            + self.pinned_shared_lane_bytes
            + self.prefill_stage_bank_bytes
            + self.prefill_stage_mapping_bytes
            + self.full_layer_prefill_bank_bytes
            + self.full_layer_prefill_mapping_bytes
        )

    # name kept for callers of the reference ledger
    total_npu_slot_bytes = total_device_slot_bytes

    @property
    def original_expert_weights_retained(self) -> bool:
        return self.original_expert_weight_bytes > 0

    def to_jsonable(self) -> dict[str, int]:
        d = {k: int(getattr(self, k)) for k in self.__dataclass_fields__}
        d["total_device_slot_bytes"] = int(self.total_device_slot_bytes)
        d["original_expert_weights_retained"] = bool(self.original_expert_weights_retained)
        return d


@dataclass(frozen=True)
class MoeExpertReleasePlan:
    """Whether original expert tensors may be dropped, and why not."""

    ready: bool
    layers_ready: tuple[int, ...]
    blockers: tuple[str, ...]


@dataclass(frozen=True)
class MoeOffloadProfileEvent:
    """One profile record (one JSONL line when a profile path is set)."""

    name: str
    layer_id: int | None
    seconds: float
    memory_ledger: MoeOffloadMemoryLedger
    payload: dict[str, object] | None = None

    def to_jsonable(self) -> dict[str, object]:
        d: dict[str, object] = {"name": self.name, "layer_id": self.layer_id, "seconds": self.seconds,
                                "memory_ledger": self.memory_ledger.to_jsonable()}
        if self.payload is not None:
            d["payload"] = self.payload
        return d


@dataclass(frozen=True)
class MoePrefillRouteStats:
    layer_id: int
    topk_cache_key: tuple
    token_counts_by_expert: dict[int, int]
    active_experts: tuple[int, ...]
    num_tokens: int
    top_k: int
    pair_offsets_by_expert: dict[int, tuple[int, ...]] | None = None


@dataclass(frozen=True)
class SlotComputeHandle:
    layer_id: int
    slot_ids: tuple[int, ...]
    leases: tuple[SlotLease, ...]


@dataclass
class PendingFixedSlotStage:
    """A decode staging whose copies are queued but not yet published."""

    layer_id: int
    active: tuple[int, ...]
    slot_ids: tuple[int, ...]
    owners: list
    ready: object | None
    hits: tuple[int, ...]
    misses: tuple[int, ...]
    log2phy: torch.Tensor
    step_id: int
    started: float
    table_updates: int = -1  # entries already written with the copies (-1: publish writes them)
    load_sync_ms: float = 0.0
    load_enqueue_ms: float = 0.0
    overflow: "DecodeOverflowStage | None" = None
    owner_updates: tuple[tuple[int, int], ...] = ()  # (slot, expert) still to write behind the table


@dataclass
class DecodeOverflowStage:
    """Routed experts of a decode step past the bank's capacity, staged into
    stage buffer `buffer_index` (slot i <- i-th expert) with the layer's own
    overflow table (expert -> stage slot, -1 elsewhere)."""

    buffer_index: int
    bank: ExpertSlotBank
    table: torch.Tensor
    experts: tuple[int, ...]
    ready: object | None


@dataclass(frozen=True)
class SlotAddressFingerprint:
    w13_data_ptr: int
    w2_data_ptr: int
    log2phy_data_ptr: int
    w13_shape: tuple[int, ...]
    w2_shape: tuple[int, ...]
    log2phy_shape: tuple[int, ...]
    device: str
    dtype: str

    def to_jsonable(self) -> dict[str, object]:
        return {k: (list(v) if isinstance(v, tuple) else v) for k, v in self.__dict__.items()}


@dataclass(frozen=True)
class FusedSharedLaneLayout:
    """Routed ids [0, routed) live in dynamic slots; shared ids follow as a
    pinned suffix of the physical bank."""

    routed_expert_count: int
    shared_expert_count: int
    pinned_logical_ids: tuple[int, ...]

    @property
    def total_logical_expert_count(self) -> int:
        return int(self.routed_expert_count + self.shared_expert_count)


class MoeOffloadRuntime:
    def __init__(self, config: MoeOffloadConfig | None = None) -> None:
        self.config = config if config is not None else MoeOffloadConfig.from_env()
        self._step_counter = itertools.count()
        self._host_store = HostExpertStore()
        self._slot_banks: dict[int, ExpertSlotBank] = {}
        self._fused_shared_lane_layouts: dict[int, FusedSharedLaneLayout] = {}
        self._prefill_stage_pool: dict[tuple, list[ExpertSlotBank]] = {}
        self._prefill_stage_banks: dict[int, list[ExpertSlotBank]] = {}
        self._prefill_stage_pool_release_events: dict[tuple, object] = {}
        self._prefill_stage_log2phy: dict[tuple, torch.Tensor] = {}
        self._full_layer_prefill_pool: dict[tuple, ExpertSlotBank] = {}
        self._full_layer_prefill_log2phy: dict[tuple, torch.Tensor] = {}
        self._original_expert_weight_bytes_by_layer: dict[int, int] = {}
        self._released_original_weight_layers: set[int] = set()
        self._expert_weight_bytes_by_layer: dict[int, int] = {}
        self._log2phy_buffers: dict[int, torch.Tensor] = {}
        # per layer: [E_total + P] int32; the first E_total entries are the
        # persistent log2phy, the last P the owner of each dynamic slot (the
        # device-side residency check: expert e is resident iff
        # owner[log2phy[e]] == e)
        self._log2phy_backing: dict[int, torch.Tensor] = {}
        self._log2phy_slot_by_expert: dict[int, dict[int, int]] = {}
        self._graph_slot_address_fingerprints: dict[int, SlotAddressFingerprint] = {}
        self._graph_slot_address_evidence: set[int] = set()
        self._slot_generation_protection_evidence: set[int] = set()
        self._transfer_engine = TransferEngine()
        self._profile_events: list[MoeOffloadProfileEvent] = []
        # JSONL destination of the profile events ("" = kept in memory only)
        self.profile_path = profile_path_from_env(self.config.profile_path)
        self._prefill_route_stats_by_layer: dict[int, MoePrefillRouteStats] = {}
        self._active_slot_ids_by_layer: dict[int, tuple[int, ...]] = {}
        self._compute_fences: dict[int, list] = {}
        # decode overflow: per-layer fixed-address tables, layers whose table
        # holds entries, and stage buffers awaiting their compute's release
        self._overflow_tables: dict[int, torch.Tensor] = {}
        self._overflow_dirty: set[int] = set()
        self._overflow_release_pending: dict[int, int] = {}
        # layers whose table holds every routed expert (static residency)
        self._full_residency_layers: set[int] = set()
        # device-planned prefill waves: plan buffers per shape, and the
        # routed-id tensors the seam handed to them (no D2H taken)
        self._device_wave_plans: dict[tuple, object] = {}
        self._device_wave_marks: dict[int, tuple] = {}
        self._layer_release_events: dict[int, object] = {}
        self._placement_plan_provider: PlacementPlanProvider | None = None
        self._fixed_slot_execution_state = threading.local()
        self._memory_ledger_cache: MoeOffloadMemoryLedger | None = None

    # ------------------------------------------------------------------ misc
    @property
    def transfer_engine(self) -> TransferEngine:
        return self._transfer_engine

    @property
    def host_store(self) -> HostExpertStore:
        return self._host_store

    def slot_bank(self, layer_id: int) -> ExpertSlotBank | None:
        return self._slot_banks.get(int(layer_id))

    def set_placement_plan_provider(self, provider: PlacementPlanProvider | None) -> None:
        """Install an external ordering provider (it never sees slot storage)."""
        self._placement_plan_provider = provider

    def next_step_id(self) -> int:
        return int(next(self._step_counter))

    def _step(self, step_id: int | None) -> int:
        return int(step_id) if step_id is not None and int(step_id) >= 0 else self.next_step_id()

    def _record_profile_event(self, name: str, *, layer_id: int | None, start: float,
                              payload: dict[str, object] | None = None) -> None:
        ev = MoeOffloadProfileEvent(name, layer_id, perf_counter() - start, self.memory_ledger(), payload)
        self._profile_events.append(ev)
        if self.profile_path:
            append_jsonl(self.profile_path, ev.to_jsonable())

    def profiling_summary(self) -> dict[str, object]:
        totals: dict[str, float] = {}
        for ev in self._profile_events:
            totals[ev.name] = totals.get(ev.name, 0.0) + ev.seconds
        return {"events": [ev.to_jsonable() for ev in self._profile_events],
                "total_seconds_by_event": totals,
                "memory_ledger": self.memory_ledger().to_jsonable()}

    def _collect_stage_profile(self, step_id: int) -> bool:
        """Decode staging events go out when a profile path (or
        LATCHMOE_PROFILE) is set, on every sample-rate-th step."""
        if not (self.profile_path or os.environ.get("LATCHMOE_PROFILE")):
            return False
        rate = _decode_profile_sample_rate()
        return rate <= 1 or int(step_id) % rate == 0

    # --------------------------------------------------------- predicates
    @property
    def should_use_fixed_slots(self) -> bool:
        return self.config.enabled and not self.config.trace_only and self.config.num_slots > 0

    def is_resident_layer(self, layer_id: int) -> bool:
        return self.config.is_resident_layer(int(layer_id))

    @contextmanager
    def suspend_fixed_slot_execution(self):
        """Temporarily route the current thread through the native path."""
        st = self._fixed_slot_execution_state
        depth = int(getattr(st, "suspend_depth", 0))
        st.suspend_depth = depth + 1
        try:
            yield
        finally:
            st.suspend_depth = depth

    def should_use_fixed_slot_plan_for_layer(self, layer_id: int) -> bool:
        if int(getattr(self._fixed_slot_execution_state, "suspend_depth", 0)) > 0:
            return False
        return self.should_use_fixed_slots and not self.is_resident_layer(int(layer_id))

    def is_static_residency_regime(self, num_logical_experts: int) -> bool:
        """Regime A: every routed expert owns a slot, log2phy never changes."""
        return int(self.config.num_slots) >= int(num_logical_experts)

    def is_static_residency_regime_for_layer(self, *, layer_id: int, fallback_routed_expert_count: int) -> bool:
        return self.is_static_residency_regime(
            self.routed_expert_count_for_layer(layer_id=layer_id, fallback=fallback_routed_expert_count)
        )

    def should_use_b2_wave_prefill(self, *, layer_id: int, active_expert_count: int, is_prefill: bool) -> bool:
        if not self.config.b2_wave_prefill or not is_prefill:
            return False
        if not self.should_use_fixed_slot_plan_for_layer(int(layer_id)):
            return False
        return int(active_expert_count) > int(self.config.num_slots)

    def should_use_b2_pair_waves(self, *, layer_id: int, active_expert_count: int) -> bool:
        if not self.config.b2_wave_prefill:
            return False
        if not self.should_use_fixed_slot_plan_for_layer(int(layer_id)):
            return False
        return int(active_expert_count) > int(self.config.num_slots)

    def is_layer_registered(self, layer_id: int) -> bool:
        return int(layer_id) in self._slot_banks

    def check_device_flags(self, *, layer_id: int | None = None) -> None:
        """Fail closed on the device status words of the native library
        (pairs a masked combine dropped because no pass placed them, one-launch
        router waits that gave up): either means an output since the last
        check is invalid.  The words are read and cleared with one small
        synchronizing copy per kernel unit, so callers make this check where
        the host already waits; with layer_id given it runs only for the
        lowest registered layer, i.e. once per forward pass."""
        if layer_id is not None and self._slot_banks and int(layer_id) != min(self._slot_banks):
            return
        if not torch.cuda.is_available():
            return
        from vllm_moe_offload_amd import native

        flags = native.device_flags(clear=True)
        unplaced, timeouts = flags[native.FLAG_UNPLACED], flags[native.FLAG_ROUTER_TIMEOUT]
        if unplaced or timeouts:
            raise RuntimeError(
                "MoE outputs since the last device check are invalid: "
                f"{unplaced} routed pairs were placed in no slot or wave, "
                f"{timeouts} one-launch router waits gave up")

    def fused_shared_lane_layout(self, layer_id: int) -> FusedSharedLaneLayout | None:
        return self._fused_shared_lane_layouts.get(int(layer_id))

    def routed_expert_count_for_layer(self, *, layer_id: int, fallback: int) -> int:
        lay = self.fused_shared_lane_layout(layer_id)
        return int(lay.routed_expert_count) if lay is not None else int(fallback)

    def total_logical_expert_count_for_layer(self, *, layer_id: int, fallback: int) -> int:
        lay = self.fused_shared_lane_layout(layer_id)
        return int(lay.total_logical_expert_count) if lay is not None else int(fallback)

    def _resolve_fused_shared_counts(self, *, layer_id: int, requested_logical_expert_count: int) -> tuple[int, int]:
        req = int(requested_logical_expert_count)
        lay = self.fused_shared_lane_layout(layer_id)
        if lay is None:
            return req, req
        routed, total = int(lay.routed_expert_count), int(lay.total_logical_expert_count)
        if req not in (routed, total):
            raise RuntimeError(
                f"fused shared lane logical count mismatch: layer={int(layer_id)} requested={req} "
                f"routed={routed} total={total}"
            )
        return routed, total

    # --------------------------------------------------------- registration
    def register_layer_for_fixed_slots(self, layer: torch.nn.Module, *, slot_device: torch.device | None = None) -> None:
        """Host-store the routed experts, build the slot bank and log2phy."""
        layer_id = int(getattr(layer, "layer_id", -1))
        if layer_id < 0:
            raise ValueError("layer.layer_id is required for fixed-slot registration")
        if layer_id in self._graph_slot_address_fingerprints:
            raise RuntimeError(
                f"layer {layer_id} fixed-slot addresses are already captured; "
                "re-registering would invalidate a graph replay"
            )
        start = perf_counter()
        w13, w2 = layer.w13_weight, layer.w2_weight
        if int(w13.shape[0]) != int(w2.shape[0]):
            raise ValueError("w13_weight and w2_weight must have the same number of experts")
        total = int(w13.shape[0])
        shared = int(getattr(layer, "n_shared_experts", 0) or 0) if bool(getattr(layer, "mix_placement", False)) else 0
        if shared > total:
            raise ValueError(f"fused shared expert count exceeds materialized expert rows: shared={shared}, total={total}")
        routed = total - shared
        if routed <= 0:
            raise ValueError(f"fused mix-placement requires at least one routed expert; total={total}, shared={shared}")
        pinned_ids = tuple(range(routed, total))
        report = self._host_store.register_layer(
            layer,
            pin_memory=self.config.should_pin_host_memory,
            clone_tensors=not is_cpu_first_layer(layer),
            routed_expert_count=routed,
        )
        self._original_expert_weight_bytes_by_layer[layer_id] = _nbytes(w13) + _nbytes(w2)
        self._released_original_weight_layers.discard(layer_id)
        self._expert_weight_bytes_by_layer[layer_id] = _nbytes(w13[0]) + _nbytes(w2[0])
        device = slot_device if slot_device is not None else w13.device
        bank = ExpertSlotBank(
            self.config.num_slots,
            tuple(int(d) for d in w13.shape[1:]),
            tuple(int(d) for d in w2.shape[1:]),
            dtype=w13.dtype,
            device=device,
            pinned_logical_ids=pinned_ids,
        )
        self._slot_banks[layer_id] = bank
        if pinned_ids:
            bank.install_pinned_weights(w13[routed:], w2[routed:])
            self._fused_shared_lane_layouts[layer_id] = FusedSharedLaneLayout(routed, shared, pinned_ids)
        else:
            self._fused_shared_lane_layouts.pop(layer_id, None)
        self._prefill_stage_banks.pop(layer_id, None)
        table = self._new_log2phy(layer_id, total, bank.num_dynamic_slots, device)
        bank.install_pinned_log2phy(table)
        self._log2phy_slot_by_expert[layer_id] = {}
        self._full_residency_layers.discard(layer_id)
        self._memory_ledger_cache = None
        self._record_profile_event(
            "register_layer_for_fixed_slots",
            layer_id=layer_id,
            start=start,
            payload={
                "host_store": report.to_jsonable(),
                "routed_expert_count": routed,
                "pinned_shared_expert_count": shared,
                "pinned_shared_logical_ids": list(pinned_ids),
            },
        )

    def register_host_buffers(self, *, layer_id: int, w13_host: torch.Tensor, w2_host: torch.Tensor,
                              slot_device: torch.device, shared_w13: torch.Tensor | None = None,
                              shared_w2: torch.Tensor | None = None) -> None:
        """Register a layer whose routed experts already sit in host buffers
        ([E, 2I, H] / [E, H, I], ideally page-locked): no device copy of the
        full layer is ever made, the buffers become the host store as they are
        (the CPU-first loading path, cpu_first_loader.py:40-177).  shared_w13 /
        shared_w2 ([S, 2I, H] / [S, H, I], any device) are fused shared
        experts: pinned suffix rows of the slot bank with logical ids
        E .. E+S-1, as a mix-placement layer registers them
        (slot_bank.py:98-115)."""
        layer_id = int(layer_id)
        if layer_id in self._graph_slot_address_fingerprints:
            raise RuntimeError(f"layer {layer_id} fixed-slot addresses are already captured")
        if (shared_w13 is None) != (shared_w2 is None):
            raise ValueError("shared_w13 and shared_w2 go together")
        holder = torch.nn.Module()
        holder.layer_id = layer_id
        holder.w13_weight = w13_host
        holder.w2_weight = w2_host
        setattr(holder, CPU_FIRST_MARKER, True)
        E = int(w13_host.shape[0])
        S = 0 if shared_w13 is None else int(shared_w13.shape[0])
        if S and (tuple(shared_w13.shape[1:]) != tuple(w13_host.shape[1:]) or
                  tuple(shared_w2.shape[1:]) != tuple(w2_host.shape[1:]) or int(shared_w2.shape[0]) != S):
            raise ValueError("fused shared experts must have the routed experts' shape")
        self._host_store.register_layer(holder, pin_memory=False, clone_tensors=False, routed_expert_count=E)
        self._original_expert_weight_bytes_by_layer[layer_id] = 0
        self._released_original_weight_layers.discard(layer_id)
        self._expert_weight_bytes_by_layer[layer_id] = _nbytes(w13_host[0]) + _nbytes(w2_host[0])
        pinned_ids = tuple(range(E, E + S))
        bank = ExpertSlotBank(self.config.num_slots, tuple(int(d) for d in w13_host.shape[1:]),
                              tuple(int(d) for d in w2_host.shape[1:]), dtype=w13_host.dtype, device=slot_device,
                              pinned_logical_ids=pinned_ids)
        self._slot_banks[layer_id] = bank
        if pinned_ids:
            bank.install_pinned_weights(shared_w13, shared_w2)
            self._fused_shared_lane_layouts[layer_id] = FusedSharedLaneLayout(E, S, pinned_ids)
        else:
            self._fused_shared_lane_layouts.pop(layer_id, None)
        self._prefill_stage_banks.pop(layer_id, None)
        table = self._new_log2phy(layer_id, E + S, bank.num_dynamic_slots, slot_device)
        if pinned_ids:
            bank.install_pinned_log2phy(table)
        self._log2phy_slot_by_expert[layer_id] = {}
        self._full_residency_layers.discard(layer_id)
        self._memory_ledger_cache = None

    # ----------------------------------------------------------- queries
    def slot_readiness_and_ready_slot_ids_for_experts(self, *, layer_id: int, expert_ids) -> tuple[dict[int, bool], dict[int, int]]:
        bank = self._slot_banks.get(int(layer_id))
        if bank is None:
            return {int(e): False for e in expert_ids}, {}
        ready: dict[int, bool] = {}
        ids: dict[int, int] = {}
        for e in expert_ids:
            slot = bank.lookup_expert_id(int(e))
            ok = slot is not None and slot.state == SlotState.READY
            ready[int(e)] = ok
            if ok:
                ids[int(e)] = int(slot.slot_id)
        return ready, ids

    def slot_readiness_for_experts(self, *, layer_id: int, expert_ids) -> dict[int, bool]:
        return self.slot_readiness_and_ready_slot_ids_for_experts(layer_id=layer_id, expert_ids=expert_ids)[0]

    def ready_slot_ids_for_experts(self, *, layer_id: int, expert_ids) -> dict[int, int]:
        return self.slot_readiness_and_ready_slot_ids_for_experts(layer_id=layer_id, expert_ids=expert_ids)[1]

    def estimate_expert_weight_bytes(self, *, layer_id: int, expert_id: int) -> int:
        return int(self._host_store.get(int(layer_id), int(expert_id)).nbytes)

    def cached_layer_expert_weight_bytes(self, *, layer_id: int) -> int:
        return int(self._expert_weight_bytes_by_layer.get(int(layer_id), 0))

    def log2phy_buffer(self, layer_id: int) -> torch.Tensor | None:
        """The persistent, fixed-address log2phy table of a layer."""
        return self._log2phy_buffers.get(int(layer_id))

    def slot_owner_buffer(self, layer_id: int) -> torch.Tensor | None:
        """Device copy of the owner of each dynamic slot of a layer (-1 none),
        written with the copies that change it."""
        b = self._log2phy_backing.get(int(layer_id))
        t = self._log2phy_buffers.get(int(layer_id))
        return None if b is None or t is None else b[int(t.numel()):]

    def _new_log2phy(self, layer_id: int, total: int, n_slots: int, device) -> torch.Tensor:
        backing = torch.full((int(total) + int(n_slots),), -1, dtype=torch.int32, device=device)
        self._log2phy_backing[int(layer_id)] = backing
        table = backing[: int(total)]
        self._log2phy_buffers[int(layer_id)] = table
        return table

    def _owner_entries(self, layer_id: int, owner_updates) -> tuple[tuple[int, ...], tuple[int, ...]]:
        """(index into the backing tensor, expert) of slot-owner changes."""
        base = int(self._log2phy_buffers[int(layer_id)].numel())
        return tuple(base + s for s, _ in owner_updates), tuple(e for _, e in owner_updates)

    # ------------------------------------------- original weight release
    def original_expert_weights_available_for_layer(self, layer_id: int) -> bool:
        return int(layer_id) not in self._released_original_weight_layers

    def plan_original_weight_release(self, *, expected_layer_ids, default_path_preserved: bool,
                                     host_store_is_complete: bool | None = None,
                                     allow_retained_original_weights: bool = False) -> MoeExpertReleasePlan:
        """Blockers to dropping the original expert tensors of the given
        layers: unregistered layers, an incomplete host store, a default path
        that needs them, or (unless allowed) original tensors still counted."""
        ids = tuple(int(i) for i in expected_layer_ids)
        blockers: list[str] = []
        if not ids:
            blockers.append("no_expected_layers")
        missing = [i for i in ids if i not in self._slot_banks]
        if missing:
            blockers.append(f"layers_not_registered:{missing}")
        if not default_path_preserved:
            blockers.append("default_path_not_preserved")
        if host_store_is_complete is False:
            blockers.append("host_store_not_marked_complete")
        blockers.extend(self._host_store.validate_complete_layers(ids).blockers)
        if self.memory_ledger().original_expert_weights_retained and not allow_retained_original_weights:
            blockers.append("original_expert_weights_still_retained")
        return MoeExpertReleasePlan(not blockers, () if blockers else ids, tuple(blockers))

    def release_original_expert_weights_if_ready(self, layer: torch.nn.Module, *,
                                                 default_path_preserved: bool = True) -> MoeExpertReleasePlan:
        """Drop one offloaded layer's original w13/w2 once its host store is
        complete (opt-in by release_original_expert_weights).  Idempotent."""
        def blocked(reason: str) -> MoeExpertReleasePlan:
            return MoeExpertReleasePlan(False, (), (reason,))

        if not self.config.release_original_expert_weights:
            return blocked("release_original_expert_weights_disabled")
        if not self.should_use_fixed_slots:
            return blocked("fixed_slots_disabled")
        layer_id = int(getattr(layer, "layer_id", -1))
        if layer_id < 0:
            return blocked("invalid_layer_id")
        if self.is_resident_layer(layer_id):
            return blocked(f"resident_layer:{layer_id}")
        if layer_id in self._released_original_weight_layers:
            return MoeExpertReleasePlan(True, (layer_id,), ())
        plan = self.plan_original_weight_release(expected_layer_ids=(layer_id,),
                                                 default_path_preserved=default_path_preserved,
                                                 allow_retained_original_weights=True)
        if not plan.ready:
            return plan
        start = perf_counter()
        freed = release_layer_original_expert_weights(layer)
        self._released_original_weight_layers.add(layer_id)
        self._original_expert_weight_bytes_by_layer[layer_id] = 0
        self._memory_ledger_cache = None
        self._record_profile_event("release_original_expert_weights", layer_id=layer_id, start=start,
                                   payload={"released_bytes": int(freed)})
        return MoeExpertReleasePlan(True, (layer_id,), ())

    # ------------------------------------------------------ memory ledger
    def memory_ledger(self) -> MoeOffloadMemoryLedger:
        if self._memory_ledger_cache is not None:
            return self._memory_ledger_cache
        stage_banks = {id(b): b for banks in self._prefill_stage_pool.values() for b in banks}
        full_banks = {id(b): b for b in self._full_layer_prefill_pool.values()}
        ledger = MoeOffloadMemoryLedger(
            registered_layers=len(self._slot_banks),
            host_experts=len(self._host_store),
            original_expert_weight_bytes=sum(self._original_expert_weight_bytes_by_layer.values()),
            host_store_bytes=int(self._host_store.total_bytes),
            slot_bank_bytes=sum(b.dynamic_bytes for b in self._slot_banks.values()),
            prefill_stage_bank_count=len(stage_banks),
            prefill_stage_bank_bytes=sum(b.total_bytes for b in stage_banks.values()),
            prefill_stage_mapping_bytes=sum(_nbytes(t) for t in self._prefill_stage_log2phy.values()),
            full_layer_prefill_bank_count=len(full_banks),
            full_layer_prefill_bank_bytes=sum(b.total_bytes for b in full_banks.values()),
            full_layer_prefill_mapping_bytes=sum(_nbytes(t) for t in self._full_layer_prefill_log2phy.values()),
            pinned_shared_lane_bytes=sum(b.pinned_bytes for b in self._slot_banks.values()),
        )
        self._memory_ledger_cache = ledger
        return ledger

    # ----------------------------------------------------- slot lifecycle
    # Compute fences: per layer, the events that end queued compute reading
    # the main bank, each with the (slot, version) generations it covers.  A
    # COMPUTING slot is released (READY) only once a fence covering its
    # current generation has completed; a slot whose generation moved on
    # while its compute was in flight is an error.
    def _note_compute_fence(self, layer_id: int, generations, event) -> None:
        self._compute_fences.setdefault(int(layer_id), []).append(
            (event, tuple((int(s), int(v)) for s, v in generations)))

    def _take_fences(self, layer_id: int, generations) -> list:
        """Remove and return the fences covering these (slot, version)
        generations; raise for a generation no fence covers."""
        fences = self._compute_fences.get(int(layer_id), [])
        wanted = set(generations)
        covered: set = set()
        taken, kept = [], []
        for ev, gens in fences:
            hit = wanted.intersection(gens)
            if hit:
                taken.append(ev)
                covered |= hit
                rest = tuple(g for g in gens if g not in wanted)
                if rest:
                    kept.append((ev, rest))
            else:
                kept.append((ev, gens))
        missing = sorted(wanted - covered)
        if missing:
            s, v = missing[0]
            raise RuntimeError(f"computing slot has no completion event: layer={int(layer_id)} slot={s} version={v}")
        self._compute_fences[int(layer_id)] = kept
        return list({id(e): e for e in taken}.values())

    def _allocate_slot_with_loading_fallback(self, bank: ExpertSlotBank, key: ExpertKey, *, step_id: int):
        try:
            return bank.allocate_for(key, step_id=step_id)
        except RuntimeError:
            if not bank.has_inflight():
                raise
            self._drain_slot_bank_inflight_work(bank)
            return bank.allocate_for(key, step_id=step_id)

    def _drain_slot_bank_inflight_work(self, bank: ExpertSlotBank) -> None:
        """Finish every in-flight copy into the bank and every queued compute
        reading it, then release the computing slots."""
        from vllm_moe_offload_amd.moe_offload.slot_bank import COMPUTING, LOADING

        if (bank._state == LOADING).any():
            self._transfer_engine.synchronize()
            still = np.flatnonzero(bank._state == LOADING).tolist()
            if still:
                raise RuntimeError(f"H2D synchronization completed without a matching ready event for slots {still}")
        comp = np.flatnonzero(bank._state == COMPUTING)
        if comp.size == 0:
            return
        layer_id = int(bank._owner_layer[comp[0]])
        gens = [(int(s), int(bank._version[s])) for s in comp]
        owners = [int(bank._owner[s]) for s in comp]
        events = self._take_fences(layer_id, gens)
        for ev in events:
            _synchronize_event(ev)
        for (sid, ver), e in zip(gens, owners):
            if int(bank._version[sid]) != ver or int(bank._owner[sid]) != e:
                raise RuntimeError(f"slot {sid} ownership changed while compute was in flight")
            if int(bank._state[sid]) == COMPUTING:
                bank.mark_ready(sid)
        if layer_id not in self._slot_generation_protection_evidence:
            self._slot_generation_protection_evidence.add(layer_id)
            self._record_profile_event(
                "slot_generation_protected_until_compute_complete",
                layer_id=layer_id,
                start=perf_counter(),
                payload={
                    "slot_ids": [g[0] for g in gens],
                    "generations": [g[1] for g in gens],
                    "expert_ids": owners,
                    "completion_events_synchronized": len(events),
                    "leases_still_match": True,
                },
            )

    @staticmethod
    def _release_allocated_loads(bank: ExpertSlotBank, loads) -> None:
        for _, slot in loads:
            if getattr(slot, "state", None) == SlotState.LOADING:
                bank.clear_slot(int(slot.slot_id), force=True)

    def begin_slot_compute(self, prepared: PreparedSlotWeights) -> SlotComputeHandle | None:
        """Mark the main-bank slots of a plan COMPUTING while kernels read them."""
        layer_id = int(prepared.mapping.layer_id)
        bank = self._slot_banks.get(layer_id)
        if bank is None or prepared.w1.data_ptr() != bank.w13_slots.data_ptr():
            return None
        slot_ids = tuple(sorted({int(s) for s in prepared.mapping.active_slot_ids}))
        if not slot_ids:
            slot_ids = tuple(int(s) for s in self._active_slot_ids_by_layer.get(layer_id, ()))
        if not slot_ids:
            return None
        owners = prepared.mapping.slot_to_expert
        if _is_current_graph_capturing():
            # the capture follows the preceding eager compute in stream order:
            # its fences are handed over, the host does not wait inside capture
            busy = [sid for sid in slot_ids if bank.slots[sid].state == SlotState.COMPUTING]
            if busy:
                try:
                    self._take_fences(layer_id, [(sid, bank.slots[sid].version) for sid in busy])
                except RuntimeError as exc:
                    raise RuntimeError(
                        "capturing slot has no completion event from the preceding eager compute: "
                        f"{str(exc).split(': ', 1)[-1]}"
                    ) from exc
                for sid in busy:
                    bank.mark_ready(sid)
        leases = []
        for sid in slot_ids:
            if sid >= len(owners):
                raise RuntimeError(f"prepared slot mapping has no owner entry for slot {sid}")
            slot = bank.slots[sid]
            want = ExpertKey(layer_id, int(owners[sid])) if owners[sid] is not None else None
            if slot.expert_key != want:
                raise RuntimeError(f"prepared mapping owner mismatch for slot {sid}: expected {want}, found {slot.expert_key}")
            if slot.state != SlotState.READY:
                raise RuntimeError(f"prepared slot {sid} is not ready for compute: {slot.state.value}")
            leases.append(slot.lease())
        for sid in slot_ids:
            bank.mark_computing(sid)
        return SlotComputeHandle(layer_id, slot_ids, tuple(leases))

    def end_slot_compute(self, handle: SlotComputeHandle | None) -> None:
        """Fence the leased slots with an event at the end of the queued
        compute (host-only banks: released at once)."""
        if handle is None:
            return
        bank = self._slot_banks.get(int(handle.layer_id))
        if bank is None:
            return
        for lease in handle.leases:
            slot = bank.slots[int(lease.slot_id)]
            if not slot.matches_lease(lease):
                raise RuntimeError(f"slot {lease.slot_id} ownership changed before compute completed")
            if slot.state != SlotState.COMPUTING:
                raise RuntimeError(f"slot {lease.slot_id} is not computing at compute completion: {slot.state.value}")
        ev = self._record_current_stream_event_or_none()
        if ev is None:
            for lease in handle.leases:
                bank.mark_ready(int(lease.slot_id))
            return
        self._layer_release_events[int(handle.layer_id)] = ev
        self._note_compute_fence(handle.layer_id, [(l.slot_id, l.version) for l in handle.leases], ev)

    def record_layer_compute(self, layer_id: int) -> None:
        """Record, on the current stream, the end of compute the caller has
        queued that reads this layer's slot bank (e.g. a graph replay, which
        bypasses begin/end_slot_compute).  The next miss copies into the bank
        wait for it on the GPU, so no slot still read by that compute is
        overwritten."""
        ev = self._record_current_stream_event_or_none()
        if ev is not None:
            self._layer_release_events[int(layer_id)] = ev
        self.end_overflow_compute(int(layer_id))

    # ------------------------------------------------------ decode staging
    def _compute_device_index(self) -> int | None:
        """Device index of the first device slot bank (None: host-only banks).
        Passing it to current_stream() skips torch's device lookup."""
        for b in self._slot_banks.values():
            if b.w13_slots.device.type == "cuda":
                idx = b.w13_slots.device.index
                return int(idx) if idx is not None else int(torch.cuda.current_device())
        return None

    def _consumer_stream(self):
        """The current stream of the slot banks' device (a no-op stream for
        host-only banks)."""
        idx = self._compute_device_index()
        return _NullStream() if idx is None else torch.cuda.current_stream(idx)

    def _record_current_stream_event_or_none(self):
        """Completion event of the compute stream (None for host-only banks)."""
        idx = self._compute_device_index()
        if idx is None:
            return None
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(idx))
        return ev

    def prepare_fixed_slot_plan(self, *, layer_id: int, active_experts, num_logical_experts: int,
                                device: torch.device | None = None, step_id: int | None = None,
                                record_stage_profile: bool = False) -> PreparedSlotWeights:
        """Stage into the main bank and return a mapping in a fresh log2phy."""
        bank = self._slot_banks.get(int(layer_id))
        if bank is None:
            raise RuntimeError(f"layer {layer_id} is not registered for fixed-slot execution")
        _, total = self._resolve_fused_shared_counts(layer_id=layer_id, requested_logical_expert_count=num_logical_experts)
        table = torch.full((total,), -1, dtype=torch.int32, device=device if device is not None else bank.w13_slots.device)
        bank.install_pinned_log2phy(table)
        saved = self._log2phy_slot_by_expert.get(int(layer_id))
        self._log2phy_slot_by_expert[int(layer_id)] = {}
        try:
            return self.prepare_fixed_slot_plan_into_log2phy(
                layer_id=layer_id, active_experts=active_experts, num_logical_experts=num_logical_experts,
                log2phy=table, step_id=step_id, record_stage_profile=record_stage_profile,
            )
        finally:
            self._log2phy_slot_by_expert[int(layer_id)] = saved if saved is not None else {}

    def prepare_fixed_slot_plan_into_log2phy(self, *, layer_id: int, active_experts, num_logical_experts: int,
                                             log2phy: torch.Tensor, step_id: int | None = None,
                                             record_stage_profile: bool = False) -> PreparedSlotWeights:
        """Decode hot path: hit/miss, one async H2D batch, consumer wait, then
        an in-place update of the changed log2phy entries."""
        pending = self._reserve_and_issue(layer_id=layer_id, active_experts=active_experts,
                                          num_logical_experts=num_logical_experts, log2phy=log2phy, step_id=step_id)
        return self._publish(pending, record_stage_profile=record_stage_profile)

    def prefetch_fixed_slot_plan(self, *, layer_id: int, active_experts, num_logical_experts: int,
                                 token_counts: dict[int, int] | None = None) -> PendingFixedSlotStage:
        """Reserve slots and queue the miss copies on the transfer stream now;
        publish later with complete_fixed_slot_plan (after the previous layer's
        kernels are queued), so the copies overlap that compute."""
        if _is_current_graph_capturing():
            raise RuntimeError("prefetch_fixed_slot_plan must run eager (outside graph capture)")
        active = resolve_placement_plan(
            self._placement_plan_provider, layer_id=int(layer_id),
            routed_experts=tuple(int(e) for e in active_experts), num_logical_experts=int(num_logical_experts),
        )
        self._assert_locked_slot_addresses(int(layer_id))
        return self._reserve_and_issue(layer_id=layer_id, active_experts=active, num_logical_experts=num_logical_experts,
                                       log2phy=self._log2phy_buffers[int(layer_id)], step_id=None,
                                       token_counts=token_counts)

    def complete_fixed_slot_plan(self, pending: PendingFixedSlotStage) -> PreparedSlotWeights:
        """Order the prefetched copies before the current stream, then publish."""
        return self._publish(pending, record_stage_profile=True)

    def _reserve_and_issue(self, *, layer_id: int, active_experts, num_logical_experts: int, log2phy: torch.Tensor,
                           step_id: int | None, token_counts: dict[int, int] | None = None) -> PendingFixedSlotStage:
        if not self.should_use_fixed_slots:
            raise RuntimeError("fixed-slot plan requested while moe offload fixed slots are disabled")
        layer_id = int(layer_id)
        if self.is_resident_layer(layer_id):
            raise RuntimeError(f"fixed-slot plan must not run on resident layer {layer_id}; use the original expert weights")
        routed, total = self._resolve_fused_shared_counts(layer_id=layer_id, requested_logical_expert_count=num_logical_experts)
        active = dedupe_preserve_order(active_experts)
        _validate_active_expert_ids(layer_id=layer_id, active_experts=active, num_logical_experts=routed)
        overflowing = len(active) > self.config.num_slots
        if overflowing and not self.can_stage_decode_overflow(layer_id=layer_id, active_expert_count=len(active)):
            raise RuntimeError(f"active expert working set size {len(active)} exceeds num_slots={self.config.num_slots}")
        if int(log2phy.numel()) != total:
            raise RuntimeError(f"log2phy buffer for layer {layer_id} has size {int(log2phy.numel())}, expected {total}")
        bank = self._slot_banks.get(layer_id)
        if bank is None:
            raise RuntimeError(f"layer {layer_id} is not registered for fixed-slot execution")
        if bank.has_inflight():
            self._drain_slot_bank_inflight_work(bank)
        step_id = self._step(step_id)
        t0 = perf_counter()
        over: tuple[int, ...] = ()
        if overflowing:
            active, over = _split_decode_overflow(bank, active, int(self.config.num_slots), token_counts)
        ids = np.fromiter(active, dtype=np.int32, count=len(active))
        # one native call plans every expert (hit: touch; miss: reserve a
        # slot, LOADING); it stops where in-flight work must finish first
        st, slot_ids, miss = bank.plan(layer_id, ids, step_id=step_id)
        base = 0
        while st < 0:
            j = base + (-st - 1)  # the expert the plan stopped at
            if not bank.has_inflight():
                self._raise_no_slot(layer_id, int(ids[j]), bank)
            self._drain_slot_bank_inflight_work(bank)
            st, rest_ids, rest_miss = bank.plan(layer_id, ids[j:], step_id=step_id)
            slot_ids[j:], miss[j:] = rest_ids, rest_miss
            if st == -1:  # stopped at the same expert with nothing left to wait for
                self._raise_no_slot(layer_id, int(ids[j]), bank)
            base = j
        slot_list = [int(v) for v in slot_ids]
        is_miss = miss.astype(bool)
        hits = tuple(int(e) for e in ids[~is_miss])
        misses = tuple(int(e) for e in ids[is_miss])
        loads = [(self._host_store.get(layer_id, e), bank.slots[sid])
                 for e, sid in zip(misses, (v for v, m in zip(slot_list, is_miss) if m))]
        ready = None
        table_updates = -1
        # overflow experts map to no slot (the second pass covers them), so a
        # stale entry of theirs cannot catch their pairs in the bank pass;
        # the slot owners behind the table (device residency) follow the misses
        tab_e, tab_s = tuple(active) + over, slot_list + [-1] * len(over)
        owner_upd = tuple((int(s_), int(e)) for e, s_, m in zip(ids, slot_list, is_miss) if m)
        t_load = perf_counter()
        load_sync_ms = load_enqueue_ms = 0.0
        if loads and not self.config.async_load:
            try:
                self._transfer_engine.load_many_sync(loads, validate_layout=False)
            except Exception:
                self._release_allocated_loads(bank, loads)
                raise
            load_sync_ms = (perf_counter() - t_load) * 1000.0
        elif loads:
            # device bank and table: the changed log2phy entries ride with the
            # copies on the transfer stream, inside their ready event
            with_table = log2phy.device.type == "cuda" and bank.w13_slots.device.type == "cuda"
            upd = self._changed_log2phy_entries(layer_id=layer_id, expert_ids=tab_e, slot_ids=tab_s) \
                if with_table else ((), ())
            persistent = log2phy.data_ptr() == self._log2phy_backing[layer_id].data_ptr()
            own = self._owner_entries(layer_id, owner_upd) if with_table and persistent else ((), ())
            extra = {}
            if own[0]:
                extra = {"table_update": (self._log2phy_backing[layer_id], upd[0] + own[0], upd[1] + own[1])}
            elif upd[0]:
                extra = {"table_update": (log2phy, upd[0], upd[1])}
            try:
                ready = self._transfer_engine.load_many_async(
                    loads, wait_event=self._layer_release_events.get(layer_id), record_event=True,
                    validate_layout=False, **extra,
                )
            except Exception:
                self._release_allocated_loads(bank, loads)
                raise
            if with_table:
                self._remember_log2phy_entries(layer_id=layer_id, expert_ids=upd[0], slot_ids=upd[1])
                table_updates = len(upd[0])
                if not persistent:  # a fresh table: the owners follow on the transfer stream
                    self._write_owner_entries(layer_id, owner_upd, stream=self._transfer_engine.stream)
                owner_upd = ()
            load_enqueue_ms = (perf_counter() - t_load) * 1000.0
        ovf = self._issue_decode_overflow(layer_id=layer_id, experts=over, total=total, step_id=step_id) \
            if over else None
        return PendingFixedSlotStage(layer_id, active, tuple(slot_list), bank.owners(), ready, hits, misses + over,
                                     log2phy, step_id, t0, table_updates, load_sync_ms, load_enqueue_ms, ovf,
                                     owner_upd)

    # ----------------------------------------------------- decode overflow
    def can_stage_decode_overflow(self, *, layer_id: int, active_expert_count: int) -> bool:
        """A decode working set past the bank fits one overflow pass: at most
        num_slots more experts, from the layer's stage buffer."""
        if not (self.config.decode_overflow and self.should_use_fixed_slot_plan_for_layer(int(layer_id))):
            return False
        n, P = int(active_expert_count), int(self.config.num_slots)
        return P < n <= 2 * P

    def decode_overflow_buffer_index(self, layer_id: int) -> int:
        """Stage buffer of a layer's overflow pass: fixed per layer (a captured
        graph records its address), alternating between neighbours so one
        layer's copies overlap the previous layer's compute."""
        return int(layer_id) % self.config.effective_prefill_buffer_count

    def _overflow_table(self, layer_id: int, total: int, device) -> torch.Tensor:
        t = self._overflow_tables.get(int(layer_id))
        if t is None or int(t.numel()) != int(total):
            t = torch.full((int(total),), -1, dtype=torch.int32, device=device)
            self._overflow_tables[int(layer_id)] = t
            self._memory_ledger_cache = None
        return t

    def decode_overflow_slot_weights(self, *, layer_id: int, n_pairs: int | None = None) -> PreparedSlotWeights | None:
        """The second pass's weights of a layer: its stage buffer and its
        overflow table, fixed addresses (what an eager call or a captured graph
        reads).  None when overflow is off or when n_pairs routed pairs cannot
        exceed the slots."""
        layer_id = int(layer_id)
        P = int(self.config.num_slots)
        if not (self.config.decode_overflow and self.should_use_fixed_slot_plan_for_layer(layer_id)):
            return None
        if n_pairs is not None and int(n_pairs) <= P:
            return None
        src = self._slot_banks.get(layer_id)
        if src is None:
            return None
        _, total = self._resolve_fused_shared_counts(
            layer_id=layer_id, requested_logical_expert_count=int(self._log2phy_buffers[layer_id].numel()))
        buf = self.decode_overflow_buffer_index(layer_id)
        stage = self._get_prefill_stage_bank(layer_id=layer_id, buffer_index=buf, template_bank=src)
        table = self._overflow_table(layer_id, total, src.w13_slots.device)
        mapping = ExpertSlotMapping(layer_id, (), table, tuple(stage.owners()), ())
        return PreparedSlotWeights(stage.w13_slots, stage.w2_slots, table, stage.physical_expert_count, mapping)

    def _issue_decode_overflow(self, *, layer_id: int, experts: tuple[int, ...], total: int,
                               step_id: int) -> DecodeOverflowStage:
        """Queue the overflow experts' copies (host rows: by construction none
        is resident) into the layer's stage buffer, with its table, after the
        buffer's previous compute has released it."""
        src = self._slot_banks[layer_id]
        buf = self.decode_overflow_buffer_index(layer_id)
        stage = self._get_prefill_stage_bank(layer_id=layer_id, buffer_index=buf, template_bank=src)
        table = self._overflow_table(layer_id, total, src.w13_slots.device)
        # the buffer's last reader recorded its release when its Python ran
        # (end_overflow_compute); a replayed graph piece records none, so the
        # copies also wait for everything queued on the compute stream so far,
        # which holds every earlier reader of this buffer (an earlier layer's
        # piece is queued before this layer's staging runs)
        wait = tuple(ev for ev in (self.prefill_stage_buffer_release_event(layer_id=layer_id, buffer_index=buf),
                                   self._record_current_stream_event_or_none()) if ev is not None)
        loads = [(self._host_store.get(layer_id, e), stage.assign_transient_slot(i, ExpertKey(layer_id, e), step_id=step_id))
                 for i, e in enumerate(experts)]
        for sid in range(len(experts), stage.num_dynamic_slots):
            stage.clear_slot(sid, force=True)
        device_path = table.device.type == "cuda" and stage.w13_slots.device.type == "cuda"
        ready = None
        try:
            if self.config.async_load and device_path:
                ready = self._transfer_engine.load_many_async(
                    loads, wait_event=wait, record_event=True, validate_layout=False,
                    table_update=(table, tuple(experts), tuple(range(len(experts))), True))
            else:
                for ev in wait:
                    _synchronize_event(getattr(ev, "event", ev))
                self._transfer_engine.load_many_sync(loads, validate_layout=False)
                values = np.full(int(table.numel()), -1, dtype=np.int32)
                values[list(experts)] = np.arange(len(experts), dtype=np.int32)
                table.copy_(torch.from_numpy(values))
        except Exception:
            self._release_allocated_loads(stage, loads)
            raise
        self._overflow_dirty.add(int(layer_id))
        return DecodeOverflowStage(buf, stage, table, tuple(experts), ready)

    def _publish_decode_overflow(self, pending: PendingFixedSlotStage) -> PreparedSlotWeights | None:
        """Order the overflow copies before the consumer and hand out the
        second pass; with no overflow this step, a table still holding the
        last one is cleared on the consumer stream (after the compute that
        read it, before the one that will)."""
        layer_id = pending.layer_id
        ovf = pending.overflow
        if ovf is None:
            if layer_id in self._overflow_dirty:
                self._overflow_tables[layer_id].fill_(-1)
                self._overflow_dirty.discard(layer_id)
            return None
        if ovf.ready is not None:
            self._wait_transfer_event(ovf.ready)
        self._overflow_release_pending[layer_id] = ovf.buffer_index
        mapping = ExpertSlotMapping(layer_id, ovf.experts, ovf.table, tuple(ovf.bank.owners()),
                                   tuple(range(len(ovf.experts))))
        return PreparedSlotWeights(ovf.bank.w13_slots, ovf.bank.w2_slots, ovf.table, ovf.bank.physical_expert_count,
                                   mapping)

    def _write_owner_entries(self, layer_id: int, owner_updates, stream=None) -> None:
        idx, val = self._owner_entries(layer_id, owner_updates)
        if not idx:
            return
        backing = self._log2phy_backing[int(layer_id)]
        if backing.device.type != "cuda":
            backing[list(idx)] = torch.tensor(val, dtype=backing.dtype)
            return
        from vllm_moe_offload_amd import native

        native.table_update_entries(backing, idx, val, stream=stream)

    def end_overflow_compute(self, layer_id: int) -> None:
        """After the compute that reads a layer's overflow pass is queued:
        its stage buffer is released for the next copies once that compute
        completes (no-op when the layer had no overflow)."""
        buf = self._overflow_release_pending.pop(int(layer_id), None)
        if buf is None:
            return
        ev = self._record_current_stream_event_or_none()
        self.remember_prefill_stage_buffer_release(layer_id=int(layer_id), buffer_index=buf, event=ev)


    def _raise_no_slot(self, layer_id: int, expert_id: int, bank: ExpertSlotBank) -> None:
        raise RuntimeError(
            f"failed to allocate expert slot for layer {layer_id} expert {expert_id} with "
            f"num_slots={self.config.num_slots}; async_load={self.config.async_load}"
        ) from RuntimeError(f"no evictable expert slots; states={bank.state_counts()}")

    def _publish(self, pending: PendingFixedSlotStage, *, record_stage_profile: bool) -> PreparedSlotWeights:
        layer_id = pending.layer_id
        bank = self._slot_banks[layer_id]
        # order the copies before the consumer, THEN publish the mapping
        t_wait = perf_counter()
        if pending.ready is not None:
            self._wait_transfer_event(pending.ready)
        t_map = perf_counter()
        active, slot_ids = pending.active, pending.slot_ids
        ovf_experts = pending.overflow.experts if pending.overflow is not None else ()
        if pending.table_updates >= 0:
            n_updates = pending.table_updates  # written on the transfer stream with the copies
        else:
            upd_e, upd_s = self._changed_log2phy_entries(layer_id=layer_id, expert_ids=tuple(active) + ovf_experts,
                                                         slot_ids=tuple(slot_ids) + (-1,) * len(ovf_experts))
            if upd_e:
                _update_log2phy_entries(pending.log2phy, expert_ids=upd_e, slot_ids=upd_s)
                self._remember_log2phy_entries(layer_id=layer_id, expert_ids=upd_e, slot_ids=upd_s)
            n_updates = len(upd_e)
        if pending.owner_updates:
            self._write_owner_entries(layer_id, pending.owner_updates)
        overflow = self._publish_decode_overflow(pending)
        mapping = ExpertSlotMapping(layer_id, active, pending.log2phy, tuple(pending.owners), tuple(slot_ids))
        self._active_slot_ids_by_layer[layer_id] = tuple(slot_ids)
        self.last_stage_stats = (len(pending.hits), len(pending.misses))
        if record_stage_profile and self._collect_stage_profile(pending.step_id):
            now = perf_counter()
            per = int(self._expert_weight_bytes_by_layer.get(layer_id, 0))
            payload = {
                "n_active": len(active),
                "n_hits": len(pending.hits),
                "n_misses": len(pending.misses),
                "hit_rate": round(len(pending.hits) / len(active), 6) if active else 0.0,
                "h2d_bytes": per * len(pending.misses),
                "stage_ms": round((now - pending.started) * 1000.0, 3),
                "load_sync_ms": round(pending.load_sync_ms, 3),
                "load_enqueue_ms": round(pending.load_enqueue_ms, 3),
                "ready_wait_ms": round((t_map - t_wait) * 1000.0, 3),
                "mapping_ms": round((now - t_map) * 1000.0, 3),
                "step_id": pending.step_id,
                "num_slots": int(self.config.num_slots),
                "mapping_mode": "persistent_log2phy",
                "log2phy_update_count": n_updates,
                "stage_mode": "main_slot_hit" if not pending.misses else (
                    "async_decode_load_many" if pending.ready is not None else "sync_decode_load"),
                "consumer_dependency_installed": True,
                "mapping_published_after_ready": True,
                "profile_sample_rate": _decode_profile_sample_rate(),
                "overflow_experts": len(ovf_experts),
            }
            if _profile_expert_lists_enabled():
                payload.update({"active_experts": list(active), "hit_experts": list(pending.hits),
                                "miss_experts": list(pending.misses)})
            else:
                payload["expert_lists"] = "omitted"
            self._record_profile_event("decode_fixed_slot_stage", layer_id=layer_id, start=t_map, payload=payload)
        return PreparedSlotWeights(bank.w13_slots, bank.w2_slots, mapping.logical_to_physical,
                                   bank.physical_expert_count, mapping, overflow)

    def _changed_log2phy_entries(self, *, layer_id: int, expert_ids, slot_ids) -> tuple[tuple[int, ...], tuple[int, ...]]:
        if len(expert_ids) != len(slot_ids):
            raise ValueError(f"expert_ids and slot_ids length mismatch: {len(expert_ids)} != {len(slot_ids)}")
        cached = self._log2phy_slot_by_expert.setdefault(int(layer_id), {})
        pairs = [(int(e), int(s)) for e, s in zip(expert_ids, slot_ids) if cached.get(int(e)) != int(s)]
        return tuple(p[0] for p in pairs), tuple(p[1] for p in pairs)

    def _remember_log2phy_entries(self, *, layer_id: int, expert_ids, slot_ids) -> None:
        cached = self._log2phy_slot_by_expert.setdefault(int(layer_id), {})
        for e, s in zip(expert_ids, slot_ids):
            cached[int(e)] = int(s)

    def stage_fixed_slot_plan(self, *, layer_id: int, active_experts, num_logical_experts: int,
                              token_counts: dict[int, int] | None = None) -> PreparedSlotWeights:
        """Eager pre-replay staging into the persistent log2phy (never inside capture)."""
        if _is_current_graph_capturing():
            raise RuntimeError(
                "stage_fixed_slot_plan must run eager (outside graph capture); it performs host decision + H2D staging"
            )
        active = resolve_placement_plan(
            self._placement_plan_provider,
            layer_id=int(layer_id),
            routed_experts=tuple(int(e) for e in active_experts),
            num_logical_experts=int(num_logical_experts),
        )
        self._assert_locked_slot_addresses(int(layer_id))
        buf = self._log2phy_buffers[int(layer_id)]
        pending = self._reserve_and_issue(layer_id=int(layer_id), active_experts=active,
                                          num_logical_experts=int(num_logical_experts), log2phy=buf, step_id=None,
                                          token_counts=token_counts)
        prepared = self._publish(pending, record_stage_profile=True)
        return PreparedSlotWeights(prepared.w1, prepared.w2, buf, prepared.physical_expert_count, prepared.mapping,
                                   prepared.overflow)

    def stage_full_residency_slot_plan(self, *, layer_id: int) -> bool:
        """Regime A: stage every routed expert once, before capture."""
        layer_id = int(layer_id)
        if not (self.should_use_fixed_slots and self.config.graph_compatible_offload):
            return False
        if self.is_resident_layer(layer_id) or not self.is_layer_registered(layer_id):
            return False
        buf = self._log2phy_buffers.get(layer_id)
        if buf is None:
            return False
        if _is_current_graph_capturing():
            if bool((buf < 0).all().item()):
                raise RuntimeError(
                    f"stage_full_residency_slot_plan called during graph capture for layer {layer_id} but its "
                    "log2phy buffer is still all -1; staging must run eager before capture"
                )
            return False
        routed, total = self._resolve_fused_shared_counts(layer_id=layer_id, requested_logical_expert_count=int(buf.numel()))
        if not self.is_static_residency_regime(routed):
            self._record_profile_event(
                "skip_full_residency_slot_plan", layer_id=layer_id, start=perf_counter(),
                payload={"reason": "regime_b_num_slots_lt_logical_experts", "num_slots": int(self.config.num_slots),
                         "routed_expert_count": routed},
            )
            return False
        self.stage_fixed_slot_plan(layer_id=layer_id, active_experts=tuple(range(routed)), num_logical_experts=total)
        self._full_residency_layers.add(layer_id)
        return True

    def is_full_residency_staged(self, layer_id: int) -> bool:
        """Every routed expert of the layer is staged and its table static
        (the per-step seam has nothing to do)."""
        return int(layer_id) in self._full_residency_layers

    def capture_safe_slot_weights(self, *, layer_id: int) -> PreparedSlotWeights | None:
        """Fixed slot tensors + fixed log2phy, no host sync, no copy: what a
        captured graph records.  Locks the address fingerprint."""
        layer_id = int(layer_id)
        bank = self._slot_banks.get(layer_id)
        buf = self._log2phy_buffers.get(layer_id)
        if bank is None or buf is None:
            return None
        self._lock_graph_slot_addresses(layer_id)
        owners: list[int | None] = [int(s.expert_key.expert_id) if s.expert_key is not None else None for s in bank.slots]
        owners.extend(int(e) for e in bank.pinned_logical_ids)
        mapping = ExpertSlotMapping(layer_id, (), buf, tuple(owners), ())
        return PreparedSlotWeights.from_slot_bank(slot_bank=bank, mapping=mapping)

    def _slot_address_fingerprint(self, layer_id: int) -> SlotAddressFingerprint:
        bank = self._slot_banks.get(int(layer_id))
        buf = self._log2phy_buffers.get(int(layer_id))
        if bank is None or buf is None:
            raise RuntimeError(f"layer {layer_id} has no fixed-slot tensors to fingerprint")
        return SlotAddressFingerprint(
            int(bank.w13_slots.data_ptr()), int(bank.w2_slots.data_ptr()), int(buf.data_ptr()),
            tuple(int(d) for d in bank.w13_slots.shape), tuple(int(d) for d in bank.w2_slots.shape),
            tuple(int(d) for d in buf.shape), str(bank.w13_slots.device), str(bank.w13_slots.dtype),
        )

    def _lock_graph_slot_addresses(self, layer_id: int) -> None:
        start = perf_counter()
        fp = self._slot_address_fingerprint(layer_id)
        old = self._graph_slot_address_fingerprints.get(int(layer_id))
        if old is None:
            self._graph_slot_address_fingerprints[int(layer_id)] = fp
            self._record_profile_event("graph_slot_address_lock", layer_id=int(layer_id), start=start, payload=fp.to_jsonable())
            return
        if old != fp:
            raise RuntimeError(f"fixed-slot address fingerprint changed for captured layer {layer_id}")
        if not _is_current_graph_capturing() and int(layer_id) not in self._graph_slot_address_evidence:
            self._graph_slot_address_evidence.add(int(layer_id))
            self._record_profile_event(
                "graph_slot_address_validate", layer_id=int(layer_id), start=start,
                payload={**fp.to_jsonable(), "matches_capture_fingerprint": True},
            )

    def _assert_locked_slot_addresses(self, layer_id: int) -> None:
        if int(layer_id) in self._graph_slot_address_fingerprints:
            self._lock_graph_slot_addresses(int(layer_id))

    def _wait_transfer_event(self, ready_event) -> None:
        if ready_event is None:
            return
        install = getattr(ready_event, "install_consumer_dependency", None)
        ev = getattr(ready_event, "event", ready_event)
        if callable(install):
            install(self._consumer_stream() if isinstance(ev, torch.cuda.Event) else _NullStream())
            return
        if isinstance(ev, torch.cuda.Event):
            self._consumer_stream().wait_event(ev)
        mark = getattr(ready_event, "mark_ready", None)
        if callable(mark):
            mark()

    def wait_prefill_stage_plan(self, ready_event) -> None:
        self._wait_transfer_event(ready_event)

    # ---------------------------------------------------- prefill waves
    def _validate_prefill_buffer_index(self, buffer_index: int) -> None:
        cap = self.config.effective_prefill_buffer_count
        if int(buffer_index) < 0 or int(buffer_index) >= cap:
            raise RuntimeError(
                f"prefill stage buffer index {int(buffer_index)} is outside prefill_buffer_count={cap}"
            )

    @staticmethod
    def _pool_key(bank: ExpertSlotBank) -> tuple:
        return (
            str(bank.w13_slots.device), str(bank.w13_slots.dtype), len(bank.slots),
            tuple(bank.pinned_logical_ids), tuple(int(d) for d in bank.w13_slots.shape[1:]),
            tuple(int(d) for d in bank.w2_slots.shape[1:]),
        )

    def _get_prefill_stage_bank(self, *, layer_id: int, buffer_index: int, template_bank: ExpertSlotBank) -> ExpertSlotBank:
        self._validate_prefill_buffer_index(buffer_index)
        banks = self._prefill_stage_pool.setdefault(self._pool_key(template_bank), [])
        self._prefill_stage_banks[int(layer_id)] = banks
        while len(banks) <= int(buffer_index):
            start = perf_counter()
            nb = ExpertSlotBank(
                len(template_bank.slots),
                tuple(int(d) for d in template_bank.w13_slots.shape[1:]),
                tuple(int(d) for d in template_bank.w2_slots.shape[1:]),
                dtype=template_bank.w13_slots.dtype,
                device=template_bank.w13_slots.device,
                pinned_logical_ids=template_bank.pinned_logical_ids,
            )
            nb.copy_pinned_weights_from(template_bank)
            banks.append(nb)
            self._memory_ledger_cache = None
            self._record_profile_event(
                "prefill_stage_bank_allocate", layer_id=int(layer_id), start=start,
                payload={"buffer_index": len(banks) - 1, "bank_bytes": int(nb.total_bytes)},
            )
        return banks[int(buffer_index)]

    def _get_prefill_stage_log2phy_buffer(self, *, template_bank: ExpertSlotBank, buffer_index: int,
                                          num_logical_experts: int, device) -> torch.Tensor:
        key = (self._pool_key(template_bank), int(buffer_index), int(num_logical_experts), str(device))
        buf = self._prefill_stage_log2phy.get(key)
        if buf is None:
            buf = torch.full((int(num_logical_experts),), -1, dtype=torch.int32, device=device)
            self._prefill_stage_log2phy[key] = buf
            self._memory_ledger_cache = None
        return buf

    def prefill_stage_buffer_release_event(self, *, layer_id: int, buffer_index: int) -> object | None:
        self._validate_prefill_buffer_index(buffer_index)
        bank = self._slot_banks.get(int(layer_id))
        if bank is None:
            return None
        return self._prefill_stage_pool_release_events.get((self._pool_key(bank), int(buffer_index)))

    def remember_prefill_stage_buffer_release(self, *, layer_id: int, buffer_index: int, event: object | None) -> None:
        self._validate_prefill_buffer_index(buffer_index)
        if event is None:
            return
        bank = self._slot_banks.get(int(layer_id))
        if bank is not None:
            self._prefill_stage_pool_release_events[(self._pool_key(bank), int(buffer_index))] = event

    def prepare_ready_slot_plan(self, *, layer_id: int, active_experts, num_logical_experts: int, device,
                                step_id: int | None = None, build_log2phy: bool = True, **_: object) -> PreparedSlotWeights:
        """Zero-copy plan for a wave whose experts are all READY in the main
        bank; any miss fails closed."""
        if not self.should_use_fixed_slots:
            raise RuntimeError("ready-slot plan requested while fixed slots are disabled")
        layer_id = int(layer_id)
        if self.is_resident_layer(layer_id):
            raise RuntimeError(f"ready-slot plan must not run on resident layer {layer_id}")
        routed, total = self._resolve_fused_shared_counts(layer_id=layer_id, requested_logical_expert_count=num_logical_experts)
        active = dedupe_preserve_order(active_experts)
        _validate_active_expert_ids(layer_id=layer_id, active_experts=active, num_logical_experts=routed)
        if len(active) > self.config.num_slots:
            raise RuntimeError(f"ready expert working set size {len(active)} exceeds num_slots={self.config.num_slots}")
        bank = self._slot_banks.get(layer_id)
        if bank is None:
            raise RuntimeError(f"layer {layer_id} is not registered for fixed-slot execution")
        step_id = self._step(step_id)
        missing: list[int] = []
        slot_ids: list[int] = []
        for e in active:
            slot = bank.lookup(ExpertKey(layer_id, e))
            if slot is None or slot.state != SlotState.READY:
                missing.append(e)
                continue
            slot.last_used_step = step_id
            slot_ids.append(int(slot.slot_id))
        if missing:
            raise RuntimeError(f"ready-slot plan requested for non-ready experts in layer {layer_id}: {missing}")
        if build_log2phy:
            mapping = ExpertSlotMapping.from_slot_bank(
                layer_id=layer_id, active_experts=active, num_logical_experts=total, slot_bank=bank, device=device
            )
        else:
            owners: list[int | None] = [None] * bank.physical_expert_count
            for logical_id in bank.pinned_logical_ids:
                owners[int(bank.pinned_slot_for_logical_id(logical_id))] = int(logical_id)
            for s in bank.slots:
                if s.expert_key is not None:
                    owners[s.slot_id] = int(s.expert_key.expert_id)
            mapping = ExpertSlotMapping(
                layer_id, active, torch.empty(0, dtype=torch.int32, device=device), tuple(owners), tuple(slot_ids),
                log2phy_valid=False,
            )
        return PreparedSlotWeights.from_slot_bank(slot_bank=bank, mapping=mapping)

    def prepare_prefill_stage_plan(self, *, layer_id: int, active_experts, num_logical_experts: int, device,
                                   buffer_index: int, async_load: bool, wait_event=None, step_id: int | None = None,
                                   build_log2phy: bool = True, known_miss: bool = False):
        """Stage one wave into stage buffer `buffer_index`: slot i <- i-th
        expert (D2D for main-bank hits, H2D for misses).  Returns
        (prepared, ready_event or None, payload)."""
        if not self.should_use_fixed_slots:
            raise RuntimeError("prefill stage plan requested while fixed slots are disabled")
        self._validate_prefill_buffer_index(int(buffer_index))
        layer_id = int(layer_id)
        if self.is_resident_layer(layer_id):
            raise RuntimeError(f"prefill stage plan must not run on resident layer {layer_id}")
        routed, total = self._resolve_fused_shared_counts(layer_id=layer_id, requested_logical_expert_count=num_logical_experts)
        active = dedupe_preserve_order(active_experts)
        _validate_active_expert_ids(layer_id=layer_id, active_experts=active, num_logical_experts=routed)
        if len(active) > self.config.num_slots:
            raise RuntimeError(f"prefill wave size {len(active)} exceeds num_slots={self.config.num_slots}")
        src = self._slot_banks.get(layer_id)
        if src is None:
            raise RuntimeError(f"layer {layer_id} is not registered for fixed-slot execution")
        stage = self._get_prefill_stage_bank(layer_id=layer_id, buffer_index=int(buffer_index), template_bank=src)
        if wait_event is None:
            wait_event = self.prefill_stage_buffer_release_event(layer_id=layer_id, buffer_index=int(buffer_index))
        table = self._get_prefill_stage_log2phy_buffer(
            template_bank=src, buffer_index=int(buffer_index), num_logical_experts=total, device=device
        )
        step_id = self._step(step_id)
        hits: list[int] = []
        misses: list[int] = []
        loads = []
        for i, e in enumerate(active):
            key = ExpertKey(layer_id, e)
            slot = (stage.assign_transient_slot if known_miss else stage.assign_slot)(i, key, step_id=step_id)
            hit = None if known_miss else src.lookup(key)
            if hit is not None and hit.state == SlotState.READY:
                hits.append(e)
                loads.append((hit.as_bundle(), slot))
            else:
                misses.append(e)
                loads.append((self._host_store.get(layer_id, e), slot))
        # the wave's table: slot i <- i-th expert, the pinned suffix, -1 elsewhere
        pairs = (tuple(active) + tuple(stage.pinned_logical_ids),
                 tuple(range(len(active))) + tuple(stage.pinned_slot_ids))
        fused_table = build_log2phy and async_load and bool(loads) and table.device.type == "cuda" \
            and stage.w13_slots.device.type == "cuda"
        if build_log2phy and not fused_table:
            values = np.full(total, -1, dtype=np.int32)
            values[list(pairs[0])] = pairs[1]
            table.copy_(torch.from_numpy(values), non_blocking=False)
        ready = None
        if loads:
            if async_load:
                extra = {"table_update": (table, pairs[0], pairs[1], True)} if fused_table else {}
                try:
                    ready = self._transfer_engine.load_many_async(loads, wait_event=wait_event, record_event=True,
                                                                  validate_layout=False, **extra)
                except Exception:
                    self._release_allocated_loads(stage, loads)
                    raise
            else:
                if wait_event is not None:
                    _synchronize_event(getattr(wait_event, "event", wait_event))
                try:
                    self._transfer_engine.load_many_sync(loads, validate_layout=False)
                except Exception:
                    self._release_allocated_loads(stage, loads)
                    raise
        for sid in range(len(active), len(stage.slots)):
            stage.clear_slot(sid)
        if async_load and ready is None:
            ready = wait_event
        mapping = ExpertSlotMapping(layer_id, active, table, tuple(stage.owners()), tuple(range(len(active))),
                                   log2phy_valid=build_log2phy)
        per = int(self._expert_weight_bytes_by_layer.get(layer_id, 0))
        payload = {
            "buffer_index": int(buffer_index),
            "hit_experts": hits,
            "miss_experts": misses,
            "h2d_bytes": per * len(misses),
            "d2d_bytes": per * len(hits),
            "log2phy_built": bool(build_log2phy),
            "known_miss": bool(known_miss),
        }
        return PreparedSlotWeights.from_slot_bank(slot_bank=stage, mapping=mapping), ready, payload

    def prepare_full_layer_prefill_plan(self, *, layer_id: int, num_logical_experts: int, device,
                                        step_id: int | None = None):
        """Blocking reference plan: the whole layer in one layout-shared bank
        with identity log2phy (the recoverable-fallback path)."""
        if not self.should_use_fixed_slots:
            raise RuntimeError("full-layer prefill plan requested while fixed slots are disabled")
        layer_id = int(layer_id)
        routed, total = self._resolve_fused_shared_counts(layer_id=layer_id, requested_logical_expert_count=num_logical_experts)
        if self.is_resident_layer(layer_id):
            raise RuntimeError(f"full-layer prefill plan must not run on resident layer {layer_id}")
        tmpl = self._slot_banks.get(layer_id)
        if tmpl is None:
            raise RuntimeError(f"layer {layer_id} is not registered for fixed-slot execution")
        buf = self._host_store.get_layer_buffer(layer_id)
        if int(buf.num_experts) != routed:
            raise RuntimeError(f"host expert count for layer {layer_id} is {buf.num_experts}, expected {routed}")
        key = (*self._pool_key(tmpl)[:2], routed, *self._pool_key(tmpl)[3:])
        reused = key in self._full_layer_prefill_pool
        bank = self._full_layer_prefill_pool.get(key)
        if bank is None:
            bank = ExpertSlotBank(
                routed, tuple(int(d) for d in tmpl.w13_slots.shape[1:]), tuple(int(d) for d in tmpl.w2_slots.shape[1:]),
                dtype=tmpl.w13_slots.dtype, device=tmpl.w13_slots.device, pinned_logical_ids=tmpl.pinned_logical_ids,
            )
            self._full_layer_prefill_pool[key] = bank
            self._memory_ledger_cache = None
        table = self._full_layer_prefill_log2phy.get(key)
        if table is None:
            values = list(range(routed)) + [int(bank.pinned_slot_for_logical_id(e)) for e in bank.pinned_logical_ids]
            table = torch.tensor(values, dtype=torch.int32, device=device)
            self._full_layer_prefill_log2phy[key] = table
            self._memory_ledger_cache = None
        step_id = self._step(step_id)
        for e in range(routed):
            bank.assign_transient_slot(e, ExpertKey(layer_id, e), step_id=step_id)
        start = perf_counter()
        try:
            bank.w13_slots[:routed].copy_(buf.w13)
            bank.w2_slots[:routed].copy_(buf.w2)
            bank.copy_pinned_weights_from(tmpl)
        except Exception:
            for sid in range(routed):
                bank.clear_slot(sid, force=True)
            raise
        for sid in range(routed):
            bank.mark_ready(sid)
        all_experts = tuple(range(routed))
        owners: list[int | None] = list(all_experts) + [int(e) for e in bank.pinned_logical_ids]
        mapping = ExpertSlotMapping(layer_id, all_experts, table, tuple(owners), all_experts)
        prepared = PreparedSlotWeights.from_slot_bank(slot_bank=bank, mapping=mapping)
        payload = {
            "execution_mode": "reference_full_layer",
            "num_logical_experts": total,
            "routed_expert_count": routed,
            "pinned_shared_expert_count": len(bank.pinned_logical_ids),
            "physical_expert_count": int(prepared.physical_expert_count),
            "h2d_bytes": int(buf.total_bytes),
            "stage_ms": round((perf_counter() - start) * 1000.0, 3),
            "pool_reused": bool(reused),
        }
        return prepared, payload

    # ------------------------------------------------------ route stats
    @staticmethod
    def _route_stats_key(*, layer_id: int, topk_ids: torch.Tensor) -> tuple:
        try:
            version = int(topk_ids._version)
        except RuntimeError:
            version = 0
        return (
            int(layer_id), str(topk_ids.device), str(topk_ids.dtype), tuple(int(d) for d in topk_ids.shape),
            tuple(int(s) for s in topk_ids.stride()), int(topk_ids.storage_offset()), int(topk_ids.numel()),
            int(topk_ids.data_ptr()), version,
        )

    def cache_prefill_route_stats(self, *, layer_id: int, topk_ids: torch.Tensor, token_counts_by_expert: dict[int, int],
                                  pair_offsets_by_expert=None) -> MoePrefillRouteStats:
        """Remember the histogram the stage seam already paid a D2H for."""
        counts = {int(e): int(c) for e, c in token_counts_by_expert.items() if int(c) > 0}
        offs = None
        if pair_offsets_by_expert is not None:
            offs = {int(e): tuple(int(o) for o in v) for e, v in pair_offsets_by_expert.items() if int(e) in counts}
        stats = MoePrefillRouteStats(
            layer_id=int(layer_id),
            topk_cache_key=self._route_stats_key(layer_id=layer_id, topk_ids=topk_ids),
            token_counts_by_expert=counts,
            active_experts=tuple(sorted(counts)),
            num_tokens=int(topk_ids.shape[0]) if topk_ids.ndim > 0 else 0,
            top_k=int(topk_ids.shape[1]) if topk_ids.ndim > 1 else 1,
            pair_offsets_by_expert=offs,
        )
        self._prefill_route_stats_by_layer[int(layer_id)] = stats
        return stats

    def consume_prefill_route_stats_record(self, *, layer_id: int, topk_ids: torch.Tensor) -> MoePrefillRouteStats | None:
        stats = self._prefill_route_stats_by_layer.pop(int(layer_id), None)
        if stats is None or stats.topk_cache_key != self._route_stats_key(layer_id=layer_id, topk_ids=topk_ids):
            return None
        return stats

    def consume_prefill_route_stats(self, *, layer_id: int, topk_ids: torch.Tensor) -> dict[int, int] | None:
        stats = self.consume_prefill_route_stats_record(layer_id=layer_id, topk_ids=topk_ids)
        return None if stats is None else dict(stats.token_counts_by_expert)

    # ------------------------------------------------- device-planned waves
    def can_run_device_waves(self, layer_id: int) -> bool:
        """Device wave planning applies: enabled, an offloaded registered layer
        on a device bank, a page-locked host store, shapes within the planner."""
        from vllm_moe_offload_amd import native

        layer_id = int(layer_id)
        if not (self.config.device_wave_prefill and self.should_use_fixed_slot_plan_for_layer(layer_id)):
            return False
        bank = self._slot_banks.get(layer_id)
        if bank is None or bank.w13_slots.device.type != "cuda":
            return False
        try:
            buf = self._host_store.get_layer_buffer(layer_id)
        except KeyError:
            return False
        routed = self.routed_expert_count_for_layer(layer_id=layer_id, fallback=buf.num_experts)
        return bool(buf.pinned) and routed <= native.WAVE_PLAN_MAX_EXPERTS and \
            bank.num_dynamic_slots <= native.WAVE_PLAN_MAX_SLOTS and buf.num_experts >= routed

    def device_wave_plan_buffer(self, *, n_routed: int, n_slots: int, max_waves: int, device):
        from vllm_moe_offload_amd import native

        key = (int(n_routed), int(n_slots), int(max_waves), str(device))
        plan = self._device_wave_plans.get(key)
        if plan is None:
            plan = native.WavePlan(n_routed, n_slots, max_waves, device)
            self._device_wave_plans[key] = plan
        return plan

    def mark_device_waves(self, *, layer_id: int, topk_ids: torch.Tensor) -> None:
        """The seam handed this layer's routed ids to the device planner."""
        self._device_wave_marks[int(layer_id)] = self._route_stats_key(layer_id=layer_id, topk_ids=topk_ids)

    def consume_device_waves(self, *, layer_id: int, topk_ids: torch.Tensor) -> bool:
        key = self._device_wave_marks.pop(int(layer_id), None)
        return key is not None and key == self._route_stats_key(layer_id=layer_id, topk_ids=topk_ids)


# ---------------------------------------------------------------------------
def _split_decode_overflow(bank: ExpertSlotBank, active: tuple[int, ...], capacity: int,
                           token_counts: dict[int, int] | None) -> tuple[tuple[int, ...], tuple[int, ...]]:
    """Split a decode working set larger than the bank: every READY resident
    expert stays in the bank pass (a hit), the other experts fill the bank's
    remaining slots by routed token count (more first, then id) and the rest
    form the overflow pass.  Which pass serves a pair does not change its
    result: each pair's row is computed alone and the combine sums in top-k
    order."""
    resident = bank.ready_resident_mask(active)
    hits = [e for e, r in zip(active, resident) if r]
    cold = [e for e, r in zip(active, resident) if not r]
    counts = token_counts or {}
    cold.sort(key=lambda e: (-int(counts.get(e, 0)), e))
    room = capacity - len(hits)
    return tuple(hits) + tuple(cold[:room]), tuple(cold[room:])


def _decode_profile_sample_rate() -> int:
    try:
        return max(1, int(os.environ.get("VLLM_ASCEND_MOE_DECODE_PROFILE_SAMPLE_RATE", "1")))
    except ValueError:
        return 1


def _profile_expert_lists_enabled() -> bool:
    return os.environ.get("VLLM_ASCEND_MOE_PROFILE_EXPERT_LISTS", "1").strip().lower() not in {"0", "false", "no", "off"}


def _synchronize_event(ev: object) -> None:
    sync = getattr(ev, "synchronize", None)
    if callable(sync):
        sync()
        return
    wait = getattr(ev, "wait", None)
    if callable(wait):
        wait()


class _NullStream:
    def wait_event(self, _event) -> None:  # host-only slot banks need no ordering
        return None


def _validate_active_expert_ids(*, layer_id: int, active_experts, num_logical_experts: int) -> None:
    bad = [int(e) for e in active_experts if int(e) < 0 or int(e) >= int(num_logical_experts)]
    if bad:
        raise ValueError(
            f"fixed-slot active expert id out of range: layer_id={int(layer_id)}, "
            f"num_logical_experts={int(num_logical_experts)}, expert_ids={bad}"
        )


def _update_log2phy_entries(log2phy: torch.Tensor, *, expert_ids, slot_ids) -> None:
    """Write the changed entries of a persistent log2phy in one operation
    (reference: runtime.py:3068-3101, one scalar write or an index_copy_)."""
    if len(expert_ids) != len(slot_ids):
        raise ValueError(f"expert_ids and slot_ids length mismatch: {len(expert_ids)} != {len(slot_ids)}")
    if not expert_ids:
        return
    if log2phy.device.type != "cuda":
        idx = torch.tensor([int(e) for e in expert_ids], dtype=torch.long)
        log2phy.index_copy_(0, idx, torch.tensor([int(v) for v in slot_ids], dtype=log2phy.dtype))
        return
    # one kernel on the current stream whose arguments carry the pairs: no
    # staging tensor, no copy, no host sync
    from vllm_moe_offload_amd import native

    native.table_update_entries(log2phy, expert_ids, slot_ids)


_runtime: MoeOffloadRuntime | None = None


def get_moe_offload_runtime() -> MoeOffloadRuntime:
    global _runtime
    if _runtime is None:
        _runtime = MoeOffloadRuntime()
    return _runtime


def reset_moe_offload_runtime() -> None:
    global _runtime
    _runtime = None
