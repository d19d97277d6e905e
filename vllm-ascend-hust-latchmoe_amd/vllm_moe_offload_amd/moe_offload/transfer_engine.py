"""Host-store -> slot transfers on a dedicated HIP transfer stream.

A batch of expert loads becomes one lmoe_stage_copy call: hipMemcpyAsync per
contiguous run (expert e, e+1, ... into slot s, s+1, ... is one copy per
weight tensor) on the transfer stream, then one hipEvent.  The consumer
(compute) stream waits on that event before the slots are published READY,
so no kernel can read a slot whose bytes are still in flight.  Leases make a
late completion for a slot that changed owner fail instead of publishing.

Reference: moe_offload/transfer_engine.py:29-342 (TransferReadyEvent lease
validation and consumer wait :29-69; load_many_async :139-187; contiguous-run
batching :205-342).  Slots on the CPU (host-only tests) take a synchronous
copy, as the reference's CPU branch does.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from vllm_moe_offload_amd.moe_offload.host_store import ExpertWeightBundle
from vllm_moe_offload_amd.moe_offload.layout import LayoutValidator
from vllm_moe_offload_amd.moe_offload.slot_bank import ExpertSlot, SlotLease, SlotState


@dataclass
class TransferReadyEvent:
    """Transfer-stream event plus the slots it makes consumable."""

    event: object | None
    leases: tuple[tuple[ExpertSlot, SlotLease], ...]
    completed: bool = False
    consumer_wait_installed: bool = False

    def install_consumer_dependency(self, consumer_stream) -> None:
        """Order the copies before consumer_stream, then publish READY."""
        if self.completed:
            return
        self._validate_loading_leases()
        if self.event is not None:
            consumer_stream.wait_event(self.event)
        self.consumer_wait_installed = True
        self.mark_ready()

    def mark_ready(self) -> None:
        if self.completed:
            return
        self._validate_loading_leases()
        for slot, _ in self.leases:
            slot.state = SlotState.READY
        self.completed = True

    def _validate_loading_leases(self) -> None:
        for slot, lease in self.leases:
            if not slot.matches_lease(lease):
                raise RuntimeError(
                    f"stale H2D completion for slot {slot.slot_id}: expected {lease.expert_key} "
                    f"v{lease.version}, found {slot.expert_key} v{slot.version}"
                )
            if slot.state != SlotState.LOADING:
                raise RuntimeError(
                    f"H2D completion for slot {slot.slot_id} requires loading state, found {slot.state.value}"
                )


Load = tuple[ExpertWeightBundle, ExpertSlot]


class TransferEngine:
    def __init__(self) -> None:
        self._h2d_stream: torch.cuda.Stream | None = None
        self._pending_ready_events: list[TransferReadyEvent] = []
        self.bytes_issued = 0
        self.copies_issued = 0

    # -- synchronous --------------------------------------------------------
    def load_sync(self, bundle: ExpertWeightBundle, slot: ExpertSlot) -> None:
        LayoutValidator.validate_copy_compatible(bundle, slot.as_bundle())
        self._copy(((bundle, slot),), stream=None)
        slot.state = SlotState.READY

    def load_many_sync(self, loads: list[Load], *, validate_layout: bool = True) -> None:
        if not loads:
            return
        if validate_layout:
            for bundle, slot in loads:
                LayoutValidator.validate_copy_compatible(bundle, slot.as_bundle())
        for _, slot in loads:
            slot.state = SlotState.LOADING
        self._copy(tuple(loads), stream=None)
        for _, slot in loads:
            slot.state = SlotState.READY

    # -- asynchronous -------------------------------------------------------
    def load_async(self, bundle: ExpertWeightBundle, slot: ExpertSlot, *, wait_event=None,
                   record_event: bool = True):
        return self.load_many_async([(bundle, slot)], wait_event=wait_event, record_event=record_event)

    def load_many_async(self, loads: list[Load], *, wait_event=None, record_event: bool = True,
                        validate_layout: bool = True, table_update=None):
        """Queue the loads on the transfer stream; returns a TransferReadyEvent
        (or None when the copy completed synchronously).  table_update =
        (device int32 table, indices, values) is written on the transfer
        stream after the copies, before the ready event (device slots only)."""
        if not loads:
            return None
        if validate_layout:
            for bundle, slot in loads:
                LayoutValidator.validate_copy_compatible(bundle, slot.as_bundle())
        if all(slot.w13.device.type == "cpu" and slot.w2.device.type == "cpu" for _, slot in loads):
            _host_wait(wait_event)
            for _, slot in loads:
                slot.state = SlotState.LOADING
            self._copy(tuple(loads), stream=None)
            for _, slot in loads:
                slot.state = SlotState.READY
            return None
        stream = self._get_h2d_stream(loads[0][1].w13.device)
        for _, slot in loads:
            slot.state = SlotState.LOADING
        done = torch.cuda.Event() if record_event else None
        self._copy(tuple(loads), stream=stream, wait_event=_torch_event(wait_event), done_event=done,
                   table_update=table_update)
        slots = tuple(slot for _, slot in loads)
        if done is None:
            stream.synchronize()
            for slot in slots:
                slot.state = SlotState.READY
            return None
        ready = TransferReadyEvent(done, tuple((s, s.lease()) for s in slots))
        self._pending_ready_events.append(ready)
        return ready

    def synchronize(self) -> None:
        """Wait for every queued copy and publish its slots READY."""
        if self._h2d_stream is not None:
            self._h2d_stream.synchronize()
        pending, self._pending_ready_events = self._pending_ready_events, []
        for ready in pending:
            ready.mark_ready()

    @property
    def stream(self) -> torch.cuda.Stream | None:
        return self._h2d_stream

    def _get_h2d_stream(self, device) -> torch.cuda.Stream:
        if self._h2d_stream is None:
            self._h2d_stream = torch.cuda.Stream(device=device)  # default priority
        return self._h2d_stream

    # -- copies -----------------------------------------------------------
    def _copy(self, loads: tuple[Load, ...], *, stream, wait_event=None, done_event=None,
              table_update=None) -> None:
        runs = contiguous_load_runs(loads)
        if stream is None:
            for run in runs:
                for bundle, slot in run:
                    slot.w13.copy_(bundle.w13)
                    slot.w2.copy_(bundle.w2)
            return
        from vllm_moe_offload_amd import native

        copies: list[tuple[int, int, int]] = []
        for run in runs:
            b0, s0 = run[0]
            n = len(run)
            for name in ("w13", "w2"):
                src, dst = getattr(b0, name), getattr(s0, name)
                nbytes = int(src.numel()) * int(src.element_size()) * n
                copies.append((int(dst.data_ptr()), int(src.data_ptr()), nbytes))
        native.stage_copy(copies, stream, wait_event=wait_event, done_event=done_event,
                          table_update=table_update)
        self.copies_issued += len(copies)
        self.bytes_issued += sum(c[2] for c in copies)


def _host_wait(wait_event) -> None:
    if wait_event is None:
        return
    ev = getattr(wait_event, "event", wait_event)
    sync = getattr(ev, "synchronize", None)
    if callable(sync):
        sync()


def _torch_event(wait_event):
    if wait_event is None:
        return None
    ev = getattr(wait_event, "event", wait_event)
    return ev if isinstance(ev, torch.cuda.Event) else None


def _next_contiguous(prev: torch.Tensor, cur: torch.Tensor) -> bool:
    if cur.device != prev.device or cur.dtype != prev.dtype:
        return False
    if tuple(cur.shape) != tuple(prev.shape) or tuple(cur.stride()) != tuple(prev.stride()):
        return False
    if not prev.is_contiguous():
        return False
    return int(cur.data_ptr()) - int(prev.data_ptr()) == int(prev.numel()) * int(prev.element_size())


def contiguous_load_runs(loads: tuple[Load, ...]) -> tuple[tuple[Load, ...], ...]:
    """Split loads into runs of consecutive experts landing in consecutive
    slots whose host and device bytes are both back to back."""
    runs: list[list[Load]] = []
    for bundle, slot in loads:
        if runs:
            pb, ps = runs[-1][-1]
            if (
                int(bundle.layer_id) == int(pb.layer_id)
                and int(bundle.expert_id) == int(pb.expert_id) + 1
                and int(slot.slot_id) == int(ps.slot_id) + 1
                and _next_contiguous(pb.w13, bundle.w13)
                and _next_contiguous(pb.w2, bundle.w2)
                and _next_contiguous(ps.w13, slot.w13)
                and _next_contiguous(ps.w2, slot.w2)
            ):
                runs[-1].append((bundle, slot))
                continue
        runs.append([(bundle, slot)])
    return tuple(tuple(r) for r in runs)
