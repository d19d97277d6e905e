"""Expert copies into slots on a dedicated transfer stream.

A batch of loads becomes a list of byte ranges: consecutive loads whose
host rows and slot rows are both back to back merge into one range per
weight tensor.  The batch then goes to the device in one call:

  * lmoe_stage_gather (default): one gather-copy kernel launch on the
    transfer stream reads page-locked host rows (or device rows) and writes
    the slots at the host link's rate, with no per-copy command overhead,
    and writes the slot-table entries that publish the batch in the same
    launch;
  * lmoe_stage_copy: one hipMemcpyAsync per range, for sources the device
    cannot read directly (pageable host memory), or when the gather entry
    refuses a range.

One event recorded after the batch orders it before its consumer (the
compute stream waits on it before the slots are published READY).  A ready
event carries the (slot, owner, version) of every slot it fills, so a late
completion for a slot that changed owner fails instead of publishing.

Reference: moe_offload/transfer_engine.py:29-342 (TransferReadyEvent and
its checks and messages, load_many_async's arguments, contiguous batching);
the reference copies with torch copy_ on its transfer stream.
"""

from __future__ import annotations

import os
from dataclasses import dataclass

import torch

from vllm_moe_offload_amd.moe_offload.host_store import ExpertWeightBundle
from vllm_moe_offload_amd.moe_offload.layout import LayoutValidator
from vllm_moe_offload_amd.moe_offload.slot_bank import ExpertSlot, SlotLease, SlotState

Load = tuple[ExpertWeightBundle, ExpertSlot]


@dataclass
class TransferReadyEvent:
    """One copy batch in flight: the event recorded after its copies on the
    transfer stream, and the (slot, lease) pairs it fills.  Completing it
    (a consumer stream's wait, or the host's) checks that every slot still
    holds the lease it was issued for and moves the slots to READY."""

    event: object | None
    leases: tuple[tuple[ExpertSlot, SlotLease], ...]
    completed: bool = False
    consumer_wait_installed: bool = False

    def _check_owners(self) -> None:
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

    def install_consumer_dependency(self, consumer_stream) -> None:
        """The consumer stream waits for the batch, then its slots are READY."""
        if self.completed:
            return
        self._check_owners()
        if self.event is not None:
            consumer_stream.wait_event(self.event)
        self.consumer_wait_installed = True
        self.mark_ready()

    def mark_ready(self) -> None:
        if self.completed:
            return
        self._check_owners()
        for slot, _ in self.leases:
            slot.state = SlotState.READY
        self.completed = True


def _span(t: torch.Tensor) -> tuple[int, int]:
    return int(t.data_ptr()), int(t.numel()) * int(t.element_size())


def contiguous_load_runs(loads) -> tuple[tuple[Load, ...], ...]:
    """Group loads into runs whose host bytes and slot bytes are both back to
    back, for w13 and for w2 (each run is then one range per tensor)."""
    runs: list[list[Load]] = []
    ends = None  # (host w13 end, host w2 end, slot w13 end, slot w2 end) of the open run
    for bundle, slot in loads:
        spans = (_span(bundle.w13), _span(bundle.w2), _span(slot.w13), _span(slot.w2))
        dense = all(t.is_contiguous() for t in (bundle.w13, bundle.w2, slot.w13, slot.w2))
        starts = tuple(p for p, _ in spans)
        if runs and dense and ends == starts and bundle.w13.device == runs[-1][-1][0].w13.device:
            runs[-1].append((bundle, slot))
        else:
            runs.append([(bundle, slot)])
        ends = tuple(p + n for p, n in spans) if dense else None
    return tuple(tuple(r) for r in runs)


def copy_ranges(loads) -> list[tuple[int, int, int]]:
    """(dst, src, bytes) per weight tensor per contiguous run."""
    out = []
    for run in contiguous_load_runs(loads):
        b0, s0 = run[0]
        for src, dst in ((b0.w13, s0.w13), (b0.w2, s0.w2)):
            out.append((int(dst.data_ptr()), int(src.data_ptr()), _span(src)[1] * len(run)))
    return out


class TransferEngine:
    def __init__(self) -> None:
        self._stream: torch.cuda.Stream | None = None
        self._in_flight: list[TransferReadyEvent] = []
        self.bytes_issued = 0
        self.copies_issued = 0
        self.batches_gathered = 0  # batches the gather kernel carried
        # "gather": page-locked sources go through the gather-copy kernel;
        # "sdma": every batch goes to the copy engines (hipMemcpyAsync),
        # which leave the compute units to the kernels they overlap
        self.copy_engine = os.environ.get("LATCHMOE_COPY_ENGINE", "gather")

    # -- synchronous -------------------------------------------------------
    def load_sync(self, bundle: ExpertWeightBundle, slot: ExpertSlot) -> None:
        self.load_many_sync([(bundle, slot)])

    def load_many_sync(self, loads: list[Load], *, validate_layout: bool = True) -> None:
        if not loads:
            return
        if validate_layout:
            for bundle, slot in loads:
                LayoutValidator.validate_copy_compatible(bundle, slot.as_bundle())
        for _, slot in loads:
            slot.state = SlotState.LOADING
        for run in contiguous_load_runs(loads):
            for bundle, slot in run:
                slot.w13.copy_(bundle.w13)
                slot.w2.copy_(bundle.w2)
        for _, slot in loads:
            slot.state = SlotState.READY
        self.copies_issued += 2 * len(loads)
        self.bytes_issued += sum(b.nbytes for b, _ in loads)

    # -- asynchronous ------------------------------------------------------
    def load_async(self, bundle: ExpertWeightBundle, slot: ExpertSlot, *, wait_event=None,
                   record_event: bool = True):
        return self.load_many_async([(bundle, slot)], wait_event=wait_event, record_event=record_event)

    def load_many_async(self, loads: list[Load], *, wait_event=None, record_event: bool = True,
                        validate_layout: bool = True, table_update=None):
        """Queue the loads on the transfer stream after wait_event (an event
        or a sequence of events); returns a TransferReadyEvent
        (None when the copy completed synchronously).  table_update =
        (device int32 table, indices, values[, fill]) is written by the same
        batch, before its ready event (device slots only); fill=True writes
        -1 into every other entry."""
        if not loads:
            return None
        if validate_layout:
            for bundle, slot in loads:
                LayoutValidator.validate_copy_compatible(bundle, slot.as_bundle())
        if all(slot.w13.device.type == "cpu" for _, slot in loads):
            _host_wait(wait_event)
            self.load_many_sync(loads, validate_layout=False)
            return None
        stream = self._transfer_stream(loads[0][1].w13.device)
        for _, slot in loads:
            slot.state = SlotState.LOADING
        done = torch.cuda.Event() if record_event else None
        ranges = copy_ranges(loads)
        self._issue(ranges, stream, _torch_events(wait_event), done, table_update,
                    direct=all(b.host_pinned or b.w13.device.type == "cuda" for b, _ in loads))
        self.copies_issued += len(ranges)
        self.bytes_issued += sum(r[2] for r in ranges)
        slots = tuple(slot for _, slot in loads)
        if done is None:
            stream.synchronize()
            for slot in slots:
                slot.state = SlotState.READY
            return None
        ready = TransferReadyEvent(done, tuple((s, s.lease()) for s in slots))
        self._in_flight.append(ready)
        return ready

    def _issue(self, ranges, stream, wait_events, done, table_update, *, direct: bool) -> None:
        from vllm_moe_offload_amd import native

        for ev in wait_events:
            stream.wait_event(ev)
        if direct and self.copy_engine == "gather" and native.stage_gather(ranges, stream, table_update=table_update):
            self.batches_gathered += 1
        else:
            native.stage_copy(ranges, stream, table_update=table_update)
        if done is not None:
            done.record(stream)

    def synchronize(self) -> None:
        """Wait for every queued copy and publish its slots READY."""
        if self._stream is not None:
            self._stream.synchronize()
        in_flight, self._in_flight = self._in_flight, []
        for ready in in_flight:
            ready.mark_ready()

    @property
    def stream(self) -> torch.cuda.Stream | None:
        return self._stream

    def _transfer_stream(self, device) -> torch.cuda.Stream:
        if self._stream is None:
            self._stream = torch.cuda.Stream(device=device)  # default priority
        return self._stream


def _waits(wait_event) -> tuple:
    """wait_event as a tuple: one event (or TransferReadyEvent), a sequence
    of them, or None."""
    if wait_event is None:
        return ()
    return tuple(wait_event) if isinstance(wait_event, (tuple, list)) else (wait_event,)


def _host_wait(wait_event) -> None:
    for w in _waits(wait_event):
        ev = getattr(w, "event", w)
        sync = getattr(ev, "synchronize", None)
        if callable(sync):
            sync()


def _torch_events(wait_event) -> tuple:
    return tuple(ev for ev in (getattr(w, "event", w) for w in _waits(wait_event))
                 if isinstance(ev, torch.cuda.Event))
