"""Address-stable expert slot bank in HBM.

Two device tensors hold every physical slot for the life of the process:
w13_slots [P, 2I, H] and w2_slots [P, H, I] (bf16, checkpoint layout, K
contiguous so the gfx950 GEMV/MFMA kernels stream rows with 16-byte loads).
Rows [0, num_slots) are the dynamic routed cache; rows after it are pinned
shared experts that LRU can never pick.  Slot ownership is versioned: every
reassignment bumps the slot's version, and a lease (slot, owner, version)
detects stale completions.

Reference: moe_offload/slot_bank.py:27-335.  Allocation policy kept exactly:
a resident expert is touched; otherwise the lowest-id EMPTY slot; otherwise
the READY slot with the smallest (last_used_step, slot_id); LOADING and
COMPUTING slots are never reassigned.
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import Enum

import torch

from vllm_moe_offload_amd.moe_offload.expert_key import ExpertKey
from vllm_moe_offload_amd.moe_offload.host_store import ExpertWeightBundle


class SlotState(str, Enum):
    EMPTY = "empty"
    LOADING = "loading"
    READY = "ready"
    COMPUTING = "computing"


@dataclass(frozen=True)
class SlotLease:
    """One ownership interval of a slot: (slot, owner, version)."""

    slot_id: int
    expert_key: ExpertKey
    version: int


@dataclass
class ExpertSlot:
    slot_id: int
    w13: torch.Tensor
    w2: torch.Tensor
    state: SlotState = SlotState.EMPTY
    expert_key: ExpertKey | None = None
    version: int = 0
    last_used_step: int = -1

    def as_bundle(self) -> ExpertWeightBundle:
        key = self.expert_key or ExpertKey(-1, -1)
        return ExpertWeightBundle(key.layer_id, key.expert_id, self.w13, self.w2)

    def lease(self) -> SlotLease:
        if self.expert_key is None:
            raise RuntimeError(f"slot {self.slot_id} has no owner")
        return SlotLease(int(self.slot_id), self.expert_key, int(self.version))

    def matches_lease(self, lease: SlotLease) -> bool:
        return (
            int(self.slot_id) == int(lease.slot_id)
            and self.expert_key == lease.expert_key
            and int(self.version) == int(lease.version)
        )


def _nbytes(t: torch.Tensor) -> int:
    return int(t.numel()) * int(t.element_size())


class ExpertSlotBank:
    def __init__(
        self,
        num_slots: int,
        w13_shape: tuple[int, ...],
        w2_shape: tuple[int, ...],
        *,
        dtype: torch.dtype,
        device: torch.device,
        pinned_logical_ids: tuple[int, ...] = (),
    ) -> None:
        if num_slots <= 0:
            raise ValueError("num_slots must be greater than 0")
        pinned = tuple(int(e) for e in pinned_logical_ids)
        if len(set(pinned)) != len(pinned):
            raise ValueError("pinned logical expert ids must be unique")
        if any(e < 0 for e in pinned):
            raise ValueError("pinned logical expert ids must be non-negative")
        self.num_dynamic_slots = int(num_slots)
        self.pinned_logical_ids = pinned
        self._pinned_slot = {e: int(num_slots) + i for i, e in enumerate(pinned)}
        rows = int(num_slots) + len(pinned)
        self.w13_slots = torch.empty((rows, *w13_shape), dtype=dtype, device=device)
        self.w2_slots = torch.empty((rows, *w2_shape), dtype=dtype, device=device)
        self.slots = [
            ExpertSlot(slot_id=i, w13=self.w13_slots[i], w2=self.w2_slots[i]) for i in range(num_slots)
        ]
        self._resident: dict[ExpertKey, int] = {}
        self._resident_by_expert_id: dict[int, int] = {}

    # -- geometry ---------------------------------------------------------
    @property
    def physical_expert_count(self) -> int:
        return int(self.w13_slots.shape[0])

    @property
    def pinned_slot_ids(self) -> tuple[int, ...]:
        return tuple(self._pinned_slot[e] for e in self.pinned_logical_ids)

    @property
    def dynamic_bytes(self) -> int:
        n = self.num_dynamic_slots
        return _nbytes(self.w13_slots[:n]) + _nbytes(self.w2_slots[:n])

    @property
    def pinned_bytes(self) -> int:
        n = self.num_dynamic_slots
        return _nbytes(self.w13_slots[n:]) + _nbytes(self.w2_slots[n:])

    @property
    def total_bytes(self) -> int:
        return _nbytes(self.w13_slots) + _nbytes(self.w2_slots)

    def pinned_slot_for_logical_id(self, logical_id: int) -> int | None:
        return self._pinned_slot.get(int(logical_id))

    # -- pinned shared suffix --------------------------------------------
    def install_pinned_weights(self, w13: torch.Tensor, w2: torch.Tensor) -> None:
        """Copy the always-resident shared rows into the suffix."""
        count = len(self.pinned_logical_ids)
        if count == 0:
            if w13.numel() or w2.numel():
                raise ValueError("cannot install pinned weights into a routed-only bank")
            return
        exp13 = tuple(int(d) for d in self.w13_slots.shape[1:])
        exp2 = tuple(int(d) for d in self.w2_slots.shape[1:])
        if (
            int(w13.shape[0]) != count
            or tuple(int(d) for d in w13.shape[1:]) != exp13
            or int(w2.shape[0]) != count
            or tuple(int(d) for d in w2.shape[1:]) != exp2
        ):
            raise ValueError(
                "pinned shared weight layout does not match slot bank: "
                f"w13={tuple(w13.shape)} expected=({count}, {exp13}); "
                f"w2={tuple(w2.shape)} expected=({count}, {exp2})"
            )
        with torch.no_grad():
            self.w13_slots[self.num_dynamic_slots:].copy_(w13)
            self.w2_slots[self.num_dynamic_slots:].copy_(w2)

    def copy_pinned_weights_from(self, source: "ExpertSlotBank") -> None:
        if self.pinned_logical_ids != source.pinned_logical_ids:
            raise ValueError("cannot copy pinned weights across different logical layouts")
        if not self.pinned_logical_ids:
            return
        with torch.no_grad():
            self.w13_slots[self.num_dynamic_slots:].copy_(source.w13_slots[source.num_dynamic_slots:])
            self.w2_slots[self.num_dynamic_slots:].copy_(source.w2_slots[source.num_dynamic_slots:])

    def install_pinned_log2phy(self, log2phy: torch.Tensor) -> None:
        for logical_id, slot_id in self._pinned_slot.items():
            if logical_id >= int(log2phy.numel()):
                raise ValueError(
                    f"log2phy does not cover pinned logical expert {logical_id}; size={int(log2phy.numel())}"
                )
            log2phy[logical_id] = slot_id

    # -- ownership ----------------------------------------------------------
    def _take(self, slot: ExpertSlot, key: ExpertKey, step_id: int, *, index: bool) -> ExpertSlot:
        if slot.expert_key is not None:
            self._resident.pop(slot.expert_key, None)
            self._resident_by_expert_id.pop(int(slot.expert_key.expert_id), None)
        slot.expert_key = key
        slot.state = SlotState.LOADING
        slot.version += 1
        slot.last_used_step = int(step_id)
        if index:
            self._resident[key] = slot.slot_id
            self._resident_by_expert_id[int(key.expert_id)] = slot.slot_id
        return slot

    def allocate_for(self, expert_key: ExpertKey, *, step_id: int) -> ExpertSlot:
        """Touch a resident expert or reserve a slot for it (state LOADING)."""
        resident = self._resident.get(expert_key)
        if resident is not None:
            slot = self.slots[resident]
            slot.last_used_step = int(step_id)
            return slot
        slot = self._first_empty_slot() or self._lru_evictable_slot()
        if slot is None:
            raise RuntimeError(f"no evictable expert slots; states={self.state_counts()}")
        return self._take(slot, expert_key, step_id, index=True)

    def assign_slot(self, slot_id: int, expert_key: ExpertKey, *, step_id: int) -> ExpertSlot:
        """Place expert_key in a given slot (moving it if resident elsewhere)."""
        slot = self.slots[int(slot_id)]
        self._require_reassignable(slot)
        other = self._resident.get(expert_key)
        if other is not None and other != int(slot_id):
            old = self.slots[other]
            old.expert_key = None
            old.state = SlotState.EMPTY
            self._resident.pop(expert_key, None)
            self._resident_by_expert_id.pop(int(expert_key.expert_id), None)
        if slot.expert_key == expert_key:
            slot.version += 1
            slot.last_used_step = int(step_id)
            slot.state = SlotState.LOADING
            self._resident[expert_key] = slot.slot_id
            self._resident_by_expert_id[int(expert_key.expert_id)] = slot.slot_id
            return slot
        return self._take(slot, expert_key, step_id, index=True)

    def assign_transient_slot(self, slot_id: int, expert_key: ExpertKey, *, step_id: int) -> ExpertSlot:
        """Place expert_key in a stage-bank slot without indexing it."""
        slot = self.slots[int(slot_id)]
        self._require_reassignable(slot)
        return self._take(slot, expert_key, step_id, index=False)

    def mark_ready(self, slot_id: int) -> None:
        self.slots[int(slot_id)].state = SlotState.READY

    def mark_computing(self, slot_id: int) -> None:
        self.slots[int(slot_id)].state = SlotState.COMPUTING

    def mark_released(self, slot_id: int) -> None:
        self.slots[int(slot_id)].state = SlotState.EMPTY

    def lookup(self, expert_key: ExpertKey) -> ExpertSlot | None:
        i = self._resident.get(expert_key)
        return None if i is None else self.slots[i]

    def lookup_expert_id(self, expert_id: int) -> ExpertSlot | None:
        i = self._resident_by_expert_id.get(int(expert_id))
        return None if i is None else self.slots[i]

    def clear_slot(self, slot_id: int, *, force: bool = False) -> None:
        slot = self.slots[int(slot_id)]
        if not force and slot.state == SlotState.COMPUTING:
            raise RuntimeError(f"slot {slot.slot_id} is computing and cannot be reassigned")
        if slot.expert_key is not None:
            self._resident.pop(slot.expert_key, None)
            self._resident_by_expert_id.pop(int(slot.expert_key.expert_id), None)
        slot.expert_key = None
        slot.state = SlotState.EMPTY

    def state_counts(self) -> dict[str, int]:
        counts = {s.value: 0 for s in SlotState}
        for slot in self.slots:
            counts[slot.state.value] += 1
        return counts

    def _first_empty_slot(self) -> ExpertSlot | None:
        return next((s for s in self.slots if s.state == SlotState.EMPTY), None)

    def _lru_evictable_slot(self) -> ExpertSlot | None:
        ready = [s for s in self.slots if s.state == SlotState.READY]
        return min(ready, key=lambda s: (s.last_used_step, s.slot_id)) if ready else None

    @staticmethod
    def _require_reassignable(slot: ExpertSlot) -> None:
        if slot.state in (SlotState.LOADING, SlotState.COMPUTING):
            raise RuntimeError(f"slot {slot.slot_id} is {slot.state.value} and cannot be reassigned")
