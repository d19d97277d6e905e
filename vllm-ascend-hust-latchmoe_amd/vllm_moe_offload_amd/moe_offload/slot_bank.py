"""Address-stable expert slot bank in HBM with its slot table.

Storage: two device tensors hold every physical slot for the life of the
process, w13_slots [P, 2I, H] and w2_slots [P, H, I] (bf16, checkpoint
layout, K contiguous for the gfx950 GEMV / MFMA kernels).  Rows [0,
num_slots) are the dynamic cache; rows past it hold pinned shared experts
that are never reassigned.

Bookkeeping is a struct of arrays, one entry per dynamic slot: state code,
owning expert id (and the layer of its key), version and last use, plus an
expert-id -> slot residency array.  The decode staging plans a whole layer
in one call of the native planner (lmoe_slot_plan, which mutates these
arrays in place); the per-slot methods below work on the same arrays.
`slots[i]` is a view of entry i, not a copy: reading or assigning
`slots[i].state` reads or writes the table.

Reference: moe_offload/slot_bank.py:27-336 (SlotState, SlotLease,
ExpertSlot, ExpertSlotBank).  The allocation policy is the reference's,
because its tests pin its exact choices: a resident expert is touched;
otherwise the lowest-id EMPTY slot; otherwise the READY slot with the
smallest (last use, slot id); LOADING and COMPUTING slots are never taken.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from enum import Enum

import numpy as np
import torch

from vllm_moe_offload_amd.moe_offload.expert_key import ExpertKey
from vllm_moe_offload_amd.moe_offload.host_store import ExpertWeightBundle


class SlotState(str, Enum):
    EMPTY = "empty"
    LOADING = "loading"
    READY = "ready"
    COMPUTING = "computing"


# state codes of the slot table (shared with the native planner)
_CODES = (SlotState.EMPTY, SlotState.LOADING, SlotState.READY, SlotState.COMPUTING)
_CODE_OF = {st: np.int8(i) for i, st in enumerate(_CODES)}
EMPTY, LOADING, READY, COMPUTING = (int(_CODE_OF[s]) for s in _CODES)


@dataclass(frozen=True)
class SlotLease:
    """One ownership interval of a slot: (slot, owner, version)."""

    slot_id: int
    expert_key: ExpertKey
    version: int


class ExpertSlot:
    """View of one slot-table entry and its weight rows."""

    __slots__ = ("_bank", "slot_id", "w13", "w2")

    def __init__(self, bank: "ExpertSlotBank", slot_id: int) -> None:
        self._bank = bank
        self.slot_id = int(slot_id)
        self.w13 = bank.w13_slots[slot_id]
        self.w2 = bank.w2_slots[slot_id]

    @property
    def state(self) -> SlotState:
        return _CODES[int(self._bank._state[self.slot_id])]

    @state.setter
    def state(self, value: SlotState) -> None:
        self._bank._state[self.slot_id] = _CODE_OF[SlotState(value)]

    @property
    def expert_key(self) -> ExpertKey | None:
        return self._bank._key_of(self.slot_id)

    @property
    def version(self) -> int:
        return int(self._bank._version[self.slot_id])

    @property
    def last_used_step(self) -> int:
        return int(self._bank._last_used[self.slot_id])

    @last_used_step.setter
    def last_used_step(self, step: int) -> None:
        self._bank._last_used[self.slot_id] = int(step)

    def as_bundle(self) -> ExpertWeightBundle:
        key = self.expert_key or ExpertKey(-1, -1)
        return ExpertWeightBundle(key.layer_id, key.expert_id, self.w13, self.w2)

    def lease(self) -> SlotLease:
        key = self.expert_key
        if key is None:
            raise RuntimeError(f"slot {self.slot_id} has no owner")
        return SlotLease(self.slot_id, key, self.version)

    def matches_lease(self, lease: SlotLease) -> bool:
        b = self._bank
        s = self.slot_id
        return (
            s == int(lease.slot_id)
            and int(b._owner[s]) == int(lease.expert_key.expert_id)
            and int(b._owner_layer[s]) == int(lease.expert_key.layer_id)
            and int(b._version[s]) == int(lease.version)
        )

    def __repr__(self) -> str:
        return f"ExpertSlot({self.slot_id}, {self.state.value}, {self.expert_key}, v{self.version})"


def _nbytes(t: torch.Tensor) -> int:
    return int(t.numel()) * int(t.element_size())


_PLAN_FN = None


def _native_plan():
    """ctypes handle of lmoe_slot_plan (host code of the kernel library)."""
    global _PLAN_FN
    if _PLAN_FN is None:
        from vllm_moe_offload_amd import native

        fn = native.load_library().lmoe_slot_plan
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                               ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
        _PLAN_FN = fn
    return _PLAN_FN


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
        n = int(num_slots)
        self.num_dynamic_slots = n
        self.pinned_logical_ids = pinned
        rows = n + len(pinned)
        self.w13_slots = torch.empty((rows, *w13_shape), dtype=dtype, device=device)
        self.w2_slots = torch.empty((rows, *w2_shape), dtype=dtype, device=device)
        # the slot table
        self._state = np.zeros(n, dtype=np.int8)
        self._owner = np.full(n, -1, dtype=np.int32)
        self._owner_layer = np.full(n, -1, dtype=np.int64)
        self._version = np.zeros(n, dtype=np.int64)
        self._last_used = np.full(n, -1, dtype=np.int64)
        self._slot_of = np.full(max(1, max(pinned, default=0) + 1), -1, dtype=np.int32)
        self.slots = [ExpertSlot(self, i) for i in range(n)]
        # planner scratch (one staging at a time) and the table's addresses
        self._plan_ids = np.empty(n, dtype=np.int32)
        self._plan_slots = np.empty(n, dtype=np.int32)
        self._plan_miss = np.empty(n, dtype=np.int8)
        self._mixed_layers = False  # keys of more than one layer held (tests)
        self._layer_seen = -1
        self._addr = None

    # -- geometry ---------------------------------------------------------
    @property
    def physical_expert_count(self) -> int:
        return int(self.w13_slots.shape[0])

    @property
    def pinned_slot_ids(self) -> tuple[int, ...]:
        return tuple(range(self.num_dynamic_slots, self.num_dynamic_slots + len(self.pinned_logical_ids)))

    @property
    def dynamic_bytes(self) -> int:
        n = self.num_dynamic_slots
        return _nbytes(self.w13_slots[:n]) + _nbytes(self.w2_slots[:n])

    @property
    def pinned_bytes(self) -> int:
        return self.total_bytes - self.dynamic_bytes

    @property
    def total_bytes(self) -> int:
        return _nbytes(self.w13_slots) + _nbytes(self.w2_slots)

    def pinned_slot_for_logical_id(self, logical_id: int) -> int | None:
        try:
            return self.num_dynamic_slots + self.pinned_logical_ids.index(int(logical_id))
        except ValueError:
            return None

    # -- pinned shared suffix --------------------------------------------
    def install_pinned_weights(self, w13: torch.Tensor, w2: torch.Tensor) -> None:
        """Copy the always-resident shared rows into the suffix."""
        n_pin = len(self.pinned_logical_ids)
        if n_pin == 0:
            if w13.numel() or w2.numel():
                raise ValueError("cannot install pinned weights into a routed-only bank")
            return
        want13 = (n_pin, *self.w13_slots.shape[1:])
        want2 = (n_pin, *self.w2_slots.shape[1:])
        if tuple(w13.shape) != tuple(want13) or tuple(w2.shape) != tuple(want2):
            raise ValueError(
                "pinned shared weight layout does not match slot bank: "
                f"w13={tuple(w13.shape)} expected={tuple(want13)}; w2={tuple(w2.shape)} expected={tuple(want2)}"
            )
        with torch.no_grad():
            self.w13_slots[self.num_dynamic_slots:].copy_(w13)
            self.w2_slots[self.num_dynamic_slots:].copy_(w2)

    def copy_pinned_weights_from(self, source: "ExpertSlotBank") -> None:
        if self.pinned_logical_ids != source.pinned_logical_ids:
            raise ValueError("cannot copy pinned weights across different logical layouts")
        if self.pinned_logical_ids:
            with torch.no_grad():
                self.w13_slots[self.num_dynamic_slots:].copy_(source.w13_slots[source.num_dynamic_slots:])
                self.w2_slots[self.num_dynamic_slots:].copy_(source.w2_slots[source.num_dynamic_slots:])

    def install_pinned_log2phy(self, log2phy: torch.Tensor) -> None:
        """Write the pinned suffix's entries of a slot table (one indexed write)."""
        if not self.pinned_logical_ids:
            return
        ids = list(self.pinned_logical_ids)
        too_big = [e for e in ids if e >= int(log2phy.numel())]
        if too_big:
            raise ValueError(f"log2phy does not cover pinned logical expert {too_big[0]}; size={int(log2phy.numel())}")
        idx = torch.tensor(ids, dtype=torch.long)
        val = torch.tensor(self.pinned_slot_ids, dtype=log2phy.dtype)
        log2phy.index_put_((idx.to(log2phy.device),), val.to(log2phy.device))

    # -- slot table ------------------------------------------------------------
    def _key_of(self, s: int) -> ExpertKey | None:
        e = int(self._owner[s])
        return None if e < 0 else ExpertKey(int(self._owner_layer[s]), e)

    def _ensure_expert(self, e: int) -> None:
        if e >= self._slot_of.size:
            grown = np.full(max(e + 1, 2 * self._slot_of.size), -1, dtype=np.int32)
            grown[: self._slot_of.size] = self._slot_of
            self._slot_of = grown
            self._addr = None

    def _addresses(self) -> tuple[int, ...]:
        if self._addr is None:
            arrs = (self._state, self._owner, self._version, self._last_used, self._slot_of,
                    self._plan_ids, self._plan_slots, self._plan_miss)
            self._addr = tuple(int(a.__array_interface__["data"][0]) for a in arrs)
        return self._addr

    def _resident_slot(self, key: ExpertKey) -> int:
        e = int(key.expert_id)
        if e < 0 or e >= self._slot_of.size:
            return -1
        s = int(self._slot_of[e])
        if s < 0 or int(self._owner[s]) != e or int(self._owner_layer[s]) != int(key.layer_id):
            return -1
        return s

    def _unindex(self, s: int) -> None:
        e = int(self._owner[s])
        if 0 <= e < self._slot_of.size and int(self._slot_of[e]) == s:
            self._slot_of[e] = -1

    def _claim(self, s: int, key: ExpertKey, step_id: int, *, indexed: bool) -> ExpertSlot:
        self._unindex(s)
        e = int(key.expert_id)
        if self._layer_seen not in (-1, int(key.layer_id)):
            self._mixed_layers = True
        self._layer_seen = int(key.layer_id)
        self._owner[s] = e
        self._owner_layer[s] = int(key.layer_id)
        self._state[s] = LOADING
        self._version[s] += 1
        self._last_used[s] = int(step_id)
        if indexed:
            self._ensure_expert(e)
            self._slot_of[e] = s
        return self.slots[s]

    def _victim(self) -> int:
        """Lowest-id EMPTY slot, else the READY slot of smallest (last use,
        id); -1 when every slot is LOADING or COMPUTING."""
        empty = np.flatnonzero(self._state == EMPTY)
        if empty.size:
            return int(empty[0])
        ready = self._state == READY
        if not ready.any():
            return -1
        return int(np.argmin(np.where(ready, self._last_used, np.iinfo(np.int64).max)))

    def allocate_for(self, expert_key: ExpertKey, *, step_id: int) -> ExpertSlot:
        """Touch a resident expert or reserve a slot for it (state LOADING)."""
        s = self._resident_slot(expert_key)
        if s >= 0:
            self._last_used[s] = int(step_id)
            return self.slots[s]
        s = self._victim()
        if s < 0:
            raise RuntimeError(f"no evictable expert slots; states={self.state_counts()}")
        return self._claim(s, expert_key, step_id, indexed=True)

    def plan(self, layer_id: int, expert_ids, *, step_id: int) -> tuple[int, np.ndarray, np.ndarray]:
        """Hit / miss and slot reservation for a list of experts of one layer,
        in one native call (lmoe_slot_plan).  Returns (status, slot ids,
        miss flags): status >= 0 is the number of misses; -(j + 1) means
        expert j needs in-flight work drained first (experts before j are
        done; call again with the rest after draining)."""
        n = len(expert_ids)
        if n > self.num_dynamic_slots:
            raise ValueError(f"{n} experts to plan exceed num_slots={self.num_dynamic_slots}")
        ids = self._plan_ids[:n]
        ids[:] = expert_ids
        if n and int(ids.max()) >= self._slot_of.size:
            self._ensure_expert(int(ids.max()))
        layer_id = int(layer_id)
        if self._mixed_layers or self._layer_seen not in (-1, layer_id):
            # residency by expert id serves one layer: entries of other
            # layers' keys (test-only mixtures) leave the index first
            for s in np.flatnonzero((self._owner >= 0) & (self._owner_layer != layer_id)):
                self._unindex(int(s))
            self._mixed_layers = False
        a = self._addresses()
        st = _native_plan()(a[0], a[1], a[2], a[3], self.num_dynamic_slots, a[4], int(self._slot_of.size),
                            a[5], n, int(step_id), a[6], a[7])
        if st >= 1000:
            raise ValueError(f"slot planning refused the expert ids (status {st})")
        slot_ids = self._plan_slots[:n].copy()
        miss = self._plan_miss[:n].copy()
        done = n if st >= 0 else -st - 1
        self._owner_layer[slot_ids[:done][miss[:done] == 1]] = layer_id
        self._layer_seen = layer_id
        return int(st), slot_ids, miss

    def assign_slot(self, slot_id: int, expert_key: ExpertKey, *, step_id: int) -> ExpertSlot:
        """Place expert_key in a given slot (moving it if resident elsewhere)."""
        s = int(slot_id)
        self._require_reassignable(s)
        other = self._resident_slot(expert_key)
        if other >= 0 and other != s:
            self._unindex(other)
            self._owner[other] = -1
            self._owner_layer[other] = -1
            self._state[other] = EMPTY
        return self._claim(s, expert_key, step_id, indexed=True)

    def assign_transient_slot(self, slot_id: int, expert_key: ExpertKey, *, step_id: int) -> ExpertSlot:
        """Place expert_key in a stage-bank slot without indexing it."""
        s = int(slot_id)
        self._require_reassignable(s)
        return self._claim(s, expert_key, step_id, indexed=False)

    def mark_ready(self, slot_id: int) -> None:
        self._state[int(slot_id)] = READY

    def mark_computing(self, slot_id: int) -> None:
        self._state[int(slot_id)] = COMPUTING

    def mark_released(self, slot_id: int) -> None:
        self._state[int(slot_id)] = EMPTY

    def lookup(self, expert_key: ExpertKey) -> ExpertSlot | None:
        s = self._resident_slot(expert_key)
        return None if s < 0 else self.slots[s]

    def ready_resident_mask(self, expert_ids) -> np.ndarray:
        """Per expert id: resident in a dynamic slot and READY."""
        ids = np.asarray(expert_ids, dtype=np.int64).reshape(-1)
        ok = (ids >= 0) & (ids < self._slot_of.size)
        s = np.full(ids.shape, -1, dtype=np.int64)
        s[ok] = self._slot_of[ids[ok]]
        ok &= (s >= 0) & (s < self.num_dynamic_slots)
        idx = np.where(ok, s, 0)
        ok &= (self._owner[idx] == ids) & (self._state[idx] == READY)
        return ok

    def lookup_expert_id(self, expert_id: int) -> ExpertSlot | None:
        e = int(expert_id)
        if e < 0 or e >= self._slot_of.size:
            return None
        s = int(self._slot_of[e])
        return None if s < 0 or int(self._owner[s]) != e else self.slots[s]

    def clear_slot(self, slot_id: int, *, force: bool = False) -> None:
        s = int(slot_id)
        if not force and int(self._state[s]) == COMPUTING:
            raise RuntimeError(f"slot {s} is computing and cannot be reassigned")
        self._unindex(s)
        self._owner[s] = -1
        self._owner_layer[s] = -1
        self._state[s] = EMPTY

    def state_counts(self) -> dict[str, int]:
        counts = np.bincount(self._state, minlength=len(_CODES))
        return {st.value: int(counts[i]) for i, st in enumerate(_CODES)}

    def has_inflight(self) -> bool:
        """Any slot LOADING or COMPUTING."""
        return bool(((self._state == LOADING) | (self._state == COMPUTING)).any())

    def owners(self) -> list[int | None]:
        """Owning expert id of every physical slot (pinned suffix included)."""
        out: list[int | None] = [int(e) if e >= 0 else None for e in self._owner.tolist()]
        out.extend(int(e) for e in self.pinned_logical_ids)
        return out

    def _require_reassignable(self, s: int) -> None:
        code = int(self._state[s])
        if code in (LOADING, COMPUTING):
            raise RuntimeError(f"slot {s} is {_CODES[code].value} and cannot be reassigned")
