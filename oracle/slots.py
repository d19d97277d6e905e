"""Fixed-slot LRU staging oracle (test infrastructure only).

Restates the decode staging decision of moe_offload/runtime.py:1636-1936 with
ExpertSlotBank.allocate_for (slot_bank.py:211-232, 318-328) as a plain table
simulation, with no slot objects, leases or tensors: for each step, experts
in staging order; a resident expert is a hit and its last-use becomes the
step; a miss takes the lowest-id empty slot, else the resident slot with the
smallest (last_use, slot_id) among slots not reserved earlier in this step
(reserved = LOADING until the batch completes), evicting its owner; the
persistent log2phy is written for the step's experts only and never cleared.

Pinned (tests/test_host_waves.py) by the reference golden trajectory
active_slot_ids == (2, 3, 0) for steps (0, 1) then (2, 3, 4) on 4 slots
(tests/test_fixed_slot_lifecycle.py:29-68) and the log2phy vectors of
tests/test_prefill_stage_runtime.py:1740-1885.
"""

from __future__ import annotations


class LruSlotTable:
    def __init__(self, num_slots: int, num_experts: int) -> None:
        self.owner = [None] * num_slots       # slot -> expert
        self.last = [-1] * num_slots          # slot -> last use step
        self.log2phy = [-1] * num_experts
        self.step = -1

    def stage(self, experts) -> tuple[tuple[int, ...], tuple[tuple[int, int], ...]]:
        """Returns (slot per expert, loads as (expert, slot))."""
        self.step += 1
        reserved: set[int] = set()
        slots: list[int] = []
        loads: list[tuple[int, int]] = []
        for e in experts:
            cur = [s for s, o in enumerate(self.owner) if o == e]
            if cur and cur[0] not in reserved:
                s = cur[0]
                self.last[s] = self.step
            elif cur:
                s = cur[0]  # reserved earlier this step for the same expert
            else:
                empty = [s for s, o in enumerate(self.owner) if o is None]
                if empty:
                    s = empty[0]
                else:
                    cands = [s for s in range(len(self.owner)) if s not in reserved]
                    s = min(cands, key=lambda q: (self.last[q], q))
                self.owner[s] = e
                self.last[s] = self.step
                reserved.add(s)
                loads.append((e, s))
            slots.append(s)
        for e, s in zip(experts, slots):
            self.log2phy[e] = s
        return tuple(slots), tuple(loads)
