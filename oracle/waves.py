"""Wave-planner oracle (test infrastructure only).

Restates the canonical capacity-bounded wave packing of
moe_offload/phase_split.py:495-554 in a different form: a heap-free,
explicit scan that assigns experts in (-count, id) order to the wave with
(smallest load, smallest index) among waves with room, starting from
ceil(n / slots) empty waves and opening a new one only when all are full.

Pinned (tests/test_host_waves.py) by the reference golden vectors
((1,), (2, 5), (3, 4)) for {1:10, 2:9, 3:8, 4:1, 5:1} / 2 slots and
((1, 2, 4, 5),) for {5:100, 1:90, 2:80, 4:70} / 4 slots
(tests/test_phase_split_b2.py:44-117), and by invariants on random
histograms: every expert in exactly one wave, waves <= slots, wave count =
ceil(n / slots), waves sorted.
"""

from __future__ import annotations

import math


def plan_waves(counts: dict[int, int], num_slots: int) -> tuple[tuple[int, ...], ...]:
    active = {int(e): int(c) for e, c in counts.items() if int(c) > 0}
    if not active:
        return ()
    experts = sorted(active.items(), key=lambda kv: (-kv[1], kv[0]))
    waves: list[dict] = [{"members": [], "load": 0} for _ in range(math.ceil(len(experts) / num_slots))]
    for e, c in experts:
        room = [i for i, w in enumerate(waves) if len(w["members"]) < num_slots]
        if not room:
            waves.append({"members": [e], "load": c})
            continue
        i = min(room, key=lambda j: (waves[j]["load"], j))
        waves[i]["members"].append(e)
        waves[i]["load"] += c
    return tuple(tuple(sorted(w["members"])) for w in waves)
