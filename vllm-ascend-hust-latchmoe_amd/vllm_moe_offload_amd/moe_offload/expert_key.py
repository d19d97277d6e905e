"""Identity of one routed expert of one layer.

Reference: moe_offload/expert_key.py (frozen, ordered (layer_id, expert_id));
kept field-for-field so keys compare and sort the same way.
"""

from dataclasses import dataclass


@dataclass(frozen=True, order=True)
class ExpertKey:
    layer_id: int
    expert_id: int
