"""Placement-plan adapter for an external MoE controller.

A controller may reorder the router-selected experts (the order in which the
staging controller reserves slots and issues copies); it may not add, drop or
duplicate an expert, and it never sees slot storage.

Reference: moe_offload/placement_plan.py:13-73 (PlacementPlanRequest,
PlacementPlan, resolve_placement_plan; the result must be an exact
permutation of the first-seen de-duplicated routed set).
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass


@dataclass(frozen=True)
class PlacementPlanRequest:
    """What the router decided for one layer, as shown to a provider."""

    layer_id: int
    routed_experts: tuple[int, ...]
    num_logical_experts: int


@dataclass(frozen=True)
class PlacementPlan:
    """A provider's staging order for the routed working set."""

    layer_id: int
    ordered_experts: tuple[int, ...]
    source: str = "external"


PlacementPlanProvider = Callable[[PlacementPlanRequest], "PlacementPlan | None"]


def _first_seen(values) -> tuple[int, ...]:
    seen: dict[int, None] = {}
    for v in values:
        seen.setdefault(int(v), None)
    return tuple(seen)


def resolve_placement_plan(
    provider: PlacementPlanProvider | None,
    *,
    layer_id: int,
    routed_experts: tuple[int, ...],
    num_logical_experts: int,
) -> tuple[int, ...]:
    """Return the staging order: the provider's plan if it is a permutation
    of the routed set, the routed order if there is no provider or no plan."""
    routed = _first_seen(routed_experts)
    if provider is None:
        return routed
    plan = provider(
        PlacementPlanRequest(
            layer_id=int(layer_id),
            routed_experts=routed,
            num_logical_experts=int(num_logical_experts),
        )
    )
    if plan is None:
        return routed
    if not isinstance(plan, PlacementPlan):
        raise TypeError("placement-plan provider must return PlacementPlan or None")
    if int(plan.layer_id) != int(layer_id):
        raise RuntimeError(f"placement plan targets layer {plan.layer_id}, expected {layer_id}")
    ordered = tuple(int(e) for e in plan.ordered_experts)
    if len(ordered) != len(routed) or sorted(ordered) != sorted(routed):
        raise RuntimeError(
            "placement plan must be a permutation of the routed expert set; "
            f"routed={routed}, planned={ordered}"
        )
    return ordered
