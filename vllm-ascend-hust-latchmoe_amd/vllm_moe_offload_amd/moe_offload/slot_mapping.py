"""Logical-expert -> physical-slot mapping handed to the fused-MoE kernels.

Reference: moe_offload/slot_mapping.py:41-187.  ExpertSlotMapping carries the
log2phy table (int32 [E_total], -1 = not staged), the owner of every slot and
the active slot ids; PreparedSlotWeights hands the kernels w1 = w13 slot bank,
w2 = w2 slot bank, log2phy and physical_expert_count = P (not E).  On the
device path the remap itself happens inside lmoe_permute, which counts pairs
whose id maps to no slot instead of reading slot[-1].
"""

from __future__ import annotations

import os
from dataclasses import dataclass

import torch

from vllm_moe_offload_amd.moe_offload.expert_key import ExpertKey
from vllm_moe_offload_amd.moe_offload.host_store import ExpertWeightBundle
from vllm_moe_offload_amd.moe_offload.layout import LayoutValidator
from vllm_moe_offload_amd.moe_offload.slot_bank import ExpertSlotBank, SlotState


def dedupe_preserve_order(values) -> tuple[int, ...]:
    seen: dict[int, None] = {}
    for v in values:
        seen.setdefault(int(v), None)
    return tuple(seen)


@dataclass(frozen=True)
class ExpertSlotMapping:
    layer_id: int
    active_experts: tuple[int, ...]
    logical_to_physical: torch.Tensor
    slot_to_expert: tuple[int | None, ...]
    active_slot_ids: tuple[int, ...]
    # False when the table was deliberately not rebuilt (a wave routed by its
    # own per-wave table); such a mapping must not be used to remap ids.
    log2phy_valid: bool = True

    @classmethod
    def from_slot_bank(
        cls,
        *,
        layer_id: int,
        active_experts: tuple[int, ...],
        num_logical_experts: int,
        slot_bank: ExpertSlotBank,
        device: torch.device,
        dtype: torch.dtype = torch.int32,
    ) -> "ExpertSlotMapping":
        if num_logical_experts <= 0:
            raise ValueError("num_logical_experts must be greater than 0")
        layer_id = int(layer_id)
        active = dedupe_preserve_order(active_experts)
        table = torch.full((int(num_logical_experts),), -1, dtype=dtype, device=device)
        owners: list[int | None] = [None] * slot_bank.physical_expert_count
        slot_bank.install_pinned_log2phy(table)
        for logical_id in slot_bank.pinned_logical_ids:
            owners[int(slot_bank.pinned_slot_for_logical_id(logical_id))] = int(logical_id)
        slot_ids: list[int] = []
        for e in active:
            if e < 0 or e >= num_logical_experts:
                raise ValueError(f"active expert {e} is outside num_logical_experts={num_logical_experts}")
            slot = slot_bank.lookup(ExpertKey(layer_id, e))
            if slot is None:
                raise RuntimeError(f"active expert {e} is not resident in layer {layer_id}")
            if slot.state != SlotState.READY:
                raise RuntimeError(f"active expert {e} slot {slot.slot_id} is not ready")
            table[e] = int(slot.slot_id)
            slot_ids.append(int(slot.slot_id))
        for slot in slot_bank.slots:
            if slot.expert_key is not None:
                owners[slot.slot_id] = int(slot.expert_key.expert_id)
        return cls(layer_id, active, table, tuple(owners), tuple(slot_ids))

    def remap_topk_ids(self, topk_ids: torch.Tensor) -> torch.Tensor:
        """phys = log2phy[topk_ids]; fails closed on unstaged experts (always on
        the host, on the device when LATCHMOE_LOG2PHY_VALIDATE is set)."""
        if not self.log2phy_valid:
            raise RuntimeError(
                "remap_topk_ids called on a mapping whose logical_to_physical was "
                "not rebuilt (log2phy_valid=False); use the wave-plan physical ids"
            )
        remapped = self.logical_to_physical[topk_ids.long()]
        check = remapped.device.type == "cpu" or bool(
            os.environ.get("LATCHMOE_LOG2PHY_VALIDATE") or os.environ.get("SEW_LOG2PHY_VALIDATE")
        )
        if check and bool((remapped < 0).any().item()):
            missing = topk_ids[remapped < 0].detach().cpu().unique().tolist()
            raise RuntimeError(f"topk_ids contain experts without ready slots: {missing}")
        return remapped


@dataclass(frozen=True)
class PreparedSlotWeights:
    w1: torch.Tensor
    w2: torch.Tensor
    log2phy: torch.Tensor
    physical_expert_count: int
    mapping: ExpertSlotMapping

    def validate_backend_ready(self, *, expected_device_type: str) -> None:
        if self.physical_expert_count <= 0:
            raise ValueError("physical_expert_count must be greater than 0")
        if self.w1.shape[0] != self.physical_expert_count:
            raise ValueError(f"w1 physical expert count mismatch: {self.w1.shape[0]} != {self.physical_expert_count}")
        if self.w2.shape[0] != self.physical_expert_count:
            raise ValueError(f"w2 physical expert count mismatch: {self.w2.shape[0]} != {self.physical_expert_count}")
        LayoutValidator.validate_backend_ready(
            ExpertWeightBundle(self.mapping.layer_id, -1, self.w1, self.w2),
            expected_device_type=expected_device_type,
        )

    @classmethod
    def from_slot_bank(cls, *, slot_bank: ExpertSlotBank, mapping: ExpertSlotMapping) -> "PreparedSlotWeights":
        return cls(
            w1=slot_bank.w13_slots,
            w2=slot_bank.w2_slots,
            log2phy=mapping.logical_to_physical,
            physical_expert_count=slot_bank.physical_expert_count,
            mapping=mapping,
        )
