"""Logical-expert -> physical-slot mapping handed to the fused-MoE kernels.

ExpertSlotMapping carries the slot table (int32 [E_total], -1 = not
staged), the owner of every physical slot and the active slot ids.
PreparedSlotWeights hands the kernels w1 = the w13 slot bank, w2 = the w2
slot bank, the table and physical_expert_count = P (not E).  On the device
path the remap itself happens inside lmoe_permute, which counts pairs whose
id maps to no slot instead of reading slot[-1].

Reference: moe_offload/slot_mapping.py:41-187 (field names, the fail-closed
checks and their messages are the reference's interface).
"""

from __future__ import annotations

import os
from dataclasses import dataclass

import numpy as np
import torch

from vllm_moe_offload_amd.moe_offload.expert_key import ExpertKey
from vllm_moe_offload_amd.moe_offload.host_store import ExpertWeightBundle
from vllm_moe_offload_amd.moe_offload.layout import LayoutValidator
from vllm_moe_offload_amd.moe_offload.slot_bank import ExpertSlotBank, SlotState


def dedupe_preserve_order(values) -> tuple[int, ...]:
    return tuple(dict.fromkeys(int(v) for v in values))


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
        """A fresh table for READY resident experts: built on the host in one
        array, then one copy to `device`."""
        n_logical = int(num_logical_experts)
        if n_logical <= 0:
            raise ValueError("num_logical_experts must be greater than 0")
        active = dedupe_preserve_order(active_experts)
        table = np.full(n_logical, -1, dtype=np.int64)
        for e, s in zip(slot_bank.pinned_logical_ids, slot_bank.pinned_slot_ids):
            if e >= n_logical:
                raise ValueError(f"log2phy does not cover pinned logical expert {e}; size={n_logical}")
            table[e] = s
        slot_ids = []
        for e in active:
            if not 0 <= e < n_logical:
                raise ValueError(f"active expert {e} is outside num_logical_experts={n_logical}")
            slot = slot_bank.lookup(ExpertKey(int(layer_id), e))
            if slot is None:
                raise RuntimeError(f"active expert {e} is not resident in layer {int(layer_id)}")
            if slot.state != SlotState.READY:
                raise RuntimeError(f"active expert {e} slot {slot.slot_id} is not ready")
            table[e] = slot.slot_id
            slot_ids.append(slot.slot_id)
        dev_table = torch.from_numpy(table).to(dtype).to(device)
        return cls(int(layer_id), active, dev_table, tuple(slot_bank.owners()), tuple(slot_ids))

    def remap_topk_ids(self, topk_ids: torch.Tensor) -> torch.Tensor:
        """phys = log2phy[topk_ids]; fails closed on unstaged experts (always on
        the host, on the device when LATCHMOE_LOG2PHY_VALIDATE is set)."""
        if not self.log2phy_valid:
            raise RuntimeError(
                "remap_topk_ids called on a mapping whose logical_to_physical was "
                "not rebuilt (log2phy_valid=False); use the wave-plan physical ids"
            )
        phys = torch.take(self.logical_to_physical, topk_ids.long())
        validate = phys.device.type == "cpu" or any(
            os.environ.get(k) for k in ("LATCHMOE_LOG2PHY_VALIDATE", "SEW_LOG2PHY_VALIDATE"))
        if validate:
            unmapped = phys < 0
            if bool(unmapped.any().item()):
                missing = sorted(set(topk_ids[unmapped].detach().cpu().tolist()))
                raise RuntimeError(f"topk_ids contain experts without ready slots: {missing}")
        return phys


@dataclass(frozen=True)
class PreparedSlotWeights:
    w1: torch.Tensor
    w2: torch.Tensor
    log2phy: torch.Tensor
    physical_expert_count: int
    mapping: ExpertSlotMapping
    # decode overflow: the stage buffer (and its table) holding the routed
    # experts past the bank's capacity, run as a second pass
    overflow: "PreparedSlotWeights | None" = None

    def validate_backend_ready(self, *, expected_device_type: str) -> None:
        P = int(self.physical_expert_count)
        if P <= 0:
            raise ValueError("physical_expert_count must be greater than 0")
        for name, t in (("w1", self.w1), ("w2", self.w2)):
            if int(t.shape[0]) != P:
                raise ValueError(f"{name} physical expert count mismatch: {int(t.shape[0])} != {P}")
        LayoutValidator.validate_backend_ready(
            ExpertWeightBundle(self.mapping.layer_id, -1, self.w1, self.w2),
            expected_device_type=expected_device_type,
        )

    @classmethod
    def from_slot_bank(cls, *, slot_bank: ExpertSlotBank, mapping: ExpertSlotMapping) -> "PreparedSlotWeights":
        return cls(slot_bank.w13_slots, slot_bank.w2_slots, mapping.logical_to_physical,
                   slot_bank.physical_expert_count, mapping)
