"""Copy-compatibility checks between a host-store bundle and a slot.

Reference: moe_offload/layout.py:42-75 — shape, dtype and stride must match
before a copy; device types are checked for backend readiness.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class LayoutSignature:
    shape: tuple[int, ...]
    dtype: torch.dtype
    stride: tuple[int, ...]
    device_type: str

    @classmethod
    def from_tensor(cls, t: torch.Tensor) -> "LayoutSignature":
        return cls(tuple(int(d) for d in t.shape), t.dtype, tuple(int(s) for s in t.stride()), t.device.type)


class LayoutValidator:
    @staticmethod
    def _check(name: str, src: torch.Tensor, dst: torch.Tensor) -> None:
        a, b = LayoutSignature.from_tensor(src), LayoutSignature.from_tensor(dst)
        for field in ("shape", "dtype", "stride"):
            if getattr(a, field) != getattr(b, field):
                raise ValueError(
                    f"{name} layout mismatch: {field} {getattr(a, field)} != {getattr(b, field)}"
                )

    @staticmethod
    def validate_copy_compatible(bundle, slot_bundle) -> None:
        LayoutValidator._check("w13", bundle.w13, slot_bundle.w13)
        LayoutValidator._check("w2", bundle.w2, slot_bundle.w2)

    @staticmethod
    def validate_bundle_matches_slot(bundle, slot_bundle) -> None:
        LayoutValidator.validate_copy_compatible(bundle, slot_bundle)
        for name in ("w13", "w2"):
            a, b = getattr(bundle, name), getattr(slot_bundle, name)
            if a.device.type != b.device.type:
                raise ValueError(f"{name} layout mismatch: device {a.device.type} != {b.device.type}")

    @staticmethod
    def validate_backend_ready(bundle, *, expected_device_type: str) -> None:
        for name in ("w13", "w2"):
            dev = getattr(bundle, name).device.type
            if dev != expected_device_type:
                raise ValueError(f"{name} backend device mismatch: {dev} != {expected_device_type}")
