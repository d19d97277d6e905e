"""Shared helpers for the tests (numpy <-> torch bf16, tolerances)."""

from __future__ import annotations

import numpy as np
import torch

from oracle.bf16 import bf16_to_f32, f32_to_bf16, normal_bf16  # noqa: F401


def to_dev_bf16(bits: np.ndarray, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


def from_dev_bf16(t: torch.Tensor) -> np.ndarray:
    """device bf16 tensor -> uint16 bits (numpy)."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def to_dev_i32(a: np.ndarray, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(device)


def rel_max_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max |got - ref| / RMS(ref), the tier's output tolerance measure."""
    ref = np.asarray(ref, dtype=np.float64)
    got = np.asarray(got, dtype=np.float64)
    rms = float(np.sqrt(np.mean(ref * ref)))
    return float(np.max(np.abs(got - ref))) / max(rms, 1e-30)


# BASELINE tolerance for bf16 layer outputs: max-abs <= 2e-2 * RMS(out)
OUT_TOL = 2e-2


def bf16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of bf16 numbers at |v| (f32 spacing scaled by 2^16)."""
    return np.abs(np.spacing(np.asarray(v, dtype=np.float32))) * np.float32(65536.0)


def ulp_mismatch_stats(got: np.ndarray, ref: np.ndarray, abs_floor: float = 0.0,
                       count_floor: float = 0.0) -> tuple[float, float]:
    """(fraction of elements off by more than one bf16 ulp + count_floor, max
    error in units of (one ulp + abs_floor)).  The floors absorb cancellation:
    an element that is a small difference of large terms carries the absolute
    rounding noise of its terms, not of its own magnitude."""
    got = np.asarray(got, dtype=np.float32)
    ref = np.asarray(ref, dtype=np.float32)
    ulp = np.maximum(bf16_ulp(ref), bf16_ulp(got))
    ulp = np.maximum(ulp, np.float32(2.0 ** -126))
    d = np.abs(got - ref)
    return float(np.mean(d > ulp + np.float32(count_floor))), float((d / (ulp + np.float32(abs_floor))).max())
