"""Hot-path configuration of the slot-bank offload runtime.

Reference: moe_offload/config.py:32-167 (MoeOffloadConfig.from_env).  The
field names and the environment variable names are kept so an existing
deployment's settings carry over; the VLLM_ASCEND_MOE_OFFLOAD_* names are read
directly from the environment (the Ascend env registry is not needed), and a
VLLM_MOE_OFFLOAD_* spelling of each is accepted as well.  Knobs of subsystems
outside the hot path (AutoConfig, GMM bucket plans, tracing) are accepted and
ignored.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field

_PREFIXES = ("VLLM_ASCEND_MOE_OFFLOAD_", "VLLM_MOE_OFFLOAD_")


def _env(name: str, default: str) -> str:
    for p in _PREFIXES:
        v = os.getenv(p + name)
        if v is not None and v.strip() != "":
            return v.strip()
    return default


def _bool(name: str, default: bool) -> bool:
    return _env(name, "1" if default else "0").lower() in {"1", "true", "yes", "on"}


def _int(name: str, default: int) -> int:
    return int(_env(name, str(default)))


def _int_set(name: str) -> frozenset[int]:
    raw = _env(name, "")
    return frozenset(int(x) for x in raw.replace(" ", "").split(",") if x)


@dataclass(frozen=True)
class MoeOffloadConfig:
    enabled: bool = False
    trace_only: bool = False
    num_slots: int = 0
    async_load: bool = False
    resident_layer_ids: frozenset[int] = field(default_factory=frozenset)
    graph_compatible_offload: bool = False
    offload_stage_seam: bool = False
    b2_wave_prefill: bool = False
    pin_host_memory: bool | None = None
    transfer_aware_wave_schedule: bool = True
    prefill_prefetch_depth: int = 1
    prefill_buffer_count: int = 2
    b2_avoid_mixed_wave_d2d: bool = True
    max_num_seqs_hint: int = 0
    profile_path: str = ""
    # expert parameters of offloaded layers are created in host memory and
    # the checkpoint loads straight into them (no full-layer device copy)
    cpu_first_load: bool = False
    # drop a layer's original expert tensors once its host store is complete
    release_original_expert_weights: bool = False
    # decode whose routed experts exceed the slots: the first num_slots run
    # from the bank, the rest (at most num_slots more) from a stage buffer in
    # a second pass of the same captured graph, instead of eager waves
    decode_overflow: bool = False
    # overflowing prefill: waves planned and staged on the device (no D2H of
    # the routed ids, no host step between the router and the expert MLP)
    device_wave_prefill: bool = False

    @classmethod
    def from_env(cls) -> "MoeOffloadConfig":
        pin = _env("PIN_HOST_MEMORY", "")
        return cls(
            enabled=_bool("ENABLED", False),
            trace_only=_bool("TRACE_ONLY", False),
            num_slots=_int("NUM_SLOTS", 0),
            async_load=_bool("ASYNC_LOAD", False),
            resident_layer_ids=_int_set("RESIDENT_LAYER_IDS"),
            graph_compatible_offload=_bool("GRAPH_COMPATIBLE", False),
            offload_stage_seam=_bool("STAGE_SEAM", False),
            b2_wave_prefill=_bool("B2_WAVE_PREFILL", False),
            pin_host_memory=None if pin == "" else pin.lower() in {"1", "true", "yes", "on"},
            transfer_aware_wave_schedule=_bool("TRANSFER_AWARE_SCHEDULE", True),
            prefill_prefetch_depth=_int("PREFILL_PREFETCH_DEPTH", 1),
            prefill_buffer_count=_int("PREFILL_BUFFER_COUNT", 2),
            b2_avoid_mixed_wave_d2d=_bool("B2_AVOID_MIXED_D2D", True),
            max_num_seqs_hint=_int("MAX_NUM_SEQS_HINT", 0),
            profile_path=_env("PROFILE_PATH", ""),
            cpu_first_load=_bool("CPU_FIRST_LOAD", False),
            release_original_expert_weights=_bool("RELEASE_ORIGINAL_EXPERT_WEIGHTS", False),
            decode_overflow=_bool("DECODE_OVERFLOW", False),
            device_wave_prefill=_bool("DEVICE_WAVE_PREFILL", False),
        )

    @property
    def should_pin_host_memory(self) -> bool:
        return bool(self.async_load) if self.pin_host_memory is None else bool(self.pin_host_memory)

    @property
    def effective_prefill_prefetch_depth(self) -> int:
        return max(0, int(self.prefill_prefetch_depth))

    @property
    def effective_prefill_buffer_count(self) -> int:
        return max(1, int(self.prefill_buffer_count))

    def is_resident_layer(self, layer_id: int) -> bool:
        return int(layer_id) in self.resident_layer_ids
