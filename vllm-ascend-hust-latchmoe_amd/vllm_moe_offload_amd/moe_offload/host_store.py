"""Host store of routed expert weights: one page-locked block per layer.

Each registered layer owns exactly two host tensors, w13 [E, 2I, H] and w2
[E, H, I] (checkpoint layout).  An expert is a pair of row views into them,
so a run of consecutive experts is one contiguous byte range of each tensor
(the copy planner merges such runs), and page-locked blocks can be read by
the device directly (the gather-copy kernel) as well as by the copy engines.
Pinning allocates page-locked memory and copies into it; existing memory is
never registered in place.  Layers registered from buffers the caller
already owns (CPU-first loading) are adopted without a copy.

Reference: moe_offload/host_store.py:25-291 (the class and field names,
register_layer's arguments and the report keys are its interface).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from vllm_moe_offload_amd.moe_offload.expert_key import ExpertKey


def _nbytes(t: torch.Tensor) -> int:
    return int(t.numel()) * int(t.element_size())


@dataclass(frozen=True)
class ExpertWeightBundle:
    layer_id: int
    expert_id: int
    w13: torch.Tensor
    w2: torch.Tensor
    w13_scale: torch.Tensor | None = None
    w2_scale: torch.Tensor | None = None
    # True when both tensors are page-locked host rows the device can read
    host_pinned: bool = False

    @property
    def key(self) -> ExpertKey:
        return ExpertKey(self.layer_id, self.expert_id)

    @property
    def nbytes(self) -> int:
        return _nbytes(self.w13) + _nbytes(self.w2)


@dataclass(frozen=True)
class HostExpertLayerBuffer:
    layer_id: int
    w13: torch.Tensor
    w2: torch.Tensor
    pinned: bool = False
    _views: list = field(default_factory=list, compare=False, repr=False)

    @property
    def num_experts(self) -> int:
        return int(self.w13.shape[0])

    @property
    def total_bytes(self) -> int:
        return _nbytes(self.w13) + _nbytes(self.w2)

    def bundle(self, expert_id: int) -> ExpertWeightBundle:
        """Row views of one expert (made once, then shared)."""
        if not self._views:
            self._views.extend(
                ExpertWeightBundle(int(self.layer_id), e, self.w13[e], self.w2[e], host_pinned=self.pinned)
                for e in range(self.num_experts)
            )
        return self._views[int(expert_id)]


@dataclass(frozen=True)
class HostStoreCompletenessReport:
    complete: bool
    layers_checked: tuple[int, ...]
    blockers: tuple[str, ...]


@dataclass(frozen=True)
class HostStoreRegisterReport:
    layer_id: int
    num_experts: int
    pin_memory_requested: bool
    pinned_tensors: int
    pin_failures: tuple[str, ...]

    @property
    def pin_memory_enabled(self) -> bool:
        return self.pin_memory_requested and not self.pin_failures

    def to_jsonable(self) -> dict[str, object]:
        return {
            "layer_id": int(self.layer_id),
            "num_experts": int(self.num_experts),
            "pin_memory_requested": bool(self.pin_memory_requested),
            "pin_memory_enabled": bool(self.pin_memory_enabled),
            "pinned_tensors": int(self.pinned_tensors),
            "pin_failures": list(self.pin_failures),
        }


def to_host_block(src: torch.Tensor, *, pin: bool, copy: bool) -> tuple[torch.Tensor, str | None]:
    """A contiguous host tensor holding src: page-locked when pin is asked
    for (a failure is reported and a plain host copy taken instead); a new
    buffer unless copy is False and src already qualifies."""
    src = src.detach()
    on_host_ok = src.device.type == "cpu" and src.is_contiguous() and (src.is_pinned() or not pin)
    if on_host_ok and not copy:
        return src, None
    if pin:
        try:
            out = torch.empty(tuple(src.shape), dtype=src.dtype, pin_memory=True)
            out.copy_(src)
            return out, None if out.is_pinned() else "pin_memory_returned_unpinned"
        except Exception as exc:  # no device runtime, or out of page-locked memory
            note = f"{type(exc).__name__}:{str(exc)[:120]}"
            return src.to("cpu", copy=True).contiguous(), note
    return src.to("cpu", copy=True).contiguous(), None


class HostExpertStore:
    """Routed expert weights of every offloaded layer, on the host."""

    def __init__(self) -> None:
        self._layers: dict[int, HostExpertLayerBuffer] = {}

    def register_layer(
        self,
        layer: torch.nn.Module,
        *,
        pin_memory: bool = False,
        clone_tensors: bool = True,
        routed_expert_count: int | None = None,
    ) -> HostStoreRegisterReport:
        """Take layer.w13_weight / layer.w2_weight rows [0, routed) into the
        layer's host block (replacing an earlier registration)."""
        layer_id = int(getattr(layer, "layer_id", -1))
        w13, w2 = layer.w13_weight, layer.w2_weight
        total = int(w13.shape[0])
        if int(w2.shape[0]) != total:
            raise ValueError("w13_weight and w2_weight must have the same number of experts")
        n = total if routed_expert_count is None else int(routed_expert_count)
        if n <= 0:
            raise ValueError("host expert store requires at least one expert")
        if n > total:
            raise ValueError(f"routed expert count exceeds materialized expert rows: routed={n}, total={total}")
        blocks, notes = [], []
        for name, t in (("w13", w13), ("w2", w2)):
            block, note = to_host_block(t[:n], pin=pin_memory, copy=clone_tensors)
            blocks.append(block)
            if note:
                notes.append(f"{name}_layer:{note}")
        pinned = [bool(b.is_pinned()) for b in blocks]
        self._layers[layer_id] = HostExpertLayerBuffer(layer_id, blocks[0], blocks[1], pinned=all(pinned))
        return HostStoreRegisterReport(layer_id, n, bool(pin_memory), sum(pinned), tuple(notes))

    def get(self, layer_id: int, expert_id: int) -> ExpertWeightBundle:
        buf = self._layers.get(int(layer_id))
        if buf is None:
            raise KeyError(ExpertKey(int(layer_id), int(expert_id)))
        e = int(expert_id)
        if not 0 <= e < buf.num_experts:
            raise KeyError(f"expert {e} is not host-managed for layer {int(layer_id)}")
        return buf.bundle(e)

    def get_layer_buffer(self, layer_id: int) -> HostExpertLayerBuffer:
        buf = self._layers.get(int(layer_id))
        if buf is None:
            raise KeyError(f"layer {int(layer_id)} is not registered in the host expert store")
        return buf

    def validate_complete_layers(self, expected_layer_ids: tuple[int, ...]) -> HostStoreCompletenessReport:
        """Every expected layer registered, its two blocks on the host, dense,
        with matching expert counts and one dtype."""
        ids = tuple(int(i) for i in expected_layer_ids)
        blockers = []
        missing = [i for i in ids if i not in self._layers]
        if missing:
            blockers.append(f"host_store_missing_layers:{missing}")
        for i in ids:
            buf = self._layers.get(i)
            if buf is None:
                continue
            for name, t in (("w13", buf.w13), ("w2", buf.w2)):
                if t.device.type != "cpu":
                    blockers.append(f"host_store_device_mismatch:layer={i},{name}={t.device.type}")
                if not t.is_contiguous():
                    blockers.append(f"host_store_layout_mismatch:layer={i},{name}_stride")
            if buf.w13.dtype != buf.w2.dtype:
                blockers.append(f"host_store_layout_mismatch:layer={i},w2_dtype")
            if int(buf.w2.shape[0]) != buf.num_experts:
                blockers.append(f"host_store_missing_experts:layer={i},experts={buf.num_experts}")
        return HostStoreCompletenessReport(not blockers, ids, tuple(blockers))

    @property
    def total_bytes(self) -> int:
        return sum(b.total_bytes for b in self._layers.values())

    def __len__(self) -> int:
        return sum(b.num_experts for b in self._layers.values())
