"""Pinned host store of routed expert weights.

One contiguous host tensor per layer and weight ([E, 2I, H] w13 and
[E, H, I] w2, checkpoint layout), pinned so hipMemcpyAsync can stream an
expert into a slot without a staging copy; per-expert bundles are views.

Reference: moe_offload/host_store.py:25-253 (ExpertWeightBundle,
HostExpertLayerBuffer, HostExpertStore.register_layer/get/get_layer_buffer,
validate_complete_layers), pinning :260-291.  Pinning allocates new
page-locked memory (torch pin_memory) and copies into it; existing memory is
never registered in place.
"""

from __future__ import annotations

from dataclasses import dataclass

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

    @property
    def num_experts(self) -> int:
        return int(self.w13.shape[0])

    @property
    def total_bytes(self) -> int:
        return _nbytes(self.w13) + _nbytes(self.w2)

    def bundle(self, expert_id: int) -> ExpertWeightBundle:
        e = int(expert_id)
        return ExpertWeightBundle(int(self.layer_id), e, self.w13[e], self.w2[e])


@dataclass(frozen=True)
class HostExpertLayerSignature:
    layer_id: int
    num_experts: int
    w13_shape: tuple[int, ...]
    w13_dtype: torch.dtype
    w13_stride: tuple[int, ...]
    w2_shape: tuple[int, ...]
    w2_dtype: torch.dtype
    w2_stride: tuple[int, ...]


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


def _host_copy(t: torch.Tensor, *, clone: bool, pin: bool) -> tuple[torch.Tensor, bool, str | None]:
    """Contiguous CPU copy of t, page-locked if requested and possible."""
    src = t.detach()
    if pin:
        try:
            if src.device.type == "cpu" and src.is_contiguous() and src.is_pinned() and not clone:
                return src, True, None
            out = torch.empty(tuple(src.shape), dtype=src.dtype, pin_memory=True)
            out.copy_(src)
            return out, bool(out.is_pinned()), None if out.is_pinned() else "pin_memory_returned_unpinned"
        except Exception as exc:  # no GPU runtime or out of pinnable memory
            err = f"{type(exc).__name__}:{str(exc)[:120]}"
            host = src.cpu().contiguous() if src.device.type != "cpu" else src.contiguous()
            return (host.clone() if clone else host), False, err
    host = src.cpu() if src.device.type != "cpu" else src
    if clone or src.device.type != "cpu":
        host = host.clone()
    host = host.contiguous()
    return host, bool(host.is_pinned()) if host.device.type == "cpu" else False, None


class HostExpertStore:
    """Routed expert weights of every offloaded layer, on the host."""

    def __init__(self) -> None:
        self._weights: dict[ExpertKey, ExpertWeightBundle] = {}
        self._by_layer: dict[int, tuple[ExpertWeightBundle, ...]] = {}
        self._layer_buffers: dict[int, HostExpertLayerBuffer] = {}
        self._signatures: dict[int, HostExpertLayerSignature] = {}

    def register_layer(
        self,
        layer: torch.nn.Module,
        *,
        pin_memory: bool = False,
        clone_tensors: bool = True,
        routed_expert_count: int | None = None,
    ) -> HostStoreRegisterReport:
        """Copy layer.w13_weight / layer.w2_weight rows [0, routed) to the host."""
        layer_id = int(getattr(layer, "layer_id", -1))
        w13 = getattr(layer, "w13_weight")
        w2 = getattr(layer, "w2_weight")
        if int(w13.shape[0]) != int(w2.shape[0]):
            raise ValueError("w13_weight and w2_weight must have the same number of experts")
        total = int(w13.shape[0])
        n = total if routed_expert_count is None else int(routed_expert_count)
        if n <= 0:
            raise ValueError("host expert store requires at least one expert")
        if n > total:
            raise ValueError(f"routed expert count exceeds materialized expert rows: routed={n}, total={total}")
        self._drop_layer(layer_id)
        w13_h, w13_pinned, e13 = _host_copy(w13[:n], clone=clone_tensors, pin=pin_memory)
        w2_h, w2_pinned, e2 = _host_copy(w2[:n], clone=clone_tensors, pin=pin_memory)
        buf = HostExpertLayerBuffer(layer_id, w13_h, w2_h)
        self._layer_buffers[layer_id] = buf
        self._signatures[layer_id] = HostExpertLayerSignature(
            layer_id=layer_id,
            num_experts=n,
            w13_shape=tuple(int(d) for d in w13_h.shape[1:]),
            w13_dtype=w13_h.dtype,
            w13_stride=tuple(int(s) for s in w13_h[0].stride()),
            w2_shape=tuple(int(d) for d in w2_h.shape[1:]),
            w2_dtype=w2_h.dtype,
            w2_stride=tuple(int(s) for s in w2_h[0].stride()),
        )
        bundles = tuple(buf.bundle(e) for e in range(n))
        for b in bundles:
            self._weights[b.key] = b
        self._by_layer[layer_id] = bundles
        failures = tuple(f for f in (f"w13_layer:{e13}" if e13 else None, f"w2_layer:{e2}" if e2 else None) if f)
        return HostStoreRegisterReport(
            layer_id=layer_id,
            num_experts=n,
            pin_memory_requested=bool(pin_memory),
            pinned_tensors=int(w13_pinned) + int(w2_pinned),
            pin_failures=failures,
        )

    def _drop_layer(self, layer_id: int) -> None:
        for key in [k for k in self._weights if k.layer_id == layer_id]:
            del self._weights[key]
        self._by_layer.pop(layer_id, None)
        self._layer_buffers.pop(layer_id, None)

    def get(self, layer_id: int, expert_id: int) -> ExpertWeightBundle:
        layer_id, expert_id = int(layer_id), int(expert_id)
        bundles = self._by_layer.get(layer_id)
        if bundles is not None:
            if 0 <= expert_id < len(bundles):
                return bundles[expert_id]
            raise KeyError(f"expert {expert_id} is not host-managed for layer {layer_id}")
        return self._weights[ExpertKey(layer_id, expert_id)]

    def get_layer_buffer(self, layer_id: int) -> HostExpertLayerBuffer:
        try:
            return self._layer_buffers[int(layer_id)]
        except KeyError as exc:
            raise KeyError(f"layer {int(layer_id)} is not registered in the host expert store") from exc

    def validate_complete_layers(self, expected_layer_ids: tuple[int, ...]) -> HostStoreCompletenessReport:
        ids = tuple(int(i) for i in expected_layer_ids)
        blockers: list[str] = []
        missing = [i for i in ids if i not in self._signatures]
        if missing:
            blockers.append(f"host_store_missing_layers:{missing}")
        for layer_id in ids:
            sig = self._signatures.get(layer_id)
            if sig is None:
                continue
            absent = []
            for e in range(sig.num_experts):
                b = self._weights.get(ExpertKey(layer_id, e))
                if b is None:
                    absent.append(e)
                    continue
                for name, shape, dtype, stride in (
                    ("w13", sig.w13_shape, sig.w13_dtype, sig.w13_stride),
                    ("w2", sig.w2_shape, sig.w2_dtype, sig.w2_stride),
                ):
                    t = getattr(b, name)
                    where = f"layer={layer_id},expert={e}"
                    if tuple(t.shape) != shape:
                        blockers.append(f"host_store_layout_mismatch:{where},{name}")
                    if t.dtype != dtype:
                        blockers.append(f"host_store_layout_mismatch:{where},{name}_dtype")
                    if tuple(t.stride()) != stride:
                        blockers.append(f"host_store_layout_mismatch:{where},{name}_stride")
                    if t.device.type != "cpu":
                        blockers.append(f"host_store_device_mismatch:{where},{name}={t.device.type}")
            if absent:
                blockers.append(f"host_store_missing_experts:layer={layer_id},experts={absent}")
        return HostStoreCompletenessReport(not blockers, ids, tuple(blockers))

    @property
    def total_bytes(self) -> int:
        return sum(b.total_bytes for b in self._layer_buffers.values())

    def __len__(self) -> int:
        return len(self._weights)
