"""CPU-first loading into the host-store layout and release of the original
expert tensors (CPU only).  Expected behaviour follows the reference's own
tests (tests/test_cpu_first_loader.py:46-297) and the release plan of
moe_offload/runtime.py:1366-1454; the checkpoint reader is checked against
safetensors files written here."""

from types import SimpleNamespace

import pytest
import torch

from vllm_moe_offload_amd.moe_offload.config import MoeOffloadConfig
from vllm_moe_offload_amd.moe_offload.cpu_first_loader import (
    CPU_FIRST_MARKER,
    CPU_FIRST_PROCESSED_MARKER,
    _can_process_cpu_first_weight_pair,
    ensure_moe_layer_id,
    layer_index_from_name,
    load_expert_checkpoint,
    maybe_create_unquantized_cpu_first_weights,
    maybe_process_unquantized_cpu_first_weights,
    maybe_register_unquantized_fixed_slot_weights,
)
from vllm_moe_offload_amd.moe_offload.runtime import MoeOffloadRuntime

safetensors_torch = pytest.importorskip("safetensors.torch")
CPU = torch.device("cpu")


class FakeMethod:
    def __init__(self, has_bias=False):
        self.moe = SimpleNamespace(is_act_and_mul=True, has_bias=has_bias)


class FakeRuntime:
    def __init__(self, config):
        self.config = config

    def should_use_fixed_slot_plan_for_layer(self, layer_id):
        return int(layer_id) == 7


class TinyLayer(torch.nn.Module):
    layer_id = 7


def _arange_layer(E=4, I=1, H=3):
    layer = TinyLayer()
    layer.w13_weight = torch.nn.Parameter(torch.arange(E * 2 * I * H, dtype=torch.float32).reshape(E, 2 * I, H),
                                          requires_grad=False)
    layer.w2_weight = torch.nn.Parameter(torch.arange(E * H * I, dtype=torch.float32).reshape(E, H, I),
                                         requires_grad=False)
    return layer


def _cfg(**kw):
    kw.setdefault("enabled", True)
    kw.setdefault("num_slots", 2)
    kw.setdefault("pin_host_memory", False)
    return MoeOffloadConfig(**kw)


def _create(layer, runtime, E=4, H=3, I=2, method=None, attrs=None):
    return maybe_create_unquantized_cpu_first_weights(
        method or FakeMethod(), layer, runtime=runtime, num_experts=E, hidden_size=H,
        intermediate_size_per_partition=I, params_dtype=torch.float32, extra_weight_attrs=attrs or {})


# ------------------------------------------------------------ layer index
def test_layer_id_from_name_and_moe_layer_id():  # reference test :46-61
    a = torch.nn.Module()
    a.layer_name = "model.layers.12.mlp.experts"
    assert ensure_moe_layer_id(a) == 12 and a.layer_id == 12
    b = torch.nn.Module()
    b.moe_layer_id = 7
    assert ensure_moe_layer_id(b) == 7 and b.layer_id == 7
    assert layer_index_from_name("model.layers.mlp") == -1
    assert layer_index_from_name("model.layers.1.mlp.experts.3") == -1  # ambiguous


def test_processing_accepts_host_or_device_pairs_only():  # reference test :62-70
    dev = SimpleNamespace(device=SimpleNamespace(type="cuda"))
    host = SimpleNamespace(device=SimpleNamespace(type="cpu"))
    meta = SimpleNamespace(device=SimpleNamespace(type="meta"))
    assert _can_process_cpu_first_weight_pair(dev, dev)
    assert _can_process_cpu_first_weight_pair(host, host)
    assert not _can_process_cpu_first_weight_pair(dev, host)
    assert not _can_process_cpu_first_weight_pair(meta, meta)


# ------------------------------------------------------------ create hook
def test_create_weights_allocates_offloaded_experts_on_host():  # reference test :73-101
    layer = TinyLayer()
    loader = object()
    assert _create(layer, FakeRuntime(_cfg(cpu_first_load=True)), attrs={"weight_loader": loader}) is True
    assert getattr(layer, CPU_FIRST_MARKER) is True
    assert layer.w13_weight.device.type == "cpu" and layer.w2_weight.device.type == "cpu"
    assert tuple(layer.w13_weight.shape) == (4, 4, 3) and tuple(layer.w2_weight.shape) == (4, 3, 2)
    assert layer.w13_weight.weight_loader is loader and layer.w2_weight.weight_loader is loader
    assert "w13_weight" in dict(layer.named_parameters())


def test_create_weights_skips_disabled_resident_and_biased_layers():  # reference test :104-121
    for rt, layer, method in (
        (FakeRuntime(_cfg(cpu_first_load=False)), TinyLayer(), None),
        (FakeRuntime(_cfg(cpu_first_load=True)), type("L", (torch.nn.Module,), {"layer_id": 3})(), None),
        (FakeRuntime(_cfg(cpu_first_load=True)), TinyLayer(), FakeMethod(has_bias=True)),
    ):
        assert _create(layer, rt, method=method) is False
        assert not hasattr(layer, "w13_weight") and not hasattr(layer, "w2_weight")


# ----------------------------------------------------------- process hook
def test_process_registers_host_blocks_without_a_copy():  # reference test :124-170
    rt = MoeOffloadRuntime(_cfg(cpu_first_load=True))
    layer = TinyLayer()
    assert _create(layer, rt)
    layer.w13_weight.data.copy_(torch.arange(layer.w13_weight.numel(), dtype=torch.float32).reshape(4, 4, 3))
    layer.w2_weight.data.copy_(torch.arange(layer.w2_weight.numel(), dtype=torch.float32).reshape(4, 3, 2))
    assert maybe_process_unquantized_cpu_first_weights(FakeMethod(), layer, runtime=rt) is True
    assert getattr(layer, CPU_FIRST_PROCESSED_MARKER) is True
    # the checkpoint layout is the kernel layout: no transpose on this device
    assert tuple(layer.w13_weight.shape) == (4, 4, 3) and tuple(layer.w2_weight.shape) == (4, 3, 2)
    assert rt.is_layer_registered(7)
    bundle = rt.host_store.get(7, 1)
    assert bundle.w13.data_ptr() == layer.w13_weight[1].data_ptr()
    assert bundle.w2.data_ptr() == layer.w2_weight[1].data_ptr()
    bank = rt.slot_bank(7)
    assert bank is not None and bank.physical_expert_count == 2
    # idempotent
    assert maybe_process_unquantized_cpu_first_weights(FakeMethod(), layer, runtime=rt) is True
    assert rt.slot_bank(7) is bank


def test_normal_loading_copies_and_retains_originals():  # reference test :173-221
    rt = MoeOffloadRuntime(_cfg(cpu_first_load=False, release_original_expert_weights=False))
    layer = _arange_layer(I=1)
    assert maybe_register_unquantized_fixed_slot_weights(layer, runtime=rt, slot_device=CPU)
    bundle = rt.host_store.get(7, 1)
    assert bundle.w13.data_ptr() != layer.w13_weight[1].data_ptr()
    assert torch.equal(bundle.w13, layer.w13_weight[1]) and torch.equal(bundle.w2, layer.w2_weight[1])
    assert tuple(layer.w13_weight.shape) == (4, 2, 3)
    first = rt.slot_bank(7)
    assert maybe_register_unquantized_fixed_slot_weights(layer, runtime=rt, slot_device=CPU)
    assert rt.slot_bank(7) is first
    assert rt.memory_ledger().original_expert_weights_retained


def test_register_skips_layers_not_on_fixed_slots():
    rt = MoeOffloadRuntime(_cfg(resident_layer_ids=frozenset({7})))
    assert maybe_register_unquantized_fixed_slot_weights(_arange_layer(), runtime=rt, slot_device=CPU) is False
    assert not rt.is_layer_registered(7)


# --------------------------------------------------------- checkpoint read
def _expert_tensors(E, I, H, dtype=torch.float32, seed=0):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(I, H, generator=g).to(dtype), torch.randn(I, H, generator=g).to(dtype),
             torch.randn(H, I, generator=g).to(dtype)) for _ in range(E)]


def _write(path, prefix, experts, names=("gate_proj", "up_proj", "down_proj"), skip=()):
    out = {}
    for e, (gate, up, down) in enumerate(experts):
        for part, (name, t) in enumerate(zip(names, (gate, up, down))):
            if (e, part) not in skip:
                out[f"{prefix}.experts.{e}.{name}.weight"] = t.contiguous()
    out[f"{prefix}.gate.weight"] = torch.zeros(len(experts), experts[0][0].shape[1])  # ignored
    safetensors_torch.save_file(out, str(path))


def _host_layer(E, I, H, dtype=torch.float32):
    layer = torch.nn.Module()
    layer.w13_weight = torch.nn.Parameter(torch.full((E, 2 * I, H), float("nan"), dtype=dtype), requires_grad=False)
    layer.w2_weight = torch.nn.Parameter(torch.full((E, H, I), float("nan"), dtype=dtype), requires_grad=False)
    return layer


def test_checkpoint_rows_are_gate_then_up_and_down(tmp_path):
    E, I, H = 5, 3, 4
    experts = _expert_tensors(E, I, H)
    # experts split over two shards, in any order
    _write(tmp_path / "a.safetensors", "model.layers.3.mlp", experts[:2])
    part2 = {f"model.layers.3.mlp.experts.{e}.{n}.weight": t
             for e in range(2, E) for n, t in zip(("gate_proj", "up_proj", "down_proj"), experts[e])}
    safetensors_torch.save_file(part2, str(tmp_path / "b.safetensors"))
    layer = _host_layer(E, I, H)
    n = load_expert_checkpoint(layer, [tmp_path / "b.safetensors", tmp_path / "a.safetensors"],
                               prefix="model.layers.3.mlp")
    assert n == E * 3 * I * H * 4
    for e, (gate, up, down) in enumerate(experts):
        assert torch.equal(layer.w13_weight[e, :I], gate)
        assert torch.equal(layer.w13_weight[e, I:], up)
        assert torch.equal(layer.w2_weight[e], down)


def test_checkpoint_mixtral_names_and_dtype_cast(tmp_path):
    E, I, H = 3, 2, 4
    experts = _expert_tensors(E, I, H, seed=1)
    _write(tmp_path / "m.safetensors", "model.layers.0.block_sparse_moe", experts, names=("w1", "w3", "w2"))
    layer = _host_layer(E, I, H, dtype=torch.bfloat16)
    load_expert_checkpoint(layer, tmp_path / "m.safetensors", prefix="model.layers.0.block_sparse_moe")
    for e, (gate, up, down) in enumerate(experts):
        assert torch.equal(layer.w13_weight[e, :I], gate.to(torch.bfloat16))
        assert torch.equal(layer.w13_weight[e, I:], up.to(torch.bfloat16))
        assert torch.equal(layer.w2_weight[e], down.to(torch.bfloat16))


def test_checkpoint_stacked_blocks(tmp_path):
    E, I, H = 3, 2, 4
    w13 = torch.randn(E, 2 * I, H)
    w2 = torch.randn(E, H, I)
    safetensors_torch.save_file({"L.experts.w13_weight": w13, "L.experts.w2_weight": w2}, str(tmp_path / "s.safetensors"))
    layer = _host_layer(E, I, H)
    load_expert_checkpoint(layer, tmp_path / "s.safetensors", prefix="L")
    assert torch.equal(layer.w13_weight, w13) and torch.equal(layer.w2_weight, w2)


def test_checkpoint_fails_closed(tmp_path):
    E, I, H = 3, 2, 4
    experts = _expert_tensors(E, I, H, seed=2)
    _write(tmp_path / "miss.safetensors", "P", experts, skip={(1, 1)})
    with pytest.raises(ValueError, match="misses 1 expert tensors.*expert 1 up"):
        load_expert_checkpoint(_host_layer(E, I, H), tmp_path / "miss.safetensors", prefix="P")
    _write(tmp_path / "dup.safetensors", "P", experts)
    with pytest.raises(ValueError, match="loaded twice"):
        load_expert_checkpoint(_host_layer(E, I, H), [tmp_path / "dup.safetensors"] * 2, prefix="P")
    with pytest.raises(ValueError, match="outside the layer's 2 experts"):
        load_expert_checkpoint(_host_layer(2, I, H), tmp_path / "dup.safetensors", prefix="P")
    with pytest.raises(ValueError, match="shape"):
        load_expert_checkpoint(_host_layer(E, I + 1, H), tmp_path / "dup.safetensors", prefix="P")


# ---------------------------------------------------------------- release
def test_release_blockers():  # runtime.py:1400-1431
    layer = _arange_layer()
    assert MoeOffloadRuntime(_cfg()).release_original_expert_weights_if_ready(layer).blockers == (
        "release_original_expert_weights_disabled",)
    assert MoeOffloadRuntime(_cfg(num_slots=0, release_original_expert_weights=True)).release_original_expert_weights_if_ready(
        layer).blockers == ("fixed_slots_disabled",)
    bad = torch.nn.Module()
    rt = MoeOffloadRuntime(_cfg(release_original_expert_weights=True, resident_layer_ids=frozenset({7})))
    assert rt.release_original_expert_weights_if_ready(bad).blockers == ("invalid_layer_id",)
    assert rt.release_original_expert_weights_if_ready(layer).blockers == ("resident_layer:7",)
    # not registered: the plan names the layer, the tensors stay
    rt = MoeOffloadRuntime(_cfg(release_original_expert_weights=True))
    plan = rt.release_original_expert_weights_if_ready(layer)
    assert not plan.ready and "layers_not_registered:[7]" in plan.blockers
    assert tuple(layer.w13_weight.shape) == (4, 2, 3)


def test_release_plan_blockers():  # runtime.py:1366-1398
    rt = MoeOffloadRuntime(_cfg())
    assert rt.plan_original_weight_release(expected_layer_ids=(), default_path_preserved=True).blockers == (
        "no_expected_layers",)
    layer = _arange_layer()
    rt.register_layer_for_fixed_slots(layer, slot_device=CPU)
    plan = rt.plan_original_weight_release(expected_layer_ids=(7,), default_path_preserved=True)
    assert plan.blockers == ("original_expert_weights_still_retained",) and plan.layers_ready == ()
    assert rt.plan_original_weight_release(expected_layer_ids=(7,), default_path_preserved=True,
                                           allow_retained_original_weights=True).layers_ready == (7,)
    plan = rt.plan_original_weight_release(expected_layer_ids=(7, 8), default_path_preserved=False,
                                           host_store_is_complete=False, allow_retained_original_weights=True)
    assert plan.blockers[:3] == ("layers_not_registered:[8]", "default_path_not_preserved",
                                 "host_store_not_marked_complete")
    assert "host_store_missing_layers:[8]" in plan.blockers


def test_release_drops_originals_and_keeps_the_slot_path():  # runtime.py:1432-1454
    rt = MoeOffloadRuntime(_cfg(num_slots=2, release_original_expert_weights=True))
    layer = _arange_layer()
    expected13, expected2 = layer.w13_weight.detach().clone(), layer.w2_weight.detach().clone()
    assert maybe_register_unquantized_fixed_slot_weights(layer, runtime=rt, slot_device=CPU)
    assert layer.w13_weight.numel() == 0 and layer.w2_weight.numel() == 0
    assert layer.w13_weight.dtype == torch.float32 and isinstance(layer.w13_weight, torch.nn.Parameter)
    assert not rt.original_expert_weights_available_for_layer(7)
    ledger = rt.memory_ledger()
    assert ledger.original_expert_weight_bytes == 0 and not ledger.original_expert_weights_retained
    ev = [e for e in rt.profiling_summary()["events"] if e["name"] == "release_original_expert_weights"]
    assert len(ev) == 1 and ev[0]["payload"]["released_bytes"] == (4 * 2 * 3 + 4 * 3 * 1) * 4
    again = rt.release_original_expert_weights_if_ready(layer)
    assert again.ready and again.layers_ready == (7,)
    # the host store still serves every expert; staging fills the slots
    prepared = rt.stage_fixed_slot_plan(layer_id=7, active_experts=(3, 1), num_logical_experts=4)
    table = prepared.log2phy.tolist()
    for e in (3, 1):
        s = table[e]
        assert torch.equal(prepared.w1[s], expected13[e]) and torch.equal(prepared.w2[s], expected2[e])


def test_cpu_first_release_keeps_the_adopted_host_blocks():
    rt = MoeOffloadRuntime(_cfg(cpu_first_load=True, release_original_expert_weights=True))
    layer = TinyLayer()
    assert _create(layer, rt)
    layer.w13_weight.data.copy_(torch.arange(48, dtype=torch.float32).reshape(4, 4, 3))
    layer.w2_weight.data.copy_(torch.arange(24, dtype=torch.float32).reshape(4, 3, 2))
    assert maybe_process_unquantized_cpu_first_weights(FakeMethod(), layer, runtime=rt)
    assert layer.w13_weight.numel() == 0
    buf = rt.host_store.get_layer_buffer(7)
    assert torch.equal(buf.w13, torch.arange(48, dtype=torch.float32).reshape(4, 4, 3))


def test_slot_layer_from_checkpoint_adopts_host_blocks(tmp_path):
    from vllm_moe_offload_amd.layer import SlotMoELayer

    E, I, H = 4, 2, 8
    experts = _expert_tensors(E, I, H, dtype=torch.bfloat16, seed=3)
    _write(tmp_path / "l.safetensors", "model.layers.2.mlp", experts)
    rt = MoeOffloadRuntime(_cfg(num_slots=4, graph_compatible_offload=True, release_original_expert_weights=True))
    layer = SlotMoELayer.from_checkpoint(
        tmp_path / "l.safetensors", prefix="model.layers.2.mlp", layer_id=2, runtime=rt, num_experts=E,
        hidden_size=H, intermediate_size=I, gate_weight=torch.zeros(E, H, dtype=torch.bfloat16), top_k=2,
        device="cpu")
    w13_ptr = layer.w13_weight.data_ptr()
    layer.register()
    buf = rt.host_store.get_layer_buffer(2)
    assert buf.w13.data_ptr() == w13_ptr  # adopted, not copied
    assert layer.w13_weight.numel() == 0  # released
    bank = rt.slot_bank(2)
    for e, (gate, up, down) in enumerate(experts):  # full residency staged every expert
        s = bank.lookup_expert_id(e).slot_id
        assert torch.equal(bank.w13_slots[s, :I], gate) and torch.equal(bank.w13_slots[s, I:], up)
        assert torch.equal(bank.w2_slots[s], down)
