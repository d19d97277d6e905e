"""Host-side staging controller, slot bank, transfer readiness and placement
plan on CPU slot banks (no GPU).  Expected values are the golden vectors of
the reference's own tests (file:line cited per test)."""

import numpy as np
import pytest
import torch

from vllm_moe_offload_amd.moe_offload import runtime as runtime_mod
from vllm_moe_offload_amd.moe_offload.config import MoeOffloadConfig
from vllm_moe_offload_amd.moe_offload.expert_key import ExpertKey
from vllm_moe_offload_amd.moe_offload.placement_plan import PlacementPlan, PlacementPlanRequest, resolve_placement_plan
from vllm_moe_offload_amd.moe_offload.runtime import MoeOffloadRuntime, _update_log2phy_entries
from vllm_moe_offload_amd.moe_offload.slot_bank import ExpertSlotBank, SlotState
from vllm_moe_offload_amd.moe_offload.slot_mapping import ExpertSlotMapping
from vllm_moe_offload_amd.moe_offload.transfer_engine import TransferEngine, TransferReadyEvent, contiguous_load_runs

CPU = torch.device("cpu")


class TinyLayer(torch.nn.Module):
    def __init__(self, layer_id=7, experts=4):
        super().__init__()
        self.layer_id = layer_id
        self.w13_weight = torch.nn.Parameter(torch.arange(experts * 2 * 3, dtype=torch.float32).reshape(experts, 2, 3))
        self.w2_weight = torch.nn.Parameter(torch.arange(experts * 3 * 2, dtype=torch.float32).reshape(experts, 3, 2))


class TinyFusedSharedLayer(TinyLayer):
    def __init__(self):
        super().__init__(layer_id=9, experts=6)
        self.mix_placement = True
        self.n_shared_experts = 2


class FakeEvent:
    def __init__(self):
        self.synchronize_calls = 0

    def synchronize(self):
        self.synchronize_calls += 1


def _rt(**kw):
    kw.setdefault("enabled", True)
    return MoeOffloadRuntime(MoeOffloadConfig(**kw))


# ---------------------------------------------------------------- slot bank
def test_slot_bank_lookup_tracks_resident_index():  # test_prefill_stage_runtime.py:40-64
    bank = ExpertSlotBank(2, (1, 1), (1, 1), dtype=torch.float32, device=CPU)
    first = bank.allocate_for(ExpertKey(7, 3), step_id=1)
    bank.mark_ready(first.slot_id)
    second = bank.assign_slot(1, ExpertKey(7, 5), step_id=2)
    bank.mark_ready(second.slot_id)
    assert bank.lookup_expert_id(3) is first and bank.lookup_expert_id(5) is second
    bank.clear_slot(first.slot_id)
    assert bank.lookup_expert_id(3) is None and bank.lookup(ExpertKey(7, 3)) is None
    bank.assign_transient_slot(second.slot_id, ExpertKey(7, 9), step_id=3)
    assert bank.lookup_expert_id(5) is None and bank.lookup_expert_id(9) is None


def test_lru_picks_first_empty_then_oldest_ready_then_lowest_id():
    bank = ExpertSlotBank(3, (1,), (1,), dtype=torch.float32, device=CPU)
    slots = [bank.allocate_for(ExpertKey(0, e), step_id=s) for e, s in ((10, 5), (11, 3), (12, 3))]
    assert [s.slot_id for s in slots] == [0, 1, 2]
    for s in slots:
        bank.mark_ready(s.slot_id)
    victim = bank.allocate_for(ExpertKey(0, 13), step_id=6)
    assert victim.slot_id == 1 and victim.version == 2 and victim.state == SlotState.LOADING
    bank.slots[2].state = SlotState.COMPUTING
    assert bank.allocate_for(ExpertKey(0, 14), step_id=7).slot_id == 0
    with pytest.raises(RuntimeError, match="no evictable"):
        bank.allocate_for(ExpertKey(0, 15), step_id=8)


# ---------------------------------------------------------------- transfer readiness
def test_transfer_ready_event_binds_owner_and_generation():  # :85-108
    bank = ExpertSlotBank(1, (1, 1), (1, 1), dtype=torch.float32, device=CPU)
    slot = bank.assign_slot(0, ExpertKey(7, 0), step_id=1)
    ready = TransferReadyEvent(object(), ((slot, slot.lease()),))
    ready.mark_ready()
    ready.mark_ready()
    assert slot.state == SlotState.READY
    slot.state = SlotState.LOADING
    stale = TransferReadyEvent(object(), ((slot, slot.lease()),))
    bank.clear_slot(0)
    repl = bank.assign_slot(0, ExpertKey(7, 1), step_id=2)
    with pytest.raises(RuntimeError, match="stale H2D completion"):
        stale.mark_ready()
    assert repl.state == SlotState.LOADING and repl.expert_key == ExpertKey(7, 1)


def test_transfer_ready_event_publishes_only_after_consumer_wait():  # :111-136
    bank = ExpertSlotBank(1, (1, 1), (1, 1), dtype=torch.float32, device=CPU)
    slot = bank.assign_slot(0, ExpertKey(7, 0), step_id=1)
    event = object()
    ready = TransferReadyEvent(event, ((slot, slot.lease()),))
    calls = []

    class Consumer:
        def wait_event(self, ev):
            assert ev is event and slot.state == SlotState.LOADING and not ready.completed
            calls.append("wait")

    ready.install_consumer_dependency(Consumer())
    assert calls == ["wait"] and ready.consumer_wait_installed and ready.completed
    assert slot.state == SlotState.READY


def test_transfer_ready_event_rejects_stale_lease_before_wait():  # :139-157
    bank = ExpertSlotBank(1, (1, 1), (1, 1), dtype=torch.float32, device=CPU)
    slot = bank.assign_slot(0, ExpertKey(7, 0), step_id=1)
    ready = TransferReadyEvent(object(), ((slot, slot.lease()),))
    bank.clear_slot(0)
    bank.assign_slot(0, ExpertKey(7, 1), step_id=2)

    class Consumer:
        def wait_event(self, _):
            raise AssertionError("must fail before the stream hand-off")

    with pytest.raises(RuntimeError, match="stale H2D completion"):
        ready.install_consumer_dependency(Consumer())


def test_contiguous_runs_batch_consecutive_experts_into_consecutive_slots():
    host = torch.arange(4 * 6, dtype=torch.float32).reshape(4, 6)
    bank = ExpertSlotBank(4, (6,), (6,), dtype=torch.float32, device=CPU)
    from vllm_moe_offload_amd.moe_offload.host_store import ExpertWeightBundle

    b = [ExpertWeightBundle(0, e, host[e], host[e]) for e in range(4)]
    loads = ((b[1], bank.slots[0]), (b[2], bank.slots[1]), (b[0], bank.slots[3]))
    runs = contiguous_load_runs(loads)
    assert [len(r) for r in runs] == [2, 1]
    TransferEngine().load_many_sync(list(loads))
    assert torch.equal(bank.w13_slots[0], host[1]) and torch.equal(bank.w13_slots[3], host[0])


# ---------------------------------------------------------------- decode staging
def test_stage_drains_prior_compute_before_reserving_sync_misses():  # test_fixed_slot_lifecycle.py:29-68
    rt = _rt(num_slots=4, graph_compatible_offload=True)
    rt.register_layer_for_fixed_slots(TinyLayer(experts=5), slot_device=CPU)
    initial = rt.stage_fixed_slot_plan(layer_id=7, active_experts=(0, 1), num_logical_experts=5)
    bank = rt._slot_banks[7]
    done = FakeEvent()
    for sid in initial.mapping.active_slot_ids:
        s = bank.slots[sid]
        s.state = SlotState.COMPUTING
    rt._note_compute_fence(7, [(sid, bank.slots[sid].version) for sid in initial.mapping.active_slot_ids], done)
    prepared = rt.stage_fixed_slot_plan(layer_id=7, active_experts=(2, 3, 4), num_logical_experts=5)
    assert done.synchronize_calls == 1
    assert all(s.state == SlotState.READY for s in bank.slots)
    assert prepared.mapping.active_slot_ids == (2, 3, 0)
    ev = [e for e in rt.profiling_summary()["events"] if e["name"] == "slot_generation_protected_until_compute_complete"]
    assert ev[-1]["payload"]["leases_still_match"] is True
    assert ev[-1]["payload"]["completion_events_synchronized"] == 1


def test_capture_handoff_releases_prior_compute_without_host_sync(monkeypatch):  # test_fixed_slot_lifecycle.py:71-103
    rt = _rt(num_slots=4, graph_compatible_offload=True)
    rt.register_layer_for_fixed_slots(TinyLayer(experts=5), slot_device=CPU)
    prepared = rt.stage_fixed_slot_plan(layer_id=7, active_experts=(0, 1), num_logical_experts=5)
    bank = rt._slot_banks[7]
    done = FakeEvent()
    for sid in prepared.mapping.active_slot_ids:
        s = bank.slots[sid]
        s.state = SlotState.COMPUTING
    rt._note_compute_fence(7, [(sid, bank.slots[sid].version) for sid in prepared.mapping.active_slot_ids], done)
    monkeypatch.setattr(runtime_mod, "_is_current_graph_capturing", lambda: True)
    cap = rt.capture_safe_slot_weights(layer_id=7)
    handle = rt.begin_slot_compute(cap)
    assert handle is not None and done.synchronize_calls == 0
    assert all(bank.slots[s].state == SlotState.COMPUTING for s in handle.slot_ids)
    assert not rt._compute_fences.get(7)


def test_stage_fixed_slot_plan_writes_persistent_log2phy(tmp_path):  # :1388-1419
    rt = _rt(num_slots=2, graph_compatible_offload=True, profile_path=str(tmp_path / "p.jsonl"))
    rt.register_layer_for_fixed_slots(TinyLayer(), slot_device=CPU)
    ptr = rt.log2phy_buffer(7).data_ptr()
    p = rt.stage_fixed_slot_plan(layer_id=7, active_experts=(3, 1), num_logical_experts=4)
    assert p.log2phy.data_ptr() == ptr
    assert rt.log2phy_buffer(7).tolist() == [-1, 1, -1, 0]
    ev = [e for e in rt.profiling_summary()["events"] if e["name"] == "decode_fixed_slot_stage"]
    assert ev[-1]["payload"]["mapping_mode"] == "persistent_log2phy"


def test_capture_locks_fingerprint_and_blocks_reregistration():  # :1422-1467, 1547-1561
    rt = _rt(num_slots=2, graph_compatible_offload=True)
    layer = TinyLayer()
    rt.register_layer_for_fixed_slots(layer, slot_device=CPU)
    p = rt.capture_safe_slot_weights(layer_id=7)
    assert p.w1.data_ptr() == rt._slot_banks[7].w13_slots.data_ptr()
    assert p.log2phy.data_ptr() == rt.log2phy_buffer(7).data_ptr()
    with pytest.raises(RuntimeError, match="addresses are already captured"):
        rt.register_layer_for_fixed_slots(layer, slot_device=CPU)
    rt.stage_fixed_slot_plan(layer_id=7, active_experts=(0, 1), num_logical_experts=4)
    ev = rt.profiling_summary()["events"]
    lock = next(e for e in ev if e["name"] == "graph_slot_address_lock")
    val = next(e for e in ev if e["name"] == "graph_slot_address_validate")
    assert val["payload"]["matches_capture_fingerprint"] is True
    for key in ("w13_data_ptr", "w2_data_ptr", "log2phy_data_ptr"):
        assert lock["payload"][key] == val["payload"][key]
    rt._slot_banks[7].w13_slots = rt._slot_banks[7].w13_slots.clone()
    with pytest.raises(RuntimeError, match="address fingerprint changed"):
        rt.stage_fixed_slot_plan(layer_id=7, active_experts=(0,), num_logical_experts=4)


def test_begin_slot_compute_refuses_loading_slot():  # :1470-1488
    rt = _rt(num_slots=1)
    rt.register_layer_for_fixed_slots(TinyLayer(), slot_device=CPU)
    p = rt.stage_fixed_slot_plan(layer_id=7, active_experts=(0,), num_logical_experts=4)
    slot = rt._slot_banks[7].slots[p.mapping.active_slot_ids[0]]
    slot.state = SlotState.LOADING
    ready = TransferReadyEvent(object(), ((slot, slot.lease()),))
    with pytest.raises(RuntimeError, match="not ready for compute"):
        rt.begin_slot_compute(p)
    ready.mark_ready()
    h = rt.begin_slot_compute(p)
    assert h is not None
    rt.end_slot_compute(h)


def test_decode_waits_before_publishing_async_mapping(monkeypatch):  # :1491-1545
    rt = _rt(num_slots=2, graph_compatible_offload=True, async_load=True)
    rt.register_layer_for_fixed_slots(TinyLayer(), slot_device=CPU)
    pending, observed = [], []

    def fake_async(loads, *, wait_event=None, record_event=True, validate_layout=True):
        assert wait_event is None and record_event and validate_layout is False  # no compute recorded yet
        pending.extend(loads)
        for b, s in loads:
            s.w13.copy_(b.w13)
            s.w2.copy_(b.w2)
            s.state = SlotState.LOADING
        return "decode-ready"

    def wait(ready):
        assert ready == "decode-ready"
        observed.append(rt.log2phy_buffer(7).tolist())
        for _, s in pending:
            s.state = SlotState.READY

    monkeypatch.setattr(rt._transfer_engine, "load_many_async", fake_async)
    monkeypatch.setattr(rt, "_wait_transfer_event", wait)
    p = rt.stage_fixed_slot_plan(layer_id=7, active_experts=(1, 2), num_logical_experts=4)
    assert observed == [[-1, -1, -1, -1]]
    assert p.log2phy.tolist() == [-1, 0, 1, -1]


def test_log2phy_updates_only_changed_and_keeps_inactive_entries():  # :1740-1885
    rt = _rt(num_slots=3)
    rt.register_layer_for_fixed_slots(TinyLayer(), slot_device=CPU)
    calls = []
    orig = runtime_mod._update_log2phy_entries

    def spy(t, *, expert_ids, slot_ids):
        calls.append((tuple(expert_ids), tuple(slot_ids)))
        orig(t, expert_ids=expert_ids, slot_ids=slot_ids)

    runtime_mod._update_log2phy_entries = spy
    try:
        rt.stage_fixed_slot_plan(layer_id=7, active_experts=(0, 1, 2), num_logical_experts=4)
        rt.stage_fixed_slot_plan(layer_id=7, active_experts=(0, 1), num_logical_experts=4)  # hit only: no rewrite
        rt.stage_fixed_slot_plan(layer_id=7, active_experts=(3, 0), num_logical_experts=4)
    finally:
        runtime_mod._update_log2phy_entries = orig
    assert calls == [((0, 1, 2), (0, 1, 2)), ((3,), (2,))]
    # expert 2 was evicted but its stale entry is kept (inactive entries are never cleared)
    assert rt.log2phy_buffer(7).tolist() == [0, 1, 2, 2]


def test_failed_loads_roll_slots_back_to_empty(monkeypatch):  # :1225-1284
    for async_load in (False, True):
        rt = _rt(num_slots=2, async_load=async_load)
        rt.register_layer_for_fixed_slots(TinyLayer(), slot_device=CPU)
        name = "load_many_async" if async_load else "load_many_sync"
        monkeypatch.setattr(rt._transfer_engine, name, lambda *a, **k: (_ for _ in ()).throw(RuntimeError("copy failed")))
        with pytest.raises(RuntimeError, match="copy failed"):
            rt.stage_fixed_slot_plan(layer_id=7, active_experts=(0, 1), num_logical_experts=4)
        bank = rt._slot_banks[7]
        assert all(s.state == SlotState.EMPTY for s in bank.slots)
        assert bank.lookup(ExpertKey(7, 0)) is None


def test_allocation_waits_for_computing_slots_before_eviction(monkeypatch):  # :1149-1200
    rt = _rt(num_slots=2)
    rt.register_layer_for_fixed_slots(TinyLayer(), slot_device=CPU)
    p = rt.prepare_fixed_slot_plan(layer_id=7, active_experts=(0, 1), num_logical_experts=4, device=CPU, step_id=1)
    bank = rt._slot_banks[7]
    ev = FakeEvent()
    monkeypatch.setattr(rt, "_record_current_stream_event_or_none", lambda: ev)
    h = rt.begin_slot_compute(p)
    rt.end_slot_compute(h)
    assert [s.state for s in bank.slots] == [SlotState.COMPUTING, SlotState.COMPUTING]
    a = rt._allocate_slot_with_loading_fallback(bank, ExpertKey(7, 2), step_id=2)
    assert ev.synchronize_calls == 1 and a.slot_id == 0 and a.state == SlotState.LOADING
    assert bank.lookup(ExpertKey(7, 0)) is None and bank.lookup(ExpertKey(7, 1)).state == SlotState.READY


def test_working_set_guard_and_range_checks():
    rt = _rt(num_slots=2)
    rt.register_layer_for_fixed_slots(TinyLayer(), slot_device=CPU)
    with pytest.raises(RuntimeError, match="exceeds num_slots"):
        rt.stage_fixed_slot_plan(layer_id=7, active_experts=(0, 1, 2), num_logical_experts=4)
    with pytest.raises(ValueError, match="out of range"):
        rt.stage_fixed_slot_plan(layer_id=7, active_experts=(4,), num_logical_experts=4)


# ---------------------------------------------------------------- fused shared lane
def test_fused_shared_lane_pins_suffix():  # :227-298
    rt = _rt(num_slots=2)
    layer = TinyFusedSharedLayer()
    w13, w2 = layer.w13_weight.detach().clone(), layer.w2_weight.detach().clone()
    rt.register_layer_for_fixed_slots(layer, slot_device=CPU)
    lay = rt.fused_shared_lane_layout(9)
    assert (lay.routed_expert_count, lay.shared_expert_count, lay.pinned_logical_ids) == (4, 2, (4, 5))
    bank = rt._slot_banks[9]
    assert len(bank.slots) == 2 and bank.physical_expert_count == 4 and bank.pinned_slot_ids == (2, 3)
    assert torch.equal(bank.w13_slots[2:], w13[4:]) and len(rt._host_store) == 4
    p = rt.prepare_fixed_slot_plan(layer_id=9, active_experts=(3, 0), num_logical_experts=4, device=CPU)
    assert p.log2phy.tolist() == [1, -1, -1, 0, 2, 3]
    assert p.mapping.slot_to_expert == (3, 0, 4, 5)
    with pytest.raises(ValueError, match="out of range"):
        rt.prepare_fixed_slot_plan(layer_id=9, active_experts=(4,), num_logical_experts=4, device=CPU)
    assert rt.stage_fixed_slot_plan(layer_id=9, active_experts=(3, 0), num_logical_experts=4).log2phy.tolist() == [1, -1, -1, 0, 2, 3]
    assert rt.capture_safe_slot_weights(layer_id=9).log2phy.tolist() == [1, -1, -1, 0, 2, 3]


def test_fused_shared_lane_prefill_and_full_layer():  # :301-339
    rt = _rt(num_slots=2)
    layer = TinyFusedSharedLayer()
    w13, w2 = layer.w13_weight.detach().clone(), layer.w2_weight.detach().clone()
    rt.register_layer_for_fixed_slots(layer, slot_device=CPU)
    st, _, payload = rt.prepare_prefill_stage_plan(layer_id=9, active_experts=(1, 3), num_logical_experts=4,
                                                   device=CPU, buffer_index=0, async_load=False)
    assert st.log2phy.tolist() == [-1, 0, -1, 1, 2, 3]
    assert st.mapping.slot_to_expert == (1, 3, 4, 5)
    assert torch.equal(st.w1[2:], w13[4:]) and payload["miss_experts"] == [1, 3]
    full, fp = rt.prepare_full_layer_prefill_plan(layer_id=9, num_logical_experts=4, device=CPU)
    assert full.physical_expert_count == 6 and full.log2phy.tolist() == [0, 1, 2, 3, 4, 5]
    assert torch.equal(full.w1, w13) and torch.equal(full.w2, w2)
    assert fp["routed_expert_count"] == 4 and fp["pinned_shared_expert_count"] == 2


# ---------------------------------------------------------------- prefill stage banks
def test_prefill_stage_plan_dedicated_buffer_and_mapping():  # :504-530
    rt = _rt(num_slots=2)
    layer = TinyLayer()
    rt.register_layer_for_fixed_slots(layer, slot_device=CPU)
    p, ready, payload = rt.prepare_prefill_stage_plan(layer_id=7, active_experts=(3, 1), num_logical_experts=4,
                                                      device=CPU, buffer_index=0, async_load=False)
    assert ready is None and payload["miss_experts"] == [3, 1]
    assert p.log2phy.tolist() == [-1, 1, -1, 0]
    assert torch.equal(p.w1[0], layer.w13_weight[3]) and torch.equal(p.w2[1], layer.w2_weight[1])


def test_prefill_stage_pool_shared_and_log2phy_fixed_per_buffer():  # :566-700
    rt = _rt(num_slots=2)
    rt.register_layer_for_fixed_slots(TinyLayer(), slot_device=CPU)
    rt.register_layer_for_fixed_slots(TinyLayer(layer_id=9), slot_device=CPU)
    a, _, _ = rt.prepare_prefill_stage_plan(layer_id=7, active_experts=(0, 1), num_logical_experts=4, device=CPU,
                                            buffer_index=0, async_load=False)
    b, _, _ = rt.prepare_prefill_stage_plan(layer_id=9, active_experts=(2,), num_logical_experts=4, device=CPU,
                                            buffer_index=0, async_load=False)
    c, _, _ = rt.prepare_prefill_stage_plan(layer_id=7, active_experts=(3,), num_logical_experts=4, device=CPU,
                                            buffer_index=1, async_load=False)
    assert a.w1.data_ptr() == b.w1.data_ptr() and a.log2phy.data_ptr() == b.log2phy.data_ptr()
    assert b.log2phy.tolist() == [-1, -1, 0, -1]
    assert c.w1.data_ptr() != a.w1.data_ptr() and c.log2phy.tolist() == [-1, -1, -1, 0]
    assert rt._prefill_stage_banks[7] is rt._prefill_stage_banks[9]
    assert rt.memory_ledger().prefill_stage_bank_count == 2
    ev = object()
    rt.remember_prefill_stage_buffer_release(layer_id=7, buffer_index=1, event=ev)
    assert rt.prefill_stage_buffer_release_event(layer_id=9, buffer_index=1) is ev
    with pytest.raises(RuntimeError, match="prefill_buffer_count=2"):
        rt.prepare_prefill_stage_plan(layer_id=7, active_experts=(0,), num_logical_experts=4, device=CPU,
                                      buffer_index=2, async_load=False)


def test_prefill_stage_plan_can_skip_log2phy():  # :725-761
    rt = _rt(num_slots=2)
    layer = TinyLayer()
    rt.register_layer_for_fixed_slots(layer, slot_device=CPU)
    primed, _, _ = rt.prepare_prefill_stage_plan(layer_id=7, active_experts=(0, 1), num_logical_experts=4, device=CPU,
                                                 buffer_index=0, async_load=False)
    p, _, payload = rt.prepare_prefill_stage_plan(layer_id=7, active_experts=(3, 2), num_logical_experts=4,
                                                  device=CPU, buffer_index=0, async_load=False, build_log2phy=False)
    assert payload["log2phy_built"] is False and p.log2phy.data_ptr() == primed.log2phy.data_ptr()
    assert p.log2phy.tolist() == [0, 1, -1, -1]
    assert torch.equal(p.w1[0], layer.w13_weight[3]) and torch.equal(p.w1[1], layer.w13_weight[2])
    with pytest.raises(RuntimeError, match="log2phy_valid=False"):
        p.mapping.remap_topk_ids(torch.tensor([[2, 3]]))


def test_ready_slot_plan_reuses_main_bank_and_fails_closed_on_miss():  # :812-936
    rt = _rt(num_slots=2)
    rt.register_layer_for_fixed_slots(TinyLayer(), slot_device=CPU)
    main = rt.prepare_fixed_slot_plan(layer_id=7, active_experts=(2, 0), num_logical_experts=4, device=CPU)
    p = rt.prepare_ready_slot_plan(layer_id=7, active_experts=(0, 2), num_logical_experts=4, device=CPU)
    assert p.w1.data_ptr() == main.w1.data_ptr() and p.log2phy.tolist() == [1, -1, 0, -1]
    assert rt.ready_slot_ids_for_experts(layer_id=7, expert_ids=(0, 1, 2)) == {0: 1, 2: 0}
    with pytest.raises(RuntimeError, match="non-ready experts"):
        rt.prepare_ready_slot_plan(layer_id=7, active_experts=(1,), num_logical_experts=4, device=CPU)


def test_full_layer_plan_identity_and_pool_reuse():  # :398-500
    rt = _rt(num_slots=2)
    a, b = TinyLayer(), TinyLayer(layer_id=8)
    with torch.no_grad():
        b.w13_weight.add_(1000)
    rt.register_layer_for_fixed_slots(a, slot_device=CPU)
    rt.register_layer_for_fixed_slots(b, slot_device=CPU)
    p1, pay1 = rt.prepare_full_layer_prefill_plan(layer_id=7, num_logical_experts=4, device=CPU)
    assert p1.log2phy.tolist() == [0, 1, 2, 3] and p1.mapping.slot_to_expert == (0, 1, 2, 3)
    assert torch.equal(p1.w1, a.w13_weight) and pay1["pool_reused"] is False
    ptr = p1.w1.data_ptr()
    p2, pay2 = rt.prepare_full_layer_prefill_plan(layer_id=8, num_logical_experts=4, device=CPU)
    assert pay2["pool_reused"] is True and p2.w1.data_ptr() == ptr and torch.equal(p2.w1, b.w13_weight)
    with pytest.raises(RuntimeError, match="host expert count.*4, expected 5"):
        rt.prepare_full_layer_prefill_plan(layer_id=7, num_logical_experts=5, device=CPU)


def test_route_stats_cache_consumed_once_and_keyed_on_tensor():  # :1934-2028
    rt = _rt(num_slots=2)
    ids = torch.tensor([[0, 1], [1, 2]], dtype=torch.int32)
    rt.cache_prefill_route_stats(layer_id=7, topk_ids=ids, token_counts_by_expert={0: 1, 1: 2, 2: 1, 3: 0})
    assert rt.consume_prefill_route_stats(layer_id=7, topk_ids=ids) == {0: 1, 1: 2, 2: 1}
    assert rt.consume_prefill_route_stats(layer_id=7, topk_ids=ids) is None
    rt.cache_prefill_route_stats(layer_id=7, topk_ids=ids, token_counts_by_expert={0: 1})
    assert rt.consume_prefill_route_stats(layer_id=7, topk_ids=ids.clone()) is None


def test_suspend_fixed_slot_execution_nested_and_exception_safe():  # :67-82
    rt = _rt(num_slots=2)
    assert rt.should_use_fixed_slot_plan_for_layer(7)
    with rt.suspend_fixed_slot_execution():
        with rt.suspend_fixed_slot_execution():
            assert not rt.should_use_fixed_slot_plan_for_layer(7)
        assert not rt.should_use_fixed_slot_plan_for_layer(7)
    assert rt.should_use_fixed_slot_plan_for_layer(7)
    with pytest.raises(RuntimeError, match="boom"):
        with rt.suspend_fixed_slot_execution():
            raise RuntimeError("boom")
    assert rt.should_use_fixed_slot_plan_for_layer(7)


def test_remap_topk_ids_fails_closed_on_host():  # :2030-2112
    bank = ExpertSlotBank(2, (1,), (1,), dtype=torch.float32, device=CPU)
    s = bank.allocate_for(ExpertKey(0, 1), step_id=0)
    bank.mark_ready(s.slot_id)
    m = ExpertSlotMapping.from_slot_bank(layer_id=0, active_experts=(1,), num_logical_experts=3, slot_bank=bank, device=CPU)
    assert m.remap_topk_ids(torch.tensor([[1]])).tolist() == [[0]]
    with pytest.raises(RuntimeError, match="without ready slots"):
        m.remap_topk_ids(torch.tensor([[2]]))


def test_update_log2phy_entries_single_and_batch():
    t = torch.full((5,), -1, dtype=torch.int32)
    _update_log2phy_entries(t, expert_ids=(3,), slot_ids=(1,))
    _update_log2phy_entries(t, expert_ids=(0, 4), slot_ids=(2, 0))
    assert t.tolist() == [2, -1, -1, 1, 0]


# ---------------------------------------------------------------- placement plan
def test_placement_plan_adapter():  # test_placement_plan_adapter.py:21-62
    seen = []

    def provider(req: PlacementPlanRequest):
        seen.append(req)
        return PlacementPlan(layer_id=req.layer_id, ordered_experts=tuple(reversed(req.routed_experts)))

    assert resolve_placement_plan(provider, layer_id=3, routed_experts=(5, 1, 5, 2), num_logical_experts=8) == (2, 1, 5)
    assert seen[0].routed_experts == (5, 1, 2)
    assert resolve_placement_plan(None, layer_id=3, routed_experts=(5, 1, 5), num_logical_experts=8) == (5, 1)
    assert resolve_placement_plan(lambda r: None, layer_id=3, routed_experts=(4,), num_logical_experts=8) == (4,)
    with pytest.raises(RuntimeError, match="must be a permutation"):
        resolve_placement_plan(lambda r: PlacementPlan(3, (1, 9)), layer_id=3, routed_experts=(1, 2), num_logical_experts=8)
    with pytest.raises(RuntimeError, match="targets layer"):
        resolve_placement_plan(lambda r: PlacementPlan(4, (1,)), layer_id=3, routed_experts=(1,), num_logical_experts=8)
    with pytest.raises(TypeError):
        resolve_placement_plan(lambda r: (1,), layer_id=3, routed_experts=(1,), num_logical_experts=8)


def test_runtime_stages_in_placement_plan_order():
    rt = _rt(num_slots=3)
    rt.register_layer_for_fixed_slots(TinyLayer(), slot_device=CPU)
    rt.set_placement_plan_provider(lambda r: PlacementPlan(r.layer_id, (2, 0, 1)))
    p = rt.stage_fixed_slot_plan(layer_id=7, active_experts=(0, 1, 2), num_logical_experts=4)
    assert p.mapping.active_experts == (2, 0, 1) and p.mapping.active_slot_ids == (0, 1, 2)
    assert rt.log2phy_buffer(7).tolist() == [1, 2, 0, -1]


def test_prefetch_then_complete_publishes_after_wait_and_orders_after_layer_compute(monkeypatch):
    """Split decode staging: copies are queued at prefetch (waiting on the
    layer's last recorded compute), the mapping is published only at
    complete, after the consumer wait."""
    rt = _rt(num_slots=2, graph_compatible_offload=True, async_load=True)
    rt.register_layer_for_fixed_slots(TinyLayer(), slot_device=CPU)
    calls, observed = [], []
    release = object()
    rt._layer_release_events[7] = release

    def fake_async(loads, *, wait_event=None, record_event=True, validate_layout=True):
        calls.append(wait_event)
        for b, s in loads:
            s.w13.copy_(b.w13)
            s.w2.copy_(b.w2)
            s.state = SlotState.LOADING
        return ("ready", tuple(s for _, s in loads))

    def wait(ready):
        observed.append(rt.log2phy_buffer(7).tolist())
        for s in ready[1]:
            s.state = SlotState.READY

    monkeypatch.setattr(rt._transfer_engine, "load_many_async", fake_async)
    monkeypatch.setattr(rt, "_wait_transfer_event", wait)
    pending = rt.prefetch_fixed_slot_plan(layer_id=7, active_experts=(2, 0), num_logical_experts=4)
    assert calls == [release]
    assert pending.misses == (2, 0) and rt.log2phy_buffer(7).tolist() == [-1, -1, -1, -1]
    p = rt.complete_fixed_slot_plan(pending)
    assert observed == [[-1, -1, -1, -1]]
    assert p.log2phy.data_ptr() == rt.log2phy_buffer(7).data_ptr()
    assert rt.log2phy_buffer(7).tolist() == [1, -1, 0, -1]
    assert rt.last_stage_stats == (0, 2)
    # all hits: no copy, nothing to wait for
    p = rt.complete_fixed_slot_plan(rt.prefetch_fixed_slot_plan(layer_id=7, active_experts=(0,), num_logical_experts=4))
    assert len(calls) == 1 and rt.last_stage_stats == (1, 0)
    assert torch.equal(p.w1[1], TinyLayer().w13_weight.detach()[0])


def test_register_host_buffers_uses_buffers_in_place():
    """CPU-first registration: the host tensors become the store as they are."""
    rt = _rt(num_slots=2, graph_compatible_offload=True)
    w13 = torch.arange(4 * 2 * 3, dtype=torch.float32).reshape(4, 2, 3)
    w2 = torch.arange(4 * 3 * 2, dtype=torch.float32).reshape(4, 3, 2) + 100
    rt.register_host_buffers(layer_id=5, w13_host=w13, w2_host=w2, slot_device=CPU)
    buf = rt.host_store.get_layer_buffer(5)
    assert buf.w13.data_ptr() == w13.data_ptr() and buf.w2.data_ptr() == w2.data_ptr()
    assert rt.log2phy_buffer(5).tolist() == [-1] * 4
    assert rt.cached_layer_expert_weight_bytes(layer_id=5) == (6 + 6) * 4
    p = rt.stage_fixed_slot_plan(layer_id=5, active_experts=(3, 1), num_logical_experts=4)
    assert rt.log2phy_buffer(5).tolist() == [-1, 1, -1, 0]
    assert torch.equal(p.w1[0], w13[3]) and torch.equal(p.w2[1], w2[1])
    rt.capture_safe_slot_weights(layer_id=5)
    with pytest.raises(RuntimeError, match="already captured"):
        rt.register_host_buffers(layer_id=5, w13_host=w13, w2_host=w2, slot_device=CPU)


# ------------------------------------------------------------ decode overflow
def _expert_rows(layer, e):
    return layer.w13_weight[e].detach(), layer.w2_weight[e].detach()


def test_decode_overflow_keeps_residents_in_the_bank_and_stages_the_rest():
    rt = _rt(num_slots=3, graph_compatible_offload=True, decode_overflow=True)
    layer = TinyLayer(experts=8)
    rt.register_layer_for_fixed_slots(layer, slot_device=CPU)
    first = rt.stage_fixed_slot_plan(layer_id=7, active_experts=(0, 1, 2), num_logical_experts=8)
    assert first.overflow is None
    p = rt.stage_fixed_slot_plan(layer_id=7, active_experts=(4, 0, 3, 1, 2), num_logical_experts=8,
                                 token_counts={3: 5, 4: 1, 0: 1, 1: 1, 2: 1})
    main = rt.log2phy_buffer(7).tolist()
    assert sorted(p.mapping.active_experts) == [0, 1, 2]  # the residents stay: three hits
    assert main[3] == -1 and main[4] == -1
    ovf = p.overflow
    assert ovf is not None and ovf.mapping.active_experts == (3, 4)  # more tokens first
    assert ovf.log2phy.tolist() == [-1, -1, -1, 0, 1, -1, -1, -1]
    for e, s in ((3, 0), (4, 1)):
        w13, w2 = _expert_rows(layer, e)
        assert torch.equal(ovf.w1[s], w13) and torch.equal(ovf.w2[s], w2)
    assert rt.decode_overflow_slot_weights(layer_id=7).log2phy.data_ptr() == ovf.log2phy.data_ptr()
    # a hot miss takes the least recently used non-active slot, a cold one overflows
    p = rt.stage_fixed_slot_plan(layer_id=7, active_experts=(6, 5, 0, 1), num_logical_experts=8,
                                 token_counts={5: 9, 6: 2, 0: 1, 1: 1})
    main = rt.log2phy_buffer(7).tolist()
    assert sorted(p.mapping.active_experts) == [0, 1, 5] and main[6] == -1
    w13, _ = _expert_rows(layer, 5)
    assert torch.equal(p.w1[main[5]], w13)
    assert p.overflow.log2phy.tolist() == [-1] * 6 + [0, -1]
    # a step without overflow clears the table the last one left
    p = rt.stage_fixed_slot_plan(layer_id=7, active_experts=(0,), num_logical_experts=8)
    assert p.overflow is None and rt.decode_overflow_slot_weights(layer_id=7).log2phy.tolist() == [-1] * 8


def test_decode_overflow_bounds_and_switch():
    rt = _rt(num_slots=2, decode_overflow=True)
    rt.register_layer_for_fixed_slots(TinyLayer(experts=8), slot_device=CPU)
    assert rt.can_stage_decode_overflow(layer_id=7, active_expert_count=4)
    assert not rt.can_stage_decode_overflow(layer_id=7, active_expert_count=5)  # past one extra pass
    assert not rt.can_stage_decode_overflow(layer_id=7, active_expert_count=2)  # fits the bank
    with pytest.raises(RuntimeError, match="exceeds num_slots=2"):
        rt.stage_fixed_slot_plan(layer_id=7, active_experts=(0, 1, 2, 3, 4), num_logical_experts=8)
    assert rt.decode_overflow_slot_weights(layer_id=7, n_pairs=2) is None  # cannot overflow
    off = _rt(num_slots=2)
    off.register_layer_for_fixed_slots(TinyLayer(experts=8), slot_device=CPU)
    with pytest.raises(RuntimeError, match="exceeds num_slots=2"):
        off.stage_fixed_slot_plan(layer_id=7, active_experts=(0, 1, 2), num_logical_experts=8)
    assert off.decode_overflow_slot_weights(layer_id=7) is None


def test_decode_overflow_split_covers_every_expert_once():
    from vllm_moe_offload_amd.moe_offload.runtime import _split_decode_overflow

    rng = np.random.default_rng(5)
    for trial in range(50):
        P = int(rng.integers(1, 9))
        rt = _rt(num_slots=P, decode_overflow=True)
        rt.register_layer_for_fixed_slots(TinyLayer(experts=24), slot_device=CPU)
        bank = rt.slot_bank(7)
        warm = tuple(int(e) for e in rng.choice(24, size=P, replace=False))
        rt.stage_fixed_slot_plan(layer_id=7, active_experts=warm, num_logical_experts=24)
        n = int(rng.integers(P + 1, 2 * P + 1))
        active = tuple(int(e) for e in rng.choice(24, size=n, replace=False))
        counts = {e: int(rng.integers(1, 9)) for e in active}
        main, over = _split_decode_overflow(bank, active, P, counts)
        assert len(main) == P and sorted(main + over) == sorted(active)
        assert set(warm) & set(active) <= set(main)  # residents are never pushed out
        prepared = rt.stage_fixed_slot_plan(layer_id=7, active_experts=active, num_logical_experts=24,
                                            token_counts=counts)
        table, otab = rt.log2phy_buffer(7).tolist(), prepared.overflow.log2phy.tolist()
        for e in active:  # every routed expert maps in exactly one of the two tables
            assert (table[e] >= 0) != (otab[e] >= 0), (trial, e)


def test_prefetch_then_complete_hands_out_the_overflow_pass():
    rt = _rt(num_slots=2, decode_overflow=True)
    rt.register_layer_for_fixed_slots(TinyLayer(experts=6), slot_device=CPU)
    pend = rt.prefetch_fixed_slot_plan(layer_id=7, active_experts=(0, 1, 2), num_logical_experts=6,
                                       token_counts={0: 1, 1: 3, 2: 2})
    assert pend.overflow is not None and pend.overflow.experts == (0,)
    prepared = rt.complete_fixed_slot_plan(pend)
    assert prepared.overflow is not None and prepared.overflow.mapping.active_experts == (0,)
    assert prepared.log2phy.data_ptr() == rt.log2phy_buffer(7).data_ptr()
    table = rt.log2phy_buffer(7).tolist()
    assert table[0] == -1 and table[1] >= 0 and table[2] >= 0


def test_slot_owner_tail_follows_every_reassignment():
    """Behind the persistent table: the owner of each dynamic slot, written
    with the same update that changes it (the device-side residency check of
    the device wave planner), while the table keeps the reference's stale
    entries for evicted experts."""
    rt = _rt(num_slots=3)
    rt.register_layer_for_fixed_slots(TinyLayer(experts=6), slot_device=CPU)
    assert rt.slot_owner_buffer(7).tolist() == [-1, -1, -1]
    rt.stage_fixed_slot_plan(layer_id=7, active_experts=(0, 1, 2), num_logical_experts=6)
    assert rt.slot_owner_buffer(7).tolist() == [0, 1, 2]
    rt.stage_fixed_slot_plan(layer_id=7, active_experts=(1, 3), num_logical_experts=6)  # 3 evicts 0
    table, owner = rt.log2phy_buffer(7).tolist(), rt.slot_owner_buffer(7).tolist()
    assert table[:4] == [0, 1, 2, 0] and owner == [3, 1, 2]  # stale table[0], exact owners
    bank = rt.slot_bank(7)
    assert owner == [int(o) for o in bank._owner[:3]]
    resident = [e for e in range(6) if 0 <= table[e] < 3 and owner[table[e]] == e]
    assert resident == [1, 2, 3]
    assert rt.log2phy_buffer(7).numel() == 6  # the table keeps its size
