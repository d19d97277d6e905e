"""Profile evidence written as JSONL with the reference's event names and
payload keys (moe_offload/profile_io.py:33-106, runtime.py:1856-1901 and
:2900-2926 there), on CPU slot banks.  The last test applies the checks the
reference's evidence verifier makes on these events
(benchmark/scripts/verify_issue7_graph_unit.py:185-251), restated here."""

import json
import threading

import torch

from vllm_moe_offload_amd.moe_offload import profile_io
from vllm_moe_offload_amd.moe_offload import runtime as runtime_mod
from vllm_moe_offload_amd.moe_offload.config import MoeOffloadConfig
from vllm_moe_offload_amd.moe_offload.phase_split import B2WavePlan
from vllm_moe_offload_amd.moe_offload.runtime import MoeOffloadRuntime
from vllm_moe_offload_amd.moe_offload.slot_bank import SlotState

CPU = torch.device("cpu")

DECODE_KEYS = {
    "n_active", "n_hits", "n_misses", "hit_rate", "h2d_bytes", "stage_ms", "load_sync_ms", "load_enqueue_ms",
    "ready_wait_ms", "mapping_ms", "step_id", "num_slots", "mapping_mode", "log2phy_update_count", "stage_mode",
    "consumer_dependency_installed", "mapping_published_after_ready", "profile_sample_rate",
}


class TinyLayer(torch.nn.Module):
    def __init__(self, layer_id=7, experts=6):
        super().__init__()
        self.layer_id = layer_id
        self.w13_weight = torch.nn.Parameter(torch.arange(experts * 2 * 3, dtype=torch.float32).reshape(experts, 2, 3))
        self.w2_weight = torch.nn.Parameter(torch.arange(experts * 3 * 2, dtype=torch.float32).reshape(experts, 3, 2))


class FakeEvent:
    def synchronize(self):
        pass


def _lines(path):
    return [json.loads(line) for line in open(path, encoding="utf-8")]


def test_writer_appends_whole_sorted_lines_from_threads(tmp_path):
    path = tmp_path / "deep" / "dir" / "events.jsonl"

    def work(t):
        for i in range(200):
            profile_io.append_jsonl(path, {"z": i, "a": t, "pad": "x" * 300})

    threads = [threading.Thread(target=work, args=(t,)) for t in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    profile_io.close_profile_writes()
    raw = open(path, encoding="utf-8").read().splitlines()
    assert len(raw) == 800
    assert all(line.startswith('{"a": ') for line in raw)  # keys sorted, no torn lines
    seen = sorted((r["a"], r["z"]) for r in map(json.loads, raw))
    assert seen == sorted((t, i) for t in range(4) for i in range(200))
    profile_io.append_jsonl("", {"ignored": True})  # empty path: nothing written


def test_path_from_config_or_environment(monkeypatch, tmp_path):
    monkeypatch.delenv("VLLM_ASCEND_MOE_GMM_PROFILE_PATH", raising=False)
    monkeypatch.setenv("VLLM_ASCEND_MOE_OFFLOAD_PROFILE_PATH", str(tmp_path / "env.jsonl"))
    assert MoeOffloadRuntime(MoeOffloadConfig()).profile_path == str(tmp_path / "env.jsonl")
    assert MoeOffloadRuntime(MoeOffloadConfig(profile_path="cfg.jsonl")).profile_path == "cfg.jsonl"
    monkeypatch.delenv("VLLM_ASCEND_MOE_OFFLOAD_PROFILE_PATH")
    rt = MoeOffloadRuntime(MoeOffloadConfig(enabled=True, num_slots=2))
    assert rt.profile_path == ""
    rt.register_layer_for_fixed_slots(TinyLayer(), slot_device=CPU)
    assert rt.profiling_summary()["events"][0]["name"] == "register_layer_for_fixed_slots"


def _rt(tmp_path, **kw):
    kw.setdefault("enabled", True)
    kw.setdefault("num_slots", 3)
    kw.setdefault("graph_compatible_offload", True)
    return MoeOffloadRuntime(MoeOffloadConfig(profile_path=str(tmp_path / "ev.jsonl"), **kw))


def test_decode_stage_event_keys_sampling_and_expert_lists(tmp_path, monkeypatch):
    rt = _rt(tmp_path)
    rt.register_layer_for_fixed_slots(TinyLayer(), slot_device=CPU)
    monkeypatch.setenv("VLLM_ASCEND_MOE_DECODE_PROFILE_SAMPLE_RATE", "2")
    for active in ((0, 1), (1, 2), (2, 3), (3, 4)):  # steps 0..3
        rt.stage_fixed_slot_plan(layer_id=7, active_experts=active, num_logical_experts=6)
    monkeypatch.setenv("VLLM_ASCEND_MOE_PROFILE_EXPERT_LISTS", "0")
    for active in ((5,), (4,)):  # steps 4, 5
        rt.stage_fixed_slot_plan(layer_id=7, active_experts=active, num_logical_experts=6)
    profile_io.close_profile_writes()
    stages = [r for r in _lines(tmp_path / "ev.jsonl") if r["name"] == "decode_fixed_slot_stage"]
    assert [r["payload"]["step_id"] for r in stages] == [0, 2, 4]  # every 2nd step
    for r in stages:
        assert DECODE_KEYS <= set(r["payload"]) and r["layer_id"] == 7
        assert set(r) == {"name", "layer_id", "seconds", "memory_ledger", "payload"}
        assert r["memory_ledger"]["registered_layers"] == 1
    first = stages[0]["payload"]
    assert first["n_misses"] == 2 and first["h2d_bytes"] == 2 * (6 + 6) * 4
    assert first["active_experts"] == [0, 1] and first["miss_experts"] == [0, 1] and first["hit_experts"] == []
    assert first["stage_mode"] == "sync_decode_load" and first["profile_sample_rate"] == 2
    third = stages[2]["payload"]
    assert third["expert_lists"] == "omitted" and "active_experts" not in third


def test_wave_plan_evidence_form():
    plan = B2WavePlan(((3, 1), (2,)), {3: 5, 1: 2, 2: 4})
    j = plan.to_jsonable()
    assert j["n_active"] == 3 and j["n_pairs"] == 11 and j["n_waves"] == 2
    assert j["waves"][0] == {"experts": [3, 1], "tokens": 7, "per_expert_tokens": {"3": 5, "1": 2}}


def test_graph_replay_issue_hook_samples_replays_only(monkeypatch, tmp_path):
    from types import SimpleNamespace

    from vllm_moe_offload_amd.patches import patch_fused_moe as pfm

    rt = _rt(tmp_path)
    monkeypatch.setattr(runtime_mod, "get_moe_offload_runtime", lambda: rt)
    ctx = SimpleNamespace(cudagraph_runtime_mode="PIECEWISE", batch_descriptor="b8")

    class CUDAGraphWrapper:
        runtime_mode = "PIECEWISE"

        def __init__(self):
            self.concrete_cudagraph_entries = {"b8": SimpleNamespace(cudagraph=object()),
                                               "b16": SimpleNamespace(cudagraph=None)}

        def __call__(self, x):
            return x + 1

    graph_mod = SimpleNamespace(CUDAGraphWrapper=CUDAGraphWrapper)
    context_mod = SimpleNamespace(get_forward_context=lambda: ctx)
    assert pfm._patch_graph_replay_profile(graph_mod, context_mod)
    assert pfm._patch_graph_replay_profile(graph_mod, context_mod)  # idempotent
    monkeypatch.setenv("VLLM_ASCEND_MOE_GRAPH_REPLAY_PROFILE_SAMPLE_RATE", "3")
    w = CUDAGraphWrapper()
    assert [w(i) for i in range(7)] == list(range(1, 8))
    ctx.batch_descriptor = "b16"  # being captured: not a replay
    w(0)
    ev = [e for e in rt.profiling_summary()["events"] if e["name"] == "graph_replay_issue"]
    assert [e["payload"]["replay_call_index"] for e in ev] == [1, 3, 6]
    assert all(e["payload"]["synchronizes_npu"] is False for e in ev)


def test_evidence_passes_the_reference_verifier_checks(tmp_path, monkeypatch):
    """Graph address lock + replay-time validation, compute-lease protection
    and H2D decode staging, as the verifier reads them from the JSONL."""
    rt = _rt(tmp_path, num_slots=3, graph_compatible_offload=False)
    rt.register_layer_for_fixed_slots(TinyLayer(), slot_device=CPU)
    rt.stage_fixed_slot_plan(layer_id=7, active_experts=(0, 1, 2), num_logical_experts=6)
    monkeypatch.setattr(runtime_mod, "_is_current_graph_capturing", lambda: True)
    rt.capture_safe_slot_weights(layer_id=7)  # capture: lock the addresses
    monkeypatch.setattr(runtime_mod, "_is_current_graph_capturing", lambda: False)
    bank = rt.slot_bank(7)
    active = rt._active_slot_ids_by_layer[7]
    for sid in active:
        bank.slots[sid].state = SlotState.COMPUTING
    rt._note_compute_fence(7, [(sid, bank.slots[sid].version) for sid in active], FakeEvent())
    rt.stage_fixed_slot_plan(layer_id=7, active_experts=(3, 4), num_logical_experts=6)  # drains, validates
    profile_io.close_profile_writes()
    by_name = {}
    for r in _lines(tmp_path / "ev.jsonl"):
        by_name.setdefault(r["name"], []).append(r)
    failures = []
    locks = {int(r["layer_id"]): r for r in by_name.get("graph_slot_address_lock", [])}
    vals = {int(r["layer_id"]): r for r in by_name.get("graph_slot_address_validate", [])}
    if not locks:
        failures.append("missing lock")
    for lid, lock in locks.items():
        v = vals.get(lid)
        if v is None:
            failures.append(f"layer {lid} lacks validation")
            continue
        for key in ("w13_data_ptr", "w2_data_ptr", "log2phy_data_ptr"):
            if lock["payload"].get(key) != v["payload"].get(key):
                failures.append(f"changed {key}")
        if v["payload"].get("matches_capture_fingerprint") is not True:
            failures.append("validation failed")
    gen = by_name.get("slot_generation_protected_until_compute_complete", [])
    if not gen or any(r["payload"].get("leases_still_match") is not True for r in gen):
        failures.append("lease evidence")
    h2d = [r for r in by_name.get("decode_fixed_slot_stage", []) if int(r["payload"].get("h2d_bytes") or 0) > 0]
    if not h2d:
        failures.append("missing H2D staging")
    for r in h2d:
        if r["payload"].get("consumer_dependency_installed") is not True or \
                r["payload"].get("mapping_published_after_ready") is not True:
            failures.append("ordering")
    assert failures == []
