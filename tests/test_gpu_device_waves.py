"""Device-planned capacity waves (lmoe_wave_plan / lmoe_wave_stage): the plan
equals the wave-packing oracle (oracle/waves.py, pinned by the reference's
golden vectors) on the same routed ids, and a layer run by device-planned,
device-staged waves equals the full layer bit for bit, eager and replayed
from a captured graph."""

import numpy as np
import pytest
import torch

from oracle import waves as owaves
from oracle.bf16 import normal_bf16
from tests._util import to_dev_bf16

pytestmark = pytest.mark.gpu


def _plan(ids_np, n_routed, P, max_waves, n_total=None):
    from vllm_moe_offload_amd import native

    plan = native.WavePlan(n_routed, P, max_waves, torch.device("cuda"))
    ids = torch.from_numpy(np.ascontiguousarray(ids_np, dtype=np.int32)).cuda()
    native.wave_plan(ids, plan, n_total=n_total)
    torch.cuda.synchronize()
    return plan.to_host()


def _counts(ids_np, n_routed):
    u, c = np.unique(ids_np[(ids_np >= 0) & (ids_np < n_routed)], return_counts=True)
    return {int(e): int(n) for e, n in zip(u, c)}


def test_device_plan_golden_vectors():
    # reference tests/test_phase_split_b2.py:44-117 (counts as routed pairs)
    ids = np.array([1] * 10 + [2] * 9 + [3] * 8 + [4, 5], dtype=np.int32)
    p = _plan(ids, 8, 2, 4)
    assert p["waves"] == ((1,), (2, 5), (3, 4)) and p["n_active"] == 5 and p["invalid"] == 0
    ids = np.array([5] * 100 + [1] * 90 + [2] * 80 + [4] * 70, dtype=np.int32)
    p = _plan(ids, 8, 4, 2)
    assert p["waves"] == ((1, 2, 4, 5),)


@pytest.mark.parametrize("seed", range(6))
def test_device_plan_equals_oracle(seed):
    rng = np.random.default_rng(100 + seed)
    for trial in range(12):
        E = int(rng.choice([8, 64, 128, 256, 1024]))
        P = int(rng.integers(1, 65))
        T, k = int(rng.integers(1, 2049)), int(rng.choice([1, 2, 6, 8]))
        k = min(k, E)
        skew = rng.zipf(1.3, size=E).astype(np.float64)
        prob = skew / skew.sum()
        ids = np.stack([rng.choice(E, size=k, replace=False, p=prob) for _ in range(T)]).astype(np.int32)
        counts = _counts(ids, E)
        P = max(P, -(-min(E, T * k) // 256))  # the planner holds at most 256 waves
        W = max(1, -(-min(E, T * k) // P))
        print(f"case plan seed={seed} trial={trial} E={E} P={P} T={T} k={k}", flush=True)
        p = _plan(ids, E, P, W)
        want = owaves.plan_waves(counts, P)
        assert p["waves"] == want, (E, P, T, k)
        assert p["n_waves"] == len(want) and p["n_active"] == len(counts)
        assert [p["counts"][e] for e in range(E)] == [counts.get(e, 0) for e in range(E)]
        for w, members in enumerate(want):
            for i, e in enumerate(members):
                assert p["wave_of"][e] == w and p["slot_of"][e] == i


def test_device_plan_shared_suffix_invalid_ids_and_capacity():
    ids = np.array([[0, 4], [1, 5], [2, 9], [-1, 3]], dtype=np.int32)  # 4,5: pinned suffix; 9, -1: invalid
    p = _plan(ids, 4, 2, 2, n_total=6)
    assert p["invalid"] == 2 and p["waves"] == owaves.plan_waves(_counts(ids, 4), 2)
    p = _plan(np.arange(8, dtype=np.int32), 8, 2, 3)  # needs 4 waves, 3 provisioned
    assert p["n_waves"] == -1


def _layer(rt_kw, E=64, H=1024, I=256, slots=16, seed=0, shared=False, layer_id=80):
    from vllm_moe_offload_amd.layer import SlotMoELayer
    from vllm_moe_offload_amd.moe_offload.config import MoeOffloadConfig
    from vllm_moe_offload_amd.moe_offload.runtime import MoeOffloadRuntime

    rng = np.random.default_rng(seed)
    w13 = normal_bf16(rng, (E, 2 * I, H), 0.02)
    w2 = normal_bf16(rng, (E, H, I), 0.02)
    wg = normal_bf16(rng, (E, H), 0.02)
    tb = lambda a: torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)  # noqa: E731
    rt = MoeOffloadRuntime(MoeOffloadConfig(enabled=True, num_slots=slots, async_load=True, pin_host_memory=True,
                                            b2_wave_prefill=True, device_wave_prefill=True, **rt_kw))
    kw = {}
    if shared:
        kw = dict(shared_w13=tb(normal_bf16(rng, (2 * I, H), 0.02)), shared_w2=tb(normal_bf16(rng, (H, I), 0.02)))
    layer = SlotMoELayer(layer_id=layer_id, runtime=rt, gate_weight=to_dev_bf16(wg), w13_weight=tb(w13),
                         w2_weight=tb(w2), top_k=8, **kw)
    layer.register()
    return layer, rt, rng


def test_device_waves_equal_full_layer_bitwise_with_main_bank_residents():
    from vllm_moe_offload_amd import fused_moe

    layer, rt, rng = _layer({})
    E, H = 64, 1024
    # a decode step first: some experts become main-bank residents (D2D sources)
    dx1 = to_dev_bf16(normal_bf16(rng, (1, H), 1.0))
    layer.forward(dx1)
    torch.cuda.synchronize()
    owner = rt.slot_owner_buffer(layer.layer_id).tolist()
    assert sum(o >= 0 for o in owner) == 8
    T = 384
    dx = to_dev_bf16(normal_bf16(rng, (T, H), 1.0))
    w, ids, _ = fused_moe.route(dx, layer.gate_weight, layer.router_spec)
    print("case device waves eager", flush=True)
    out_d = fused_moe.run_device_waves(rt, layer_id=layer.layer_id, hidden=dx, topk_weights=w, topk_ids=ids,
                                       num_logical_experts=E).clone()
    out_f = fused_moe.run_full_layer(rt, layer_id=layer.layer_id, hidden=dx, topk_weights=w, topk_ids=ids,
                                     num_logical_experts=E).clone()
    out_h, report = fused_moe.run_wave_prefill(rt, layer_id=layer.layer_id, hidden=dx, topk_weights=w,
                                               topk_ids=ids, num_logical_experts=E)
    out_h = out_h.clone()
    torch.cuda.synchronize()
    assert len(report.waves) >= 3
    assert torch.equal(out_d.view(torch.int16), out_f.view(torch.int16))
    assert torch.equal(out_d.view(torch.int16), out_h.view(torch.int16))


def test_device_waves_captured_graph_replays_new_routes_and_the_seam_takes_no_d2h():
    from vllm_moe_offload_amd import fused_moe
    from vllm_moe_offload_amd.ops.fused_moe.moe_offload_stage_op import PHASE_PREFILL

    layer, rt, rng = _layer({}, seed=3, layer_id=81)
    E, H, T, k = 64, 1024, 256, 8
    static_x = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    static_w = torch.empty((T, k), dtype=torch.bfloat16, device="cuda")
    static_ids = torch.empty((T, k), dtype=torch.int32, device="cuda")
    out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")

    def run():
        fused_moe.run_device_waves(rt, layer_id=81, hidden=static_x, topk_weights=static_w, topk_ids=static_ids,
                                   num_logical_experts=E, out=out)

    def load(x):
        w, ids, _ = fused_moe.route(x, layer.gate_weight, layer.router_spec)
        static_x.copy_(x)
        static_w.copy_(w)
        static_ids.copy_(ids)

    load(to_dev_bf16(normal_bf16(rng, (T, H), 1.0)))
    run()  # eager warm-up allocates the plan and the stage buffers
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    for step in range(3):
        print(f"case device waves replay {step}", flush=True)
        x = to_dev_bf16(normal_bf16(rng, (T, H), 1.0))
        load(x)
        g.replay()
        got = out.clone()
        ref = fused_moe.run_full_layer(rt, layer_id=81, hidden=static_x, topk_weights=static_w, topk_ids=static_ids,
                                       num_logical_experts=E).clone()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), step
    # the seam: a prefill-phase call hands the ids to the device planner
    x = to_dev_bf16(normal_bf16(rng, (T, H), 1.0))
    w, ids, _ = fused_moe.route(x, layer.gate_weight, layer.router_spec)
    ref = fused_moe.run_full_layer(rt, layer_id=81, hidden=x, topk_weights=w, topk_ids=ids,
                                   num_logical_experts=E).clone()
    got = layer.forward(x, phase=PHASE_PREFILL).clone()
    torch.cuda.synchronize()
    assert not rt._prefill_route_stats_by_layer and not rt._device_wave_marks
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_device_waves_with_a_pinned_shared_expert():
    from vllm_moe_offload_amd import fused_moe

    layer, rt, rng = _layer({}, seed=5, shared=True, layer_id=82)
    E, H, T = 64, 1024, 128
    dx = to_dev_bf16(normal_bf16(rng, (T, H), 1.0))
    w, ids, _ = fused_moe.route(dx, layer.gate_weight, layer.router_spec)
    assert int((ids == E).sum().item()) == T  # the shared suffix rides in every token's top-k
    print("case device waves shared", flush=True)
    out_d = fused_moe.run_device_waves(rt, layer_id=82, hidden=dx, topk_weights=w, topk_ids=ids,
                                       num_logical_experts=E + 1).clone()
    out_f = fused_moe.run_full_layer(rt, layer_id=82, hidden=dx, topk_weights=w, topk_ids=ids,
                                     num_logical_experts=E + 1).clone()
    torch.cuda.synchronize()
    assert torch.equal(out_d.view(torch.int16), out_f.view(torch.int16))
