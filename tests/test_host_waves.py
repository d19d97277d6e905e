"""Wave planner, async schedule, pair builders and combine helpers (CPU), with
the reference's golden vectors (tests/test_phase_split_b2.py lines cited) and
product-vs-oracle checks of the wave packing and of long LRU trajectories."""

import numpy as np
import pytest
import torch

from oracle import slots as oslots
from oracle import waves as owaves
from vllm_moe_offload_amd.moe_offload.config import MoeOffloadConfig
from vllm_moe_offload_amd.moe_offload.phase_split import (
    B2DirectScatterPayload,
    B2WaveFallback,
    build_b2_device_wave_microbatch_plans,
    build_b2_native_combine_inputs,
    build_b2_pair_microbatch,
    build_b2_pair_microbatch_from_index,
    build_b2_routed_pair_index,
    build_b2_wave_microbatch_plans,
    count_routed_tokens_by_expert,
    count_shared_suffix_pairs,
    direct_scatter_add_b2_permuted_output,
    direct_scatter_add_b2_permuted_outputs,
    materialize_b2_pair_microbatches_from_plans,
    plan_b2_prefill_async_schedule,
    plan_balanced_b2_waves,
    scatter_add_b2_pair_output,
    scatter_add_b2_pair_outputs,
    simulate_b2_prefill_issue_log,
)
from vllm_moe_offload_amd.moe_offload.runtime import MoeOffloadRuntime


def test_count_routed_tokens():  # :25-41
    ids = torch.tensor([[1, 3], [3, 4], [1, 4], [7, 3]], dtype=torch.int32)
    assert count_routed_tokens_by_expert(ids) == {1: 2, 3: 3, 4: 2, 7: 1}


def test_balanced_waves_golden_and_canonical():  # :44-127
    counts = {1: 10, 2: 9, 3: 8, 4: 1, 5: 1}
    plans = [plan_balanced_b2_waves(counts, num_slots=2, slot_readiness=r)
             for r in ({}, {3: True}, {e: True for e in counts})]
    assert plans[0].waves == plans[1].waves == plans[2].waves == ((1,), (2, 5), (3, 4))
    loads = [plans[0].wave_tokens(w) for w in plans[0].waves]
    assert max(loads) - min(loads) <= 8
    assert plan_balanced_b2_waves({1: 10, 2: 9, 3: 8, 4: 7}, num_slots=4, slot_readiness={1: True}).waves == ((1, 2, 3, 4),)
    p = plan_balanced_b2_waves({5: 100, 1: 90, 2: 80, 4: 70}, num_slots=4)
    assert p.waves == ((1, 2, 4, 5),) and p.wave_tokens(p.waves[0]) == 340
    assert plan_balanced_b2_waves({1: 10, 2: 100, 5: 90}, num_slots=3, slot_readiness={1: True}).waves == ((1, 2, 5),)


def test_waves_match_oracle_on_realistic_histograms():
    rng = np.random.default_rng(0)
    for trial in range(200):
        E = int(rng.choice([16, 64, 128, 256]))
        slots = int(rng.integers(1, 65))
        counts = {int(e): int(c) for e, c in enumerate(rng.zipf(1.3, size=E)) if rng.random() < 0.9}
        got = plan_balanced_b2_waves(counts, slots).waves
        assert got == owaves.plan_waves(counts, slots)
        flat = [e for w in got for e in w]
        assert sorted(flat) == sorted(counts) and all(len(w) <= slots for w in got)
        assert len(got) == -(-len(counts) // slots) and all(list(w) == sorted(w) for w in got)


def test_schedule_golden_vectors():  # :197-322
    s = plan_b2_prefill_async_schedule(((1, 2), (3,), (4, 5), (6,)),
                                       slot_readiness={1: True, 2: True, 3: True, 4: False, 5: False, 6: False})
    assert (s.compute_order, s.hit_wave_indices, s.staged_wave_indices, s.staged_issue_order) == ((0, 1, 2, 3), (0, 1), (2, 3), (2, 3))
    assert (s.prefetch_depth, s.buffer_count, s.initial_stage_count) == (1, 2, 1)
    assert s.to_jsonable()["staged_issue_order"] == [2, 3]

    s = plan_b2_prefill_async_schedule(((1,), (2,), (3,), (4,), (5,)), slot_readiness={1: True}, prefetch_depth=2, buffer_count=3)
    assert s.staged_issue_order == (1, 2, 3, 4) and s.initial_stage_count == 2
    log = simulate_b2_prefill_issue_log(s)
    assert log[:2] == (("issue_stage", 1), ("issue_stage", 2))
    assert log.index(("issue_stage", 2)) < log.index(("compute", 1))
    assert log.index(("issue_stage", 3)) < log.index(("compute", 2))

    s = plan_b2_prefill_async_schedule(((1,), (2,), (3,)), slot_readiness={1: True}, prefetch_depth=0, buffer_count=3)
    assert s.initial_stage_count == 0
    assert simulate_b2_prefill_issue_log(s)[:3] == (("issue_hit", 0), ("compute", 0), ("issue_stage", 1))

    s = plan_b2_prefill_async_schedule(((1,), (2,), (3,), (4,)), slot_readiness={1: True, 2: True},
                                       h2d_bytes_by_wave={2: 100, 3: 1000},
                                       compute_cost_by_wave={0: 1.0, 1: 10.0, 2: 5.0, 3: 4.0}, transfer_aware=True)
    assert s.transfer_aware and s.compute_order == (1, 0, 3, 2) and s.staged_issue_order == (3, 2)
    assert s.to_jsonable()["estimated_h2d_bytes_by_wave"] == [0, 0, 100, 1000]
    log = simulate_b2_prefill_issue_log(s, prefetch_depth=1, buffer_count=2)
    assert log[0] == ("issue_stage", 3)
    assert log.index(("issue_stage", 2)) < log.index(("compute", 3))

    s = plan_b2_prefill_async_schedule(((1,), (2,), (3,)), slot_readiness={1: True}, prefetch_depth=0,
                                       h2d_bytes_by_wave={2: 1000, 1: 1}, compute_cost_by_wave={0: 100.0}, transfer_aware=True)
    assert not s.transfer_aware and s.compute_order == (0, 1, 2) and s.staged_issue_order == (1, 2)

    s = plan_b2_prefill_async_schedule(((1,), (2,), (3,), (4,)), slot_readiness={1: True, 2: True})
    log = simulate_b2_prefill_issue_log(s, prefetch_depth=1, buffer_count=2)
    assert log[:5] == (("issue_stage", 2), ("issue_hit", 0), ("compute", 0), ("issue_hit", 1), ("compute", 1))
    assert log.index(("issue_stage", 3)) < log.index(("compute", 2))
    assert log[-2:] == (("compute", 2), ("compute", 3))


def test_pair_microbatch_golden_vector():  # :325-365
    hidden = torch.arange(12, dtype=torch.float32).reshape(4, 3)
    ids = torch.tensor([[1, 3], [3, 4], [1, 4], [7, 3]], dtype=torch.long)
    w = torch.tensor([[0.1, 0.3], [0.4, 0.5], [0.6, 0.7], [0.8, 0.9]])
    l2p = torch.full((8,), -1, dtype=torch.long)
    l2p[3], l2p[4] = 0, 2
    mb = build_b2_pair_microbatch(hidden, ids, w, l2p, wave_experts=(3, 4))
    assert mb.num_pairs == 5
    assert mb.restore_token_indices.tolist() == [0, 1, 1, 2, 3]
    assert mb.logical_expert_ids.tolist() == [3, 3, 4, 4, 3]
    assert mb.topk_ids.squeeze(1).tolist() == [0, 0, 2, 2, 0]
    assert torch.allclose(mb.topk_weights.squeeze(1), torch.tensor([0.3, 0.4, 0.5, 0.7, 0.9]))
    assert torch.equal(mb.hidden_states, hidden[mb.restore_token_indices])
    idx = build_b2_routed_pair_index(ids, w)
    mb2 = build_b2_pair_microbatch_from_index(hidden, idx, l2p, (3, 4))
    for a, b in zip((mb.topk_ids, mb.topk_weights, mb.restore_token_indices), (mb2.topk_ids, mb2.topk_weights, mb2.restore_token_indices)):
        assert torch.equal(a, b)


def test_positional_vs_main_bank_slots():  # :130-194
    idx = build_b2_routed_pair_index(torch.tensor([[1, 2], [2, 3], [3, 4], [4, 1]]), torch.ones(4, 2))
    wave = plan_balanced_b2_waves({1: 10, 2: 9, 3: 8, 4: 7}, num_slots=4).waves[0]
    p = build_b2_wave_microbatch_plans(idx, (wave,), physical_slot_by_expert={4: 0})[0]
    pos = {e: i for i, e in enumerate(wave)}
    assert p.physical_slot_ids.tolist() == [pos[int(e)] for e in p.logical_expert_ids.tolist()]
    idx = build_b2_routed_pair_index(torch.tensor([[1, 2], [2, 1]]), torch.ones(2, 2))
    p = build_b2_wave_microbatch_plans(idx, ((1, 2),), physical_slot_by_expert={1: 5, 2: 7})[0]
    assert dict(zip(p.logical_expert_ids.tolist(), p.physical_slot_ids.tolist())) == {1: 5, 2: 7}


def test_device_wave_planner_golden():  # :1220-1334
    ids = torch.tensor([[3, 1], [2, 3], [0, 2]], dtype=torch.long)
    w = torch.tensor([[0.6, 0.4], [0.7, 0.3], [0.8, 0.2]])
    plans = build_b2_device_wave_microbatch_plans(ids, ((0, 3), (1, 2)), num_logical_experts=4,
                                                  active_experts=(0, 1, 2, 3), wave_pair_counts=(3, 3))
    mbs = materialize_b2_pair_microbatches_from_plans(torch.arange(12.0).reshape(3, 4), w, plans)
    assert torch.cat([p.pair_offsets for p in plans]).sort().values.tolist() == list(range(6))
    assert plans[0].physical_slot_ids.tolist() == [1, 1, 0]
    assert plans[1].physical_slot_ids.tolist() == [0, 1, 1]
    assert sum(m.num_pairs for m in mbs) == 6
    assert torch.cat([m.restore_token_indices for m in mbs]).sort().values.tolist() == [0, 0, 1, 1, 2, 2]
    for active, n in ((tuple(range(128)), 4), (tuple(range(127)), 4), ((0, 127), 1)):
        waves = tuple(tuple(active[s:s + 32]) for s in range(0, len(active), 32))
        plans = build_b2_device_wave_microbatch_plans(torch.tensor(active).reshape(-1, 1), waves, num_logical_experts=128,
                                                      active_experts=active, wave_pair_counts=tuple(len(x) for x in waves))
        assert len(plans) == n
        assert torch.cat([p.pair_offsets for p in plans]).sort().values.tolist() == list(range(len(active)))
    with pytest.raises(ValueError, match="waves do not match"):
        build_b2_device_wave_microbatch_plans(torch.tensor([[0], [127]]), ((0,),), num_logical_experts=128,
                                              active_experts=(0, 127), wave_pair_counts=(2,))
    with pytest.raises(ValueError, match="invalid or uncovered top-k IDs"):
        build_b2_device_wave_microbatch_plans(torch.tensor([[0], [128]]), ((0,),), num_logical_experts=128, active_experts=(0,))
    with pytest.raises(ValueError, match="do not match current top-k contents"):
        build_b2_device_wave_microbatch_plans(torch.tensor([[0], [0], [1]]), ((0,), (1,)), num_logical_experts=2,
                                              active_experts=(0, 1), wave_pair_counts=(1, 2))


def test_scatter_and_native_combine_golden():  # :863-1117
    full = torch.zeros(4, 2)
    out = scatter_add_b2_pair_output(full, torch.tensor([[1.0, 1], [2, 2], [3, 3], [4, 4]]), torch.tensor([0, 1, 1, 3]))
    assert out is full and full.tolist() == [[1, 1], [5, 5], [0, 0], [4, 4]]
    b = scatter_add_b2_pair_outputs(torch.zeros(4, 2), (torch.tensor([[1.0, 1], [2, 2]]), torch.tensor([[3.0, 3], [4, 4], [5, 5]]), torch.empty(0, 2)),
                                    (torch.tensor([0, 1]), torch.tensor([1, 3, 0]), torch.empty(0, dtype=torch.long)))
    assert b.tolist() == [[6, 6], [5, 5], [0, 0], [4, 4]]
    payloads = (
        B2DirectScatterPayload(torch.tensor([[3.0, 30.0], [1.0, 10.0], [5.0, 50.0]]), torch.tensor([2, 0, 1], dtype=torch.int32),
                               torch.tensor([[0.5], [0.7], [0.9]]), torch.tensor([0, 1, 0])),
        B2DirectScatterPayload(torch.tensor([[4.0, 40.0], [2.0, 20.0]]), torch.tensor([1, 0], dtype=torch.int32),
                               torch.tensor([[0.25], [0.75]]), torch.tensor([2, 1])),
    )
    batched = direct_scatter_add_b2_permuted_outputs(torch.zeros(3, 2), payloads)
    assert torch.allclose(batched, torch.tensor([[3.4, 34.0], [5.1, 51.0], [0.5, 5.0]]))
    canon = tuple(B2DirectScatterPayload(torch.tensor([[v]]), torch.tensor([0], dtype=torch.int32), torch.tensor([[1.0]]),
                                         torch.tensor([0]), wave_index=i) for i, v in ((2, 1.0), (1, -1.0e8), (0, 1.0e8)))
    assert direct_scatter_add_b2_permuted_outputs(torch.zeros(1, 1), canon).item() == 1.0
    o = torch.zeros(1, 1)
    direct_scatter_add_b2_permuted_output(o, permuted_tokens=torch.tensor([[2.0]], dtype=torch.bfloat16),
                                          expanded_row_idx=torch.tensor([0], dtype=torch.int32),
                                          topk_weights=torch.tensor([[0.5]], dtype=torch.bfloat16),
                                          restore_token_indices=torch.tensor([0]))
    assert o.dtype == torch.float32 and o.item() == 1.0
    meta = object()
    pl = (
        B2DirectScatterPayload(torch.tensor([[30.0], [10.0]]), torch.tensor([1, 0], dtype=torch.int32), torch.ones(2, 1),
                               torch.tensor([0, 1]), wave_index=0, pair_offsets=torch.tensor([1, 3]), combine_metadata=meta),
        B2DirectScatterPayload(torch.tensor([[20.0], [40.0]]), torch.tensor([0, 1], dtype=torch.int32), torch.ones(2, 1),
                               torch.tensor([0, 1]), wave_index=1, pair_offsets=torch.tensor([0, 2]), combine_metadata=meta),
    )
    perm, expanded, m = build_b2_native_combine_inputs(pl, total_pairs=4)
    assert perm.tolist() == [[30.0], [10.0], [20.0], [40.0]] and expanded.tolist() == [2, 1, 3, 0] and m is meta
    with pytest.raises(B2WaveFallback, match="pair coverage"):
        build_b2_native_combine_inputs(pl[:1], total_pairs=4)


# ---------------------------------------------------------------- LRU trajectories vs oracle
class _Layer(torch.nn.Module):
    def __init__(self, E):
        super().__init__()
        self.layer_id = 3
        self.w13_weight = torch.nn.Parameter(torch.zeros(E, 2, 1))
        self.w2_weight = torch.nn.Parameter(torch.zeros(E, 1, 1))


def test_lru_golden_trajectory_of_reference_matches_oracle():
    t = oslots.LruSlotTable(4, 5)
    t.stage((0, 1))
    assert t.stage((2, 3, 4))[0] == (2, 3, 0)  # test_fixed_slot_lifecycle.py:29-68


def test_long_lru_trajectories_match_oracle():
    """Zipf-skewed decode routing over many steps: slot per expert, loads and
    the persistent log2phy agree with the independent table simulation."""
    rng = np.random.default_rng(1)
    E, slots = 32, 8
    rt = MoeOffloadRuntime(MoeOffloadConfig(enabled=True, num_slots=slots))
    rt.register_layer_for_fixed_slots(_Layer(E), slot_device=torch.device("cpu"))
    table = oslots.LruSlotTable(slots, E)
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    p = p / p.sum()
    order = rng.permutation(E)
    misses = 0
    for step in range(400):
        k = int(rng.integers(1, slots + 1))
        active = tuple(sorted(int(order[i]) for i in rng.choice(E, size=k, replace=False, p=p)))
        prepared = rt.stage_fixed_slot_plan(layer_id=3, active_experts=active, num_logical_experts=E)
        want_slots, loads = table.stage(active)
        misses += len(loads)
        assert prepared.mapping.active_slot_ids == want_slots
        assert rt.log2phy_buffer(3).tolist() == table.log2phy
    assert 0 < misses < 400 * slots


def test_shared_suffix_pair_count_ignores_ids_past_the_layer():
    """Only ids in [routed, total) are shared-suffix pairs: an id at or past
    total is in no wave and no suffix, so the coverage check (waves + shared
    == T * k) fails closed on it (phase_split.py:1808-1812)."""
    ids = torch.tensor([[0, 4], [1, 5], [2, 6], [3, 9], [-1, 4]], dtype=torch.int32)  # routed 4, total 6
    assert count_shared_suffix_pairs(ids, 4, 6) == 3        # the 4, 5, 4 entries
    assert count_shared_suffix_pairs(ids, 4, 4) == 0        # no suffix
    counts = {e: c for e, c in count_routed_tokens_by_expert(ids).items() if e < 4}
    covered = sum(counts.values()) + count_shared_suffix_pairs(ids, 4, 6)
    assert covered == 7 < ids.numel()                                   # 6, 9 and -1 are uncovered
