"""Fail-closed coverage on every multi-pass path (waves, device waves, the
decode overflow pass) and the reference's one recoverable error.

The reference refuses a wave split that does not cover every routed pair
exactly once (moe_offload/phase_split.py:1808-1812) and recovers from that
B2WaveFallback by running the blocking full layer
(patches/patch_fused_moe.py:2281-2298).  Here: eager paths raise before any
wave runs and fall back; captured paths cannot raise, so the single combine
masks every pair no pass placed (never a stale y row) and counts it in the
device status words (lmoe_device_flags), which the runtime checks at its host
sync points."""

import numpy as np
import pytest
import torch

from oracle import mlp as omlp
from oracle.bf16 import bf16_to_f32, normal_bf16
from tests._util import OUT_TOL, from_dev_bf16, rel_max_err, to_dev_bf16

pytestmark = pytest.mark.gpu


def _mods():
    from vllm_moe_offload_amd import fused_moe, native
    from vllm_moe_offload_amd.layer import SlotMoELayer
    from vllm_moe_offload_amd.moe_offload import phase_split
    from vllm_moe_offload_amd.moe_offload.config import MoeOffloadConfig
    from vllm_moe_offload_amd.moe_offload.runtime import MoeOffloadRuntime

    return fused_moe, native, phase_split, SlotMoELayer, MoeOffloadConfig, MoeOffloadRuntime


def _tb(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def _layer(layer_id, *, E=64, H=1024, I=256, slots=16, seed=0, shared=False, **cfg):
    fused_moe, native, phase_split, SlotMoELayer, Cfg, Runtime = _mods()
    rng = np.random.default_rng(seed)
    w13 = normal_bf16(rng, (E, 2 * I, H), 0.02)
    w2 = normal_bf16(rng, (E, H, I), 0.02)
    wg = normal_bf16(rng, (E, H), 0.02)
    rt = Runtime(Cfg(enabled=True, num_slots=slots, async_load=True, pin_host_memory=True, b2_wave_prefill=True,
                     **cfg))
    kw = {}
    sh = None
    if shared:
        sh = (normal_bf16(rng, (2 * I, H), 0.02), normal_bf16(rng, (H, I), 0.02))
        kw = dict(shared_w13=_tb(sh[0]), shared_w2=_tb(sh[1]), scoring_func="sigmoid", use_grouped_topk=True,
                  num_expert_group=8, topk_group=4, routed_scaling_factor=2.5)
    layer = SlotMoELayer(layer_id=layer_id, runtime=rt, gate_weight=to_dev_bf16(wg), w13_weight=_tb(w13),
                         w2_weight=_tb(w2), top_k=8, **kw)
    layer.register()
    return layer, rt, rng, (w13, w2, sh)


def _zero_weight_twin(w, ids, t, j, valid_id=0):
    """(w, ids) with pair (t, j) moved to a valid expert at weight 0: the
    combine then adds exactly +0 for it, the bits of dropping the pair."""
    w2, i2 = w.clone(), ids.clone()
    w2[t, j] = 0
    i2[t, j] = valid_id
    return w2, i2


def test_masked_combine_drops_unplaced_pairs_and_counts_them():
    _, native, *_ = _mods()
    native.device_flags(clear=True)
    rng = np.random.default_rng(5)
    T, k, H = 5, 4, 256
    y = to_dev_bf16(normal_bf16(rng, (T * k, H), 1.0))
    w = to_dev_bf16(normal_bf16(rng, (T, k), 0.5))
    mask = torch.arange(T * k, dtype=torch.int32, device="cuda")
    dropped = [3, 9, 17]
    mask[dropped] = -1
    out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    native.combine(y, w, out, row_mask=mask)
    wz = w.clone().view(-1)
    wz[dropped] = 0
    ref = torch.empty_like(out)
    native.combine(y, wz.view(T, k), ref)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert native.device_flags(clear=True)[native.FLAG_UNPLACED] == len(dropped)
    assert native.device_flags(clear=True) == [0] * native.FLAG_COUNT


def test_host_waves_with_a_shared_suffix_refuse_an_id_past_the_layer():
    fused_moe, native, phase_split, *_ = _mods()
    layer, rt, rng, _ = _layer(90, shared=True, seed=1)
    E, T = 64, 96
    dx = to_dev_bf16(normal_bf16(rng, (T, 1024), 1.0))
    w, ids, _ = fused_moe.route(dx, layer.gate_weight, layer.router_spec)
    assert int(ids.shape[1]) == 9 and int(ids[0, 8]) == E  # the pinned suffix column
    bad = ids.clone()
    bad[5, 2] = E + 1  # past the routed experts and the suffix
    print("case host waves, shared suffix, id past the layer", flush=True)
    with pytest.raises(phase_split.B2WaveFallback, match="coverage"):
        fused_moe.run_wave_prefill(rt, layer_id=90, hidden=dx, topk_weights=w, topk_ids=bad, num_logical_experts=E)
    # the recovery runs the full layer, whose remap fails closed on the id
    with pytest.raises(RuntimeError, match="without ready slots"):
        fused_moe.run_overflow_prefill(rt, layer_id=90, hidden=dx, topk_weights=w, topk_ids=bad,
                                       num_logical_experts=E, device_planned=False)
    native.device_flags(clear=True)


def test_forced_wave_fallback_runs_the_full_layer_and_matches_the_oracle(tmp_path):
    fused_moe, native, phase_split, *_ = _mods()
    layer, rt, rng, (w13, w2, _) = _layer(91, seed=2)
    rt.profile_path = str(tmp_path / "ev.jsonl")
    E, T, k = 64, 384, 8
    x = normal_bf16(rng, (T, 1024), 1.0)
    dx = to_dev_bf16(x)
    w, ids, _ = fused_moe.route(dx, layer.gate_weight, layer.router_spec)
    counts = phase_split.count_routed_tokens_by_expert(ids)
    stale = dict(counts)
    stale.pop(max(stale))  # a stale histogram: one expert missing from the plan
    print("case forced fallback", flush=True)
    out = fused_moe.run_overflow_prefill(rt, layer_id=91, hidden=dx, topk_weights=w, topk_ids=ids,
                                         num_logical_experts=E, device_planned=False,
                                         token_counts_by_expert=stale).clone()
    full = fused_moe.run_full_layer(rt, layer_id=91, hidden=dx, topk_weights=w, topk_ids=ids,
                                    num_logical_experts=E).clone()
    waves, _ = fused_moe.run_wave_prefill(rt, layer_id=91, hidden=dx, topk_weights=w, topk_ids=ids,
                                          num_logical_experts=E, token_counts_by_expert=counts)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), full.view(torch.int16))
    assert torch.equal(out.view(torch.int16), waves.view(torch.int16))
    ref = omlp.moe_layer(x, ids.cpu().numpy(), from_dev_bf16(w), None, w13, w2)
    assert rel_max_err(bf16_to_f32(from_dev_bf16(out)), ref) <= OUT_TOL
    names = [e.name for e in rt._profile_events]
    assert "b2_full_layer_fallback" in names
    ev = rt._profile_events[names.index("b2_full_layer_fallback")]
    assert "coverage" in ev.payload["fallback_reason"]
    assert native.device_flags(clear=True) == [0] * native.FLAG_COUNT


def test_device_waves_fail_closed_eager_and_mask_and_flag_under_capture():
    fused_moe, native, phase_split, *_ = _mods()
    layer, rt, rng, _ = _layer(92, seed=3, device_wave_prefill=True)
    E, T, k = 64, 384, 8
    dx = to_dev_bf16(normal_bf16(rng, (T, 1024), 1.0))
    w, ids, _ = fused_moe.route(dx, layer.gate_weight, layer.router_spec)
    bad = ids.clone()
    bad[7, 3] = E + 3
    print("case device waves eager, id past the layer", flush=True)
    with pytest.raises(phase_split.B2WaveFallback, match="in no wave"):
        fused_moe.run_device_waves(rt, layer_id=92, hidden=dx, topk_weights=w, topk_ids=bad, num_logical_experts=E)
    with pytest.raises(RuntimeError, match="without ready slots"):
        fused_moe.run_overflow_prefill(rt, layer_id=92, hidden=dx, topk_weights=w, topk_ids=bad,
                                       num_logical_experts=E, device_planned=True)
    native.device_flags(clear=True)
    # captured on valid routes, replayed with the bad id: the pair is masked
    # (its y row still holds the previous replay's value) and counted
    static_w, static_ids = w.clone(), ids.clone()
    out = torch.empty((T, 1024), dtype=torch.bfloat16, device="cuda")

    def run():
        fused_moe.run_device_waves(rt, layer_id=92, hidden=dx, topk_weights=static_w, topk_ids=static_ids,
                                   num_logical_experts=E, out=out)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    g.replay()
    torch.cuda.synchronize()
    assert native.device_flags(clear=True) == [0] * native.FLAG_COUNT
    print("case device waves replay, id past the layer", flush=True)
    static_ids.copy_(bad)
    g.replay()
    torch.cuda.synchronize()
    got = out.clone()
    assert native.device_flags(clear=True)[native.FLAG_UNPLACED] == 1
    wz, iz = _zero_weight_twin(w, ids, 7, 3, valid_id=int(ids[7, 3]))
    ref = fused_moe.run_full_layer(rt, layer_id=92, hidden=dx, topk_weights=wz, topk_ids=iz,
                                   num_logical_experts=E).clone()
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    with pytest.raises(RuntimeError, match="invalid"):
        static_ids.copy_(bad)
        g.replay()
        torch.cuda.synchronize()
        rt.check_device_flags()
    rt.check_device_flags()  # cleared by the failed check


def test_decode_overflow_pass_masks_a_pair_in_neither_table_and_flags_it():
    fused_moe, native, phase_split, SlotMoELayer, Cfg, Runtime = _mods()
    rng = np.random.default_rng(44)
    E, H, I, k, T = 64, 1024, 256, 8, 16
    w13 = normal_bf16(rng, (E, 2 * I, H), 0.02)
    w2 = normal_bf16(rng, (E, H, I), 0.02)
    gate = to_dev_bf16(normal_bf16(rng, (E, H), 0.02))
    common = dict(enabled=True, async_load=True, pin_host_memory=True, graph_compatible_offload=True)
    rt_a = Runtime(Cfg(num_slots=32, decode_overflow=True, **common))
    rt_b = Runtime(Cfg(num_slots=64, **common))
    la = SlotMoELayer(layer_id=93, runtime=rt_a, gate_weight=gate, w13_weight=_tb(w13), w2_weight=_tb(w2), top_k=k)
    lb = SlotMoELayer(layer_id=94, runtime=rt_b, gate_weight=gate, w13_weight=_tb(w13), w2_weight=_tb(w2), top_k=k)
    la.register()
    lb.register()
    dx = to_dev_bf16(normal_bf16(rng, (T, H), 1.0))
    w, ids, _ = fused_moe.route(dx, gate, la.router_spec)
    flat = ids.cpu().flatten().tolist()
    counts = {e: flat.count(e) for e in set(flat)}
    pa = rt_a.stage_fixed_slot_plan(layer_id=93, active_experts=tuple(sorted(counts)), num_logical_experts=E,
                                    token_counts=counts)
    assert pa.overflow is not None, "the case needs more experts than the bank's slots"
    rt_b.stage_fixed_slot_plan(layer_id=94, active_experts=tuple(sorted(counts)), num_logical_experts=E)
    native.device_flags(clear=True)
    bad = ids.clone()
    bad[3, 5] = E + 2  # in neither the bank's table nor the overflow table
    print("case decode overflow pass, pair in neither table", flush=True)
    ovf = rt_a.decode_overflow_slot_weights(layer_id=93, n_pairs=T * k)
    bank_a, bank_b = rt_a.slot_bank(93), rt_b.slot_bank(94)
    out_a, _ = fused_moe._fused_experts_ws(dx, w, bad, bank_a.w13_slots, bank_a.w2_slots, rt_a.log2phy_buffer(93),
                                           overflow=ovf)
    out_a = out_a.clone()
    torch.cuda.synchronize()
    assert native.device_flags(clear=True)[native.FLAG_UNPLACED] == 1
    wz, iz = _zero_weight_twin(w, ids, 3, 5, valid_id=int(ids[3, 5]))
    out_b = fused_moe.fused_experts(dx, wz, iz, bank_b.w13_slots, bank_b.w2_slots, rt_b.log2phy_buffer(94)).clone()
    torch.cuda.synchronize()
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16))
    assert native.device_flags(clear=True) == [0] * native.FLAG_COUNT
