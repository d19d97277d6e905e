"""The DeepSeek-V3-style layer at its own working set
on the GPU: 256 routed experts in a page-locked host store, a 64-slot bank,
the shared expert pinned in the bank's suffix (id 256, weight 1 on every
token), H 7168, I 2048, grouped sigmoid router with a selection-only bias,
routed_scaling_factor 2.5.

* a 2048-token prefill touches every routed expert: device-planned waves
  (H2D inside) and host-planned waves equal the blocking full layer bit for
  bit, and sampled y rows match the oracle's expert MLP;
* decode batches go through the staging op: 8 tokens on the LRU bank (plus
  one overflow pass when their union passes 64 experts), 32 tokens (about
  160 experts, past what one overflow pass holds) on the device-planned
  waves; every output equals the resident layer's bit for bit, and sampled
  tokens match the oracle within 2e-2 x RMS.
Reference: runtime.py:2035-2258 (stage banks), patch_fused_moe.py:2300-2441
(fused shared lane), :2443-3470 (waves)."""

import gc

import numpy as np
import pytest
import torch

from oracle import mlp as omlp
from oracle.bf16 import bf16_to_f32
from tests._util import OUT_TOL, from_dev_bf16, rel_max_err, ulp_mismatch_stats

pytestmark = pytest.mark.gpu

H, E, I, K, P = 7168, 256, 2048, 8, 64
NT = E + 1


@pytest.fixture(scope="module")
def c5():
    from vllm_moe_offload_amd import fused_moe
    from vllm_moe_offload_amd.moe_offload.config import MoeOffloadConfig
    from vllm_moe_offload_amd.moe_offload.runtime import MoeOffloadRuntime

    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(7168)
    w13 = torch.empty((NT, 2 * I, H), dtype=torch.bfloat16, device=dev)
    w2 = torch.empty((NT, H, I), dtype=torch.bfloat16, device=dev)
    for e in range(NT):
        w13[e].copy_(torch.randn((2 * I, H), generator=g, device=dev) * 0.02)
        w2[e].copy_(torch.randn((H, I), generator=g, device=dev) * 0.02)
    gate = (torch.randn((E, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    bias = (torch.randn((E,), generator=g, device=dev) * 0.01).float()
    h13 = torch.empty((E, 2 * I, H), dtype=torch.bfloat16, pin_memory=True)
    h2 = torch.empty((E, H, I), dtype=torch.bfloat16, pin_memory=True)
    for e in range(E):
        h13[e].copy_(w13[e])
        h2[e].copy_(w2[e])
    rt = MoeOffloadRuntime(MoeOffloadConfig(enabled=True, num_slots=P, async_load=True, pin_host_memory=True,
                                            graph_compatible_offload=True, decode_overflow=True,
                                            b2_wave_prefill=True, device_wave_prefill=True))
    rt.register_host_buffers(layer_id=0, w13_host=h13, w2_host=h2, slot_device=dev,
                             shared_w13=w13[E:], shared_w2=w2[E:])
    spec = fused_moe.RouterSpec(top_k=K, scoring_func="sigmoid", use_grouped_topk=True, num_expert_group=8,
                                topk_group=4, routed_scaling_factor=2.5, e_score_correction_bias=bias, n_shared=1)
    torch.cuda.synchronize()
    yield dict(rt=rt, w13=w13, w2=w2, gate=gate, spec=spec, g=g,
               l2p=torch.arange(NT, dtype=torch.int32, device=dev))
    del rt, w13, w2, h13, h2
    fused_moe.clear_workspaces()
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _oracle_tokens(c, x, w, ids, tokens):
    """The oracle layer (routed + shared, f32 before the final cast) of the
    given tokens, over a compact bank of just their experts."""
    ids_s = ids[tokens].cpu().numpy()
    used = np.unique(ids_s)
    local = {int(e): i for i, e in enumerate(used)}
    w13 = np.stack([from_dev_bf16(c["w13"][int(e)]) for e in used])
    w2 = np.stack([from_dev_bf16(c["w2"][int(e)]) for e in used])
    ids_l = np.vectorize(lambda e: local[int(e)])(ids_s).astype(np.int32)
    return omlp.moe_layer(from_dev_bf16(x[tokens]), ids_l, from_dev_bf16(w[tokens]), None, w13, w2)


def test_c5_prefill_2048_waves_equal_full_layer_and_oracle(c5):
    from vllm_moe_offload_amd import fused_moe

    rt, T = c5["rt"], 2048
    x = (torch.randn((T, H), generator=c5["g"], device="cuda")).to(torch.bfloat16)
    w, ids, _ = fused_moe.route(x, c5["gate"], c5["spec"])
    ids_np = ids.cpu().numpy()
    assert np.unique(ids_np[:, :K]).size == E and (ids_np[:, K] == E).all()
    print("case c5 prefill: device-planned waves", flush=True)
    out_d = fused_moe.run_device_waves(rt, layer_id=0, hidden=x, topk_weights=w, topk_ids=ids,
                                       num_logical_experts=NT).clone()
    print("case c5 prefill: host-planned waves", flush=True)
    out_h, report = fused_moe.run_wave_prefill(rt, layer_id=0, hidden=x, topk_weights=w, topk_ids=ids,
                                               num_logical_experts=NT)
    out_h = out_h.clone()
    y_h = fused_moe.get_workspace(T, K + 1, rt.slot_bank(0).physical_expert_count, H, I, x.device,
                                  tag="waves").y.clone()
    print("case c5 prefill: full layer", flush=True)
    out_f = fused_moe.run_full_layer(rt, layer_id=0, hidden=x, topk_weights=w, topk_ids=ids,
                                     num_logical_experts=NT).clone()
    torch.cuda.synchronize()
    print(f"waves {len(report.waves)} sizes {[len(v) for v in report.waves]} h2d {report.h2d_bytes}", flush=True)
    assert len(report.waves) == 4 and all(len(v) <= P for v in report.waves)
    assert report.h2d_bytes >= (E - P) * 3 * H * I * 2
    for name, got in (("device waves", out_d), ("host waves", out_h)):
        ndiff = int((got.view(torch.int16) != out_f.view(torch.int16)).sum().item())
        assert ndiff == 0, f"{name}: {ndiff} elements differ from the full layer"
    rng = np.random.default_rng(6)
    pairs = rng.choice(T * (K + 1), size=24, replace=False)
    x_np = bf16_to_f32(from_dev_bf16(x))
    got = bf16_to_f32(from_dev_bf16(y_h))[pairs]
    ref = np.empty_like(got)
    for i, p in enumerate(pairs):
        e = int(ids_np.reshape(-1)[p])
        ref[i] = omlp.expert_mlp(x_np[p // (K + 1)][None, :], bf16_to_f32(from_dev_bf16(c5["w13"][e])),
                                 bf16_to_f32(from_dev_bf16(c5["w2"][e])))[0]
    rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
    frac, max_ulps = ulp_mismatch_stats(got, ref, abs_floor=rms / 256, count_floor=rms / 4096)
    print(f"  sampled y: frac>1ulp {frac:.2e} max {max_ulps:.2f} ulp", flush=True)
    assert frac <= 1e-3 and max_ulps <= 2.0
    tokens = [0, 777, 2047]
    want = _oracle_tokens(c5, x, w, ids, tokens)
    assert rel_max_err(bf16_to_f32(from_dev_bf16(out_f[tokens])), want) <= OUT_TOL


@pytest.mark.parametrize("B,branch", [(8, "bank"), (32, "device_waves")])
def test_c5_decode_through_the_staging_op(c5, B, branch):
    from vllm_moe_offload_amd import fused_moe
    from vllm_moe_offload_amd.ops.fused_moe.moe_offload_stage_op import PHASE_DECODE, stage_topk_for_layer

    rt = c5["rt"]
    bank = rt.slot_bank(0)
    for step in range(3):
        x = (torch.randn((B, H), generator=c5["g"], device="cuda")).to(torch.bfloat16)
        w, ids, _ = fused_moe.route(x, c5["gate"], c5["spec"])
        n_routed = int(ids[:, :K].unique().numel())
        stage_topk_for_layer(rt, ids, 0, NT, PHASE_DECODE)
        took = "device_waves" if rt.consume_device_waves(layer_id=0, topk_ids=ids) else "bank"
        print(f"case c5 decode B={B} step {step}: {n_routed} routed experts, {took}", flush=True)
        assert took == branch
        if took == "device_waves":
            out = fused_moe.run_device_waves(rt, layer_id=0, hidden=x, topk_weights=w, topk_ids=ids,
                                             num_logical_experts=NT)
        else:
            ovf = rt.decode_overflow_slot_weights(layer_id=0, n_pairs=int(ids.numel()))
            out, _ = fused_moe._fused_experts_ws(x, w, ids, bank.w13_slots, bank.w2_slots, rt.log2phy_buffer(0),
                                                 overflow=ovf)
            rt.record_layer_compute(0)
        out = out.clone()
        ref = fused_moe.fused_experts(x, w, ids, c5["w13"], c5["w2"], c5["l2p"]).clone()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), step
        if step == 0:
            tokens = [0, B // 2, B - 1]
            want = _oracle_tokens(c5, x, w, ids, tokens)
            assert rel_max_err(bf16_to_f32(from_dev_bf16(out[tokens])), want) <= OUT_TOL
    rt.check_device_flags()
