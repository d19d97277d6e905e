#!/usr/bin/env python3
"""Benchmark of the slot-indexed fused-MoE hot path on one MI355X.

Headline (value): Qwen3-30B-A3B-shaped decode, 48 MoE layers, 64 slots per
layer, batch 1 — MoE-layer microseconds per token per layer, measured as the
hipGraph replay of the 48-layer decode compute (per layer: gate GEMV, top-k,
slot remap + permutation, gate_up GEMV + SiLU*mul, down GEMV + combine)
after the step's eager staging has made every routed expert resident.  Also reported in the same JSON line:

  decode[B]   B in --batches: graph-replayed layer us/token, layer HBM GB/s,
              slot-miss rate of the Zipf-skewed router, and the eager
              staging-inclusive step time (D2H of the ids, LRU, H2D)
  roofline    dominant kernel (gate_up GEMV + SiLU*mul at B=1; the down
              GEMV + combine beside it), timed with HIP events over launches
              rotating through the 48 layers
  prefill     4096 tokens, 48 slots, uniform router: capacity waves with one
              combine (compute TFLOP/s and MFMA fraction; staged wall time;
              H2D GB/s), against the blocking full layer; torch.bmm
              (hipBLASLt) on the same per-slot shapes as a reference point
  staging     forced k misses per layer per step (k in 1, 4, 8): H2D GB/s on
              the transfer stream and the fraction of compute overlapped,
              with per-layer graph replays and stable slot addresses
  deepseek    DeepSeek-V3-style layer (H 7168, E 256 + 1 shared, I 2048,
              grouped sigmoid router): every expert resident (kernels on the
              real working set), and staged through a 64-slot bank and a
              page-locked host store (decode B 1/8/32, 2048-token prefill)
  cpu_baseline  the numpy oracle of the same layer on the host cores

Synthetic data: weights N(0, 0.02) bf16 and hidden states N(0, 1) from fixed
seeds.  To bound page-locked host memory the 48 layers share one 128-expert
pinned host store (1.2 GB); every miss still moves its full 9,437,184 bytes.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "vllm-ascend-hust-latchmoe_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA

H, E, I, K = 2048, 128, 768, 8  # Qwen3-30B-A3B MoE layer
EXPERT_BYTES = 3 * H * I * 2    # 9,437,184


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def zipf_bias(seed: int, n: int = E, s: float = 1.1) -> list[float]:
    """Seeded Zipf(s) rank permutation mapped linearly onto [-2, +2] logits."""
    import numpy as np

    rng = np.random.default_rng(seed)
    ranks = rng.permutation(n) + 1
    logp = -s * np.log(ranks.astype(np.float64))
    lo, hi = -s * math.log(n), 0.0
    return list((-2.0 + 4.0 * (logp - lo) / (hi - lo)).astype(np.float32))


class Timer:
    """HIP-event timer on a stream."""

    def __init__(self, stream=None):
        import torch

        self.stream = stream or torch.cuda.current_stream()
        self.a = torch.cuda.Event(enable_timing=True)
        self.b = torch.cuda.Event(enable_timing=True)

    def __enter__(self):
        self.a.record(self.stream)
        return self

    def __exit__(self, *exc):
        self.b.record(self.stream)

    def ms(self) -> float:
        self.b.synchronize()
        return float(self.a.elapsed_time(self.b))


def time_queued(fn, reps: int) -> float:
    """Mean ms per call of fn over reps calls (HIP events on the current
    stream).  One untimed call is queued first, so the device is busy while
    the host issues the timed calls: the first timed call does not wait for
    the host."""
    fn()
    with Timer() as t:
        for _ in range(reps):
            fn()
    return t.ms() / reps


# ---------------------------------------------------------------------------
# C2: 48-layer decode
# ---------------------------------------------------------------------------
class DecodeModel:
    def __init__(self, n_layers: int, num_slots: int, host_w13, host_w2, seed: int = 1):
        import torch

        from vllm_moe_offload_amd.fused_moe import RouterSpec
        from vllm_moe_offload_amd.moe_offload.config import MoeOffloadConfig
        from vllm_moe_offload_amd.moe_offload.runtime import MoeOffloadRuntime

        self.L = n_layers
        self.rt = MoeOffloadRuntime(MoeOffloadConfig(enabled=True, num_slots=num_slots, async_load=True,
                                                     graph_compatible_offload=True, b2_wave_prefill=True,
                                                     decode_overflow=True))
        dev = torch.device("cuda")
        g = torch.Generator(device=dev)
        self.gates, self.specs = [], []
        for l in range(n_layers):
            g.manual_seed(seed * 1000 + l)
            self.gates.append((torch.randn((E, H), generator=g, device=dev) * 0.02).to(torch.bfloat16))
            # the Zipf skew is a gate bias (added to the logits before the softmax)
            bias = torch.tensor(zipf_bias(seed * 7919 + l), dtype=torch.float32, device=dev)
            self.specs.append(RouterSpec(top_k=K, scoring_func="softmax", renormalize=True, logit_bias=bias))
            self.rt.register_host_buffers(layer_id=l, w13_host=host_w13, w2_host=host_w2, slot_device=dev)

    def bank(self, l):
        return self.rt.slot_bank(l)


def _route(x, model, l, w_out, ids_out, logits_out):
    """Gate GEMV then top-k selection (two launches)."""
    from vllm_moe_offload_amd import native

    native.router_gate(x, model.gates[l], logits_out)
    native.router_topk(logits_out, K, logit_bias=model.specs[l].logit_bias, w_bf16=w_out, ids=ids_out)


def _interval_overlap(a: list[tuple[float, float]], b: list[tuple[float, float]]) -> float:
    """Total length of a's intervals covered by the union of b's (ms)."""
    merged: list[list[float]] = []
    for s0, s1 in sorted(b):
        if merged and s0 <= merged[-1][1]:
            merged[-1][1] = max(merged[-1][1], s1)
        else:
            merged.append([s0, s1])
    tot = 0.0
    for a0, a1 in a:
        for m0, m1 in merged:
            lo, hi = max(a0, m0), min(a1, m1)
            if hi > lo:
                tot += hi - lo
    return tot


def bench_decode(model: DecodeModel, B: int, steps: int, warmup: int, seed: int, budget_s: float) -> dict:
    """B tokens per step through the 48 layers, staged per layer while the
    previous layer computes.  Per step: eager routing of every layer and one
    D2H of the ids (the seam), then the per-layer pipeline: publish layer l's
    copies (the compute stream waits on their ready event), queue layer
    l + 1's misses on the transfer stream (prefetch), replay layer l's
    captured decode graph, record the compute that reads layer l's bank.
    Each replay is bracketed by HIP events recorded after the copy wait;
    that interval also holds any wait for the host to submit the replay, so
    it is reported as the pipelined layer interval, not as compute.  A layer
    whose working set exceeds its slots (by at most the slot count) stages
    the excess into its stage buffer and replays the graph captured with the
    overflow pass; a larger excess would run eager capacity waves.  The
    compute rate (the headline) is the 48-layer graph replayed over the
    staged, HBM-resident step: one replay, timed with HIP events (on a step
    with overflow layers, the variant with every layer's overflow pass; the
    stage buffers then hold the last layers' overflow experts, the same
    work)."""
    import numpy as np
    import torch

    from vllm_moe_offload_amd import fused_moe

    dev = torch.device("cuda")
    L = model.L
    rt = model.rt
    engine = rt.transfer_engine
    gx = torch.Generator(device=dev)
    gx.manual_seed(seed + B)
    n_inputs = steps + warmup
    xs = torch.randn((n_inputs, B, H), generator=gx, device=dev).to(torch.bfloat16)
    static_x = torch.empty((B, H), dtype=torch.bfloat16, device=dev)
    logits = [torch.empty((B, E), dtype=torch.bfloat16, device=dev) for _ in range(L)]
    ws_w = [torch.empty((B, K), dtype=torch.bfloat16, device=dev) for _ in range(L)]
    ws_ids = [torch.empty((B, K), dtype=torch.int32, device=dev) for _ in range(L)]
    outs = [torch.empty((B, H), dtype=torch.bfloat16, device=dev) for _ in range(L)]
    P = model.bank(0).physical_expert_count
    ws = fused_moe.get_workspace(B, K, P, H, I, dev, tag=f"bench{B}")
    cap = rt.config.num_slots

    def compute_layer(l, two=False):
        # the slot table is final (staged from the eager routing of this
        # step), so selection and permutation run as one launch
        bank = model.bank(l)
        ovf = rt.decode_overflow_slot_weights(layer_id=l, n_pairs=B * K) if two else None
        fused_moe.decode_layer(static_x, model.gates[l], model.specs[l], bank.w13_slots, bank.w2_slots,
                               rt.log2phy_buffer(l), workspace=ws, out=outs[l], logits_out=logits[l],
                               w_out=ws_w[l], ids_out=ws_ids[l], overflow=ovf)

    counts: list[dict[int, int]] = [{} for _ in range(L)]

    def route_all(i: int) -> list[tuple[int, ...]]:
        static_x.copy_(xs[i])
        for l in range(L):
            _route(static_x, model, l, ws_w[l], ws_ids[l], logits[l])
        ids_host = torch.stack(ws_ids).cpu().numpy()  # one D2H for all layers' ids
        out = []
        for l in range(L):
            u, c = np.unique(ids_host[l], return_counts=True)
            counts[l] = dict(zip(u.tolist(), c.tolist()))
            out.append(tuple(u.tolist()))
        return out

    stats = {"hits": 0, "misses": 0, "overflow_layers": 0}
    graphs: dict = {}  # (layer, overflow pass) -> graph
    big: dict = {}  # overflow pass -> the 48-layer graph
    ev0 = [torch.cuda.Event(enable_timing=True) for _ in range(L)]
    ev1 = [torch.cuda.Event(enable_timing=True) for _ in range(L)]
    tx0 = [torch.cuda.Event(enable_timing=True) for _ in range(L)]
    tx1 = [torch.cuda.Event(enable_timing=True) for _ in range(L)]
    base = torch.cuda.Event(enable_timing=True)

    def prefetch(l, a):
        if len(a[l]) > cap and not rt.can_stage_decode_overflow(layer_id=l, active_expert_count=len(a[l])):
            return None
        s = engine._transfer_stream(dev)
        tx0[l].record(s)
        p = rt.prefetch_fixed_slot_plan(layer_id=l, active_experts=a[l], num_logical_experts=E, token_counts=counts[l])
        tx1[l].record(s)
        return p

    def capture(l, two):
        torch.cuda.synchronize()
        rt.capture_safe_slot_weights(layer_id=l)  # lock slot addresses
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            compute_layer(l, two)
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            compute_layer(l, two)
        return g

    def pipelined_step(a, timed: bool):
        """Returns (compute ms, overflow ms, compute intervals, copy intervals,
        eager layers, overflow-pass layers)."""
        comp = torch.cuda.current_stream()
        base.record(comp)
        pend = prefetch(0, a)
        waves_ms = 0.0
        eager_layers = []
        n_two = 0
        for l in range(L):
            two = False
            if pend is not None:
                prepared = rt.complete_fixed_slot_plan(pend)
                two = prepared.overflow is not None
                assert two == (pend.overflow is not None), "staged overflow lost before compute"
                stats["hits"] += len(pend.hits)
                stats["misses"] += len(pend.misses)
            nxt = prefetch(l + 1, a) if l + 1 < L else None
            if pend is None:
                ev0[l].record(comp)
                fused_moe.run_wave_prefill(rt, layer_id=l, hidden=static_x, topk_weights=ws_w[l],
                                           topk_ids=ws_ids[l], num_logical_experts=E, out=outs[l])
                ev1[l].record(comp)
                eager_layers.append(l)
            else:
                n_two += int(two)
                g = graphs.get((l, two))
                if g is None:
                    g = graphs[(l, two)] = capture(l, two)
                ev0[l].record(comp)
                g.replay()
                ev1[l].record(comp)
            rt.record_layer_compute(l)
            pend = nxt
        ev1[L - 1].synchronize()
        torch.cuda.synchronize()
        comp_iv, copy_iv, c_ms = [], [], 0.0
        for l in range(L):
            t0, t1 = base.elapsed_time(ev0[l]), base.elapsed_time(ev1[l])
            if l in eager_layers:
                waves_ms += t1 - t0
            else:
                c_ms += t1 - t0
                comp_iv.append((t0, t1))
        if timed:
            for l in range(L):
                if l not in eager_layers:
                    copy_iv.append((base.elapsed_time(tx0[l]), base.elapsed_time(tx1[l])))
        return c_ms, waves_ms, comp_iv, copy_iv, len(eager_layers), n_two

    def capture_big(two):
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for l in range(L):
                compute_layer(l, two)
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for l in range(L):
                compute_layer(l, two)
        for l in range(L):
            rt.record_layer_compute(l)
        return g

    t_begin = time.perf_counter()
    for i in range(warmup):
        pipelined_step(route_all(i), timed=False)
    torch.cuda.synchronize()
    fp0 = [rt._slot_address_fingerprint(l) for l in range(L)]
    resident_ms = []
    stats["hits"] = stats["misses"] = 0
    comp_ms, wave_ms, step_ms, U, ov_num, ov_den, n_eager, n_over = [], [], [], [], 0.0, 0.0, [], []
    done = 0
    for i in range(warmup, warmup + steps):
        if time.perf_counter() - t_begin > budget_s and done >= 8:
            break
        t0 = time.perf_counter()
        a = route_all(i)
        U.append(sum(len(x) for x in a) / L)
        c, w, civ, tiv, ne, n2 = pipelined_step(a, timed=True)
        step_ms.append((time.perf_counter() - t0) * 1000.0)
        ov_num += _interval_overlap(civ, tiv)
        ov_den += sum(t1 - t0_ for t0_, t1 in civ)
        n_eager.append(ne)
        n_over.append(n2)
        if ne == 0:
            comp_ms.append(c)
            two = n2 > 0
            if two not in big:
                big[two] = capture_big(two)
            # the same step again with every layer resident: one replay
            with Timer() as t:
                big[two].replay()
            resident_ms.append(t.ms())
            for l in range(L):
                rt.record_layer_compute(l)
        else:
            wave_ms.append(c + w)
        done += 1
    torch.cuda.synchronize()
    assert fp0 == [rt._slot_address_fingerprint(l) for l in range(L)], "slot addresses moved"
    res: dict = {"B": B, "steps_run": done, "steps_all_graph": len(comp_ms),
                 "steps_with_wave_layers": len(wave_ms),
                 "wave_layers_per_step": round(sum(n_eager) / max(1, len(n_eager)), 2),
                 "overflow_pass_layers_per_step": round(sum(n_over) / max(1, len(n_over)), 2)}
    res["slot_miss_rate"] = round(stats["misses"] / max(1, stats["hits"] + stats["misses"]), 4)
    u = sum(U) / max(1, len(U))
    res["distinct_experts_per_layer"] = round(u, 2)
    layer_bytes = u * EXPERT_BYTES + E * H * 2 + 2 * B * H * 2
    res["algorithmic_bytes_per_layer"] = int(layer_bytes)
    res["pipelined_step_ms_mean"] = round(sum(step_ms) / max(1, len(step_ms)), 3)
    res["compute_under_copies_frac"] = round(ov_num / ov_den, 4) if ov_den > 0 else 0.0
    if comp_ms:
        ms = sorted(comp_ms)
        res["pipelined_layer_interval_us_mean"] = round(sum(ms) / len(ms) * 1000.0 / L, 3)
    if wave_ms:
        res["steps_with_waves_compute_ms_mean"] = round(sum(wave_ms) / len(wave_ms), 3)
    # the compute rate: the 48-layer graph over each staged, resident step
    if resident_ms:
        ms = sorted(resident_ms)
        mean = sum(ms) / len(ms)
        us_layer = mean * 1000.0 / L
        res.update(
            graph_replays=len(ms),
            graph_ms_per_step_mean=round(mean, 4),
            graph_ms_per_step_median=round(ms[len(ms) // 2], 4),
            graph_ms_p10=round(ms[len(ms) // 10], 4),
            graph_ms_p90=round(ms[(9 * len(ms)) // 10], 4),
            us_per_layer=round(us_layer, 3),
            us_per_token_per_layer=round(us_layer / B, 3),
            layer_hbm_gbs=round(layer_bytes / (us_layer * 1e-6) / 1e9, 1),
        )
        res["layer_hbm_frac"] = round(res["layer_hbm_gbs"] / HBM_PEAK_GBS, 4)
    res["_state"] = (ws_w, ws_ids, static_x)
    return res


def bench_decode_roofline(model: DecodeModel, state, reps: int = 10) -> dict:
    """Dominant decode kernel at B=1: the gate_up GEMV + SiLU*mul (two thirds
    of the layer's bytes), 48*reps launches rotating through the 48 layers'
    slot banks (29 GB, far beyond the 256 MB MALL), captured in one graph so
    they run back to back, timed with HIP events on the stream they are
    launched on.  Same measurement for the down GEMV + combine."""
    import torch

    from vllm_moe_offload_amd import native

    ws_w, ws_ids, x = state
    L = model.L
    dev = torch.device("cuda")
    B = x.shape[0]
    P = model.bank(0).physical_expert_count
    perms, acts = [], []
    out = torch.empty((B, H), dtype=torch.bfloat16, device=dev)
    for l in range(L):
        p = native.Permutation.allocate(B * K, P, dev)
        native.permute(ws_ids[l], p, log2phy=model.rt.log2phy_buffer(l))
        perms.append(p)
        acts.append(torch.empty((B * K, I), dtype=torch.bfloat16, device=dev))
    torch.cuda.synchronize()
    U = [int(perms[l].meta[native.META_ACTIVE].item()) for l in range(L)]
    u = sum(U) / L

    def gateup():
        for _ in range(reps):
            for l in range(L):
                native.gateup_silu(x, K, model.bank(l).w13_slots, perms[l], acts[l], path=native.LMOE_PATH_GEMV)

    def down():
        for _ in range(reps):
            for l in range(L):
                native.down_combine(acts[l], ws_w[l], model.bank(l).w2_slots, perms[l], out)

    res = {}
    for name, fn, byts in (
        ("gateup_gemv_kernel", gateup, u * (2 * I * H * 2) + B * H * 2 + B * K * I * 2),
        ("down_combine_gemv_kernel", down, u * (H * I * 2) + B * K * I * 2 + B * H * 2),
    ):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        g.replay()
        stream = torch.cuda.current_stream()
        with Timer(stream) as t:
            g.replay()
        ms = t.ms()
        avg_us = ms * 1000.0 / (reps * L)
        res[name] = {"avg_launch_us": round(avg_us, 3), "bytes_per_launch": int(byts),
                     "achieved_gbs": round(byts / (avg_us * 1e-6) / 1e9, 1), "launches": reps * L}
    res["distinct_slots_per_launch"] = round(u, 2)
    # calibration for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE: one device copy
    # of exactly 64 MiB (read 64 MiB, write 64 MiB)
    src = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    res["calibration_copy_bytes"] = int(src.numel())
    return res


# ---------------------------------------------------------------------------
# C3: multi-wave prefill
# ---------------------------------------------------------------------------
def bench_prefill(host_w13, host_w2, T: int = 4096, slots: int = 48, reps: int = 5) -> dict:
    import torch

    from vllm_moe_offload_amd import fused_moe, native
    from vllm_moe_offload_amd.fused_moe import RouterSpec, route
    from vllm_moe_offload_amd.moe_offload.config import MoeOffloadConfig
    from vllm_moe_offload_amd.moe_offload.runtime import MoeOffloadRuntime

    dev = torch.device("cuda")
    rt = MoeOffloadRuntime(MoeOffloadConfig(enabled=True, num_slots=slots, async_load=True, b2_wave_prefill=True))
    rt.register_host_buffers(layer_id=0, w13_host=host_w13, w2_host=host_w2, slot_device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(4096)
    gate = (torch.randn((E, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    x = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
    spec = RouterSpec(top_k=K)
    w, ids, _ = route(x, gate, spec)
    torch.cuda.synchronize()
    pairs = T * K
    flops = 2.0 * pairs * 3 * H * I
    router_flops = 2.0 * T * H * E
    res: dict = {"T": T, "slots": slots, "algorithmic_gflop": round((flops + router_flops) / 1e9, 2)}

    # staged multi-wave layer (H2D from the pinned host store each call)
    fused_moe.run_wave_prefill(rt, layer_id=0, hidden=x, topk_weights=w, topk_ids=ids, num_logical_experts=E)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    nrep = 2
    for _ in range(nrep):
        out_w, rep = fused_moe.run_wave_prefill(rt, layer_id=0, hidden=x, topk_weights=w, topk_ids=ids, num_logical_experts=E)
    torch.cuda.synchronize()
    staged_ms = (time.perf_counter() - t0) * 1000.0 / nrep
    res.update(waves=len(rep.waves), wave_sizes=[len(v) for v in rep.waves], staged_wave_ms=round(staged_ms, 2),
               staged_h2d_gb=round(rep.h2d_bytes / 1e9, 3),
               staged_effective_h2d_gbs=round(rep.h2d_bytes / (staged_ms * 1e-3) / 1e9, 1))

    # the same layer with the waves planned and staged on the device (no D2H
    # of the ids, no host step per wave), eager and as one captured graph
    rt_d = MoeOffloadRuntime(MoeOffloadConfig(enabled=True, num_slots=slots, async_load=True, b2_wave_prefill=True,
                                              device_wave_prefill=True))
    rt_d.register_host_buffers(layer_id=0, w13_host=host_w13, w2_host=host_w2, slot_device=dev)
    out_d = torch.empty((T, H), dtype=torch.bfloat16, device=dev)

    def device_waves():
        fused_moe.run_device_waves(rt_d, layer_id=0, hidden=x, topk_weights=w, topk_ids=ids, num_logical_experts=E,
                                   out=out_d)

    device_waves()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(nrep):
        device_waves()
    torch.cuda.synchronize()
    dev_ms = (time.perf_counter() - t0) * 1000.0 / nrep
    s_cap = torch.cuda.Stream()
    s_cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s_cap):
        device_waves()
    torch.cuda.current_stream().wait_stream(s_cap)
    g_d = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_d):
        device_waves()
    with Timer() as t:
        for _ in range(nrep):
            g_d.replay()
    graph_ms = t.ms() / nrep
    torch.cuda.synchronize()
    res.update(device_planned_staged_wave_ms=round(dev_ms, 2), device_planned_graph_ms=round(graph_ms, 2),
               device_planned_equal_host_planned_bitwise=bool(torch.equal(out_d.view(torch.int16),
                                                                          out_w.view(torch.int16))))
    del g_d

    # compute-only: all waves' experts resident in per-wave banks
    full, _ = rt.prepare_full_layer_prefill_plan(layer_id=0, num_logical_experts=E, device=dev)
    torch.cuda.synchronize()
    wave_banks = []
    for wv in rep.waves:
        idx = torch.tensor(wv, dtype=torch.long, device=dev)
        w13 = full.w1.index_select(0, idx).contiguous()
        w2 = full.w2.index_select(0, idx).contiguous()
        l2p = torch.full((E,), -1, dtype=torch.int32, device=dev)
        l2p[idx] = torch.arange(len(wv), dtype=torch.int32, device=dev)
        wave_banks.append((w13, w2, l2p))
    perm = native.Permutation.allocate(pairs, max(len(v) for v in rep.waves), dev)
    perms_w = [native.Permutation.allocate(pairs, wb[0].shape[0], dev) for wb in wave_banks]
    act = torch.empty((pairs, I), dtype=torch.bfloat16, device=dev)
    y = torch.empty((pairs, H), dtype=torch.bfloat16, device=dev)
    out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)

    wave_bm = [native.prefill_block_m(len(wv), H, I, dev) for wv in rep.waves]

    def waves_compute():
        for (w13, w2, l2p), pw, bm in zip(wave_banks, perms_w, wave_bm):
            native.permute(ids, pw, log2phy=l2p, skip_unmapped=True, block_m=bm)
            native.grouped_mlp(x, K, w13, w2, pw, act, y, path=native.LMOE_PATH_MFMA)
        native.combine(y, w, out)

    ws_full = fused_moe.get_workspace(T, K, E, H, I, dev, tag="bench-full")

    def full_compute():
        fused_moe.fused_experts(x, w, ids, full.w1, full.w2, full.log2phy, path=native.LMOE_PATH_MFMA, workspace=ws_full)

    def gemm_only():
        for (w13, w2, l2p), pw in zip(wave_banks, perms_w):
            native.grouped_mlp(x, K, w13, w2, pw, act, y, path=native.LMOE_PATH_MFMA)

    for fn in (waves_compute, full_compute):
        fn()
    torch.cuda.synchronize()
    for name, fn in (("waves_compute", waves_compute), ("full_layer_compute", full_compute), ("grouped_gemm_only", gemm_only)):
        ms = time_queued(fn, reps)
        tf = flops / (ms * 1e-3) / 1e12
        res[f"{name}_ms"] = round(ms, 3)
        res[f"{name}_tflops"] = round(tf, 1)
        res[f"{name}_mfma_frac"] = round(tf / BF16_PEAK_TFLOPS, 4)
    # per-wave grouped GEMM time and the row-tile height each wave ran with
    per_wave = []
    for (w13, w2, l2p), pw, bm in zip(wave_banks, perms_w, wave_bm):
        native.permute(ids, pw, log2phy=l2p, skip_unmapped=True, block_m=bm)
        ms = time_queued(lambda: native.grouped_mlp(x, K, w13, w2, pw, act, y, path=native.LMOE_PATH_MFMA), reps)
        per_wave.append(round(ms, 3))
    res["wave_block_m"] = wave_bm
    res["wave_gemm_ms"] = per_wave
    res["wave_max_pairs_per_slot"] = [int(pw.counts.max().item()) for pw in perms_w]
    torch.cuda.synchronize()
    same = torch.equal(out.view(torch.int16), ws_full.out[:T].view(torch.int16))
    res["waves_equal_full_layer_bitwise"] = bool(same)

    # the full layer's two grouped GEMMs alone (all 128 slots resident)
    bm_full = native.prefill_block_m(E, H, I, dev, n_pairs=pairs)
    perm_full = native.Permutation.allocate(pairs, E, dev)
    native.permute(ids, perm_full, log2phy=full.log2phy, block_m=bm_full)
    ms = time_queued(lambda: native.grouped_mlp(x, K, full.w1, full.w2, perm_full, act, y,
                                                path=native.LMOE_PATH_MFMA), reps)
    res["full_gemm_only_ms"] = round(ms, 3)
    res["full_gemm_only_tflops"] = round(flops / (ms * 1e-3) / 1e12, 1)
    del perm_full
    res["library_bmm"] = bench_library_bmm((E, len(rep.waves[0])), M=pairs // E, reps=reps)
    return res


def bench_library_bmm(slot_counts, M: int, reps: int = 5) -> dict:
    """The vendor library on the same per-slot shapes, as a reference point
    for the grouped GEMMs: torch.bmm (hipBLASLt) over S slots of a uniform
    M rows each, gate-up [S, M, H] x [S, H, 2I] and down [S, M, I] x [S, I, H],
    contiguous operands.  It does less than the grouped kernels (no row
    gather, no SiLU*mul, no ragged slots, no padding), so its time is a floor
    for what a library GEMM call per pass would take, not a parity check."""
    import torch

    dev = torch.device("cuda")
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    out = {}
    for S in slot_counts:
        r = {}
        total_us = 0.0
        for name, k_dim, n_dim in (("gate_up", H, 2 * I), ("down", I, H)):
            a = torch.randn((S, M, k_dim), generator=g, device=dev).to(torch.bfloat16)
            b = (torch.randn((S, k_dim, n_dim), generator=g, device=dev) * 0.02).to(torch.bfloat16).contiguous()
            c = torch.bmm(a, b)
            us = time_queued(lambda: torch.bmm(a, b, out=c), reps) * 1000.0
            total_us += us
            r[f"{name}_us"] = round(us, 1)
            r[f"{name}_tflops"] = round(2.0 * S * M * k_dim * n_dim / (us * 1e-6) / 1e12, 1)
            del a, b, c
        r["both_us"] = round(total_us, 1)
        r["both_tflops"] = round(2.0 * S * M * 3 * H * I / (total_us * 1e-6) / 1e12, 1)
        out[f"S{S}_M{M}"] = r
    torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------------------
# C4: staging stress with prefetch under per-layer graph replay
# ---------------------------------------------------------------------------
def bench_staging(model: DecodeModel, ks=(1, 4, 8), steps: int = 16, seed: int = 99) -> dict:
    """Per step and layer, exactly k experts that are not resident plus 8-k
    resident ones.  (a) copies alone: every layer's misses queued back to
    back on the transfer stream; (b) pipelined under per-layer graph
    replays: layer l+1's copies are queued (prefetch) before layer l's graph
    is replayed, the compute stream waits for them (complete) right before
    layer l+1.  Overlap comes from event timestamps on both streams inside
    the pipelined run: the share of compute time during which a copy batch
    was in flight."""
    import numpy as np
    import torch

    from vllm_moe_offload_amd import fused_moe

    dev = torch.device("cuda")
    L = model.L
    rt = model.rt
    engine = rt.transfer_engine
    rng = np.random.default_rng(seed)
    B = 1
    x = torch.randn((B, H), device=dev).to(torch.bfloat16)
    w_all = torch.full((L, B, K), 1.0 / K, dtype=torch.bfloat16, device=dev)
    ids_all = torch.zeros((L, B, K), dtype=torch.int32, device=dev)
    ids_host = torch.zeros((L, B, K), dtype=torch.int32, pin_memory=True)
    out_l = [torch.empty((B, H), dtype=torch.bfloat16, device=dev) for _ in range(L)]
    P = model.bank(0).physical_expert_count
    ws = fused_moe.get_workspace(B, K, P, H, I, dev, tag="bench-stage")

    def resident(l):
        return [s.expert_key.expert_id for s in model.bank(l).slots if s.expert_key is not None]

    for l in range(L):
        if len(resident(l)) < K:  # fill an empty bank with a random set of experts
            first = tuple(int(e) for e in rng.permutation(E)[: rt.config.num_slots])
            rt.stage_fixed_slot_plan(layer_id=l, active_experts=first, num_logical_experts=E)
    torch.cuda.synchronize()
    for l in range(L):
        ids_all[l, 0].copy_(torch.tensor(resident(l)[:K], dtype=torch.int32))
    graphs = []
    for l in range(L):
        bank = model.bank(l)

        def piece(l=l, bank=bank):
            fused_moe.fused_experts(x, w_all[l], ids_all[l], bank.w13_slots, bank.w2_slots, rt.log2phy_buffer(l),
                                    out=out_l[l], workspace=ws)

        piece()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            piece()
        graphs.append(g)

    def plan_step(k: int):
        plan = []
        for l in range(L):
            res = resident(l)
            non = sorted(set(range(E)) - set(res))
            miss = list(rng.choice(non, size=k, replace=False))
            hit = list(rng.choice(res, size=K - k, replace=False)) if K - k > 0 else []
            # hits first: staging runs in list order (as the reference's), so a
            # miss listed before a hit could evict that hit's slot
            plan.append(tuple(int(e) for e in hit + miss))
        return plan

    def load_ids(plan):
        ids_host.copy_(torch.tensor(plan, dtype=torch.int32).view(L, B, K))
        ids_all.copy_(ids_host, non_blocking=True)

    compute = torch.cuda.current_stream()
    tstream = engine._transfer_stream(dev)
    torch.cuda.synchronize()
    tc = []
    for _ in range(3):
        with Timer(compute) as t:
            for g in graphs:
                g.replay()
        tc.append(t.ms())
    tc_ms = min(tc)
    fp = [rt._slot_address_fingerprint(l) for l in range(L)]
    base = torch.cuda.Event(enable_timing=True)
    c0 = [torch.cuda.Event(enable_timing=True) for _ in range(L)]
    c1 = [torch.cuda.Event(enable_timing=True) for _ in range(L)]
    x0 = [torch.cuda.Event(enable_timing=True) for _ in range(L)]
    x1 = [torch.cuda.Event(enable_timing=True) for _ in range(L)]
    out: dict = {"compute_only_ms_per_step": round(tc_ms, 3)}
    for k in ks:
        # (a) copies alone: all layers prefetched back to back on the transfer stream
        plan = plan_step(k)
        torch.cuda.synchronize()
        b0 = engine.bytes_issued
        t0 = time.perf_counter()
        with Timer(tstream) as tt:
            pend = [rt.prefetch_fixed_slot_plan(layer_id=l, active_experts=plan[l], num_logical_experts=E)
                    for l in range(L)]
        host_issue_ms = (time.perf_counter() - t0) * 1000.0
        first_misses = sum(len(p_.misses) for p_ in pend)
        th_ms = tt.ms()
        h2d_bytes = engine.bytes_issued - b0
        for l in range(L):
            rt.complete_fixed_slot_plan(pend[l])
        torch.cuda.synchronize()
        # (b) pipelined under per-layer graph replays
        tb, nb, host_ms, miss_counts, ov, cs = [], 0, [], [], 0.0, 0.0
        for _ in range(steps):
            plan = plan_step(k)
            torch.cuda.synchronize()
            b0 = engine.bytes_issued
            t0 = time.perf_counter()
            base.record(compute)
            load_ids(plan)
            x0[0].record(tstream)
            pending = rt.prefetch_fixed_slot_plan(layer_id=0, active_experts=plan[0], num_logical_experts=E)
            x1[0].record(tstream)
            step_misses = 0
            for l in range(L):
                step_misses += len(pending.misses)
                rt.complete_fixed_slot_plan(pending)
                nxt = None
                if l + 1 < L:
                    x0[l + 1].record(tstream)
                    nxt = rt.prefetch_fixed_slot_plan(layer_id=l + 1, active_experts=plan[l + 1],
                                                      num_logical_experts=E)
                    x1[l + 1].record(tstream)
                c0[l].record(compute)
                graphs[l].replay()
                c1[l].record(compute)
                rt.record_layer_compute(l)
                pending = nxt
            host_ms.append((time.perf_counter() - t0) * 1000.0)
            miss_counts.append(step_misses)
            torch.cuda.synchronize()
            tb.append(base.elapsed_time(c1[L - 1]))
            nb += engine.bytes_issued - b0
            comp_iv = [(base.elapsed_time(c0[l]), base.elapsed_time(c1[l])) for l in range(L)]
            copy_iv = [(base.elapsed_time(x0[l]), base.elapsed_time(x1[l])) for l in range(L)]
            ov += _interval_overlap(comp_iv, copy_iv)
            cs += sum(b - a for a, b in comp_iv)
        tb_ms = sum(tb) / len(tb)
        assert fp == [rt._slot_address_fingerprint(l) for l in range(L)], "slot addresses moved"
        out[f"k{k}"] = {
            "h2d_bytes_per_step": int(h2d_bytes),
            "h2d_only_misses": int(first_misses),
            "h2d_only_ms": round(th_ms, 3),
            "h2d_gbs": round(h2d_bytes / (th_ms * 1e-3) / 1e9, 2),
            "host_issue_ms": round(host_issue_ms, 3),
            "pipelined_step_ms": round(tb_ms, 3),
            "pipelined_host_ms": round(sum(host_ms) / len(host_ms), 3),
            "pipelined_h2d_gbs": round(nb / steps / (tb_ms * 1e-3) / 1e9, 2),
            "compute_under_copies_frac": round(ov / cs, 4) if cs > 0 else 0.0,
            "pipelined_compute_ms": round(cs / steps, 3),
            "misses_per_step": sorted(set(miss_counts)),
            "steps": steps,
        }
    out["copy_path"] = "gather kernel" if engine.batches_gathered else "hipMemcpyAsync"
    out["slot_addresses_stable_across_replays"] = True
    return out


# ---------------------------------------------------------------------------
# C5: DeepSeek-V3-style layer (compute, resident slots)
# ---------------------------------------------------------------------------
def bench_deepseek(batches=(1, 8, 32), prefill_tokens: int = 2048, reps: int = 20,
                   staged_steps=(12, 6, 3), prefill_steps: int = 2) -> dict:
    """DeepSeek-V3-style layer (C5) at its own working set: 256 routed
    experts and one shared expert (H 7168, I 2048, grouped sigmoid router,
    bias for selection only, scale 2.5; the shared expert appended to every
    token's top-8 as a pinned suffix id with weight 1).

    resident   all 257 experts in one 257-slot bank (identity table): the
               kernels on the bytes and flops of the real working set
               (distinct experts per step reported), graph-replayed
    staged     the configuration's 64-slot bank, the 256 routed experts in a
               page-locked host store, the shared expert pinned in the bank:
               every step goes through the staging op (vllm::moe_offload_stage)
               -- an LRU bank (plus one overflow pass) up to 128 experts,
               device-planned waves with their H2D inside past that and for
               the prefill -- and is timed whole (eager, copies included);
               H2D bytes and the resident leg's compute time for the same
               batch are reported beside it, and every staged output is
               compared with the resident bank on the same routing
    """
    import torch

    from vllm_moe_offload_amd import fused_moe, native
    from vllm_moe_offload_amd.moe_offload.config import MoeOffloadConfig
    from vllm_moe_offload_amd.moe_offload.runtime import MoeOffloadRuntime
    from vllm_moe_offload_amd.ops.fused_moe.moe_offload_stage_op import (PHASE_DECODE, PHASE_PREFILL,
                                                                         stage_topk_for_layer)

    dev = torch.device("cuda")
    Hd, Ed, Id, Kd, P = 7168, 256, 2048, 8, 64
    NT = Ed + 1  # routed + the shared expert
    g = torch.Generator(device=dev)
    g.manual_seed(7168)
    t0 = time.perf_counter()
    w13 = torch.empty((NT, 2 * Id, Hd), dtype=torch.bfloat16, device=dev)
    w2 = torch.empty((NT, Hd, Id), dtype=torch.bfloat16, device=dev)
    for e in range(NT):
        w13[e].copy_(torch.randn((2 * Id, Hd), generator=g, device=dev) * 0.02)
        w2[e].copy_(torch.randn((Hd, Id), generator=g, device=dev) * 0.02)
    gate = (torch.randn((Ed, Hd), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    bias = (torch.randn((Ed,), generator=g, device=dev) * 0.01).float()
    l2p = torch.arange(NT, dtype=torch.int32, device=dev)
    per_expert = 3 * Hd * Id * 2
    spec = fused_moe.RouterSpec(top_k=Kd, scoring_func="sigmoid", use_grouped_topk=True, num_expert_group=8,
                                topk_group=4, routed_scaling_factor=2.5, e_score_correction_bias=bias, n_shared=1)
    res: dict = {"experts": {"routed": Ed, "shared": 1, "slots": P, "bytes_per_expert": per_expert}}
    log(f"deepseek: weights {time.perf_counter() - t0:.1f}s")

    def timed(step, n):
        step()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        with torch.cuda.graph(graph):
            step()
        graph.replay()
        with Timer() as t:
            for _ in range(n):
                graph.replay()
        return t.ms() / n

    # ---- resident: every expert in HBM, graph-replayed ----
    resident: dict = {}
    for B in batches:
        x = torch.randn((B, Hd), generator=g, device=dev).to(torch.bfloat16)
        logits = torch.empty((B, Ed), dtype=torch.bfloat16, device=dev)
        wv = torch.empty((B, Kd + 1), dtype=torch.bfloat16, device=dev)
        idv = torch.empty((B, Kd + 1), dtype=torch.int32, device=dev)
        ws = fused_moe.get_workspace(B, Kd + 1, NT, Hd, Id, dev, tag=f"ds{B}")
        out = torch.empty((B, Hd), dtype=torch.bfloat16, device=dev)

        def step():
            fused_moe.decode_layer(x, gate, spec, w13, w2, l2p, workspace=ws, out=out, logits_out=logits,
                                   w_out=wv, ids_out=idv)

        ms = timed(step, reps)
        U = int(ws.perm.meta[native.META_ACTIVE].item())
        byts = U * per_expert + Ed * Hd * 2 + 2 * B * Hd * 2
        resident[f"decode_B{B}"] = {
            "us_per_layer": round(ms * 1000, 2), "us_per_token": round(ms * 1000 / B, 2),
            "distinct_experts": U, "hbm_gbs": round(byts / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    T = prefill_tokens
    x = torch.randn((T, Hd), generator=g, device=dev).to(torch.bfloat16)
    logits = torch.empty((T, Ed), dtype=torch.bfloat16, device=dev)
    wv = torch.empty((T, Kd + 1), dtype=torch.bfloat16, device=dev)
    idv = torch.empty((T, Kd + 1), dtype=torch.int32, device=dev)
    ws = fused_moe.get_workspace(T, Kd + 1, NT, Hd, Id, dev, tag=f"ds{T}")
    out = torch.empty((T, Hd), dtype=torch.bfloat16, device=dev)

    def pstep():
        w, ids, _ = fused_moe.route(x, gate, spec, logits_out=logits, w_out=wv, ids_out=idv)
        fused_moe.fused_experts(x, w, ids, w13, w2, l2p, out=out, workspace=ws, path=native.LMOE_PATH_MFMA)

    ms = timed(pstep, 5)
    U = int(ws.perm.meta[native.META_ACTIVE].item())
    flops = 2.0 * T * (Kd + 1) * 3 * Hd * Id + 2.0 * T * Hd * Ed
    byts = U * per_expert + Ed * Hd * 2 + T * Hd * 2 * 2 + T * (Kd + 1) * Hd * 2 * 2
    tf = flops / (ms * 1e-3) / 1e12
    resident[f"prefill_T{T}"] = {"ms": round(ms, 3), "tflops": round(tf, 1),
                                 "mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4), "distinct_experts": U,
                                 "weight_bytes": U * per_expert,
                                 "hbm_frac": round(byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    res["resident"] = resident
    fused_moe.clear_workspaces()
    log(f"deepseek resident: {resident}")

    # ---- staged: 64 slots, the routed experts in page-locked host memory ----
    t0 = time.perf_counter()
    h13 = torch.empty((Ed, 2 * Id, Hd), dtype=torch.bfloat16, pin_memory=True)
    h2 = torch.empty((Ed, Hd, Id), dtype=torch.bfloat16, pin_memory=True)
    for e in range(Ed):
        h13[e].copy_(w13[e])
        h2[e].copy_(w2[e])
    rt = MoeOffloadRuntime(MoeOffloadConfig(enabled=True, num_slots=P, async_load=True, pin_host_memory=True,
                                            graph_compatible_offload=True, decode_overflow=True,
                                            b2_wave_prefill=True, device_wave_prefill=True))
    rt.register_host_buffers(layer_id=0, w13_host=h13, w2_host=h2, slot_device=dev,
                             shared_w13=w13[Ed:], shared_w2=w2[Ed:])
    bank = rt.slot_bank(0)
    log(f"deepseek: pinned host store {time.perf_counter() - t0:.1f}s")

    def staged_step(x, phase):
        """One layer step through the seam: route, stage op, experts; returns
        (out, w, ids, branch, h2d bytes, distinct routed experts)."""
        w, ids, _ = fused_moe.route(x, gate, spec)
        owner = set(int(o) for o in rt.slot_owner_buffer(0).tolist())
        bytes0 = rt.transfer_engine.bytes_issued
        stage_topk_for_layer(rt, ids, 0, NT, phase)
        routed = set(int(e) for e in ids[:, :Kd].unique().tolist())
        if rt.consume_device_waves(layer_id=0, topk_ids=ids):
            out = fused_moe.run_device_waves(rt, layer_id=0, hidden=x, topk_weights=w, topk_ids=ids,
                                             num_logical_experts=NT)
            branch, h2d = "device_waves", len(routed - owner) * per_expert
        else:
            ovf = rt.decode_overflow_slot_weights(layer_id=0, n_pairs=int(ids.numel()))
            out, _ = fused_moe._fused_experts_ws(x, w, ids, bank.w13_slots, bank.w2_slots, rt.log2phy_buffer(0),
                                                 overflow=ovf)
            rt.record_layer_compute(0)
            branch = "bank+overflow" if ovf is not None else "bank"
            h2d = rt.transfer_engine.bytes_issued - bytes0
        return out, w, ids, branch, h2d, len(routed)

    def check(out, x, w, ids):
        ref = fused_moe.fused_experts(x, w, ids, w13, w2, l2p)
        d = (out.float() - ref.float()).abs().max().item()
        rms = ref.float().pow(2).mean().sqrt().item()
        return bool(torch.equal(out.view(torch.int16), ref.view(torch.int16))), d / max(rms, 1e-30)

    staged: dict = {}
    legs = [(f"decode_B{B}", B, PHASE_DECODE, n) for B, n in zip(batches, staged_steps)]
    legs.append((f"prefill_T{T}", T, PHASE_PREFILL, prefill_steps))
    for name, B, phase, n in legs:
        x = torch.randn((B, Hd), generator=g, device=dev).to(torch.bfloat16)
        staged_step(x, phase)  # warm: the bank fills, workspaces and stage buffers exist
        torch.cuda.synchronize()
        ms, h2d, distinct, branches, exact, err = [], 0, [], set(), True, 0.0
        for i in range(n):
            x = torch.randn((B, Hd), generator=g, device=dev).to(torch.bfloat16)
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            out, w, ids, branch, hb, nd = staged_step(x, phase)
            torch.cuda.synchronize()
            ms.append((time.perf_counter() - t1) * 1000.0)
            h2d += hb
            distinct.append(nd)
            branches.add(branch)
            same, e = check(out, x, w, ids)
            exact, err = exact and same, max(err, e)
        mean_ms = sum(ms) / len(ms)
        comp = resident.get(name, {})
        comp_ms = comp.get("ms", comp.get("us_per_layer", 0.0) / 1000.0)
        staged[name] = {
            "ms_per_step": round(mean_ms, 3), "steps": n, "branches": sorted(branches),
            "distinct_routed_experts_mean": round(sum(distinct) / len(distinct), 1),
            "h2d_bytes_per_step": int(h2d / n), "h2d_gbs": round(h2d / n / (mean_ms * 1e-3) / 1e9, 1),
            "resident_compute_ms": round(comp_ms, 3),
            "bitwise_equal_to_resident": exact, "max_abs_err_over_rms_vs_resident": round(err, 6)}
        log(f"deepseek staged {name}: {staged[name]}")
    res["staged"] = staged
    del rt, bank, h13, h2, w13, w2
    fused_moe.clear_workspaces()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


# ---------------------------------------------------------------------------
# CPU baseline: the oracle of one layer on the host cores
# ---------------------------------------------------------------------------
def _cpu_model() -> str:
    """The host CPU: model name plus family / model / stepping (a virtual
    machine may report only a generic name), and the logical CPUs."""
    fields: dict[str, str] = {}
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                fields.setdefault(k.strip().lower(), v.strip())
    except OSError:
        pass
    name = fields.get("model name", "unknown")
    ident = ", ".join(f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields)
    extra = f"{ident}, " if ident else ""
    return f"{name} ({extra}{os.cpu_count()} logical CPUs)"


def bench_cpu_baseline(budget_s: float = 8.0) -> dict:
    """The numpy oracle on the host cores, on bounded samples of the bench's
    workloads (about 25 s in all):

    * decode (C2): one Qwen3-shaped layer per step at B = 1, 4, 16, 64 --
      gate, softmax top-8, the routed experts' SwiGLU MLP with f32
      accumulation, combine; B = 1 is the headline `value`;
    * prefill (C3): the 4096-token routing restricted to 16 of the 128
      experts (~4096 pairs, ~256 rows per expert as in C3), GFLOP/s;
    * staging (C4): expert copies (gate_up + down, 9.4 MB each) from one
      host buffer to another, the CPU form of the host-store -> slot copy.

    Expert weights are generated and stacked outside the timed regions."""
    import numpy as np

    from oracle import mlp as omlp
    from oracle import router as orouter
    from oracle.bf16 import normal_bf16

    rng = np.random.default_rng(5)
    wg = normal_bf16(rng, (E, H), 0.02)
    # 16 distinct weight sets stand in for the 128 experts (expert e uses set
    # e % 16): the oracle converts and multiplies each routed expert's weights
    # whatever their values, and generating 128 sets would take longer than
    # the legs themselves
    pool = [(normal_bf16(rng, (2 * I, H), 0.02), normal_bf16(rng, (H, I), 0.02)) for _ in range(16)]

    def expert(e: int):
        return pool[e % len(pool)]

    def decode_leg(B: int, budget: float) -> tuple[float, int]:
        """3 untimed steps, then the median step of at least 10 (more while
        the budget lasts), per token."""
        times = []
        t_start = time.perf_counter()
        step = 0
        while len(times) < 10 or time.perf_counter() - t_start < budget:
            x = normal_bf16(rng, (B, H), 1.0)
            t0 = time.perf_counter()
            ids, _, wb = orouter.softmax_topk(orouter.gate_logits(x, wg), K)
            t_route = time.perf_counter() - t0
            used = np.unique(ids)
            l2p = np.full(E, -1, dtype=np.int32)
            l2p[used] = np.arange(used.size, dtype=np.int32)
            w13 = np.stack([expert(int(e))[0] for e in used])
            w2 = np.stack([expert(int(e))[1] for e in used])
            t1 = time.perf_counter()
            omlp.moe_layer(x, ids, wb, l2p, w13, w2)
            if step >= 3:
                times.append(t_route + (time.perf_counter() - t1))
            step += 1
        return float(np.median(times)) / B * 1e6, len(times)

    decode = {}
    for B, budget in ((1, budget_s), (4, 3.0), (16, 3.0), (64, 3.0)):
        us, steps = decode_leg(B, budget)
        decode[f"B{B}"] = {"us_per_token_per_layer": round(us, 1), "timed_steps": steps}

    # C3 sample: 4096 tokens routed uniformly, the pairs of 16 experts
    T3, n3 = 4096, 16
    ids3 = np.stack([rng.permutation(E)[:K] for _ in range(T3)]).astype(np.int32)
    x3 = normal_bf16(rng, (T3, H), 1.0)
    slot3 = np.where(ids3 < n3, ids3, -1).astype(np.int32)
    w13_3 = np.stack([expert(e)[0] for e in range(n3)])
    w2_3 = np.stack([expert(e)[1] for e in range(n3)])
    pairs3 = int((slot3 >= 0).sum())
    t0 = time.perf_counter()
    omlp.grouped_mlp(x3, slot3, K, w13_3, w2_3)
    t3 = time.perf_counter() - t0
    prefill_gflops = 2.0 * pairs3 * 3 * H * I / t3 / 1e9

    # C4 sample: expert copies host -> host (one thread)
    src = [np.concatenate([expert(e)[0].reshape(-1), expert(e)[1].reshape(-1)]) for e in range(n3)]
    dst = [np.empty_like(a) for a in src]
    copied, t_copy = 0, 0.0
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < 2.0 or copied == 0:
        t0 = time.perf_counter()
        for a, b in zip(src, dst):
            np.copyto(b, a)
        t_copy += time.perf_counter() - t0
        copied += sum(a.nbytes for a in src)

    cores = int(os.environ.get("OMP_NUM_THREADS") or (os.cpu_count() or 1))
    return {"value": decode["B1"]["us_per_token_per_layer"], "unit": "us/token/layer (decode B=1)",
            "cores": cores, "kind": "port", "cpu_model": _cpu_model(),
            "sample": f"numpy oracle: decode B=1/4/16/64 of one Qwen3-shaped MoE layer (gate, softmax top-8, "
                      f"routed f32-accumulated SwiGLU experts, combine; median step after 3 untimed, at least 10 "
                      f"timed, B=1 for {budget_s:.0f} s); prefill: "
                      f"{pairs3} pairs of a 4096-token routing on {n3} of the 128 experts; staging: "
                      f"{n3} expert copies host->host, one thread; BLAS threads up to {cores}",
            "decode": decode,
            "prefill_gflops": round(prefill_gflops, 1), "prefill_sample_pairs": pairs3,
            "prefill_sample_s": round(t3, 2),
            "host_copy_gbs": round(copied / t_copy / 1e9, 2), "host_copy_threads": 1}


# ---------------------------------------------------------------------------
def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="timed decode steps per batch size")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batches", default="1,4,16,64")
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--slots", type=int, default=64)
    ap.add_argument("--skip", default="", help="comma list of: prefill,staging,deepseek,cpu")
    ap.add_argument("--budget-s", type=float, default=30.0, help="wall-clock cap per decode batch size")
    ap.add_argument("--stage-steps", type=int, default=16)
    ap.add_argument("--out", default="")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; multi-GPU runs are not part of it"}))
        return 2
    skip = set(x for x in args.skip.split(",") if x)

    import torch

    from vllm_moe_offload_amd import native

    native.load_library()
    dev = torch.device("cuda")
    torch.manual_seed(0)
    t_setup = time.perf_counter()
    # shared 128-expert pinned host store (checkpoint layout)
    host_w13 = torch.empty((E, 2 * I, H), dtype=torch.bfloat16, pin_memory=True)
    host_w2 = torch.empty((E, H, I), dtype=torch.bfloat16, pin_memory=True)
    g = torch.Generator(device=dev)
    g.manual_seed(128)
    for e in range(E):
        host_w13[e].copy_((torch.randn((2 * I, H), generator=g, device=dev) * 0.02).to(torch.bfloat16))
        host_w2[e].copy_((torch.randn((H, I), generator=g, device=dev) * 0.02).to(torch.bfloat16))
    model = DecodeModel(args.layers, args.slots, host_w13, host_w2)
    log(f"setup {time.perf_counter() - t_setup:.1f}s")

    decode = {}
    roof = None
    t_run0 = time.perf_counter()
    for B in [int(b) for b in args.batches.split(",") if b]:
        t0 = time.perf_counter()
        r = bench_decode(model, B, args.steps, args.warmup, seed=17, budget_s=args.budget_s)
        state = r.pop("_state")
        if B == 1:
            roof = bench_decode_roofline(model, state)
        decode[f"B{B}"] = r
        log(f"decode B={B}: {r} ({time.perf_counter() - t0:.1f}s)")
    t_decode = time.perf_counter() - t_run0
    prefill = staging = deepseek = cpu = None
    if "prefill" not in skip:
        t0 = time.perf_counter()
        prefill = bench_prefill(host_w13, host_w2)
        log(f"prefill: {prefill} ({time.perf_counter() - t0:.1f}s)")
    if "staging" not in skip:
        t0 = time.perf_counter()
        staging = bench_staging(model, steps=args.stage_steps)
        log(f"staging: {staging} ({time.perf_counter() - t0:.1f}s)")
    del model
    torch.cuda.empty_cache()
    if "deepseek" not in skip:
        t0 = time.perf_counter()
        deepseek = bench_deepseek()
        log(f"deepseek: {deepseek} ({time.perf_counter() - t0:.1f}s)")
    if "cpu" not in skip:
        cpu = bench_cpu_baseline()
        log(f"cpu baseline: {cpu}")

    b1 = decode.get("B1", {})
    value = b1.get("us_per_token_per_layer")
    steps_ms = b1.get("graph_ms_per_step_mean")
    line = {
        "metric": "MoE-layer us/token decode (HBM GB/s %peak); prefill TFLOP/s; H2D GB/s",
        "value": value,
        "unit": "us/token/layer (decode, B=1, 48-layer hipGraph replay)",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": steps_ms,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (weights N(0,0.02) bf16, hidden N(0,1), Zipf(1.1) router bias from fixed seeds)",
        "config": {"workload": "C2 Qwen3-30B-A3B-shaped decode: 48 MoE layers, hidden 2048, 128 experts, top-8, "
                               "intermediate 768, 64 slots/layer, pinned host store, hipGraph-captured step",
                   "layers": args.layers, "slots": args.slots, "batch": 1},
        "roofline": None,
        "cpu_baseline": cpu,
        "decode": decode,
        "prefill": prefill,
        "staging": staging,
        "deepseek_v3_style": deepseek,
    }
    if roof is not None:
        gu = roof["gateup_gemv_kernel"]
        line["roofline"] = {"bound": "hbm", "achieved": gu["achieved_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": round(gu["achieved_gbs"] / HBM_PEAK_GBS, 4), "traffic": None,
                            "kernel": "gateup_gemv_kernel (decode B=1)", "avg_launch_us": gu["avg_launch_us"],
                            "bytes_per_launch": gu["bytes_per_launch"],
                            "distinct_slots_per_launch": roof["distinct_slots_per_launch"],
                            "down_combine_gemv_kernel": roof["down_combine_gemv_kernel"]}
        if b1.get("layer_hbm_gbs"):
            # the headline's own fraction: the whole layer's algorithmic
            # bytes over its graph-replayed time (value)
            line["roofline"]["layer"] = {"bytes": b1.get("algorithmic_bytes_per_layer"),
                                         "us": b1.get("us_per_layer"), "achieved": b1["layer_hbm_gbs"],
                                         "frac": b1.get("layer_hbm_frac")}
        traffic_file = ROOT / "profiles" / "gateup_gemv_decode_b1_traffic.json"
        if traffic_file.exists():
            try:
                line["roofline"]["traffic"] = json.loads(traffic_file.read_text()).get("hbm_bytes_per_launch")
            except Exception:
                pass
    text = json.dumps(line)
    print(text, flush=True)
    if args.out:
        Path(args.out).write_text(text + "\n")
    log(f"decode phase {t_decode:.1f}s total")
    # return page-locked and device memory while the runtime is fully up: a
    # page-locked block left in torch's host cache would be freed by the
    # allocator's destructor in static teardown, after a profiler attached to
    # the runtime may have shut down
    del host_w13, host_w2
    before = dict(torch.cuda.host_memory_stats()) if hasattr(torch.cuda, "host_memory_stats") else {}
    after = native.release_device_resources()
    log("page-locked host cache: reserved "
        f"{before.get('reserved_bytes.current', before.get('segment.current', 'n/a'))} -> "
        f"{after.get('reserved_bytes.current', after.get('segment.current', 'n/a'))} "
        f"(keys {sorted(k for k in after if 'current' in k)[:6]})")
    return 0


if __name__ == "__main__":
    sys.exit(main())
