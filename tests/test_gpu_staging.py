"""Staging under graph replay and the full-size
capacity-wave prefill (config C3), on the GPU.

C4: eight Qwen3-shaped layers (H 2048, I 768, one 128-expert page-locked host
store shared by the layers, 64 slots each), one token per step.  Every step
names, per layer, 8 - k experts already resident followed by exactly k that
are not (the reference stages in list order, so misses listed last never
evict a hit of the same step).  The per-layer pipeline of the decode loop:
complete layer l's prefetched copies, prefetch layer l + 1 (its copies wait
on the transfer stream for the compute that last read its bank), replay
layer l's captured graph, record the compute that reads layer l's bank.
Every layer's output at every step must equal, bit for bit, an eager pass
of the same kernels over a bank that holds all 128 experts; slot addresses
never move.  Mirrors reference transfer_engine.py:139-187 (event-ordered
batches), runtime.py:1636-1936 (hit/miss, LRU, consumer wait before
publish) and tests/test_prefill_stage_runtime.py:504-760 (stage buffer
reuse after release).

C3: 4096 tokens, 48 slots, a gate without bias (every expert touched), three
staged waves with one combine against the blocking full layer, bit for bit;
sampled pair rows of y against the oracle's expert MLP.
"""

import numpy as np
import pytest
import torch

from oracle import mlp as omlp
from oracle.bf16 import bf16_to_f32
from tests._util import from_dev_bf16, ulp_mismatch_stats

pytestmark = pytest.mark.gpu

H, I, E, K = 2048, 768, 128, 8


def _rand_bf16(g, shape, std):
    return (torch.randn(shape, generator=g, device="cuda") * std).to(torch.bfloat16)


@pytest.fixture(scope="module")
def qwen_experts():
    """All 128 Qwen3-shaped experts: device copies (the reference bank) and
    one page-locked host store."""
    g = torch.Generator(device="cuda").manual_seed(4242)
    w13 = _rand_bf16(g, (E, 2 * I, H), 0.02)
    w2 = _rand_bf16(g, (E, H, I), 0.02)
    h13 = torch.empty(w13.shape, dtype=torch.bfloat16, pin_memory=True)
    h2 = torch.empty(w2.shape, dtype=torch.bfloat16, pin_memory=True)
    h13.copy_(w13)
    h2.copy_(w2)
    torch.cuda.synchronize()
    return w13, w2, h13, h2


def test_c4_pipelined_staging_under_graph_replay_bit_exact(qwen_experts):
    from vllm_moe_offload_amd import fused_moe
    from vllm_moe_offload_amd.moe_offload.config import MoeOffloadConfig
    from vllm_moe_offload_amd.moe_offload.runtime import MoeOffloadRuntime

    full13, full2, h13, h2 = qwen_experts
    L, slots, B, steps = 8, 64, 1, 6
    dev = torch.device("cuda")
    rt = MoeOffloadRuntime(MoeOffloadConfig(enabled=True, num_slots=slots, async_load=True,
                                            graph_compatible_offload=True))
    for l in range(L):
        rt.register_host_buffers(layer_id=l, w13_host=h13, w2_host=h2, slot_device=dev)
    rng = np.random.default_rng(2026)
    # fill every bank with a random half of the experts (one batch per layer)
    for l in range(L):
        first = tuple(int(e) for e in rng.permutation(E)[:slots])
        rt.stage_fixed_slot_plan(layer_id=l, active_experts=first, num_logical_experts=E)
    torch.cuda.synchronize()

    g = torch.Generator(device="cuda").manual_seed(7)
    x = _rand_bf16(g, (B, H), 1.0)
    w_all = torch.rand((L, B, K), generator=g, device="cuda")
    w_all = (w_all / w_all.sum(-1, keepdim=True)).to(torch.bfloat16)
    ids_all = torch.zeros((L, B, K), dtype=torch.int32, device=dev)
    ids_host = torch.zeros((L, B, K), dtype=torch.int32, pin_memory=True)
    out_l = [torch.zeros((B, H), dtype=torch.bfloat16, device=dev) for _ in range(L)]
    P = rt.slot_bank(0).physical_expert_count
    ws = fused_moe.get_workspace(B, K, P, H, I, dev, tag="test-c4")
    ws_ref = fused_moe.get_workspace(B, K, E, H, I, dev, tag="test-c4-ref")

    def resident(l):
        return [s.expert_key.expert_id for s in rt.slot_bank(l).slots if s.expert_key is not None]

    for l in range(L):
        ids_all[l, 0].copy_(torch.tensor(resident(l)[:K], dtype=torch.int32))
    graphs = []
    for l in range(L):
        bank = rt.slot_bank(l)

        def piece(l=l, bank=bank):
            fused_moe.fused_experts(x, w_all[l], ids_all[l], bank.w13_slots, bank.w2_slots, rt.log2phy_buffer(l),
                                    out=out_l[l], workspace=ws)

        piece()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            piece()
        graphs.append(gr)
    fp = [rt._slot_address_fingerprint(l) for l in range(L)]

    for k in (1, 4, 8):
        for step in range(steps):
            print(f"case c4 k={k} step={step}", flush=True)
            plan = []
            for l in range(L):
                res = resident(l)
                non = sorted(set(range(E)) - set(res))
                miss = [int(e) for e in rng.choice(non, size=k, replace=False)]
                hit = [int(e) for e in rng.choice(res, size=K - k, replace=False)] if K > k else []
                plan.append(tuple(hit + miss))
            ids_host.copy_(torch.tensor(plan, dtype=torch.int32).view(L, B, K))
            ids_all.copy_(ids_host, non_blocking=True)
            pending = rt.prefetch_fixed_slot_plan(layer_id=0, active_experts=plan[0], num_logical_experts=E)
            for l in range(L):
                assert len(pending.misses) == k and tuple(pending.misses) == plan[l][K - k:], (k, step, l)
                rt.complete_fixed_slot_plan(pending)
                nxt = None
                if l + 1 < L:
                    nxt = rt.prefetch_fixed_slot_plan(layer_id=l + 1, active_experts=plan[l + 1],
                                                      num_logical_experts=E)
                graphs[l].replay()
                rt.record_layer_compute(l)
                pending = nxt
            torch.cuda.synchronize()
            assert fp == [rt._slot_address_fingerprint(l) for l in range(L)], "slot addresses moved"
            for l in range(L):
                ref = fused_moe.fused_experts(x, w_all[l], ids_all[l], full13, full2, None, workspace=ws_ref)
                torch.cuda.synchronize()
                same = torch.equal(ref.view(torch.int16), out_l[l].view(torch.int16))
                assert same, f"k={k} step={step} layer={l}: replayed output differs from the resident bank"
                # the table maps exactly this step's experts to slots that own them
                l2p = rt.log2phy_buffer(l).cpu().numpy()
                bank = rt.slot_bank(l)
                for e in plan[l]:
                    s = int(l2p[e])
                    assert s >= 0 and bank.slots[s].expert_key.expert_id == e


def test_c3_full_size_waves_equal_full_layer_bitwise(qwen_experts):
    """4096 tokens over 128 experts with 48 slots: three staged waves and one
    combine equal the blocking full layer bit for bit; y rows of sampled pairs
    are held to the oracle's expert MLP (two bf16 ulp with a cancellation
    floor, as the grouped-MLP parity tests)."""
    from vllm_moe_offload_amd import fused_moe
    from vllm_moe_offload_amd.fused_moe import RouterSpec
    from vllm_moe_offload_amd.moe_offload.config import MoeOffloadConfig
    from vllm_moe_offload_amd.moe_offload.runtime import MoeOffloadRuntime

    full13, full2, h13, h2 = qwen_experts
    T, slots = 4096, 48
    dev = torch.device("cuda")
    rt = MoeOffloadRuntime(MoeOffloadConfig(enabled=True, num_slots=slots, async_load=True,
                                            b2_wave_prefill=True))
    rt.register_host_buffers(layer_id=0, w13_host=h13, w2_host=h2, slot_device=dev)
    g = torch.Generator(device="cuda").manual_seed(33)
    x = _rand_bf16(g, (T, H), 1.0)
    gate = _rand_bf16(g, (E, H), 0.02)
    w, ids, _ = fused_moe.route(x, gate, RouterSpec(top_k=K))
    out_w, report = fused_moe.run_wave_prefill(rt, layer_id=0, hidden=x, topk_weights=w, topk_ids=ids,
                                               num_logical_experts=E)
    out_w = out_w.clone()
    y_w = fused_moe.get_workspace(T, K, slots, H, I, x.device, tag="waves").y.clone()
    out_f = fused_moe.run_full_layer(rt, layer_id=0, hidden=x, topk_weights=w, topk_ids=ids,
                                     num_logical_experts=E).clone()
    torch.cuda.synchronize()
    ids_np = ids.cpu().numpy()
    print(f"waves {len(report.waves)} sizes {[len(v) for v in report.waves]} h2d {report.h2d_bytes}", flush=True)
    assert np.unique(ids_np).size == E
    assert len(report.waves) == 3 and all(len(v) <= slots for v in report.waves)
    assert report.h2d_bytes > 0
    ndiff = int((out_w.view(torch.int16) != out_f.view(torch.int16)).sum().item())
    assert ndiff == 0, f"{ndiff} elements differ between the waves and the full layer"
    # sampled y rows against the oracle's expert MLP
    rng = np.random.default_rng(5)
    pairs = rng.choice(T * K, size=48, replace=False)
    x_np = bf16_to_f32(from_dev_bf16(x))
    got = bf16_to_f32(from_dev_bf16(y_w))[pairs]
    ref = np.empty_like(got)
    for i, p in enumerate(pairs):
        e = int(ids_np.reshape(-1)[p])
        ref[i] = omlp.expert_mlp(x_np[p // K][None, :], bf16_to_f32(from_dev_bf16(full13[e])),
                                 bf16_to_f32(from_dev_bf16(full2[e])))[0]
    rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
    frac, max_ulps = ulp_mismatch_stats(got, ref, abs_floor=rms / 256, count_floor=rms / 4096)
    print(f"  sampled y: frac>1ulp {frac:.2e} max {max_ulps:.2f} ulp", flush=True)
    assert frac <= 1e-3 and max_ulps <= 2.0


def test_stage_gather_copies_and_publishes_the_table():
    """lmoe_stage_gather: ranges from page-locked host memory and from device
    memory into device memory, more ranges than one launch holds, and the
    slot-table entries (pairs only, or the whole table with -1 elsewhere)
    written by the same batch; the ready event orders it all before the
    compute stream."""
    from vllm_moe_offload_amd import native

    g = torch.Generator(device="cuda").manual_seed(11)
    n_rows, row = 80, 48 * 1024  # 96 KiB rows
    src_dev = torch.randint(-30000, 30000, (n_rows, row), generator=g, device="cuda", dtype=torch.int16)
    src_host = torch.empty((n_rows, row), dtype=torch.int16, pin_memory=True)
    src_host.copy_(src_dev)
    dst = torch.zeros((n_rows, row), dtype=torch.int16, device="cuda")
    rng = np.random.default_rng(3)
    order = rng.permutation(n_rows)
    copies = []
    for i, r in enumerate(order[:70]):  # 70 ranges: three launches
        src = src_host if i % 3 else src_dev
        copies.append((int(dst[i].data_ptr()), int(src[int(r)].data_ptr()), row * 2))
    table = torch.full((300,), 7, dtype=torch.int32, device="cuda")
    idx = tuple(int(v) for v in rng.permutation(300)[:150])  # 150 pairs: two table launches
    val = tuple(range(150))
    stream = torch.cuda.Stream()
    done = torch.cuda.Event()
    assert native.stage_gather(copies, stream, table_update=(table, idx, val))
    done.record(stream)
    torch.cuda.current_stream().wait_event(done)
    want = torch.stack([src_dev[int(r)] for r in order[:70]])
    assert torch.equal(dst[:70], want)
    assert torch.equal(dst[70:], torch.zeros_like(dst[70:]))
    t = table.cpu().numpy()
    exp = np.full(300, 7, dtype=np.int32)
    exp[list(idx)] = val
    np.testing.assert_array_equal(t, exp)
    # fill: every entry not among the pairs becomes -1
    assert native.stage_gather(copies[:2], stream, table_update=(table, idx[:40], val[:40], True))
    torch.cuda.current_stream().wait_stream(stream)
    exp = np.full(300, -1, dtype=np.int32)
    exp[list(idx[:40])] = val[:40]
    np.testing.assert_array_equal(table.cpu().numpy(), exp)
    # misaligned ranges are refused before anything is queued
    assert not native.stage_gather([(int(dst[0].data_ptr()) + 8, int(src_dev[0].data_ptr()), 64)], stream)
    # torch reports pageable memory as not page-locked (the same runtime
    # query the library's range check makes), so the transfer engine sends
    # such sources to the copy engines
    assert not torch.empty(64, dtype=torch.int16).is_pinned() and src_host.is_pinned()


def test_transfer_engine_takes_copy_engines_for_pageable_sources():
    """Host rows that are not page-locked go through hipMemcpyAsync; the
    batch still lands and publishes."""
    from vllm_moe_offload_amd.moe_offload.expert_key import ExpertKey
    from vllm_moe_offload_amd.moe_offload.host_store import ExpertWeightBundle
    from vllm_moe_offload_amd.moe_offload.slot_bank import ExpertSlotBank, SlotState
    from vllm_moe_offload_amd.moe_offload.transfer_engine import TransferEngine

    bank = ExpertSlotBank(4, (64, 32), (32, 32), dtype=torch.bfloat16, device=torch.device("cuda"))
    host13 = torch.randn((3, 64, 32)).to(torch.bfloat16)   # pageable
    host2 = torch.randn((3, 32, 32)).to(torch.bfloat16)
    eng = TransferEngine()
    loads = []
    for e in range(3):
        slot = bank.allocate_for(ExpertKey(0, e), step_id=1)
        loads.append((ExpertWeightBundle(0, e, host13[e], host2[e]), slot))
    table = torch.full((3,), -1, dtype=torch.int32, device="cuda")
    ready = eng.load_many_async(loads, table_update=(table, (0, 1, 2), (0, 1, 2)))
    ready.install_consumer_dependency(torch.cuda.current_stream())
    assert eng.batches_gathered == 0
    assert all(s.state == SlotState.READY for _, s in loads)
    assert torch.equal(bank.w13_slots[:3].cpu(), host13) and torch.equal(bank.w2_slots[:3].cpu(), host2)
    assert table.tolist() == [0, 1, 2]
