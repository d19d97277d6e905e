"""Pins the CPU oracle against things other than itself: the reference's
golden vectors, closed forms, brute force on tiny inputs and independent
library routines.  CPU only."""

import itertools
import math

import numpy as np
import pytest
import torch

from oracle import mlp as omlp
from oracle import permute as operm
from oracle import router as orouter
from oracle.bf16 import bf16_to_f32, f32_to_bf16, round_bf16


# ---------------------------------------------------------------- bf16
def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * 10,
        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.4e38, -3.4e38, 1e-40, np.inf, -np.inf], dtype=np.float32),
        # exact ties between two bf16 values (round half to even)
        (bf16_to_f32(np.arange(0x3F80, 0x3FA0, dtype=np.uint16)).view(np.uint32) + 0x8000).view(np.float32),
    ])
    ours = f32_to_bf16(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)


# ---------------------------------------------------------------- router
def test_exp_nonpos_within_two_ulp_of_float64():
    x = np.concatenate([np.linspace(-86.0, 0.0, 200001, dtype=np.float32),
                        -np.abs(np.random.default_rng(1).standard_normal(100000)).astype(np.float32)])
    got = orouter.exp_nonpos(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(got - ref) / ulp) <= 2.0
    assert orouter.exp_nonpos(np.array([0.0], np.float32))[0] == 1.0
    assert orouter.exp_nonpos(np.array([-87.0, -1000.0, -np.inf], np.float32)).tolist() == [0.0, 0.0, 0.0]


def test_sigmoid_against_float64():
    x = np.linspace(-30, 30, 100001, dtype=np.float32)
    got = orouter.sigmoid(x).astype(np.float64)
    ref = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    assert np.max(np.abs(got - ref) / np.spacing(ref.astype(np.float32))) <= 3.0


def test_softmax_probs_against_float64():
    rng = np.random.default_rng(2)
    lg = rng.standard_normal((64, 128)).astype(np.float32) * 3
    p = orouter.softmax_probs(lg).astype(np.float64)
    z = lg.astype(np.float64)
    ref = np.exp(z - z.max(1, keepdims=True))
    ref /= ref.sum(1, keepdims=True)
    # x - max rounds in f32: relative error grows like |x| * 2^-24
    assert np.max(np.abs(p - ref) / ref) < 2e-6
    np.testing.assert_allclose(p.sum(1), 1.0, rtol=1e-6)


def _brute_topk(score, k, eligible=None):
    idx = [i for i in range(len(score)) if eligible is None or eligible[i]]
    # selection sort with explicit (value desc, id asc) rule
    out = []
    for _ in range(k):
        best = None
        for i in idx:
            if i in out:
                continue
            if best is None or score[i] > score[best] or (score[i] == score[best] and i < best):
                best = i
        out.append(best)
    return out


def test_softmax_topk_selection_brute_force_with_ties():
    rng = np.random.default_rng(3)
    for _ in range(200):
        E = int(rng.integers(4, 20))
        k = int(rng.integers(1, E + 1))
        lg = (rng.integers(-3, 4, size=(1, E)) * 0.5).astype(np.float32)  # many ties
        ids, w, wb = orouter.softmax_topk(lg, k)
        p = orouter.softmax_probs(lg)[0]
        assert ids[0].tolist() == _brute_topk(p.tolist(), k)
        assert len(set(ids[0].tolist())) == k
        np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-6)


def test_softmax_correction_bias_selects_only_and_logit_bias_shifts_logits():
    """The correction bias moves the choice, never the weights; the logit bias
    is the same as adding it to the logits first."""
    rng = np.random.default_rng(31)
    for _ in range(200):
        E = int(rng.integers(4, 20))
        k = int(rng.integers(1, E + 1))
        lg = (rng.integers(-3, 4, size=(1, E)) * 0.5).astype(np.float32)
        bias = (rng.integers(-2, 3, size=E) * 0.125).astype(np.float32)
        ids, w, _ = orouter.softmax_topk(lg, k, bias=bias, renorm=False)
        p = orouter.softmax_probs(lg)[0]
        sel = (p + bias).astype(np.float32)
        want = _brute_topk(sel.tolist(), k)
        assert ids[0].tolist() == want
        np.testing.assert_array_equal(w[0], p[want])  # unbiased probabilities
        ids2, w2, _ = orouter.softmax_topk(lg, k, logit_bias=bias)
        ids3, w3, _ = orouter.softmax_topk((lg + bias).astype(np.float32), k)
        np.testing.assert_array_equal(ids2, ids3)
        np.testing.assert_array_equal(w2, w3)
    # a large bias on one expert selects it although its probability is low
    lg = np.array([[2.0, 1.0, 0.0, -1.0]], np.float32)
    ids, w, _ = orouter.softmax_topk(lg, 2, bias=np.array([0, 0, 0, 5.0], np.float32), renorm=False)
    p = orouter.softmax_probs(lg)[0]
    assert ids[0].tolist() == [3, 0]
    assert w[0].tolist() == [p[3], p[0]]


def test_renorm_golden_vector_of_reference():
    """weights [1, 3] -> [0.25, 0.75] (reference tests/test_patch_fused_moe.py:560)."""
    w, wb = orouter._finish(np.array([[1.0, 3.0]], np.float32), True, 1.0)
    assert w.tolist() == [[0.25, 0.75]]
    assert bf16_to_f32(wb).tolist() == [[0.25, 0.75]]
    # clamp_min(eps): an all-zero row stays zero instead of NaN
    w0, _ = orouter._finish(np.array([[0.0, 0.0]], np.float32), True, 1.0)
    assert w0.tolist() == [[0.0, 0.0]]


def test_grouped_sigmoid_brute_force():
    rng = np.random.default_rng(4)
    for _ in range(100):
        G = int(rng.choice([2, 4]))
        gs = int(rng.choice([2, 3, 4]))
        E = G * gs
        TG = int(rng.integers(1, G + 1))
        k = int(rng.integers(1, TG * gs + 1))
        lg = (rng.integers(-4, 5, size=(1, E)) * 0.25).astype(np.float32)
        bias = (rng.integers(-2, 3, size=E) * 0.125).astype(np.float32)
        ids, w, _ = orouter.grouped_sigmoid_topk(lg, k, bias=bias, n_group=G, topk_group=TG, scale=2.5)
        s = orouter.sigmoid(lg)[0]
        sb = (s + bias).astype(np.float32)
        gscore = []
        for g in range(G):
            vals = sorted(sb[g * gs:(g + 1) * gs].tolist(), reverse=True)
            gscore.append(np.float32(vals[0]) + np.float32(vals[1]))
        kept = _brute_topk(gscore, TG)
        elig = [(e // gs) in kept for e in range(E)]
        want = _brute_topk(sb.tolist(), k, elig)
        assert ids[0].tolist() == want
        ref_w = s[want] / max(float(np.float32(sum(np.float32(v) for v in s[want]))), np.finfo(np.float32).eps) * 2.5
        np.testing.assert_allclose(w[0], ref_w, rtol=1e-6)


def test_gate_logits_exact_on_integer_scaled_inputs():
    rng = np.random.default_rng(5)
    xi = rng.integers(-8, 9, size=(3, 64))
    wi = rng.integers(-8, 9, size=(5, 64))
    x = f32_to_bf16(xi.astype(np.float32) / 8)
    w = f32_to_bf16(wi.astype(np.float32) / 16)
    got = orouter.gate_logits(x, w, out_f32=True)
    np.testing.assert_array_equal(got, (xi @ wi.T).astype(np.float32) / 128)


# ---------------------------------------------------------------- permute
def test_histogram_golden_vector_of_reference():
    """reference tests/test_phase_split_b2.py:25-41."""
    ids = np.array([[1, 3], [3, 4], [1, 4], [7, 3]])
    assert operm.count_routed_tokens_by_expert(ids) == {1: 2, 3: 3, 4: 2, 7: 1}
    p = operm.init_routing(ids, 8)
    assert p.counts.tolist() == [0, 2, 0, 3, 2, 0, 0, 1]


def test_wave_filter_golden_vector_of_reference():
    """reference tests/test_phase_split_b2.py:325-365: wave (3, 4), log2phy
    3->0, 4->2: pairs in flat order tokens [0,1,1,2,3], logical [3,3,4,4,3],
    slots [0,0,2,2,0]."""
    ids = np.array([[1, 3], [3, 4], [1, 4], [7, 3]])
    l2p = np.full(8, -1)
    l2p[3], l2p[4] = 0, 2
    p = operm.init_routing(ids, 3, log2phy=l2p, skip_unmapped=True)
    flat_pairs = np.sort(p.sorted_pairs)
    assert (flat_pairs // 2).tolist() == [0, 1, 1, 2, 3]
    assert ids.reshape(-1)[flat_pairs].tolist() == [3, 3, 4, 4, 3]
    assert p.slot_of[flat_pairs].tolist() == [0, 0, 2, 2, 0]
    assert p.errors == 0


def _check_launch_order(active, counts):
    """Every listed pair of slots is in launch order, by a pairwise
    comparator: heavy (>= 16 pairs and >= 1/16 of all) before light, heavy by
    descending count then slot, light by slot."""
    total = sum(counts)

    def heavy(s):
        return counts[s] >= 16 and 16 * counts[s] >= total

    for i in range(len(active)):
        for j in range(i + 1, len(active)):
            a, b = active[i], active[j]
            if heavy(a) != heavy(b):
                assert heavy(a), (active, counts)
            elif heavy(a):
                assert counts[a] > counts[b] or (counts[a] == counts[b] and a < b), (active, counts)
            else:
                assert a < b, (active, counts)


def test_active_launch_order_hand_vectors():
    # 84 pairs: the 1/16 bound is 5.25, so count >= 16 decides
    ids = np.repeat(np.arange(7), [0, 17, 3, 20, 17, 15, 12]).reshape(-1, 1)
    assert operm.init_routing(ids, 7).active.tolist() == [3, 1, 4, 2, 5, 6]
    # 400 pairs: 20 pairs are under 1/16 of them, 80 and 300 are not
    ids = np.repeat(np.arange(3), [20, 300, 80]).reshape(-1, 1)
    assert operm.init_routing(ids, 3).active.tolist() == [1, 2, 0]
    # 200 pairs: 8 pairs are under the 16-pair bound, 42 and 150 are not
    ids = np.repeat(np.arange(3), [8, 150, 42]).reshape(-1, 1)
    assert operm.init_routing(ids, 3).active.tolist() == [1, 2, 0]
    # one token, distinct slots: slot order (the one-token kernels use rank = position)
    assert operm.init_routing(np.array([[5, 1, 7, 2]]), 8).active.tolist() == [1, 2, 5, 7]


def test_active_launch_order_skewed_counts():
    rng = np.random.default_rng(11)
    for _ in range(200):
        P = int(rng.integers(1, 200))
        n = int(rng.integers(0, 600))
        pz = 1.0 / np.arange(1, P + 1) ** rng.uniform(0.0, 2.0)
        ids = rng.choice(P, size=n, p=pz / pz.sum()).reshape(-1, 1)
        p = operm.init_routing(ids, P)
        assert sorted(p.active.tolist()) == [s for s in range(P) if p.counts[s] > 0]
        assert sum(1 for s in range(P) if p.counts[s] >= 16 and 16 * p.counts[s] >= n) <= 16
        _check_launch_order(p.active.tolist(), p.counts.tolist())


def test_init_routing_brute_force_and_invariants():
    rng = np.random.default_rng(6)
    for _ in range(300):
        T, k, P = int(rng.integers(1, 9)), int(rng.integers(1, 4)), int(rng.integers(1, 7))
        ids = rng.integers(-1, P + 1, size=(T, k))
        p = operm.init_routing(ids, P)
        flat = ids.reshape(-1)
        # brute force: insertion order by (slot, flat index)
        want = [i for s in range(P) for i in range(flat.size) if flat[i] == s]
        assert p.sorted_pairs.tolist() == want
        assert p.errors == int(np.sum((flat < 0) | (flat >= P)))
        for i in range(flat.size):
            if 0 <= flat[i] < P:
                assert p.sorted_pairs[p.row_idx[i]] == i
            else:
                assert p.row_idx[i] == -1
        assert p.offsets[-1] == len(want)
        assert sorted(p.active.tolist()) == [s for s in range(P) if p.counts[s] > 0]
        _check_launch_order(p.active.tolist(), p.counts.tolist())
        tiles = [math.ceil(c / 2) for c in p.counts]
        q = operm.init_routing(ids, P, block_m=2)
        assert q.tile_off.tolist() == [0] + list(itertools.accumulate(tiles))


# ---------------------------------------------------------------- mlp / combine
def test_expert_mlp_against_float64_triple_loop():
    rng = np.random.default_rng(7)
    n, H, I = 3, 16, 8
    x = round_bf16(rng.standard_normal((n, H)).astype(np.float32))
    w13 = round_bf16((rng.standard_normal((2 * I, H)) * 0.3).astype(np.float32))
    w2 = round_bf16((rng.standard_normal((H, I)) * 0.3).astype(np.float32))
    got = omlp.expert_mlp(x, w13, w2)
    ref = np.zeros((n, H))
    for r in range(n):
        g = [sum(float(x[r, h]) * float(w13[i, h]) for h in range(H)) for i in range(I)]
        u = [sum(float(x[r, h]) * float(w13[I + i, h]) for h in range(H)) for i in range(I)]
        a = [gi / (1 + math.exp(-gi)) * ui for gi, ui in zip(g, u)]
        for h in range(H):
            ref[r, h] = sum(a[i] * float(w2[h, i]) for i in range(I))
    # three bf16 rounding points: relative error a few bf16 ulps
    assert np.max(np.abs(got - ref)) <= 4 * 2 ** -8 * np.max(np.abs(ref)) + 1e-6


def test_combine_golden_vectors_of_reference():
    """weighted gather+scatter vectors of tests/test_phase_split_b2.py:923-1016
    ([[3.4, 34], [5.1, 51], [0.5, 5]]) restated as flat-pair combines."""
    # payload 1: unpermute [2,0,1] gathers [5,50], [3,30], [1,10] with weights
    # .5, .7, .9 for tokens 0, 1, 0; payload 2: unpermute [1,0] gathers
    # [2,20], [4,40] with weights .25, .75 for tokens 2, 1
    pairs = {0: [([5.0, 50.0], 0.5), ([1.0, 10.0], 0.9)],
             1: [([3.0, 30.0], 0.7), ([4.0, 40.0], 0.75)],
             2: [([2.0, 20.0], 0.25)]}
    T, k = 3, 2
    y = np.zeros((T * k, 2), np.float32)
    w = np.zeros((T, k), np.float32)
    for t, lst in pairs.items():
        for j, (row, wt) in enumerate(lst):
            y[t * k + j] = row
            w[t, j] = wt
    # weights are exact in f32 but not in bf16: use the f32 arithmetic of the
    # combine with weights already bf16-representable
    wb = f32_to_bf16(w)
    out = omlp.combine(y, wb, round_output=False)
    ref = np.array([[3.4, 34.0], [5.1, 51.0], [0.5, 5.0]], np.float32)
    np.testing.assert_allclose(out, ref, rtol=5e-3)
    assert omlp.combine(np.array([[1.0], [1e8], [-1e8]], np.float32)[[1, 2, 0]], f32_to_bf16(np.ones((1, 3), np.float32)),
                        round_output=False)[0, 0] == 1.0


def test_wave_split_invariance_of_oracle():
    rng = np.random.default_rng(8)
    T, k, E, H, I = 6, 3, 9, 16, 8
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    x = f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    w13 = f32_to_bf16((rng.standard_normal((E, 2 * I, H)) * 0.3).astype(np.float32))
    w2 = f32_to_bf16((rng.standard_normal((E, H, I)) * 0.3).astype(np.float32))
    wb = f32_to_bf16(rng.random((T, k)).astype(np.float32))
    single = omlp.combine(omlp.grouped_mlp(x, operm.remap(ids, None, E), k, w13, w2), wb)
    y = np.zeros((T * k, H), np.float32)
    for wave in (np.arange(0, 4), np.arange(4, 9)):
        l2p = np.full(E, -1)
        l2p[wave] = np.arange(wave.size)
        slot = operm.remap(ids, l2p, wave.size, skip_unmapped=True)
        part = omlp.grouped_mlp(x, slot, k, w13[wave], w2[wave])
        y[slot >= 0] = part[slot >= 0]
    np.testing.assert_array_equal(omlp.combine(y, wb), single)
