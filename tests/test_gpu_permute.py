"""GPU parity of lmoe_permute / lmoe_gather_rows against the oracle (bit-exact)."""

import numpy as np
import pytest
import torch

from oracle import permute as orc
from tests._util import from_dev_bf16, to_dev_bf16, to_dev_i32

pytestmark = pytest.mark.gpu


def _native():
    from vllm_moe_offload_amd import native

    return native


def _check(perm, ref, n_pairs):
    torch.cuda.synchronize()
    placed = ref.placed
    np.testing.assert_array_equal(perm.counts.cpu().numpy(), ref.counts)
    np.testing.assert_array_equal(perm.offsets.cpu().numpy(), ref.offsets)
    np.testing.assert_array_equal(perm.sorted_pairs.cpu().numpy()[:placed], ref.sorted_pairs)
    np.testing.assert_array_equal(perm.row_idx.cpu().numpy()[:n_pairs], ref.row_idx)
    na = ref.active.size
    np.testing.assert_array_equal(perm.active.cpu().numpy()[:na], ref.active)
    assert (perm.active.cpu().numpy()[na:] == -1).all()  # -1 past the active slots
    np.testing.assert_array_equal(perm.tile_off.cpu().numpy(), ref.tile_off)
    meta = perm.meta.cpu().numpy()
    assert meta[0] == na
    assert meta[1] == placed
    assert meta[2] == ref.errors
    assert meta[3] == ref.tile_off[-1]


@pytest.mark.parametrize("block_m", [128, 256, 320])
@pytest.mark.parametrize("T,k,E,P,use_map", [
    (1, 8, 128, 64, True),
    (8, 8, 128, 32, False),
    (16, 8, 128, 64, True),     # one wave, two pairs per lane
    (24, 8, 128, 64, True),     # one wave, four pairs per lane (partly filled)
    (32, 8, 1024, 1024, False), # one wave: 256 pairs, 16 slots per lane
    (40, 6, 8, 8, False),       # one wave, ~30 pairs per slot across the pair groups
    (64, 8, 128, 64, True),
    (128, 8, 128, 128, False),
    (129, 8, 128, 64, True),
    (4096, 8, 128, 48, True),
    (2048, 8, 256, 256, False),
    (5000, 8, 1024, 1024, False),  # 40 chunks x 1024 slots: scan over the table in global memory
    (3, 1, 5, 3, True),
])
def test_permute_matches_oracle(T, k, E, P, use_map, block_m):
    native = _native()
    print(f"case permute T={T} k={k} E={E} P={P} map={use_map} block_m={block_m}", flush=True)
    rng = np.random.default_rng(T * 31 + P)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    log2phy = None
    if use_map:
        log2phy = np.full(E, -1, dtype=np.int32)
        chosen = rng.permutation(E)[: min(P, E)]
        log2phy[chosen] = rng.permutation(P)[: chosen.size]
    perm = native.Permutation.allocate(T * k, P, "cuda")
    native.permute(to_dev_i32(ids), perm, log2phy=None if log2phy is None else to_dev_i32(log2phy),
                   block_m=block_m)
    _check(perm, orc.init_routing(ids, P, log2phy=log2phy, block_m=block_m), T * k)


@pytest.mark.parametrize("N,P,s", [
    (128, 128, 1.2),    # one wave
    (256, 1024, 1.5),   # one wave, 16 slots per lane
    (512, 128, 1.1),    # one block
    (1024, 256, 1.3),   # one block, full chunk
    (8192, 64, 1.3),    # multi-block
    (16000, 1024, 1.0), # multi-block, scan over the table in global memory
])
def test_permute_heavy_first_order_matches_oracle(N, P, s):
    """Zipf-skewed slots (plus a run of equal heavy counts): the active list
    leads with the heavy slots, ties by slot, as the oracle orders them."""
    native = _native()
    print(f"case permute heavy-first N={N} P={P} s={s}", flush=True)
    rng = np.random.default_rng(N + P)
    pz = 1.0 / (rng.permutation(P) + 1.0) ** s
    ids = rng.choice(P, size=N, p=pz / pz.sum()).astype(np.int32)
    # four slots with the same heavy count: equal counts are ordered by slot
    tie = max(8, N // 12)
    ids[: 4 * tie] = np.repeat(rng.permutation(P)[:4], tie)
    ids = ids.reshape(-1, 1)
    for block_m in (128, 320):
        perm = native.Permutation.allocate(N, P, "cuda")
        native.permute(to_dev_i32(ids), perm, block_m=block_m)
        ref = orc.init_routing(ids, P, block_m=block_m)
        assert ((ref.counts >= orc.HEAVY_MIN_PAIRS) & (16 * ref.counts >= ref.placed)).sum() >= 2
        _check(perm, ref, N)


@pytest.mark.parametrize("N,P", [(64, 16), (200, 16), (5000, 40)])
def test_permute_skip_unmapped_wave_filter(N, P):
    native = _native()
    rng = np.random.default_rng(N)
    E = 2 * P
    ids = rng.integers(0, E, size=N).astype(np.int32)
    log2phy = np.full(E, -1, dtype=np.int32)
    wave = rng.permutation(E)[:P]
    log2phy[np.sort(wave)] = np.arange(P, dtype=np.int32)
    perm = native.Permutation.allocate(N, P, "cuda")
    native.permute(to_dev_i32(ids), perm, log2phy=to_dev_i32(log2phy), skip_unmapped=True)
    ref = orc.init_routing(ids, P, log2phy=log2phy, skip_unmapped=True, block_m=native.MFMA_BLOCK_M)
    assert ref.errors == 0
    _check(perm, ref, N)


def test_permute_counts_invalid_ids_as_errors():
    native = _native()
    ids = np.array([[0, 1], [2, 9], [-3, 1]], dtype=np.int32)
    log2phy = np.array([0, 1, -1, 2], dtype=np.int32)
    perm = native.Permutation.allocate(6, 3, "cuda")
    native.permute(to_dev_i32(ids), perm, log2phy=to_dev_i32(log2phy))
    ref = orc.init_routing(ids, 3, log2phy=log2phy, block_m=native.MFMA_BLOCK_M)
    assert ref.errors == 3  # expert 2 unstaged, id 9 and id -3 out of range
    _check(perm, ref, 6)


def test_gather_rows_is_expanded_x():
    native = _native()
    rng = np.random.default_rng(3)
    T, k, E, H = 24, 4, 16, 256
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    x = rng.integers(0, 1 << 15, size=(T, H)).astype(np.uint16)
    perm = native.Permutation.allocate(T * k, E, "cuda")
    native.permute(to_dev_i32(ids), perm)
    out = native.gather_rows(to_dev_bf16(x), k, perm)
    ref = orc.init_routing(ids, E, block_m=native.MFMA_BLOCK_M)
    np.testing.assert_array_equal(from_dev_bf16(out), orc.expanded_x(x, ref, k))


def test_permute_is_stable_across_repeated_launches():
    native = _native()
    rng = np.random.default_rng(11)
    ids = rng.integers(0, 64, size=(4096, 8)).astype(np.int32)
    perm = native.Permutation.allocate(ids.size, 64, "cuda")
    d = to_dev_i32(ids)
    native.permute(d, perm)
    first = perm.sorted_pairs.clone()
    for _ in range(3):
        native.permute(d, perm)
    torch.cuda.synchronize()
    assert torch.equal(first, perm.sorted_pairs)


@pytest.mark.parametrize("n_table,n", [(128, 1), (128, 9), (300, 150)])  # 150: three launches of 64
def test_table_update_writes_exactly_the_pairs(n_table, n):
    """lmoe_table_update (the staging path's log2phy write) against numpy."""
    from vllm_moe_offload_amd import native

    print(f"case table-update n_table={n_table} n={n}", flush=True)
    rng = np.random.default_rng(n_table + n)
    init = rng.integers(-1, 64, n_table).astype(np.int32)
    table = torch.from_numpy(init.copy()).cuda()
    idx = rng.permutation(n_table)[:n].astype(np.int32)
    val = rng.integers(-1, 64, n).astype(np.int32)
    native.table_update_entries(table, idx.tolist(), val.tolist())
    torch.cuda.synchronize()
    ref = init.copy()
    ref[idx] = val
    np.testing.assert_array_equal(table.cpu().numpy(), ref)


def _perm_arrays(perm, n):
    torch.cuda.synchronize()
    return {name: getattr(perm, name).cpu().numpy()[: (n if name in ("sorted_pairs", "row_idx") else None)]
            for name in ("counts", "offsets", "sorted_pairs", "row_idx", "active", "tile_off")} | \
        {"meta": perm.meta.cpu().numpy()[:4]}


@pytest.mark.parametrize("N,Pa,Pb,E,overlap,bad", [
    (128, 64, 64, 128, False, False),    # one wave per table
    (512, 64, 64, 128, False, False),    # the B=64 decode build: one workgroup per table
    (1024, 64, 300, 600, False, True),   # the largest one-launch build, ids outside both tables
    (200, 40, 1500, 3000, False, False),  # a table past the wave form: workgroups
    (256, 64, 64, 100, True, False),     # overlapping tables: the later build's rows win
    (0, 8, 8, 16, False, False),         # empty batch
])
def test_permute_two_tables_equals_two_builds(N, Pa, Pb, E, overlap, bad):
    """lmoe_permute_two_tables (bank table in skip mode 1, overflow table in
    skip mode 2, one launch) writes every output as lmoe_permute(a, 1) then
    lmoe_permute(b, 2) on the same row_idx, and both match the oracle."""
    native = _native()
    rng = np.random.default_rng(N + Pb)
    ids = rng.integers(0, E, size=N).astype(np.int32)
    if bad and N:  # ids past the tables: skipped silently by both builds
        ids[rng.integers(0, N, size=7)] = E + 5
        ids[3] = -2
    experts = rng.permutation(E)
    la = np.full(E, -1, dtype=np.int32)
    lb = np.full(E, -1, dtype=np.int32)
    na = min(Pa, E // 2)
    la[experts[:na]] = rng.permutation(Pa)[:na]
    if overlap:
        lb[experts[:Pb]] = rng.permutation(Pb)[: min(Pb, E)]
    else:
        nb = min(Pb, E - na - 3)
        lb[experts[na:na + nb]] = rng.permutation(Pb)[:nb]
        if bad:  # entries that are no slot of their table: errors of each build
            la[experts[-1]] = Pa + 5
            lb[experts[-2]] = -7
            ids[5], ids[6] = experts[-1], experts[-2]
    print(f"case two tables N={N} Pa={Pa} Pb={Pb} overlap={overlap} bad={bad}", flush=True)
    d_ids, d_la, d_lb = to_dev_i32(ids.reshape(-1, 1) if N else ids), to_dev_i32(la), to_dev_i32(lb)
    seq_a, seq_b = native.Permutation.allocate(N, Pa, "cuda"), native.Permutation.allocate(N, Pb, "cuda")
    one_a, one_b = native.Permutation.allocate(N, Pa, "cuda"), native.Permutation.allocate(N, Pb, "cuda")
    for p in (seq_a, seq_b, one_a, one_b):  # stale contents the builds must overwrite
        for t in (p.counts, p.offsets, p.sorted_pairs, p.row_idx, p.active, p.tile_off):
            t.fill_(7)
    native.permute(d_ids, seq_a, log2phy=d_la, skip_unmapped=True)
    native.permute(d_ids, seq_b, log2phy=d_lb, keep_rows=True, row_idx=seq_a.row_idx)
    lib = native.load_library()
    st = lib.lmoe_permute_two_tables(
        native._ptr(d_ids), N, native.MFMA_BLOCK_M, native._ptr(one_a.row_idx),
        native._ptr(d_la), E, Pa, native._ptr(one_a.counts), native._ptr(one_a.offsets),
        native._ptr(one_a.sorted_pairs), native._ptr(one_a.active), native._ptr(one_a.tile_off),
        native._ptr(one_a.meta), native._ptr(d_lb), E, Pb, native._ptr(one_b.counts), native._ptr(one_b.offsets),
        native._ptr(one_b.sorted_pairs), native._ptr(one_b.active), native._ptr(one_b.tile_off),
        native._ptr(one_b.meta), None)
    assert st == 0
    got_a, got_b = _perm_arrays(one_a, N), _perm_arrays(one_b, N)
    want_a, want_b = _perm_arrays(seq_a, N), _perm_arrays(seq_b, N)
    for name in got_a:
        if name == "sorted_pairs":  # positions past the placed pairs are not written
            pa, pb = int(want_a["meta"][1]), int(want_b["meta"][1])
            np.testing.assert_array_equal(got_a[name][:pa], want_a[name][:pa])
            np.testing.assert_array_equal(got_b[name][:pb], want_b[name][:pb])
            continue
        np.testing.assert_array_equal(got_a[name], want_a[name], err_msg=name)
        if name != "row_idx":  # the second build's row_idx lives in the first's buffer
            np.testing.assert_array_equal(got_b[name], want_b[name], err_msg=name)
    # the oracle: each table's build, row_idx from the later build where it places
    ra = orc.init_routing(ids, Pa, log2phy=la, skip_unmapped=True, block_m=native.MFMA_BLOCK_M)
    rb = orc.init_routing(ids, Pb, log2phy=lb, skip_unmapped=True, block_m=native.MFMA_BLOCK_M)
    np.testing.assert_array_equal(got_a["counts"], ra.counts)
    np.testing.assert_array_equal(got_b["counts"], rb.counts)
    np.testing.assert_array_equal(got_a["sorted_pairs"][: ra.placed], ra.sorted_pairs)
    np.testing.assert_array_equal(got_b["sorted_pairs"][: rb.placed], rb.sorted_pairs)
    np.testing.assert_array_equal(got_a["active"][: ra.active.size], ra.active)
    np.testing.assert_array_equal(got_b["active"][: rb.active.size], rb.active)
    rows = np.where(rb.row_idx >= 0, rb.row_idx, ra.row_idx)
    np.testing.assert_array_equal(got_a["row_idx"], rows)
    assert got_a["meta"][2] == ra.errors and got_b["meta"][2] == rb.errors
    if bad and N:
        assert ra.errors > 0 and rb.errors > 0
    if overlap:
        assert ((ra.row_idx >= 0) & (rb.row_idx >= 0)).any()


def test_permute_two_tables_refuses_builds_past_one_workgroup():
    """More than 1024 pairs: LMOE_ERR_SHAPE before any launch (the wrapper
    then runs the two builds one after the other)."""
    native = _native()
    lib = native.load_library()
    z = torch.zeros(4096, dtype=torch.int32, device="cuda")
    p = z.data_ptr()
    st = lib.lmoe_permute_two_tables(p, 1025, 256, p, p, 8, 8, p, p, p, p, p, p, p, 8, 8, p, p, p, p, p, p, None)
    assert st == native.LMOE_ERR_SHAPE
    st = lib.lmoe_permute_two_tables(p, 16, 256, p, None, 8, 8, p, p, p, p, p, p, p, 8, 8, p, p, p, p, p, p, None)
    assert st == native.LMOE_ERR_ARG
    # the wrapper's fallback: the two builds
    N, P = 2048, 16
    rng = np.random.default_rng(5)
    ids = to_dev_i32(rng.integers(0, 32, size=N).astype(np.int32))
    la = np.full(32, -1, dtype=np.int32)
    lb = np.full(32, -1, dtype=np.int32)
    la[:16], lb[16:] = np.arange(16), np.arange(16)
    a, b = native.Permutation.allocate(N, P, "cuda"), native.Permutation.allocate(N, P, "cuda")
    native.permute_two_tables(ids, a, to_dev_i32(la), b, to_dev_i32(lb))
    torch.cuda.synchronize()
    assert int(a.meta[1]) + int(b.meta[1]) == N and (a.row_idx >= 0).all()
