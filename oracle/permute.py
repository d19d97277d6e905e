"""Permutation oracle (test infrastructure only).

Restates the token->slot remap and the init-routing sort:
  * remap: slot = log2phy[id] (moe_offload/slot_mapping.py:116-140);
  * init routing (npu_moe_init_routing_v2 as called at
    patches/patch_fused_moe.py:668-701 with expert_capacity=-1,
    drop_pad_mode=0, expert_tokens_num_type=1): stable sort of the flat
    (token, k) pairs by slot, expanded_row_idx[p] = sorted position of pair p,
    expanded_x[pos] = x[pair // k], count histogram per slot;
  * wave membership: a pair whose slot is -1 belongs to another wave and is
    left out (the per-wave expert table of
    phase_split.build_b2_device_wave_microbatch_plans, :1224-1384).

Pinning (tests/test_oracle_core.py): the reference golden histogram
{1: 2, 3: 3, 4: 2, 7: 1} (tests/test_phase_split_b2.py:25-41); the pair
microbatch vectors of tests/test_phase_split_b2.py:325-365 (restore tokens
[0, 1, 1, 2, 3], logical [3, 3, 4, 4, 3], slots [0, 0, 2, 2, 0]); a
brute-force insertion sort over random small inputs; invariants
(sorted_pairs is a permutation, row_idx its inverse, slots non-decreasing,
flat order kept inside each slot).

The active-slot list is this build's own launch order (the reference has
no such list): a heavy slot (count >= 16 and 16 * count >= placed pairs)
first, by descending count then ascending slot, then every other slot
with count > 0 in ascending slot order.  Pinned by a brute-force pairwise
check over random skewed counts (tests/test_oracle_core.py).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class OraclePermutation:
    slot_of: np.ndarray       # [N] slot per flat pair, -1 skipped, -2 error
    counts: np.ndarray        # [P]
    offsets: np.ndarray       # [P+1]
    sorted_pairs: np.ndarray  # [placed]
    row_idx: np.ndarray       # [N] sorted position or -1
    active: np.ndarray        # [num_active] slots with count > 0, launch order (active_order)
    tile_off: np.ndarray      # [P+1]
    errors: int

    @property
    def placed(self) -> int:
        return int(self.offsets[-1])


def remap(ids: np.ndarray, log2phy: np.ndarray | None, n_slots: int, *, skip_unmapped: bool = False) -> np.ndarray:
    """Slot of every flat pair: >= 0 placed, -1 skipped (wave filter), -2 error."""
    flat = np.asarray(ids, dtype=np.int64).reshape(-1)
    if log2phy is None:
        s = flat.copy()
    else:
        table = np.asarray(log2phy, dtype=np.int64)
        ok = (flat >= 0) & (flat < table.size)
        outside = -1 if skip_unmapped else -(1 << 40)
        s = np.where(ok, table[np.clip(flat, 0, max(table.size - 1, 0))], outside)
    out = np.where((s >= 0) & (s < n_slots), s, -2)
    if skip_unmapped:
        out = np.where(s == -1, -1, out)
    return out.astype(np.int64)


HEAVY_MIN_PAIRS = 16


def active_order(counts: np.ndarray) -> np.ndarray:
    """Slots with count > 0 in launch order: heavy slots (count >= 16 and
    16 * count >= total) by descending count, ties ascending slot, then the
    rest in ascending slot order."""
    c = np.asarray(counts, dtype=np.int64)
    placed = int(c.sum())
    heavy = (c >= HEAVY_MIN_PAIRS) & (16 * c >= placed)
    hs = np.nonzero(heavy)[0]
    hs = hs[np.lexsort((hs, -c[hs]))]
    light = np.nonzero((c > 0) & ~heavy)[0]
    return np.concatenate([hs, light]).astype(np.int64)


def init_routing(
    ids: np.ndarray,
    n_slots: int,
    *,
    log2phy: np.ndarray | None = None,
    skip_unmapped: bool = False,
    block_m: int = 128,
) -> OraclePermutation:
    slot_of = remap(ids, log2phy, n_slots, skip_unmapped=skip_unmapped)
    N = slot_of.size
    placed_mask = slot_of >= 0
    counts = np.bincount(slot_of[placed_mask], minlength=n_slots).astype(np.int64)[:n_slots]
    offsets = np.zeros(n_slots + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(counts)
    order = np.nonzero(placed_mask)[0]
    order = order[np.argsort(slot_of[order], kind="stable")]
    row_idx = np.full(N, -1, dtype=np.int64)
    row_idx[order] = np.arange(order.size)
    tiles = (counts + block_m - 1) // block_m
    tile_off = np.zeros(n_slots + 1, dtype=np.int64)
    tile_off[1:] = np.cumsum(tiles)
    return OraclePermutation(
        slot_of=slot_of,
        counts=counts,
        offsets=offsets,
        sorted_pairs=order.astype(np.int64),
        row_idx=row_idx,
        active=active_order(counts),
        tile_off=tile_off,
        errors=int(np.count_nonzero(slot_of == -2)),
    )


def expanded_x(x: np.ndarray, perm: OraclePermutation, top_k: int) -> np.ndarray:
    return np.asarray(x)[perm.sorted_pairs // top_k]


def count_routed_tokens_by_expert(ids: np.ndarray) -> dict[int, int]:
    """Histogram of non-negative ids (phase_split.py:479-492)."""
    flat = np.asarray(ids).reshape(-1)
    flat = flat[flat >= 0]
    u, c = np.unique(flat, return_counts=True)
    return {int(a): int(b) for a, b in zip(u, c) if b > 0}
