// Permutation building blocks shared by the permutation kernels and the
// fused decode router: token->slot remap through log2phy, count histogram per
// physical slot, stable counting sort of the flat (token, k) pairs by slot,
// active-slot list and the MFMA tile table.
//
// Reference behaviour: ExpertSlotMapping.remap_topk_ids
// (moe_offload/slot_mapping.py:116-140, phys = log2phy[ids], fail closed on
// -1) feeding npu_moe_init_routing_v2 (patches/patch_fused_moe.py:668-701:
// stable sort by expert, expanded_row_idx, count-type histogram).  The wave
// filter (skip_unmapped) plays the role of the per-wave expert table of
// phase_split.build_b2_device_wave_microbatch_plans (:1224-1384).
//
// Integer work only; every output is bit-exact and independent of launch
// shape.  Pairs of one chunk (1024 pairs) are ranked with wave64 ballots.
#pragma once

#include "lmoe_device.h"

namespace lmoe {

constexpr int kChunk = 1024;       // pairs per block
constexpr int kMaxSlots = 8192;    // LDS histogram bound
// skip mode 2: as mode 1, and a pair this build leaves out keeps the row_idx
// an earlier pass of the same layer wrote, so that after the passes row_idx
// is >= 0 exactly for the pairs some pass placed (the combine's row mask)
constexpr int kSkipKeepRows = 2;

// slot of expert id `id`: >= 0 placed, -1 skipped silently, -2 error
__device__ __forceinline__ int map_id(int id, const int32_t* __restrict__ log2phy, int n_log2phy,
                                      int P, int skip) {
  int s;
  if (log2phy != nullptr) {
    // in wave mode an id the table does not cover belongs to another pass
    if (id < 0 || id >= n_log2phy) return skip ? -1 : -2;
    s = log2phy[id];
  } else {
    s = id;
  }
  if (s >= 0 && s < P) return s;
  if (skip && s == -1) return -1;
  return -2;
}

// slot of pair p, as map_id
__device__ __forceinline__ int map_pair(const int32_t* ids, int p,
                                        const int32_t* __restrict__ log2phy,
                                        int n_log2phy, int P, int skip) {
  return map_id(ids[p], log2phy, n_log2phy, P, skip);
}

// A later pass's table whose pairs keep the row_idx that pass writes: a
// build given one leaves those entries alone, so that two builds of one
// layer (the bank, then the overflow table in skip mode 2) can run at the
// same time and give the row_idx of the two run one after the other.  A null
// table (the default) keeps nothing.
struct RowKeep {
  const int32_t* log2phy = nullptr;
  int n_log2phy = 0;
  int P = 0;
};

__device__ __forceinline__ bool kept_row(const RowKeep& keep, const int32_t* ids, int p) {
  return keep.log2phy != nullptr && map_pair(ids, p, keep.log2phy, keep.n_log2phy, keep.P, 1) >= 0;
}

// Per-build state past the four counts: the build counter advances (the
// one thread that publishes meta).
__device__ __forceinline__ void publish_build(int32_t* meta) {
  // no-return atomic: the publishing thread does not wait for the old value
  __hip_atomic_fetch_add(meta + LMOE_META_GEN, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t match_key(int key, int nbits) {
  uint64_t m = __ballot(1);
  for (int b = 0; b < nbits; ++b) {
    const bool bit = (key >> b) & 1;
    const uint64_t bb = __ballot(bit);
    m &= bit ? bb : ~bb;
  }
  return m;
}

// Exclusive scan over a block of 1024 threads.  Returns the exclusive prefix
// of v; *total receives the block sum.  Uses scan_lds[32].
__device__ int block_exclusive_scan(int v, int* scan_lds, int* total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const int inc = wave_inclusive_sum(v);
  if (lane == 63) scan_lds[wave] = inc;
  __syncthreads();
  if (wave == 0) {
    // the wave totals scanned by one wave (nw <= 16 lanes) instead of one
    // thread walking them through LDS
    const int t = lane < nw ? scan_lds[lane] : 0;
    const int tinc = wave_inclusive_sum(t);
    if (lane < nw) scan_lds[lane] = tinc - t;
    if (lane == 63) scan_lds[nw] = tinc;
  }
  __syncthreads();
  const int excl = scan_lds[wave] + inc - v;
  *total = scan_lds[nw];
  __syncthreads();
  return excl;
}

// Launch order of the active-slot list.  The decode GEMVs give the a-th
// active slot the a-th row of their grid, and the hardware dispatches rows in
// order; a workgroup's time grows with its slot's pair count, so one hot slot
// dispatched late ends the kernel long after the rest (one slot of 60 of 512
// pairs: 35 us past the others).  A heavy slot, one holding at least 1/16 of
// the placed pairs and at least kHeavyMinPairs of them, therefore comes
// first, heaviest first (ties: ascending slot); every other active slot
// follows in ascending slot order, which keeps light and moderately loaded
// slots mixed (moving those forward as well measured 1-4% slower, and a
// bound of 8 pairs cost the 16-token decode layer 1%).  The 1/16 bound
// admits at most 16 heavy slots.  The order changes no output bits: every
// kernel writes by sorted position, never by active rank.
constexpr int kHeavyMinPairs = 16;
constexpr int kMaxHeavy = 16;

__device__ __forceinline__ bool heavy_slot(int count, int placed) {
  return count >= kHeavyMinPairs && 16 * count >= placed;
}

// Order key of a heavy slot: a larger key is listed first (higher count,
// then lower slot); never 0, the value of an empty entry of a key list.
__device__ __forceinline__ uint64_t heavy_key(int count, int s) {
  return (static_cast<uint64_t>(count) << 32) | (0xffffffffu - static_cast<uint32_t>(s));
}

// The same order in 32 bits, for count < 65536 and s < 65536.
__device__ __forceinline__ uint32_t heavy_key16(int count, int s) {
  return (static_cast<uint32_t>(count) << 16) | (0xffffu - static_cast<uint32_t>(s));
}

// Rank of key among the kMaxHeavy entries of an LDS key list (empty entries
// 0): the reads are independent, so all of them are in flight at once.
template <typename K>
__device__ __forceinline__ int heavy_rank(const K* keys, K key) {
  int rank = 0;
#pragma unroll
  for (int j = 0; j < kMaxHeavy; ++j) rank += keys[j] > key;
  return rank;
}

// Scan counts[0..P) held in LDS (hist) into offsets/active/tile_off; writes
// counts, offsets, active (in the launch order above), tile_off and
// meta[ACTIVE, PAIRS, TILES], and replaces hist[s] by offsets[s] in place
// (each s is owned by one thread).  PUBLISH false: only the in-place
// conversion (a workgroup that needs the offsets but is not the one that
// writes the outputs).
template <bool PUBLISH = true>
__device__ void scan_slots(int* hist, int P, int block_m, int* scan_lds,
                           int32_t* counts, int32_t* offsets, int32_t* active,
                           int32_t* tile_off, int32_t* meta) {
  // keys of the heavy slots in slot order, empty entries 0
  __shared__ uint64_t heavy_keys[kMaxHeavy];
  const int per = (P + blockDim.x - 1) / blockDim.x;
  const int s0 = threadIdx.x * per;
  if (threadIdx.x < kMaxHeavy) heavy_keys[threadIdx.x] = 0;
  int csum = 0, tsum = 0;
  for (int i = 0; i < per; ++i) {
    const int s = s0 + i;
    if (s < P) {
      const int c = hist[s];
      csum += c;
      tsum += (c + block_m - 1) / block_m;
    }
  }
  int ctot, hltot, ttot;
  int cpre = block_exclusive_scan(csum, scan_lds, &ctot);
  // heavy slots (high half) and light active slots (low half: at most
  // kMaxSlots < 65536) in one scan
  int hl = 0;
  for (int i = 0; i < per; ++i) {
    const int s = s0 + i;
    if (s < P) {
      const int c = hist[s];
      hl += heavy_slot(c, ctot) ? (1 << 16) : (c > 0);
    }
  }
  const int hlpre = block_exclusive_scan(hl, scan_lds, &hltot);
  const int nh = hltot >> 16;
  const int atot = nh + (hltot & 0xffff);
  int lpre = nh + (hlpre & 0xffff);
  if (__builtin_expect(hl >> 16, 0)) {
    int h = hlpre >> 16;
    for (int i = 0; i < per; ++i) {
      const int s = s0 + i;
      if (s < P && heavy_slot(hist[s], ctot)) heavy_keys[h++] = heavy_key(hist[s], s);
    }
  }
  // the scan's barriers also publish the keys (and, in the one before,
  // order their clearing before the writes)
  int tpre = block_exclusive_scan(tsum, scan_lds, &ttot);
  for (int i = 0; i < per; ++i) {
    const int s = s0 + i;
    if (s < P) {
      const int c = hist[s];
      if (PUBLISH) {
        counts[s] = c;
        offsets[s] = cpre;
        tile_off[s] = tpre;
        if (__builtin_expect(heavy_slot(c, ctot), 0)) active[heavy_rank(heavy_keys, heavy_key(c, s))] = s;
        else if (c > 0) active[lpre++] = s;
      }
      hist[s] = cpre;
      cpre += c;
      tpre += (c + block_m - 1) / block_m;
    }
  }
  if (!PUBLISH) return;
  // active[a] = -1 past the active slots: kernels that serve "the a-th
  // active slot" read one value (no dependent load of meta first)
  for (int a = atot + threadIdx.x; a < P; a += blockDim.x) active[a] = -1;
  if (threadIdx.x == 0) {
    offsets[P] = ctot;
    tile_off[P] = ttot;
    meta[LMOE_META_ACTIVE] = atot;
    meta[LMOE_META_PAIRS] = ctot;
    meta[LMOE_META_TILES] = ttot;
    publish_build(meta);
  }
}

// Stable ranks of one chunk.  slot[] is this thread's slot (>= 0 placed),
// run_base[s] holds the next free position of slot s and is advanced.
__device__ int chunk_positions(int s, int nbits, int* run_base) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const bool placed = s >= 0;
  const int key = placed ? s : (1 << nbits) - 1;
  const uint64_t m = match_key(key, nbits);
  const int rank = __popcll(m & lanemask_lt(lane));
  const int cnt = __popcll(m);
  const bool last = lane == 63 - __clzll(m);
  int pos = -1;
  for (int w = 0; w < nw; ++w) {
    if (wave == w && placed) {
      const int b = run_base[s];
      pos = b + rank;
      if (last) run_base[s] = b + cnt;
    }
    __syncthreads();
  }
  return pos;
}

__device__ __forceinline__ int key_bits(int P) {
  // keys 0..P (P = "not placed" sentinel fits when (1<<nbits)-1 >= P)
  int nbits = 1;
  while ((1 << nbits) - 1 < P) ++nbits;
  return nbits;
}

// Whole permutation of N <= kChunk pairs by one block.  ids may live in
// global memory or LDS; hist is LDS of P ints, scan_lds 33 ints, err_lds one.
// Thread i owns pairs i + c * blockDim.x.
__device__ __forceinline__ void permute_block(
    const int32_t* ids, int N, const int32_t* __restrict__ log2phy,
    int n_log2phy, int P, int skip, int block_m, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ sorted_pairs,
    int32_t* __restrict__ row_idx, int32_t* __restrict__ active,
    int32_t* __restrict__ tile_off, int32_t* __restrict__ meta, int* hist,
    int* scan_lds, int* err_lds, RowKeep keep = {}) {
  for (int s = threadIdx.x; s < P; s += blockDim.x) hist[s] = 0;
  if (threadIdx.x == 0) *err_lds = 0;
  __syncthreads();
  constexpr int kSmallChunks = kChunk / 64;
  int sl[kSmallChunks];
#pragma unroll
  for (int c = 0; c < kSmallChunks; ++c) {
    const int p = threadIdx.x + c * blockDim.x;
    sl[c] = -1;
    if (p < N) {
      const int s = map_pair(ids, p, log2phy, n_log2phy, P, skip);
      sl[c] = s;
      if (s >= 0) atomicAdd(&hist[s], 1);
      if (s == -2) atomicAdd(err_lds, 1);
    }
  }
  __syncthreads();
  scan_slots(hist, P, block_m, scan_lds, counts, offsets, active, tile_off, meta);
  if (threadIdx.x == 0) meta[LMOE_META_ERRORS] = *err_lds;
  __syncthreads();  // hist now holds offsets: the running base of each slot
  const int nb = key_bits(P);
#pragma unroll
  for (int c = 0; c < kSmallChunks; ++c) {
    if (c * static_cast<int>(blockDim.x) < N) {  // uniform across the block
      const int p = threadIdx.x + c * blockDim.x;
      const int s = sl[c] >= 0 ? sl[c] : -1;
      const int pos = chunk_positions(s, nb, hist);  // chunks in pair order: stable
      if (p < N) {
        if ((pos >= 0 || skip != kSkipKeepRows) && !kept_row(keep, ids, p)) row_idx[p] = pos;
        if (pos >= 0) sorted_pairs[pos] = p;
      }
    }
  }
}

// One wave permutes N <= 64 * PPL pairs over P <= 64 * SPL slots (the
// decode sizes) with ballots, shuffles and LDS, but no block barrier: pair
// p = 64 g + lane belongs to group g of lane `lane`, slot s is owned by lane
// s / SPL.  Groups are ranked in order, so pairs of one slot keep their flat
// order.  Same outputs as permute_block.  lds: wave_perm_lds_ints(P) ints of
// the calling wave's own LDS.
constexpr int kWavePermMaxSlotsPerLane = 16;
constexpr int kWavePermMaxPairsPerLane = 4;

// Per-slot outputs of one lane's slots s0 .. s0 + SPL - 1 (counts c, running
// pair and tile prefixes cpre / tpre): counts, offsets, tile_off, the slot's
// running base in lds, and the active entry of each slot with pairs at
// positions lpos, lpos + 1, ...; with SKIP_HEAVY the heavy slots are left out
// (the caller lists them).
template <int SPL, bool SKIP_HEAVY>
__device__ __forceinline__ void wave_slot_outputs(const int (&c)[SPL], int s0, int P, int block_m,
                                                  int ctot, int cpre, int tpre, int lpos,
                                                  int32_t* __restrict__ counts,
                                                  int32_t* __restrict__ offsets,
                                                  int32_t* __restrict__ tile_off,
                                                  int32_t* __restrict__ active, int* lds) {
#pragma unroll
  for (int i = 0; i < SPL; ++i) {
    const int sl = s0 + i;
    if (sl < P) {
      counts[sl] = c[i];
      offsets[sl] = cpre;
      tile_off[sl] = tpre;
      if (c[i] > 0 && !(SKIP_HEAVY && heavy_slot(c[i], ctot))) active[lpos++] = sl;
      lds[sl] = cpre;  // running base of the slot
      cpre += c[i];
      tpre += (c[i] + block_m - 1) / block_m;
    }
  }
}

template <int SPL, int PPL>
__device__ __forceinline__ void permute_wave(
    const int32_t* ids, int N, const int32_t* __restrict__ log2phy, int n_log2phy, int P,
    int skip, int block_m, int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ sorted_pairs, int32_t* __restrict__ row_idx,
    int32_t* __restrict__ active, int32_t* __restrict__ tile_off, int32_t* __restrict__ meta,
    int* lds, RowKeep keep = {}) {
  const int lane = threadIdx.x & 63;
  const int nbits = key_bits(P);
  int s[PPL], rank[PPL], cnt[PPL];
  int errs = 0;
#pragma unroll
  for (int g = 0; g < PPL; ++g) {
    const int p = g * kWave + lane;
    const bool have = p < N;
    s[g] = have ? map_pair(ids, p, log2phy, n_log2phy, P, skip) : -1;
    errs += __popcll(__ballot(have && s[g] == -2));
  }
#pragma unroll
  for (int i = 0; i < SPL; ++i) lds[lane * SPL + i] = 0;
  wave_lds_sync();
  // pairs of the same slot within each group, this pair's rank among them,
  // and the slot counts (the group's first pair of a slot adds the group's
  // count; one LDS add per slot and group)
#pragma unroll
  for (int g = 0; g < PPL; ++g) {
    const bool placed = s[g] >= 0;
    const uint64_t m = match_key(placed ? s[g] : (1 << nbits) - 1, nbits);
    rank[g] = __popcll(m & lanemask_lt(lane));
    cnt[g] = __popcll(m);
    if (placed && rank[g] == 0) {
      if constexpr (PPL == 1) lds[s[g]] = cnt[g];  // one group: one writer per slot
      else atomicAdd(&lds[s[g]], cnt[g]);
    }
  }
  wave_lds_sync();
  // this lane's slots s0 .. s0+SPL-1: counts, then wave-wide prefixes
  const int s0 = lane * SPL;
  int c[SPL];
  int csum = 0, asum = 0, tsum = 0;
#pragma unroll
  for (int i = 0; i < SPL; ++i) {
    c[i] = (s0 + i < P) ? lds[s0 + i] : 0;
    csum += c[i];
    asum += c[i] > 0;
    tsum += (c[i] + block_m - 1) / block_m;
  }
  const int cinc = wave_inclusive_sum(csum);
  int cpre = cinc - csum;
  const int ctot = read_lane_i32(cinc, 63);
  // launch order (heavy_slot): whether the wave holds a heavy slot (one
  // ballot; the rare heavy case counts them again)
  bool lane_heavy = false;
#pragma unroll
  for (int i = 0; i < SPL; ++i) lane_heavy |= heavy_slot(c[i], ctot);
  const bool any_heavy = __builtin_amdgcn_ballot_w64(lane_heavy) != 0ull;
  int apre, atot, tpre, ttot;
  if constexpr (SPL == 1) {
    // one slot per lane: the active prefix is a ballot count
    const uint64_t am = __builtin_amdgcn_ballot_w64(asum > 0);
    apre = static_cast<int>(__popcll(am & lanemask_lt(lane)));
    atot = static_cast<int>(__popcll(am));
  } else {
    const int ainc = wave_inclusive_sum(asum);
    apre = ainc - asum;
    atot = read_lane_i32(ainc, 63);
  }
  if (SPL == 1 && N <= block_m) {
    // no slot holds more than block_m pairs: one tile per active slot, so
    // the tile prefix is the active prefix in slot order
    tpre = apre;
    ttot = atot;
  } else {
    const int tinc = wave_inclusive_sum(tsum);
    tpre = tinc - tsum;
    ttot = read_lane_i32(tinc, 63);
  }
  // uniform; marked unlikely so that the branch is laid out after the
  // kernel's straight-line path
  if (__builtin_expect(any_heavy, 0)) {
    // heavy keys in lds[64 SPL .. + kMaxHeavy) (slot order, empty entries
    // 0); lane j < nh ranks key j against all of them and lists its slot.
    // Light slots follow the nh heavy ones: active slots before this lane's,
    // less the heavy ones.  (counts <= N <= 256 and slots < 1024 here:
    // 32-bit keys)
    int hsum = 0;
#pragma unroll
    for (int i = 0; i < SPL; ++i) hsum += heavy_slot(c[i], ctot);
    const int hinc = wave_inclusive_sum(hsum);
    const int hpre = hinc - hsum;
    const int nh = read_lane_i32(hinc, 63);
    uint32_t* keys = reinterpret_cast<uint32_t*>(lds + kWave * SPL);
    if (lane < kMaxHeavy && lane >= nh) keys[lane] = 0;
    int h = hpre;
#pragma unroll
    for (int i = 0; i < SPL; ++i)
      if (heavy_slot(c[i], ctot)) keys[h++] = heavy_key16(c[i], s0 + i);
    wave_lds_sync();
    if (lane < nh) {
      const uint32_t key = keys[lane];
      active[heavy_rank(keys, key)] = static_cast<int>(0xffffu - (key & 0xffffu));
    }
    wave_lds_sync();  // every lane has read its counts and the keys before lds is reused
    wave_slot_outputs<SPL, true>(c, s0, P, block_m, ctot, cpre, tpre, apre + nh - hpre, counts,
                                 offsets, tile_off, active, lds);
  } else {
    wave_lds_sync();  // every lane has read its counts before lds is reused
    wave_slot_outputs<SPL, false>(c, s0, P, block_m, ctot, cpre, tpre, apre, counts, offsets,
                                  tile_off, active, lds);
  }
  // active[a] = -1 past the active slots (see scan_slots)
  for (int a = atot + lane; a < P; a += kWave) active[a] = -1;
  if (lane == 0) {
    offsets[P] = ctot;
    tile_off[P] = ttot;
    meta[LMOE_META_ACTIVE] = atot;
    meta[LMOE_META_PAIRS] = ctot;
    meta[LMOE_META_ERRORS] = errs;
    meta[LMOE_META_TILES] = ttot;
    publish_build(meta);
  }
  // groups in flat order: read the slot's running base, then its first
  // pair of the group advances it past the group's pairs
#pragma unroll
  for (int g = 0; g < PPL; ++g) {
    wave_lds_sync();
    const int p = g * kWave + lane;
    const bool placed = s[g] >= 0;
    const int pos = placed ? lds[s[g]] + rank[g] : -1;
    if constexpr (PPL > 1) {
      wave_lds_sync();
      if (placed && rank[g] == 0) lds[s[g]] = pos + cnt[g];
    }
    if (p < N) {
      if ((pos >= 0 || skip != kSkipKeepRows) && !kept_row(keep, ids, p)) row_idx[p] = pos;
      if (pos >= 0) sorted_pairs[pos] = p;
    }
  }
}

// Slots per lane of permute_wave for P slots (0 when P exceeds the wave path).
__host__ __device__ inline int wave_perm_spl(int P) {
  const int need = (P + 63) / 64;
  int spl = 1;
  while (spl < need) spl <<= 1;
  return spl <= kWavePermMaxSlotsPerLane ? spl : 0;
}

// Pairs per lane of permute_wave for N pairs (0 when N exceeds the wave path).
__host__ __device__ inline int wave_perm_ppl(int N) {
  return N <= kWave ? 1 : N <= 2 * kWave ? 2 : N <= 4 * kWave ? 4 : 0;
}

// LDS ints permute_wave needs for P slots: the count table of 64 slots per
// lane and the heavy-slot key list.
__host__ __device__ inline int wave_perm_lds_ints(int P) {
  return kWave * wave_perm_spl(P) + kMaxHeavy;
}

// Whether one wave permutes N pairs over P slots.
__host__ __device__ inline bool wave_perm_fits(int N, int P) {
  return wave_perm_ppl(N) > 0 && wave_perm_spl(P) > 0;
}

// permute_wave with PPL pairs per lane for any P <= 64 *
// kWavePermMaxSlotsPerLane (lds: wave_perm_lds_ints(P) ints).  PPL is a
// template parameter of the callers' kernels: one pair layout per kernel
// keeps the latency-bound routers' code (and registers) small.
template <int PPL>
__device__ __forceinline__ void permute_wave_any(
    const int32_t* ids, int N, const int32_t* __restrict__ log2phy, int n_log2phy, int P,
    int skip, int block_m, int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ sorted_pairs, int32_t* __restrict__ row_idx,
    int32_t* __restrict__ active, int32_t* __restrict__ tile_off, int32_t* __restrict__ meta,
    int* lds, RowKeep keep = {}) {
  const int spl = wave_perm_spl(P);
#define LMOE_PW(S)                                                                                  \
  permute_wave<S, PPL>(ids, N, log2phy, n_log2phy, P, skip, block_m, counts, offsets, sorted_pairs, \
                       row_idx, active, tile_off, meta, lds, keep)
  if (spl <= 1) LMOE_PW(1);
  else if (spl == 2) LMOE_PW(2);
  else if (spl == 4) LMOE_PW(4);
  else if (spl == 8) LMOE_PW(8);
  else LMOE_PW(16);
#undef LMOE_PW
}

}  // namespace lmoe
