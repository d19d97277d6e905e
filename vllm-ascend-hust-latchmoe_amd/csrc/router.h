// Router kernels shared by router.hip and the per-scoring translation units:
// gate rows (bf16 GEMV, f32 accumulation), expert selection (softmax top-k,
// or sigmoid + correction bias + group-limited top-k, one wave64 per token)
// and the one-launch decode routers that add the permutation.
//
// Reference behaviour: moe_router_op.py:191-278 (gate then select_experts),
// renorm contract patches/patch_fused_moe.py:597-632
// (w / w.sum().clamp_min(eps)), grouped sigmoid as configured for the
// DeepSeek-V3-style layer (bias for selection only, sum of the two best scores
// per group, keep topk_group groups, renormalise, then scale).
#pragma once

#include "gemm_lds.h"
#include "gemm_mfma.h"
#include "permute.h"
#include "select.h"

namespace lmoe {

constexpr int kGateMaxChunks = 16;  // H <= 16 * 512 = 8192 in the GEMV path
constexpr int kGateShortChunks = 4;  // the one-launch router's short-row gate: H <= 2048
// threads of every one-token one-launch router: the gate form's eight gate
// rows per block, which also covers the slot scan up to kMaxSlots / 16
constexpr int kOneTokenRouterThreads = 512;
// router gate at large T: 64-row x 128-expert tiles, 2 waves, 4-stage ring
using DenseGateTile = SmallTile;
constexpr int kGateTok = 4;         // tokens per reduction in the gate GEMV
// one-launch router: tagged logit words from int32 offset 64 of sync (256
// bytes past the arrival counter), and the re-reads of a stale word
constexpr int kRouterWordsOffset = 64;
constexpr int kRouterSpinLimit = 1 << 16;
static_assert(kRouterWordsOffset + 2 * 16 * 256 == LMOE_ROUTER_SYNC_WORDS, "sync layout");

// A logit as the selection reads it (bf16 logits are rounded first).
__device__ __forceinline__ float selected_logit(float acc, int logits_f32) {
  return logits_f32 ? acc : bf16_to_f32(static_cast<uint16_t>(f32_to_bf16_bits(acc)));
}

// Store logit o: the logits output, and with words (the one-launch router)
// the same value as a tagged word, (tag << 32) | f32 bits, by an
// agent-scope atomic store that the selecting workgroup reads back.
__device__ __forceinline__ void store_logit(void* __restrict__ logits, int logits_f32, size_t o,
                                            float acc, uint64_t* __restrict__ words, uint32_t tag) {
  if (logits_f32) {
    reinterpret_cast<float*>(logits)[o] = acc;
  } else {
    reinterpret_cast<uint16_t*>(logits)[o] = static_cast<uint16_t>(f32_to_bf16_bits(acc));
  }
  if (words != nullptr) {
    const uint64_t word = (static_cast<uint64_t>(tag) << 32) |
                          __float_as_uint(selected_logit(acc, logits_f32));
    __hip_atomic_store(words + o, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// logits[t][e] of one expert e for tokens [t0, t1), by the calling wave.
// The expert row stays in registers (one 16-byte chunk per 512 columns per
// lane) while the token rows stream through L1.  ONE: t1 == t0 + 1 (the
// kernel holds only the single-token code).  words: see store_logit.  FULL:
// H == NC * 512, so the chunk loads need no guards (the guards' zeroed
// registers and exec-masked loads come before the first load issues).
template <int NC, bool ONE, bool FULL = false>
__device__ __forceinline__ void gate_row(const uint16_t* __restrict__ x,
                                         const uint16_t* __restrict__ wg, int t0, int t1,
                                         int H, int E, int e, void* __restrict__ logits,
                                         int logits_f32, uint64_t* __restrict__ words = nullptr,
                                         uint32_t tag = 0) {
  const int lane = threadIdx.x & 63;
  const uint16_t* wrow = wg + static_cast<size_t>(e) * H;

  uint4 w[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int h = c * 512 + lane * 8;
    w[c] = load16_g<!FULL>(wrow, h, h < H);
  }
  // kGateTok tokens per reduction (x rows in flight together; the same
  // lane-pair tree per token as a lone wave_sum, so the logits do not depend
  // on how tokens are grouped)
  if constexpr (ONE) {
    const uint16_t* xr = x + static_cast<size_t>(t0) * H;
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int h = c * 512 + lane * 8;
      acc = dot8(load16_g<!FULL>(xr, h, h < H), w[c], acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) store_logit(logits, logits_f32, static_cast<size_t>(t0) * E + e, acc, words, tag);
  } else {
    for (int tb = t0; tb < t1; tb += kGateTok) {
      const uint16_t* xr[kGateTok];
#pragma unroll
      for (int g = 0; g < kGateTok; ++g)
        xr[g] = x + static_cast<size_t>(tb + g < t1 ? tb + g : t1 - 1) * H;
      float v[kGateTok];
#pragma unroll
      for (int g = 0; g < kGateTok; ++g) v[g] = 0.0f;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int h = c * 512 + lane * 8;
#pragma unroll
        for (int g = 0; g < kGateTok; ++g) v[g] = dot8(load16_if(xr[g], h, h < H), w[c], v[g]);
      }
      // lane l ends with the total of token tb + l / 16
      const float acc = reduce_scatter<kGateTok, 5, 0>(v, lane);
      const int t = tb + (lane >> 4);
      if ((lane & 15) == 0 && t < t1)
        store_logit(logits, logits_f32, static_cast<size_t>(t) * E + e, acc, words, tag);
    }
  }
}

// Expert selection and the permutation of the selected pairs in one block,
// for a slot table that is final before the router runs (decode replay
// after staging).  Wave t selects token t (T <= kFusedTopkTokens); the ids
// go to LDS and feed the same permutation code as lmoe_permute (one wave, or
// the whole block), so every output equals what lmoe_router_topk followed by
// lmoe_permute writes.
constexpr int kFusedTopkTokens = 16;

// LDS of the selection of T <= kFusedTopkTokens tokens and the permutation
// of their pairs.
template <int EPL>
struct TopkPermuteLds {
  SelectLds<EPL> sel[kFusedTopkTokens];
  int32_t ids[kFusedTopkTokens * kMaxK];
  int scan[33];
  int err;
};

// Logits of token t from the one-launch router's tagged words (expert
// j*64 + lane, -inf beyond E).  A word whose tag is not this launch's holds
// an earlier launch's logit, or this launch's store is not visible here
// yet: it is read again (agent scope) until its tag matches, at most
// kRouterSpinLimit rounds; past them meta[LMOE_META_ROUTER_TIMEOUT] becomes 1
// and the value read is used.
template <int EPL>
__device__ __forceinline__ void load_logits_tagged(const uint64_t* words, uint32_t tag, int t,
                                                   int E, float (&lg)[EPL], int32_t* meta) {
  const int lane = threadIdx.x & 63;
  uint64_t wv[EPL];
  bool ok = true;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = j * kWave + lane;
    wv[j] = e < E ? __hip_atomic_load(words + static_cast<size_t>(t) * E + e, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT)
                  : static_cast<uint64_t>(tag) << 32;
    ok = ok && static_cast<uint32_t>(wv[j] >> 32) == tag;
  }
  for (int spin = 0; __builtin_amdgcn_ballot_w64(!ok) != 0; ++spin) {
    if (spin == kRouterSpinLimit) {
      if (lane == 0) {
        __hip_atomic_store(meta + LMOE_META_ROUTER_TIMEOUT, 1, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        add_device_flag(LMOE_FLAG_ROUTER_TIMEOUT, 1);
      }
      break;
    }
    __builtin_amdgcn_s_sleep(1);
    ok = true;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int e = j * kWave + lane;
      if (static_cast<uint32_t>(wv[j] >> 32) != tag)
        wv[j] = __hip_atomic_load(words + static_cast<size_t>(t) * E + e, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
      ok = ok && static_cast<uint32_t>(wv[j] >> 32) == tag;
    }
  }
#pragma unroll
  for (int j = 0; j < EPL; ++j)
    lg[j] = j * kWave + lane < E ? __uint_as_float(static_cast<uint32_t>(wv[j])) : -INFINITY;
}

// One token's pairs in pair order, for the one-token MLP kernels (which read
// active[a] as the slot of position a, a pair of its own, and row_idx[p] as
// pair p's position): lane j < kw holds pair j's expert e.  The placed pairs
// take positions 0, 1, ... in pair order (a pair whose id maps to no slot
// of the table is left out, and counted in meta[LMOE_META_ERRORS] unless
// skip allows it, as map_id decides): active[pos] = its slot,
// sorted_pairs[pos] = j, row_idx[j] = pos or -1, active[a] = -1 from the
// placed count on (every a < P).  meta ACTIVE and PAIRS = the placed pairs,
// ERRORS, and the build count advances; counts, offsets, tile_off and
// meta[TILES] are not written.  With distinct slots this is the sorted
// permutation with the slots in pair order: the one-token kernels compute
// every value as from it.
__device__ __forceinline__ void pair_order_outputs(int e, int lane, int kw,
                                                   const int32_t* __restrict__ log2phy,
                                                   int n_log2phy, int P, int skip,
                                                   int32_t* __restrict__ sorted_pairs,
                                                   int32_t* __restrict__ row_idx,
                                                   int32_t* __restrict__ active,
                                                   int32_t* __restrict__ meta) {
  const int s = lane < kw ? map_id(e, log2phy, n_log2phy, P, skip) : -1;
  const bool placed = s >= 0;
  const uint64_t pm = __ballot(placed);
  const int pos = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(pm >> 32),
                                            __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(pm), 0));
  const int n_placed = __popcll(pm);
  const int n_err = __popcll(__ballot(s == -2));
  if (lane < kw) row_idx[lane] = placed ? pos : -1;
  if (placed) {
    sorted_pairs[pos] = lane;
    active[pos] = s;
  }
  for (int a = n_placed + lane; a < P; a += kWave) active[a] = -1;
  if (lane == 0) {
    meta[LMOE_META_ACTIVE] = n_placed;
    meta[LMOE_META_PAIRS] = n_placed;
    meta[LMOE_META_ERRORS] = n_err;
    publish_build(meta);
  }
}

// PPL > 0: one wave permutes with PPL pairs per lane; PPL == 0: the block
// permutation (more pairs or slots than one wave takes).  SCORE: the
// scoring (LMOE_SCORING_*), sp.scoring must agree.  words (the one-launch
// router): the logits come from its tagged words, see load_logits_tagged.
// PPL < 0: one token in pair order (pair_order_outputs) instead of the
// permutation.
template <int EPL, int PPL, int SCORE>
__device__ __forceinline__ void select_and_permute(
    const void* __restrict__ logits, int logits_f32, int T, const SelectParams& sp,
    float* __restrict__ w_f32, uint16_t* __restrict__ w_bf16, int32_t* __restrict__ ids,
    const int32_t* __restrict__ log2phy, int n_log2phy, int P, int skip, int block_m,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ sorted_pairs, int32_t* __restrict__ row_idx,
    int32_t* __restrict__ active, int32_t* __restrict__ tile_off, int32_t* __restrict__ meta,
    int* hist, TopkPermuteLds<EPL>& L, const uint64_t* words = nullptr, uint32_t tag = 0) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  if (wave < T) {
    float bv[EPL], lb[EPL], lg[EPL];
    load_bias<EPL>(sp, bv, lb);
    if (words != nullptr) load_logits_tagged<EPL>(words, tag, wave, sp.E, lg, meta);
    else load_logits<EPL>(logits, logits_f32, wave, sp.E, lg);
    int e;
    float w;
    select_token<EPL, SCORE>(sp, lg, bv, lb, L.sel[wave], e, w);
    const int kw = sp.k + sp.n_shared;
    if (lane >= sp.k) {
      // the pinned shared-expert suffix: ids E, E + 1, ..., weight 1
      e = sp.E + lane - sp.k;
      w = 1.0f;
    }
    if (lane < kw) {
      const int o = wave * kw + lane;
      ids[o] = e;
      L.ids[o] = e;
      w_bf16[o] = static_cast<uint16_t>(f32_to_bf16_bits(w));
      if (w_f32 != nullptr) w_f32[o] = w;
    }
    if constexpr (PPL < 0) {
      pair_order_outputs(e, lane, kw, log2phy, n_log2phy, P, skip, sorted_pairs, row_idx, active,
                         meta);
      return;
    }
  }
  if constexpr (PPL < 0) return;  // one token: wave 0 wrote everything
  __syncthreads();
  const int n_pairs = T * (sp.k + sp.n_shared);
  if constexpr (PPL > 0) {
    if (wave == 0)
      permute_wave_any<PPL>(L.ids, n_pairs, log2phy, n_log2phy, P, skip, block_m, counts,
                            offsets, sorted_pairs, row_idx, active, tile_off, meta, hist);
  } else {
    permute_block(L.ids, n_pairs, log2phy, n_log2phy, P, skip, block_m, counts, offsets,
                  sorted_pairs, row_idx, active, tile_off, meta, hist, L.scan, &L.err);
  }
}

// Pair layout of the routers' permutation: pairs per lane of the one-wave
// path, 0 for the block path.
__host__ inline int router_perm_ppl(int n_pairs, int n_slots) {
  return wave_perm_fits(n_pairs, n_slots) ? wave_perm_ppl(n_pairs) : 0;
}

template <int EPL, int PPL, int SCORE>
__global__ __launch_bounds__(1024) void topk_permute_kernel(
    const void* __restrict__ logits, int logits_f32, int T, SelectParams sp,
    float* __restrict__ w_f32, uint16_t* __restrict__ w_bf16, int32_t* __restrict__ ids,
    const int32_t* __restrict__ log2phy, int n_log2phy, int P, int skip, int block_m,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ sorted_pairs, int32_t* __restrict__ row_idx,
    int32_t* __restrict__ active, int32_t* __restrict__ tile_off, int32_t* __restrict__ meta) {
  extern __shared__ int hist[];  // [max(P, wave_perm_lds_ints(P))]
  __shared__ TopkPermuteLds<EPL> L;
  select_and_permute<EPL, PPL, SCORE>(logits, logits_f32, T, sp, w_f32, w_bf16, ids, log2phy,
                                      n_log2phy, P, skip, block_m, counts, offsets,
                                      sorted_pairs, row_idx, active, tile_off, meta, hist, L);
}

// Gate, selection and permutation in one launch.  Block (b, g)'s waves
// compute the logits of experts b * nw + wave for the tokens of group g
// (kGateTok tokens per group, gridDim.y groups) and store them, to the
// logits output and as tagged words in sync (value | this launch's build
// number << 32, agent-scope atomic stores); the block then counts itself in
// with an atomic add on sync[0].  The last block to arrive (the add returns
// the grid size - 1) resets sync[0] to 0 for the next launch and runs the
// selection and the permutation, reading the words back and reading again
// any whose tag is not yet this launch's.  Only that last block ever waits,
// for stores that every other block has already issued.  Calls that may run
// concurrently need separate sync buffers, and a sync buffer serves one
// permutation (one meta).  ONE: T == 1.  FULL: H == NC * 512 (see gate_row).
template <int NC, int EPL, int PPL, int SCORE, bool ONE, bool FULL = false>
__global__ __launch_bounds__(ONE ? kOneTokenRouterThreads : 1024) void gate_topk_permute_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wg, int T, int H,
    void* __restrict__ logits, int logits_f32, SelectParams sp, float* __restrict__ w_f32,
    uint16_t* __restrict__ w_bf16, int32_t* __restrict__ ids,
    const int32_t* __restrict__ log2phy, int n_log2phy, int P, int skip, int block_m,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ sorted_pairs, int32_t* __restrict__ row_idx,
    int32_t* __restrict__ active, int32_t* __restrict__ tile_off, int32_t* __restrict__ meta,
    int32_t* __restrict__ sync) {
  extern __shared__ int hist[];  // [max(P, wave_perm_lds_ints(P))]
  __shared__ TopkPermuteLds<EPL> L;
  __shared__ int32_t l2p_lds[kMaxE];
  __shared__ int last;
  const int nw = blockDim.x >> 6;
  const int e = blockIdx.x * nw + (threadIdx.x >> 6);
  // every block copies the slot table while its gate rows load, so that the
  // last one remaps the selected ids from LDS (no table: the identity).  The
  // selected ids are below E + n_shared <= kMaxE, so the first kMaxE entries
  // cover them; the permutation then reads the table with LDS loads only,
  // not with generic loads that would also wait for the global stores of
  // the selection
  const int n_tab = log2phy != nullptr ? min(n_log2phy, kMaxE) : min(sp.E + sp.n_shared, kMaxE);
  for (int i = threadIdx.x; i < n_tab; i += blockDim.x) l2p_lds[i] = log2phy != nullptr ? log2phy[i] : i;
  // this launch's tag: the build it makes (every block reads the count
  // before it counts in, and the count advances only after the last one has)
  const uint32_t tag = static_cast<uint32_t>(__hip_atomic_load(
                           meta + LMOE_META_GEN, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) + 1u;
  uint64_t* words = reinterpret_cast<uint64_t*>(sync + kRouterWordsOffset);
  const int t0 = ONE ? 0 : static_cast<int>(blockIdx.y) * kGateTok;
  const int t1 = ONE ? T : min(T, t0 + kGateTok);
  if (e < sp.E && t0 < t1)
    gate_row<NC, ONE, FULL>(x, wg, t0, t1, H, sp.E, e, logits, logits_f32, words, tag);
  // every wave's logits are issued before thread 0 counts the block in (not
  // waited for: waiting for the stores to complete cost 0.35 us per layer,
  // more than the last block's occasional second read)
  __syncthreads();
  if (threadIdx.x == 0) {
    // no release / acquire fences (with them the decode layer took 0.2 us
    // longer): the count only elects the last block, and the tags tell it
    // which words it still has to read again
    const int prev = __hip_atomic_fetch_add(sync, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = prev == static_cast<int>(gridDim.x * gridDim.y) - 1;
    if (last) __hip_atomic_store(sync, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last) return;
  select_and_permute<EPL, PPL, SCORE>(logits, logits_f32, T, sp, w_f32, w_bf16, ids, l2p_lds,
                                      n_tab, P, skip, block_m, counts, offsets, sorted_pairs,
                                      row_idx, active, tile_off, meta, hist, L, words, tag);
}

inline int check_select(int T, int E, int k, int n_shared, int scoring, int n_group,
                        int topk_group) {
  if (T < 0 || E <= 0 || k <= 0 || n_shared < 0) return LMOE_ERR_ARG;
  if (E > kMaxE || k + n_shared > kMaxK || k > E) return LMOE_ERR_SHAPE;
  if (scoring != LMOE_SCORING_SOFTMAX && scoring != LMOE_SCORING_SIGMOID)
    return LMOE_ERR_UNSUPPORTED;
  if (scoring == LMOE_SCORING_SIGMOID && n_group > 1) {
    if (n_group > 64 || E % n_group != 0 || E / n_group < 2) return LMOE_ERR_SHAPE;
    if (topk_group <= 0 || topk_group > n_group) return LMOE_ERR_SHAPE;
    if (k > topk_group * (E / n_group)) return LMOE_ERR_SHAPE;
  }
  return LMOE_OK;
}

inline SelectParams make_select(int E, int k, int n_shared, int scoring, const float* bias,
                                const float* logit_bias, int n_group, int topk_group,
                                int renorm, float routed_scale) {
  SelectParams sp;
  sp.E = E;
  sp.k = k;
  sp.n_shared = n_shared;
  sp.scoring = scoring;
  sp.bias = bias;
  sp.logit_bias = logit_bias;
  sp.n_group = scoring == LMOE_SCORING_SIGMOID ? (n_group > 1 ? n_group : 1) : 1;
  sp.topk_group = topk_group;
  sp.renorm = renorm;
  sp.routed_scale = routed_scale;
  return sp;
}

// Arguments of the one-launch routers (gate fields unused by the
// selection + permutation form).
struct RouterPermuteArgs {
  const void* x;
  const void* wg;
  int H;
  int32_t* sync;
  void* logits;
  int logits_f32;
  int T;
  SelectParams sp;
  float* w_f32;
  uint16_t* w_bf16;
  int32_t* ids;
  const int32_t* log2phy;
  int n_log2phy;
  int n_slots;
  int skip;
  int block_m;
  int32_t* counts;
  int32_t* offsets;
  int32_t* sorted_pairs;
  int32_t* row_idx;
  int32_t* active;
  int32_t* tile_off;
  int32_t* meta;
  bool pairs;  // one token: pair-order outputs instead of the permutation
};

// Block size and dynamic LDS of the one-launch routers: enough waves for
// the tokens (and, gate form, at least eight gate rows per block: 16
// workgroups count in for 128 experts; measured 0.24 us faster than 32
// workgroups of four rows, and 8 of sixteen rows slower again), the
// permutation's pairs and its slot scan.
inline void router_launch_shape(const RouterPermuteArgs& a, bool gate, int* threads,
                                size_t* lds) {
  const int n_pairs = a.T * (a.sp.k + a.sp.n_shared);
  int t = n_pairs > a.n_slots / 16 ? n_pairs : a.n_slots / 16;
  t = t > a.T * 64 ? t : a.T * 64;
  if (gate) t = t > 512 ? t : 512;
  t = ((t + 63) / 64) * 64;
  t = t < 64 ? 64 : (t > kChunk ? kChunk : t);
  *threads = t;
  size_t l = sizeof(int) * static_cast<size_t>(a.n_slots);
  if (wave_perm_fits(n_pairs, a.n_slots)) {
    const size_t w = sizeof(int) * static_cast<size_t>(wave_perm_lds_ints(a.n_slots));
    l = w > l ? w : l;
  }
  *lds = l;
}

// Selection + permutation launch for one scoring mode.  E <= 128 runs with
// two experts per lane, E <= 256 with four: larger per-lane widths work for
// fewer experts, and fewer instantiations keep the build and the code small.
template <int SCORE>
int launch_topk_permute(const RouterPermuteArgs& a, hipStream_t stream) {
  int threads;
  size_t lds;
  router_launch_shape(a, false, &threads, &lds);
  const int ppl = router_perm_ppl(a.T * (a.sp.k + a.sp.n_shared), a.n_slots);
#define LMOE_TP(EPL, Q)                                                                            \
  hipLaunchKernelGGL((topk_permute_kernel<EPL, Q, SCORE>), dim3(1), dim3(threads), lds, stream,    \
                     a.logits, a.logits_f32, a.T, a.sp, a.w_f32, a.w_bf16, a.ids, a.log2phy,      \
                     a.n_log2phy, a.n_slots, a.skip, a.block_m, a.counts, a.offsets,              \
                     a.sorted_pairs, a.row_idx, a.active, a.tile_off, a.meta)
#define LMOE_TP_Q(EPL)                  \
  do {                                  \
    if (ppl == 1) LMOE_TP(EPL, 1);      \
    else if (ppl == 2) LMOE_TP(EPL, 2); \
    else if (ppl == 4) LMOE_TP(EPL, 4); \
    else LMOE_TP(EPL, 0);               \
  } while (0)
  if (a.sp.E <= 128) LMOE_TP_Q(2);
  else LMOE_TP_Q(4);
#undef LMOE_TP_Q
#undef LMOE_TP
  LMOE_RETURN_LAUNCH();
}

// Gate + selection + permutation launch for one scoring mode (NC = 4 for
// H <= 2048, 16 up to 8192; experts per lane as launch_topk_permute).
template <int SCORE>
int launch_gate_topk_permute(const RouterPermuteArgs& a, hipStream_t stream) {
  int threads;
  size_t lds;
  router_launch_shape(a, true, &threads, &lds);
  const int nw = threads / 64;
  const int blocks = (a.sp.E + nw - 1) / nw;
  // several tokens: one block row per kGateTok tokens, so no wave walks
  // the token groups in turn
  const int tgroups = a.T == 1 ? 1 : (a.T + kGateTok - 1) / kGateTok;
  // -1: the one-token pair-order outputs (pair_order_outputs)
  const int ppl = a.pairs ? -1 : router_perm_ppl(a.T * (a.sp.k + a.sp.n_shared), a.n_slots);
  if (a.pairs && a.T != 1) return LMOE_ERR_SHAPE;
  const uint16_t* x = static_cast<const uint16_t*>(a.x);
  const uint16_t* wg = static_cast<const uint16_t*>(a.wg);
#define LMOE_GTP_F(NC, EPL, Q, ONE, FULL)                                                        \
  hipLaunchKernelGGL((gate_topk_permute_kernel<NC, EPL, Q, SCORE, ONE, FULL>),                   \
                     dim3(blocks, tgroups), \
                     dim3(threads), lds, stream, x, wg, a.T, a.H, a.logits, a.logits_f32, a.sp, \
                     a.w_f32, a.w_bf16, a.ids, a.log2phy, a.n_log2phy, a.n_slots, a.skip,       \
                     a.block_m, a.counts, a.offsets, a.sorted_pairs, a.row_idx, a.active,       \
                     a.tile_off, a.meta, a.sync)
#define LMOE_GTP(NC, EPL, Q, ONE) LMOE_GTP_F(NC, EPL, Q, ONE, false)
  // one token, rows of exactly NC chunks: the gate loads without guards
#define LMOE_GTP_Q(NC, EPL)                          \
  do {                                               \
    if (a.T == 1 && a.H == (NC)*512) {               \
      if (ppl < 0) LMOE_GTP_F(NC, EPL, -1, true, true); \
      else if (ppl == 1) LMOE_GTP_F(NC, EPL, 1, true, true); \
      else LMOE_GTP_F(NC, EPL, 0, true, true);       \
    } else if (a.T == 1) {                           \
      if (ppl < 0) LMOE_GTP(NC, EPL, -1, true);      \
      else if (ppl == 1) LMOE_GTP(NC, EPL, 1, true); \
      else LMOE_GTP(NC, EPL, 0, true);               \
    } else {                                         \
      if (ppl == 1) LMOE_GTP(NC, EPL, 1, false);     \
      else if (ppl == 2) LMOE_GTP(NC, EPL, 2, false); \
      else if (ppl == 4) LMOE_GTP(NC, EPL, 4, false); \
      else LMOE_GTP(NC, EPL, 0, false);              \
    }                                                \
  } while (0)
#define LMOE_GTP_E(NC)                  \
  do {                                  \
    if (a.sp.E <= 128) LMOE_GTP_Q(NC, 2); \
    else LMOE_GTP_Q(NC, 4);             \
  } while (0)
  // one-token launches run kOneTokenRouterThreads threads (the launch bound
  // that gives the long-row gate its registers)
  if (a.T == 1 && threads != kOneTokenRouterThreads) return LMOE_ERR_UNSUPPORTED;
  if (a.H <= kGateShortChunks * 512) {
    LMOE_GTP_E(4);
  } else {
    // long rows: one token only (the entry point refuses more)
    if (a.T != 1) return LMOE_ERR_SHAPE;
    if (a.sp.E <= 128) {
      if (ppl < 0) LMOE_GTP(16, 2, -1, true);
      else if (ppl == 1) LMOE_GTP(16, 2, 1, true);
      else LMOE_GTP(16, 2, 0, true);
    } else {
      if (ppl < 0) LMOE_GTP(16, 4, -1, true);
      else if (ppl == 1) LMOE_GTP(16, 4, 1, true);
      else LMOE_GTP(16, 4, 0, true);
    }
  }
#undef LMOE_GTP_E
#undef LMOE_GTP_Q
#undef LMOE_GTP
#undef LMOE_GTP_F
  LMOE_RETURN_LAUNCH();
}

// Each scoring mode's launches are instantiated in a translation unit of
// its own (router_fused_softmax.hip, router_fused_sigmoid.hip), compiled in
// parallel.
extern template int launch_topk_permute<LMOE_SCORING_SOFTMAX>(const RouterPermuteArgs&, hipStream_t);
extern template int launch_topk_permute<LMOE_SCORING_SIGMOID>(const RouterPermuteArgs&, hipStream_t);
extern template int launch_gate_topk_permute<LMOE_SCORING_SOFTMAX>(const RouterPermuteArgs&,
                                                                    hipStream_t);
extern template int launch_gate_topk_permute<LMOE_SCORING_SIGMOID>(const RouterPermuteArgs&,
                                                                    hipStream_t);

}  // namespace lmoe
