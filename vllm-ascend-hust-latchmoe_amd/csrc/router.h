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

#include "gemm_mfma.h"
#include "permute.h"
#include "select.h"

namespace lmoe {

constexpr int kGateMaxChunks = 16;  // H <= 16 * 512 = 8192 in the GEMV path
constexpr int kGateTok = 4;         // tokens per reduction in the gate GEMV

// logits[t][e] of one expert e for tokens [t0, t1), by the calling wave.
// The expert row stays in registers (one 16-byte chunk per 512 columns per
// lane) while the token rows stream through L1.  ONE: t1 == t0 + 1 (the
// kernel holds only the single-token code).
template <int NC, bool ONE>
__device__ __forceinline__ void gate_row(const uint16_t* __restrict__ x,
                                         const uint16_t* __restrict__ wg, int t0, int t1,
                                         int H, int E, int e, void* __restrict__ logits,
                                         int logits_f32) {
  const int lane = threadIdx.x & 63;
  const uint16_t* wrow = wg + static_cast<size_t>(e) * H;

  uint4 w[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int h = c * 512 + lane * 8;
    w[c] = load16_if(wrow, h, h < H);
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
      acc = dot8(load16_if(xr, h, h < H), w[c], acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) {
      const size_t o = static_cast<size_t>(t0) * E + e;
      if (logits_f32) {
        reinterpret_cast<float*>(logits)[o] = acc;
      } else {
          reinterpret_cast<uint16_t*>(logits)[o] =
              static_cast<uint16_t>(f32_to_bf16_bits(acc));
        }
      }
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
      if ((lane & 15) == 0 && t < t1) {
        const size_t o = static_cast<size_t>(t) * E + e;
        if (logits_f32) {
          reinterpret_cast<float*>(logits)[o] = acc;
        } else {
          reinterpret_cast<uint16_t*>(logits)[o] =
              static_cast<uint16_t>(f32_to_bf16_bits(acc));
        }
      }
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

// PPL > 0: one wave permutes with PPL pairs per lane; PPL == 0: the block
// permutation (more pairs or slots than one wave takes).  SCORE: the
// scoring (LMOE_SCORING_*), sp.scoring must agree.
template <int EPL, int PPL, int SCORE>
__device__ __forceinline__ void select_and_permute(
    const void* __restrict__ logits, int logits_f32, int T, const SelectParams& sp,
    float* __restrict__ w_f32, uint16_t* __restrict__ w_bf16, int32_t* __restrict__ ids,
    const int32_t* __restrict__ log2phy, int n_log2phy, int P, int skip, int block_m,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ sorted_pairs, int32_t* __restrict__ row_idx,
    int32_t* __restrict__ active, int32_t* __restrict__ tile_off, int32_t* __restrict__ meta,
    int* hist, TopkPermuteLds<EPL>& L) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  if (wave < T) {
    float bv[EPL], lb[EPL], lg[EPL];
    load_bias<EPL>(sp, bv, lb);
    load_logits<EPL>(logits, logits_f32, wave, sp.E, lg);
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
  }
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
  extern __shared__ int hist[];  // [max(P, 64 * wave_perm_spl(P))]
  __shared__ TopkPermuteLds<EPL> L;
  select_and_permute<EPL, PPL, SCORE>(logits, logits_f32, T, sp, w_f32, w_bf16, ids, log2phy,
                                      n_log2phy, P, skip, block_m, counts, offsets,
                                      sorted_pairs, row_idx, active, tile_off, meta, hist, L);
}

// Gate, selection and permutation in one launch.  Block (b, g)'s waves
// compute the logits of experts b * nw + wave for the tokens of group g
// (kGateTok tokens per group, gridDim.y groups) and store them; the block
// then counts itself in with a release fence and an atomic add on *sync.
// The last block to arrive (the add returns the grid size - 1) takes an
// acquire fence, resets *sync to 0 for the next launch, and runs the
// selection and the permutation over everything the others stored.  No block
// ever waits for another: the last one only starts once all have finished
// their stores.  Calls that may run concurrently need separate sync words.
// ONE: T == 1.
template <int NC, int EPL, int PPL, int SCORE, bool ONE>
__global__ __launch_bounds__(1024) void gate_topk_permute_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wg, int T, int H,
    void* __restrict__ logits, int logits_f32, SelectParams sp, float* __restrict__ w_f32,
    uint16_t* __restrict__ w_bf16, int32_t* __restrict__ ids,
    const int32_t* __restrict__ log2phy, int n_log2phy, int P, int skip, int block_m,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ sorted_pairs, int32_t* __restrict__ row_idx,
    int32_t* __restrict__ active, int32_t* __restrict__ tile_off, int32_t* __restrict__ meta,
    int32_t* __restrict__ sync) {
  extern __shared__ int hist[];  // [max(P, 64 * wave_perm_spl(P))]
  __shared__ TopkPermuteLds<EPL> L;
  __shared__ int32_t l2p_lds[kMaxE];
  __shared__ int last;
  const int nw = blockDim.x >> 6;
  const int e = blockIdx.x * nw + (threadIdx.x >> 6);
  // every block copies the slot table while its gate rows load, so that the
  // last one remaps the selected ids from LDS
  const bool l2p_in_lds = log2phy != nullptr && n_log2phy <= kMaxE;
  if (l2p_in_lds)
    for (int i = threadIdx.x; i < n_log2phy; i += blockDim.x) l2p_lds[i] = log2phy[i];
  const int t0 = ONE ? 0 : static_cast<int>(blockIdx.y) * kGateTok;
  const int t1 = ONE ? T : min(T, t0 + kGateTok);
  if (e < sp.E && t0 < t1) gate_row<NC, ONE>(x, wg, t0, t1, H, sp.E, e, logits, logits_f32);
  __syncthreads();  // every wave's logits are stored before thread 0 counts the block in
  if (threadIdx.x == 0) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const int prev = __hip_atomic_fetch_add(sync, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = prev == static_cast<int>(gridDim.x * gridDim.y) - 1;
    if (last) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      __hip_atomic_store(sync, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  if (!last) return;
  select_and_permute<EPL, PPL, SCORE>(logits, logits_f32, T, sp, w_f32, w_bf16, ids,
                                      l2p_in_lds ? l2p_lds : log2phy, n_log2phy, P, skip,
                                      block_m, counts, offsets, sorted_pairs, row_idx, active,
                                      tile_off, meta, hist, L);
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
    const size_t w = sizeof(int) * kWave * static_cast<size_t>(wave_perm_spl(a.n_slots));
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
  const int ppl = router_perm_ppl(a.T * (a.sp.k + a.sp.n_shared), a.n_slots);
  const uint16_t* x = static_cast<const uint16_t*>(a.x);
  const uint16_t* wg = static_cast<const uint16_t*>(a.wg);
#define LMOE_GTP(NC, EPL, Q, ONE)                                                                 \
  hipLaunchKernelGGL((gate_topk_permute_kernel<NC, EPL, Q, SCORE, ONE>), dim3(blocks, tgroups), \
                     dim3(threads), lds, stream, x, wg, a.T, a.H, a.logits, a.logits_f32, a.sp, \
                     a.w_f32, a.w_bf16, a.ids, a.log2phy, a.n_log2phy, a.n_slots, a.skip,       \
                     a.block_m, a.counts, a.offsets, a.sorted_pairs, a.row_idx, a.active,       \
                     a.tile_off, a.meta, a.sync)
#define LMOE_GTP_Q(NC, EPL)                          \
  do {                                               \
    if (a.T == 1) {                                  \
      if (ppl == 1) LMOE_GTP(NC, EPL, 1, true);      \
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
  if (a.H <= 4 * 512) LMOE_GTP_E(4);
  else LMOE_GTP_E(16);
#undef LMOE_GTP_E
#undef LMOE_GTP_Q
#undef LMOE_GTP
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
