// Router entry points: gate linear (bf16 GEMV, f32 accumulation; dense MFMA
// GEMM for many tokens), expert selection, and the one-launch decode routers
// whose kernels are instantiated per scoring mode in
// router_fused_softmax.hip / router_fused_sigmoid.hip.
//
// Reference behaviour: moe_router_op.py:191-278 (gate then select_experts),
// renorm contract patches/patch_fused_moe.py:597-632.
#include "router.h"

namespace lmoe {

// logits[t][e] for e = 4*blockIdx.x + wave, tokens of block row blockIdx.y.
// FULL: H == NC * 512 (unguarded chunk loads, see gate_row).
template <int NC, bool FULL>
__global__ __launch_bounds__(256) void gate_gemv_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wg, int T,
    int H, int E, int tokens_per_block, void* __restrict__ logits,
    int logits_f32) {
  const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (e >= E) return;
  const int t0 = blockIdx.y * tokens_per_block;
  const int t1 = min(T, t0 + tokens_per_block);
  if (t1 - t0 == 1) gate_row<NC, true, FULL>(x, wg, t0, t1, H, E, e, logits, logits_f32);
  else gate_row<NC, false, FULL>(x, wg, t0, t1, H, E, e, logits, logits_f32);
}

// One wave per token; EPL experts per lane (EPL*64 >= E).
template <int EPL, int SCORE>
__global__ __launch_bounds__(256) void topk_kernel(
    const void* __restrict__ logits, int logits_f32, int T, SelectParams sp,
    float* __restrict__ w_f32, uint16_t* __restrict__ w_bf16,
    int32_t* __restrict__ ids) {
  __shared__ SelectLds<EPL> lds[4];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  float bv[EPL], lb[EPL], lg[EPL];
  load_bias<EPL>(sp, bv, lb);
  load_logits<EPL>(logits, logits_f32, t < T ? t : 0, sp.E, lg);
  int e;
  float w;
  select_token<EPL, SCORE>(sp, lg, bv, lb, lds[wave], e, w);
  const int kw = sp.k + sp.n_shared;
  if (lane >= sp.k) {
    // the pinned shared-expert suffix: ids E, E + 1, ..., weight 1
    e = sp.E + lane - sp.k;
    w = 1.0f;
  }
  if (t < T && lane < kw) {
    const size_t o = static_cast<size_t>(t) * kw + lane;
    ids[o] = e;
    w_bf16[o] = static_cast<uint16_t>(f32_to_bf16_bits(w));
    if (w_f32 != nullptr) w_f32[o] = w;
  }
}

}  // namespace lmoe

using namespace lmoe;

extern "C" int lmoe_router_gate(const void* x, const void* wg, int T, int H,
                                int E, void* logits, int logits_f32,
                                hipStream_t stream) {
  if (T < 0 || H <= 0 || E <= 0) return LMOE_ERR_ARG;
  if (H % 8 != 0 || H > kGateMaxChunks * 512) return LMOE_ERR_SHAPE;
  if (T == 0) return LMOE_OK;  // an empty batch: nothing read or written
  if (x == nullptr || wg == nullptr || logits == nullptr) return LMOE_ERR_ARG;
  if (T > 64 && H % DenseGateTile::BK == 0 && E % 8 == 0 &&
      ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(wg) |
        reinterpret_cast<uintptr_t>(logits)) & 15u) == 0) {
    // large token counts: one dense bf16 MFMA GEMM, logits = x . wg^T, with
    // 64 x 128 tiles and four stages of operands in flight per workgroup
    // (a few dozen tiles, each a long K chain: the chain's stages, not the
    // tile count, set the time)
    GemmArgs g{};
    g.a = static_cast<const uint16_t*>(x);
    g.w = static_cast<const uint16_t*>(wg);
    g.w_slot_stride = 0;
    g.N = E;
    g.K = H;
    g.M_dense = T;
    g.out = logits;
    g.out_f32 = logits_f32;
    const int grid = lds_gemm_grid((T + DenseGateTile::BM - 1) / DenseGateTile::BM,
                                   (E + DenseGateTile::BN - 1) / DenseGateTile::BN);
    hipLaunchKernelGGL((grouped_gemm_lds_kernel<kDense, DenseGateTile>), dim3(grid),
                       dim3(DenseGateTile::THREADS), 0, stream, g);
    LMOE_RETURN_LAUNCH();
  }
  if (T > 64) {
    // large token counts, other shapes: the 128 x 128 register-staged GEMM
    GemmArgs g{};
    g.a = static_cast<const uint16_t*>(x);
    g.w = static_cast<const uint16_t*>(wg);
    g.w_slot_stride = 0;
    g.N = E;
    g.K = H;
    g.M_dense = T;
    g.out = logits;
    g.out_f32 = logits_f32;
    hipLaunchKernelGGL(grouped_gemm_kernel<kDense>,
                       dim3((T + kBM - 1) / kBM, (E + kBN - 1) / kBN), dim3(256),
                       0, stream, g);
    LMOE_RETURN_LAUNCH();
  }
  // kGateTok tokens per block: blocks (bx, by) read the same weight rows
  // (from L2 after the first, and on one XCD when E / 4 is a multiple of 8)
  const int tpb = kGateTok;
  dim3 grid((E + 3) / 4, (T + tpb - 1) / tpb);
  const int nc = (H + 511) / 512;
#define LMOE_GATE1(NC, FULL)                                                                \
  hipLaunchKernelGGL((gate_gemv_kernel<NC, FULL>), grid, dim3(256), 0, stream,                \
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(wg), T, H, E, \
                     tpb, logits, logits_f32)
#define LMOE_GATE(NC)                              \
  do {                                             \
    if (H == (NC)*512) LMOE_GATE1(NC, true);       \
    else LMOE_GATE1(NC, false);                    \
  } while (0)
  if (nc <= 4) LMOE_GATE(4);
  else if (nc <= 8) LMOE_GATE(8);
  else LMOE_GATE(16);
#undef LMOE_GATE
#undef LMOE_GATE1
  LMOE_RETURN_LAUNCH();
}

extern "C" int lmoe_router_topk(const void* logits, int logits_f32, int T,
                                int E, int k, int n_shared, int scoring, const float* bias,
                                const float* logit_bias, int n_group, int topk_group, int renorm,
                                float routed_scale, float* w_f32,
                                uint16_t* w_bf16, int32_t* ids,
                                hipStream_t stream) {
  const int st = check_select(T, E, k, n_shared, scoring, n_group, topk_group);
  if (st != LMOE_OK) return st;
  if (T == 0) return LMOE_OK;  // an empty batch: nothing read or written
  if (logits == nullptr || w_bf16 == nullptr || ids == nullptr)
    return LMOE_ERR_ARG;
  const SelectParams sp =
      make_select(E, k, n_shared, scoring, bias, logit_bias, n_group, topk_group, renorm,
                  routed_scale);
  const dim3 grid((T + 3) / 4);
#define LMOE_TK(EPL, S) \
  hipLaunchKernelGGL((topk_kernel<EPL, S>), grid, dim3(256), 0, stream, logits, logits_f32, T, sp, w_f32, w_bf16, ids)
#define LMOE_TK_E(S)                 \
  do {                               \
    if (E <= 64) LMOE_TK(1, S);      \
    else if (E <= 128) LMOE_TK(2, S); \
    else if (E <= 256) LMOE_TK(4, S); \
    else LMOE_TK(8, S);              \
  } while (0)
  if (scoring == LMOE_SCORING_SOFTMAX) LMOE_TK_E(LMOE_SCORING_SOFTMAX);
  else LMOE_TK_E(LMOE_SCORING_SIGMOID);
#undef LMOE_TK_E
#undef LMOE_TK
  LMOE_RETURN_LAUNCH();
}

extern "C" int lmoe_router_topk_permute(
    const void* logits, int logits_f32, int T, int E, int k, int n_shared, int scoring,
    const float* bias, const float* logit_bias, int n_group, int topk_group, int renorm,
    float routed_scale, float* w_f32, uint16_t* w_bf16,
    int32_t* ids, const int32_t* log2phy, int n_log2phy, int n_slots, int skip_unmapped,
    int block_m, int32_t* counts, int32_t* offsets, int32_t* sorted_pairs, int32_t* row_idx,
    int32_t* active, int32_t* tile_off, int32_t* meta, hipStream_t stream) {
  int st = check_select(T, E, k, n_shared, scoring, n_group, topk_group);
  if (st != LMOE_OK) return st;
  if (n_slots <= 0 || block_m <= 0) return LMOE_ERR_ARG;
  if (log2phy != nullptr && n_log2phy <= 0) return LMOE_ERR_ARG;
  // one block: a token per wave, the whole permutation in LDS
  if (T > kFusedTopkTokens || E > 256 || n_slots > kMaxSlots) return LMOE_ERR_SHAPE;
  // an empty batch still builds its (empty) permutation
  if (T == 0)
    return lmoe_permute(nullptr, 0, log2phy, n_log2phy, n_slots, skip_unmapped, block_m, counts,
                        offsets, sorted_pairs, row_idx, active, tile_off, meta, nullptr, 0,
                        stream);
  if (logits == nullptr || w_bf16 == nullptr || ids == nullptr || counts == nullptr ||
      offsets == nullptr || sorted_pairs == nullptr || row_idx == nullptr ||
      active == nullptr || tile_off == nullptr || meta == nullptr)
    return LMOE_ERR_ARG;
  RouterPermuteArgs ra{};
  ra.T = T;
  ra.logits = const_cast<void*>(logits);
  ra.logits_f32 = logits_f32;
  ra.sp = make_select(E, k, n_shared, scoring, bias, logit_bias, n_group, topk_group, renorm,
                      routed_scale);
  ra.w_f32 = w_f32;
  ra.w_bf16 = w_bf16;
  ra.ids = ids;
  ra.log2phy = log2phy;
  ra.n_log2phy = n_log2phy;
  ra.n_slots = n_slots;
  ra.skip = skip_unmapped ? 1 : 0;
  ra.block_m = block_m;
  ra.counts = counts;
  ra.offsets = offsets;
  ra.sorted_pairs = sorted_pairs;
  ra.row_idx = row_idx;
  ra.active = active;
  ra.tile_off = tile_off;
  ra.meta = meta;
  return scoring == LMOE_SCORING_SOFTMAX ? launch_topk_permute<LMOE_SCORING_SOFTMAX>(ra, stream)
                                         : launch_topk_permute<LMOE_SCORING_SIGMOID>(ra, stream);
}

extern "C" int lmoe_router_gate_topk_pairs(
    const void* x, const void* wg, int H, int E, void* logits, int logits_f32, int k,
    int n_shared, int scoring, const float* bias, const float* logit_bias, int n_group,
    int topk_group, int renorm, float routed_scale, float* w_f32, uint16_t* w_bf16, int32_t* ids,
    const int32_t* log2phy, int n_log2phy, int n_slots, int skip_unmapped, int32_t* sorted_pairs,
    int32_t* row_idx, int32_t* active, int32_t* meta, int32_t* sync, hipStream_t stream) {
  if (H <= 0) return LMOE_ERR_ARG;
  int st = check_select(1, E, k, n_shared, scoring, n_group, topk_group);
  if (st != LMOE_OK) return st;
  if (n_slots <= 0) return LMOE_ERR_ARG;
  if (log2phy != nullptr && n_log2phy <= 0) return LMOE_ERR_ARG;
  if (H % 8 != 0 || H > kGateMaxChunks * 512) return LMOE_ERR_SHAPE;
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(wg)) & 15u)
    return LMOE_ERR_SHAPE;
  if (E > 256 || n_slots > kMaxSlots) return LMOE_ERR_SHAPE;
  if (x == nullptr || wg == nullptr || logits == nullptr || w_bf16 == nullptr || ids == nullptr ||
      sorted_pairs == nullptr || row_idx == nullptr || active == nullptr || meta == nullptr ||
      sync == nullptr)
    return LMOE_ERR_ARG;
  if (reinterpret_cast<uintptr_t>(sync) & 7u) return LMOE_ERR_SHAPE;  // u64 tagged words
  RouterPermuteArgs ra{};
  ra.x = x;
  ra.wg = wg;
  ra.H = H;
  ra.sync = sync;
  ra.T = 1;
  ra.logits = logits;
  ra.logits_f32 = logits_f32;
  ra.sp = make_select(E, k, n_shared, scoring, bias, logit_bias, n_group, topk_group, renorm,
                      routed_scale);
  ra.w_f32 = w_f32;
  ra.w_bf16 = w_bf16;
  ra.ids = ids;
  ra.log2phy = log2phy;
  ra.n_log2phy = n_log2phy;
  ra.n_slots = n_slots;
  ra.skip = skip_unmapped ? 1 : 0;
  ra.block_m = 1;  // no tile table
  ra.sorted_pairs = sorted_pairs;
  ra.row_idx = row_idx;
  ra.active = active;
  ra.meta = meta;
  ra.pairs = true;
  return scoring == LMOE_SCORING_SOFTMAX
             ? launch_gate_topk_permute<LMOE_SCORING_SOFTMAX>(ra, stream)
             : launch_gate_topk_permute<LMOE_SCORING_SIGMOID>(ra, stream);
}

extern "C" int lmoe_router_gate_topk_permute(
    const void* x, const void* wg, int T, int H, int E, void* logits, int logits_f32, int k,
    int n_shared, int scoring, const float* bias, const float* logit_bias, int n_group,
    int topk_group, int renorm, float routed_scale,
    float* w_f32, uint16_t* w_bf16, int32_t* ids, const int32_t* log2phy, int n_log2phy,
    int n_slots, int skip_unmapped, int block_m, int32_t* counts, int32_t* offsets,
    int32_t* sorted_pairs, int32_t* row_idx, int32_t* active, int32_t* tile_off, int32_t* meta,
    int32_t* sync, hipStream_t stream) {
  if (T < 0 || H <= 0) return LMOE_ERR_ARG;
  int st = check_select(T, E, k, n_shared, scoring, n_group, topk_group);
  if (st != LMOE_OK) return st;
  if (n_slots <= 0 || block_m <= 0) return LMOE_ERR_ARG;
  if (log2phy != nullptr && n_log2phy <= 0) return LMOE_ERR_ARG;
  if (H % 8 != 0 || H > kGateMaxChunks * 512) return LMOE_ERR_SHAPE;
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(wg)) & 15u)
    return LMOE_ERR_SHAPE;
  // the last block holds the whole selection and permutation
  if (T > kFusedTopkTokens || E > 256 || n_slots > kMaxSlots) return LMOE_ERR_SHAPE;
  // rows past 2048 columns: one token only (the several-token forms of the
  // long-row gate spill ~810 bytes per lane, and two launches are faster
  // above one token anyway)
  if (T > 1 && H > kGateShortChunks * 512) return LMOE_ERR_SHAPE;
  // an empty batch still builds its (empty) permutation
  if (T == 0)
    return lmoe_permute(nullptr, 0, log2phy, n_log2phy, n_slots, skip_unmapped, block_m, counts,
                        offsets, sorted_pairs, row_idx, active, tile_off, meta, nullptr, 0,
                        stream);
  if (x == nullptr || wg == nullptr || logits == nullptr || w_bf16 == nullptr || ids == nullptr ||
      counts == nullptr || offsets == nullptr || sorted_pairs == nullptr || row_idx == nullptr ||
      active == nullptr || tile_off == nullptr || meta == nullptr || sync == nullptr)
    return LMOE_ERR_ARG;
  if (reinterpret_cast<uintptr_t>(sync) & 7u) return LMOE_ERR_SHAPE;  // u64 tagged words
  RouterPermuteArgs ra{};
  ra.x = x;
  ra.wg = wg;
  ra.H = H;
  ra.sync = sync;
  ra.T = T;
  ra.logits = logits;
  ra.logits_f32 = logits_f32;
  ra.sp = make_select(E, k, n_shared, scoring, bias, logit_bias, n_group, topk_group, renorm,
                      routed_scale);
  ra.w_f32 = w_f32;
  ra.w_bf16 = w_bf16;
  ra.ids = ids;
  ra.log2phy = log2phy;
  ra.n_log2phy = n_log2phy;
  ra.n_slots = n_slots;
  ra.skip = skip_unmapped ? 1 : 0;
  ra.block_m = block_m;
  ra.counts = counts;
  ra.offsets = offsets;
  ra.sorted_pairs = sorted_pairs;
  ra.row_idx = row_idx;
  ra.active = active;
  ra.tile_off = tile_off;
  ra.meta = meta;
  return scoring == LMOE_SCORING_SOFTMAX
             ? launch_gate_topk_permute<LMOE_SCORING_SOFTMAX>(ra, stream)
             : launch_gate_topk_permute<LMOE_SCORING_SIGMOID>(ra, stream);
}
