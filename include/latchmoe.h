/*
 * latchmoe.h — C ABI of liblatchmoe_hip.so, the MI355X (gfx950) kernels of
 * the slot-indexed fused-MoE hot path.
 *
 * Every entry point is `extern "C"`, takes plain device pointers, sizes and a
 * hipStream_t, never throws, allocates nothing, and returns an int status:
 *   0                      success
 *   1 .. 999               a hipError_t from the launch or copy
 *   LMOE_ERR_* (>= 1000)   an argument error detected on the host before any
 *                          device work was queued
 * lmoe_status_string() names a status.  All launches are asynchronous on the
 * given stream and are legal inside hipStreamBeginCapture/EndCapture (no
 * allocation, no host synchronisation, no memset node).
 *
 * An empty batch (T == 0 tokens, or n_pairs == 0) is legal everywhere: the
 * call checks its sizes, then returns 0 without reading its token-sized
 * operands, which may be null (an empty device tensor has no address).  The
 * entry points that build a permutation still write it, empty (zero counts,
 * no active slot), so a caller never reads the previous batch's.
 *
 * Tensor conventions (row-major, element types in brackets):
 *   x         [T, H]        bf16   hidden states (T tokens)
 *   logits    [T, E]        bf16 or f32
 *   ids       [T, k]        i32    logical expert ids, flat pair p = t*k + j
 *   w13_slots [P, 2I, H]    bf16   slot bank, rows 0..I-1 gate, I..2I-1 up
 *   w2_slots  [P, H, I]     bf16   slot bank, down projection
 *   log2phy   [E_total]     i32    logical expert -> physical slot, -1 = none
 *
 * Reference interfaces replaced (paths relative to the LatchMoE repository):
 *   lmoe_router_gate   gate(hidden) in ops/fused_moe/moe_router_op.py:228-231
 *   lmoe_router_topk   select_experts (moe_router_op.py:108-124) with the
 *                      renorm contract of patches/patch_fused_moe.py:597-632
 *   lmoe_router_topk_permute  select_experts then remap + init routing in
 *                      one launch (decode with a final slot table)
 *   lmoe_router_gate_topk_permute  gate, select_experts, remap + init
 *                      routing in one launch (same decode case)
 *   lmoe_permute       log2phy remap moe_offload/slot_mapping.py:116-140 and
 *                      npu_moe_init_routing_v2, patch_fused_moe.py:668-701
 *                      (stable sort by slot, expanded_row_idx, count histogram)
 *   lmoe_gather_rows   expanded_x output of the same init-routing call
 *   lmoe_grouped_mlp   npu_grouped_matmul x2 + npu_swiglu (_apply_mlp,
 *                      patch_fused_moe.py:3772-3774, hooks :4249-4302)
 *   lmoe_combine       npu_moe_token_unpermute, patch_fused_moe.py:3363-3366,
 *                      and the single native combine of :3342-3379
 *   lmoe_fused_moe_decode  GMM1+swiglu+GMM2+unpermute of the decode
 *                      fused_experts call (patch_fused_moe.py:3946-4009)
 *   lmoe_down_combine  GMM2 + unpermute of the same call
 *   lmoe_stage_copy    TransferEngine.load_many_async H2D batch + ready event,
 *                      moe_offload/transfer_engine.py:139-187, 205-228
 */
#ifndef LATCHMOE_H
#define LATCHMOE_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LMOE_ABI_VERSION 8

enum { LMOE_SKIP_KEEP_ROWS = 2 }; /* lmoe_permute skip_unmapped mode */

/* Device status words (lmoe_device_flags). */
enum {
  LMOE_FLAG_UNPLACED = 0,        /* pairs a masked combine dropped: no pass
                                    placed them (an id outside every table) */
  LMOE_FLAG_ROUTER_TIMEOUT = 1,  /* one-launch router waits that gave up: the
                                    routing of that step is invalid */
  LMOE_FLAG_COUNT = 4
};

enum {
  LMOE_OK = 0,
  LMOE_ERR_ARG = 1000,         /* null pointer or negative size */
  LMOE_ERR_SHAPE = 1001,       /* a dimension the kernels do not support */
  LMOE_ERR_WORKSPACE = 1002,   /* workspace smaller than required */
  LMOE_ERR_UNSUPPORTED = 1003  /* an option combination with no kernel */
};

/* Scoring functions of lmoe_router_topk. */
enum { LMOE_SCORING_SOFTMAX = 0, LMOE_SCORING_SIGMOID = 1 };

/* Kernel-path selectors of lmoe_grouped_mlp. */
enum { LMOE_PATH_AUTO = 0, LMOE_PATH_GEMV = 1, LMOE_PATH_MFMA = 2 };

/* Slots of the meta[] output of lmoe_permute. */
enum {
  LMOE_META_ACTIVE = 0,  /* number of slots with at least one pair          */
  LMOE_META_PAIRS = 1,   /* number of pairs placed in the sorted order      */
  LMOE_META_ERRORS = 2,  /* pairs dropped because their id did not map      */
  LMOE_META_TILES = 3,   /* sum over slots of ceil(count / block_m)         */
  LMOE_META_GEN = 4,     /* builds of this permutation so far (+1 per build) */
  LMOE_META_ROUTER_TIMEOUT = 6,  /* lmoe_router_gate_topk_permute: 1 if the
                                    selection gave up waiting for a logit
                                    (sticky: the library never clears it; the
                                    same event adds to LMOE_FLAG_ROUTER_TIMEOUT) */
  LMOE_META_COUNT = 64           /* int32 words; the others are reserved */
};

/* int32 words of the sync buffer of lmoe_router_gate_topk_permute: [0] the
 * arrival count, from [64] the tagged logit words (u64, T x E <= 16 x 256). */
enum { LMOE_ROUTER_SYNC_WORDS = 64 + 2 * 16 * 256 };

const char* lmoe_status_string(int status);
int lmoe_abi_version(void);

/* Device status of the current device, summed over the library's kernels:
 * flags[LMOE_FLAG_COUNT] receives the words (LMOE_FLAG_UNPLACED,
 * LMOE_FLAG_ROUTER_TIMEOUT); with clear, nonzero words are reset to 0.
 * Synchronizes stream (a host check point: call it where the host already
 * waits, e.g. beside the staging op's read of the routed ids).  A nonzero
 * word means an output since the last clear is invalid.  No counterpart in
 * the reference, whose host code sees every routed id before the experts
 * run; this library's captured and device-planned paths do not. */
int lmoe_device_flags(int32_t* flags, int clear, hipStream_t stream);

/* Gate linear: logits[t][e] = sum_h x[t][h] * wg[e][h], f32 accumulation,
 * stored as bf16 (round to nearest even) or f32.  Replaces the gate matmul of
 * moe_router_op.py:228-231. */
int lmoe_router_gate(const void* x, const void* wg, int T, int H, int E,
                     void* logits, int logits_f32, hipStream_t stream);

/* Expert selection.  l = logits + logit_bias (logit_bias may be NULL: the
 * router gate's linear bias, one f32 add before scoring).
 * scoring = LMOE_SCORING_SOFTMAX: p = f32 softmax over E of l.
 * scoring = LMOE_SCORING_SIGMOID: p = sigmoid(l).  The selection score is
 * p + bias (bias = e_score_correction_bias, may be NULL: used for selection
 * only, as vLLM's grouped_topk and CANN's gating top-k use it); with
 * sigmoid and n_group > 1, n_group contiguous groups ranked by the sum of
 * their two largest selection scores, the topk_group best groups kept; the
 * k largest selection scores (inside the kept groups); weights = p.
 * Ties break toward the lower expert (or group) id.  Output order is the
 * selection order (descending score).  If renorm, w /= max(sum(w), FLT_EPSILON)
 * (sum in selection order); then w *= routed_scale.  w_f32 may be NULL.
 * Rows of w / ids are k + n_shared wide: columns k .. k + n_shared - 1 hold
 * the pinned shared-expert suffix, ids E, E + 1, ... with weight 1 (outside
 * the renormalisation), the mix-placement suffix that select_experts appends
 * (patch_fused_moe.py:4697-4727; checked as ids [E, E + S) at :2338-2370).
 * E <= 512, k + n_shared <= 16, n_group <= 64.  Replaces select_experts
 * (moe_router_op.py:108-124, patch_fused_moe.py:597-632). */
int lmoe_router_topk(const void* logits, int logits_f32, int T, int E, int k,
                     int n_shared, int scoring, const float* bias,
                     const float* logit_bias, int n_group,
                     int topk_group, int renorm, float routed_scale,
                     float* w_f32, uint16_t* w_bf16, int32_t* ids,
                     hipStream_t stream);

/* lmoe_router_topk followed by lmoe_permute (same arguments, same outputs,
 * bit for bit) in one launch, for a slot table that is final before the
 * router runs: the decode replay after staging, where the reference calls
 * select_experts (moe_router_op.py:108-124) and then remap + init routing
 * (slot_mapping.py:116-140, patch_fused_moe.py:668-701) back to back.
 * Returns LMOE_ERR_SHAPE when T > 16, E > 256 or n_slots > 8192 (then use
 * the two calls). */
int lmoe_router_topk_permute(const void* logits, int logits_f32, int T, int E,
                             int k, int n_shared, int scoring, const float* bias,
                             const float* logit_bias,
                             int n_group, int topk_group, int renorm,
                             float routed_scale, float* w_f32,
                             uint16_t* w_bf16, int32_t* ids,
                             const int32_t* log2phy, int n_log2phy,
                             int n_slots, int skip_unmapped, int block_m,
                             int32_t* counts, int32_t* offsets,
                             int32_t* sorted_pairs, int32_t* row_idx,
                             int32_t* active, int32_t* tile_off,
                             int32_t* meta, hipStream_t stream);

/* lmoe_router_gate, lmoe_router_topk and lmoe_permute (same arguments, same
 * outputs, bit for bit; logits is still written, without the logit bias,
 * as lmoe_router_gate writes it) in one launch, for the same
 * final-table decode case as lmoe_router_topk_permute: gate(hidden)
 * (moe_router_op.py:228-231), select_experts (:108-124) and remap + init
 * routing (slot_mapping.py:116-140, patch_fused_moe.py:668-701).  The gate
 * workgroups store their logits, also as tagged words in sync (the logit |
 * the build number this launch makes, meta[LMOE_META_GEN] + 1, << 32, by
 * agent-scope atomic stores: no cache write-back or invalidate), and count
 * themselves in on sync[0]; the last one to arrive resets sync[0] to 0,
 * reads the words back (again where a tag is not yet this launch's; a wait
 * that gives up sets meta[LMOE_META_ROUTER_TIMEOUT], the result is then
 * undefined) and runs the selection and the permutation.  sync is
 * LMOE_ROUTER_SYNC_WORDS int32, 8-byte aligned, zero before the first call;
 * it serves one permutation (one meta), and calls that may run concurrently
 * need separate sync buffers.
 * Returns LMOE_ERR_SHAPE when T > 16, T > 1 with H > 2048 (long rows: one
 * token only), E > 256, n_slots > 8192, H % 8 != 0,
 * H > 8192, x / wg are not 16-byte aligned or sync is not 8-byte aligned
 * (then use the separate calls). */
int lmoe_router_gate_topk_permute(const void* x, const void* wg, int T, int H,
                                  int E, void* logits, int logits_f32, int k,
                                  int n_shared, int scoring, const float* bias,
                                  const float* logit_bias, int n_group,
                                  int topk_group, int renorm,
                                  float routed_scale, float* w_f32,
                                  uint16_t* w_bf16, int32_t* ids,
                                  const int32_t* log2phy, int n_log2phy,
                                  int n_slots, int skip_unmapped, int block_m,
                                  int32_t* counts, int32_t* offsets,
                                  int32_t* sorted_pairs, int32_t* row_idx,
                                  int32_t* active, int32_t* tile_off,
                                  int32_t* meta, int32_t* sync,
                                  hipStream_t stream);

/* One token (T == 1): lmoe_router_gate_topk_permute's gate and selection
 * (the same logits, w_f32, w_bf16 and ids, bit for bit, and the same sync
 * and meta protocol), then the token's pairs in pair order instead of the
 * slot-sorted permutation: the placed pairs take positions 0, 1, ... in
 * pair order, active[pos] = the slot of the pos-th placed pair,
 * sorted_pairs[pos] = that pair, row_idx[j] = pair j's position or -1, and
 * active[a] = -1 for a from the placed count to n_slots - 1; meta[ACTIVE]
 * = meta[PAIRS] = the placed pairs, meta[ERRORS] as lmoe_permute counts
 * them, GEN advanced; counts, offsets and tile_off are not touched.  A pair
 * whose id maps to no slot is placed nowhere (skip_unmapped as in
 * lmoe_permute).  With distinct slots (a router-fed token) this is a
 * permutation of the one-token kernels' form (every slot serves one pair,
 * position a is active rank a): lmoe_fused_moe_decode with distinct_slots
 * gives the same bits from it as from the sorted permutation.  It saves the
 * sort at the end of the router's dependent chain.  No counterpart in the
 * reference, whose permutation is always slot-sorted
 * (patch_fused_moe.py:668-701); the gate and selection replace
 * moe_router_op.py:108-124, 228-231.  LMOE_ERR_SHAPE as
 * lmoe_router_gate_topk_permute with T = 1. */
int lmoe_router_gate_topk_pairs(const void* x, const void* wg, int H, int E,
                                void* logits, int logits_f32, int k,
                                int n_shared, int scoring, const float* bias,
                                const float* logit_bias, int n_group,
                                int topk_group, int renorm, float routed_scale,
                                float* w_f32, uint16_t* w_bf16, int32_t* ids,
                                const int32_t* log2phy, int n_log2phy,
                                int n_slots, int skip_unmapped,
                                int32_t* sorted_pairs, int32_t* row_idx,
                                int32_t* active, int32_t* meta, int32_t* sync,
                                hipStream_t stream);

/* Bytes of device workspace lmoe_permute needs for n_pairs pairs, n_slots. */
size_t lmoe_permute_workspace_bytes(int n_pairs, int n_slots);

/* Slot remap, count histogram and stable counting sort of the flat pairs.
 * slot(p) = log2phy ? log2phy[ids[p]] : ids[p].  A pair whose id is outside
 * [0, n_log2phy) or whose slot is outside [0, n_slots) is left out of the
 * sorted order; it is counted in meta[LMOE_META_ERRORS] unless skip_unmapped
 * is set and the slot is -1 or the id lies outside the table (a pair of
 * another wave).  skip_unmapped = 2 (LMOE_SKIP_KEEP_ROWS) skips as 1 does and
 * leaves row_idx[p] untouched for every pair it does not place: a layer run
 * in several passes over one row_idx (the first pass with 0 or 1, the later
 * ones with 2) ends with row_idx[p] >= 0 exactly for the pairs some pass
 * placed, the row mask of its single combine.  Other values: LMOE_ERR_ARG.
 * Outputs: counts[s]; offsets[s] = exclusive prefix of counts (offsets[P] =
 * placed pairs); sorted_pairs[offsets[s] + r] = the r-th pair of slot s in
 * flat order; row_idx[p] = sorted position of pair p or -1; active[a] = a-th
 * slot with count > 0 in launch order, -1 for a >= meta[LMOE_META_ACTIVE]:
 * first the heavy slots (count >= 16 and 16 * count >= placed pairs; at most
 * 16) by descending count, ties by ascending slot, then the other slots with
 * count > 0 in ascending slot order (the decode kernels give active rank a
 * grid row a, so a hot slot starts first instead of ending the kernel late;
 * no output depends on the order);
 * tile_off[s] = sum over s' < s of
 * ceil(counts[s'] / block_m); meta[LMOE_META_COUNT] (ACTIVE, PAIRS, ERRORS,
 * TILES; GEN advanced; the other words are not written).
 * Replaces slot_mapping.py:116-140 + npu_moe_init_routing_v2
 * (patch_fused_moe.py:668-701: expert_capacity=-1, drop_pad_mode=0,
 * expert_tokens_num_type=1). */
int lmoe_permute(const int32_t* ids, int n_pairs, const int32_t* log2phy,
                 int n_log2phy, int n_slots, int skip_unmapped, int block_m,
                 int32_t* counts, int32_t* offsets, int32_t* sorted_pairs,
                 int32_t* row_idx, int32_t* active, int32_t* tile_off,
                 int32_t* meta, void* workspace, size_t workspace_bytes,
                 hipStream_t stream);

/* The two builds of a decode layer whose routed experts exceed its bank, in
 * one launch: table a (the bank, skip_unmapped = 1) and table b (the
 * overflow stage buffer, LMOE_SKIP_KEEP_ROWS) over the same ids, each into
 * its own outputs (counts_x .. meta_x, as lmoe_permute writes them), row_idx
 * shared.  Every output equals lmoe_permute(a, 1) followed by
 * lmoe_permute(b, 2) on the same row_idx.  Both tables required; n_pairs <=
 * 1024 (one workgroup per table; larger builds: LMOE_ERR_SHAPE, run the two
 * lmoe_permute calls).  No workspace.  No single counterpart in the
 * reference, which remaps and routes one expert table per pass
 * (slot_mapping.py:116-140 + patch_fused_moe.py:668-701 per wave). */
int lmoe_permute_two_tables(
    const int32_t* ids, int n_pairs, int block_m, int32_t* row_idx,
    const int32_t* log2phy_a, int n_log2phy_a, int n_slots_a, int32_t* counts_a,
    int32_t* offsets_a, int32_t* sorted_pairs_a, int32_t* active_a,
    int32_t* tile_off_a, int32_t* meta_a, const int32_t* log2phy_b,
    int n_log2phy_b, int n_slots_b, int32_t* counts_b, int32_t* offsets_b,
    int32_t* sorted_pairs_b, int32_t* active_b, int32_t* tile_off_b,
    int32_t* meta_b, hipStream_t stream);

/* expanded_x: x_sorted[pos] = x[sorted_pairs[pos] / k] for pos < n_pairs
 * (positions past meta[LMOE_META_PAIRS] are left untouched). */
int lmoe_gather_rows(const void* x, int H, int k, const int32_t* sorted_pairs,
                     const int32_t* meta, int n_pairs, void* x_sorted,
                     hipStream_t stream);

/* Grouped SwiGLU MLP over the permuted pairs, reading weights only through
 * the slot bank.  For each placed pair p in slot s (token t = p / k):
 *   act[pos]  = silu(W13_s[0:I] x_t) * (W13_s[I:2I] x_t)    bf16, f32 math
 *   y[p]      = W2_s act[pos]                                 bf16, f32 acc.
 * act is a [n_pairs, I] bf16 workspace in sorted order; y is [T*k, H] bf16
 * indexed by flat pair (rows of unplaced pairs are left untouched).
 * path = LMOE_PATH_GEMV (weight-streaming, small slot groups),
 * LMOE_PATH_MFMA (bf16 MFMA tiles, block_m must equal the block_m given to
 * lmoe_permute: 320 = one workgroup per CU with equal shares of 32-column
 * blocks of 320-row tiles, 256 = a grid of 256 x 256 tiles, 128 = 128 x 128
 * tiles; 320 needs H % 64 == 0) or
 * LMOE_PATH_AUTO.  H % 8 == 0, I % 64 == 0.  Every block_m gives the same
 * bits. */
int lmoe_grouped_mlp(const void* x, int T, int H, int I, int k,
                     const void* w13_slots, const void* w2_slots, int n_slots,
                     const int32_t* offsets, const int32_t* sorted_pairs,
                     const int32_t* active, const int32_t* tile_off,
                     const int32_t* meta, int n_pairs, int block_m, int path,
                     void* act, void* y, hipStream_t stream);

/* The two halves of lmoe_grouped_mlp, callable on their own (same argument
 * meaning): GMM1 + SwiGLU into act, and GMM2 from act into y.  Replace the
 * separate npu_grouped_matmul + npu_swiglu and npu_grouped_matmul calls of
 * _apply_mlp (patch_fused_moe.py:3772-3774). */
int lmoe_gateup_silu(const void* x, int T, int H, int I, int k,
                     const void* w13_slots, int n_slots, const int32_t* offsets,
                     const int32_t* sorted_pairs, const int32_t* active,
                     const int32_t* tile_off, const int32_t* meta, int n_pairs,
                     int block_m, int path, void* act, hipStream_t stream);
int lmoe_down(const void* act, int H, int I, const void* w2_slots, int n_slots,
              const int32_t* offsets, const int32_t* sorted_pairs,
              const int32_t* active, const int32_t* tile_off,
              const int32_t* meta, int n_pairs, int block_m, int path, void* y,
              hipStream_t stream);

/* Both decode passes of a layer whose routed experts exceed its bank, in one
 * gate_up and one down launch (the GEMV path): pass a is the bank (w13_a,
 * w2_a, n_slots_a and its permutation, built with skip_unmapped), pass b the
 * overflow stage buffer (w13_b, w2_b, n_slots_b and its permutation, built
 * with skip mode 2 over the same ids).  act is one [n_pairs, I] bf16
 * workspace: pass a's rows at its sorted positions, pass b's after pass a's
 * meta_a[LMOE_META_PAIRS] placed pairs.  y is [T*k, H] indexed by flat pair,
 * as lmoe_grouped_mlp writes it; every value has the bits of
 * lmoe_grouped_mlp(path GEMV) over each pass.  The two tables must map
 * disjoint experts (an overflow expert maps to -1 in the bank table): a pair
 * both place is written by both passes in no set order, and pass b's rows
 * that would fall past act's n_pairs rows are not computed.  Rows up to 4096
 * columns (H <= 4096, I <= 4096), act and w2 16-byte aligned; else
 * LMOE_ERR_SHAPE (run the passes one by one).  No counterpart in the reference, which executes a
 * working set past the slot count as bounded pair waves one after the other
 * (moe_offload/runtime.py:1215-1232); here the decode overflow's two passes
 * share their launches. */
int lmoe_decode_mlp_two_passes(const void* x, int T, int H, int I, int k,
                               const void* w13_a, const void* w2_a, int n_slots_a,
                               const int32_t* offsets_a, const int32_t* sorted_pairs_a,
                               const int32_t* active_a, const int32_t* meta_a,
                               const void* w13_b, const void* w2_b, int n_slots_b,
                               const int32_t* offsets_b, const int32_t* sorted_pairs_b,
                               const int32_t* active_b, int n_pairs, void* act, void* y,
                               hipStream_t stream);

/* Weighted combine: out[t] = sum_{j<k} w[t][j] * y[t*k+j], f32 accumulation
 * in j order, one rounding to bf16.  y is [T*k, H] bf16 indexed by flat pair
 * (as lmoe_grouped_mlp writes it, over one or several waves); row_idx (may be
 * NULL) masks pairs: a pair with row_idx[p] < 0 contributes nothing.  add (may be NULL) is a
 * [T, H] bf16 term added before rounding (resident shared expert).  Replaces
 * npu_moe_token_unpermute (patch_fused_moe.py:3363-3366, semantics
 * phase_split.py:1649-1656) and the single native combine (:3342-3379). */
int lmoe_combine(const void* y, const int32_t* row_idx, const uint16_t* w,
                 int T, int k, int H, const void* add, void* out,
                 hipStream_t stream);

/* The second half of lmoe_fused_moe_decode on its own: down GEMV from act
 * (sorted order) fused with the weighted combine into out (same argument
 * meaning).  Replaces npu_grouped_matmul GMM2 + npu_moe_token_unpermute of
 * the decode call (patch_fused_moe.py:3772-3774, :3363-3366). */
int lmoe_down_combine(const void* act, int T, int H, int I, int k,
                      const void* w2_slots, int n_slots, const uint16_t* w,
                      const int32_t* offsets, const int32_t* row_idx,
                      const int32_t* active, const int32_t* meta,
                      const void* add, void* out, hipStream_t stream);

/* Decode MoE for small pair counts:
 *   out[t] = (add ? add[t] : 0) + sum_j w[t][j] * W2_s(t,j) act[pos(t,j)].
 * gate_up GEMV + SiLU*mul into act (sorted order), then either the down GEMV
 * fused with the weighted combine (each workgroup owns a few output columns
 * of every token; two launches, used for T*k <= 16 or y == NULL), or, for
 * more pairs with a y workspace ([T*k, H] bf16, flat pair order on return),
 * the down GEMV per (row block, slot) into y and the combine (three
 * launches: no workgroup walks the slots in turn).  Both give the same out
 * bit for bit.  Each slot's weights are read once however many tokens chose
 * it.  distinct_slots != 0 promises that no slot serves two pairs of one
 * token (true for ids from the routers, which pick distinct experts, through
 * a slot table, which maps distinct experts to distinct slots); with one
 * token it selects kernels that take active rank a as sorted position a.
 * Ids from elsewhere pass 0 (the general kernels; same bits when the
 * promise holds).  Needs T*k <= 1024, H % 8 == 0, I % 64 == 0, I <= 4096,
 * H <= 8192; x, slot banks, act and y 16-byte aligned.  Permutation arrays
 * as produced by lmoe_permute; with one token and distinct_slots, also the
 * pair-order form of lmoe_router_gate_topk_pairs (its one-token kernels
 * read only active[] and row_idx[], not offsets or sorted_pairs), with the
 * same out bit for bit. */
int lmoe_fused_moe_decode(const void* x, int T, int H, int I, int k,
                          const void* w13_slots, const void* w2_slots,
                          int n_slots, const uint16_t* w,
                          const int32_t* offsets, const int32_t* sorted_pairs,
                          const int32_t* row_idx, const int32_t* active,
                          const int32_t* meta, const void* add, void* act,
                          void* y, void* out, int distinct_slots,
                          hipStream_t stream);

/* Size of the per-device scratch array of lmoe_fused_moe_decode_noalloc. */
#define LMOE_NOALLOC_SCRATCH_BYTES (8u << 20)

/* lmoe_fused_moe_decode (same arguments, same out bit for bit) without the
 * act / y workspaces: they live in a library-owned __device__ array of
 * LMOE_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends.  No
 * counterpart in the reference: for callers that cannot allocate (code under
 * hipGraph capture, serving loops or harnesses that forbid hipMalloc).  The
 * call allocates nothing.  Limits, both checked before any device work:
 * T*k <= 1024 (the decode body's, else LMOE_ERR_SHAPE) and
 * align256(T*k*I*2) + align256(T*k*H*2) <= LMOE_NOALLOC_SCRATCH_BYTES (else
 * LMOE_ERR_WORKSPACE), i.e. T <= min(1024 / k, what the array holds):
 * Qwen3 shape (H 2048, I 768, k 8) T <= 128 (the array alone would hold
 * 186), DeepSeek-V3 expert shape with the shared pair (H 7168, I 2048,
 * k 9) T <= 50.  Every call on
 * one GPU shares that GPU's array: calls that may overlap on one GPU race and
 * must be ordered by the caller. */
int lmoe_fused_moe_decode_noalloc(const void* x, int T, int H, int I, int k,
                                  const void* w13_slots, const void* w2_slots,
                                  int n_slots, const uint16_t* w,
                                  const int32_t* offsets,
                                  const int32_t* sorted_pairs,
                                  const int32_t* row_idx, const int32_t* active,
                                  const int32_t* meta, const void* add,
                                  void* out, int distinct_slots,
                                  hipStream_t stream);

/* Batched host->device (or device->device) expert copies on a transfer
 * stream: optionally wait on wait_event, then for i < n copy bytes[i] from
 * src[i] to dst[i] with hipMemcpyAsync, then record done_event (may be NULL).
 * Replaces TransferEngine.load_many_async (transfer_engine.py:139-187) with
 * the contiguous-run batching of :205-228 done by the caller. */
int lmoe_stage_copy(void* const* dst, const void* const* src,
                    const size_t* bytes, int n, hipStream_t transfer_stream,
                    hipEvent_t wait_event, hipEvent_t done_event);

/* Batched expert copies by a gather-copy kernel on the transfer stream:
 * optionally wait on wait_event, then for i < n copy bytes[i] from src[i] to
 * dst[i] (sources: page-locked host memory mapped for the device at the same
 * address, or device memory; destinations: device memory), then
 * table[idx[p]] = val[p] for p < n_tab (fill != 0: every other entry of the
 * n_table-entry table becomes -1), then record done_event (may be NULL).
 * One launch per 32 copies; the table rides with the last one (fill: at
 * most 128 pairs).  Every range
 * is checked before anything is queued: a range outside one runtime
 * allocation, or a source the device cannot read at its host address
 * (pageable memory), returns LMOE_ERR_ARG, and bytes or addresses not
 * multiples of 16 LMOE_ERR_SHAPE (use lmoe_stage_copy then).  Replaces
 * TransferEngine.load_many_async (transfer_engine.py:139-187) with the
 * contiguous-run batching of :205-228 done by the caller, and the
 * persistent-log2phy write (runtime.py:3068-3101) or the stage-bank table
 * build (runtime.py:2035-2258) that publishes the batch. */
int lmoe_stage_gather(void* const* dst, const void* const* src,
                      const size_t* bytes, int n, int32_t* table, int n_table,
                      const int32_t* idx, const int32_t* val, int n_tab,
                      int fill, hipStream_t transfer_stream,
                      hipEvent_t wait_event, hipEvent_t done_event);

/* Host-side slot planning of one decode staging over a slot table held as
 * arrays (no device work): state[s] (0 EMPTY, 1 LOADING, 2 READY,
 * 3 COMPUTING), owner[s] (expert id, -1 none), version[s], last_used[s] for
 * s < n_slots, and slot_of[e] (slot of resident expert e, -1 none) for
 * e < n_experts.  For each active[j] in order: a resident READY expert is a
 * hit (last_used = step); otherwise the lowest-id EMPTY slot, else the READY
 * slot of smallest (last_used, id), is reserved: its previous owner loses
 * residency, owner = expert, state LOADING, version + 1, last_used = step.
 * slot_ids[j] is the slot, miss[j] 1 for a reservation.  Returns the number
 * of misses, or -(j + 1) when expert j needs in-flight work drained first
 * (resident but LOADING / COMPUTING, or every slot LOADING / COMPUTING;
 * experts before j are planned), or LMOE_ERR_ARG.  Replaces the staging
 * loop of prepare_fixed_slot_plan_into_log2phy (runtime.py:1636-1936) with
 * ExpertSlotBank.allocate_for (slot_bank.py:211-336). */
int lmoe_slot_plan(int8_t* state, int32_t* owner, int64_t* version,
                   int64_t* last_used, int n_slots, int32_t* slot_of,
                   int n_experts, const int32_t* active, int n_active,
                   int64_t step, int32_t* slot_ids, int8_t* miss);

/* table[idx[i]] = val[i] for i < n, on stream; the idx must be distinct
 * (LMOE_ERR_ARG otherwise).  idx and val are HOST arrays read during the
 * call; the pairs travel as kernel arguments (no staging buffer, no copy),
 * so the update is capturable and can follow a stage copy batch on the
 * transfer stream, inside the same ready event.  Every idx must lie in
 * [0, n_table).  Replaces the persistent-log2phy write of
 * _update_log2phy_entries (moe_offload/runtime.py:3068-3101: one scalar
 * write, or an index_copy_ of the changed entries). */
int lmoe_table_update(int32_t* table, int n_table, const int32_t* idx,
                      const int32_t* val, int n, hipStream_t stream);

/* Bytes of the int32 plan buffer of lmoe_wave_plan / lmoe_wave_stage for
 * n_routed <= 1024 experts, n_slots <= 1024 stage slots and max_waves <= 256
 * waves; -1 outside those bounds. */
long long lmoe_wave_plan_bytes(int n_routed, int n_slots, int max_waves);

/* Capacity waves of a prefill layer planned on the device, one workgroup on
 * stream: histogram of ids[0..n_pairs) over the routed experts
 * [0, n_routed) (ids in [n_routed, n_total) are a pinned shared suffix, any
 * other id is counted as invalid), experts taken in (-count, id) order, each
 * into the wave of (least routed pairs, lowest index) among the
 * ceil(n_active / n_slots) waves with room, members ascending per wave.
 * plan: [0] waves (-1 when more than max_waves), [1] active experts, [2]
 * invalid ids, [3] 0, counts[n_routed], wave_of[n_routed],
 * slot_of[n_routed] (position in its wave, -1 inactive), size[max_waves],
 * members[max_waves][n_slots] (-1 padded).  Replaces the host planning of
 * phase_split.plan_balanced_b2_waves (moe_offload/phase_split.py:495-554)
 * after count_routed_tokens_by_expert's D2H (:479-492), and the expert ->
 * wave / slot maps of build_b2_device_wave_microbatch_plans (:1224-1384). */
int lmoe_wave_plan(const int32_t* ids, int n_pairs, int n_routed, int n_total,
                   int n_slots, int max_waves, int32_t* plan, hipStream_t stream);

/* Stage wave `wave` of a device plan, on stream (the transfer stream): for
 * member i (expert e) copy w13_expert_bytes and w2_expert_bytes into stage
 * slot i of stage_w13 / stage_w2, from main-bank slot s = main_table[e] when
 * s is in [0, main_slots) and main_owner[s] == e (the table keeps stale
 * entries of evicted experts; main_owner[s] is the slot's current expert),
 * else from host row e of host_w13 / host_w2
 * (page-locked host blocks of n_routed experts, read by the device at their
 * host address); then write stage_table[0..n_table): members -> i, ids
 * n_routed .. n_routed + n_pinned - 1 -> pinned_slot0 + j for wave 0 only,
 * -1 elsewhere.  A wave past the plan's count copies nothing and writes an
 * all -1 table.  Sizes and addresses must be multiples of 16.  Replaces the
 * stage-bank fill of prepare_prefill_stage_plan (runtime.py:2035-2258:
 * D2D for main-bank hits, H2D for misses, the per-wave table). */
int lmoe_wave_stage(const int32_t* plan, int n_routed, int n_slots, int max_waves,
                    int wave, const int32_t* main_table, const int32_t* main_owner,
                    const void* main_w13, const void* main_w2, int main_slots,
                    const void* host_w13,
                    const void* host_w2, void* stage_w13, void* stage_w2,
                    long long w13_expert_bytes, long long w2_expert_bytes,
                    int32_t* stage_table, int n_table, int n_pinned,
                    int pinned_slot0, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* LATCHMOE_H */
