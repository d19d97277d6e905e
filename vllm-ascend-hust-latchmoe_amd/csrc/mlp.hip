// Grouped SwiGLU expert MLP over the slot bank, and the weighted combine.
//
// Decode (few pairs per slot): weight-streaming GEMV kernels.  Every weight
// row is read from HBM exactly once with 16-byte non-temporal loads, all of a
// wave's rows in flight at once; token rows and act rows come from L2.  The
// down projection is fused with the weighted combine (one workgroup owns R
// output columns for every token), so the decode layer body is permute + two
// kernels.  (A single launch would need a cross-block hand-off of act; the
// agent-scope fences that takes write back / invalidate a whole XCD L2 each
// and cost far more than a kernel boundary, which in a captured graph is
// back to back.)
// Prefill (hundreds of pairs per slot): bf16 MFMA grouped GEMM, gemm_mfma.h.
//
// Reference behaviour: npu_grouped_matmul (GMM1) + npu_swiglu + GMM2 inside
// _apply_mlp (patches/patch_fused_moe.py:3772-3774, hooks :4249-4302) reading
// w1/w2 = slot bank (PreparedSlotWeights, slot_mapping.py:143-187), then
// npu_moe_token_unpermute (:3363-3366; out[t] = sum_j w[t,j] y[row(t,j)],
// phase_split.py:1649-1656).
#include "gemm_lds.h"
#include "gemm_part.h"

namespace lmoe {

// Several tokens: block (bx, slot s) of the gate_up GEMV, the slot's pairs
// p0 .. p0 + n - 1 (act rows p0 + r of act).  Each wave holds its row pair's
// weights in registers and the slot's tokens stream past one at a time; with
// TWO, two at a time (one reduction of four values and one barrier per two
// tokens; the reduction pairs lanes 32, 16, 8, 4, 2, 1 apart for every
// value as the two-value one does, so each act value has the same bits).
template <int NC, bool FULL, bool TWO = false>
__device__ __forceinline__ void gateup_tokens(const uint16_t* __restrict__ x, int H, int I,
                                              int topk, const uint16_t* __restrict__ w13, int s,
                                              int p0, int n,
                                              const int32_t* __restrict__ sorted_pairs,
                                              uint16_t* __restrict__ act) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  // [token parity][wave][gate total, up total]
  __shared__ __attribute__((aligned(16))) float s_gu[2][4][2];
  // I % 64 == 0 (the entry points check it), so every wave's row is < I and
  // all four waves meet the barrier of every pair
  const int i = blockIdx.x * 4 + wave;
  const uint16_t* grow = w13 + (static_cast<size_t>(s) * 2 * I + i) * H;
  const uint16_t* urow = grow + static_cast<size_t>(I) * H;
  uint4 wg[NC], wu[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int h = c * 512 + lane * 8;
    wg[c] = load_stream16_g<!FULL>(grow, h, h < H);
    wu[c] = load_stream16_g<!FULL>(urow, h, h < H);
  }
  int r = 0;
  if constexpr (TWO) {
    // [step parity][token][wave][gate total, up total]
    __shared__ __attribute__((aligned(16))) float s_gu2[2][2][4][2];
    for (int it = 0; r + 1 < n; r += 2, ++it) {
      const uint16_t* xr0 = x + static_cast<size_t>(sorted_pairs[p0 + r] / topk) * H;
      const uint16_t* xr1 = x + static_cast<size_t>(sorted_pairs[p0 + r + 1] / topk) * H;
      float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int h = c * 512 + lane * 8;
        const uint4 xv0 = load16_g<!FULL>(xr0, h, h < H);
        const uint4 xv1 = load16_g<!FULL>(xr1, h, h < H);
        v[0] = dot8(xv0, wg[c], v[0]);
        v[1] = dot8(xv0, wu[c], v[1]);
        v[2] = dot8(xv1, wg[c], v[2]);
        v[3] = dot8(xv1, wu[c], v[3]);
      }
      // lanes 0..15 end with token r's gate total, 16..31 its up total,
      // 32..47 and 48..63 token r + 1's
      const float tot = reduce_scatter<4, 5, 0>(v, lane);
      if ((lane & 15) == 0) s_gu2[it & 1][lane >> 5][wave][(lane >> 4) & 1] = tot;
      __syncthreads();
      if (wave == 0 && lane < 4) {
        const int tk = lane >> 1;
        const float4 gu = *reinterpret_cast<const float4*>(&s_gu2[it & 1][tk][2 * (lane & 1)][0]);
        *reinterpret_cast<uint32_t*>(act + static_cast<size_t>(p0 + r + tk) * I + blockIdx.x * 4 +
                                     2 * (lane & 1)) = swiglu_bf16x2(gu.x, gu.y, gu.z, gu.w);
      }
    }
  }
  for (; r < n; ++r) {
    const int t = sorted_pairs[p0 + r] / topk;
    const uint16_t* xr = x + static_cast<size_t>(t) * H;
    float v[2] = {0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int h = c * 512 + lane * 8;
      const uint4 xv = load16_g<!FULL>(xr, h, h < H);
      v[0] = dot8(xv, wg[c], v[0]);
      v[1] = dot8(xv, wu[c], v[1]);
    }
    // lanes 0..31 end with the gate total, 32..63 with the up total; lanes
    // 0 and 32 leave them in LDS (double-buffered by pair parity, one
    // barrier per pair), and wave 0's lanes 0 and 1 form the block's four
    // act values, two per lane, and store them as one 8-byte piece: one
    // SwiGLU sequence per block and pair instead of one per wave (the
    // paired form gives each value the bits of the single one)
    const float tot = reduce_scatter<2, 5, 0>(v, lane);
    if ((lane & 31) == 0) s_gu[r & 1][wave][lane >> 5] = tot;
    __syncthreads();
    if (wave == 0 && lane < 2) {
      const float4 gu = *reinterpret_cast<const float4*>(&s_gu[r & 1][2 * lane][0]);
      // I % 64 == 0: the four columns blockIdx.x * 4 .. + 3 are all < I
      *reinterpret_cast<uint32_t*>(act + static_cast<size_t>(p0 + r) * I + blockIdx.x * 4 + 2 * lane) =
          swiglu_bf16x2(gu.x, gu.y, gu.z, gu.w);
    }
  }
}

// ---------------------------------------------------------------------------
// gate_up GEMV + SiLU*mul, rows up to 4096 columns.  grid (ceil(I/4),
// max_active), 4 waves.  Block (bx, a) serves the a-th active slot (active[] /
// offsets[] of the permutation); each wave owns one row pair i (gate row i
// and up row I+i, 2*NC 16-byte chunks per lane, loaded non-temporally).  The
// slot's tokens stream past one at a time (x rows from L2); act is written in
// sorted order.  Longer rows: gateup_gemv_cols_kernel.  (Reducing
// several tokens per step needs twice the registers, and the lost occupancy
// costs more than the shorter chain saves: measured slower at B = 4 and 16.)
// ---------------------------------------------------------------------------
template <int NC, bool ONE, bool FULL, bool TWO = false>
__global__ __launch_bounds__(256) void gateup_gemv_kernel(
    const uint16_t* __restrict__ x, int H, int I, int topk,
    const uint16_t* __restrict__ w13, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ sorted_pairs, const int32_t* __restrict__ active,
    const int32_t* __restrict__ meta, uint16_t* __restrict__ act) {
  const int a = blockIdx.y;  // < n_slots: active[] has an entry (-1 past the active slots)
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  if (ONE) {
    // one token: its x row needs no index, so it is loaded before active[a]
    // returns, and the weight rows wait on that one load only
    uint4 xv[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int h = c * 512 + lane * 8;
      xv[c] = load16_g<!FULL>(x, h, h < H);
    }
    const int s = active[a];
    const int i = blockIdx.x * 4 + wave;
    if (s < 0 || i >= I) return;
    const uint16_t* grow = w13 + (static_cast<size_t>(s) * 2 * I + i) * H;
    const uint16_t* urow = grow + static_cast<size_t>(I) * H;
    float v[2] = {0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int h = c * 512 + lane * 8;
      v[0] = dot8(xv[c], load_stream16_g<!FULL>(grow, h, h < H), v[0]);
      v[1] = dot8(xv[c], load_stream16_g<!FULL>(urow, h, h < H), v[1]);
    }
    const float tot = reduce_scatter<2, 5, 0>(v, lane);
    const float up = read_lane(tot, 32);  // lane 32 holds the up total
    if (lane == 0) act[static_cast<size_t>(a) * I + i] = swiglu_bf16(tot, up);
    return;
  }
  const int s = active[a];
  if (s < 0) return;  // uniform over the block
  const int p0 = offsets[s];
  gateup_tokens<NC, FULL, TWO>(x, H, I, topk, w13, s, p0, offsets[s + 1] - p0, sorted_pairs, act);
}

// Both passes of a decode layer whose working set exceeds its bank (the
// bank and the overflow stage buffer, each with its own permutation) in one
// gate_up launch: grid rows below max_active_a serve the bank's active
// slots, the rest the overflow's.  The overflow pass's act rows follow the
// bank pass's placed pairs (meta_a[LMOE_META_PAIRS]), so one act buffer of
// n_pairs rows holds both when the two tables map disjoint experts (each
// pair placed by at most one pass); second_rows keeps an overflow slot's
// rows inside the buffer otherwise.  Each block runs gateup_tokens as the
// one-pass kernel does: the same bits.
__device__ __forceinline__ int second_rows(int base, int p0, int n, int n_pairs) {
  const int room = n_pairs - base - p0;
  return n < room ? n : room;
}

template <int NC, bool FULL, bool TWO>
__global__ __launch_bounds__(256) void gateup_gemv_two_kernel(
    const uint16_t* __restrict__ x, int H, int I, int topk, int n_pairs, int max_active_a,
    const uint16_t* __restrict__ w13_a, const int32_t* __restrict__ offsets_a,
    const int32_t* __restrict__ sorted_pairs_a, const int32_t* __restrict__ active_a,
    const int32_t* __restrict__ meta_a, const uint16_t* __restrict__ w13_b,
    const int32_t* __restrict__ offsets_b, const int32_t* __restrict__ sorted_pairs_b,
    const int32_t* __restrict__ active_b, uint16_t* __restrict__ act) {
  const bool second = static_cast<int>(blockIdx.y) >= max_active_a;
  const int a = second ? blockIdx.y - max_active_a : blockIdx.y;
  const int32_t* offsets = second ? offsets_b : offsets_a;
  const int s = (second ? active_b : active_a)[a];
  if (s < 0) return;  // uniform over the block
  const int p0 = offsets[s];
  const int base = second ? meta_a[LMOE_META_PAIRS] : 0;
  int n = offsets[s + 1] - p0;
  if (second) n = second_rows(base, p0, n, n_pairs);  // uniform over the block
  if (n <= 0) return;
  gateup_tokens<NC, FULL, TWO>(x, H, I, topk, second ? w13_b : w13_a, s, p0, n,
                          second ? sorted_pairs_b : sorted_pairs_a,
                          act + static_cast<size_t>(base) * I);
}

// ---------------------------------------------------------------------------
// gate_up GEMV + SiLU*mul with the columns split over the waves.  grid
// (ceil(I/RP), max_active), 4 waves.  Block (bx, a) owns the RP row pairs
// i0 = RP bx .. i0 + RP - 1 of the a-th active slot; wave w holds chunks w,
// w + 4, w + 8, ... (512 columns each, 16 bytes per lane, non-temporal) of
// all 2 RP rows (gate i, up i for each i), so each token's x row is read
// once per block, a quarter by each wave, instead of once per wave and row
// pair.  The four waves' partial sums meet in LDS (double-buffered by token
// parity, one barrier per token) and wave 0 adds them in wave order.  Every
// token's act is computed the same way whatever the batch, so one token
// alone gives the bits it gets in a batch.  ONE: T == 1 with every slot
// serving one pair (active rank a is position a, the x row is row 0), as in
// gateup_gemv_kernel: offsets and sorted_pairs are not read.
// ---------------------------------------------------------------------------
template <int NC, int RP, bool ONE>
__global__ __launch_bounds__(256) void gateup_gemv_cols_kernel(
    const uint16_t* __restrict__ x, int H, int I, int topk,
    const uint16_t* __restrict__ w13, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ sorted_pairs, const int32_t* __restrict__ active,
    uint16_t* __restrict__ act) {
  constexpr int CPW = (NC + 3) / 4;  // chunks per wave
  constexpr int NR = 2 * RP;         // rows: gate i0, up i0, gate i0 + 1, ...
  constexpr int LB = (NR >= 8) ? 3 : (NR >= 4) ? 2 : 1;
  static_assert((1 << LB) == NR, "2 RP must be a power of two");
  __shared__ float s_part[2][4][NR];  // [token parity][wave][row]
  const int a = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int s = active[a];
  if (s < 0) return;  // uniform over the block
  const int i0 = blockIdx.x * RP;
  uint4 wr[NR][CPW];
  {
    const uint16_t* g0 = w13 + (static_cast<size_t>(s) * 2 * I) * H;
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      // rows past I (the last block of a ragged I) load row 0 and are not stored
      const int i = i0 + (j >> 1);
      const uint16_t* row = g0 + (static_cast<size_t>((j & 1) * I) + (i < I ? i : 0)) * H;
#pragma unroll
      for (int q = 0; q < CPW; ++q) {
        const int h = (wave + 4 * q) * 512 + lane * 8;
        wr[j][q] = load_stream16_if(row, h, h < H);
      }
    }
  }
  const int p0 = ONE ? a : offsets[s];
  const int n = ONE ? 1 : offsets[s + 1] - p0;
  int t_next = (!ONE && n > 0) ? sorted_pairs[p0] / topk : 0;
  for (int r = 0; r < n; ++r) {
    const int t = t_next;
    if (!ONE && r + 1 < n) t_next = sorted_pairs[p0 + r + 1] / topk;
    const uint16_t* xr = x + static_cast<size_t>(t) * H;
    float v[NR];
#pragma unroll
    for (int j = 0; j < NR; ++j) v[j] = 0.0f;
#pragma unroll
    for (int q = 0; q < CPW; ++q) {
      const int h = (wave + 4 * q) * 512 + lane * 8;
      const uint4 xv = load16_if(xr, h, h < H);
#pragma unroll
      for (int j = 0; j < NR; ++j) v[j] = dot8(xv, wr[j][q], v[j]);
    }
    // lane groups of 64 / NR end with one row's partial sum each
    const float tot = reduce_scatter<NR, 5, 0>(v, lane);
    if ((lane & ((64 >> LB) - 1)) == 0) s_part[r & 1][wave][lane >> (6 - LB)] = tot;
    __syncthreads();
    if (wave == 0 && lane < RP && i0 + lane < I) {
      float g = 0.0f, u = 0.0f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        g += s_part[r & 1][w][2 * lane];
        u += s_part[r & 1][w][2 * lane + 1];
      }
      act[static_cast<size_t>(p0 + r) * I + i0 + lane] = swiglu_bf16(g, u);
    }
  }
}

// ---------------------------------------------------------------------------
// down GEMV + weighted combine (n_pairs <= 1024).  grid ceil(H/R): block b
// owns output rows h0 = R*b .. R*b+R-1 for EVERY active slot, so the combine
// needs nothing from other blocks.  Half wave hw (8 per block) takes the
// active slots a = hw, hw+8, ...: it holds the slot's R W2 rows (DNC
// 16-byte chunks per lane and row, non-temporal), with PF also loading the
// next slot's rows while it computes, streams the slot's act rows one pair at
// a time (sorted order, from L2) and leaves y[pos][r] (bf16 values) in LDS;
// then the block
// combines its R columns of every token in j order.
// ---------------------------------------------------------------------------
constexpr int kFusedMaxPairs = 1024;
constexpr int kDnMaxRows = 4;

// FULL: I == DNC * 256 and H % R == 0 (W2 rows and act chunks unguarded).
template <int DNC, int R, bool PF, bool ONE, bool FULL = false>
__global__ __launch_bounds__(256) void down_combine_gemv_kernel(
    const uint16_t* __restrict__ act, int I, int H, int T, int topk,
    const uint16_t* __restrict__ w2, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ active, int P,
    const int32_t* __restrict__ row_idx, const uint16_t* __restrict__ wts,
    const uint16_t* __restrict__ add, uint16_t* __restrict__ out) {
  constexpr int LV = (R >= 4) ? 2 : 1;
  __shared__ float s_y[kFusedMaxPairs * kDnMaxRows];
  __shared__ __attribute__((aligned(16))) int s_pos[kFusedMaxPairs];
  __shared__ __attribute__((aligned(16))) float s_w[kFusedMaxPairs];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int l5 = lane & 31;
  const int half = lane >> 5;
  const int hw = (tid >> 6) * 2 + half;
  const int h0 = blockIdx.x * R;

  uint4 wcur[R][DNC], wnxt[PF ? R : 1][PF ? DNC : 1];
  auto load_rows = [&](int s, auto& w) {
    const uint16_t* base2 = w2 + static_cast<size_t>(s) * H * I;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int h = h0 + r;
#pragma unroll
      for (int c = 0; c < DNC; ++c) {
        const int col = c * 256 + l5 * 8;
        w[r][c] = load_stream16_g<!FULL>(base2, h * I + col, h < H && col < I);
      }
    }
  };
  // active[] is -1 past the active slots, so one load per rank decides
  int rank = hw;
  int s_cur = rank < P ? active[rank] : -1;
  if (s_cur >= 0) load_rows(s_cur, wcur);
  // the combine's per-pair inputs, loaded behind the first W2 rows so they
  // arrive with them instead of one dependent round trip per pair at the end
  const int NP = T * topk;
  int pre_pos[kFusedMaxPairs / 256];
  float pre_w[kFusedMaxPairs / 256];
#pragma unroll
  for (int u = 0; u < kFusedMaxPairs / 256; ++u) {
    const int p = tid + u * 256;
    pre_pos[u] = p < NP ? row_idx[p] : -1;
    pre_w[u] = p < NP ? bf16_to_f32(wts[p]) : 0.0f;
    if (blockIdx.x == 0 && p < NP && pre_pos[u] < 0) add_device_flag(LMOE_FLAG_UNPLACED, 1);
  }
  // add term of this thread's first output (T * R <= 256 covers decode)
  const float pre_add = (add != nullptr && tid < T * R && h0 + tid % R < H)
                            ? bf16_to_f32(add[static_cast<size_t>(tid / R) * H + h0 + tid % R])
                            : 0.0f;
  // both halves of a wave run the loop together (shuffles span the wave)
  while (__ballot(s_cur >= 0) != 0ull) {
    const int nrank = rank + 8;
    const int s_nxt = (s_cur >= 0 && nrank < P) ? active[nrank] : -1;
    if constexpr (PF) {
      if (s_nxt >= 0) load_rows(s_nxt, wnxt);
    }
    // one token: active rank r is sorted position r and serves one pair
    const int p0 = s_cur >= 0 ? (ONE ? rank : offsets[s_cur]) : 0;
    const int n = s_cur >= 0 ? (ONE ? 1 : offsets[s_cur + 1] - p0) : 0;
    const int n_other = __shfl_xor(n, 32, kWave);
    const int n_max = n > n_other ? n : n_other;
    for (int q = 0; q < n_max; ++q) {
      float v[R];
#pragma unroll
      for (int r = 0; r < R; ++r) v[r] = 0.0f;
      {
        // the two half waves may have different token counts: loads past a
        // half wave's count are clamped to act[0] and zeroed
        const uint16_t* ar = act + static_cast<size_t>(q < n ? p0 + q : 0) * I;
#pragma unroll
        for (int c = 0; c < DNC; ++c) {
          const int col = c * 256 + l5 * 8;
          const uint4 av = load16_if(ar, col, q < n && (FULL || col < I));
#pragma unroll
          for (int r = 0; r < R; ++r) v[r] = dot8(av, wcur[r][c], v[r]);
        }
      }
      // reduce over the 32 lanes of each half wave: lane holds row r
      const float tot = reduce_scatter<R, 4, 0>(v, lane);
      const int r = scatter_index<4, 0, LV>(lane);
      if ((l5 & ((1 << (5 - LV)) - 1)) == 0 && q < n)
        s_y[(p0 + q) * kDnMaxRows + r] = round_bf16(tot);  // GMM2 output is bf16
    }
    rank = nrank;
    s_cur = s_nxt;
    if constexpr (PF) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < DNC; ++c) wcur[r][c] = wnxt[r][c];
    } else {
      if (s_cur >= 0) load_rows(s_cur, wcur);
    }
  }
#pragma unroll
  for (int u = 0; u < kFusedMaxPairs / 256; ++u) {
    s_pos[tid + u * 256] = pre_pos[u];
    s_w[tid + u * 256] = pre_w[u];
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kFusedMaxPairs * kDnMaxRows / 256; ++u) {
    const int qq = tid + u * 256;
    if (qq >= T * R) break;
    const int t = qq / R;
    const int r = qq % R;
    const int h = h0 + r;
    if (h >= H) continue;
    float acc = 0.0f;
    int j = 0;
    if (topk % 4 == 0) {
      // four pairs per step: one 16-byte read each of positions and weights,
      // then the four y reads in flight together (summed in pair order)
      for (; j < topk; j += 4) {
        const int p = t * topk + j;
        const int4 pos4 = *reinterpret_cast<const int4*>(&s_pos[p]);
        const float4 w4 = *reinterpret_cast<const float4*>(&s_w[p]);
        const float y0 = pos4.x >= 0 ? s_y[pos4.x * kDnMaxRows + r] : 0.0f;
        const float y1 = pos4.y >= 0 ? s_y[pos4.y * kDnMaxRows + r] : 0.0f;
        const float y2 = pos4.z >= 0 ? s_y[pos4.z * kDnMaxRows + r] : 0.0f;
        const float y3 = pos4.w >= 0 ? s_y[pos4.w * kDnMaxRows + r] : 0.0f;
        if (pos4.x >= 0) acc += w4.x * y0;
        if (pos4.y >= 0) acc += w4.y * y1;
        if (pos4.z >= 0) acc += w4.z * y2;
        if (pos4.w >= 0) acc += w4.w * y3;
      }
    }
    for (; j < topk; ++j) {
      const int p = t * topk + j;
      const int pos = s_pos[p];
      if (pos >= 0) acc += s_w[p] * s_y[pos * kDnMaxRows + r];
    }
    if (add != nullptr)
      acc += u == 0 ? pre_add : bf16_to_f32(add[static_cast<size_t>(t) * H + h]);
    out[static_cast<size_t>(t) * H + h] = static_cast<uint16_t>(f32_to_bf16_bits(acc));
  }
}

// ---------------------------------------------------------------------------
// down GEMV per (row block, slot), y in bf16.  grid (ceil(H / (8 R)),
// max_active); half wave hw of block (bx, a) owns rows h0 = (8 bx + hw) R ..
// h0 + R - 1 of the a-th active slot: DNC 16-byte chunks per lane and row
// (non-temporal), then the slot's act rows one pair at a time (sorted order,
// from L2).  Every (slot, row block) is its own workgroup, so a slot's rows
// are streamed by many CUs at once and no workgroup walks the slots in turn.
// y row = flat pair (sorted_pairs[pos]).  Per value the reduction is the
// lane-pair tree of down_combine_gemv_kernel, so y equals its LDS values bit
// for bit.
// ---------------------------------------------------------------------------
// FULL: I == DNC * 256 and H % (8 R) == 0, so no chunk or row is guarded.
// Block (bx, slot s) of the down GEMV: the slot's pairs p0 .. p0 + n - 1,
// act row pos read at act + pos * I (act already offset for a second pass).
template <int DNC, int R, bool FULL>
__device__ __forceinline__ void down_rows_body(const uint16_t* __restrict__ act, int I, int H,
                                               const uint16_t* __restrict__ w2, int s, int p0,
                                               int n, const int32_t* __restrict__ sorted_pairs,
                                               uint16_t* __restrict__ y) {
  constexpr int LV = (R >= 4) ? 2 : 1;
  const int lane = threadIdx.x & 63;
  const int l5 = lane & 31;
  const int hw = (threadIdx.x >> 6) * 2 + (lane >> 5);
  const int h0 = (blockIdx.x * 8 + hw) * R;
  // both halves of a wave serve the same slot: loop bounds are wave-uniform
  const uint16_t* base2 = w2 + static_cast<size_t>(s) * H * I;
  uint4 w[R][DNC];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int h = h0 + r;
#pragma unroll
    for (int c = 0; c < DNC; ++c) {
      const int col = c * 256 + l5 * 8;
      w[r][c] = load_stream16_g<!FULL>(base2, h * I + col, h < H && col < I);
    }
  }
  for (int q = 0; q < n; ++q) {
    const int pos = p0 + q;
    const uint16_t* ar = act + static_cast<size_t>(pos) * I;
    const int dst = sorted_pairs[pos];
    float v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = 0.0f;
#pragma unroll
    for (int c = 0; c < DNC; ++c) {
      const int col = c * 256 + l5 * 8;
      const uint4 av = load16_g<!FULL>(ar, col, col < I);
#pragma unroll
      for (int r = 0; r < R; ++r) v[r] = dot8(av, w[r][c], v[r]);
    }
    // reduce over the 32 lanes of each half wave: lane holds row r
    const float tot = reduce_scatter<R, 4, 0>(v, lane);
    const int r = scatter_index<4, 0, LV>(lane);
    if ((l5 & ((1 << (5 - LV)) - 1)) == 0 && (FULL || h0 + r < H))
      y[static_cast<size_t>(dst) * H + h0 + r] = static_cast<uint16_t>(f32_to_bf16_bits(tot));
  }
}

template <int DNC, int R, bool FULL>
__global__ __launch_bounds__(256) void down_rows_kernel(
    const uint16_t* __restrict__ act, int I, int H,
    const uint16_t* __restrict__ w2, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ sorted_pairs, const int32_t* __restrict__ active,
    uint16_t* __restrict__ y) {
  const int a = blockIdx.y;  // < n_slots: active[] has an entry (-1 past the active slots)
  const int s = active[a];
  if (s < 0) return;
  const int p0 = offsets[s];
  down_rows_body<DNC, R, FULL>(act, I, H, w2, s, p0, offsets[s + 1] - p0, sorted_pairs, y);
}

// The down GEMV of both passes (see gateup_gemv_two_kernel): grid rows below
// max_active_a serve the bank's active slots, the rest the overflow's, whose
// act rows follow the bank pass's placed pairs.  y is indexed by flat pair,
// which each pair has in at most one pass.
template <int DNC, int R, bool FULL>
__global__ __launch_bounds__(256) void down_rows_two_kernel(
    const uint16_t* __restrict__ act, int I, int H, int n_pairs, int max_active_a,
    const uint16_t* __restrict__ w2_a, const int32_t* __restrict__ offsets_a,
    const int32_t* __restrict__ sorted_pairs_a, const int32_t* __restrict__ active_a,
    const int32_t* __restrict__ meta_a, const uint16_t* __restrict__ w2_b,
    const int32_t* __restrict__ offsets_b, const int32_t* __restrict__ sorted_pairs_b,
    const int32_t* __restrict__ active_b, uint16_t* __restrict__ y) {
  const bool second = static_cast<int>(blockIdx.y) >= max_active_a;
  const int a = second ? blockIdx.y - max_active_a : blockIdx.y;
  const int32_t* offsets = second ? offsets_b : offsets_a;
  const int s = (second ? active_b : active_a)[a];
  if (s < 0) return;
  const int p0 = offsets[s];
  const int base = second ? meta_a[LMOE_META_PAIRS] : 0;
  int n = offsets[s + 1] - p0;
  if (second) n = second_rows(base, p0, n, n_pairs);  // the rows gate_up wrote
  if (n <= 0) return;
  down_rows_body<DNC, R, FULL>(act + static_cast<size_t>(base) * I, I, H, second ? w2_b : w2_a, s,
                               p0, n, second ? sorted_pairs_b : sorted_pairs_a, y);
}

// ---------------------------------------------------------------------------
// weighted combine, y indexed by flat pair.  grid (T, ceil(H/2048)); each
// thread owns 8 consecutive columns.  The k rows of its token are loaded
// together (up to kCombineStep per step, independent of row_idx, which only
// masks; every load is issued, from a clamped address where j >= topk),
// then added in j order.  Eight per step: the 4096-token, top-8 combine
// took 23.7 us against 26.2 us with sixteen (same bits).
// ---------------------------------------------------------------------------
constexpr int kCombineStep = 8;

__global__ __launch_bounds__(256) void combine_kernel(
    const uint16_t* __restrict__ y, const int32_t* __restrict__ row_idx,
    const uint16_t* __restrict__ w, int T, int topk, int H,
    const uint16_t* __restrict__ add, uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  const int h = (blockIdx.y * 256 + threadIdx.x) * 8;
  if (t >= T || h >= H) return;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
  uint4 av = make_uint4(0u, 0u, 0u, 0u);
  if (add != nullptr) av = *reinterpret_cast<const uint4*>(add + static_cast<size_t>(t) * H + h);
  for (int j0 = 0; j0 < topk; j0 += kCombineStep) {
    uint4 v[kCombineStep];
    float wj[kCombineStep];
    bool use[kCombineStep];
#pragma unroll
    for (int jj = 0; jj < kCombineStep; ++jj) {
      const int j = j0 + jj;
      const int p = t * topk + j;
      const bool in = j < topk;
      use[jj] = in && (row_idx == nullptr || row_idx[p] >= 0);
      // a pair no pass placed: counted once (first column block of the token)
      if (in && !use[jj] && blockIdx.y == 0 && threadIdx.x == 0)
        add_device_flag(LMOE_FLAG_UNPLACED, 1);
      wj[jj] = in ? bf16_to_f32(w[p]) : 0.0f;
      const uint4 yv =
          *reinterpret_cast<const uint4*>(y + (in ? static_cast<size_t>(p) * H + h : 0));
      v[jj] = in ? yv : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int jj = 0; jj < kCombineStep; ++jj) {
      if (use[jj]) {
        const float q = wj[jj];
        acc[0] += q * bf16lo(v[jj].x);
        acc[1] += q * bf16hi(v[jj].x);
        acc[2] += q * bf16lo(v[jj].y);
        acc[3] += q * bf16hi(v[jj].y);
        acc[4] += q * bf16lo(v[jj].z);
        acc[5] += q * bf16hi(v[jj].z);
        acc[6] += q * bf16lo(v[jj].w);
        acc[7] += q * bf16hi(v[jj].w);
      }
    }
  }
  if (add != nullptr) {
    acc[0] += bf16lo(av.x);
    acc[1] += bf16hi(av.x);
    acc[2] += bf16lo(av.y);
    acc[3] += bf16hi(av.y);
    acc[4] += bf16lo(av.z);
    acc[5] += bf16hi(av.z);
    acc[6] += bf16lo(av.w);
    acc[7] += bf16hi(av.w);
  }
  uint4 o;
  o.x = pack_bf16x2(acc[0], acc[1]);
  o.y = pack_bf16x2(acc[2], acc[3]);
  o.z = pack_bf16x2(acc[4], acc[5]);
  o.w = pack_bf16x2(acc[6], acc[7]);
  *reinterpret_cast<uint4*>(out + static_cast<size_t>(t) * H + h) = o;
}

// ---------------------------------------------------------------------------
// launch helpers
// ---------------------------------------------------------------------------
// one: T == 1 (every slot serves at most one pair; log2phy maps distinct
// experts to distinct slots).  Past kTwoTokenMinPairs pairs the several-token
// form takes its tokens two at a time (half the block barriers: same box,
// B=4 43.35 -> 42.96, B=16 78.57 -> 77.83, B=64 178.3 -> 175.3 us per
// decode layer).
constexpr int kTwoTokenMinPairs = 16;

static int launch_gateup_gemv(const uint16_t* x, int H, int I, int topk,
                              const uint16_t* w13, const int32_t* offsets,
                              const int32_t* sorted_pairs, const int32_t* active,
                              const int32_t* meta, int max_active, bool one, int n_pairs,
                              uint16_t* act, hipStream_t stream) {
  const bool two = !one && n_pairs > kTwoTokenMinPairs;
  const int nc = (H + 511) / 512;
  const dim3 g4((I + 3) / 4, max_active);
  // long rows: the column-split kernel.  (For H <= 4096 it measured 3%
  // faster at 16 tokens but 0.7 us slower at one token, and one layout must
  // serve every batch size, so the row-per-wave kernels stay there.)
  const bool cols = nc > 8;
  // rows of exactly NC chunks of 512 columns load without guards
#define LMOE_GU0(NC, ONE, FULL, TWO)                                                          \
  hipLaunchKernelGGL((gateup_gemv_kernel<NC, ONE, FULL, TWO>), g4, dim3(256), 0, stream, x, H, \
                     I, topk, w13, offsets, sorted_pairs, active, meta, act)
#define LMOE_GU1(NC, ONE, TWO)                     \
  do {                                             \
    if (H == (NC)*512) LMOE_GU0(NC, ONE, true, TWO); \
    else LMOE_GU0(NC, ONE, false, TWO);            \
  } while (0)
#define LMOE_GU(NC)                     \
  do {                                  \
    if (one) LMOE_GU1(NC, true, false); \
    else if (two) LMOE_GU1(NC, false, true); \
    else LMOE_GU1(NC, false, false);    \
  } while (0)
#define LMOE_GC(NC, RP, ONE)                                                                 \
  hipLaunchKernelGGL((gateup_gemv_cols_kernel<NC, RP, ONE>), dim3((I + (RP)-1) / (RP),         \
                     max_active), dim3(256), 0, stream, x, H, I, topk, w13, offsets,              \
                     sorted_pairs, active, act)
  if (cols) {
    // the four waves split each row's columns and share every x row (for
    // one token too, so that a token's act does not depend on its batch)
    if (nc > 16) return LMOE_ERR_SHAPE;
    if (one) LMOE_GC(16, 2, true);
    else LMOE_GC(16, 2, false);
    return LMOE_OK;
  }
#undef LMOE_GC
  if (nc <= 2) LMOE_GU(2);
  else if (nc <= 4) LMOE_GU(4);
  else LMOE_GU(8);
#undef LMOE_GU
#undef LMOE_GU1
#undef LMOE_GU0
  return LMOE_OK;
}

// down_rows_kernel launch: R = 2 rows per half wave, 16 rows per workgroup
// (measured faster than 4 at B = 4 and 16: twice the workgroups, fewer
// registers).
static int launch_down_rows(const uint16_t* act, int H, int I, const uint16_t* w2,
                            const int32_t* offsets, const int32_t* sorted_pairs,
                            const int32_t* active, int max_active, uint16_t* y,
                            hipStream_t stream) {
  const int dnc = (I + 255) / 256;
#define LMOE_DR1(DNC, R, FULL)                                                               \
  hipLaunchKernelGGL((down_rows_kernel<DNC, R, FULL>), dim3((H + 8 * (R)-1) / (8 * (R)),       \
                     max_active), dim3(256), 0, stream, act, I, H, w2, offsets, sorted_pairs,   \
                     active, y)
#define LMOE_DR(DNC, R)                                                   \
  do {                                                                    \
    if (I == (DNC)*256 && H % (8 * (R)) == 0) LMOE_DR1(DNC, R, true);     \
    else LMOE_DR1(DNC, R, false);                                         \
  } while (0)
  if (dnc <= 2) LMOE_DR(2, 2);
  else if (dnc <= 3) LMOE_DR(3, 2);
  else if (dnc <= 4) LMOE_DR(4, 2);
  else if (dnc <= 8) LMOE_DR(8, 2);
  else if (dnc <= 16) LMOE_DR(16, 2);
  else return LMOE_ERR_SHAPE;
#undef LMOE_DR
#undef LMOE_DR1
  return LMOE_OK;
}

static void launch_combine(const uint16_t* y, const int32_t* row_idx, const uint16_t* w, int T,
                           int k, int H, const uint16_t* add, uint16_t* out, hipStream_t stream) {
  hipLaunchKernelGGL(combine_kernel, dim3(T, (H + 2047) / 2048), dim3(256), 0, stream, y, row_idx,
                     w, T, k, H, add, out);
}

// ---------------------------------------------------------------------------
// grouped MFMA GEMM launch (prefill).  block_m is the tile height the
// permutation's tile table was built with: 320 runs the block-range kernel
// (gemm_part.h: one workgroup per CU, equal column-block shares), 256 the
// direct-to-LDS 256 x 256 tile grid (both: K a multiple of 64, 16-byte
// aligned operands), 128 the register-staged 128 x 128 kernel.
// ---------------------------------------------------------------------------
using PrefillTile = LdsTile<256, 256, 2, 4, 2>;

// Workgroups of the block-range kernel: one per CU, a multiple of 8 (one
// share per XCD), queried once per device.
static int part_grid() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 64 && cached[dev] > 0) return cached[dev];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  const int grid = ((cus + 7) / 8) * 8;
  if (dev < 64) cached[dev] = grid;
  return grid;
}

// The block-range kernel forms operand offsets in 32 bits: activation row r
// starts at r * K, the rows read are token rows (gate-up: sorted pair / topk
// < ceil(n_pairs / topk)) or sorted positions (down: < n_pairs), and a
// weight row lies inside one slot of w_slot_stride elements.  All of them
// must end below 2^31.
template <int MODE>
static bool part_offsets_fit(const GemmArgs& g, int n_pairs) {
  const long long a_rows =
      MODE == kGateUp ? (static_cast<long long>(n_pairs) + g.topk - 1) / g.topk : n_pairs;
  const long long lim = 0x7fffffffLL;
  return a_rows * g.K <= lim && g.w_slot_stride <= lim;
}

template <int MODE>
static int launch_grouped_mfma(GemmArgs g, int n_pairs, int max_active, int block_m,
                               hipStream_t stream) {
  if (block_m != PartTile::BM && block_m != PrefillTile::BM && block_m != kBM)
    return LMOE_ERR_UNSUPPORTED;
  const int ub_tiles = n_pairs / block_m + max_active + 1;
  g.block_m = block_m;
  const bool aligned = ((reinterpret_cast<uintptr_t>(g.a) | reinterpret_cast<uintptr_t>(g.w) |
                         reinterpret_cast<uintptr_t>(g.out)) & 15u) == 0;
  if (!aligned) return LMOE_ERR_SHAPE;
  if (block_m == PartTile::BM) {
    if (g.K % PartTile::BK != 0 || g.N % 8 != 0) return LMOE_ERR_SHAPE;
    if (!part_offsets_fit<MODE>(g, n_pairs)) return LMOE_ERR_SHAPE;  // take block_m 256
    hipLaunchKernelGGL((grouped_gemm_part_kernel<MODE, PartTile>), dim3(part_grid()),
                       dim3(PartTile::THREADS), 0, stream, g);
    return LMOE_OK;
  }
  if (block_m == PrefillTile::BM && g.K % PrefillTile::BK == 0 && g.N % 8 == 0) {
    const int col_tile = (MODE == kGateUp) ? PrefillTile::BN / 2 : PrefillTile::BN;
    const int grid = lds_gemm_grid(ub_tiles, (g.N + col_tile - 1) / col_tile);
    hipLaunchKernelGGL((grouped_gemm_lds_kernel<MODE, PrefillTile>), dim3(grid),
                       dim3(PrefillTile::THREADS), 0, stream, g);
    return LMOE_OK;
  }
  const int col_tile = (MODE == kGateUp) ? kBN / 2 : kBN;
  hipLaunchKernelGGL(grouped_gemm_kernel<MODE>,
                     dim3(ub_tiles, (g.N + col_tile - 1) / col_tile, block_m / kBM), dim3(256),
                     0, stream, g);
  return LMOE_OK;
}

}  // namespace lmoe

LMOE_FLAGS_UNIT(mlp)

using namespace lmoe;

static long long slot_elems_w13(int H, int I) { return 2LL * I * H; }
static long long slot_elems_w2(int H, int I) { return 1LL * H * I; }

static int check_mlp_args(int T, int H, int I, int k, int n_slots, int n_pairs) {
  if (T < 0 || H <= 0 || I <= 0 || k <= 0 || n_slots <= 0 || n_pairs < 0) return LMOE_ERR_ARG;
  if (H % 8 != 0 || I % 64 != 0 || I > 8192 || H > 8192) return LMOE_ERR_SHAPE;
  return LMOE_OK;
}

static int resolve_path(int path, int n_pairs) {
  return path == LMOE_PATH_AUTO ? (n_pairs <= 256 ? LMOE_PATH_GEMV : LMOE_PATH_MFMA) : path;
}

extern "C" int lmoe_gateup_silu(const void* x, int T, int H, int I, int k,
                                const void* w13_slots, int n_slots,
                                const int32_t* offsets, const int32_t* sorted_pairs,
                                const int32_t* active, const int32_t* tile_off,
                                const int32_t* meta, int n_pairs, int block_m,
                                int path, void* act, hipStream_t stream) {
  int st = check_mlp_args(T, H, I, k, n_slots, n_pairs);
  if (st != LMOE_OK) return st;
  if (n_pairs == 0) return LMOE_OK;  // an empty batch: nothing read or written
  if (x == nullptr || w13_slots == nullptr || offsets == nullptr || sorted_pairs == nullptr ||
      active == nullptr || meta == nullptr || act == nullptr)
    return LMOE_ERR_ARG;
  path = resolve_path(path, n_pairs);
  const int max_active = n_pairs < n_slots ? n_pairs : n_slots;
  if (path == LMOE_PATH_GEMV) {
    // general form: a caller's permutation may give one slot several pairs
    // of the one token
    st = launch_gateup_gemv(static_cast<const uint16_t*>(x), H, I, k,
                            static_cast<const uint16_t*>(w13_slots), offsets, sorted_pairs,
                            active, meta, max_active, false, n_pairs,
                            static_cast<uint16_t*>(act), stream);
    if (st != LMOE_OK) return st;
    LMOE_RETURN_LAUNCH();
  }
  if (path != LMOE_PATH_MFMA) return LMOE_ERR_UNSUPPORTED;
  if (tile_off == nullptr) return LMOE_ERR_ARG;
  GemmArgs g{};
  g.topk = k;
  g.offsets = offsets;
  g.sorted_pairs = sorted_pairs;
  g.tile_off = tile_off;
  g.meta = meta;
  g.P = n_slots;
  g.a = static_cast<const uint16_t*>(x);
  g.w = static_cast<const uint16_t*>(w13_slots);
  g.w_slot_stride = slot_elems_w13(H, I);
  g.N = I;
  g.K = H;
  g.I = I;
  g.out = act;
  st = launch_grouped_mfma<kGateUp>(g, n_pairs, max_active, block_m, stream);
  if (st != LMOE_OK) return st;
  LMOE_RETURN_LAUNCH();
}

extern "C" int lmoe_down(const void* act, int H, int I, const void* w2_slots, int n_slots,
                         const int32_t* offsets, const int32_t* sorted_pairs,
                         const int32_t* active, const int32_t* tile_off,
                         const int32_t* meta, int n_pairs, int block_m, int path,
                         void* y, hipStream_t stream) {
  int st = check_mlp_args(1, H, I, 1, n_slots, n_pairs);
  if (st != LMOE_OK) return st;
  if (n_pairs == 0) return LMOE_OK;  // an empty batch: nothing read or written
  if (act == nullptr || w2_slots == nullptr || offsets == nullptr || sorted_pairs == nullptr ||
      active == nullptr || meta == nullptr || y == nullptr)
    return LMOE_ERR_ARG;
  path = resolve_path(path, n_pairs);
  const int max_active = n_pairs < n_slots ? n_pairs : n_slots;
  const uint16_t* actb = static_cast<const uint16_t*>(act);
  const uint16_t* w2 = static_cast<const uint16_t*>(w2_slots);
  uint16_t* yb = static_cast<uint16_t*>(y);
  if (path == LMOE_PATH_GEMV) {
    if ((reinterpret_cast<uintptr_t>(act) | reinterpret_cast<uintptr_t>(w2_slots)) & 15u)
      return LMOE_ERR_SHAPE;
    st = launch_down_rows(actb, H, I, w2, offsets, sorted_pairs, active, max_active, yb, stream);
    if (st != LMOE_OK) return st;
    LMOE_RETURN_LAUNCH();
  }
  if (path != LMOE_PATH_MFMA) return LMOE_ERR_UNSUPPORTED;
  if (tile_off == nullptr) return LMOE_ERR_ARG;
  GemmArgs g{};
  g.topk = 1;
  g.offsets = offsets;
  g.sorted_pairs = sorted_pairs;
  g.tile_off = tile_off;
  g.meta = meta;
  g.P = n_slots;
  g.a = actb;
  g.w = w2;
  g.w_slot_stride = slot_elems_w2(H, I);
  g.N = H;
  g.K = I;
  g.out = yb;
  st = launch_grouped_mfma<kDown>(g, n_pairs, max_active, block_m, stream);
  if (st != LMOE_OK) return st;
  LMOE_RETURN_LAUNCH();
}

extern "C" int lmoe_grouped_mlp(const void* x, int T, int H, int I, int k,
                                const void* w13_slots, const void* w2_slots,
                                int n_slots, const int32_t* offsets,
                                const int32_t* sorted_pairs,
                                const int32_t* active, const int32_t* tile_off,
                                const int32_t* meta, int n_pairs, int block_m,
                                int path, void* act, void* y,
                                hipStream_t stream) {
  int st = check_mlp_args(T, H, I, k, n_slots, n_pairs);
  if (st != LMOE_OK) return st;
  if (n_pairs == 0) return LMOE_OK;
  if (w2_slots == nullptr || y == nullptr) return LMOE_ERR_ARG;
  st = lmoe_gateup_silu(x, T, H, I, k, w13_slots, n_slots, offsets, sorted_pairs, active,
                            tile_off, meta, n_pairs, block_m, path, act, stream);
  if (st != LMOE_OK) return st;
  return lmoe_down(act, H, I, w2_slots, n_slots, offsets, sorted_pairs, active, tile_off, meta,
                   n_pairs, block_m, path, y, stream);
}

extern "C" int lmoe_decode_mlp_two_passes(
    const void* x, int T, int H, int I, int k, const void* w13_a, const void* w2_a, int n_slots_a,
    const int32_t* offsets_a, const int32_t* sorted_pairs_a, const int32_t* active_a,
    const int32_t* meta_a, const void* w13_b, const void* w2_b, int n_slots_b,
    const int32_t* offsets_b, const int32_t* sorted_pairs_b, const int32_t* active_b,
    int n_pairs, void* act, void* y, hipStream_t stream) {
  int st = check_mlp_args(T, H, I, k, n_slots_a, n_pairs);
  if (st != LMOE_OK) return st;
  if (n_slots_b <= 0) return LMOE_ERR_ARG;
  if (n_pairs == 0) return LMOE_OK;  // an empty batch: nothing read or written
  if (x == nullptr || w13_a == nullptr || w2_a == nullptr || offsets_a == nullptr ||
      sorted_pairs_a == nullptr || active_a == nullptr || meta_a == nullptr ||
      w13_b == nullptr || w2_b == nullptr || offsets_b == nullptr || sorted_pairs_b == nullptr ||
      active_b == nullptr || act == nullptr || y == nullptr)
    return LMOE_ERR_ARG;
  // the row-per-wave GEMVs only (rows up to 4096 columns)
  const int nc = (H + 511) / 512;
  const int dnc = (I + 255) / 256;
  if (nc > 8 || dnc > 16) return LMOE_ERR_SHAPE;
  if ((reinterpret_cast<uintptr_t>(act) | reinterpret_cast<uintptr_t>(w2_a) |
       reinterpret_cast<uintptr_t>(w2_b)) & 15u)
    return LMOE_ERR_SHAPE;
  const int max_a = n_pairs < n_slots_a ? n_pairs : n_slots_a;
  const int max_b = n_pairs < n_slots_b ? n_pairs : n_slots_b;
  const uint16_t* xb = static_cast<const uint16_t*>(x);
  const uint16_t* w13a = static_cast<const uint16_t*>(w13_a);
  const uint16_t* w13b = static_cast<const uint16_t*>(w13_b);
  uint16_t* actb = static_cast<uint16_t*>(act);
  const dim3 g4((I + 3) / 4, max_a + max_b);
#define LMOE_GU3(NC, FULL, TWO)                                                                \
  hipLaunchKernelGGL((gateup_gemv_two_kernel<NC, FULL, TWO>), g4, dim3(256), 0, stream, xb, H, I, \
                     k, n_pairs, max_a, w13a, offsets_a, sorted_pairs_a, active_a, meta_a, w13b,    \
                     offsets_b, sorted_pairs_b, active_b, actb)
#define LMOE_GU2(NC, FULL)                                   \
  do {                                                       \
    if (n_pairs > kTwoTokenMinPairs) LMOE_GU3(NC, FULL, true); \
    else LMOE_GU3(NC, FULL, false);                          \
  } while (0)
#define LMOE_GU2N(NC)                     \
  do {                                    \
    if (H == (NC)*512) LMOE_GU2(NC, true); \
    else LMOE_GU2(NC, false);             \
  } while (0)
  if (nc <= 2) LMOE_GU2N(2);
  else if (nc <= 4) LMOE_GU2N(4);
  else LMOE_GU2N(8);
#undef LMOE_GU2N
#undef LMOE_GU2
#undef LMOE_GU3
  const uint16_t* w2a = static_cast<const uint16_t*>(w2_a);
  const uint16_t* w2b = static_cast<const uint16_t*>(w2_b);
  uint16_t* yb = static_cast<uint16_t*>(y);
  // R = 2 rows per half wave, as launch_down_rows
#define LMOE_DR2(DNC, FULL)                                                                       \
  hipLaunchKernelGGL((down_rows_two_kernel<DNC, 2, FULL>), dim3((H + 15) / 16, max_a + max_b),    \
                     dim3(256), 0, stream, actb, I, H, n_pairs, max_a, w2a, offsets_a, sorted_pairs_a,    \
                     active_a, meta_a, w2b, offsets_b, sorted_pairs_b, active_b, yb)
#define LMOE_DR2N(DNC)                                          \
  do {                                                          \
    if (I == (DNC)*256 && H % 16 == 0) LMOE_DR2(DNC, true);     \
    else LMOE_DR2(DNC, false);                                  \
  } while (0)
  if (dnc <= 2) LMOE_DR2N(2);
  else if (dnc <= 3) LMOE_DR2N(3);
  else if (dnc <= 4) LMOE_DR2N(4);
  else if (dnc <= 8) LMOE_DR2N(8);
  else LMOE_DR2N(16);
#undef LMOE_DR2N
#undef LMOE_DR2
  LMOE_RETURN_LAUNCH();
}

// one: a single token whose pairs sit in distinct slots (active rank a is
// sorted position a), the precondition of the ONE kernels.
static int down_combine_impl(const void* act, int T, int H, int I, int k,
                             const void* w2_slots, int n_slots, const uint16_t* w,
                             const int32_t* offsets, const int32_t* row_idx,
                             const int32_t* active, const int32_t* meta,
                             const void* add, void* out, bool one, hipStream_t stream) {
  if (T < 0 || H <= 0 || I <= 0 || k <= 0 || n_slots <= 0) return LMOE_ERR_ARG;
  if (H % 8 != 0 || I % 64 != 0 || I > 4096 || H > 8192) return LMOE_ERR_SHAPE;
  if (T * k > kFusedMaxPairs) return LMOE_ERR_SHAPE;
  if (T == 0) return LMOE_OK;  // an empty batch: nothing read or written
  if (act == nullptr || w2_slots == nullptr || w == nullptr || offsets == nullptr ||
      row_idx == nullptr || active == nullptr || meta == nullptr || out == nullptr)
    return LMOE_ERR_ARG;
  if ((reinterpret_cast<uintptr_t>(act) | reinterpret_cast<uintptr_t>(w2_slots)) & 15u)
    return LMOE_ERR_SHAPE;
  const int dnc = (I + 255) / 256;
#define LMOE_DC(DNC, R, PF)                                                                    \
  do {                                                                                         \
    const dim3 grid((H + R - 1) / R);                                                          \
    const uint16_t* a_ = static_cast<const uint16_t*>(act);                                    \
    const uint16_t* w2_ = static_cast<const uint16_t*>(w2_slots);                              \
    const uint16_t* add_ = static_cast<const uint16_t*>(add);                                  \
    uint16_t* out_ = static_cast<uint16_t*>(out);                                              \
    if (one && k <= 8 && I == (DNC)*256 && H % (R) == 0)                                       \
      /* one slot per half wave (ranks < k <= 8): no next-slot prefetch; rows of whole chunks */ \
      hipLaunchKernelGGL((down_combine_gemv_kernel<DNC, R, false, true, true>), grid, dim3(256), \
                         0, stream, a_, I, H, T, k, w2_, offsets, active, n_slots, row_idx, w,  \
                         add_, out_);                                                          \
    else if (one && k <= 8)                                                                    \
      hipLaunchKernelGGL((down_combine_gemv_kernel<DNC, R, false, true>), grid, dim3(256), 0,   \
                         stream, a_, I, H, T, k, w2_, offsets, active, n_slots, row_idx, w,     \
                         add_, out_);                                                          \
    else if (one)                                                                              \
      hipLaunchKernelGGL((down_combine_gemv_kernel<DNC, R, PF, true>), grid, dim3(256), 0,      \
                         stream, a_, I, H, T, k, w2_, offsets, active, n_slots, row_idx, w,     \
                         add_, out_);                                                          \
    else                                                                                       \
      hipLaunchKernelGGL((down_combine_gemv_kernel<DNC, R, PF, false>), grid, dim3(256), 0,     \
                         stream, a_, I, H, T, k, w2_, offsets, active, n_slots, row_idx, w,     \
                         add_, out_);                                                          \
  } while (0)
  if (dnc <= 2) LMOE_DC(2, 4, true);
  else if (dnc <= 3) LMOE_DC(3, 4, true);
  else if (dnc <= 4) LMOE_DC(4, 4, true);
  // I up to 2048: two rows per half wave (half the weight registers of
  // four) measured 41 / 52 us against 53 / 70 us for four at H 7168 with
  // 8 / 9 active slots (at I 768 the two are alike)
  else if (dnc <= 8) LMOE_DC(8, 2, false);
  else if (dnc <= 16) LMOE_DC(16, 2, false);
  else return LMOE_ERR_SHAPE;
#undef LMOE_DC
  LMOE_RETURN_LAUNCH();
}

extern "C" int lmoe_down_combine(const void* act, int T, int H, int I, int k,
                                 const void* w2_slots, int n_slots, const uint16_t* w,
                                 const int32_t* offsets, const int32_t* row_idx,
                                 const int32_t* active, const int32_t* meta,
                                 const void* add, void* out, hipStream_t stream) {
  return down_combine_impl(act, T, H, I, k, w2_slots, n_slots, w, offsets, row_idx, active, meta,
                           add, out, false, stream);
}

extern "C" int lmoe_fused_moe_decode(const void* x, int T, int H, int I, int k,
                                     const void* w13_slots, const void* w2_slots,
                                     int n_slots, const uint16_t* w,
                                     const int32_t* offsets,
                                     const int32_t* sorted_pairs,
                                     const int32_t* row_idx,
                                     const int32_t* active, const int32_t* meta,
                                     const void* add, void* act, void* y, void* out,
                                     int distinct_slots, hipStream_t stream) {
  if (T < 0 || H <= 0 || I <= 0 || k <= 0 || n_slots <= 0) return LMOE_ERR_ARG;
  if (H % 8 != 0 || I % 64 != 0 || I > 4096 || H > 8192) return LMOE_ERR_SHAPE;
  const int n_pairs = T * k;
  if (n_pairs > kFusedMaxPairs) return LMOE_ERR_SHAPE;
  if (T == 0) return LMOE_OK;  // an empty batch: nothing read or written
  if (x == nullptr || w13_slots == nullptr || w2_slots == nullptr || w == nullptr ||
      offsets == nullptr || sorted_pairs == nullptr || row_idx == nullptr ||
      active == nullptr || meta == nullptr || act == nullptr || out == nullptr)
    return LMOE_ERR_ARG;
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w13_slots) |
       reinterpret_cast<uintptr_t>(w2_slots) | reinterpret_cast<uintptr_t>(act) |
       reinterpret_cast<uintptr_t>(y)) & 15u)
    return LMOE_ERR_SHAPE;
  const int max_active = n_pairs < n_slots ? n_pairs : n_slots;
  const bool one = T == 1 && distinct_slots != 0;
  int st = launch_gateup_gemv(static_cast<const uint16_t*>(x), H, I, k,
                              static_cast<const uint16_t*>(w13_slots), offsets,
                              sorted_pairs, active, meta, max_active, one, n_pairs,
                              static_cast<uint16_t*>(act), stream);
  if (st != LMOE_OK) return st;
  if (y != nullptr && T > 1 && n_pairs > 16) {
    // slots serving several tokens: down per (row block, slot) into y (flat
    // pair order), then the combine.  Up to 16 pairs (two slots per half
    // wave of the fused kernel) the fused down + combine is faster: 27.7
    // against 28.9 us per layer at 2 tokens, equal at 4, slower from 8 on;
    // both give the same bits.
    st = launch_down_rows(static_cast<const uint16_t*>(act), H, I,
                          static_cast<const uint16_t*>(w2_slots), offsets, sorted_pairs, active,
                          max_active, static_cast<uint16_t*>(y), stream);
    if (st != LMOE_OK) return st;
    launch_combine(static_cast<const uint16_t*>(y), row_idx, w, T, k, H,
                   static_cast<const uint16_t*>(add), static_cast<uint16_t*>(out), stream);
    LMOE_RETURN_LAUNCH();
  }
  return down_combine_impl(act, T, H, I, k, w2_slots, n_slots, w, offsets, row_idx, active, meta,
                           add, out, one, stream);
}

extern "C" int lmoe_combine(const void* y, const int32_t* row_idx,
                            const uint16_t* w, int T, int k, int H,
                            const void* add, void* out, hipStream_t stream) {
  if (T < 0 || k <= 0 || H <= 0) return LMOE_ERR_ARG;
  if (H % 8 != 0) return LMOE_ERR_SHAPE;
  if (T == 0) return LMOE_OK;  // an empty batch: nothing read or written
  if (y == nullptr || w == nullptr || out == nullptr) return LMOE_ERR_ARG;
  launch_combine(static_cast<const uint16_t*>(y), row_idx, w, T, k, H,
                 static_cast<const uint16_t*>(add), static_cast<uint16_t*>(out), stream);
  LMOE_RETURN_LAUNCH();
}
