// bf16 MFMA grouped "NT" GEMM for gfx950: C[m][n] = sum_k A[m][k] * W[n][k]
// with f32 accumulation, A rows gathered per slot group, W read from the slot
// bank ([P, N, K] row-major, K contiguous, i.e. the checkpoint layout).
//
// Work unit: a 128 x 128 output tile computed by 256 threads (2 x 2 waves of
// 64 x 64), K staged through LDS 64 columns at a time with a register
// prefetch of the next K step (one barrier per step).  Matrix core op:
// v_mfma_f32_32x32x16_bf16 (lane l holds A[l%32][8*(l/32)..+8],
// B[8*(l/32)..+8][l%32]; accumulator element r of lane l is
// C[8*(r/4) + 4*(l/32) + r%4][l%32]).
//
// Modes
//   kGateUp : W = W13_s [2I, H].  A tile of 128 gate columns is really 64
//             gate rows (i0..i0+63) and the matching 64 up rows (I+i0..), so
//             the epilogue forms act = silu(gate) * up in registers and
//             writes act[pos][i] (sorted position order).
//   kDown   : W = W2_s [H, I], A = act rows; writes y[pair][h] (flat pair).
//   kDense  : one group of M rows (router gate at large T); writes bf16/f32.
#pragma once

#include "lmoe_device.h"

namespace lmoe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

enum GemmMode { kGateUp = 0, kDown = 1, kDense = 2 };

constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kBK = 64;
constexpr int kLdsStride = kBK + 8;  // bf16 elements per LDS row (16 B pad)

struct GemmArgs {
  const uint16_t* a;      // x [T, K] (gate-up, dense) or act [pairs, K] (down)
  const uint16_t* w;      // slot bank base
  long long w_slot_stride;  // elements per slot
  int N;                  // output columns (gate-up: I; down: H; dense: E)
  int K;
  int I;                  // gate-up: offset of the up rows
  int topk;               // pairs per token
  const int32_t* offsets;       // [P+1]
  const int32_t* sorted_pairs;  // [pairs]
  const int32_t* tile_off;      // [P+1]
  const int32_t* meta;
  int P;
  int M_dense;            // dense: number of rows
  int block_m;            // rows per tile of tile_off (a multiple of kBM); grouped modes
  void* out;
  int out_f32;            // dense only
};

__device__ __forceinline__ int find_tile_slot(const int32_t* tile_off, int P,
                                              int tile) {
  // largest s with tile_off[s] <= tile and tile_off[s+1] > tile
  int lo = 0, hi = P;  // tile_off[lo] <= tile < tile_off[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (tile_off[mid] <= tile) lo = mid; else hi = mid;
  }
  return lo;
}

template <int MODE>
__global__ __launch_bounds__(256) void grouped_gemm_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][kBM * kLdsStride];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][kBN * kLdsStride];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;   // 0..1 : 64-row half
  const int wn = wave & 1;    // 0..1 : 64-col half (gate-up: 32 i each)

  // ---- work unit -> (slot, first row, rows) ----
  int slot = 0, row0 = 0, rows = 0;
  if (MODE == kDense) {
    row0 = blockIdx.x * kBM;
    if (row0 >= g.M_dense) return;
    rows = min(kBM, g.M_dense - row0);
  } else {
    // tile_off counts tiles of g.block_m rows; blockIdx.z picks the kBM-row
    // part of the tile this workgroup computes
    const int tile = blockIdx.x;
    if (tile >= g.meta[LMOE_META_TILES]) return;
    slot = find_tile_slot(g.tile_off, g.P, tile);
    const int p0 = g.offsets[slot];
    const int n = g.offsets[slot + 1] - p0;
    row0 = p0 + (tile - g.tile_off[slot]) * g.block_m + blockIdx.z * kBM;
    rows = min(kBM, p0 + n - row0);
    if (rows <= 0) return;
  }
  const int n0 = blockIdx.y * (MODE == kGateUp ? kBN / 2 : kBN);

  const uint16_t* wbase = g.w + static_cast<long long>(slot) * g.w_slot_stride;

  // ---- per-thread global load assignment: 4 rows x 16 B per operand ----
  // thread -> rows r = tid/8 + 32*q (q < 4), k chunk (tid%8)*8
  const int lr = tid >> 3;
  const int lk = (tid & 7) * 8;
  const uint16_t* a_src[4];
  bool a_ok[4];
  const uint16_t* b_src[4];
  bool b_ok[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = lr + 32 * q;
    a_ok[q] = r < rows;
    int arow = 0;
    if (a_ok[q]) {
      const int pos = row0 + r;
      if (MODE == kGateUp) arow = g.sorted_pairs[pos] / g.topk;
      else arow = pos;  // down: act row = sorted position; dense: row
    }
    a_src[q] = g.a + static_cast<long long>(arow) * g.K + lk;
    int wrow;
    if (MODE == kGateUp) wrow = (r < 64) ? (n0 + r) : (g.I + n0 + r - 64);
    else wrow = n0 + r;
    b_ok[q] = (MODE == kGateUp) ? ((r < 64 ? n0 + r : n0 + r - 64) < g.N)
                                : (wrow < g.N);
    b_src[q] = wbase + static_cast<long long>(b_ok[q] ? wrow : 0) * g.K + lk;
  }

  uint4 ra[4], rb[4];
  auto gload = [&](int kt) {
    const int koff = kt * kBK;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bool kin = koff + lk < g.K;
      ra[q] = (a_ok[q] && kin) ? *reinterpret_cast<const uint4*>(a_src[q] + koff)
                               : make_uint4(0u, 0u, 0u, 0u);
      rb[q] = (b_ok[q] && kin) ? *reinterpret_cast<const uint4*>(b_src[q] + koff)
                               : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = lr + 32 * q;
      *reinterpret_cast<uint4*>(&As[buf][r * kLdsStride + lk]) = ra[q];
      *reinterpret_cast<uint4*>(&Bs[buf][r * kLdsStride + lk]) = rb[q];
    }
  };

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int KT = (g.K + kBK - 1) / kBK;
  gload(0);
  sstore(0);
  __syncthreads();

  // fragment rows: A rows wm*64 + mi*32 + lane%32; B rows depend on mode
  const int frag_k = (lane >> 5) * 8;
  int brow[2];
  if (MODE == kGateUp) {
    brow[0] = wn * 32 + (lane & 31);        // gate rows 0..63 of the tile
    brow[1] = 64 + wn * 32 + (lane & 31);   // matching up rows
  } else {
    brow[0] = wn * 64 + (lane & 31);
    brow[1] = wn * 64 + 32 + (lane & 31);
  }

  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      bf16x8_t af[2], bfr[2];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) {
        const int r = wm * 64 + mi * 32 + (lane & 31);
        af[mi] = *reinterpret_cast<const bf16x8_t*>(
            &As[cur][r * kLdsStride + ks * 16 + frag_k]);
      }
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) {
        bfr[ni] = *reinterpret_cast<const bf16x8_t*>(
            &Bs[cur][brow[ni] * kLdsStride + ks * 16 + frag_k]);
      }
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              af[mi], bfr[ni], acc[mi][ni], 0, 0, 0);
    }
    if (kt + 1 < KT) sstore(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue ----
  const int col = lane & 31;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = wm * 64 + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      if (m >= rows) continue;
      const int pos = row0 + m;
      if (MODE == kGateUp) {
        const int i = n0 + wn * 32 + col;
        if (i < g.N) {
          reinterpret_cast<uint16_t*>(g.out)[static_cast<long long>(pos) * g.I + i] =
              swiglu_bf16(acc[mi][0][r], acc[mi][1][r]);
        }
      } else {
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
          const int n = n0 + wn * 64 + ni * 32 + col;
          if (n >= g.N) continue;
          const float v = acc[mi][ni][r];
          if (MODE == kDown) {
            const int pair = g.sorted_pairs[pos];
            reinterpret_cast<uint16_t*>(g.out)[static_cast<long long>(pair) * g.N + n] =
                static_cast<uint16_t>(f32_to_bf16_bits(v));
          } else if (g.out_f32) {
            reinterpret_cast<float*>(g.out)[static_cast<long long>(pos) * g.N + n] = v;
          } else {
            reinterpret_cast<uint16_t*>(g.out)[static_cast<long long>(pos) * g.N + n] =
                static_cast<uint16_t>(f32_to_bf16_bits(v));
          }
        }
      }
    }
  }
}

}  // namespace lmoe
