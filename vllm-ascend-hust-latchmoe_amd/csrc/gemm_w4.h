// bf16 MFMA grouped "NT" GEMM for gfx950, 256 x 256 block tile, four waves:
// C[m][n] = sum_k A[m][k] * W[n][k], f32 accumulation, A rows gathered per
// slot group, W read from the slot bank ([P, N, K] row-major, K contiguous).
//
// One wave per SIMD, each owning a 128 x 128 sub-tile (16 accumulator
// blocks of v_mfma_f32_32x32x16_bf16, 256 f32 per lane).  Per k16 step a wave
// reads 4 A + 4 B fragments (8 KiB) for 16 MFMAs, i.e. 64 B/clk of LDS per
// CU at the MFMA peak.
//
// Operands travel HBM/L2 -> LDS with buffer_load_dwordx4 ... lds (16 bytes
// per lane, no register staging) into a ring of STAGES buffers of BK = 32
// columns (A 256 x 64 B, B 256 x 64 B = 32 KiB per stage).  One load
// instruction fills 16 LDS rows of 64 bytes, lane l landing at row l/4,
// position l%4; LDS holds logical 16-byte chunk c of row r at position
// c ^ sw(r), sw(r) = ((r/2)%4) ^ ((r/8)%2), which makes a fragment read (32
// rows, one chunk each) hit distinct banks per 8 lanes over 128 bytes and
// per 16 lanes over 256 bytes.
//
// Pipeline: stage kt+STAGES is issued into stage kt's buffer right after
// the barrier that ends stage kt's reads, so about STAGES-1 stages of MFMA
// time cover the load latency.  The barrier sits before the last k16 step of
// a stage: the first fragments of stage kt+1 are read while that step's
// MFMAs run, so the MFMA pipe does not drain at stage boundaries.
//
// The MFMA takes the weight fragment as its first operand (C^T): lane l
// holds row l%32 of an A block and accumulator element r is
// C[l%32][8*(r/4) + 4*(l/32) + r%4].  Every output element accumulates its
// K/16 MFMA steps in increasing k, the same sequence as grouped_gemm_kernel,
// so both kernels give identical bits.
//
// Epilogue: the bf16 tile goes to LDS (8-byte writes) and leaves in 16-byte
// row-contiguous stores; the down mode's destination rows (pair ids) are
// read into LDS at the start.
//
// Work order: the (row tile, column tile) items are split into 8 contiguous
// chunks, one per XCD (workgroup b runs on XCD b % 8), so the column tiles of
// one row tile and the row tiles of one slot meet in the same L2.
//
// Modes (as grouped_gemm_kernel): kGateUp forms act = silu(gate) * up from a
// B tile whose rows 0..127 are gate rows i0.. and rows 128..255 the matching
// up rows I+i0..; kDown writes y[pair][h] in flat pair order.
#pragma once

#include <type_traits>

#include "gemm_mfma.h"

namespace lmoe {

struct W4 {
  static constexpr int BM = 256, BN = 256, BK = 32, STAGES = 4;
  static constexpr int WM = 2, WN = 2, NW = 4, THREADS = 256;
  static constexpr int WTM = 128, WTN = 128, NI = 4, NJ = 4;
  static constexpr int KS = BK / 16;                  // k16 steps per stage
  static constexpr int ROW_BYTES = BK * 2;            // 64
  static constexpr int A_BYTES = BM * ROW_BYTES;      // 16 KiB
  static constexpr int B_BYTES = BN * ROW_BYTES;      // 16 KiB
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int QA = A_BYTES / 1024 / NW;      // 4 loads per wave per stage
  static constexpr int QB = B_BYTES / 1024 / NW;      // 4
  static constexpr int Q = QA + QB;
  static constexpr int RING_BYTES = STAGES * STAGE_BYTES;   // 128 KiB
  static constexpr int out_cols(int mode) { return mode == kGateUp ? BN / 2 : BN; }
  static constexpr int out_pitch(int mode) { return out_cols(mode) * 2 + 16; }
  static constexpr int OUT_BYTES = BM * (BN * 2 + 16);
  static constexpr int MAIN_BYTES = RING_BYTES > OUT_BYTES ? RING_BYTES : OUT_BYTES;
  static constexpr int LDS_BYTES = MAIN_BYTES + BM * 4;
  static_assert(LDS_BYTES <= 160 * 1024, "LDS footprint too large");
};

// s_waitcnt immediate (gfx9 encoding): vmcnt <= vm, lgkmcnt <= lgkm, expcnt any
constexpr int waitcnt_imm(int vm, int lgkm) {
  return (vm & 0xf) | ((vm >> 4) << 14) | (0x7 << 4) | ((lgkm & 0xf) << 8);
}

// Wait until at most `stages` stages (of Q loads each) of this wave's
// operand loads are in flight and its LDS reads are done, then meet the
// other waves.  The waitcnt builtin keeps the compiler's own counter model
// informed; the empty asm statements keep memory operations on their side.
template <int Q>
__device__ __forceinline__ void stage_barrier(int stages) {
  if (stages >= 3) __builtin_amdgcn_s_waitcnt(waitcnt_imm(3 * Q, 0));
  else if (stages == 2) __builtin_amdgcn_s_waitcnt(waitcnt_imm(2 * Q, 0));
  else if (stages == 1) __builtin_amdgcn_s_waitcnt(waitcnt_imm(Q, 0));
  else __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
  // raw buffer over 2 GiB - 1 bytes (offsets are checked on the host)
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           0x7fffffff, 0x00020000);
}

__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t r, char* lds, int voff,
                                                  int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16,
                                           voff, soff, 0, 0);
}

__device__ __forceinline__ int w4_swizzle(int r) { return ((r >> 1) & 3) ^ ((r >> 3) & 1); }

template <int MODE>
__global__ __launch_bounds__(W4::THREADS) __attribute__((amdgpu_waves_per_eu(1, 1)))
void grouped_gemm_w4_kernel(GemmArgs g) {
  using C = W4;
  __shared__ __attribute__((aligned(1024))) char smem[C::LDS_BYTES];
  int* s_rowid = reinterpret_cast<int*>(smem + C::MAIN_BYTES);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1;
  const int wn = wave & 1;

  // ---- work item: XCD-contiguous chunks of (row tile, column tile) ----
  const int col_tile = (MODE == kGateUp) ? C::BN / 2 : C::BN;
  const int NT = (g.N + col_tile - 1) / col_tile;
  const int total = g.meta[LMOE_META_TILES] * NT;
  const int chunk = (total + 7) >> 3;
  const int jj = blockIdx.x >> 3;
  if (jj >= chunk) return;
  const int w = (blockIdx.x & 7) * chunk + jj;
  if (w >= total) return;
  const int tile = w / NT;
  const int n0 = (w - tile * NT) * col_tile;
  const int slot = find_tile_slot(g.tile_off, g.P, tile);
  const int p0 = g.offsets[slot];
  const int row0 = p0 + (tile - g.tile_off[slot]) * C::BM;
  const int rows = min(C::BM, g.offsets[slot + 1] - row0);
  if (MODE == kDown) {
    for (int t = tid; t < C::BM; t += C::THREADS)
      s_rowid[t] = g.sorted_pairs[row0 + (t < rows ? t : 0)];
  }

  // ---- per-lane buffer offsets of this wave's load instructions ----
  // instruction q fills rows 16*gq .. 16*gq+15: the lane lands at row
  // 16*gq + l/4, position l%4, and loads logical chunk (l%4) ^ sw(l/4)
  const int lrow = lane >> 2;
  const int lchunk_bytes = ((lane & 3) ^ w4_swizzle(lrow)) * 16;
  const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(g.a);
  const __amdgpu_buffer_rsrc_t b_rsrc =
      make_rsrc(g.w + static_cast<long long>(slot) * g.w_slot_stride);
  const int krow_bytes = g.K * 2;
  int a_voff[C::QA], b_voff[C::QB];
#pragma unroll
  for (int q = 0; q < C::QA; ++q) {
    const int r = (wave * C::QA + q) * 16 + lrow;
    const int pos = row0 + (r < rows ? r : 0);
    const int arow = (MODE == kGateUp) ? g.sorted_pairs[pos] / g.topk : pos;
    a_voff[q] = arow * krow_bytes + lchunk_bytes;
  }
#pragma unroll
  for (int q = 0; q < C::QB; ++q) {
    const int r = (wave * C::QB + q) * 16 + lrow;
    int wrow;
    if (MODE == kGateUp) {
      const int half = r >> 7;
      int i = n0 + (r & 127);
      if (i >= g.N) i = n0;  // column past I: any valid row, output dropped
      wrow = half * g.I + i;
    } else {
      wrow = n0 + r < g.N ? n0 + r : n0;
    }
    b_voff[q] = wrow * krow_bytes + lchunk_bytes;
  }

  auto issue = [&](int kt, int buf) {
    char* st = smem + buf * C::STAGE_BYTES;
    const int soff = kt * C::ROW_BYTES;
#pragma unroll
    for (int q = 0; q < C::QA; ++q)
      buffer_load_lds16(a_rsrc, st + (wave * C::QA + q) * 1024, a_voff[q], soff);
#pragma unroll
    for (int q = 0; q < C::QB; ++q)
      buffer_load_lds16(b_rsrc, st + C::A_BYTES + (wave * C::QB + q) * 1024, b_voff[q], soff);
  };

  f32x16_t acc[C::NI][C::NJ];
#pragma unroll
  for (int i = 0; i < C::NI; ++i)
#pragma unroll
    for (int j = 0; j < C::NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // fragment rows: block base (multiple of 32) + l%32, so sw(row) = sw(l%16)
  const int frow = lane & 31;
  const int fhi = lane >> 5;
  const int fsw = w4_swizzle(lane & 15);
  int a_off[C::NI], b_off[C::NJ];
#pragma unroll
  for (int i = 0; i < C::NI; ++i) a_off[i] = (wm * C::WTM + i * 32 + frow) * C::ROW_BYTES;
#pragma unroll
  for (int j = 0; j < C::NJ; ++j) {
    const int br = (MODE == kGateUp) ? ((j >> 1) * 128 + wn * 64 + (j & 1) * 32)
                                     : (wn * C::WTN + j * 32);
    b_off[j] = C::A_BYTES + (br + frow) * C::ROW_BYTES;
  }
  const int wave_rows = rows - wm * C::WTM;
  const int ni_live = wave_rows <= 0 ? 0 : min(C::NI, (wave_rows + 31) >> 5);

  const int KT = g.K / C::BK;
#pragma unroll
  for (int s = 0; s < C::STAGES; ++s)
    if (s < KT) issue(s, s);
  stage_barrier<C::Q>(min(C::STAGES - 1, KT - 1));

  // NL = 32-row blocks computed (1, 2 or 4; rounding a partial tile up
  // only adds discarded rows); instantiated per count so the k loop is
  // straight-line code.
  auto main_loop = [&](auto nl_tag) {
    constexpr int NL = decltype(nl_tag)::value;
    bf16x8_t fb[2][C::NJ], fa[2][NL > 0 ? NL : 1];
    auto read_frags = [&](int buf, int ks, int set) {
      const char* st = smem + buf * C::STAGE_BYTES;
      const int cpos = ((2 * ks + fhi) ^ fsw) * 16;
#pragma unroll
      for (int j = 0; j < C::NJ; ++j)
        fb[set][j] = *reinterpret_cast<const bf16x8_t*>(st + b_off[j] + cpos);
#pragma unroll
      for (int i = 0; i < NL; ++i)
        fa[set][i] = *reinterpret_cast<const bf16x8_t*>(st + a_off[i] + cpos);
    };
    auto mfma_block = [&](int set) {
#pragma unroll
      for (int i = 0; i < NL; ++i)
#pragma unroll
        for (int j = 0; j < C::NJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[set][j], fa[set][i],
                                                               acc[i][j], 0, 0, 0);
    };
    if constexpr (NL > 0) read_frags(0, 0, 0);
    int buf = 0;
    for (int kt = 0; kt < KT; ++kt) {
      // k16 step 0 of stage kt (fragments in set 0); step 1 read meanwhile
      if constexpr (NL > 0) {
        read_frags(buf, 1, 1);
        mfma_block(0);
      }
      // stage kt+1 landed, everyone's reads of stage kt done
      stage_barrier<C::Q>(min(C::STAGES - 2, KT - 2 - kt));
      if (kt + C::STAGES < KT) issue(kt + C::STAGES, buf);
      const int nbuf = (buf + 1 == C::STAGES) ? 0 : buf + 1;
      if constexpr (NL > 0) {
        if (kt + 1 < KT) read_frags(nbuf, 0, 0);
        mfma_block(1);
      }
      buf = nbuf;
    }
  };
  if (ni_live > 2) main_loop(std::integral_constant<int, 4>{});
  else if (ni_live == 2) main_loop(std::integral_constant<int, 2>{});
  else if (ni_live == 1) main_loop(std::integral_constant<int, 1>{});
  else main_loop(std::integral_constant<int, 0>{});

  // ---- epilogue: bf16 tile -> LDS -> 16-byte row stores ----
  constexpr int BNO = C::out_cols(MODE);
  constexpr int PITCH = C::out_pitch(MODE);
  stage_barrier<C::Q>(0);  // every wave is done with the operand ring
  {
    const int cb = (MODE == kGateUp ? wn * 64 : wn * C::WTN) + 4 * fhi;
#pragma unroll
    for (int i = 0; i < C::NI; ++i) {
      if (i >= ni_live) continue;
      char* rowp = smem + (wm * C::WTM + 32 * i + frow) * PITCH;
      constexpr int JO = (MODE == kGateUp) ? C::NJ / 2 : C::NJ;
#pragma unroll
      for (int j = 0; j < JO; ++j) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          uint32_t lo, hi;
          if (MODE == kGateUp) {
            // gate block j (j = 0,1) pairs with up block j + 2
            lo = static_cast<uint32_t>(swiglu_bf16(acc[i][j][4 * q + 0], acc[i][j + 2][4 * q + 0])) |
                 (static_cast<uint32_t>(swiglu_bf16(acc[i][j][4 * q + 1], acc[i][j + 2][4 * q + 1])) << 16);
            hi = static_cast<uint32_t>(swiglu_bf16(acc[i][j][4 * q + 2], acc[i][j + 2][4 * q + 2])) |
                 (static_cast<uint32_t>(swiglu_bf16(acc[i][j][4 * q + 3], acc[i][j + 2][4 * q + 3])) << 16);
          } else {
            lo = pack_bf16x2(acc[i][j][4 * q + 0], acc[i][j][4 * q + 1]);
            hi = pack_bf16x2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
          }
          *reinterpret_cast<uint2*>(rowp + (cb + j * 32 + 8 * q) * 2) = make_uint2(lo, hi);
        }
      }
    }
  }
  stage_barrier<C::Q>(0);
  constexpr int CPR = BNO / 8;  // 16-byte chunks per output row
  for (int e = tid; e < C::BM * CPR; e += C::THREADS) {
    const int m = e / CPR;
    if (m >= rows) break;  // rows are visited in order: the rest are past too
    const int c = e - m * CPR;
    const int n = n0 + c * 8;
    if (n >= g.N) continue;
    const uint4 v = *reinterpret_cast<const uint4*>(smem + m * PITCH + c * 16);
    uint16_t* dst;
    if (MODE == kGateUp) {
      dst = reinterpret_cast<uint16_t*>(g.out) + static_cast<long long>(row0 + m) * g.I + n;
    } else {
      dst = reinterpret_cast<uint16_t*>(g.out) + static_cast<long long>(s_rowid[m]) * g.N + n;
    }
    *reinterpret_cast<uint4*>(dst) = v;
  }
}

// Launch size for up to ub_tiles row tiles: a multiple of 8 workgroups with
// ceil(items / 8) per XCD.
__host__ inline int w4_grid(int ub_tiles, int n_col_tiles) {
  const long long items = static_cast<long long>(ub_tiles) * n_col_tiles;
  return static_cast<int>(8 * ((items + 7) / 8));
}

}  // namespace lmoe
