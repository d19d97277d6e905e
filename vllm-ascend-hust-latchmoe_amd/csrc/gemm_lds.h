// bf16 MFMA grouped "NT" GEMM for gfx950 with direct-to-LDS operand loads:
// C[m][n] = sum_k A[m][k] * W[n][k], f32 accumulation, A rows gathered per
// slot group, W read from the slot bank ([P, N, K] row-major, K contiguous).
//
// Block tile BM x BN, K staged BK (64 or 32) columns at a time through a
// STAGES-deep ring of LDS buffers.  Operands go HBM/L2 -> LDS with
// global_load_lds_dwordx4 (16 bytes per lane, no register staging): one
// instruction fills 1 KiB of LDS rows (BK 64: 8 rows of 128 bytes, lane l
// landing at row l/8, 16-byte chunk l%8; BK 32: 16 rows of 64 bytes, row l/4,
// chunk l%4).  LDS holds logical chunk c of row r at position c ^ sw(r), so
// the lane loads the chunk that belongs at its landing position:
//   BK 64: sw(r) = (r%8) ^ ((r/8)%2)
//   BK 32: sw(r) = ((r/2) ^ (r/8)) % 4
// A fragment read (32 rows, one chunk each) then hits distinct banks both per
// 8 lanes over 128 bytes and per 16 lanes over 256 bytes.  The 32-column
// stage halves the ring's footprint, so the same LDS holds twice the stages
// and twice the loads in flight ahead of the MFMAs.
//
// Waves form a WM x WN grid; a wave owns a (BM/WM) x (BN/WN) sub-tile as
// 32x32 blocks of v_mfma_f32_32x32x16_bf16 with the weight fragment as the
// first operand, i.e. the wave computes C^T: lane l holds W rows
// W[l%32][8*(l/32)..+8] and A rows A[l%32][8*(l/32)..+8], and accumulator
// element r of lane l is C[l%32][8*(r/4) + 4*(l/32) + r%4], four consecutive
// output columns per register quad.  Every output element accumulates its
// K/16 MFMA steps in increasing k, the same sequence as grouped_gemm_kernel,
// so both kernels give identical bits.
//
// Epilogue: the bf16 tile goes to LDS (8-byte writes) and leaves in 16-byte
// row-contiguous stores; the down mode's destination rows (pair ids) are
// read into LDS once at the start.
//
// Work order: the (row tile, column tile) items are split into 8 contiguous
// chunks, one per XCD (workgroup b runs on XCD b % 8), so the column tiles of
// one row tile and the row tiles of one slot meet in the same L2.
//
// Modes (as grouped_gemm_kernel): kGateUp forms act = silu(gate) * up from a
// B tile whose first BN/2 rows are gate rows i0.. and last BN/2 the matching
// up rows I+i0..; kDown writes y[pair][h] in flat pair order.
#pragma once

#include <type_traits>

#include "gemm_mfma.h"

namespace lmoe {

// Swizzle of staged row r (see the header): the chunk position that logical
// chunk c of row r occupies is c ^ lds_swz<BK>(r).
template <int BK>
__device__ __forceinline__ int lds_swz(int r) {
  static_assert(BK == 64 || BK == 32, "staged rows are 128 or 64 bytes");
  return BK == 64 ? ((r & 7) ^ ((r >> 3) & 1)) : (((r >> 1) ^ (r >> 3)) & 3);
}

template <int BM_, int BN_, int WM_, int WN_, int STAGES_, int BK_ = 64>
struct LdsTile {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_, STAGES = STAGES_;
  static constexpr int NW = WM * WN;
  static constexpr int THREADS = NW * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int NI = WTM / 32, NJ = WTN / 32;
  static constexpr int ROWB = BK * 2;        // bytes of one staged row
  static constexpr int CPR = BK / 8;         // 16-byte chunks per staged row
  static constexpr int RPL = 1024 / ROWB;    // rows one load instruction fills
  static constexpr int A_BYTES = BM * BK * 2, B_BYTES = BN * BK * 2;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int QA = A_BYTES / 1024 / NW;  // load instructions per wave per stage
  static constexpr int QB = B_BYTES / 1024 / NW;
  static constexpr int Q = QA + QB;
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be whole 32x32 blocks");
  static_assert(QA * NW * 1024 == A_BYTES && QB * NW * 1024 == B_BYTES,
                "operand tiles must split evenly into 1 KiB loads per wave");
  // output tile staged in LDS: BM rows x BNO bf16 (down: BN, gate-up: BN/2)
  static constexpr int out_cols(int mode) { return mode == kGateUp ? BN / 2 : BN; }
  static constexpr int out_pitch(int mode) { return out_cols(mode) * 2 + 16; }
  static constexpr int RING_BYTES = STAGES * STAGE_BYTES;
  static constexpr int OUT_BYTES = BM * (BN * 2 + 16);  // the larger (down) tile
  static constexpr int MAIN_BYTES = RING_BYTES > OUT_BYTES ? RING_BYTES : OUT_BYTES;
  static constexpr int LDS_BYTES = MAIN_BYTES + BM * 4;  // + destination row ids
  static_assert(STAGES >= 2 && LDS_BYTES <= 160 * 1024, "LDS footprint too large");
};

// Wait until at most N of this wave's vector-memory loads are in flight (and
// every LDS access has completed), then meet the other waves.  Inline asm so
// the compiler neither adds a full vmcnt(0) (as a workgroup fence would) nor
// moves LDS reads across the barrier.
template <int N>
__device__ __forceinline__ void vm_wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

__device__ __forceinline__ void load_lds16(const uint16_t* src, char* lds) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                   (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

__device__ __forceinline__ bf16x8_t lds_read16(const char* p) {
  return *reinterpret_cast<const bf16x8_t*>(p);
}

template <int MODE, class C>
__global__ __launch_bounds__(C::THREADS) void grouped_gemm_lds_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) char smem[C::LDS_BYTES];
  int* s_rowid = reinterpret_cast<int*>(smem + C::MAIN_BYTES);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave-uniform by construction; readfirstlane lets the compiler keep the
  // wave's tile coordinates (and the branches on them) scalar
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / C::WN;
  const int wn = wave % C::WN;

  // ---- work item: XCD-contiguous chunks of (row tile, column tile) ----
  // (kDense: one group of g.M_dense rows, no tile table)
  const int col_tile = (MODE == kGateUp) ? C::BN / 2 : C::BN;
  const int NT = (g.N + col_tile - 1) / col_tile;
  const int n_tiles = (MODE == kDense) ? (g.M_dense + C::BM - 1) / C::BM : g.meta[LMOE_META_TILES];
  const int total = n_tiles * NT;
  const int chunk = (total + 7) >> 3;
  const int jj = blockIdx.x >> 3;
  if (jj >= chunk) return;
  const int w = (blockIdx.x & 7) * chunk + jj;
  if (w >= total) return;
  const int tile = w / NT;
  const int n0 = (w - tile * NT) * col_tile;
  const int slot = (MODE == kDense) ? 0 : find_tile_slot(g.tile_off, g.P, tile);
  const int p0 = (MODE == kDense) ? 0 : g.offsets[slot];
  const int row0 = p0 + (tile - (MODE == kDense ? 0 : g.tile_off[slot])) * C::BM;
  const int rows = min(C::BM, (MODE == kDense ? g.M_dense : g.offsets[slot + 1]) - row0);
  const uint16_t* wbase = g.w + static_cast<long long>(slot) * g.w_slot_stride;
  if (MODE == kDown) {
    for (int t = tid; t < C::BM; t += C::THREADS)
      s_rowid[t] = g.sorted_pairs[row0 + (t < rows ? t : 0)];
  }

  // ---- per-lane source rows for this wave's load instructions ----
  // instruction q fills rows RPL*gq .. RPL*gq+RPL-1; the lane lands at row
  // RPL*gq + l/CPR, position l%CPR, and loads the logical chunk stored
  // there: (l%CPR) ^ sw(row)
  const int lrow = lane / C::CPR;
  const int lpos = lane % C::CPR;
  const uint16_t* a_src[C::QA];
  const uint16_t* b_src[C::QB];
#pragma unroll
  for (int q = 0; q < C::QA; ++q) {
    const int gq = wave * C::QA + q;
    const int r = gq * C::RPL + lrow;
    const int pos = row0 + (r < rows ? r : 0);
    const int arow = (MODE == kGateUp) ? g.sorted_pairs[pos] / g.topk : pos;
    const int lchunk = (lpos ^ lds_swz<C::BK>(r)) * 8;
    a_src[q] = g.a + static_cast<long long>(arow) * g.K + lchunk;
  }
#pragma unroll
  for (int q = 0; q < C::QB; ++q) {
    const int gq = wave * C::QB + q;
    const int r = gq * C::RPL + lrow;
    const int lchunk = (lpos ^ lds_swz<C::BK>(r)) * 8;
    int wrow;
    if (MODE == kGateUp) {
      const int half = r / (C::BN / 2);
      int i = n0 + r - half * (C::BN / 2);
      if (i >= g.N) i = n0;  // column past I: any valid row, output dropped
      wrow = half * g.I + i;
    } else {
      wrow = n0 + r < g.N ? n0 + r : n0;
    }
    b_src[q] = wbase + static_cast<long long>(wrow) * g.K + lchunk;
  }

  auto issue = [&](int kt, int buf) {
    char* st = smem + buf * C::STAGE_BYTES;
    const int koff = kt * C::BK;
#pragma unroll
    for (int q = 0; q < C::QA; ++q) load_lds16(a_src[q] + koff, st + (wave * C::QA + q) * 1024);
#pragma unroll
    for (int q = 0; q < C::QB; ++q)
      load_lds16(b_src[q] + koff, st + C::A_BYTES + (wave * C::QB + q) * 1024);
  };

  f32x16_t acc[C::NI][C::NJ];
#pragma unroll
  for (int i = 0; i < C::NI; ++i)
#pragma unroll
    for (int j = 0; j < C::NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // fragment reads: row base + l%32 (bases are multiples of 32, so
  // sw(row) = sw(l%32)), logical chunk 2*ks + l/32
  const int frow = lane & 31;
  const int fhi = lane >> 5;
  const int fsw = lds_swz<C::BK>(frow);
  int a_off[C::NI], b_off[C::NJ];
#pragma unroll
  for (int i = 0; i < C::NI; ++i) a_off[i] = (wm * C::WTM + i * 32 + frow) * C::ROWB;
#pragma unroll
  for (int j = 0; j < C::NJ; ++j) {
    int br;
    if (MODE == kGateUp) {
      constexpr int HJ = C::NJ / 2;
      br = (j < HJ) ? wn * (C::WTN / 2) + j * 32
                    : C::BN / 2 + wn * (C::WTN / 2) + (j - HJ) * 32;
    } else {
      br = wn * C::WTN + j * 32;
    }
    b_off[j] = C::A_BYTES + (br + frow) * C::ROWB;
  }
  // 32-row blocks of this wave that hold at least one valid row
  const int wave_rows = rows - wm * C::WTM;
  const int ni_live = wave_rows <= 0 ? 0 : min(C::NI, (wave_rows + 31) >> 5);

  const int KT = g.K / C::BK;
#pragma unroll
  for (int s = 0; s < C::STAGES - 1; ++s)
    if (s < KT) issue(s, s);

  // NL = 32-row blocks computed; instantiated per count so the k loop is
  // straight-line code (blocks past the valid rows would only add discarded
  // rows, so a partial tile rounds NL up to 1, NI/2 or NI)
  auto main_loop = [&](auto nl_tag) {
    constexpr int NL = decltype(nl_tag)::value;
    int buf = 0;
    for (int kt = 0; kt < KT; ++kt) {
      // stage kt landed (loads of the later stages may stay in flight) and
      // every wave is done with the buffer the next issue overwrites
      const int ahead = KT - 1 - kt;
      if (C::STAGES >= 4 && ahead >= 2) vm_wait_barrier<(C::STAGES >= 4 ? 2 : 0) * C::Q>();
      else if (C::STAGES >= 3 && ahead >= 1) vm_wait_barrier<(C::STAGES >= 3 ? 1 : 0) * C::Q>();
      else vm_wait_barrier<0>();
      if (kt + C::STAGES - 1 < KT) {
        int nb = buf + C::STAGES - 1;
        if (nb >= C::STAGES) nb -= C::STAGES;
        issue(kt + C::STAGES - 1, nb);
      }
      if constexpr (NL > 0) {
        // fragments double-buffered in registers: the reads of k16 step
        // ks+1 are in flight while the MFMAs of step ks run
        const char* st = smem + buf * C::STAGE_BYTES;
        bf16x8_t bfr[2][C::NJ], af[2][NL];
        auto read_frags = [&](int ks, int slot) {
          const int cpos = ((2 * ks + fhi) ^ fsw) * 16;
#pragma unroll
          for (int j = 0; j < C::NJ; ++j) bfr[slot][j] = lds_read16(st + b_off[j] + cpos);
#pragma unroll
          for (int i = 0; i < NL; ++i) af[slot][i] = lds_read16(st + a_off[i] + cpos);
        };
        read_frags(0, 0);
#pragma unroll
        for (int ks = 0; ks < C::BK / 16; ++ks) {
          if (ks + 1 < C::BK / 16) read_frags(ks + 1, (ks + 1) & 1);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int i = 0; i < NL; ++i)
#pragma unroll
            for (int j = 0; j < C::NJ; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[ks & 1][j], af[ks & 1][i],
                                                                   acc[i][j], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      buf = (buf + 1 == C::STAGES) ? 0 : buf + 1;
    }
  };
  constexpr int kHalf = C::NI >= 4 ? C::NI / 2 : C::NI;
  if (ni_live > kHalf) main_loop(std::integral_constant<int, C::NI>{});
  else if (ni_live > 1) main_loop(std::integral_constant<int, kHalf>{});
  else if (ni_live == 1) main_loop(std::integral_constant<int, 1>{});
  else main_loop(std::integral_constant<int, 0>{});

  // ---- kDense with f32 output: straight from the accumulators (lane l%32
  // holds row 32 i + l%32, its 16 values are 4 runs of 4 columns) ----
  if constexpr (MODE == kDense) {
    if (g.out_f32) {
      const int m0 = wm * C::WTM + frow;
      const int cb = wn * C::WTN + 4 * fhi;
#pragma unroll
      for (int i = 0; i < C::NI; ++i) {
        const int m = m0 + 32 * i;
        if (i >= ni_live || m >= rows) continue;
        float* orow = reinterpret_cast<float*>(g.out) + static_cast<long long>(row0 + m) * g.N;
#pragma unroll
        for (int j = 0; j < C::NJ; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int n = n0 + cb + j * 32 + 8 * q;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (n + e < g.N) orow[n + e] = acc[i][j][4 * q + e];
          }
      }
      return;
    }
  }

  // ---- epilogue: bf16 tile -> LDS -> 16-byte row stores ----
  constexpr int BNO = C::out_cols(MODE);
  constexpr int PITCH = C::out_pitch(MODE);
  vm_wait_barrier<0>();  // every wave is done reading the operand ring
  {
    const int m = wm * C::WTM + frow;  // + 32 * i
    const int cb = (MODE == kGateUp ? wn * (C::WTN / 2) : wn * C::WTN) + 4 * fhi;
#pragma unroll
    for (int i = 0; i < C::NI; ++i) {
      if (i >= ni_live) continue;
      char* rowp = smem + (m + 32 * i) * PITCH;
      constexpr int JO = (MODE == kGateUp) ? C::NJ / 2 : C::NJ;
#pragma unroll
      for (int j = 0; j < JO; ++j) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          uint32_t lo, hi;
          if (MODE == kGateUp) {
            lo = swiglu_bf16x2(acc[i][j][4 * q + 0], acc[i][j + JO][4 * q + 0],
                               acc[i][j][4 * q + 1], acc[i][j + JO][4 * q + 1]);
            hi = swiglu_bf16x2(acc[i][j][4 * q + 2], acc[i][j + JO][4 * q + 2],
                               acc[i][j][4 * q + 3], acc[i][j + JO][4 * q + 3]);
          } else {
            lo = pack_bf16x2(acc[i][j][4 * q + 0], acc[i][j][4 * q + 1]);
            hi = pack_bf16x2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
          }
          *reinterpret_cast<uint2*>(rowp + (cb + j * 32 + 8 * q) * 2) = make_uint2(lo, hi);
        }
      }
    }
  }
  vm_wait_barrier<0>();
  constexpr int CPR = BNO / 8;  // 16-byte chunks per output row
  for (int e = tid; e < C::BM * CPR; e += C::THREADS) {
    const int m = e / CPR;
    if (m >= rows) break;  // rows are filled in order, so later e are past too
    const int c = e - m * CPR;
    const int n = n0 + c * 8;
    if (n >= g.N) continue;
    const uint4 v = *reinterpret_cast<const uint4*>(smem + m * PITCH + c * 16);
    uint16_t* dst;
    if (MODE == kGateUp) {
      dst = reinterpret_cast<uint16_t*>(g.out) + static_cast<long long>(row0 + m) * g.I + n;
    } else if (MODE == kDense) {
      dst = reinterpret_cast<uint16_t*>(g.out) + static_cast<long long>(row0 + m) * g.N + n;
    } else {
      dst = reinterpret_cast<uint16_t*>(g.out) + static_cast<long long>(s_rowid[m]) * g.N + n;
    }
    *reinterpret_cast<uint4*>(dst) = v;
  }
}

// 64-row x 128-column tiles with four stages of operands in flight: for a
// few dozen tiles whose time is the K chain (the router gate over many
// tokens)
using SmallTile = LdsTile<64, 128, 1, 2, 4>;

// Upper bound on launched workgroups for up to ub_tiles row tiles: the grid
// is a multiple of 8 with ceil(items / 8) workgroups per XCD.
__host__ inline int lds_gemm_grid(int ub_tiles, int n_col_tiles) {
  const long long items = static_cast<long long>(ub_tiles) * n_col_tiles;
  return static_cast<int>(8 * ((items + 7) / 8));
}

}  // namespace lmoe
