// Prefill grouped GEMM with the work split evenly over the CUs.
//
// The unit of work is a block of 32 output columns of one row tile (a slot's
// rows, up to BM = 320 of them: one tile covers a slot of up to 320 pairs,
// the typical ~256 of a prefill wave plus its spread).  Blocks are grouped
// into units of up to BN/2 (gate-up) or BN (down) columns, aligned within
// the row tile.  The grid holds one workgroup per CU, and each runs whole
// units (a unit's time is set by its K loop, ~2.5 us per 64 K-columns
// whatever its width, so narrower pieces of a unit would not finish sooner).
// A slot of up to 320 pairs is one row tile, so the usual prefill slot (~256
// pairs plus spread) streams each weight block once; the 256-row tiles of
// grouped_gemm_lds_kernel cut such slots into a full tile and a remainder
// tile that streams the same weights again.  The full Qwen3-shaped layer
// (128 slots, 6 gate-up units per row tile) is exactly 3 units per CU.
//
// Each XCD (workgroup b runs on XCD b % 8) owns an eighth of the units, in
// row-tile order, and its workgroups take them round-robin, so the units of
// one row tile run at the same time on one XCD and read their activation
// rows through its L2 once.  Assigning each workgroup a contiguous range
// instead ran a row tile's units one after another on one CU, re-reading the
// activation rows from HBM each time: the DeepSeek-V3-style prefill (16
// gate-up units per row tile) took 6.8 ms against 5.2 ms round-robin.
//
// A sub-tile is the 256-row kernel's tile (grouped_gemm_lds_kernel) grown to
// 320 rows: 8 waves as 2 x 4, each owning 160 x 64 (5 x 2 blocks of
// v_mfma_f32_32x32x16_bf16 with the weight fragment first), operands staged
// 64 K-columns at a time by direct-to-LDS loads into a two-stage ring (LDS
// rows of 128 bytes, swizzled as there).  A stage is 72 load instructions of
// 1 KiB (40 for the 320 activation rows, 32 for the 256 weight rows), dealt
// round-robin over the waves, and each wave waits for its own count.  A row
// tile of at most 128 rows is staged as 128 rows (16 + 32 loads, 48 KiB) in
// a three-stage ring of the same LDS, its waves owning 64 x 64: two stages of
// weight rows in flight instead of one.  Rows past the tile's valid rows and
// weight rows of columns outside the sub-tile load a valid row whose result
// is dropped, so the count per stage is fixed; waves without live columns
// skip their MFMAs, and a wave computes only its live 32-row blocks.  Every
// output element accumulates its K/16 MFMA steps in increasing k, the order
// of the other grouped kernels, so all of them (and both geometries) give
// identical bits.
//
// Epilogue through LDS as in grouped_gemm_lds_kernel; the down tile (320 x 256
// bf16 = 169 KB with padding) does not fit beside nothing else in 160 KB, so
// it leaves in two halves, one per wave row.
#pragma once

#include <type_traits>

#include "gemm_lds.h"

namespace lmoe {

// Stage geometry of a unit: BM staged activation rows, BN weight rows (gate-up:
// BN/2 gate rows then the matching up rows), 64 K-columns per stage, a ring
// of STAGES buffers, 8 waves as 2 x 4.
template <int BM_, int STAGES_>
struct PartStage {
  static constexpr int BM = BM_, BN = 256, BK = 64, STAGES = STAGES_, WM = 2, WN = 4;
  static constexpr int NW = WM * WN;
  static constexpr int THREADS = NW * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;  // 160 x 64 or 64 x 64
  static constexpr int NI = WTM / 32, NJ = WTN / 32;  // 5 x 2 or 2 x 2
  static constexpr int ROWB = BK * 2;                 // 128-byte staged rows
  static constexpr int CPR = BK / 8;                  // 8 chunks per row
  static constexpr int RPL = 1024 / ROWB;             // 8 rows per load
  static constexpr int A_LOADS = BM / RPL, B_LOADS = BN / RPL;  // 40 or 16, and 32
  static constexpr int LOADS = A_LOADS + B_LOADS;     // 72 or 48 per stage
  static constexpr int Q_HI = (LOADS + NW - 1) / NW;  // waves below LOADS % NW
  static constexpr int Q_LO = LOADS / NW;             // the others
  static constexpr int A_BYTES = BM * ROWB, B_BYTES = BN * ROWB;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;              // 72 or 48 KiB
  static constexpr int RING_BYTES = STAGES * STAGE_BYTES;            // 144 KiB either way
  static constexpr int GU_OUT_BYTES = BM * ((BN / 2) * 2 + 16);
  static constexpr int DN_OUT_BYTES = (BM / 2) * (BN * 2 + 16);      // per half
  static constexpr int MAIN_BYTES = RING_BYTES;
  static_assert(GU_OUT_BYTES <= MAIN_BYTES && DN_OUT_BYTES <= MAIN_BYTES, "epilogue staging");
  static_assert(A_LOADS * RPL == BM && B_LOADS * RPL == BN, "whole 1 KiB loads");
  static_assert(STAGES >= 2 && STAGES <= 4, "the stage waits allow up to two later stages");
  static_assert(WTM % 32 == 0 && WTM * 2 == BM, "the down epilogue stages one wave row at a time");
};

// The row tile (block_m 320) and the wide unit: two 72 KiB stages, one in
// flight while the other is multiplied.
using PartTile = PartStage<320, 2>;
// Units of row tiles with at most 128 rows (a slot of few pairs: the
// DeepSeek-V3-style prefill routes ~64 pairs to each of 256 experts): the
// same 144 KiB ring as three 48 KiB stages, so two stages of weight rows are
// in flight while the third is multiplied (that prefill: 5.17 -> 4.79 ms;
// 4.94 ms with the 128-row stages in two buffers).
using PartSkinny = PartStage<128, 3>;
constexpr int kPartMainBytes =
    PartTile::MAIN_BYTES > PartSkinny::MAIN_BYTES ? PartTile::MAIN_BYTES : PartSkinny::MAIN_BYTES;
constexpr int kPartLdsBytes = kPartMainBytes + PartTile::BM * 4;  // + destination row ids (down)
static_assert(kPartLdsBytes <= 160 * 1024, "LDS footprint too large");

// Columns (32-column blocks) of one sub-tile: gate-up BN/2 act columns
// (BN weight rows, gate then up), down BN output columns.
template <int MODE, class C>
constexpr int part_max_blocks() {
  return (MODE == kGateUp ? C::BN / 2 : C::BN) / 32;
}

// Chooses NL = n (the live 32-row blocks, 0..N) as a compile-time constant.
template <int N, class F>
__device__ __forceinline__ void part_live_dispatch(int n, F&& f) {
  if constexpr (N == 0) {
    f(std::integral_constant<int, 0>{});
  } else {
    if (n >= N) f(std::integral_constant<int, N>{});
    else part_live_dispatch<N - 1>(n, f);
  }
}

// One unit: output columns [n0, n0 + 32 * w) of the row tile whose rows
// [row0, row0 + rows) (rows <= S::BM) belong to `slot`, staged with geometry S.
template <int MODE, class S>
__device__ __forceinline__ void part_unit(const GemmArgs& g, char* smem, int* s_rowid, int tid,
                                          int lane, int wave, int slot, int row0, int rows,
                                          int n0, int w) {
  const int wm = wave / S::WN;
  const int wn = wave % S::WN;
  const int frow = lane & 31;
  const int fhi = lane >> 5;
  const int fsw = lds_swz<S::BK>(frow);
  const int KT = g.K / S::BK;
  const uint16_t* wbase = g.w + static_cast<long long>(slot) * g.w_slot_stride;
  if (MODE == kDown) {
    for (int t = tid; t < S::BM; t += S::THREADS)
      s_rowid[t] = g.sorted_pairs[row0 + (t < rows ? t : 0)];
  }

  // per-lane sources of this wave's load instructions: load t = wave + NW*q
  // of a stage fills LDS bytes [1024 t, 1024 t + 1024) of it, activation
  // rows for t < A_LOADS, weight rows after; the lane lands at row
  // RPL*t' + l/CPR, position l%CPR, and loads the logical chunk stored there.
  // Offsets are 32-bit element offsets from the operand bases: the launch
  // refuses (LMOE_ERR_SHAPE) an activation operand whose rows reach 2^31
  // elements (part_offsets_fit), and a weight offset stays inside one slot
  const int lrow = lane / S::CPR;
  const int lpos = lane % S::CPR;
  const int nq = wave < S::LOADS % S::NW ? S::Q_HI : S::Q_LO;
  int src[S::Q_HI];
#pragma unroll
  for (int q = 0; q < S::Q_HI; ++q) {
    const int t = wave + S::NW * q;
    if (t < S::A_LOADS) {
      const int rr = t * S::RPL + lrow;
      const int pos = row0 + (rr < rows ? rr : 0);
      const int arow = (MODE == kGateUp) ? g.sorted_pairs[pos] / g.topk : pos;
      src[q] = arow * g.K + (lpos ^ lds_swz<S::BK>(rr)) * 8;
    } else {
      const int rr = (t - S::A_LOADS) * S::RPL + lrow;
      int wrow;
      if (MODE == kGateUp) {
        // gate rows n0.., then the matching up rows I + n0..
        const int half = rr / (S::BN / 2);
        const int c = rr - half * (S::BN / 2);
        const int i = (c < 32 * w && n0 + c < g.N) ? n0 + c : n0;
        wrow = half * g.I + i;
      } else {
        wrow = (rr < 32 * w && n0 + rr < g.N) ? n0 + rr : n0;
      }
      src[q] = wrow * g.K + (lpos ^ lds_swz<S::BK>(rr)) * 8;
    }
  }

  auto issue = [&](int kt, int buf) {
    char* st = smem + buf * S::STAGE_BYTES;
    const int koff = kt * S::BK;
#pragma unroll
    for (int q = 0; q < S::Q_HI; ++q) {
      const int t = wave + S::NW * q;
      if (q < nq) load_lds16((t < S::A_LOADS ? g.a : wbase) + (src[q] + koff), st + t * 1024);
    }
  };
  // stage kt landed: at most `ahead` later stages of this wave's loads
  // (nq each) still in flight; then meet the other waves
  auto wait_stage = [&](int ahead) {
    if (nq == S::Q_HI) {
      if (ahead >= 2) vm_wait_barrier<2 * S::Q_HI>();
      else if (ahead == 1) vm_wait_barrier<S::Q_HI>();
      else vm_wait_barrier<0>();
    } else {
      if (ahead >= 2) vm_wait_barrier<2 * S::Q_LO>();
      else if (ahead == 1) vm_wait_barrier<S::Q_LO>();
      else vm_wait_barrier<0>();
    }
  };

  f32x16_t acc[S::NI][S::NJ];
#pragma unroll
  for (int i = 0; i < S::NI; ++i)
#pragma unroll
    for (int j = 0; j < S::NJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  int a_off[S::NI], b_off[S::NJ];
#pragma unroll
  for (int i = 0; i < S::NI; ++i) a_off[i] = (wm * S::WTM + i * 32 + frow) * S::ROWB;
#pragma unroll
  for (int j = 0; j < S::NJ; ++j) {
    int br;
    if (MODE == kGateUp) {
      constexpr int HJ = S::NJ / 2;
      br = (j < HJ) ? wn * (S::WTN / 2) + j * 32
                    : S::BN / 2 + wn * (S::WTN / 2) + (j - HJ) * 32;
    } else {
      br = wn * S::WTN + j * 32;
    }
    b_off[j] = S::A_BYTES + (br + frow) * S::ROWB;
  }
  // this wave's live 32-row blocks and whether any of its columns is live
  const int wave_rows = rows - wm * S::WTM;
  const bool cols_live = (MODE == kGateUp) ? (wn * (S::WTN / 2) < 32 * w) : (wn * S::WTN < 32 * w);
  const int ni_live = (wave_rows <= 0 || !cols_live) ? 0 : min(S::NI, (wave_rows + 31) >> 5);

#pragma unroll
  for (int s = 0; s < S::STAGES - 1; ++s)
    if (s < KT) issue(s, s);
  auto main_loop = [&](auto nl_tag) {
    constexpr int NL = decltype(nl_tag)::value;
    int buf = 0;
    for (int kt = 0; kt < KT; ++kt) {
      // stage kt landed and every wave is done with the buffer the next
      // issue overwrites (the one stage kt-1 was multiplied from)
      wait_stage(min(S::STAGES - 2, KT - 1 - kt));
      if (kt + S::STAGES - 1 < KT) {
        int nb = buf + S::STAGES - 1;
        if (nb >= S::STAGES) nb -= S::STAGES;
        issue(kt + S::STAGES - 1, nb);
      }
      if constexpr (NL > 0) {
        const char* st = smem + buf * S::STAGE_BYTES;
        bf16x8_t bfr[2][S::NJ], af[2][NL];
        auto read_frags = [&](int ks, int sl) {
          const int cpos = ((2 * ks + fhi) ^ fsw) * 16;
#pragma unroll
          for (int j = 0; j < S::NJ; ++j) bfr[sl][j] = lds_read16(st + b_off[j] + cpos);
#pragma unroll
          for (int i = 0; i < NL; ++i) af[sl][i] = lds_read16(st + a_off[i] + cpos);
        };
        read_frags(0, 0);
#pragma unroll
        for (int ks = 0; ks < S::BK / 16; ++ks) {
          if (ks + 1 < S::BK / 16) read_frags(ks + 1, (ks + 1) & 1);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int i = 0; i < NL; ++i)
#pragma unroll
            for (int j = 0; j < S::NJ; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[ks & 1][j], af[ks & 1][i],
                                                                   acc[i][j], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      buf = (buf + 1 == S::STAGES) ? 0 : buf + 1;
    }
  };
  // NL: 32-row blocks computed, exactly the live ones: a slot of ~256
  // pairs leaves the second wave row 3 of its 5 blocks, and MFMAs on
  // padding rows cost time (6% of the full-layer gate-up, same box)
  part_live_dispatch<S::NI>(ni_live, main_loop);

  // ---- epilogue: bf16 tile -> LDS -> 16-byte row stores ----
  vm_wait_barrier<0>();  // every wave is done reading the operand ring
  const int cb_base = (MODE == kGateUp ? wn * (S::WTN / 2) : wn * S::WTN) + 4 * fhi;
  const int n_end = min(g.N, n0 + 32 * w);
  if constexpr (MODE == kGateUp) {
    constexpr int PITCH = (S::BN / 2) * 2 + 16;
    constexpr int HJ = S::NJ / 2;
    const int m = wm * S::WTM + frow;
#pragma unroll
    for (int i = 0; i < S::NI; ++i) {
      if (i >= ni_live) continue;
      char* rowp = smem + (m + 32 * i) * PITCH;
#pragma unroll
      for (int j = 0; j < HJ; ++j) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t lo = swiglu_bf16x2(acc[i][j][4 * q + 0], acc[i][j + HJ][4 * q + 0],
                                            acc[i][j][4 * q + 1], acc[i][j + HJ][4 * q + 1]);
          const uint32_t hi = swiglu_bf16x2(acc[i][j][4 * q + 2], acc[i][j + HJ][4 * q + 2],
                                            acc[i][j][4 * q + 3], acc[i][j + HJ][4 * q + 3]);
          *reinterpret_cast<uint2*>(rowp + (cb_base + j * 32 + 8 * q) * 2) = make_uint2(lo, hi);
        }
      }
    }
    vm_wait_barrier<0>();
    constexpr int CPR = (S::BN / 2) / 8;  // 16-byte chunks per staged row
    for (int e = tid; e < S::BM * CPR; e += S::THREADS) {
      const int mm = e / CPR;
      if (mm >= rows) break;
      const int c = e - mm * CPR;
      const int n = n0 + c * 8;
      if (n >= n_end) continue;
      const uint4 v = *reinterpret_cast<const uint4*>(smem + mm * PITCH + c * 16);
      *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(g.out) +
                                static_cast<long long>(row0 + mm) * g.I + n) = v;
    }
    vm_wait_barrier<0>();  // the staged rows are read before the next sub-tile loads
  } else {
    constexpr int PITCH = S::BN * 2 + 16;
    constexpr int CPR = S::BN / 8;
#pragma unroll
    for (int h = 0; h < S::WM; ++h) {
      if (wm == h) {
#pragma unroll
        for (int i = 0; i < S::NI; ++i) {
          if (i >= ni_live) continue;
          char* rowp = smem + (frow + 32 * i) * PITCH;
#pragma unroll
          for (int j = 0; j < S::NJ; ++j) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const uint32_t lo = pack_bf16x2(acc[i][j][4 * q + 0], acc[i][j][4 * q + 1]);
              const uint32_t hi = pack_bf16x2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
              *reinterpret_cast<uint2*>(rowp + (cb_base + j * 32 + 8 * q) * 2) =
                  make_uint2(lo, hi);
            }
          }
        }
      }
      vm_wait_barrier<0>();
      const int hrows = min(S::WTM, rows - h * S::WTM);
      for (int e = tid; e < S::WTM * CPR; e += S::THREADS) {
        const int mm = e / CPR;
        if (mm >= hrows) break;
        const int c = e - mm * CPR;
        const int n = n0 + c * 8;
        if (n >= n_end) continue;
        const uint4 v = *reinterpret_cast<const uint4*>(smem + mm * PITCH + c * 16);
        *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(g.out) +
                                  static_cast<long long>(s_rowid[h * S::WTM + mm]) * g.N + n) = v;
      }
      vm_wait_barrier<0>();  // staged rows read before the next half / sub-tile
    }
  }
}

template <int MODE, class C>
__global__ __launch_bounds__(C::THREADS) void grouped_gemm_part_kernel(GemmArgs g) {
  static_assert(PartSkinny::THREADS == C::THREADS && PartSkinny::BN == C::BN,
                "both unit geometries share the workgroup and the column blocks");
  __shared__ __attribute__((aligned(1024))) char smem[kPartLdsBytes];
  int* s_rowid = reinterpret_cast<int*>(smem + kPartMainBytes);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int MAXB = part_max_blocks<MODE, C>();

  // ---- this workgroup's units ----
  // units: MAXB-block column groups of a row tile, aligned within it (the
  // last one of a row tile may be narrower), numbered row-major (tile,
  // unit).  XCD x (workgroup b runs on XCD b % 8) owns the units
  // [U * x / 8, U * (x + 1) / 8), and its workgroups take them round-robin:
  // local workgroup j runs units ux0 + j, ux0 + j + G/8, ...  So the units of
  // one row tile, which read the same activation rows, run at the same time
  // on one XCD and meet in its L2, instead of one after another.
  const int NB = (g.N + 31) >> 5;
  const int UPT = (NB + MAXB - 1) / MAXB;  // units per row tile
  const long long U = static_cast<long long>(g.meta[LMOE_META_TILES]) * UPT;
  const int GX = gridDim.x >> 3;  // workgroups per XCD (the grid is a multiple of 8)
  const int xcd = blockIdx.x & 7;
  const long long ux1 = U * (xcd + 1) / 8;

  for (long long u = U * xcd / 8 + (blockIdx.x >> 3); u < ux1; u += GX) {
    // ---- sub-tile: row tile `tile`, output columns [32 cb, 32 (cb + w)) ----
    const int tile = static_cast<int>(u / UPT);
    const int cb = static_cast<int>(u - static_cast<long long>(tile) * UPT) * MAXB;
    // one unit: up to MAXB blocks, ending at the row tile's end
    const int w = min(MAXB, NB - cb);
    const int slot = find_tile_slot(g.tile_off, g.P, tile);
    const int p0 = g.offsets[slot];
    const int row0 = p0 + (tile - g.tile_off[slot]) * C::BM;
    const int rows = min(C::BM, g.offsets[slot + 1] - row0);
    // rows is uniform over the workgroup, and so is the geometry
    if (rows <= PartSkinny::BM)
      part_unit<MODE, PartSkinny>(g, smem, s_rowid, tid, lane, wave, slot, row0, rows, cb * 32, w);
    else
      part_unit<MODE, C>(g, smem, s_rowid, tid, lane, wave, slot, row0, rows, cb * 32, w);
  }
}

}  // namespace lmoe
