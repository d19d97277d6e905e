// Decode MoE layer body straight from the router output, in two launches
// with no cross-block synchronisation inside either:
//   1. gate_up GEMV + SiLU*mul  -> act [T*k, I] (flat pair order)
//   2. down GEMV + weighted combine -> out [T, H]
// Both derive the slot grouping of the pairs themselves from ids + log2phy
// (an LDS bitmap of the used slots ranked by popcount prefix: active slot a
// is the a-th smallest used slot id; each slot's pairs in flat order), which
// costs two dependent L2 reads per block and replaces a permutation launch.
// Each expert's weights are read from HBM once per launch, however many of
// the T tokens chose it.
//
// (Cross-block hand-off inside one launch would need agent-scope release /
// acquire fences; on this part they write back / invalidate a whole XCD L2
// each and cost far more than a kernel boundary, which in a captured graph
// is back to back.)
//
// Rounding points follow the reference: gate and up leave GMM1 as bf16, the
// SwiGLU output is bf16, y = GMM2 output is bf16, the combine accumulates in
// f32 in j order and rounds once.
//
// Reference behaviour: ExpertSlotMapping.remap_topk_ids
// (moe_offload/slot_mapping.py:116-140) + npu_moe_init_routing_v2
// (patches/patch_fused_moe.py:668-701) + npu_grouped_matmul x2 + npu_swiglu
// (_apply_mlp, :3772-3774) + npu_moe_token_unpermute (:3363-3366), i.e. the
// decode fused_experts call of patch_fused_moe.py:3946-4009.
#include "lmoe_device.h"

namespace lmoe {

constexpr int kDecMaxPairs = 512;
constexpr int kDecMaxSlots = 8192;
constexpr int kDecWords = kDecMaxSlots / 32;
constexpr int kDnMaxRows = 4;  // output rows per down block (at most)

struct DecodeArgs {
  const uint16_t* x;
  int T, H, I, k;
  const int32_t* ids;
  const int32_t* log2phy;
  int n_log2phy;
  const uint16_t* w13;
  const uint16_t* w2;
  int P;
  const uint16_t* wts;
  const uint16_t* add;
  uint16_t* out;
  uint16_t* act;  // [N, I] by flat pair
  int32_t* meta;
};

// Sum V values per lane over the lanes that differ in bits LO..HI of the lane
// id, leaving ONE total per lane: the first log2(V) steps exchange halves of
// the value set (a reduce-scatter), the rest are plain butterfly adds.  On
// return, the lane holds value index scatter_index<HI, LO, log2 V>(lane).
template <int V, int HI, int LO>
__device__ __forceinline__ float reduce_scatter(float (&v)[V], int lane) {
  constexpr int L = (V >= 16) ? 4 : (V >= 8) ? 3 : (V >= 4) ? 2 : (V >= 2) ? 1 : 0;
  static_assert((1 << L) == V, "V must be a power of two <= 16");
  static_assert(HI - LO + 1 >= L, "not enough lane bits");
#pragma unroll
  for (int b = 0; b < L; ++b) {
    const int bit = HI - b;
    const int half = V >> (b + 1);
    const bool upper = (lane >> bit) & 1;
#pragma unroll
    for (int i = 0; i < half; ++i) {
      const float send = upper ? v[i] : v[half + i];
      const float keep = upper ? v[half + i] : v[i];
      v[i] = keep + __shfl_xor(send, 1 << bit, kWave);
    }
  }
  float r = v[0];
#pragma unroll
  for (int bit = HI - L; bit >= LO; --bit) r += __shfl_xor(r, 1 << bit, kWave);
  return r;
}

template <int HI, int LO, int L>
__device__ __forceinline__ int scatter_index(int lane) {
  int idx = 0;
#pragma unroll
  for (int b = 0; b < L; ++b) idx = (idx << 1) | ((lane >> (HI - b)) & 1);
  return idx;
}

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte streaming load of weights that are read once per launch.
__device__ __forceinline__ uint4 load_stream16(const uint16_t* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Slot grouping of the pairs: s_slot[p] = slot of pair p (-1 if it does not
// map), s_bits = bitmap of the used slots, s_wpre = exclusive popcount prefix
// per 32-slot word.
struct Grouping {
  int s_slot[kDecMaxPairs];
  uint32_t s_bits[kDecWords];
  int s_wpre[kDecWords];
  int s_scan[8];
  int na, err, placed;
};

// Every thread of a 256-thread block calls it.
__device__ void build_grouping(const DecodeArgs& a, Grouping& g) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int N = a.T * a.k;
  const int nwords = (a.P + 31) >> 5;
  if (tid == 0) {
    g.err = 0;
    g.placed = 0;
  }
  for (int w = tid; w < nwords; w += 256) g.s_bits[w] = 0u;
  __syncthreads();
  int err = 0, placed = 0;
  for (int p = tid; p < N; p += 256) {
    const int id = a.ids[p];
    int s = -2;
    if (a.log2phy != nullptr) {
      if (id >= 0 && id < a.n_log2phy) s = a.log2phy[id];
    } else {
      s = id;
    }
    if (s >= 0 && s < a.P) {
      atomicOr(&g.s_bits[s >> 5], 1u << (s & 31));
      ++placed;
    } else {
      s = -1;
      ++err;
    }
    g.s_slot[p] = s;
  }
  if (err) atomicAdd(&g.err, err);
  if (placed) atomicAdd(&g.placed, placed);
  __syncthreads();
  // exclusive prefix of the word popcounts (nwords <= 256 threads)
  const int c = tid < nwords ? __popc(g.s_bits[tid]) : 0;
  int inc = c;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(inc, o, kWave);
    if (lane >= o) inc += t;
  }
  if (lane == 63) g.s_scan[wave] = inc;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += g.s_scan[w];
  if (tid < nwords) g.s_wpre[tid] = base + inc - c;
  if (tid == 255) g.na = base + inc;
  __syncthreads();
}

// slot id of active rank r (r < g.na)
__device__ __forceinline__ int slot_of_rank(const Grouping& g, int nwords, int r) {
  int lo = 0, hi = nwords - 1;  // largest w with s_wpre[w] <= r
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (g.s_wpre[mid] <= r) lo = mid; else hi = mid - 1;
  }
  uint32_t bits = g.s_bits[lo];
  for (int q = r - g.s_wpre[lo]; q > 0; --q) bits &= bits - 1u;
  return lo * 32 + (__ffs(bits) - 1);
}

// ---------------------------------------------------------------------------
// gate_up + SiLU*mul.  grid (gu_units, max_active): block (sub, a) owns rows
// i = (4*sub + wave)*GR .. +GR of the a-th active slot; the weight rows stay
// in registers while that slot's tokens stream past, 4 at a time.
// GNC: 512-column chunks of an H row; GR: row pairs per wave.
// ---------------------------------------------------------------------------
template <int GNC, int GR>
__global__ __launch_bounds__(256) void moe_decode_gateup_kernel(DecodeArgs a) {
  __shared__ Grouping g;
  __shared__ int s_list[kDecMaxPairs];
  __shared__ int s_n, s_myslot;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int N = a.T * a.k;
  const int I = a.I;
  const int H = a.H;
  const int nwords = (a.P + 31) >> 5;
  build_grouping(a, g);
  const int slot_rank = blockIdx.y;
  if (blockIdx.x == 0 && slot_rank == 0 && tid == 0) {
    a.meta[LMOE_META_ACTIVE] = g.na;
    a.meta[LMOE_META_PAIRS] = g.placed;
    a.meta[LMOE_META_ERRORS] = g.err;
  }
  if (slot_rank >= g.na) return;
  if (tid == 0) s_myslot = slot_of_rank(g, nwords, slot_rank);
  __syncthreads();
  const int myslot = s_myslot;
  if (wave == 0) {
    int cnt = 0;
    for (int base = 0; base < N; base += 64) {
      const int p = base + lane;
      const bool m = p < N && g.s_slot[p] == myslot;
      const uint64_t bm = __ballot(m);
      if (m) s_list[cnt + __popcll(bm & lanemask_lt(lane))] = p;
      cnt += __popcll(bm);
    }
    if (lane == 0) s_n = cnt;
  }
  __syncthreads();
  const int n = s_n;

  const int i0 = (blockIdx.x * 4 + wave) * GR;
  const uint16_t* base13 = a.w13 + static_cast<size_t>(myslot) * 2 * I * H;
  uint4 wg[GR][GNC], wu[GR][GNC];
#pragma unroll
  for (int r = 0; r < GR; ++r) {
    const int i = i0 + r;
#pragma unroll
    for (int c = 0; c < GNC; ++c) {
      const int h = c * 512 + lane * 8;
      if (i < I && h < H) {
        wg[r][c] = load_stream16(base13 + static_cast<size_t>(i) * H + h);
        wu[r][c] = load_stream16(base13 + static_cast<size_t>(I + i) * H + h);
      } else {
        wg[r][c] = make_uint4(0u, 0u, 0u, 0u);
        wu[r][c] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
  }
  constexpr int V = 2 * GR * 4;
  constexpr int LV = (V >= 16) ? 4 : (V >= 8) ? 3 : 2;
  for (int q0 = 0; q0 < n; q0 += 4) {
    float v[V];
#pragma unroll
    for (int z = 0; z < V; ++z) v[z] = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (q0 + q < n) {
        const int t = s_list[q0 + q] / a.k;
        const uint16_t* xr = a.x + static_cast<size_t>(t) * H;
#pragma unroll
        for (int c = 0; c < GNC; ++c) {
          const int h = c * 512 + lane * 8;
          if (h < H) {
            const uint4 xv = *reinterpret_cast<const uint4*>(xr + h);
#pragma unroll
            for (int r = 0; r < GR; ++r) {
              v[r * 4 + q] = dot8(xv, wg[r][c], v[r * 4 + q]);
              v[GR * 4 + r * 4 + q] = dot8(xv, wu[r][c], v[GR * 4 + r * 4 + q]);
            }
          }
        }
      }
    }
    // value index z = which * (4 GR) + r * 4 + q; after the reduction lane l
    // holds z = scatter_index(l): "which" (gate 0 / up 1) is lane bit 5
    const float tot = reduce_scatter<V, 5, 0>(v, lane);
    const float other = __shfl_xor(tot, 32, kWave);
    const int z = scatter_index<5, 0, LV>(lane);
    constexpr int kLow = 6 - LV;
    if ((lane & 32) == 0 && (lane & ((1 << kLow) - 1)) == 0) {
      const int r = (z >> 2) % GR;
      const int q = z & 3;
      const int i = i0 + r;
      if (q0 + q < n && i < I) {
        const int p = s_list[q0 + q];
        a.act[static_cast<size_t>(p) * I + i] = swiglu_bf16(tot, other);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// down + weighted combine.  grid ceil(H / R): block b owns output rows
// h0 = R*b .. R*b+R-1 for EVERY active slot, so its combine needs nothing
// from other blocks.  Half wave hw (8 per block) takes the active slots
// a = hw, hw + 8, ...: it holds the slot's R W2 rows (DNC 16-byte chunks per
// lane and row), with PF also loading the next slot's while it computes,
// streams the slot's act rows from L2 and leaves y[p][h] (bf16 values) in
// LDS; then the block combines its R columns of every token in j order.
// ---------------------------------------------------------------------------
template <int DNC, int R, bool PF>
__global__ __launch_bounds__(256) void moe_decode_down_kernel(DecodeArgs a) {
  constexpr int kDnRows = R;
  constexpr int V = 4 * R;
  constexpr int LV = (V >= 16) ? 4 : (V >= 8) ? 3 : 2;
  __shared__ Grouping g;
  __shared__ float s_y[kDecMaxPairs * kDnMaxRows];
  __shared__ int s_list[8][kDecMaxPairs];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int half = lane >> 5;
  const int l5 = lane & 31;
  const int hw = wave * 2 + half;
  const int N = a.T * a.k;
  const int I = a.I;
  const int H = a.H;
  const int nwords = (a.P + 31) >> 5;
  build_grouping(a, g);
  const int na = g.na;
  const int h0 = blockIdx.x * kDnRows;

  uint4 wcur[kDnRows][DNC], wnxt[PF ? kDnRows : 1][PF ? DNC : 1];
  int rank = hw;
  int s_cur = rank < na ? slot_of_rank(g, nwords, rank) : -1;
  if (s_cur >= 0) {
    const uint16_t* base2 = a.w2 + static_cast<size_t>(s_cur) * H * I;
#pragma unroll
    for (int r = 0; r < kDnRows; ++r) {
      const int h = h0 + r;
#pragma unroll
      for (int c = 0; c < DNC; ++c) {
        const int col = c * 256 + l5 * 8;
        wcur[r][c] = (h < H && col < I) ? load_stream16(base2 + static_cast<size_t>(h) * I + col)
                                        : make_uint4(0u, 0u, 0u, 0u);
      }
    }
  }
  // both halves of a wave run the loop together (ballots), each on its own
  // slot sequence; a half with no slot left idles until the other finishes
  while (__ballot(s_cur >= 0) != 0ull) {
    const int nrank = rank + 8;
    const int s_nxt = (s_cur >= 0 && nrank < na) ? slot_of_rank(g, nwords, nrank) : -1;
    if (PF && s_nxt >= 0) {
      const uint16_t* base2 = a.w2 + static_cast<size_t>(s_nxt) * H * I;
#pragma unroll
      for (int r = 0; r < kDnRows; ++r) {
        const int h = h0 + r;
#pragma unroll
        for (int c = 0; c < DNC; ++c) {
          const int col = c * 256 + l5 * 8;
          wnxt[PF ? r : 0][PF ? c : 0] =
              (h < H && col < I) ? load_stream16(base2 + static_cast<size_t>(h) * I + col)
                                 : make_uint4(0u, 0u, 0u, 0u);
        }
      }
    }
    // pairs of s_cur in flat order (per half wave)
    int* list = s_list[hw];
    int n = 0;
    for (int base = 0; base < N; base += 32) {
      const int p = base + l5;
      const bool m = s_cur >= 0 && p < N && g.s_slot[p] == s_cur;
      const uint64_t bm = __ballot(m);
      const uint32_t mine = static_cast<uint32_t>(half ? (bm >> 32) : bm);
      if (m) list[n + __popc(mine & ((1u << l5) - 1u))] = p;
      n += __popc(mine);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int n_other = __shfl_xor(n, 32, kWave);
    const int n_max = n > n_other ? n : n_other;
    for (int q0 = 0; q0 < n_max; q0 += 4) {
      float v[V];
#pragma unroll
      for (int z = 0; z < V; ++z) v[z] = 0.0f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (q0 + q < n) {
          const uint16_t* ar = a.act + static_cast<size_t>(list[q0 + q]) * I;
#pragma unroll
          for (int c = 0; c < DNC; ++c) {
            const int col = c * 256 + l5 * 8;
            if (col < I) {
              const uint4 av = *reinterpret_cast<const uint4*>(ar + col);
#pragma unroll
              for (int r = 0; r < kDnRows; ++r) v[r * 4 + q] = dot8(av, wcur[r][c], v[r * 4 + q]);
            }
          }
        }
      }
      // reduce over the 32 lanes of each half wave: lane holds z = r*4 + q
      const float tot = reduce_scatter<V, 4, 0>(v, lane);
      const int z = scatter_index<4, 0, LV>(lane);
      if ((l5 & ((1 << (5 - LV)) - 1)) == 0) {
        const int r = z >> 2;
        const int q = z & 3;
        if (q0 + q < n) s_y[list[q0 + q] * kDnRows + r] = round_bf16(tot);  // GMM2 output is bf16
      }
    }
    rank = nrank;
    s_cur = s_nxt;
    if (PF) {
#pragma unroll
      for (int r = 0; r < kDnRows; ++r)
#pragma unroll
        for (int c = 0; c < DNC; ++c) wcur[r][c] = wnxt[PF ? r : 0][PF ? c : 0];
    } else if (s_cur >= 0) {
      const uint16_t* base2 = a.w2 + static_cast<size_t>(s_cur) * H * I;
#pragma unroll
      for (int r = 0; r < kDnRows; ++r) {
        const int h = h0 + r;
#pragma unroll
        for (int c = 0; c < DNC; ++c) {
          const int col = c * 256 + l5 * 8;
          wcur[r][c] = (h < H && col < I) ? load_stream16(base2 + static_cast<size_t>(h) * I + col)
                                          : make_uint4(0u, 0u, 0u, 0u);
        }
      }
    }
  }
  __syncthreads();
  for (int qq = tid; qq < a.T * kDnRows; qq += 256) {
    const int t = qq / kDnRows;
    const int r = qq % kDnRows;
    const int h = h0 + r;
    if (h >= H) continue;
    float acc = 0.0f;
    for (int j = 0; j < a.k; ++j) {
      const int p = t * a.k + j;
      if (g.s_slot[p] >= 0) acc += bf16_to_f32(a.wts[p]) * s_y[p * kDnRows + r];
    }
    if (a.add != nullptr) acc += bf16_to_f32(a.add[static_cast<size_t>(t) * H + h]);
    a.out[static_cast<size_t>(t) * H + h] = static_cast<uint16_t>(f32_to_bf16_bits(acc));
  }
}

}  // namespace lmoe

using namespace lmoe;

namespace {

struct DecodeShape {
  int gnc, gr, dnc;
};

DecodeShape pick_shape(int H, int I) {
  DecodeShape s{};
  const int g = (H + 511) / 512;
  s.gnc = g <= 4 ? 4 : g <= 8 ? 8 : g <= 14 ? 14 : 16;
  s.gr = s.gnc <= 4 ? 2 : 1;
  const int d = (I + 255) / 256;
  s.dnc = d <= 3 ? 3 : d <= 4 ? 4 : d <= 8 ? 8 : 16;
  return s;
}

}  // namespace

extern "C" int lmoe_moe_decode(const void* x, int T, int H, int I, int k,
                               const int32_t* ids, const int32_t* log2phy,
                               int n_log2phy, const void* w13_slots,
                               const void* w2_slots, int n_slots,
                               const uint16_t* w, const void* add, void* out,
                               void* act, int32_t* meta, hipStream_t stream) {
  if (x == nullptr || ids == nullptr || w13_slots == nullptr ||
      w2_slots == nullptr || w == nullptr || out == nullptr || act == nullptr ||
      meta == nullptr)
    return LMOE_ERR_ARG;
  if (T <= 0 || H <= 0 || I <= 0 || k <= 0 || n_slots <= 0) return LMOE_ERR_ARG;
  if (log2phy != nullptr && n_log2phy <= 0) return LMOE_ERR_ARG;
  const int N = T * k;
  if (N > kDecMaxPairs || n_slots > kDecMaxSlots) return LMOE_ERR_SHAPE;
  if (H % 8 != 0 || I % 8 != 0 || H > 16 * 512 || I > 16 * 256) return LMOE_ERR_SHAPE;
  const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w13_slots) |
                          reinterpret_cast<uintptr_t>(w2_slots) | reinterpret_cast<uintptr_t>(act);
  if (align & 15u) return LMOE_ERR_SHAPE;
  const DecodeShape s = pick_shape(H, I);
  DecodeArgs args{};
  args.x = static_cast<const uint16_t*>(x);
  args.T = T;
  args.H = H;
  args.I = I;
  args.k = k;
  args.ids = ids;
  args.log2phy = log2phy;
  args.n_log2phy = n_log2phy;
  args.w13 = static_cast<const uint16_t*>(w13_slots);
  args.w2 = static_cast<const uint16_t*>(w2_slots);
  args.P = n_slots;
  args.wts = w;
  args.add = static_cast<const uint16_t*>(add);
  args.out = static_cast<uint16_t*>(out);
  args.act = static_cast<uint16_t*>(act);
  args.meta = meta;
  const int max_active = N < n_slots ? N : n_slots;
  const dim3 gu_grid((I + 4 * s.gr - 1) / (4 * s.gr), max_active);
  switch (s.gnc) {
    case 4: hipLaunchKernelGGL((moe_decode_gateup_kernel<4, 2>), gu_grid, dim3(256), 0, stream, args); break;
    case 8: hipLaunchKernelGGL((moe_decode_gateup_kernel<8, 1>), gu_grid, dim3(256), 0, stream, args); break;
    case 14: hipLaunchKernelGGL((moe_decode_gateup_kernel<14, 1>), gu_grid, dim3(256), 0, stream, args); break;
    default: hipLaunchKernelGGL((moe_decode_gateup_kernel<16, 1>), gu_grid, dim3(256), 0, stream, args); break;
  }
  switch (s.dnc) {
    case 3:
      hipLaunchKernelGGL((moe_decode_down_kernel<3, 4, true>), dim3((H + 3) / 4), dim3(256), 0, stream, args);
      break;
    case 4:
      hipLaunchKernelGGL((moe_decode_down_kernel<4, 4, true>), dim3((H + 3) / 4), dim3(256), 0, stream, args);
      break;
    case 8:
      hipLaunchKernelGGL((moe_decode_down_kernel<8, 4, false>), dim3((H + 3) / 4), dim3(256), 0, stream, args);
      break;
    default:
      hipLaunchKernelGGL((moe_decode_down_kernel<16, 2, false>), dim3((H + 1) / 2), dim3(256), 0, stream, args);
      break;
  }
  LMOE_RETURN_LAUNCH();
}
