// Decode MoE layer body in one launch: slot remap + grouping of the pairs by
// slot, gate_up GEMV + SiLU*mul, down GEMV, weighted combine.
//
// Work units are handed out in launch order by a device-scope ticket
// counter: first every gate_up unit (slot-major: all units of the first
// active slot, then the next ...), then every down unit.  A down unit loads
// its W2 rows first, then waits until all gate_up units of its slot have
// published their act rows.  Every unit it can wait for holds a smaller
// ticket, so it is already resident and never waits itself: the launch
// always drains.  The wait is also bounded (about a second); a timeout is
// counted in meta[LMOE_META_STALLS] instead of spinning on.  The last down
// unit of each output column tile (per-tile counter) combines the tokens of
// that tile.  All counters are returned to zero by the launch itself (the
// last unit to finish resets the shared ones), so the workspace needs to be
// zeroed once, at allocation, and never again: graph replays need no memset.
//
// Every block derives the slot grouping itself from ids + log2phy (an LDS
// bitmap of the slots, ranked by popcount prefix, so active slot a is the
// a-th smallest slot id, and each slot's pairs in flat order), which costs
// two dependent L2 reads and replaces a separate permutation launch.
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
constexpr int kDecSpinLimit = 1 << 22;  // x s_sleep(8) ~ 2e9 cycles

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
  uint16_t* y;    // [N, H] by flat pair
  int32_t* sync;  // [2 + max_active + dn_per_slot], zero between launches
  int32_t* meta;
  int max_active;
  int gu_per_slot;
  int dn_per_slot;
};

// Sum V values per lane over the lanes that differ in bits LO..HI of the lane
// id, leaving ONE total per lane: the first log2(V) steps exchange halves of
// the value set (a reduce-scatter), the rest are plain butterfly adds.  On
// return, the lane holds value index
//   sum_{b < log2 V} ((lane >> (HI - b)) & 1) << (log2 V - 1 - b).
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

__device__ __forceinline__ void release_agent() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
}
__device__ __forceinline__ void acquire_agent() {
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

// GNC: 512-column chunks of an H row (gate_up); GR: row pairs per wave.
// DNC: 256-column chunks of an I row (down, one row per half wave);
// DS: row steps per wave (2 rows per step).
template <int GNC, int GR, int DNC, int DS>
__global__ __launch_bounds__(256) void moe_decode_kernel(DecodeArgs a) {
  __shared__ int s_slot[kDecMaxPairs];
  __shared__ uint32_t s_bits[kDecWords];
  __shared__ int s_wpre[kDecWords];
  __shared__ int s_list[kDecMaxPairs];
  __shared__ int s_scan[8];
  __shared__ int s_ticket, s_na, s_err, s_placed, s_myslot, s_n, s_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int N = a.T * a.k;
  const int I = a.I;
  const int H = a.H;

  if (tid == 0) {
    s_ticket = __hip_atomic_fetch_add(&a.sync[0], 1, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
    s_err = 0;
    s_placed = 0;
  }
  const int nwords = (a.P + 31) >> 5;
  for (int w = tid; w < nwords; w += 256) s_bits[w] = 0u;
  __syncthreads();
  // ---- slot of every pair, slot bitmap
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
      atomicOr(&s_bits[s >> 5], 1u << (s & 31));
      ++placed;
    } else {
      s = -1;
      ++err;
    }
    s_slot[p] = s;
  }
  if (err) atomicAdd(&s_err, err);
  if (placed) atomicAdd(&s_placed, placed);
  __syncthreads();
  // ---- exclusive prefix of the word popcounts (nwords <= 256 threads)
  {
    const int c = tid < nwords ? __popc(s_bits[tid]) : 0;
    int inc = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(inc, o, kWave);
      if (lane >= o) inc += t;
    }
    if (lane == 63) s_scan[wave] = inc;
    __syncthreads();
    int base = 0;
    for (int w = 0; w < wave; ++w) base += s_scan[w];
    if (tid < nwords) s_wpre[tid] = base + inc - c;
    if (tid == 255) s_na = base + inc;
  }
  __syncthreads();
  const int na = s_na;
  const int ticket = s_ticket;
  const int n_gu = a.max_active * a.gu_per_slot;
  const bool is_gu = ticket < n_gu;
  const int u = is_gu ? ticket : ticket - n_gu;
  const int slot_rank = is_gu ? u / a.gu_per_slot : u / a.dn_per_slot;
  const int sub = is_gu ? u % a.gu_per_slot : u % a.dn_per_slot;
  const bool has_work = slot_rank < na;

  if (ticket == 0) {
    if (tid == 0) {
      a.meta[LMOE_META_ACTIVE] = na;
      a.meta[LMOE_META_PAIRS] = s_placed;
      a.meta[LMOE_META_ERRORS] = s_err;
    }
  }
  if (has_work) {
    // ---- the slot of rank slot_rank and its pairs in flat order
    if (tid == 0) {
      int lo = 0, hi = nwords - 1;  // largest w with s_wpre[w] <= slot_rank
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_wpre[mid] <= slot_rank) lo = mid; else hi = mid - 1;
      }
      uint32_t bits = s_bits[lo];
      for (int r = slot_rank - s_wpre[lo]; r > 0; --r) bits &= bits - 1u;
      s_myslot = lo * 32 + (__ffs(bits) - 1);
    }
    __syncthreads();
    const int myslot = s_myslot;
    if (wave == 0) {
      int cnt = 0;
      for (int base = 0; base < N; base += 64) {
        const int p = base + lane;
        const bool m = p < N && s_slot[p] == myslot;
        const uint64_t bm = __ballot(m);
        if (m) s_list[cnt + __popcll(bm & lanemask_lt(lane))] = p;
        cnt += __popcll(bm);
      }
      if (lane == 0) s_n = cnt;
    }
    __syncthreads();
    const int n = s_n;

    if (is_gu) {
      // ================= gate_up rows i0 .. i0+GR-1 of slot myslot
      const int i0 = (sub * 4 + wave) * GR;
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
        // value index z = which * (4 GR) + r * 4 + q; after the reduction
        // lane l holds z = scatter_index(l), "which" is lane bit 5
        const float tot = reduce_scatter<V, 5, 0>(v, lane);
        const float other = __shfl_xor(tot, 32, kWave);
        const int z = scatter_index<5, 0, LV>(lane);
        const int low_bits = 6 - LV;
        if ((lane & 32) == 0 && (lane & ((1 << low_bits) - 1)) == 0) {
          const int r = (z >> 2) % GR;
          const int q = z & 3;
          const int i = i0 + r;
          if (q0 + q < n && i < I) {
            const int p = s_list[q0 + q];
            a.act[static_cast<size_t>(p) * I + i] = swiglu_bf16(tot, other);
          }
        }
      }
      release_agent();
      __syncthreads();
      if (tid == 0)
        __hip_atomic_fetch_add(&a.sync[2 + slot_rank], 1, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    } else {
      // ================= down rows of tile sub, slot myslot
      const int half = lane >> 5;
      const int l5 = lane & 31;
      const int rows_per_unit = 4 * 2 * DS;
      const int hbase = sub * rows_per_unit + wave * 2 * DS;
      const uint16_t* base2 = a.w2 + static_cast<size_t>(myslot) * H * I;
      uint4 wv[DS][DNC];
#pragma unroll
      for (int st = 0; st < DS; ++st) {
        const int h = hbase + st * 2 + half;
#pragma unroll
        for (int c = 0; c < DNC; ++c) {
          const int col = c * 256 + l5 * 8;
          wv[st][c] = (h < H && col < I)
                          ? load_stream16(base2 + static_cast<size_t>(h) * I + col)
                          : make_uint4(0u, 0u, 0u, 0u);
        }
      }
      // wait for the act rows of this slot
      if (tid == 0) {
        int spins = 0;
        while (__hip_atomic_load(&a.sync[2 + slot_rank], __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT) < a.gu_per_slot) {
          __builtin_amdgcn_s_sleep(8);
          if (++spins > kDecSpinLimit) {
            atomicAdd(&a.meta[LMOE_META_STALLS], 1);
            break;
          }
        }
      }
      __syncthreads();
      acquire_agent();
      constexpr int V = 4 * DS;
      constexpr int LV = (V >= 16) ? 4 : (V >= 8) ? 3 : 2;
      for (int q0 = 0; q0 < n; q0 += 4) {
        float v[V];
#pragma unroll
        for (int z = 0; z < V; ++z) v[z] = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (q0 + q < n) {
            const uint16_t* ar = a.act + static_cast<size_t>(s_list[q0 + q]) * I;
#pragma unroll
            for (int c = 0; c < DNC; ++c) {
              const int col = c * 256 + l5 * 8;
              if (col < I) {
                const uint4 av = *reinterpret_cast<const uint4*>(ar + col);
#pragma unroll
                for (int st = 0; st < DS; ++st) v[st * 4 + q] = dot8(av, wv[st][c], v[st * 4 + q]);
              }
            }
          }
        }
        const float tot = reduce_scatter<V, 4, 0>(v, lane);
        const int z = scatter_index<4, 0, LV>(lane);
        const int low_bits = 5 - LV;
        if ((l5 & ((1 << low_bits) - 1)) == 0) {
          const int st = z >> 2;
          const int q = z & 3;
          const int h = hbase + st * 2 + half;
          if (q0 + q < n && h < H) {
            const int p = s_list[q0 + q];
            a.y[static_cast<size_t>(p) * H + h] =
                static_cast<uint16_t>(f32_to_bf16_bits(tot));
          }
        }
      }
    }
  }

  // ---- combine: the last down unit of each column tile
  if (!is_gu && slot_rank < (na > 0 ? na : 1)) {
    release_agent();
    __syncthreads();
    if (tid == 0) {
      const int expect = na > 0 ? na : 1;
      const int done = __hip_atomic_fetch_add(&a.sync[2 + a.max_active + sub], 1,
                                              __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      s_last = done == expect - 1;
    }
    __syncthreads();
    if (s_last) {
      acquire_agent();
      const int R = 4 * 2 * DS;
      const int h0 = sub * R;
      for (int qq = tid; qq < a.T * R; qq += 256) {
        const int t = qq / R;
        const int h = h0 + qq % R;
        if (h >= H) continue;
        float acc = 0.0f;
        for (int j = 0; j < a.k; ++j) {
          const int p = t * a.k + j;
          if (s_slot[p] >= 0)
            acc += bf16_to_f32(a.wts[p]) * bf16_to_f32(a.y[static_cast<size_t>(p) * H + h]);
        }
        if (a.add != nullptr) acc += bf16_to_f32(a.add[static_cast<size_t>(t) * H + h]);
        a.out[static_cast<size_t>(t) * H + h] = static_cast<uint16_t>(f32_to_bf16_bits(acc));
      }
      if (tid == 0)
        __hip_atomic_store(&a.sync[2 + a.max_active + sub], 0, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  // ---- the last unit to finish returns the shared counters to zero
  __syncthreads();
  if (tid == 0) {
    const int fin = __hip_atomic_fetch_add(&a.sync[1], 1, __ATOMIC_ACQ_REL,
                                           __HIP_MEMORY_SCOPE_AGENT);
    if (fin == static_cast<int>(gridDim.x) - 1) {
      for (int i = 0; i < a.max_active; ++i)
        __hip_atomic_store(&a.sync[2 + i], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&a.sync[0], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&a.sync[1], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

struct DecodeShape {
  int gnc, gr, dnc, ds;
};

static DecodeShape pick_shape(int H, int I) {
  DecodeShape s{};
  const int g = (H + 511) / 512;
  s.gnc = g <= 4 ? 4 : g <= 8 ? 8 : g <= 14 ? 14 : 16;
  s.gr = s.gnc <= 4 ? 2 : 1;
  const int d = (I + 255) / 256;
  s.dnc = d <= 3 ? 3 : d <= 4 ? 4 : d <= 8 ? 8 : 16;
  s.ds = s.dnc <= 4 ? 4 : s.dnc <= 8 ? 2 : 1;
  return s;
}

static int decode_units(const DecodeShape& s, int H, int I, int* gu, int* dn) {
  *gu = (I + 4 * s.gr - 1) / (4 * s.gr);
  *dn = (H + 8 * s.ds - 1) / (8 * s.ds);
  return 0;
}

}  // namespace lmoe

using namespace lmoe;

extern "C" size_t lmoe_moe_decode_sync_words(int n_pairs, int n_slots, int H, int I) {
  if (n_pairs <= 0 || n_slots <= 0 || H <= 0 || I <= 0) return 0;
  const DecodeShape s = pick_shape(H, I);
  int gu, dn;
  decode_units(s, H, I, &gu, &dn);
  const int max_active = n_pairs < n_slots ? n_pairs : n_slots;
  return static_cast<size_t>(2 + max_active + dn);
}

#define LMOE_DECODE_LAUNCH(G, GR_, D, DS_)                                      \
  hipLaunchKernelGGL((moe_decode_kernel<G, GR_, D, DS_>), grid, dim3(256), 0,   \
                     stream, args)

extern "C" int lmoe_moe_decode(const void* x, int T, int H, int I, int k,
                               const int32_t* ids, const int32_t* log2phy,
                               int n_log2phy, const void* w13_slots,
                               const void* w2_slots, int n_slots,
                               const uint16_t* w, const void* add, void* out,
                               void* act, void* y, int32_t* sync,
                               size_t sync_words, int32_t* meta,
                               hipStream_t stream) {
  if (x == nullptr || ids == nullptr || w13_slots == nullptr ||
      w2_slots == nullptr || w == nullptr || out == nullptr || act == nullptr ||
      y == nullptr || sync == nullptr || meta == nullptr)
    return LMOE_ERR_ARG;
  if (T <= 0 || H <= 0 || I <= 0 || k <= 0 || n_slots <= 0) return LMOE_ERR_ARG;
  if (log2phy != nullptr && n_log2phy <= 0) return LMOE_ERR_ARG;
  const int N = T * k;
  if (N > kDecMaxPairs || n_slots > kDecMaxSlots) return LMOE_ERR_SHAPE;
  if (H % 8 != 0 || I % 8 != 0 || H > 16 * 512 || I > 16 * 256) return LMOE_ERR_SHAPE;
  if (sync_words < lmoe_moe_decode_sync_words(N, n_slots, H, I)) return LMOE_ERR_WORKSPACE;
  const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w13_slots) |
                          reinterpret_cast<uintptr_t>(w2_slots) | reinterpret_cast<uintptr_t>(act) |
                          reinterpret_cast<uintptr_t>(y);
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
  args.y = static_cast<uint16_t*>(y);
  args.sync = sync;
  args.meta = meta;
  args.max_active = N < n_slots ? N : n_slots;
  decode_units(s, H, I, &args.gu_per_slot, &args.dn_per_slot);
  const dim3 grid(args.max_active * (args.gu_per_slot + args.dn_per_slot));
  if (s.gnc == 4 && s.dnc == 3) LMOE_DECODE_LAUNCH(4, 2, 3, 4);
  else if (s.gnc == 4 && s.dnc == 4) LMOE_DECODE_LAUNCH(4, 2, 4, 4);
  else if (s.gnc == 4 && s.dnc == 8) LMOE_DECODE_LAUNCH(4, 2, 8, 2);
  else if (s.gnc == 4) LMOE_DECODE_LAUNCH(4, 2, 16, 1);
  else if (s.gnc == 8 && s.dnc == 3) LMOE_DECODE_LAUNCH(8, 1, 3, 4);
  else if (s.gnc == 8 && s.dnc == 4) LMOE_DECODE_LAUNCH(8, 1, 4, 4);
  else if (s.gnc == 8 && s.dnc == 8) LMOE_DECODE_LAUNCH(8, 1, 8, 2);
  else if (s.gnc == 8) LMOE_DECODE_LAUNCH(8, 1, 16, 1);
  else if (s.gnc == 14 && s.dnc == 3) LMOE_DECODE_LAUNCH(14, 1, 3, 4);
  else if (s.gnc == 14 && s.dnc == 4) LMOE_DECODE_LAUNCH(14, 1, 4, 4);
  else if (s.gnc == 14 && s.dnc == 8) LMOE_DECODE_LAUNCH(14, 1, 8, 2);
  else if (s.gnc == 14) LMOE_DECODE_LAUNCH(14, 1, 16, 1);
  else if (s.dnc == 3) LMOE_DECODE_LAUNCH(16, 1, 3, 4);
  else if (s.dnc == 4) LMOE_DECODE_LAUNCH(16, 1, 4, 4);
  else if (s.dnc == 8) LMOE_DECODE_LAUNCH(16, 1, 8, 2);
  else LMOE_DECODE_LAUNCH(16, 1, 16, 1);
  LMOE_RETURN_LAUNCH();
}
