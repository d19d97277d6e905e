// One-token decode body in ONE launch: gate_up GEMV + SiLU*mul and the down
// GEMV + weighted combine, with the down projection's weights in flight
// while gate_up still runs.
//
// The grid is two groups of workgroups.  The first n_gu are the gate_up
// producers (as gateup_gemv_kernel's one-token path: workgroup (bx, a) owns
// row pairs 4 bx .. 4 bx + 3 of the a-th active slot, one wave each).  The
// rest are the down consumers (as down_combine_gemv_kernel's one-token path:
// workgroup b owns output rows R b .. R b + R - 1 for every pair; half wave
// hw holds the W2 rows of active rank hw).  A consumer issues its W2 loads
// first, then takes the act values as producers publish them.
//
// Hand-off without cache flushes: every act value travels as one 32-bit
// word (bf16 value | 16-bit tag) written and read by agent-scope atomic
// accesses, so a reader sees a whole word or an older one; the tag is the
// permutation's build count (meta[LMOE_META_GEN], advanced by the build
// that precedes this launch), so a word of an earlier launch is never
// taken.  Producer progress goes up a counter tree in meta (16 first-level
// counters per rank, one per rank, then the number of ranks done; the
// build zeroed them; 256 bytes apart), which only tells a consumer when to
// start reading (one thread polls the ranks-done count): a word whose tag
// does not match yet is read again.  No counter has more than a few dozen
// increments (contended agent-scope atomics are slow), and nothing is left
// to reset.  Every wait is bounded: past kSpinLimit polls
// meta[LMOE_META_DECODE_TIMEOUT] becomes 1 and the wave goes on, so no wave
// can wait for ever.
//
// Producers have the lower workgroup ids, and workgroups are dispatched in
// id order on every XCD, so every producer is resident or finished before a
// consumer on its XCD waits: the wait ends.  Values are computed exactly as
// by the two-kernel path (same reductions, same roundings), so out is equal
// bit for bit.
//
// Reference behaviour: the decode fused_experts call of
// patches/patch_fused_moe.py:3946-4009 (GMM1 + swiglu + GMM2 + unpermute).
#include "lmoe_device.h"

namespace {

using namespace lmoe;

constexpr int kOneMaxK = 8;   // pairs of the token (one per half wave)
constexpr int kOneRows = 4;   // output rows per consumer workgroup
constexpr int kFan = 16;      // first-level counters per rank
constexpr long long kSpinLimit = 1LL << 22;

// hand-off counters in meta (zeroed by the permutation build), 256 bytes
// apart: kept together in a few cache lines, the producers' atomics all
// queued at one memory channel and the last of them finished ~13 us late
constexpr int kLevel1 = 0;                        // [kOneMaxK][kFan]
constexpr int kLevel2 = kLevel1 + kOneMaxK * kFan;  // [kOneMaxK]
constexpr int kLevel3 = kLevel2 + kOneMaxK;         // ranks done
static_assert(kLevel3 + 1 <= LMOE_META_DECODE_COUNTERS, "meta holds the hand-off counters");

__device__ __forceinline__ int32_t* counter(int32_t* meta, int c) {
  return meta + LMOE_META_DECODE_HINT + c * LMOE_META_DECODE_STRIDE;
}

struct DecodeOneArgs {
  const uint16_t* x;
  int H, I, k, ranks;
  const uint16_t* w13;
  const uint16_t* w2;
  const int32_t* active;
  const int32_t* row_idx;
  const uint16_t* wts;
  const uint16_t* add;
  uint32_t* words;  // [ranks, I] tagged act values
  uint16_t* out;
  int32_t* meta;
  int n_gu, gu_per_slot, n_dn;
};

__device__ __forceinline__ int ld_agent(const int32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void give_up(int32_t* meta) {
  __hip_atomic_store(meta + LMOE_META_DECODE_TIMEOUT, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int NC, int DNC>
__global__ __launch_bounds__(256) void decode_one_kernel(DecodeOneArgs a) {
  constexpr int R = kOneRows;
  constexpr int LV = 2;  // log2(R / 1) bits of the row index in the lane id
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // the build count, written by the build this launch follows in stream
  // order: a plain (cached) load sees it
  const uint32_t tag = static_cast<uint32_t>(a.meta[LMOE_META_GEN]) << 16;
  if (static_cast<int>(blockIdx.x) < a.n_gu) {
    // ---------------- producer: gate_up row pair of one active slot
    const int ar = blockIdx.x / a.gu_per_slot;
    const int i = (blockIdx.x % a.gu_per_slot) * 4 + wave;
    uint4 xv[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int h = c * 512 + lane * 8;
      xv[c] = load16_if(a.x, h, h < a.H);
    }
    const int s = a.active[ar];
    if (s >= 0 && i < a.I) {
      const uint16_t* grow = a.w13 + (static_cast<size_t>(s) * 2 * a.I + i) * a.H;
      const uint16_t* urow = grow + static_cast<size_t>(a.I) * a.H;
      float v[2] = {0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int h = c * 512 + lane * 8;
        v[0] = dot8(xv[c], load_stream16_if(grow, h, h < a.H), v[0]);
        v[1] = dot8(xv[c], load_stream16_if(urow, h, h < a.H), v[1]);
      }
      const float tot = reduce_scatter<2, 5, 0>(v, lane);
      const float up = read_lane(tot, 32);
      if (lane == 0)
        __hip_atomic_store(a.words + static_cast<size_t>(ar) * a.I + i, tag | swiglu_bf16(tot, up),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (tid == 0) {
      // first level: producer workgroups bx, bx + kFan, ... of this rank;
      // the one that completes its counter moves the rank's counter
      const int bx = blockIdx.x % a.gu_per_slot;
      const int f = bx % kFan;
      const int members = (a.gu_per_slot - f + kFan - 1) / kFan;
      const int done = __hip_atomic_fetch_add(counter(a.meta, kLevel1 + ar * kFan + f), 1,
                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (done == members - 1) {
        // ... and the one that completes the rank moves the ranks-done count
        const int fans = a.gu_per_slot < kFan ? a.gu_per_slot : kFan;
        const int d2 = __hip_atomic_fetch_add(counter(a.meta, kLevel2 + ar), 1, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
        if (d2 == fans - 1)
          __hip_atomic_fetch_add(counter(a.meta, kLevel3), 1, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    return;
  }
  // ------------------ consumer: R output rows of every pair, then combine
  __shared__ float s_y[kOneMaxK * R];
  __shared__ int s_pos[kOneMaxK];
  __shared__ float s_w[kOneMaxK];
  const int b = blockIdx.x - a.n_gu;
  const int l5 = lane & 31;
  const int hw = wave * 2 + (lane >> 5);
  const int h0 = b * R;
  const int s = hw < a.ranks ? a.active[hw] : -1;
  uint4 wr[R][DNC];
  if (s >= 0) {
    const uint16_t* base2 = a.w2 + static_cast<size_t>(s) * a.H * a.I;
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int c = 0; c < DNC; ++c) {
        const int col = c * 256 + l5 * 8;
        wr[r][c] = load_stream16_if(base2, (h0 + r) * a.I + col, h0 + r < a.H && col < a.I);
      }
    }
  }
  // the combine's inputs, loaded while the weights are in flight
  if (tid < kOneMaxK) {
    s_pos[tid] = tid < a.k ? a.row_idx[tid] : -1;
    s_w[tid] = tid < a.k ? bf16_to_f32(a.wts[tid]) : 0.0f;
  }
  const float addv = (a.add != nullptr && tid < R && h0 + tid < a.H) ? bf16_to_f32(a.add[h0 + tid]) : 0.0f;
  // start reading once the producers of every rank are done (a hint only)
  if (tid == 0) {
    long long n = 0;
    while (ld_agent(counter(a.meta, kLevel3)) < a.ranks) {
      if (++n >= kSpinLimit) {
        give_up(a.meta);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  __syncthreads();
  if (__ballot(s >= 0) != 0ull) {
    float v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = 0.0f;
    // every word of the lane's act columns in flight at once, as ordinary
    // 16-byte loads through this XCD's L2 (the launch began with the L2
    // invalidated, so a line holds either a word of this launch or, if it
    // was filled before the producer's write-through landed, an older one),
    // then the tags checked; words not yet of this launch are read again
    // past the L2 (agent-scope loads).  Through the L2, the 512 consumers'
    // reads of the same 8 x I words reach memory once per XCD instead of
    // once per consumer.
    const uint32_t* row = a.words + static_cast<size_t>(s >= 0 ? hw : 0) * a.I;
    uint32_t wv[DNC][8];
    bool ok[DNC];
#pragma unroll
    for (int c = 0; c < DNC; ++c) {
      const int col = c * 256 + l5 * 8;
      ok[c] = s >= 0 && col < a.I;
      const uint4* q = reinterpret_cast<const uint4*>(row + (ok[c] ? col : 0));
      const uint4 lo = q[0], hi = q[1];
      wv[c][0] = lo.x; wv[c][1] = lo.y; wv[c][2] = lo.z; wv[c][3] = lo.w;
      wv[c][4] = hi.x; wv[c][5] = hi.y; wv[c][6] = hi.z; wv[c][7] = hi.w;
    }
    long long n = 0;
    while (true) {
      bool fresh = true;
#pragma unroll
      for (int c = 0; c < DNC; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) fresh = fresh && (!ok[c] || (wv[c][j] & 0xffff0000u) == tag);
      if (__ballot(!fresh) == 0ull) break;
      if (++n >= kSpinLimit) {
        give_up(a.meta);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int c = 0; c < DNC; ++c) {
        const int col = c * 256 + l5 * 8;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (ok[c] && (wv[c][j] & 0xffff0000u) != tag)
            wv[c][j] = __hip_atomic_load(row + col + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
#pragma unroll
    for (int c = 0; c < DNC; ++c) {
      uint32_t w8[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) w8[j] = ok[c] ? (wv[c][j] & 0xffffu) : 0u;
      const uint4 av = make_uint4(w8[0] | (w8[1] << 16), w8[2] | (w8[3] << 16), w8[4] | (w8[5] << 16),
                                  w8[6] | (w8[7] << 16));
#pragma unroll
      for (int r = 0; r < R; ++r) v[r] = dot8(av, wr[r][c], v[r]);
    }
    const float tot = reduce_scatter<R, 4, 0>(v, lane);
    const int r = scatter_index<4, 0, LV>(lane);
    if ((l5 & ((1 << (5 - LV)) - 1)) == 0 && s >= 0) s_y[hw * R + r] = round_bf16(tot);
  }
  __syncthreads();
  if (tid < R && h0 + tid < a.H) {
    float acc = 0.0f;
    for (int j = 0; j < a.k; ++j) {
      const int p = s_pos[j];
      if (p >= 0) acc += s_w[j] * s_y[p * R + tid];
    }
    if (a.add != nullptr) acc += addv;
    a.out[h0 + tid] = static_cast<uint16_t>(f32_to_bf16_bits(acc));
  }
}

}  // namespace

extern "C" int lmoe_decode_one(const void* x, int H, int I, int k, const void* w13_slots,
                               const void* w2_slots, int n_slots, const uint16_t* w,
                               const int32_t* row_idx, const int32_t* active, const void* add,
                               void* words, void* out, int32_t* meta, hipStream_t stream) {
  if (x == nullptr || w13_slots == nullptr || w2_slots == nullptr || w == nullptr ||
      row_idx == nullptr || active == nullptr || words == nullptr || out == nullptr || meta == nullptr)
    return LMOE_ERR_ARG;
  if (H <= 0 || I <= 0 || k <= 0 || n_slots <= 0) return LMOE_ERR_ARG;
  if (H % 8 != 0 || I % 64 != 0 || I > 4096 || H > 8192) return LMOE_ERR_SHAPE;
  // the shapes whose two-kernel path runs the same per-value reductions
  // (row-per-wave gate_up, four down rows per half wave): equal bits
  const int nc = (H + 511) / 512;
  const int dnc = (I + 255) / 256;
  if (k > kOneMaxK || nc > 8 || dnc > 4) return LMOE_ERR_UNSUPPORTED;
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w13_slots) |
       reinterpret_cast<uintptr_t>(w2_slots) | reinterpret_cast<uintptr_t>(words)) & 15u)
    return LMOE_ERR_SHAPE;
  DecodeOneArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.H = H;
  a.I = I;
  a.k = k;
  a.ranks = k < n_slots ? k : n_slots;
  a.w13 = static_cast<const uint16_t*>(w13_slots);
  a.w2 = static_cast<const uint16_t*>(w2_slots);
  a.active = active;
  a.row_idx = row_idx;
  a.wts = w;
  a.add = static_cast<const uint16_t*>(add);
  a.words = static_cast<uint32_t*>(words);
  a.out = static_cast<uint16_t*>(out);
  a.meta = meta;
  a.gu_per_slot = (I + 3) / 4;
  a.n_gu = a.gu_per_slot * a.ranks;
  a.n_dn = (H + kOneRows - 1) / kOneRows;
  const dim3 grid(a.n_gu + a.n_dn);
#define LMOE_D1(NC_, DNC_) hipLaunchKernelGGL((decode_one_kernel<NC_, DNC_>), grid, dim3(256), 0, stream, a)
#define LMOE_D1_DNC(NC_)                \
  do {                                  \
    if (dnc <= 2) LMOE_D1(NC_, 2);      \
    else if (dnc <= 3) LMOE_D1(NC_, 3); \
    else LMOE_D1(NC_, 4);               \
  } while (0)
  if (nc <= 2) LMOE_D1_DNC(2);
  else if (nc <= 4) LMOE_D1_DNC(4);
  else LMOE_D1_DNC(8);
#undef LMOE_D1_DNC
#undef LMOE_D1
  LMOE_RETURN_LAUNCH();
}
