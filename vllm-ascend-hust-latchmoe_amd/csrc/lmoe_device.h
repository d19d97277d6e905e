// Device helpers shared by the latchmoe gfx950 kernels: bf16 packing,
// wave64 reductions and the one exp/sigmoid routine used by the router.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "latchmoe.h"

namespace lmoe {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// device status words (lmoe_device_flags)
// ---------------------------------------------------------------------------
// Each translation unit holds its own copy per GPU (the build has no
// relocatable device code): [LMOE_FLAG_UNPLACED] pairs a masked combine
// dropped because no pass placed them, [LMOE_FLAG_ROUTER_TIMEOUT] one-launch
// router waits that gave up.  Kernels only add to them (vector atomics);
// lmoe_device_flags sums every unit's words and clears them.  Unused copies
// cost 16 bytes.
static __device__ __attribute__((aligned(16))) int32_t g_lmoe_flags[LMOE_FLAG_COUNT];

__device__ __forceinline__ void add_device_flag(int f, int v) {
  __hip_atomic_fetch_add(&g_lmoe_flags[f], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The device address of this unit's words on the current device (nullptr
// on failure); defined once per unit by LMOE_FLAGS_UNIT(name).
#define LMOE_FLAGS_UNIT(name)                                                    \
  namespace lmoe {                                                               \
  void* flags_address_##name() {                                                 \
    void* p = nullptr;                                                           \
    return hipGetSymbolAddress(&p, HIP_SYMBOL(g_lmoe_flags)) == hipSuccess ? p \
                                                                           : nullptr; \
  }                                                                              \
  }

// ---------------------------------------------------------------------------
// bf16 <-> f32
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16lo(uint32_t packed) {
  return __uint_as_float(packed << 16);
}
__device__ __forceinline__ float bf16hi(uint32_t packed) {
  return __uint_as_float(packed & 0xffff0000u);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

// Round-to-nearest-even f32 -> bf16 (NaN stays NaN).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu) != 0u) {
    return (u >> 16) | 0x0040u;
  }
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ float round_bf16(float f) {
  return __uint_as_float(f32_to_bf16_bits(f) << 16);
}
// SwiGLU with the reference's op boundaries: gate and up leave GMM1 as bf16,
// the activation is formed in f32 and leaves as bf16 (returned as bits).
__device__ __forceinline__ uint16_t swiglu_bf16(float gate_acc, float up_acc);
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
// Two f32 -> packed bf16 pair (lo in bits 0..15), round to nearest even: one
// v_cvt_pk_bf16_f32 on gfx950 (same bits as f32_to_bf16_bits for every
// non-NaN input; NaNs stay NaN).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// One packed bf16 pair dot: acc + a.lo*b.lo + a.hi*b.hi in one
// v_dot2c_f32_bf16 (f32 accumulation; no unpacking to f32 first).
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), acc, false);
}
// dot of 8 bf16 pairs held in two uint4, accumulated into acc pair by pair
// in element order (four dot2 steps).
__device__ __forceinline__ float dot8(const uint4 a, const uint4 b, float acc) {
  acc = dot2(a.x, b.x, acc);
  acc = dot2(a.y, b.y, acc);
  acc = dot2(a.z, b.z, acc);
  acc = dot2(a.w, b.w, acc);
  return acc;
}
__device__ __forceinline__ float dot4(const uint2 a, const uint2 b, float acc) {
  acc = dot2(a.x, b.x, acc);
  acc = dot2(a.y, b.y, acc);
  return acc;
}

// ---------------------------------------------------------------------------
// wave64 lane exchanges and reductions, without the LDS crossbar
// ---------------------------------------------------------------------------
// lane_xor<M>(v) is v of lane (lane ^ M).  Distances 32 and 16 use the gfx950
// permlane swaps (v_permlane32_swap: upper half of the first operand with
// the lower half of the second; v_permlane16_swap: odd rows of the first
// with even rows of the second), 8 a row rotate, 4 a half-row mirror (^7)
// then a quad reversal (^3), 2 and 1 quad permutes.  Every step pairs lane i
// with lane i ^ M, so a butterfly built from them adds in the same tree as a
// shuffle butterfly and gives the same bits.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
constexpr int kDppQuadXor1 = 0xb1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4e;     // quad_perm [2,3,0,1]
constexpr int kDppQuadXor3 = 0x1b;     // quad_perm [3,2,1,0]
constexpr int kDppHalfRowMirror = 0x141;
constexpr int kDppRowRor8 = 0x128;

// Swap through the permlane instructions: on return a holds, in lanes with
// bit M clear, their own a and in the others the partner's b; b holds the
// partner's a resp. their own b.  With a == b: {a, b} = {own, partner} in
// some order, so a commutative op of the two is the butterfly step.
template <int M>
__device__ __forceinline__ void permlane_swap(float& a, float& b) {
  static_assert(M == 32 || M == 16, "permlane swaps exist for 32 and 16");
  const uint32_t ua = __float_as_uint(a), ub = __float_as_uint(b);
  if constexpr (M == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(ua, ub, false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane16_swap(ua, ub, false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
  }
}

template <int M>
__device__ __forceinline__ float lane_xor(float v) {
  if constexpr (M == 32 || M == 16) {
    float a = v, b = v;
    permlane_swap<M>(a, b);
    return (__lane_id() & M) ? a : b;
  } else if constexpr (M == 8) {
    return dpp_f32<kDppRowRor8>(v);
  } else if constexpr (M == 4) {
    return dpp_f32<kDppQuadXor3>(dpp_f32<kDppHalfRowMirror>(v));
  } else if constexpr (M == 2) {
    return dpp_f32<kDppQuadXor2>(v);
  } else {
    static_assert(M == 1, "lane distance must be a power of two <= 32");
    return dpp_f32<kDppQuadXor1>(v);
  }
}

// v of lane l (wave-uniform l), broadcast through a scalar register
__device__ __forceinline__ float read_lane(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// v (op) v of lane ^ M, for a commutative op
template <int M, typename Op>
__device__ __forceinline__ float xor_step(float v, Op op) {
  if constexpr (M == 32 || M == 16) {
    float a = v, b = v;
    permlane_swap<M>(a, b);
    return op(a, b);
  } else {
    return op(v, lane_xor<M>(v));
  }
}

struct AddOp {
  __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};
struct MaxOp {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

// Butterfly over all 64 lanes: every lane ends with the same value.
__device__ __forceinline__ float wave_sum(float v) {
  v = xor_step<32>(v, AddOp{});
  v = xor_step<16>(v, AddOp{});
  v = xor_step<8>(v, AddOp{});
  v = xor_step<4>(v, AddOp{});
  v = xor_step<2>(v, AddOp{});
  return xor_step<1>(v, AddOp{});
}
__device__ __forceinline__ float wave_max(float v) {
  v = xor_step<32>(v, MaxOp{});
  v = xor_step<16>(v, MaxOp{});
  v = xor_step<8>(v, MaxOp{});
  v = xor_step<4>(v, MaxOp{});
  v = xor_step<2>(v, MaxOp{});
  return xor_step<1>(v, MaxOp{});
}

// Unsigned max over the wave: row rotates by 8, 4, 2, 1 (each lane then
// holds its row's max), then the two permlane swaps across rows.  Every
// lane ends with the wave's max.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ uint32_t umax32(uint32_t a, uint32_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = umax32(v, dpp_u32<0x128>(v));  // row_ror:8
  v = umax32(v, dpp_u32<0x124>(v));  // row_ror:4
  v = umax32(v, dpp_u32<0x122>(v));  // row_ror:2
  v = umax32(v, dpp_u32<0x121>(v));  // row_ror:1
  float a = __uint_as_float(v), b = a;
  permlane_swap<16>(a, b);
  v = umax32(__float_as_uint(a), __float_as_uint(b));
  a = __uint_as_float(v);
  b = a;
  permlane_swap<32>(a, b);
  return umax32(__float_as_uint(a), __float_as_uint(b));
}

// The same max as a wave-uniform (scalar) value: row maxima by DPP, then
// the four rows' lanes 0, 16, 32, 48 read into scalar registers.
__device__ __forceinline__ uint32_t wave_max_u32_uniform(uint32_t v) {
  v = umax32(v, dpp_u32<0x128>(v));  // row_ror:8
  v = umax32(v, dpp_u32<0x124>(v));  // row_ror:4
  v = umax32(v, dpp_u32<0x122>(v));  // row_ror:2
  v = umax32(v, dpp_u32<0x121>(v));  // row_ror:1
  const uint32_t r0 = __builtin_amdgcn_readlane(static_cast<int>(v), 0);
  const uint32_t r1 = __builtin_amdgcn_readlane(static_cast<int>(v), 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(static_cast<int>(v), 32);
  const uint32_t r3 = __builtin_amdgcn_readlane(static_cast<int>(v), 48);
  return umax32(umax32(r0, r1), umax32(r2, r3));
}

// Inclusive prefix sum over the wave's 64 lanes (lane l: v of lanes 0..l),
// all in DPP: row shifts by 1, 2, 4, 8 (zero fill at the row start) give
// the prefix within each row of 16; row_bcast:15 adds row 0's total to row
// 1 and row 2's to row 3; row_bcast:31 adds lane 31's prefix (rows 0-1) to
// rows 2 and 3.  Integer adds: exact in any order.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_i32_zero(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, true);
}
__device__ __forceinline__ int wave_inclusive_sum(int v) {
  v += dpp_i32_zero<0x111, 0xf>(v);  // row_shr:1
  v += dpp_i32_zero<0x112, 0xf>(v);  // row_shr:2
  v += dpp_i32_zero<0x114, 0xf>(v);  // row_shr:4
  v += dpp_i32_zero<0x118, 0xf>(v);  // row_shr:8
  v += dpp_i32_zero<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_i32_zero<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}
__device__ __forceinline__ int read_lane_i32(int v, int l) {
  return __builtin_amdgcn_readlane(v, l);
}

// One reduce-scatter step over lane bit M: lanes with the bit clear end with
// lo + partner's lo, the others with hi + partner's hi.
template <int M>
__device__ __forceinline__ float exchange_add(float lo, float hi, int lane) {
  if constexpr (M == 32 || M == 16) {
    permlane_swap<M>(lo, hi);
    return lo + hi;
  } else {
    const bool upper = (lane & M) != 0;
    const float send = upper ? lo : hi;
    const float keep = upper ? hi : lo;
    return keep + lane_xor<M>(send);
  }
}

template <int BIT, int LO>
__device__ __forceinline__ float butterfly_sum(float r) {
  if constexpr (BIT >= LO) {
    r = xor_step<(1 << BIT)>(r, AddOp{});
    return butterfly_sum<BIT - 1, LO>(r);
  } else {
    return r;
  }
}

template <int V, int B, int HI>
__device__ __forceinline__ void scatter_steps(float (&v)[V], int lane) {
  if constexpr ((V >> (B + 1)) >= 1) {
    constexpr int half = V >> (B + 1);
#pragma unroll
    for (int i = 0; i < half; ++i) v[i] = exchange_add<(1 << (HI - B))>(v[i], v[half + i], lane);
    scatter_steps<V, B + 1, HI>(v, lane);
  }
}

// Sum V values per lane over the lanes that differ in bits LO..HI of the lane
// id, leaving ONE total per lane: the first log2(V) steps exchange halves of
// the value set (a reduce-scatter: V-1 exchanges instead of V*(HI-LO+1)), the
// rest are plain butterfly adds.  On return, the lane holds value index
// scatter_index<HI, LO, log2 V>(lane).
template <int V, int HI, int LO>
__device__ __forceinline__ float reduce_scatter(float (&v)[V], int lane) {
  constexpr int L = (V >= 16) ? 4 : (V >= 8) ? 3 : (V >= 4) ? 2 : (V >= 2) ? 1 : 0;
  static_assert((1 << L) == V, "V must be a power of two <= 16");
  static_assert(HI - LO + 1 >= L, "not enough lane bits");
  static_assert(HI <= 5 && LO >= 0, "lane bits of a wave64");
  scatter_steps<V, 0, HI>(v, lane);
  return butterfly_sum<HI - L, LO>(v[0]);
}

template <int HI, int LO, int L>
__device__ __forceinline__ int scatter_index(int lane) {
  int idx = 0;
#pragma unroll
  for (int b = 0; b < L; ++b) idx = (idx << 1) | ((lane >> (HI - b)) & 1);
  return idx;
}

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte streaming (non-temporal) load of weights read once per launch:
// measured 7.1 TB/s on a 4 GiB read against 6.2 TB/s for plain loads.
__device__ __forceinline__ uint4 load_stream16(const uint16_t* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// 16-byte loads issued by every lane whatever the guard: where !ok the
// address is clamped to p itself (a valid element) and the value replaced
// by zeros.  A load inside a lane-dependent branch is waited for before the
// branch ends, so per-chunk guarded loads complete one after another (a
// decode GEMV measured 1.05 us slower out of 10); these stay in flight
// together.
__device__ __forceinline__ uint4 load_stream16_if(const uint16_t* p, int off, bool ok) {
  const uint4 v = load_stream16(p + (ok ? off : 0));
  return ok ? v : make_uint4(0u, 0u, 0u, 0u);
}
__device__ __forceinline__ uint4 load16_if(const uint16_t* p, int off, bool ok) {
  const uint4 v = *reinterpret_cast<const uint4*>(p + (ok ? off : 0));
  return ok ? v : make_uint4(0u, 0u, 0u, 0u);
}

// The two guarded loads with the guard dropped when the caller knows it holds
// (CHECK false: the chunks tile the row exactly).  A guarded load costs its
// lanes a zeroed register set and an exec-masked load per chunk; in the
// multi-token GEMV loops that is a quarter of the instructions per token.
template <bool CHECK>
__device__ __forceinline__ uint4 load16_g(const uint16_t* p, int off, bool ok) {
  if constexpr (CHECK) return load16_if(p, off, ok);
  else return *reinterpret_cast<const uint4*>(p + off);
}
template <bool CHECK>
__device__ __forceinline__ uint4 load_stream16_g(const uint16_t* p, int off, bool ok) {
  if constexpr (CHECK) return load_stream16_if(p, off, ok);
  else return load_stream16(p + off);
}

// Order LDS traffic of one wave: stores before the fence are seen by every
// lane's loads after it.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint64_t lanemask_lt(int lane) {
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// ---------------------------------------------------------------------------
// exp for x <= 0 and sigmoid, written out operation by operation so the CPU
// restatement (numpy float32) reproduces every rounding: Cody-Waite reduction
// x = n*ln2 + r with ln2 split into a 9-bit head (n*head exact) and a tail,
// then exp(r) by its degree-7 Taylor polynomial in Horner form (truncation
// error < 6e-9 relative on |r| <= ln2/2), then an exact scaling by 2^n.
// Inputs below -86 return 0 so every non-zero result is a normal float.
// No FMA contraction: each product and sum is rounded on its own.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float exp_nonpos(float x) {
#pragma clang fp contract(off)
  if (!(x >= -86.0f)) return 0.0f;
  const float n = rintf(x * 0x1.715476p+0f);   // log2(e), f32 0x3fb8aa3b
  float r = x - n * 0x1.63p-1f;                 // ln2 head 0.693359375
  r = r - n * -0x1.bd0106p-13f;                 // ln2 tail, 0xb95e8083
  float p = 0x1.a01a02p-13f;                    // 1/5040, 0x39500d01
  p = p * r + 0x1.6c16c2p-10f;                  // 1/720,  0x3ab60b61
  p = p * r + 0x1.111112p-7f;                   // 1/120,  0x3c088889
  p = p * r + 0x1.555556p-5f;                   // 1/24,   0x3d2aaaab
  p = p * r + 0x1.555556p-3f;                   // 1/6,    0x3e2aaaab
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  return ldexpf(p, static_cast<int>(n));
}

__device__ __forceinline__ float sigmoid_det(float x) {
#pragma clang fp contract(off)
  // 1 / (1 + exp(-x)) for x >= 0, exp(x) / (1 + exp(x)) below, without a
  // branch: one exp and one division per value whichever side each lane is on
  const bool pos = x >= 0.0f;
  const float e = exp_nonpos(pos ? -x : x);
  return (pos ? 1.0f : e) / (1.0f + e);
}

__device__ __forceinline__ float silu_f32(float g) {
  // silu(g) = g / (1 + exp(-g)) with the hardware exp and reciprocal (a
  // floating-point path checked against tolerance, not bit-exactly)
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

// act = silu(gate) * up at the reference's op boundaries: gate and up leave
// GMM1 as bf16, the product is formed in f32 and leaves as bf16.  Two
// outputs per call (packed, lo first): the bf16 roundings are paired
// v_cvt_pk_bf16_f32 instructions.
__device__ __forceinline__ uint32_t swiglu_bf16x2(float g0, float u0, float g1, float u1) {
  const uint32_t gp = pack_bf16x2(g0, g1);
  const uint32_t up = pack_bf16x2(u0, u1);
  const float gr0 = bf16lo(gp), gr1 = bf16hi(gp);
  const float ur0 = bf16lo(up), ur1 = bf16hi(up);
  return pack_bf16x2(silu_f32(gr0) * ur0, silu_f32(gr1) * ur1);
}

__device__ __forceinline__ uint16_t swiglu_bf16(float gate_acc, float up_acc) {
  return static_cast<uint16_t>(swiglu_bf16x2(gate_acc, up_acc, 0.0f, 0.0f) & 0xffffu);
}

}  // namespace lmoe

// Host-side status helper shared by the entry points.
#define LMOE_RETURN_LAUNCH()                              \
  do {                                                    \
    hipError_t _e = hipGetLastError();                    \
    return _e == hipSuccess ? LMOE_OK : static_cast<int>(_e); \
  } while (0)
