// Device helpers shared by the latchmoe gfx950 kernels: bf16 packing,
// wave64 reductions and the one exp/sigmoid routine used by the router.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "latchmoe.h"

namespace lmoe {

constexpr int kWave = 64;

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
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

// dot of 8 bf16 pairs held in two uint4, accumulated into acc in element order
__device__ __forceinline__ float dot8(const uint4 a, const uint4 b, float acc) {
  acc += bf16lo(a.x) * bf16lo(b.x);
  acc += bf16hi(a.x) * bf16hi(b.x);
  acc += bf16lo(a.y) * bf16lo(b.y);
  acc += bf16hi(a.y) * bf16hi(b.y);
  acc += bf16lo(a.z) * bf16lo(b.z);
  acc += bf16hi(a.z) * bf16hi(b.z);
  acc += bf16lo(a.w) * bf16lo(b.w);
  acc += bf16hi(a.w) * bf16hi(b.w);
  return acc;
}
__device__ __forceinline__ float dot4(const uint2 a, const uint2 b, float acc) {
  acc += bf16lo(a.x) * bf16lo(b.x);
  acc += bf16hi(a.x) * bf16hi(b.x);
  acc += bf16lo(a.y) * bf16lo(b.y);
  acc += bf16hi(a.y) * bf16hi(b.y);
  return acc;
}

// ---------------------------------------------------------------------------
// wave64 reductions (butterfly: every lane ends with the same value)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
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
  if (x >= 0.0f) {
    const float e = exp_nonpos(-x);
    return 1.0f / (1.0f + e);
  }
  const float e = exp_nonpos(x);
  return e / (1.0f + e);
}

__device__ __forceinline__ float silu_f32(float g) {
  // silu(g) = g / (1 + exp(-g)); plain device expf is fine here (FP path
  // checked against tolerance, not bit-exactly).
  return g / (1.0f + __expf(-g));
}

__device__ __forceinline__ uint16_t swiglu_bf16(float gate_acc, float up_acc) {
  const float g = round_bf16(gate_acc);
  const float u = round_bf16(up_acc);
  return static_cast<uint16_t>(f32_to_bf16_bits(silu_f32(g) * u));
}

}  // namespace lmoe

// Host-side status helper shared by the entry points.
#define LMOE_RETURN_LAUNCH()                              \
  do {                                                    \
    hipError_t _e = hipGetLastError();                    \
    return _e == hipSuccess ? LMOE_OK : static_cast<int>(_e); \
  } while (0)
