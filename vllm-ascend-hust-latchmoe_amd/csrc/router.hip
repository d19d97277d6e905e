// Router kernels: gate linear (bf16 GEMV, f32 accumulation) and expert
// selection (softmax top-k, or sigmoid + correction bias + group-limited
// top-k), one wave64 per token.
//
// Reference behaviour: moe_router_op.py:191-278 (gate then select_experts),
// renorm contract patches/patch_fused_moe.py:597-632
// (w / w.sum().clamp_min(eps)), grouped sigmoid as configured for the
// DeepSeek-V3-style layer (bias for selection only, sum of the two best scores
// per group, keep topk_group groups, renormalise, then scale).
#include <float.h>

#include "gemm_mfma.h"

namespace lmoe {

constexpr int kGateMaxChunks = 16;  // H <= 16 * 512 = 8192 in the GEMV path
constexpr int kMaxEPL = 8;          // E <= 8 * 64 = 512 experts per token
constexpr int kMaxK = 16;

// logits[t][e] for e = 4*blockIdx.x + wave, tokens [t0, t1).  The expert row
// stays in registers (one 16-byte chunk per 512 columns per lane) while the
// token rows stream through L1.
__global__ __launch_bounds__(256) void gate_gemv_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wg, int T,
    int H, int E, int tokens_per_block, void* __restrict__ logits,
    int logits_f32) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int e = blockIdx.x * 4 + wave;
  if (e >= E) return;
  const int t0 = blockIdx.y * tokens_per_block;
  const int t1 = min(T, t0 + tokens_per_block);
  const uint16_t* wrow = wg + static_cast<size_t>(e) * H;

  uint4 w[kGateMaxChunks];
#pragma unroll
  for (int c = 0; c < kGateMaxChunks; ++c) {
    const int h = c * 512 + lane * 8;
    w[c] = (h < H) ? *reinterpret_cast<const uint4*>(wrow + h)
                   : make_uint4(0u, 0u, 0u, 0u);
  }
  for (int t = t0; t < t1; ++t) {
    const uint16_t* xr = x + static_cast<size_t>(t) * H;
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < kGateMaxChunks; ++c) {
      const int h = c * 512 + lane * 8;
      if (h < H) acc = dot8(*reinterpret_cast<const uint4*>(xr + h), w[c], acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) {
      const size_t o = static_cast<size_t>(t) * E + e;
      if (logits_f32) {
        reinterpret_cast<float*>(logits)[o] = acc;
      } else {
        reinterpret_cast<uint16_t*>(logits)[o] =
            static_cast<uint16_t>(f32_to_bf16_bits(acc));
      }
    }
  }
}

// (value desc, id asc) ordering used by every selection step.
__device__ __forceinline__ bool better(float v, int e, float v2, int e2) {
  return (v > v2) || (v == v2 && e < e2);
}

// Wave-wide arg-best: all lanes return the winning (value, id).
__device__ __forceinline__ void wave_argbest(float& v, int& e) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float v2 = __shfl_xor(v, o, kWave);
    const int e2 = __shfl_xor(e, o, kWave);
    if (better(v2, e2, v, e)) {
      v = v2;
      e = e2;
    }
  }
}

// One wave per token; lane l holds experts e = j*64 + l, j < kMaxEPL.
__global__ __launch_bounds__(256) void topk_kernel(
    const void* __restrict__ logits, int logits_f32, int T, int E, int k,
    int scoring, const float* __restrict__ bias, int n_group, int topk_group,
    int renorm, float routed_scale, float* __restrict__ w_f32,
    uint16_t* __restrict__ w_bf16, int32_t* __restrict__ ids) {
  __shared__ float sel_lds[4][kMaxEPL * kWave];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  const bool token_ok = t < T;
  const int tt = token_ok ? t : 0;

  float lg[kMaxEPL];
#pragma unroll
  for (int j = 0; j < kMaxEPL; ++j) {
    const int e = j * kWave + lane;
    float v = -INFINITY;
    if (e < E) {
      const size_t o = static_cast<size_t>(tt) * E + e;
      v = logits_f32 ? reinterpret_cast<const float*>(logits)[o]
                     : bf16_to_f32(reinterpret_cast<const uint16_t*>(logits)[o]);
    }
    lg[j] = v;
  }

  float sel[kMaxEPL];   // selection score
  float wgt[kMaxEPL];   // weight carried by a selected expert
  bool elig[kMaxEPL];
  if (scoring == LMOE_SCORING_SOFTMAX) {
    if (bias != nullptr) {
      // additive per-expert logit bias (rounded once, before the softmax)
#pragma unroll
      for (int j = 0; j < kMaxEPL; ++j) {
        const int e = j * kWave + lane;
        if (e < E) lg[j] = lg[j] + bias[e];
      }
    }
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < kMaxEPL; ++j) m = fmaxf(m, lg[j]);
    m = wave_max(m);
    float ex[kMaxEPL];
    float local = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxEPL; ++j) {
      const int e = j * kWave + lane;
      ex[j] = (e < E) ? exp_nonpos(lg[j] - m) : 0.0f;
      local = (j == 0) ? ex[0] : local + ex[j];
    }
    const float s = wave_sum(local);
#pragma unroll
    for (int j = 0; j < kMaxEPL; ++j) {
      const int e = j * kWave + lane;
      const float p = ex[j] / s;
      sel[j] = p;
      wgt[j] = p;
      elig[j] = e < E;
    }
  } else {
#pragma unroll
    for (int j = 0; j < kMaxEPL; ++j) {
      const int e = j * kWave + lane;
      const float sg = sigmoid_det(lg[j]);
      const float sb = (e < E && bias != nullptr) ? sg + bias[e] : sg;
      sel[j] = sb;
      wgt[j] = sg;
      elig[j] = e < E;
    }
    if (n_group > 1) {
      const int gs = E / n_group;
#pragma unroll
      for (int j = 0; j < kMaxEPL; ++j) {
        const int e = j * kWave + lane;
        if (e < E) sel_lds[wave][e] = sel[j];
      }
      __syncthreads();
      // group score = best + second best selection score of the group
      float gscore = -INFINITY;
      if (lane < n_group) {
        float m1 = -INFINITY, m2 = -INFINITY;
        for (int i = 0; i < gs; ++i) {
          const float v = sel_lds[wave][lane * gs + i];
          if (v > m1) {
            m2 = m1;
            m1 = v;
          } else if (v > m2) {
            m2 = v;
          }
        }
        gscore = m1 + m2;
      }
      uint64_t kept = 0ull;
      bool gtaken = false;
      for (int it = 0; it < topk_group; ++it) {
        float v = (lane < n_group && !gtaken) ? gscore : -INFINITY;
        int g = (lane < n_group && !gtaken) ? lane : 0x7fffffff;
        wave_argbest(v, g);
        if (g >= 0 && g < 64) kept |= 1ull << g;
        if (lane == g) gtaken = true;
      }
#pragma unroll
      for (int j = 0; j < kMaxEPL; ++j) {
        const int e = j * kWave + lane;
        elig[j] = (e < E) && ((kept >> (e / gs)) & 1ull);
      }
    }
  }

  // k rounds of wave arg-best; lane-local candidates scanned in ascending j,
  // i.e. ascending expert id, so the first maximum is the lowest id.
  uint32_t taken = 0u;
  int sel_e[kMaxK];
  float sel_w[kMaxK];
#pragma unroll
  for (int it = 0; it < kMaxK; ++it) {
    sel_e[it] = 0;
    sel_w[it] = 0.0f;
    if (it < k) {
      float bv = -INFINITY;
      int be = 0x7fffffff;
      float bw = 0.0f;
#pragma unroll
      for (int j = 0; j < kMaxEPL; ++j) {
        const int e = j * kWave + lane;
        if (elig[j] && !((taken >> j) & 1u) && better(sel[j], e, bv, be)) {
          bv = sel[j];
          be = e;
          bw = wgt[j];
        }
      }
      float v = bv;
      int e = be;
      wave_argbest(v, e);
      const bool found = e >= 0 && e < E;
      const int owner = found ? (e & 63) : 0;
      const float w = __shfl(bw, owner, kWave);
      if (found && lane == owner) taken |= 1u << (e >> 6);
      if (!found) e = -1;  // no eligible expert left: an id no table maps
      sel_e[it] = e;
      sel_w[it] = w;
    }
  }

  float sum = sel_w[0];
#pragma unroll
  for (int it = 1; it < kMaxK; ++it)
    if (it < k) sum = sum + sel_w[it];
  const float denom = fmaxf(sum, FLT_EPSILON);

  if (token_ok && lane < k) {
    int my_e = 0;
    float my_w = 0.0f;
#pragma unroll
    for (int it = 0; it < kMaxK; ++it) {
      if (lane == it) {
        my_e = sel_e[it];
        my_w = sel_w[it];
      }
    }
    float w = renorm ? my_w / denom : my_w;
    w = w * routed_scale;
    const size_t o = static_cast<size_t>(t) * k + lane;
    ids[o] = my_e;
    w_bf16[o] = static_cast<uint16_t>(f32_to_bf16_bits(w));
    if (w_f32 != nullptr) w_f32[o] = w;
  }
}

}  // namespace lmoe

using namespace lmoe;

extern "C" int lmoe_router_gate(const void* x, const void* wg, int T, int H,
                                int E, void* logits, int logits_f32,
                                hipStream_t stream) {
  if (x == nullptr || wg == nullptr || logits == nullptr) return LMOE_ERR_ARG;
  if (T < 0 || H <= 0 || E <= 0) return LMOE_ERR_ARG;
  if (H % 8 != 0 || H > kGateMaxChunks * 512) return LMOE_ERR_SHAPE;
  if (T == 0) return LMOE_OK;
  if (T > 64) {
    // large token counts: one dense bf16 MFMA GEMM, logits = x . wg^T
    GemmArgs g{};
    g.a = static_cast<const uint16_t*>(x);
    g.w = static_cast<const uint16_t*>(wg);
    g.w_slot_stride = 0;
    g.N = E;
    g.K = H;
    g.M_dense = T;
    g.out = logits;
    g.out_f32 = logits_f32;
    hipLaunchKernelGGL(grouped_gemm_kernel<kDense>,
                       dim3((T + kBM - 1) / kBM, (E + kBN - 1) / kBN), dim3(256),
                       0, stream, g);
    LMOE_RETURN_LAUNCH();
  }
  const int tpb = 16;
  dim3 grid((E + 3) / 4, (T + tpb - 1) / tpb);
  hipLaunchKernelGGL(gate_gemv_kernel, grid, dim3(256), 0, stream,
                     static_cast<const uint16_t*>(x),
                     static_cast<const uint16_t*>(wg), T, H, E, tpb, logits,
                     logits_f32);
  LMOE_RETURN_LAUNCH();
}

extern "C" int lmoe_router_topk(const void* logits, int logits_f32, int T,
                                int E, int k, int scoring, const float* bias,
                                int n_group, int topk_group, int renorm,
                                float routed_scale, float* w_f32,
                                uint16_t* w_bf16, int32_t* ids,
                                hipStream_t stream) {
  if (logits == nullptr || w_bf16 == nullptr || ids == nullptr)
    return LMOE_ERR_ARG;
  if (T < 0 || E <= 0 || k <= 0) return LMOE_ERR_ARG;
  if (E > kMaxEPL * kWave || k > kMaxK || k > E) return LMOE_ERR_SHAPE;
  if (scoring != LMOE_SCORING_SOFTMAX && scoring != LMOE_SCORING_SIGMOID)
    return LMOE_ERR_UNSUPPORTED;
  if (scoring == LMOE_SCORING_SIGMOID && n_group > 1) {
    if (n_group > 64 || E % n_group != 0 || E / n_group < 2) return LMOE_ERR_SHAPE;
    if (topk_group <= 0 || topk_group > n_group) return LMOE_ERR_SHAPE;
    if (k > topk_group * (E / n_group)) return LMOE_ERR_SHAPE;
  }
  if (T == 0) return LMOE_OK;
  dim3 grid((T + 3) / 4);
  hipLaunchKernelGGL(topk_kernel, grid, dim3(256), 0, stream, logits,
                     logits_f32, T, E, k, scoring, bias,
                     scoring == LMOE_SCORING_SIGMOID ? n_group : 1, topk_group,
                     renorm, routed_scale, w_f32, w_bf16, ids);
  LMOE_RETURN_LAUNCH();
}
