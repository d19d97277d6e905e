// Expert selection for one token per wave64: softmax top-k, or sigmoid +
// correction bias + group-limited top-k, with renormalisation and scaling.
//
// Selection order is (score desc, expert id asc), the order torch.topk gives
// with ties to the lower id.  Instead of k serial rounds of wave arg-max
// (a chain of 12 cross-lane shuffles per round), the k best are found by
// ranking:
//   1. every lane takes the best of its own experts (e = j*64 + lane);
//   2. the lane maxima are ranked against each other through LDS; the value
//      of the lane maximum of rank k-1 is a lower bound on the k-th best
//      score (k distinct experts reach it), so only experts at or above it
//      can be selected;
//   3. those candidates (usually k..2k) are compacted with ballots and each
//      is ranked against the others; rank r < k lands in output slot r.
// The rank of a candidate among candidates equals its rank among all
// experts, because every expert that beats a candidate is a candidate too.
//
// Reference behaviour: moe_router_op.py:191-278 (gate then select_experts),
// renorm contract patches/patch_fused_moe.py:597-632
// (w / w.sum().clamp_min(eps)), grouped sigmoid as configured for the
// DeepSeek-V3-style layer (bias for selection only, sum of the two best
// scores per group, keep topk_group groups, renormalise, then scale).
#pragma once

#include <float.h>

#include "lmoe_device.h"

namespace lmoe {

constexpr int kMaxEPL = 8;  // E <= 8 * 64 = 512 experts per token
constexpr int kMaxK = 16;
constexpr int kMaxE = kMaxEPL * kWave;

struct SelectParams {
  int E;
  int k;
  int scoring;
  const float* bias;
  int n_group;
  int topk_group;
  int renorm;
  float routed_scale;
};

// Per-wave LDS scratch of one selection over up to EPL*64 experts.  Score/id
// pairs are interleaved so one 16-byte LDS read returns two entries; the
// ranking loops are unrolled so all their reads are in flight together (a
// rolled loop waits for each read in turn: ~120 cycles x 64).
template <int EPL>
struct SelectLds {
  float2 lm[kWave];         // (score, id as float bits) of every lane maximum
  float2 cand[EPL * kWave]; // (score, id bits) of the candidates
  float c_w[EPL * kWave];
  float c_s[EPL * kWave];   // score table of the groups (grouped sigmoid)
  float gsc[kWave];
  float o_w[kMaxK];
  int o_e[kMaxK];
};

// (value desc, id asc) ordering used by every selection step.  Written
// without short-circuit evaluation: as `a || (b && c)` the compiler emits a
// divergent branch (and a separate LDS read and wait) per comparison, which
// serialises the unrolled ranking loops.
__device__ __forceinline__ bool better(float v, int e, float v2, int e2) {
  const bool gt = v > v2;
  const bool eq = v == v2;
  const bool lt = e < e2;
  return gt | (eq & lt);
}

// Order LDS traffic of one wave: stores before the fence are seen by every
// lane's loads after it.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Selects the k experts of one token from its logits lg[j] (expert j*64 +
// lane, -inf beyond E; EPL*64 >= E).  Lane l < k returns the l-th selected
// expert id (-1 if fewer than k are eligible) and its final f32 weight.
template <int EPL>
__device__ __forceinline__ void select_token(const SelectParams& sp,
                                             float (&lg)[EPL],
                                             SelectLds<EPL>& L, int& out_e,
                                             float& out_w) {
  const int lane = threadIdx.x & 63;
  const int E = sp.E;
  const int k = sp.k;
  float sel[EPL];  // selection score
  float wgt[EPL];  // weight carried by a selected expert
  bool elig[EPL];
  if (sp.scoring == LMOE_SCORING_SOFTMAX) {
    if (sp.bias != nullptr) {
      // additive per-expert logit bias (rounded once, before the softmax)
#pragma unroll
      for (int j = 0; j < EPL; ++j) {
        const int e = j * kWave + lane;
        if (e < E) lg[j] = lg[j] + sp.bias[e];
      }
    }
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < EPL; ++j) m = fmaxf(m, lg[j]);
    m = wave_max(m);
    float ex[EPL];
    float local = 0.0f;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int e = j * kWave + lane;
      ex[j] = (e < E) ? exp_nonpos(lg[j] - m) : 0.0f;
      local = (j == 0) ? ex[0] : local + ex[j];
    }
    const float s = wave_sum(local);
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int e = j * kWave + lane;
      const float p = ex[j] / s;
      sel[j] = p;
      wgt[j] = p;
      elig[j] = e < E;
    }
  } else {
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int e = j * kWave + lane;
      const float sg = sigmoid_det(lg[j]);
      const float sb = (e < E && sp.bias != nullptr) ? sg + sp.bias[e] : sg;
      sel[j] = sb;
      wgt[j] = sg;
      elig[j] = e < E;
    }
    if (sp.n_group > 1) {
      const int ng = sp.n_group;
      const int gs = E / ng;
#pragma unroll
      for (int j = 0; j < EPL; ++j) {
        const int e = j * kWave + lane;
        if (e < E) L.c_s[e] = sel[j];
      }
      wave_lds_sync();
      // group score = best + second best selection score of the group
      float gscore = -INFINITY;
      if (lane < ng) {
        float m1 = -INFINITY, m2 = -INFINITY;
        int i = 0;
        for (; i + 4 <= gs; i += 4) {
          float q[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) q[u] = L.c_s[lane * gs + i + u];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            if (q[u] > m1) {
              m2 = m1;
              m1 = q[u];
            } else if (q[u] > m2) {
              m2 = q[u];
            }
          }
        }
        for (; i < gs; ++i) {
          const float v = L.c_s[lane * gs + i];
          if (v > m1) {
            m2 = m1;
            m1 = v;
          } else if (v > m2) {
            m2 = v;
          }
        }
        gscore = m1 + m2;
        L.gsc[lane] = gscore;
      }
      wave_lds_sync();
      // keep the topk_group best groups (ties to the lower group id)
      int r = 0;
#pragma unroll 8
      for (int g = 0; g < ng; ++g) r += better(L.gsc[g], g, gscore, lane) ? 1 : 0;
      const uint64_t kept = __ballot(lane < ng && r < sp.topk_group);
#pragma unroll
      for (int j = 0; j < EPL; ++j) {
        const int e = j * kWave + lane;
        elig[j] = (e < E) && ((kept >> (e / gs)) & 1ull);
      }
      wave_lds_sync();  // c_s is reused below
    }
  }

  // 1. lane maxima
  float m = -INFINITY;
  int me = 0x7fffffff;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = j * kWave + lane;
    if (elig[j] && better(sel[j], e, m, me)) {
      m = sel[j];
      me = e;
    }
  }
  L.lm[lane] = make_float2(m, __int_as_float(me));
  if (lane < kMaxK) {
    L.o_e[lane] = -1;
    L.o_w[lane] = 0.0f;
  }
  wave_lds_sync();
  // 2. threshold: value of the lane maximum of rank k-1 (-inf if fewer than
  //    k lanes hold an eligible expert)
  int r = 0;
  {
    const float4* lm4 = reinterpret_cast<const float4*>(L.lm);
#pragma unroll
    for (int l = 0; l < kWave / 2; ++l) {
      const float4 q = lm4[l];
      r += better(q.x, __float_as_int(q.y), m, me) ? 1 : 0;
      r += better(q.z, __float_as_int(q.w), m, me) ? 1 : 0;
    }
  }
  const uint64_t at = __ballot(me != 0x7fffffff && r == k - 1);
  const float thr = at ? __shfl(m, __ffsll(static_cast<long long>(at)) - 1, kWave)
                       : -INFINITY;
  // 3. compact the candidates, in ascending expert id order
  int C = 0;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = j * kWave + lane;
    const bool c = elig[j] && sel[j] >= thr;
    const uint64_t bm = __ballot(c);
    if (c) {
      const int idx = C + __popcll(bm & lanemask_lt(lane));
      L.cand[idx] = make_float2(sel[j], __int_as_float(e));
      L.c_w[idx] = wgt[j];
    }
    C += __popcll(bm);
  }
  // pad to a multiple of 8 with entries that beat nothing (C <= E <= EPL*64,
  // a multiple of 8, so the padded range stays inside cand[])
  const int C8 = (C + 7) >> 3;
  if (lane < 8 && C + lane < C8 * 8) L.cand[C + lane] = make_float2(-INFINITY, __int_as_float(0x7fffffff));
  wave_lds_sync();
  const float4* cand4 = reinterpret_cast<const float4*>(L.cand);
  for (int i0 = 0; i0 < C; i0 += kWave) {
    const int i = i0 + lane;
    const float2 me2 = i < C ? L.cand[i] : make_float2(-INFINITY, __int_as_float(0x7fffffff));
    const float cs = me2.x;
    const int ce = __float_as_int(me2.y);
    int rr = 0;
    for (int b = 0; b < C8; ++b) {
      float4 q[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) q[u] = cand4[b * 4 + u];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        rr += better(q[u].x, __float_as_int(q[u].y), cs, ce) ? 1 : 0;
        rr += better(q[u].z, __float_as_int(q[u].w), cs, ce) ? 1 : 0;
      }
    }
    if (i < C && rr < k) {
      L.o_e[rr] = ce;
      L.o_w[rr] = L.c_w[i];
    }
  }
  wave_lds_sync();
  // renormalise in selection order, scale
  float ow[kMaxK];
  {
    const float4* o4 = reinterpret_cast<const float4*>(L.o_w);
#pragma unroll
    for (int u = 0; u < kMaxK / 4; ++u) {
      const float4 q = o4[u];
      ow[4 * u] = q.x;
      ow[4 * u + 1] = q.y;
      ow[4 * u + 2] = q.z;
      ow[4 * u + 3] = q.w;
    }
  }
  float sum = ow[0];
#pragma unroll
  for (int it = 1; it < kMaxK; ++it)
    if (it < k) sum = sum + ow[it];
  const float denom = fmaxf(sum, FLT_EPSILON);
  out_e = -1;
  out_w = 0.0f;
  if (lane < k) {
    out_e = L.o_e[lane];
    const float w = sp.renorm ? L.o_w[lane] / denom : L.o_w[lane];
    out_w = w * sp.routed_scale;
  }
  wave_lds_sync();  // the scratch may be reused by the next token
}

// Logits of token t in the lane layout (expert j*64 + lane), -inf beyond E.
template <int EPL>
__device__ __forceinline__ void load_logits(const void* logits, int logits_f32,
                                            int t, int E, float (&lg)[EPL]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = j * kWave + lane;
    float v = -INFINITY;
    if (e < E) {
      const size_t o = static_cast<size_t>(t) * E + e;
      v = logits_f32 ? reinterpret_cast<const float*>(logits)[o]
                     : bf16_to_f32(reinterpret_cast<const uint16_t*>(logits)[o]);
    }
    lg[j] = v;
  }
}

}  // namespace lmoe
