// Expert selection for one token per wave64: softmax top-k, or sigmoid +
// group-limited top-k, with renormalisation and scaling.  Two optional
// per-expert f32 biases: a logit bias added to the logits before scoring
// (the router gate's linear bias), and the correction bias
// (e_score_correction_bias), added to the scores for selection only: the
// weights are the unbiased scores, for softmax and sigmoid alike.
//
// Selection order is (score desc, expert id asc), the order torch.topk gives
// with ties to the lower id.  Each score becomes an order-preserving 32-bit
// key; k rounds of wave arg-max (an unsigned max over the wave through DPP
// row rotates and the permlane swaps, then a ballot on equality that picks
// the lowest id among equal keys) produce the experts already in selection
// order, with no sort, compaction or LDS ranking.
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
  int n_shared;  // shared-expert suffix appended to every token (ids E.., weight 1)
  int scoring;
  const float* bias;        // correction bias: selection only
  const float* logit_bias;  // added to the logits before scoring
  int n_group;
  int topk_group;
  int renorm;
  float routed_scale;
};

// Per-wave LDS scratch of one selection: the score table and group scores
// of the grouped sigmoid (the other scorings use none).
template <int EPL>
struct SelectLds {
  float c_s[EPL * kWave];   // score table of the groups (grouped sigmoid)
  float gsc[kWave];
};

// Order-preserving 32-bit key of a score: key(a) > key(b) <=> a > b, -0
// made +0 first (so equal scores have equal keys); score_of_key inverts it.
__device__ __forceinline__ uint32_t score_key(float v) {
  const uint32_t u = __float_as_uint(v + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float score_of_key(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

// One top-two merge step with the lane M apart: (a1 >= a2) and the
// partner's (b1 >= b2) become the two largest of the four.
template <int M>
__device__ __forceinline__ void top2_step(uint32_t& a1, uint32_t& a2) {
  const uint32_t b1 = __float_as_uint(lane_xor<M>(__uint_as_float(a1)));
  const uint32_t b2 = __float_as_uint(lane_xor<M>(__uint_as_float(a2)));
  const uint32_t lo = a1 < b1 ? a1 : b1;
  a1 = umax32(a1, b1);
  a2 = umax32(lo, umax32(a2, b2));
}

// The two largest keys (a copy of the largest counts as the second) over
// the aligned block of 2^LG lanes holding this lane; every lane of the block
// ends with them.
template <int LG>
__device__ __forceinline__ void block_top2_key(uint32_t& a1, uint32_t& a2) {
  if constexpr (LG >= 6) top2_step<32>(a1, a2);
  if constexpr (LG >= 5) top2_step<16>(a1, a2);
  if constexpr (LG >= 4) top2_step<8>(a1, a2);
  if constexpr (LG >= 3) top2_step<4>(a1, a2);
  if constexpr (LG >= 2) top2_step<2>(a1, a2);
  top2_step<1>(a1, a2);
}

// Group scores (best + second best selection score) of groups of 2^LG
// experts, which are aligned lane blocks of one register: a top-two
// butterfly over the blocks' keys.  The score of group g goes to gsc[g]
// (g < ng).
template <int LG, int EPL>
__device__ __forceinline__ void group_scores_pow2(const float (&sel)[EPL], int ng, float* gsc) {
  constexpr int GS = 1 << LG;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    uint32_t k1 = score_key(sel[j]), k2 = 0u;
    block_top2_key<LG>(k1, k2);
    const float gsum = score_of_key(k1) + score_of_key(k2);
    const int g = (j * kWave + lane) >> LG;
    if ((lane & (GS - 1)) == 0 && g < ng) gsc[g] = gsum;
  }
}

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

// Selects the k experts of one token from its logits lg[j] (expert j*64 +
// lane, -inf beyond E; EPL*64 >= E), the correction bias bv[j] and the
// logit bias lb[j] (load_bias; used only when sp.bias / sp.logit_bias are
// set).  SCORE (LMOE_SCORING_*) is a
// template parameter so that a kernel holds only the code of its scoring.
// Lane l < k returns the l-th selected expert id (-1 if fewer than k are
// eligible) and its final f32 weight.
template <int EPL, int SCORE>
__device__ __forceinline__ void select_token(const SelectParams& sp,
                                             float (&lg)[EPL], const float (&bv)[EPL],
                                             const float (&lb)[EPL], SelectLds<EPL>& L,
                                             int& out_e, float& out_w) {
  const int lane = threadIdx.x & 63;
  const int E = sp.E;
  const int k = sp.k;
  float sel[EPL];  // selection score
  float wgt[EPL];  // weight carried by a selected expert
  bool elig[EPL];
  if (sp.logit_bias != nullptr) {
    // additive per-expert logit bias (one f32 rounding, before scoring)
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int e = j * kWave + lane;
      if (e < E) lg[j] = lg[j] + lb[j];
    }
  }
  if constexpr (SCORE == LMOE_SCORING_SOFTMAX) {
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
      sel[j] = (e < E && sp.bias != nullptr) ? p + bv[j] : p;
      wgt[j] = p;
      elig[j] = e < E;
    }
  } else {
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int e = j * kWave + lane;
      const float sg = sigmoid_det(lg[j]);
      const float sb = (e < E && sp.bias != nullptr) ? sg + bv[j] : sg;
      sel[j] = sb;
      wgt[j] = sg;
      elig[j] = e < E;
    }
    if (sp.n_group > 1) {
      const int ng = sp.n_group;
      const int gs = E / ng;
      // group score = best + second best selection score of the group
      float gscore = -INFINITY;
      const int lg2 = 31 - __builtin_clz(gs);
      if (gs == (1 << lg2) && lg2 >= 4 && lg2 <= 6) {
        // groups of 16, 32 or 64 experts (DeepSeek-V3: 256 experts in 8
        // groups of 32) are aligned lane blocks of one register
        if (lg2 == 5) group_scores_pow2<5>(sel, ng, L.gsc);
        else if (lg2 == 4) group_scores_pow2<4>(sel, ng, L.gsc);
        else group_scores_pow2<6>(sel, ng, L.gsc);
        wave_lds_sync();
        if (lane < ng) gscore = L.gsc[lane];
      } else {
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
          const int e = j * kWave + lane;
          if (e < E) L.c_s[e] = sel[j];
        }
        wave_lds_sync();
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
      }
      wave_lds_sync();
      // keep the topk_group best groups (ties to the lower group id)
      int r = 0;
#pragma unroll 8
      for (int g = 0; g < ng; ++g) r += better(L.gsc[g], g, gscore, lane) ? 1 : 0;
      const uint64_t kept = __ballot(lane < ng && r < sp.topk_group);
      // group of expert e: e / gs (a shift for the power-of-two sizes)
      const bool pow2 = (gs & (gs - 1)) == 0;
      const int sh = pow2 ? 31 - __builtin_clz(gs) : 0;
#pragma unroll
      for (int j = 0; j < EPL; ++j) {
        const int e = j * kWave + lane;
        const int g = pow2 ? (e >> sh) : e / gs;
        elig[j] = (e < E) && ((kept >> g) & 1ull);
      }
      wave_lds_sync();  // the scratch may be reused by the next token
    }
  }

  // 1. order-preserving 32-bit keys: key(a) > key(b) <=> a > b for scores
  //    (-0 is made +0 so equal scores tie and go to the lower id); key 0
  //    marks an expert that is not eligible
  uint32_t key[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const uint32_t u = __float_as_uint(sel[j] + 0.0f);
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    key[j] = elig[j] ? o : 0u;
  }
  // 2. k rounds of wave arg-max, without branches.  Round r takes the
  //    largest key left (the lowest id among equal keys), writes its id and
  //    weight into lane r and clears it; the weights are summed in
  //    selection order as they come.  Once the largest key left is 0 (fewer
  //    than k experts are eligible) the remaining rounds write -1 and 0.
  int my_e = -1;
  float my_w = 0.0f;
  float sum = 0.0f;
  for (int r = 0; r < k; ++r) {
    uint32_t lm = key[0];
#pragma unroll
    for (int j = 1; j < EPL; ++j) lm = lm > key[j] ? lm : key[j];
    const uint32_t best = wave_max_u32_uniform(lm);
    uint64_t bm[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) bm[j] = __builtin_amdgcn_ballot_w64(key[j] == best);
    uint64_t bsel = bm[EPL - 1];
    int wj = EPL - 1;
#pragma unroll
    for (int j = EPL - 2; j >= 0; --j) {
      if (bm[j] != 0ull) {
        bsel = bm[j];
        wj = j;
      }
    }
    const bool ok = best != 0u;
    const int wl = static_cast<int>(__builtin_ctzll(bsel | (1ull << 63)));  // in [0, 63]
    float w = read_lane(wgt[0], wl);
#pragma unroll
    for (int j = 1; j < EPL; ++j) {
      const float wjv = read_lane(wgt[j], wl);
      w = (j == wj) ? wjv : w;
    }
    w = ok ? w : 0.0f;
    sum = (r == 0) ? w : sum + w;
    const bool mine = lane == r;
    my_e = mine ? (ok ? wj * kWave + wl : -1) : my_e;
    my_w = mine ? w : my_w;
#pragma unroll
    for (int j = 0; j < EPL; ++j) key[j] = (j == wj && lane == wl) ? 0u : key[j];
  }
  // 3. renormalise (sum in selection order), scale
  const float denom = fmaxf(sum, FLT_EPSILON);
  out_e = -1;
  out_w = 0.0f;
  if (lane < k) {
    out_e = my_e;
    const float w = sp.renorm ? my_w / denom : my_w;
    out_w = w * sp.routed_scale;
  }
}

// Correction bias bv and logit bias lb in the lane layout (0 where absent).
// Issued before the logits so that all loads are in flight together.
template <int EPL>
__device__ __forceinline__ void load_bias(const SelectParams& sp, float (&bv)[EPL],
                                          float (&lb)[EPL]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = j * kWave + lane;
    bv[j] = (sp.bias != nullptr && e < sp.E) ? sp.bias[e] : 0.0f;
    lb[j] = (sp.logit_bias != nullptr && e < sp.E) ? sp.logit_bias[e] : 0.0f;
  }
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
