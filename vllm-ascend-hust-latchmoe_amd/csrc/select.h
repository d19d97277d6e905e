// Expert selection for one token per wave64: softmax top-k, or sigmoid +
// correction bias + group-limited top-k, with renormalisation and scaling.
//
// Selection order is (score desc, expert id asc), the order torch.topk gives
// with ties to the lower id.  Instead of k serial rounds of wave arg-max,
// each score becomes an order-preserving 32-bit key and a most-significant-
// bit-first radix select (one ballot per expert slot and bit, stopping once
// the prefix found is shared by exactly the experts still needed) finds the
// k-th largest key's prefix; the taken experts (the lowest ids among equal
// keys) are compacted with ballots and only those k are ranked against each
// other through LDS.
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
  float2 cand[EPL * kWave]; // (key bits, id bits) of the taken experts
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

// Selects the k experts of one token from its logits lg[j] (expert j*64 +
// lane, -inf beyond E; EPL*64 >= E) and the correction bias bv[j]
// (load_bias; used only when sp.bias is set).  SCORE (LMOE_SCORING_*) is a
// template parameter so that a kernel holds only the code of its scoring.
// Lane l < k returns the l-th selected expert id (-1 if fewer than k are
// eligible) and its final f32 weight.
template <int EPL, int SCORE>
__device__ __forceinline__ void select_token(const SelectParams& sp,
                                             float (&lg)[EPL], const float (&bv)[EPL],
                                             SelectLds<EPL>& L, int& out_e,
                                             float& out_w) {
  const int lane = threadIdx.x & 63;
  const int E = sp.E;
  const int k = sp.k;
  float sel[EPL];  // selection score
  float wgt[EPL];  // weight carried by a selected expert
  bool elig[EPL];
  if constexpr (SCORE == LMOE_SCORING_SOFTMAX) {
    if (sp.bias != nullptr) {
      // additive per-expert logit bias (rounded once, before the softmax)
#pragma unroll
      for (int j = 0; j < EPL; ++j) {
        const int e = j * kWave + lane;
        if (e < E) lg[j] = lg[j] + bv[j];
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
      const float sb = (e < E && sp.bias != nullptr) ? sg + bv[j] : sg;
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
  // 2. radix select, most significant bit first.  Invariant: thr holds the
  //    bits above b of the k-th largest key (tmask marks them), `match`
  //    experts share that prefix and `need` of them are still to be taken.
  //    Stops as soon as match == need (all of them are taken), or after bit
  //    0 with ties on the full key (the lowest ids are taken).
  int match = 0;
#pragma unroll
  for (int j = 0; j < EPL; ++j) match += __popcll(__builtin_amdgcn_ballot_w64(key[j] != 0u));
  uint32_t thr = 0u, tmask = 0u;
  int need = k;
  for (int b = 31; b >= 0 && match > need; --b) {
    const uint32_t tgt = (thr >> b) | 1u;  // prefix with bit b set
    int c1 = 0;
#pragma unroll
    for (int j = 0; j < EPL; ++j) c1 += __popcll(__builtin_amdgcn_ballot_w64((key[j] >> b) == tgt));
    if (c1 >= need) {
      thr |= 1u << b;
      match = c1;
    } else {
      need -= c1;
      match -= c1;
    }
    tmask |= 1u << b;
  }
  // 3. the taken experts (k, or every eligible one if fewer), compacted in
  //    id order, then each ranked among the others by (key desc, id asc)
  if (lane < kMaxK) {
    L.o_e[lane] = -1;
    L.o_w[lane] = 0.0f;
  }
  int C = 0, eq_before = 0;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = j * kWave + lane;
    const uint32_t pre = key[j] & tmask;
    const bool live = key[j] != 0u;
    const bool eq = live & (pre == thr);
    const uint64_t beq = __builtin_amdgcn_ballot_w64(eq);
    const int eq_rank = eq_before + static_cast<int>(__popcll(beq & lanemask_lt(lane)));
    const bool take = live & ((pre > thr) | (eq & (eq_rank < need)));
    eq_before += __popcll(beq);
    const uint64_t bt = __builtin_amdgcn_ballot_w64(take);
    if (take) {
      const int idx = C + __popcll(bt & lanemask_lt(lane));
      L.cand[idx] = make_float2(__uint_as_float(key[j]), __int_as_float(e));
      L.c_w[idx] = wgt[j];
    }
    C += __popcll(bt);
  }
  // pad to kMaxK entries with key 0 (beats nothing)
  if (lane >= C && lane < kMaxK) L.cand[lane] = make_float2(__uint_as_float(0u), __int_as_float(0x7fffffff));
  wave_lds_sync();
  if (lane < C) {
    const float2 me2 = L.cand[lane];
    const uint32_t mk = __float_as_uint(me2.x);
    const int mid = __float_as_int(me2.y);
    const float4* cand4 = reinterpret_cast<const float4*>(L.cand);
    int rr = 0;
#pragma unroll
    for (int u = 0; u < kMaxK / 2; ++u) {
      const float4 q = cand4[u];
      const uint32_t k0 = __float_as_uint(q.x), k1 = __float_as_uint(q.z);
      const int i0 = __float_as_int(q.y), i1 = __float_as_int(q.w);
      rr += ((k0 > mk) | ((k0 == mk) & (i0 < mid))) ? 1 : 0;
      rr += ((k1 > mk) | ((k1 == mk) & (i1 < mid))) ? 1 : 0;
    }
    L.o_e[rr] = mid;
    L.o_w[rr] = L.c_w[lane];
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

// Correction bias in the lane layout (0 where absent).  Issued before the
// logits so that both loads are in flight together.
template <int EPL>
__device__ __forceinline__ void load_bias(const SelectParams& sp, float (&bv)[EPL]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = j * kWave + lane;
    bv[j] = (sp.bias != nullptr && e < sp.E) ? sp.bias[e] : 0.0f;
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
