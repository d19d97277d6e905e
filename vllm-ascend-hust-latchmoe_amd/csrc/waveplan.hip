// Device-side capacity-wave planning and plan-driven staging for an
// overflowing prefill layer: no host round trip between the router and the
// expert MLP.
//
//   wave_plan_kernel   one workgroup: histogram of the routed ids, experts in
//                      (-count, id) order, each placed in the wave with
//                      (least load, lowest index) among ceil(n / P) waves with
//                      room; members listed ascending per wave.
//   wave_stage_kernel  for one wave index: copy its members' weights into a
//                      stage buffer (from the main-bank slot when the layer's
//                      slot table maps the expert to a slot that it owns,
//                      from its host row otherwise) and write the
//                      stage buffer's table (expert -> stage slot, -1
//                      elsewhere).  A wave index past the plan's count copies
//                      nothing and writes an all -1 table, so a caller can
//                      launch a fixed number of waves (graph capture) and the
//                      extra ones compute nothing.
//
// Reference behaviour: phase_split.plan_balanced_b2_waves
// (moe_offload/phase_split.py:495-554; membership by routed count only, never
// by residency), build_b2_device_wave_microbatch_plans (:1224-1384: the
// expert -> wave and expert -> slot maps built once, pairs compacted on the
// device) and the per-wave stage-bank fill of prepare_prefill_stage_plan
// (runtime.py:2035-2258: slot i <- i-th expert of the wave, D2D for main-bank
// hits, H2D for misses).
//
// Plan buffer (int32, lmoe_wave_plan_bytes): [0] waves, [1] active experts,
// [2] ids outside [0, n_total), [3] reserved, then counts[n_routed],
// wave_of[n_routed], slot_of[n_routed], size[max_waves],
// members[max_waves * n_slots].
#include "lmoe_device.h"

namespace {

using namespace lmoe;

constexpr int kPlanThreads = 1024;
constexpr int kPlanMaxExperts = 1024;
constexpr int kPlanMaxWaves = 256;
constexpr int kPlanMaxSlots = 1024;
constexpr int kPlanHeader = 4;

struct PlanView {
  int32_t* hdr;
  int32_t* counts;
  int32_t* wave_of;
  int32_t* slot_of;
  int32_t* size;
  int32_t* members;
};

__host__ __device__ inline PlanView plan_view(int32_t* base, int n_routed, int max_waves) {
  PlanView v;
  v.hdr = base;
  v.counts = base + kPlanHeader;
  v.wave_of = v.counts + n_routed;
  v.slot_of = v.wave_of + n_routed;
  v.size = v.slot_of + n_routed;
  v.members = v.size + max_waves;
  return v;
}

__host__ __device__ inline long long plan_words(int n_routed, int n_slots, int max_waves) {
  return kPlanHeader + 3LL * n_routed + max_waves + static_cast<long long>(max_waves) * n_slots;
}

__global__ __launch_bounds__(kPlanThreads) void wave_plan_kernel(
    const int32_t* __restrict__ ids, int n_pairs, int n_routed, int n_total, int P,
    int max_waves, int32_t* __restrict__ plan) {
  __shared__ int s_cnt[kPlanMaxExperts];
  __shared__ int s_sorted[kPlanMaxExperts];
  __shared__ int s_wave[kPlanMaxExperts];
  __shared__ int s_size[kPlanMaxWaves];
  __shared__ int s_nact, s_invalid;
  const int tid = threadIdx.x;
  PlanView v = plan_view(plan, n_routed, max_waves);
  for (int e = tid; e < n_routed; e += kPlanThreads) {
    s_cnt[e] = 0;
    s_wave[e] = -1;
  }
  for (int w = tid; w < max_waves; w += kPlanThreads) s_size[w] = 0;
  if (tid == 0) {
    s_nact = 0;
    s_invalid = 0;
  }
  __syncthreads();
  // histogram; ids in [n_routed, n_total) are the pinned shared suffix
  for (int p = tid; p < n_pairs; p += kPlanThreads) {
    const int id = ids[p];
    if (id >= 0 && id < n_routed) atomicAdd(&s_cnt[id], 1);
    else if (id < 0 || id >= n_total) atomicAdd(&s_invalid, 1);
  }
  __syncthreads();
  // rank of each active expert in (-count, id) order: the keys are distinct
  for (int e = tid; e < n_routed; e += kPlanThreads) {
    const int c = s_cnt[e];
    if (c <= 0) continue;
    int r = 0;
    for (int f = 0; f < n_routed; ++f) {
      const int cf = s_cnt[f];
      r += (cf > c || (cf == c && f < e)) ? 1 : 0;
    }
    s_sorted[r] = e;
    atomicAdd(&s_nact, 1);
  }
  __syncthreads();
  const int n_act = s_nact;
  const int n_waves = (n_act + P - 1) / P;
  // greedy placement by one wave of lanes: lane l holds waves l, l + 64, ...
  if (tid < kWave) {
    constexpr int kPer = kPlanMaxWaves / kWave;
    long long load[kPer];
    int size[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      load[j] = 0;
      size[j] = 0;
    }
    const bool fits = n_waves <= max_waves;
    for (int r = 0; fits && r < n_act; ++r) {
      const int e = s_sorted[r];
      const int c = s_cnt[e];
      long long best = 0x7fffffffffffffffLL;
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int w = tid + j * kWave;
        if (w < n_waves && size[j] < P) {
          const long long key = load[j] * kPlanMaxWaves + w;
          best = key < best ? key : best;
        }
      }
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) {
        const long long o = __shfl_xor(best, off, kWave);
        best = o < best ? o : best;
      }
      const int w = static_cast<int>(best % kPlanMaxWaves);  // some wave has room
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        if (tid + j * kWave == w) {
          load[j] += c;
          size[j] += 1;
        }
      }
      if (tid == 0) s_wave[e] = w;
    }
  }
  __syncthreads();
  // members ascending within each wave
  for (int e = tid; e < n_routed; e += kPlanThreads) {
    const int w = s_wave[e];
    int pos = -1;
    if (w >= 0) {
      pos = 0;
      for (int f = 0; f < e; ++f) pos += s_wave[f] == w ? 1 : 0;
      v.members[static_cast<long long>(w) * P + pos] = e;
      atomicAdd(&s_size[w], 1);
    }
    v.counts[e] = s_cnt[e];
    v.wave_of[e] = w;
    v.slot_of[e] = pos;
  }
  __syncthreads();
  for (int w = tid; w < max_waves; w += kPlanThreads) {
    v.size[w] = s_size[w];
    for (int i = s_size[w]; i < P; ++i) v.members[static_cast<long long>(w) * P + i] = -1;
  }
  if (tid == 0) {
    v.hdr[0] = n_waves <= max_waves ? n_waves : -1;
    v.hdr[1] = n_act;
    v.hdr[2] = s_invalid;
    v.hdr[3] = 0;
  }
}

constexpr int kStageGrid = 128;        // workgroups (every XCD gets 16)
constexpr int kStageThreads = 256;
constexpr int kStageUnroll = 8;
constexpr long long kStageItem16 = 16384;  // 16-byte words per work item (256 KiB)

struct StageArgs {
  const int32_t* plan;
  int n_routed, P, max_waves, wave;
  const int32_t* main_table;  // expert -> main slot (entries of evicted experts may be stale)
  const int32_t* main_owner;  // main slot -> owning expert, -1 none
  int main_slots;
  const uint4* main13;
  const uint4* main2;
  const uint4* host13;
  const uint4* host2;
  uint4* stage13;
  uint4* stage2;
  long long n16_13, n16_2;  // 16-byte words per expert
  int32_t* table;
  int n_table, n_pinned, pinned_slot0;
};

__global__ __launch_bounds__(kStageThreads) void wave_stage_kernel(StageArgs a) {
  PlanView v = plan_view(const_cast<int32_t*>(a.plan), a.n_routed, a.max_waves);
  const int n_waves = v.hdr[0];
  const bool live = a.wave < n_waves;
  const int n = live ? v.size[a.wave] : 0;
  const long long it13 = (a.n16_13 + kStageItem16 - 1) / kStageItem16;
  const long long it2 = (a.n16_2 + kStageItem16 - 1) / kStageItem16;
  const long long per = it13 + it2;
  const long long total = static_cast<long long>(n) * per;
  const int32_t* mem = v.members + static_cast<long long>(a.wave) * a.P;
  for (long long c = blockIdx.x; c < total; c += gridDim.x) {
    const int i = static_cast<int>(c / per);
    const long long r = c % per;
    const int e = mem[i];
    const int s = a.main_table[e];
    const bool hit = s >= 0 && s < a.main_slots && a.main_owner[s] == e;
    const bool first = r < it13;
    const long long n16 = first ? a.n16_13 : a.n16_2;
    const long long beg = (first ? r : r - it13) * kStageItem16;
    const long long end = min(beg + kStageItem16, n16);
    const uint4* __restrict__ src =
        first ? (hit ? a.main13 + s * n16 : a.host13 + e * n16)
              : (hit ? a.main2 + s * n16 : a.host2 + e * n16);
    uint4* __restrict__ dst = (first ? a.stage13 : a.stage2) + static_cast<long long>(i) * n16;
    for (long long j = beg + threadIdx.x; j < end; j += kStageUnroll * kStageThreads) {
      uint4 t[kStageUnroll];
#pragma unroll
      for (int u = 0; u < kStageUnroll; ++u) {
        const long long q = j + u * kStageThreads;
        t[u] = q < end ? src[q] : make_uint4(0u, 0u, 0u, 0u);
      }
#pragma unroll
      for (int u = 0; u < kStageUnroll; ++u) {
        const long long q = j + u * kStageThreads;
        if (q < end) dst[q] = t[u];
      }
    }
  }
  // the stage table: members -> their stage slots, the pinned suffix with
  // the first wave only, -1 elsewhere (consumers wait for the whole launch)
  if (blockIdx.x == 0) {
    for (int e = threadIdx.x; e < a.n_table; e += kStageThreads) {
      int val = -1;
      if (e < a.n_routed) {
        if (live && v.wave_of[e] == a.wave) val = v.slot_of[e];
      } else if (e < a.n_routed + a.n_pinned) {
        if (a.wave == 0) val = a.pinned_slot0 + (e - a.n_routed);
      }
      a.table[e] = val;
    }
  }
}

}  // namespace

extern "C" long long lmoe_wave_plan_bytes(int n_routed, int n_slots, int max_waves) {
  if (n_routed <= 0 || n_routed > kPlanMaxExperts || n_slots <= 0 || n_slots > kPlanMaxSlots ||
      max_waves <= 0 || max_waves > kPlanMaxWaves)
    return -1;
  return plan_words(n_routed, n_slots, max_waves) * 4;
}

extern "C" int lmoe_wave_plan(const int32_t* ids, int n_pairs, int n_routed, int n_total, int n_slots,
                              int max_waves, int32_t* plan, hipStream_t stream) {
  // an empty batch (n_pairs 0, ids may be null) plans zero waves
  if ((n_pairs > 0 && ids == nullptr) || plan == nullptr || n_pairs < 0) return LMOE_ERR_ARG;
  if (lmoe_wave_plan_bytes(n_routed, n_slots, max_waves) < 0 || n_total < n_routed)
    return LMOE_ERR_SHAPE;
  hipLaunchKernelGGL(wave_plan_kernel, dim3(1), dim3(kPlanThreads), 0, stream, ids, n_pairs,
                     n_routed, n_total, n_slots, max_waves, plan);
  LMOE_RETURN_LAUNCH();
}

extern "C" int lmoe_wave_stage(const int32_t* plan, int n_routed, int n_slots, int max_waves,
                               int wave, const int32_t* main_table, const int32_t* main_owner,
                               const void* main_w13,
                               const void* main_w2, int main_slots, const void* host_w13,
                               const void* host_w2, void* stage_w13, void* stage_w2,
                               long long w13_expert_bytes, long long w2_expert_bytes,
                               int32_t* stage_table, int n_table, int n_pinned,
                               int pinned_slot0, hipStream_t stream) {
  if (plan == nullptr || main_table == nullptr || main_owner == nullptr || main_w13 == nullptr ||
      main_w2 == nullptr ||
      host_w13 == nullptr || host_w2 == nullptr || stage_w13 == nullptr || stage_w2 == nullptr ||
      stage_table == nullptr)
    return LMOE_ERR_ARG;
  if (lmoe_wave_plan_bytes(n_routed, n_slots, max_waves) < 0 || wave < 0 || wave >= max_waves ||
      main_slots <= 0 || n_pinned < 0 || pinned_slot0 < n_slots || n_table < n_routed + n_pinned)
    return LMOE_ERR_SHAPE;
  if (w13_expert_bytes <= 0 || w2_expert_bytes <= 0 || ((w13_expert_bytes | w2_expert_bytes) & 15))
    return LMOE_ERR_SHAPE;
  const uintptr_t al = reinterpret_cast<uintptr_t>(main_w13) | reinterpret_cast<uintptr_t>(main_w2) |
                       reinterpret_cast<uintptr_t>(host_w13) | reinterpret_cast<uintptr_t>(host_w2) |
                       reinterpret_cast<uintptr_t>(stage_w13) | reinterpret_cast<uintptr_t>(stage_w2);
  if (al & 15u) return LMOE_ERR_SHAPE;
  StageArgs a{};
  a.plan = plan;
  a.n_routed = n_routed;
  a.P = n_slots;
  a.max_waves = max_waves;
  a.wave = wave;
  a.main_table = main_table;
  a.main_owner = main_owner;
  a.main_slots = main_slots;
  a.main13 = static_cast<const uint4*>(main_w13);
  a.main2 = static_cast<const uint4*>(main_w2);
  a.host13 = static_cast<const uint4*>(host_w13);
  a.host2 = static_cast<const uint4*>(host_w2);
  a.stage13 = static_cast<uint4*>(stage_w13);
  a.stage2 = static_cast<uint4*>(stage_w2);
  a.n16_13 = w13_expert_bytes / 16;
  a.n16_2 = w2_expert_bytes / 16;
  a.table = stage_table;
  a.n_table = n_table;
  a.n_pinned = n_pinned;
  a.pinned_slot0 = pinned_slot0;
  hipLaunchKernelGGL(wave_stage_kernel, dim3(kStageGrid), dim3(kStageThreads), 0, stream, a);
  LMOE_RETURN_LAUNCH();
}
