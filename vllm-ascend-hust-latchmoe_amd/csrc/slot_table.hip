// Host-side slot planner of the decode staging: hit / miss and slot
// reservation over a slot table kept as arrays (one entry per slot: state,
// owning expert, version, last use) plus the expert -> slot residency array.
// The Python slot bank owns these arrays (numpy) and hands them over by
// pointer; nothing here touches the device.
//
// Reference behaviour: the staging loop of
// MoeOffloadRuntime.prepare_fixed_slot_plan_into_log2phy
// (moe_offload/runtime.py:1636-1936) with the allocation policy of
// ExpertSlotBank.allocate_for (moe_offload/slot_bank.py:211-336): a READY
// resident expert is a hit; otherwise the lowest-id EMPTY slot, else the
// READY slot with the smallest (last use, slot id); LOADING and COMPUTING
// slots are never taken.
#include <stdint.h>

#include "latchmoe.h"

namespace {

// slot state codes (COMPUTING = 3 is never taken, like LOADING)
constexpr int8_t kEmpty = 0;
constexpr int8_t kLoading = 1;
constexpr int8_t kReady = 2;

// The slot to reserve, or -1 when every slot is LOADING or COMPUTING.
int pick_slot(const int8_t* state, const int64_t* last_used, int n_slots) {
  int best = -1;
  for (int s = 0; s < n_slots; ++s) {
    if (state[s] == kEmpty) return s;
    if (state[s] == kReady && (best < 0 || last_used[s] < last_used[best])) best = s;
  }
  return best;
}

}  // namespace

extern "C" int lmoe_slot_plan(int8_t* state, int32_t* owner, int64_t* version, int64_t* last_used,
                              int n_slots, int32_t* slot_of, int n_experts, const int32_t* active,
                              int n_active, int64_t step, int32_t* slot_ids, int8_t* miss) {
  if (n_slots <= 0 || n_experts <= 0 || n_active < 0) return LMOE_ERR_ARG;
  if (state == nullptr || owner == nullptr || version == nullptr || last_used == nullptr ||
      slot_of == nullptr || (n_active > 0 && (active == nullptr || slot_ids == nullptr || miss == nullptr)))
    return LMOE_ERR_ARG;
  for (int j = 0; j < n_active; ++j)
    if (active[j] < 0 || active[j] >= n_experts) return LMOE_ERR_ARG;
  int misses = 0;
  for (int j = 0; j < n_active; ++j) {
    const int e = active[j];
    int s = slot_of[e];
    if (s >= 0 && s < n_slots && owner[s] == e) {
      if (state[s] != kReady) return -(j + 1);  // its copy or its compute is in flight
      last_used[s] = step;
      slot_ids[j] = s;
      miss[j] = 0;
      continue;
    }
    s = pick_slot(state, last_used, n_slots);
    if (s < 0) return -(j + 1);  // wait for in-flight work to free a slot
    const int prev = owner[s];
    if (prev >= 0 && prev < n_experts && slot_of[prev] == s) slot_of[prev] = -1;
    owner[s] = e;
    slot_of[e] = s;
    state[s] = kLoading;
    version[s] += 1;
    last_used[s] = step;
    slot_ids[j] = s;
    miss[j] = 1;
    ++misses;
  }
  return misses;
}
