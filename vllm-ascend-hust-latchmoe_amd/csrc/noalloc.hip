// lmoe_fused_moe_decode_noalloc: the decode layer body with its act / y
// workspaces in a library-owned device array instead of caller memory, for
// callers that cannot allocate (code under graph capture, serving loops
// that forbid allocation).  It allocates nothing: the array is a
// file-scope __device__ object that every GPU the library runs on holds for
// the life of the process.
//
// In host code `scratch` names a host-side stand-in, not a device address.
// Its device address is looked up once per device, with that device
// current, by hipGetSymbolAddress, and only that address is ever handed to
// kernels.  Every call on one GPU shares that GPU's array: calls that may
// overlap on one GPU (two streams, two threads) race and must be ordered by
// the caller.  The array is never cleared: the decode kernels write every
// act / y row they read in the same call.
#include <hip/hip_runtime.h>

#include <mutex>

#include "latchmoe.h"

namespace {

constexpr size_t kScratchBytes = static_cast<size_t>(LMOE_NOALLOC_SCRATCH_BYTES);
constexpr int kMaxDevices = 64;
constexpr int kDecodeMaxPairs = 1024;  // lmoe_fused_moe_decode: T * k <= 1024

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of this device's scratch array (looked up on the first
// call on the device).  Returns a hipError_t status (0 on success).
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return LMOE_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return static_cast<int>(e);
    if (p == nullptr) return static_cast<int>(hipErrorInvalidSymbol);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return LMOE_OK;
}

size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

}  // namespace

extern "C" int lmoe_fused_moe_decode_noalloc(const void* x, int T, int H, int I, int k,
                                             const void* w13_slots, const void* w2_slots,
                                             int n_slots, const uint16_t* w,
                                             const int32_t* offsets, const int32_t* sorted_pairs,
                                             const int32_t* row_idx, const int32_t* active,
                                             const int32_t* meta, const void* add, void* out,
                                             int distinct_slots, hipStream_t stream) {
  if (T < 0 || H <= 0 || I <= 0 || k <= 0) return LMOE_ERR_ARG;
  const size_t n_pairs = static_cast<size_t>(T) * static_cast<size_t>(k);
  // the decode body's own pair limit, checked here too so that no call past
  // it reaches the array-size check below with a misleading status
  if (n_pairs > static_cast<size_t>(kDecodeMaxPairs)) return LMOE_ERR_SHAPE;
  const size_t act_bytes = align256(n_pairs * static_cast<size_t>(I) * 2);
  const size_t y_bytes = align256(n_pairs * static_cast<size_t>(H) * 2);
  if (act_bytes + y_bytes > kScratchBytes) return LMOE_ERR_WORKSPACE;
  if (T == 0) return LMOE_OK;
  void* base = nullptr;
  const int st = scratch_address(&base);
  if (st != LMOE_OK) return st;
  char* act = static_cast<char*>(base);
  char* y = act + act_bytes;
  return lmoe_fused_moe_decode(x, T, H, I, k, w13_slots, w2_slots, n_slots, w, offsets,
                               sorted_pairs, row_idx, active, meta, add, act, y, out,
                               distinct_slots, stream);
}
