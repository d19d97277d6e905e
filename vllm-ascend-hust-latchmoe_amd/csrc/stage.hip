// Host-side entry points: batched expert staging copies on a transfer stream,
// the slot-table update that publishes them, status strings and the ABI
// version.
//
// Reference behaviour: TransferEngine.load_many_async
// (moe_offload/transfer_engine.py:139-187): the transfer stream first waits
// for the slot's release event, every copy of the batch is queued on it, and
// one event recorded after the batch orders the copies before their consumer
// (TransferReadyEvent.install_consumer_dependency, :38-47).  The persistent
// log2phy entries that change are written after the copies
// (_update_log2phy_entries, moe_offload/runtime.py:3068-3101).
#include "lmoe_device.h"

namespace {

constexpr int kTableUpdateBatch = 64;  // pairs per launch (kernel argument bytes: 516)

struct TableUpdate {
  int n;
  int idx[kTableUpdateBatch];
  int val[kTableUpdateBatch];
};

// table[u.idx[i]] = u.val[i] for i < u.n; the pairs travel as kernel
// arguments, so no staging buffer or copy precedes the launch
__global__ __launch_bounds__(64) void table_update_kernel(int32_t* __restrict__ table,
                                                          TableUpdate u) {
  const int i = threadIdx.x;
  if (i < u.n) table[u.idx[i]] = u.val[i];
}

// ---------------------------------------------------------------------------
// Gather copy: one launch moves a batch of expert copies (page-locked host
// memory or device memory -> device memory) with 16-byte vector loads and
// stores, and writes the slot-table entries that publish them.  The batch is
// cut into 256 KiB work items, dealt round-robin to kGatherGrid workgroups;
// each lane keeps eight 16-byte loads in flight.  Measured on the MI355X
// host link: 52-56 GB/s (a single large hipMemcpyAsync reaches the same),
// with no per-copy command overhead, from 16 workgroups as from 128; the
// smaller grid leaves the CUs to the compute kernels the copies overlap (the
// B=1 decode step with prefetched misses: 7.5 ms against 8.0 ms).
// Everything rides in the kernel arguments: no descriptor buffer, no copy
// precedes the launch.
// ---------------------------------------------------------------------------
constexpr int kGatherMax = 32;        // copies per launch
constexpr int kGatherTab = 128;       // slot-table pairs per launch
constexpr int kGatherGrid = 16;       // workgroups (a multiple of 8: every XCD gets 2)
constexpr long long kGatherItem16 = 16384;  // 16-byte words per work item (256 KiB)
constexpr int kGatherThreads = 256;
constexpr int kGatherUnroll = 8;

struct GatherArgs {
  int n;                               // copies
  int n_tab;                           // table pairs
  int fill;                            // 1: entries not among the pairs become -1
  int n_table;                         // table length (fill)
  int32_t* table;                      // may be null
  long long item_end[kGatherMax];      // inclusive prefix of the copies' work items
  const uint4* src[kGatherMax];
  uint4* dst[kGatherMax];
  long long n16[kGatherMax];
  int32_t tidx[kGatherTab];
  int32_t tval[kGatherTab];
};

__global__ __launch_bounds__(kGatherThreads) void stage_gather_kernel(GatherArgs a) {
  const long long total = a.n > 0 ? a.item_end[a.n - 1] : 0;
  for (long long c = blockIdx.x; c < total; c += gridDim.x) {
    int i = 0;
    while (c >= a.item_end[i]) ++i;  // uniform; c < total keeps i < n
    const long long beg = (c - (i == 0 ? 0 : a.item_end[i - 1])) * kGatherItem16;
    const long long end = min(beg + kGatherItem16, a.n16[i]);
    const uint4* __restrict__ s = a.src[i];
    uint4* __restrict__ d = a.dst[i];
    for (long long j = beg + threadIdx.x; j < end; j += kGatherUnroll * kGatherThreads) {
      uint4 v[kGatherUnroll];
#pragma unroll
      for (int u = 0; u < kGatherUnroll; ++u) {
        const long long q = j + u * kGatherThreads;
        v[u] = q < end ? s[q] : make_uint4(0u, 0u, 0u, 0u);
      }
#pragma unroll
      for (int u = 0; u < kGatherUnroll; ++u) {
        const long long q = j + u * kGatherThreads;
        if (q < end) d[q] = v[u];
      }
    }
  }
  // the table publishes the copied slots; its consumers wait for the whole
  // launch (the batch's ready event), so the order against the copies
  // inside the launch does not matter
  if (blockIdx.x == 0 && a.table != nullptr) {
    if (a.fill) {
      for (int e = threadIdx.x; e < a.n_table; e += kGatherThreads) {
        int v = -1;
        for (int p = 0; p < a.n_tab; ++p) v = a.tidx[p] == e ? a.tval[p] : v;
        a.table[e] = v;
      }
    } else {
      for (int p = threadIdx.x; p < a.n_tab; p += kGatherThreads) a.table[a.tidx[p]] = a.tval[p];
    }
  }
}

// True when [p, p + bytes) lies inside one allocation the HIP runtime knows
// (device memory, or page-locked host memory mapped for the device); *dev
// is the address the device uses for p.
bool gpu_accessible_range(const void* p, size_t bytes, const void** dev) {
  hipPointerAttribute_t at;
  if (hipPointerGetAttributes(&at, p) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  const void* dp = nullptr;
  if (at.type == hipMemoryTypeDevice) dp = p;
  else if (at.type == hipMemoryTypeHost && at.devicePointer != nullptr) dp = at.devicePointer;
  else return false;
  void* base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, const_cast<void*>(dp)) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  const uintptr_t b = reinterpret_cast<uintptr_t>(base);
  const uintptr_t q = reinterpret_cast<uintptr_t>(dp);
  if (q < b || q - b > size || bytes > size - (q - b)) return false;
  *dev = dp;
  return true;
}

}  // namespace

extern "C" int lmoe_abi_version(void) { return LMOE_ABI_VERSION; }

namespace lmoe {
void* flags_address_mlp();
void* flags_address_router_softmax();
void* flags_address_router_sigmoid();
}  // namespace lmoe

extern "C" int lmoe_device_flags(int32_t* flags, int clear, hipStream_t stream) {
  if (flags == nullptr) return LMOE_ERR_ARG;
  // the units whose kernels add to their status words
  static void* (*const units[])() = {lmoe::flags_address_mlp, lmoe::flags_address_router_softmax,
                                     lmoe::flags_address_router_sigmoid};
  constexpr int kUnits = sizeof(units) / sizeof(units[0]);
  static const int32_t zeros[LMOE_FLAG_COUNT] = {0};
  for (int f = 0; f < LMOE_FLAG_COUNT; ++f) flags[f] = 0;
  for (int u = 0; u < kUnits; ++u) {
    void* p = units[u]();
    if (p == nullptr) return LMOE_ERR_ARG;
    int32_t w[LMOE_FLAG_COUNT];
    hipError_t e = hipMemcpyAsync(w, p, sizeof(w), hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return static_cast<int>(e);
    bool any = false;
    for (int f = 0; f < LMOE_FLAG_COUNT; ++f) {
      flags[f] += w[f];
      any = any || w[f] != 0;
    }
    if (clear && any) {
      e = hipMemcpyAsync(p, zeros, sizeof(zeros), hipMemcpyHostToDevice, stream);
      if (e == hipSuccess) e = hipStreamSynchronize(stream);
      if (e != hipSuccess) return static_cast<int>(e);
    }
  }
  return LMOE_OK;
}

extern "C" const char* lmoe_status_string(int status) {
  switch (status) {
    case LMOE_OK: return "ok";
    case LMOE_ERR_ARG: return "invalid argument (null pointer or negative size)";
    case LMOE_ERR_SHAPE: return "unsupported shape";
    case LMOE_ERR_WORKSPACE: return "workspace too small";
    case LMOE_ERR_UNSUPPORTED: return "unsupported option combination";
    default: break;
  }
  if (status > 0 && status < 1000)
    return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}

extern "C" int lmoe_stage_copy(void* const* dst, const void* const* src,
                               const size_t* bytes, int n,
                               hipStream_t transfer_stream,
                               hipEvent_t wait_event, hipEvent_t done_event) {
  if (n < 0 || (n > 0 && (dst == nullptr || src == nullptr || bytes == nullptr)))
    return LMOE_ERR_ARG;
  for (int i = 0; i < n; ++i)
    if (bytes[i] > 0 && (dst[i] == nullptr || src[i] == nullptr)) return LMOE_ERR_ARG;
  hipError_t e = hipSuccess;
  if (wait_event != nullptr) {
    e = hipStreamWaitEvent(transfer_stream, wait_event, 0);
    if (e != hipSuccess) return static_cast<int>(e);
  }
  for (int i = 0; i < n; ++i) {
    if (bytes[i] == 0) continue;
    e = hipMemcpyAsync(dst[i], src[i], bytes[i], hipMemcpyDefault, transfer_stream);
    if (e != hipSuccess) return static_cast<int>(e);
  }
  if (done_event != nullptr) {
    e = hipEventRecord(done_event, transfer_stream);
    if (e != hipSuccess) return static_cast<int>(e);
  }
  return LMOE_OK;
}

extern "C" int lmoe_table_update(int32_t* table, int n_table, const int32_t* idx,
                                 const int32_t* val, int n, hipStream_t stream) {
  if (n < 0 || n_table < 0 || (n > 0 && (table == nullptr || idx == nullptr || val == nullptr)))
    return LMOE_ERR_ARG;
  for (int i = 0; i < n; ++i) {
    if (idx[i] < 0 || idx[i] >= n_table) return LMOE_ERR_ARG;
    for (int j = 0; j < i; ++j)
      if (idx[j] == idx[i]) return LMOE_ERR_ARG;  // the writes of one launch are unordered
  }
  for (int i0 = 0; i0 < n; i0 += kTableUpdateBatch) {
    TableUpdate u;
    u.n = n - i0 < kTableUpdateBatch ? n - i0 : kTableUpdateBatch;
    for (int i = 0; i < u.n; ++i) {
      u.idx[i] = idx[i0 + i];
      u.val[i] = val[i0 + i];
    }
    hipLaunchKernelGGL(table_update_kernel, dim3(1), dim3(kTableUpdateBatch), 0, stream, table, u);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return static_cast<int>(e);
  }
  return LMOE_OK;
}

extern "C" int lmoe_stage_gather(void* const* dst, const void* const* src, const size_t* bytes,
                                 int n, int32_t* table, int n_table, const int32_t* idx,
                                 const int32_t* val, int n_tab, int fill,
                                 hipStream_t transfer_stream, hipEvent_t wait_event,
                                 hipEvent_t done_event) {
  if (n < 0 || n_tab < 0 || n_table < 0) return LMOE_ERR_ARG;
  if (n > 0 && (dst == nullptr || src == nullptr || bytes == nullptr)) return LMOE_ERR_ARG;
  if ((n_tab > 0 || fill) && (table == nullptr || n_table <= 0)) return LMOE_ERR_ARG;
  if (n_tab > 0 && (idx == nullptr || val == nullptr)) return LMOE_ERR_ARG;
  if (fill && n_tab > kGatherTab) return LMOE_ERR_SHAPE;  // a filled table is one launch
  for (int i = 0; i < n_tab; ++i) {
    if (idx[i] < 0 || idx[i] >= n_table) return LMOE_ERR_ARG;
    for (int j = 0; j < i; ++j)
      if (idx[j] == idx[i]) return LMOE_ERR_ARG;  // the writes of one launch are unordered
  }
  // every range is checked before anything is queued: a source the device
  // cannot read at the same address (pageable memory), or a range that
  // leaves its allocation, is refused, and the caller takes lmoe_stage_copy
  for (int i = 0; i < n; ++i) {
    if (bytes[i] == 0) continue;
    if (dst[i] == nullptr || src[i] == nullptr) return LMOE_ERR_ARG;
    if ((bytes[i] & 15u) ||
        ((reinterpret_cast<uintptr_t>(dst[i]) | reinterpret_cast<uintptr_t>(src[i])) & 15u))
      return LMOE_ERR_SHAPE;
    const void* sp = nullptr;
    const void* dp = nullptr;
    if (!gpu_accessible_range(src[i], bytes[i], &sp) || sp != src[i]) return LMOE_ERR_ARG;
    if (!gpu_accessible_range(dst[i], bytes[i], &dp) || dp != dst[i]) return LMOE_ERR_ARG;
  }
  hipError_t e = hipSuccess;
  if (wait_event != nullptr) {
    e = hipStreamWaitEvent(transfer_stream, wait_event, 0);
    if (e != hipSuccess) return static_cast<int>(e);
  }
  int i0 = 0, t0 = 0;
  do {
    GatherArgs a{};
    long long items = 0;
    a.n = 0;
    for (; i0 < n && a.n < kGatherMax; ++i0) {
      if (bytes[i0] == 0) continue;
      a.src[a.n] = static_cast<const uint4*>(src[i0]);
      a.dst[a.n] = static_cast<uint4*>(dst[i0]);
      a.n16[a.n] = static_cast<long long>(bytes[i0] / 16);
      items += (a.n16[a.n] + kGatherItem16 - 1) / kGatherItem16;
      a.item_end[a.n] = items;
      ++a.n;
    }
    const bool last = i0 >= n;
    if (last && table != nullptr && (n_tab > 0 || fill)) {
      // the table rides with the last launch (pairs past kGatherTab: extra
      // launches below)
      a.table = table;
      a.n_table = n_table;
      a.fill = fill;
      a.n_tab = n_tab - t0 < kGatherTab ? n_tab - t0 : kGatherTab;
      for (int p = 0; p < a.n_tab; ++p) {
        a.tidx[p] = idx[t0 + p];
        a.tval[p] = val[t0 + p];
      }
      t0 += a.n_tab;
    }
    if (a.n > 0 || a.table != nullptr) {
      const int grid = items > kGatherGrid ? kGatherGrid : (items > 0 ? static_cast<int>(items) : 1);
      hipLaunchKernelGGL(stage_gather_kernel, dim3(grid), dim3(kGatherThreads), 0, transfer_stream,
                         a);
      e = hipGetLastError();
      if (e != hipSuccess) return static_cast<int>(e);
    }
  } while (i0 < n);
  while (t0 < n_tab) {  // remaining table pairs (no fill), after every copy
    GatherArgs a{};
    a.table = table;
    a.n_table = n_table;
    a.n_tab = n_tab - t0 < kGatherTab ? n_tab - t0 : kGatherTab;
    for (int p = 0; p < a.n_tab; ++p) {
      a.tidx[p] = idx[t0 + p];
      a.tval[p] = val[t0 + p];
    }
    t0 += a.n_tab;
    hipLaunchKernelGGL(stage_gather_kernel, dim3(1), dim3(kGatherThreads), 0, transfer_stream, a);
    e = hipGetLastError();
    if (e != hipSuccess) return static_cast<int>(e);
  }
  if (done_event != nullptr) {
    e = hipEventRecord(done_event, transfer_stream);
    if (e != hipSuccess) return static_cast<int>(e);
  }
  return LMOE_OK;
}
