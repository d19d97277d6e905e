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

}  // namespace

extern "C" int lmoe_abi_version(void) { return LMOE_ABI_VERSION; }

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
