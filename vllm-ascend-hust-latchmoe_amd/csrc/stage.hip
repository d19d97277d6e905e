// Host-side entry points: batched expert staging copies on a transfer stream,
// status strings and the ABI version.
//
// Reference behaviour: TransferEngine.load_many_async
// (moe_offload/transfer_engine.py:139-187): the transfer stream first waits
// for the slot's release event, every copy of the batch is queued on it, and
// one event recorded after the batch orders the copies before their consumer
// (TransferReadyEvent.install_consumer_dependency, :38-47).
#include "lmoe_device.h"

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
