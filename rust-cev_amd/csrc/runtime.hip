// Runtime helpers of the C ABI for hosts with no HIP binding of their own
// (the Rust host: candle has no HIP device, so the FFI crate holds device
// buffers as raw pointers and uses these to move them).
#include <hip/hip_runtime.h>
#include <string.h>

#include "cev_internal.h"

namespace {
int32_t hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return CEV_OK;
  return cev_fail(CEV_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}
}  // namespace

extern "C" int32_t cev_device_info(int32_t device, char* name, size_t name_len, int32_t* n_cus, int64_t* hbm_bytes, int32_t* clock_mhz) {
  hipDeviceProp_t p;
  int32_t rc = hip_status(hipGetDeviceProperties(&p, device), "hipGetDeviceProperties");
  if (rc) return rc;
  if (name && name_len) {
    strncpy(name, p.gcnArchName, name_len - 1);
    name[name_len - 1] = 0;
  }
  if (n_cus) *n_cus = p.multiProcessorCount;
  if (hbm_bytes) *hbm_bytes = (int64_t)p.totalGlobalMem;
  if (clock_mhz) *clock_mhz = p.clockRate / 1000;
  return CEV_OK;
}

extern "C" int32_t cev_malloc(void** ptr, size_t bytes) {
  CEV_CHECK_ARG(ptr != nullptr, "cev_malloc: null output");
  return hip_status(hipMalloc(ptr, bytes), "hipMalloc");
}

extern "C" int32_t cev_free(void* ptr) { return hip_status(hipFree(ptr), "hipFree"); }

extern "C" int32_t cev_memcpy_h2d(void* dst, const void* src, size_t bytes, cev_stream stream) {
  return hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream), "hipMemcpyAsync h2d");
}

extern "C" int32_t cev_memcpy_d2h(void* dst, const void* src, size_t bytes, cev_stream stream) {
  return hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream), "hipMemcpyAsync d2h");
}

extern "C" int32_t cev_memcpy_d2d(void* dst, const void* src, size_t bytes, cev_stream stream) {
  return hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream), "hipMemcpyAsync d2d");
}

extern "C" int32_t cev_stream_create(cev_stream* stream) {
  CEV_CHECK_ARG(stream != nullptr, "cev_stream_create: null output");
  hipStream_t s;
  int32_t rc = hip_status(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
  if (rc) return rc;
  *stream = (cev_stream)s;
  return CEV_OK;
}

extern "C" int32_t cev_stream_destroy(cev_stream stream) { return hip_status(hipStreamDestroy((hipStream_t)stream), "hipStreamDestroy"); }

extern "C" int32_t cev_stream_synchronize(cev_stream stream) {
  return hip_status(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
}

// Timing events: record two on a stream around the launches to time, wait
// for the second, then read the milliseconds between them.
extern "C" int32_t cev_event_create(cev_event* event) {
  CEV_CHECK_ARG(event != nullptr, "cev_event_create: null output");
  hipEvent_t e;
  int32_t rc = hip_status(hipEventCreate(&e), "hipEventCreate");
  if (rc) return rc;
  *event = (cev_event)e;
  return CEV_OK;
}

extern "C" int32_t cev_event_destroy(cev_event event) { return hip_status(hipEventDestroy((hipEvent_t)event), "hipEventDestroy"); }

extern "C" int32_t cev_event_record(cev_event event, cev_stream stream) {
  CEV_CHECK_ARG(event != nullptr, "cev_event_record: null event");
  return hip_status(hipEventRecord((hipEvent_t)event, (hipStream_t)stream), "hipEventRecord");
}

extern "C" int32_t cev_event_synchronize(cev_event event) {
  CEV_CHECK_ARG(event != nullptr, "cev_event_synchronize: null event");
  return hip_status(hipEventSynchronize((hipEvent_t)event), "hipEventSynchronize");
}

extern "C" int32_t cev_event_elapsed_ms(cev_event start, cev_event end, float* ms) {
  CEV_CHECK_ARG(start != nullptr && end != nullptr && ms != nullptr, "cev_event_elapsed_ms: null argument");
  return hip_status(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end), "hipEventElapsedTime");
}
