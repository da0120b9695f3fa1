// Backend shim: the HIP runtime calls that ROCmBackend makes through hip-python
// (offload_runtime/backends/rocm_backend.py:46-119), exported as a plain C ABI so the
// Python backend needs no hip-python.  Streams keep the default priority.
#include <string.h>

#include "mx_common.h"

extern "C" const char* mx_error_string(int status) {
  switch (status) {
    case MX_OK: return "ok";
    case MX_ERR_INVALID: return "invalid argument";
    case MX_ERR_UNSUPPORTED: return "unsupported configuration";
    case MX_ERR_WORKSPACE: return "workspace too small";
    case MX_ERR_ALIGNMENT: return "weight pointer not 16-byte aligned";
    default: break;
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "unknown error";
}

extern "C" int mx_get_device_count(int32_t* count) {
  if (!count) return MX_ERR_INVALID;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  *count = (e == hipSuccess) ? n : 0;
  return mx_status(e);
}

extern "C" int mx_device_info(int32_t device, MxDeviceInfo* info) {
  if (!info) return MX_ERR_INVALID;
  hipDeviceProp_t p;
  hipError_t e = hipGetDeviceProperties(&p, device);
  if (e != hipSuccess) return mx_status(e);
  memset(info, 0, sizeof(*info));
  strncpy(info->name, p.name, sizeof(info->name) - 1);
  strncpy(info->arch, p.gcnArchName, sizeof(info->arch) - 1);
  info->cu_count = p.multiProcessorCount;
  info->clock_khz = p.clockRate;
  info->mem_clock_khz = p.memoryClockRate;
  info->mem_bus_width = p.memoryBusWidth;
  info->total_mem = (int64_t)p.totalGlobalMem;
  info->l2_bytes = p.l2CacheSize;
  info->lds_per_block = (int32_t)p.sharedMemPerBlock;
  return MX_OK;
}

extern "C" int mx_set_device(int32_t device) { return mx_status(hipSetDevice(device)); }

extern "C" int mx_device_sync(void) { return mx_status(hipDeviceSynchronize()); }

extern "C" int mx_malloc(void** ptr, size_t nbytes) {
  if (!ptr) return MX_ERR_INVALID;
  *ptr = nullptr;
  return mx_status(hipMalloc(ptr, nbytes ? nbytes : 1));
}

extern "C" int mx_free(void* ptr) { return ptr ? mx_status(hipFree(ptr)) : MX_OK; }

extern "C" int mx_host_malloc(void** ptr, size_t nbytes) {
  if (!ptr) return MX_ERR_INVALID;
  *ptr = nullptr;
  return mx_status(hipHostMalloc(ptr, nbytes ? nbytes : 1, 0));
}

extern "C" int mx_host_free(void* ptr) { return ptr ? mx_status(hipHostFree(ptr)) : MX_OK; }

static int mx_copy(void* dst, const void* src, size_t n, hipMemcpyKind kind, void* stream) {
  if (n == 0) return MX_OK;
  if (!dst || !src) return MX_ERR_INVALID;
  return mx_status(hipMemcpyAsync(dst, src, n, kind, (hipStream_t)stream));
}

extern "C" int mx_memcpy_h2d_async(void* dst, const void* src, size_t nbytes, void* stream) {
  return mx_copy(dst, src, nbytes, hipMemcpyHostToDevice, stream);
}

extern "C" int mx_memcpy_d2h_async(void* dst, const void* src, size_t nbytes, void* stream) {
  return mx_copy(dst, src, nbytes, hipMemcpyDeviceToHost, stream);
}

extern "C" int mx_memcpy_d2d_async(void* dst, const void* src, size_t nbytes, void* stream) {
  return mx_copy(dst, src, nbytes, hipMemcpyDeviceToDevice, stream);
}

extern "C" int mx_stream_create(void** stream, int32_t nonblocking) {
  if (!stream) return MX_ERR_INVALID;
  hipStream_t s = nullptr;
  hipError_t e = hipStreamCreateWithFlags(&s, nonblocking ? hipStreamNonBlocking : hipStreamDefault);
  *stream = (void*)s;
  return mx_status(e);
}

extern "C" int mx_stream_destroy(void* stream) {
  return stream ? mx_status(hipStreamDestroy((hipStream_t)stream)) : MX_OK;
}

extern "C" int mx_stream_sync(void* stream) {
  return mx_status(hipStreamSynchronize((hipStream_t)stream));
}

extern "C" int mx_event_create(void** event, int32_t timing) {
  if (!event) return MX_ERR_INVALID;
  hipEvent_t ev = nullptr;
  hipError_t e = hipEventCreateWithFlags(&ev, timing ? hipEventDefault : hipEventDisableTiming);
  *event = (void*)ev;
  return mx_status(e);
}

extern "C" int mx_event_record(void* event, void* stream) {
  if (!event) return MX_ERR_INVALID;
  return mx_status(hipEventRecord((hipEvent_t)event, (hipStream_t)stream));
}

extern "C" int mx_event_wait(void* stream, void* event) {
  if (!event) return MX_ERR_INVALID;
  return mx_status(hipStreamWaitEvent((hipStream_t)stream, (hipEvent_t)event, 0));
}

extern "C" int mx_event_sync(void* event) {
  if (!event) return MX_ERR_INVALID;
  return mx_status(hipEventSynchronize((hipEvent_t)event));
}

extern "C" int mx_event_query(void* event, int32_t* done) {
  if (!event || !done) return MX_ERR_INVALID;
  hipError_t e = hipEventQuery((hipEvent_t)event);
  if (e == hipSuccess) { *done = 1; return MX_OK; }
  if (e == hipErrorNotReady) { *done = 0; return MX_OK; }
  return mx_status(e);
}

extern "C" int mx_event_destroy(void* event) {
  return event ? mx_status(hipEventDestroy((hipEvent_t)event)) : MX_OK;
}

extern "C" int mx_event_elapsed_ms(float* ms, void* start, void* end) {
  if (!ms || !start || !end) return MX_ERR_INVALID;
  return mx_status(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end));
}
