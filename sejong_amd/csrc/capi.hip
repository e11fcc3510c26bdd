// Status strings, last-error message and device identification.
// Error text follows the reference's Error::Message / Error::Capacity /
// "HIP {code}: {str}" forms (crates/sejong-core/src/lib.rs:8-24,
// crates/sejong-gpu/src/hip.rs:47-57).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "common.h"

static thread_local char g_last_error[1024] = "";

namespace sjh {
ProfHook& prof_hook() {
  static thread_local ProfHook h;
  return h;
}
GradSq& grad_sq() {
  static thread_local GradSq g;
  return g;
}
int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}
int hip_check(hipError_t e, const char* what) {
  return fail(SJ_ERR_HIP, "%s: HIP %d: %s", what, (int)e, hipGetErrorString(e));
}
}  // namespace sjh

extern "C" const char* sj_status_string(int status) {
  switch (status) {
    case SJ_OK: return "ok";
    case SJ_ERR_INVALID: return "invalid argument or shape";
    case SJ_ERR_CAPACITY: return "capacity exceeded";
    case SJ_ERR_HIP: return "HIP runtime error";
    case SJ_ERR_UNSUPPORTED: return "unsupported dtype or layout";
    case SJ_ERR_NONFINITE: return "nonfinite clipping gradient";
    case SJ_ERR_IO: return "file read or write error";
    default: return "unknown status";
  }
}

extern "C" const char* sj_last_error(void) { return g_last_error; }

extern "C" int sj_device_info(char* arch, size_t arch_len, int* compute_units) {
  int dev = 0;
  SJ_HIP(hipGetDevice(&dev));
  hipDeviceProp_t prop;
  SJ_HIP(hipGetDeviceProperties(&prop, dev));
  if (arch && arch_len) {
    strncpy(arch, prop.gcnArchName, arch_len - 1);
    arch[arch_len - 1] = 0;
  }
  if (compute_units) *compute_units = prop.multiProcessorCount;
  return SJ_OK;
}

// ------------------------------------------------ device memory and events
// Host utilities mirroring the reference Engine's empty / from_* / to_*
// transfers (crates/sejong-gpu/src/lib.rs:234-365) for callers that do not
// bring their own HIP allocator (the test harness and bench.py).

extern "C" int sj_alloc(size_t bytes, void** ptr) {
  SJ_REQUIRE(ptr, "alloc: null");
  hipError_t e = hipMalloc(ptr, bytes ? bytes : 256);
  if (e != hipSuccess) {
    size_t fr = 0, tot = 0;
    hipMemGetInfo(&fr, &tot);
    return sjh::fail(SJ_ERR_CAPACITY, "allocation: required %zu bytes, available %zu bytes", bytes, fr);
  }
  return SJ_OK;
}

extern "C" int sj_free(void* ptr) {
  if (ptr) SJ_HIP(hipFree(ptr));
  return SJ_OK;
}

extern "C" int sj_memory_info(size_t* free_bytes, size_t* total_bytes) {
  SJ_REQUIRE(free_bytes && total_bytes, "memory info: null");
  SJ_HIP(hipMemGetInfo(free_bytes, total_bytes));
  return SJ_OK;
}

extern "C" int sj_upload(void* dst, const void* src, size_t bytes) {
  SJ_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return SJ_OK;
}

extern "C" int sj_download(void* dst, const void* src, size_t bytes) {
  SJ_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return SJ_OK;
}

extern "C" int sj_synchronize(void* stream) {
  if (stream)
    SJ_HIP(hipStreamSynchronize((hipStream_t)stream));
  else
    SJ_HIP(hipDeviceSynchronize());
  return SJ_OK;
}

extern "C" int sj_event_create(void** ev) {
  SJ_REQUIRE(ev, "event: null");
  hipEvent_t e;
  SJ_HIP(hipEventCreate(&e));
  *ev = (void*)e;
  return SJ_OK;
}

extern "C" int sj_event_destroy(void* ev) {
  if (ev) SJ_HIP(hipEventDestroy((hipEvent_t)ev));
  return SJ_OK;
}

extern "C" int sj_event_record(void* ev, void* stream) {
  SJ_HIP(hipEventRecord((hipEvent_t)ev, (hipStream_t)stream));
  return SJ_OK;
}

extern "C" int sj_event_elapsed(void* start, void* end, float* ms) {
  SJ_REQUIRE(ms, "event_elapsed: null");
  SJ_HIP(hipEventSynchronize((hipEvent_t)end));
  SJ_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end));
  return SJ_OK;
}
