// Runtime part of the C-ABI: errors, device memory, the library stream, events.
//
// Mirrors the capability/error conventions of the reference extension
// (native/src/module.cpp:13-17 `with_cuda`, :221-227 `flash_sdpa_available`;
// errors surface as exceptions with the runtime's message, sdpa_cuda.cu:10-14):
// here every call returns a status and the message is read with nml_last_error().
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "common.hpp"
#include "nimbleml_hip.h"

namespace nml {

namespace {
thread_local char g_err[1024] = {0};
hipStream_t g_stream = nullptr;
bool g_stream_owned = false;
std::mutex g_init_mu;
}  // namespace

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

hipStream_t stream() { return g_stream; }

// A second library stream (default priority, like the first) for work the library forks
// off the library stream and joins back with events; created on first use.
namespace {
hipStream_t g_stream2 = nullptr;
}

hipStream_t stream2() {
  std::lock_guard<std::mutex> lock(g_init_mu);
  if (g_stream2 == nullptr && hipStreamCreateWithFlags(&g_stream2, hipStreamNonBlocking) != hipSuccess)
    g_stream2 = nullptr;
  return g_stream2;
}

bool is_stream2(hipStream_t s) { return s != nullptr && s == g_stream2; }

}  // namespace nml

using nml::set_error;

extern "C" {

const char* nml_last_error(void) { return nml::g_err; }

int nml_with_hip(void) { return 1; }

int nml_hip_available(int* device_count) {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) n = 0;
  if (device_count) *device_count = n;
  return 0;
}

int nml_init(int device) {
  std::lock_guard<std::mutex> lock(nml::g_init_mu);
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
    set_error("no HIP device is visible (hipGetDeviceCount found none)");
    return -1;
  }
  NML_REQUIRE(device >= 0 && device < n, "device %d out of range (found %d)", device, n);
  NML_HIP(hipSetDevice(device));
  if (nml::g_stream == nullptr) {
    // Default priority on purpose: streams of different priorities are not used.
    NML_HIP(hipStreamCreateWithFlags(&nml::g_stream, hipStreamNonBlocking));
    nml::g_stream_owned = true;
  }
  return 0;
}

int nml_get_stream(void** out) {
  *out = reinterpret_cast<void*>(nml::g_stream);
  return 0;
}

int nml_set_stream(void* s) {
  nml::g_stream = reinterpret_cast<hipStream_t>(s);
  nml::g_stream_owned = false;
  return 0;
}

int nml_device_info(char* name, size_t name_len, int* cu_count, size_t* total_mem) {
  int dev = 0;
  NML_HIP(hipGetDevice(&dev));
  hipDeviceProp_t p;
  NML_HIP(hipGetDeviceProperties(&p, dev));
  if (name && name_len) {
    snprintf(name, name_len, "%s (%s)", p.name, p.gcnArchName);
  }
  if (cu_count) *cu_count = p.multiProcessorCount;
  if (total_mem) *total_mem = p.totalGlobalMem;
  return 0;
}

int nml_malloc(size_t bytes, void** out) {
  *out = nullptr;
  if (bytes == 0) bytes = 256;
  NML_HIP(hipMalloc(out, bytes));
  return 0;
}

// Waits for the library stream first: callers (Python's GC) may free a buffer
// that queued kernels still read.
int nml_free(void* p) {
  if (!p) return 0;
  if (nml::g_stream) NML_HIP(hipStreamSynchronize(nml::g_stream));
  NML_HIP(hipFree(p));
  return 0;
}

int nml_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  if (!bytes) return 0;
  NML_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, nml::g_stream));
  NML_HIP(hipStreamSynchronize(nml::g_stream));
  return 0;
}

int nml_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  if (!bytes) return 0;
  NML_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, nml::g_stream));
  NML_HIP(hipStreamSynchronize(nml::g_stream));
  return 0;
}

int nml_memcpy_d2d(void* dst, const void* src, size_t bytes) {
  if (!bytes) return 0;
  NML_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, nml::g_stream));
  return 0;
}

int nml_memset(void* dst, int value, size_t bytes) {
  if (!bytes) return 0;
  NML_HIP(hipMemsetAsync(dst, value, bytes, nml::g_stream));
  return 0;
}

int nml_synchronize(void) {
  NML_HIP(hipStreamSynchronize(nml::g_stream));
  return 0;
}

int nml_event_create(void** ev) {
  hipEvent_t e;
  NML_HIP(hipEventCreate(&e));
  *ev = reinterpret_cast<void*>(e);
  return 0;
}

int nml_event_record(void* ev) {
  NML_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(ev), nml::g_stream));
  return 0;
}

int nml_event_elapsed_ms(void* start, void* end, float* ms) {
  NML_HIP(hipEventSynchronize(reinterpret_cast<hipEvent_t>(end)));
  NML_HIP(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                              reinterpret_cast<hipEvent_t>(end)));
  return 0;
}

int nml_event_destroy(void* ev) {
  if (ev) NML_HIP(hipEventDestroy(reinterpret_cast<hipEvent_t>(ev)));
  return 0;
}

}  // extern "C"
