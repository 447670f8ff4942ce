// HIP runtime for the hist engine: one device, one stream, explicit device
// memory and event timing.  Replaces the reference's Metal runtime
// (src/runtime.mm:37-455): no unified memory, so results are copied back
// explicitly; no indirect dispatch, so kernels read device-side work counts.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>
#include <string>

#include "device_common.hpp"

namespace mgb {
namespace {
thread_local std::string g_error;
hipStream_t g_stream = nullptr;
int g_device = -1;
std::mutex g_init_mutex;
hipEvent_t g_events[16] = {};
}  // namespace

hipStream_t stream() { return g_stream; }
void set_error(std::string message) { g_error = std::move(message); }

int check(hipError_t status, const char* what) {
  if (status == hipSuccess) return 0;
  set_error(std::string(what) + ": " + hipGetErrorString(status));
  return -1;
}

static int ensure_init() {
  if (g_stream) return 0;
  return mgb_init(0);
}

}  // namespace mgb

using namespace mgb;

extern "C" {

int mgb_init(int device) {
  std::lock_guard<std::mutex> lock(g_init_mutex);
  if (g_stream) return device == g_device ? 0 : (set_error("mgb_init: already bound to another device"), -1);
  int count = 0;
  MGB_CHECK(hipGetDeviceCount(&count));
  if (device < 0 || device >= count) {
    set_error("mgb_init: no HIP device " + std::to_string(device));
    return -1;
  }
  MGB_CHECK(hipSetDevice(device));
  // Default priority on purpose: streams of different priorities are not used.
  MGB_CHECK(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
  for (auto& e : g_events) MGB_CHECK(hipEventCreate(&e));
  g_device = device;
  return 0;
}

const char* mgb_last_error(void) { return g_error.c_str(); }

int mgb_device_count(int* count) {
  MGB_CHECK(hipGetDeviceCount(count));
  return 0;
}

int mgb_malloc(void** ptr, size_t bytes) {
  if (ensure_init()) return -1;
  *ptr = nullptr;
  if (!bytes) return 0;
  MGB_CHECK(hipMalloc(ptr, bytes));
  return 0;
}

int mgb_free(void* ptr) {
  if (!ptr) return 0;
  MGB_CHECK(hipFree(ptr));
  return 0;
}

int mgb_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  if (ensure_init()) return -1;
  if (!bytes) return 0;
  MGB_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
  MGB_CHECK(hipStreamSynchronize(g_stream));
  return 0;
}

int mgb_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  if (ensure_init()) return -1;
  if (!bytes) return 0;
  MGB_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
  MGB_CHECK(hipStreamSynchronize(g_stream));
  return 0;
}

int mgb_memcpy_d2d(void* dst, const void* src, size_t bytes) {
  if (ensure_init()) return -1;
  if (!bytes) return 0;
  MGB_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_stream));
  return 0;
}

int mgb_memset(void* dst, int value, size_t bytes) {
  if (ensure_init()) return -1;
  if (!bytes) return 0;
  MGB_CHECK(hipMemsetAsync(dst, value, bytes, g_stream));
  return 0;
}

int mgb_synchronize(void) {
  if (ensure_init()) return -1;
  MGB_CHECK(hipStreamSynchronize(g_stream));
  return 0;
}

int mgb_event_record(int slot) {
  if (ensure_init()) return -1;
  if (slot < 0 || slot >= 16) { set_error("mgb_event_record: slot out of range"); return -1; }
  MGB_CHECK(hipEventRecord(g_events[slot], g_stream));
  return 0;
}

int mgb_event_elapsed_ms(int begin_slot, int end_slot, float* ms) {
  if (begin_slot < 0 || begin_slot >= 16 || end_slot < 0 || end_slot >= 16) {
    set_error("mgb_event_elapsed_ms: slot out of range");
    return -1;
  }
  MGB_CHECK(hipEventSynchronize(g_events[end_slot]));
  MGB_CHECK(hipEventElapsedTime(ms, g_events[begin_slot], g_events[end_slot]));
  return 0;
}

}  // extern "C"
