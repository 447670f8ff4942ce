// HIP runtime for the hist engine: one device, one stream, explicit device
// memory and event timing.  Replaces the reference's Metal runtime
// (src/runtime.mm:37-455): no unified memory, so results are copied back
// explicitly; no indirect dispatch, so kernels read device-side work counts.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <functional>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "device_common.hpp"

namespace mgb {
namespace {
thread_local std::string g_error;
hipStream_t g_stream = nullptr;
int g_device = -1;
std::mutex g_init_mutex;
hipEvent_t g_events[16] = {};
}  // namespace

struct Profile {
  bool on = false;
  std::vector<hipEvent_t> free_events;
  struct Pending { int kind; hipEvent_t begin, end; };
  std::vector<Pending> pending;
  double ms[MGB_PROF_KINDS] = {};
  uint64_t launches[MGB_PROF_KINDS] = {};
  hipEvent_t take() {
    hipEvent_t e = nullptr;
    if (!free_events.empty()) { e = free_events.back(); free_events.pop_back(); }
    // No system-scope fence when the event completes: the timestamps bracket
    // the kernel alone, as the profiler's dispatch records do.
    else if (hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess) e = nullptr;
    return e;
  }
};
Profile g_profile;

hipStream_t stream() { return g_stream; }

bool prof_events(int kind, hipEvent_t* begin, hipEvent_t* end) {
  if (!g_profile.on || kind < 0 || kind >= MGB_PROF_KINDS) return false;
  *begin = g_profile.take();
  *end = g_profile.take();
  if (*begin && *end) return true;
  if (*begin) g_profile.free_events.push_back(*begin);
  if (*end) g_profile.free_events.push_back(*end);
  return false;
}

void prof_record(int kind, hipEvent_t begin, hipEvent_t end) { g_profile.pending.push_back({kind, begin, end}); }

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

int bound_device() { return ensure_init() ? -1 : g_device; }

bool profiling_enabled() { return g_profile.on; }

// Model data copied back to the host (a drain of queued rounds: every
// round's node records) lands in one pinned buffer kept for the process:
// no page faults on freshly allocated host memory and no staging of a
// pageable copy (262,144 x 64: 2 MB per fit, 0.22 ms of device idle at the
// end of every fit before).  Grows to the largest request, in 4 MiB steps.
namespace {
std::mutex g_pinned_mutex;
uint8_t* g_pinned = nullptr;
size_t g_pinned_bytes = 0;
}  // namespace

int download_pinned(const void* src, size_t bytes, const std::function<void(const uint8_t*)>& use) {
  if (ensure_init()) return -1;
  std::lock_guard<std::mutex> lock(g_pinned_mutex);
  if (g_pinned_bytes < bytes) {
    if (g_pinned) MGB_CHECK(hipHostFree(g_pinned));
    g_pinned = nullptr;
    g_pinned_bytes = 0;
    const size_t step = size_t(4) << 20;
    const size_t want = (bytes + step - 1) / step * step;
    void* p = nullptr;
    MGB_CHECK(hipHostMalloc(&p, want, hipHostMallocDefault));
    g_pinned = static_cast<uint8_t*>(p);
    g_pinned_bytes = want;
  }
  if (bytes) {
    MGB_CHECK(hipMemcpyAsync(g_pinned, src, bytes, hipMemcpyDeviceToHost, g_stream));
    MGB_CHECK(hipStreamSynchronize(g_stream));
  }
  use(g_pinned);
  return 0;
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
  // Blocks the allocator gives back (beyond what it keeps, below) return to
  // the device's default pool; keep up to 4 GiB of it mapped between passes
  // instead of releasing it at every synchronisation.
  hipMemPool_t pool = nullptr;
  MGB_CHECK(hipDeviceGetDefaultMemPool(&pool, device));
  uint64_t keep = uint64_t(4) << 30;
  MGB_CHECK(hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep));
  g_device = device;
  return 0;
}

const char* mgb_last_error(void) { return g_error.c_str(); }

int mgb_device_count(int* count) {
  MGB_CHECK(hipGetDeviceCount(count));
  return 0;
}

// Device buffers are stream-ordered allocations from the device's default
// pool on the library's one stream (the reference pools its round buffers,
// src/learner.cpp:25-35), and a freed buffer is kept by the library for the
// next request of about its size instead of going back to HIP: a
// hipFreeAsync costs 0.35-1.2 ms of host time on this runtime even on an idle
// stream, which after a synchronisation (the end of the quantile sketch, a
// booster's teardown) is time the device waits (262,144 x 64: about 2 ms of
// frees and 0.5 ms of allocations per fit).  Every use of a buffer is ordered
// on the one stream, so a kept buffer handed out again is only touched after
// the work that used it.  At most kCacheBytes are kept; larger frees, and
// everything kept when an allocation fails, go back to the pool.
namespace {
std::mutex g_alloc_mutex;
std::multimap<size_t, void*> g_kept;         // freed blocks by size
std::unordered_map<void*, size_t> g_blocks;  // every block handed out, by address
size_t g_kept_bytes = 0;
constexpr size_t kCacheBytes = size_t(8) << 30;

// Block sizes: 256-byte multiples up to 1 MiB, then 2 MiB multiples, so that
// buffers of nearly equal size share blocks.
size_t block_bytes(size_t bytes) {
  const size_t g = bytes <= (size_t(1) << 20) ? 256 : (size_t(2) << 20);
  return (bytes + g - 1) / g * g;
}

// Returns every kept block to the pool (caller holds g_alloc_mutex).
void release_kept() {
  for (auto& kv : g_kept) (void)hipFreeAsync(kv.second, g_stream);
  g_kept.clear();
  g_kept_bytes = 0;
}
}  // namespace

int mgb_malloc(void** ptr, size_t bytes) {
  if (ensure_init()) return -1;
  *ptr = nullptr;
  if (!bytes) return 0;
  const size_t want = block_bytes(bytes);
  std::lock_guard<std::mutex> lock(g_alloc_mutex);
  // The smallest kept block that fits, unless it is more than twice the size.
  auto it = g_kept.lower_bound(want);
  if (it != g_kept.end() && it->first / 2 <= want) {
    *ptr = it->second;
    g_kept_bytes -= it->first;
    g_blocks[*ptr] = it->first;
    g_kept.erase(it);
    return 0;
  }
  hipError_t status = hipMallocAsync(ptr, want, g_stream);
  if (status != hipSuccess && !g_kept.empty()) {
    (void)hipGetLastError();
    release_kept();
    status = hipMallocAsync(ptr, want, g_stream);
  }
  if (status != hipSuccess) {
    *ptr = nullptr;
    return check(status, "hipMallocAsync");
  }
  g_blocks[*ptr] = want;
  return 0;
}

int mgb_free(void* ptr) {
  if (!ptr) return 0;
  if (ensure_init()) return -1;
  std::lock_guard<std::mutex> lock(g_alloc_mutex);
  auto it = g_blocks.find(ptr);
  if (it == g_blocks.end()) {
    set_error("mgb_free: not a buffer from mgb_malloc");
    return -1;
  }
  const size_t bytes = it->second;
  g_blocks.erase(it);
  if (g_kept_bytes + bytes <= kCacheBytes) {
    g_kept.emplace(bytes, ptr);
    g_kept_bytes += bytes;
    return 0;
  }
  MGB_CHECK(hipFreeAsync(ptr, g_stream));
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

int mgb_memcpy_h2d_async(void* dst, const void* src, size_t bytes) {
  if (ensure_init()) return -1;
  if (!bytes) return 0;
  MGB_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
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

int mgb_profile_enable(int on) {
  if (ensure_init()) return -1;
  g_profile.on = on != 0;
  return 0;
}

int mgb_profile_collect(void) {
  if (ensure_init()) return -1;
  MGB_CHECK(hipStreamSynchronize(g_stream));
  for (auto& p : g_profile.pending) {
    float ms = 0;
    MGB_CHECK(hipEventElapsedTime(&ms, p.begin, p.end));
    g_profile.ms[p.kind] += ms;
    g_profile.launches[p.kind] += 1;
    g_profile.free_events.push_back(p.begin);
    g_profile.free_events.push_back(p.end);
  }
  g_profile.pending.clear();
  return 0;
}

int mgb_profile_read(double* ms, uint64_t* launches, int kinds) {
  for (int k = 0; k < kinds && k < MGB_PROF_KINDS; ++k) {
    if (ms) ms[k] = g_profile.ms[k];
    if (launches) launches[k] = g_profile.launches[k];
  }
  return 0;
}

int mgb_profile_reset(void) {
  for (int k = 0; k < MGB_PROF_KINDS; ++k) { g_profile.ms[k] = 0; g_profile.launches[k] = 0; }
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
