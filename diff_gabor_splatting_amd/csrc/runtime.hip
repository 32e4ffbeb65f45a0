// Error reporting and optional per-family kernel timing for the C ABI.
#include <cstdarg>
#include <mutex>
#include <string>
#include <vector>

#include "common.hpp"

namespace gs {
namespace {

thread_local std::string g_error;

struct PendingEvent {
  int family;
  hipEvent_t start;
  hipEvent_t stop;
};

struct Profiler {
  std::mutex mutex;
  bool enabled = false;
  std::vector<PendingEvent> pending;
  double total_ms[GS_PROF_COUNT] = {};
  int64_t launches[GS_PROF_COUNT] = {};
};

Profiler& profiler() {
  static Profiler p;
  return p;
}

// Fold completed event pairs into the totals; the caller holds the mutex.
int drain(Profiler& p) {
  int status = GS_OK;
  for (auto& e : p.pending) {
    if (status == GS_OK) {
      hipError_t err = hipEventSynchronize(e.stop);
      float ms = 0.f;
      if (err == hipSuccess) err = hipEventElapsedTime(&ms, e.start, e.stop);
      if (err != hipSuccess) {
        status = hip_status(err, "profile event");
      } else {
        p.total_ms[e.family] += ms;
        p.launches[e.family] += 1;
      }
    }
    (void)hipEventDestroy(e.start);
    (void)hipEventDestroy(e.stop);
  }
  p.pending.clear();
  return status;
}

}  // namespace

void set_error(const char* fmt, ...) {
  char buffer[512];
  va_list args;
  va_start(args, fmt);
  vsnprintf(buffer, sizeof(buffer), fmt, args);
  va_end(args);
  g_error = buffer;
}

void clear_error() { g_error.clear(); }

int hip_status(hipError_t err, const char* what) {
  if (err == hipSuccess) return GS_OK;
  set_error("%s failed: %s", what, hipGetErrorString(err));
  return GS_ERR_HIP;
}

int launch_status(const char* kernel) {
  hipError_t err = hipGetLastError();
  if (err == hipSuccess) return GS_OK;
  set_error("launch of %s failed: %s", kernel, hipGetErrorString(err));
  return GS_ERR_HIP;
}

ProfileScope::ProfileScope(int family, hipStream_t stream) : family_(family), stream_(stream) {
  Profiler& p = profiler();
  std::lock_guard<std::mutex> lock(p.mutex);
  if (!p.enabled) return;
  if (hipEventCreate(&start_) != hipSuccess) {
    start_ = nullptr;
    return;
  }
  if (hipEventRecord(start_, stream_) != hipSuccess) {
    (void)hipEventDestroy(start_);
    start_ = nullptr;
  }
}

ProfileScope::~ProfileScope() {
  if (!start_) return;
  Profiler& p = profiler();
  std::lock_guard<std::mutex> lock(p.mutex);
  hipEvent_t stop = nullptr;
  if (hipEventCreate(&stop) != hipSuccess || hipEventRecord(stop, stream_) != hipSuccess) {
    if (stop) (void)hipEventDestroy(stop);
    (void)hipEventDestroy(start_);
    return;
  }
  p.pending.push_back({family_, start_, stop});
}

}  // namespace gs

extern "C" {

const char* gs_last_error(void) { return gs::g_error.c_str(); }

int gs_abi_version(void) { return 13; }

int gs_profile_enable(int32_t enable) {
  gs::clear_error();
  gs::Profiler& p = gs::profiler();
  std::lock_guard<std::mutex> lock(p.mutex);
  int status = gs::drain(p);
  p.enabled = enable != 0;
  if (p.enabled) {
    for (int i = 0; i < GS_PROF_COUNT; ++i) {
      p.total_ms[i] = 0.0;
      p.launches[i] = 0;
    }
  }
  return status;
}

int gs_profile_read(int32_t family, double* total_ms, int64_t* launches) {
  gs::clear_error();
  GS_REQUIRE(family >= 0 && family < GS_PROF_COUNT, GS_ERR_ARGUMENT, "unknown kernel family %d",
             family);
  GS_REQUIRE(total_ms && launches, GS_ERR_ARGUMENT, "null output pointer");
  gs::Profiler& p = gs::profiler();
  std::lock_guard<std::mutex> lock(p.mutex);
  int status = gs::drain(p);
  *total_ms = p.total_ms[family];
  *launches = p.launches[family];
  return status;
}

}  // extern "C"
