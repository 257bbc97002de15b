// ABI housekeeping: version and the thread-local error string (the convention of
// deps/sentencepiece_bridge.cpp:11-16 and 83-87 in the reference).
#include "common.h"

#include <atomic>
#include <mutex>
#include <string>
#include <vector>

namespace reels {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(REELS_HIP_EHIP, std::string(what) + ": " + hipGetErrorString(e));
  return REELS_HIP_OK;
}

// ---- kernel timing instrumentation ----------------------------------------------------------
namespace {
struct TraceRec {
  const char* name;
  hipEvent_t start, stop;
};
std::mutex g_trace_mu;
std::vector<TraceRec> g_trace;  // events are created once and reused across trace sessions
int g_trace_used = 0, g_trace_cap = 0;
std::atomic<bool> g_trace_on{false};
std::string g_trace_only;  // record only kernels whose name contains this (empty: all)
thread_local bool g_trace_skip = false;  // the current launch is not recorded
}  // namespace

void trace_before(hipStream_t st, const char* name) {
  g_trace_skip = false;
  if (!g_trace_on) return;
  std::lock_guard<std::mutex> lk(g_trace_mu);
  if (!g_trace_on || g_trace_used >= g_trace_cap) return;
  if (!g_trace_only.empty() && std::string(name).find(g_trace_only) == std::string::npos) {
    g_trace_skip = true;
    return;
  }
  if (g_trace_used == (int)g_trace.size()) {
    TraceRec r{name, nullptr, nullptr};
    if (hipEventCreate(&r.start) != hipSuccess || hipEventCreate(&r.stop) != hipSuccess) {
      g_trace_on = false;
      return;
    }
    g_trace.push_back(r);
  }
  TraceRec& r = g_trace[g_trace_used];
  r.name = name;
  if (hipEventRecord(r.start, st) != hipSuccess) g_trace_on = false;
}

void trace_after(hipStream_t st) {
  if (!g_trace_on || g_trace_skip) return;
  std::lock_guard<std::mutex> lk(g_trace_mu);
  if (!g_trace_on || g_trace_used >= g_trace_cap) return;
  if (hipEventRecord(g_trace[g_trace_used].stop, st) != hipSuccess) g_trace_on = false;
  ++g_trace_used;
}

}  // namespace reels

extern "C" int reels_hip_trace_start(int capacity) {
  using namespace reels;
  clear_error();
  if (capacity < 0) return fail(REELS_HIP_EINVAL, "reels_hip_trace_start: capacity < 0");
  std::lock_guard<std::mutex> lk(g_trace_mu);
  g_trace_used = 0;
  g_trace_cap = capacity;
  g_trace_on = true;
  return REELS_HIP_OK;
}

extern "C" int reels_hip_trace_only(const char* name_part) {
  using namespace reels;
  clear_error();
  std::lock_guard<std::mutex> lk(g_trace_mu);
  g_trace_only = name_part ? name_part : "";
  return REELS_HIP_OK;
}

extern "C" int reels_hip_trace_stop(void) {
  using namespace reels;
  std::lock_guard<std::mutex> lk(g_trace_mu);
  g_trace_on = false;
  return g_trace_used;
}

extern "C" int reels_hip_trace_get(int index, const char** name, float* ms) {
  using namespace reels;
  clear_error();
  std::lock_guard<std::mutex> lk(g_trace_mu);
  if (index < 0 || index >= g_trace_used || name == nullptr || ms == nullptr)
    return fail(REELS_HIP_EINVAL, "reels_hip_trace_get: bad index or NULL output");
  *name = g_trace[index].name;
  float t = 0.0f;
  hipError_t e = hipEventElapsedTime(&t, g_trace[index].start, g_trace[index].stop);
  if (e != hipSuccess)
    return fail(REELS_HIP_EHIP, std::string("reels_hip_trace_get: ") + hipGetErrorString(e));
  *ms = t;
  return REELS_HIP_OK;
}

extern "C" int reels_hip_abi_version(void) { return REELS_HIP_ABI_VERSION; }

extern "C" const char* reels_hip_last_error(void) { return reels::g_last_error.c_str(); }
