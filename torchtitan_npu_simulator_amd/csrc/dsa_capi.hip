// C-ABI plumbing shared by every entry point: thread-local error text, version, and the
// optional per-kernel HIP-event timing.
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "dsa_common.h"

namespace dsa {

static thread_local std::string g_last_error;

int set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(DSA_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return DSA_OK;
}

// ---- per-kernel timing: event pairs recorded around launches while enabled ----
namespace {
struct TimingRecord {
  const char* name;  // a string literal at the launch site
  hipEvent_t e0, e1;
};
struct TimingSummary {
  std::string name;
  double total_ms;
  int64_t launches;
};
std::atomic<bool> g_timing_on{false};
std::mutex g_timing_mu;
std::vector<TimingRecord> g_timing_records;
std::vector<TimingSummary> g_timing_summary;
bool g_timing_summarised = false;

void destroy_records() {
  for (auto& r : g_timing_records) {
    hipEventDestroy(r.e0);
    hipEventDestroy(r.e1);
  }
  g_timing_records.clear();
}
}  // namespace

bool kernel_timing_on() { return g_timing_on.load(std::memory_order_relaxed); }

void kernel_timing_begin(hipStream_t st, hipEvent_t* ev) {
  if (hipEventCreate(&ev[0]) != hipSuccess) {
    ev[0] = nullptr;
    return;
  }
  if (hipEventCreate(&ev[1]) != hipSuccess || hipEventRecord(ev[0], st) != hipSuccess) {
    hipEventDestroy(ev[0]);
    if (ev[1]) hipEventDestroy(ev[1]);
    ev[0] = ev[1] = nullptr;
  }
}

void kernel_timing_end(const char* name, hipStream_t st, hipEvent_t* ev) {
  if (hipEventRecord(ev[1], st) != hipSuccess) {
    hipEventDestroy(ev[0]);
    hipEventDestroy(ev[1]);
    return;
  }
  std::lock_guard<std::mutex> lk(g_timing_mu);
  g_timing_records.push_back({name, ev[0], ev[1]});
  g_timing_summarised = false;
}

}  // namespace dsa

extern "C" int dsa_kernel_timing(int enable) {
  using namespace dsa;
  std::lock_guard<std::mutex> lk(g_timing_mu);
  if (enable) {  // a fresh window: earlier records are dropped
    destroy_records();
    g_timing_summary.clear();
    g_timing_summarised = false;
  }
  g_timing_on.store(enable != 0);
  return DSA_OK;
}

extern "C" int dsa_kernel_timing_count(void) {
  using namespace dsa;
  std::lock_guard<std::mutex> lk(g_timing_mu);
  if (!g_timing_summarised) {
    g_timing_summary.clear();
    for (auto& r : g_timing_records) {
      if (hipEventSynchronize(r.e1) != hipSuccess) return -set_error(DSA_ERR_LAUNCH, "dsa_kernel_timing_count: event");
      float ms = 0.f;
      if (hipEventElapsedTime(&ms, r.e0, r.e1) != hipSuccess)
        return -set_error(DSA_ERR_LAUNCH, "dsa_kernel_timing_count: elapsed time");
      TimingSummary* t = nullptr;
      for (auto& x : g_timing_summary)
        if (x.name == r.name) t = &x;
      if (!t) {
        g_timing_summary.push_back({r.name, 0.0, 0});
        t = &g_timing_summary.back();
      }
      t->total_ms += ms;
      t->launches += 1;
    }
    g_timing_summarised = true;
  }
  return (int)g_timing_summary.size();
}

extern "C" int dsa_kernel_timing_get(int i, char* name, int64_t name_cap, double* total_ms, int64_t* launches) {
  using namespace dsa;
  std::lock_guard<std::mutex> lk(g_timing_mu);
  if (!g_timing_summarised || i < 0 || i >= (int)g_timing_summary.size())
    return set_error(DSA_ERR_INVALID_ARG, "dsa_kernel_timing_get: entry %d (call dsa_kernel_timing_count first)", i);
  const TimingSummary& t = g_timing_summary[i];
  if (name && name_cap > 0) {
    std::strncpy(name, t.name.c_str(), (size_t)name_cap - 1);
    name[name_cap - 1] = 0;
  }
  if (total_ms) *total_ms = t.total_ms;
  if (launches) *launches = t.launches;
  return DSA_OK;
}

extern "C" const char* dsa_last_error(void) { return dsa::g_last_error.c_str(); }

extern "C" int dsa_abi_version(void) { return 17; }
