// profile.cpp -- optional per-kernel launch timing with HIP events.
//
// When enabled (cfa_profile_enable(1)), every kernel launch made by the
// library is bracketed by two hipEvents recorded on the stream the kernel is
// launched on, so the elapsed time between them is that kernel's duration on
// that stream (plus the ~µs event granularity).  Records accumulate until
// cfa_profile_reset(); cfa_profile_query() synchronises on the recorded
// events and sums the durations of one kernel name.  Disabled (the default),
// the launch path only reads one atomic flag.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "abi_internal.hpp"

namespace cfa {
namespace prof {

namespace {
struct Record {
  const char *name;
  hipEvent_t start, stop;
};
std::atomic<int> g_enabled{0};
std::mutex g_mu;
std::vector<Record> g_records;
std::vector<hipEvent_t> g_pool;

hipEvent_t take_event() {
  if (!g_pool.empty()) {
    hipEvent_t e = g_pool.back();
    g_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}
}  // namespace

bool enabled() { return g_enabled.load(std::memory_order_relaxed) != 0; }

void *begin(const char *name, hipStream_t stream) {
  std::lock_guard<std::mutex> lock(g_mu);
  Record r{name, take_event(), take_event()};
  if (!r.start || !r.stop) return nullptr;
  if (hipEventRecord(r.start, stream) != hipSuccess) return nullptr;
  g_records.push_back(r);
  return reinterpret_cast<void *>(g_records.size());
}

void end(void *token, hipStream_t stream) {
  if (!token) return;
  std::lock_guard<std::mutex> lock(g_mu);
  const size_t i = reinterpret_cast<size_t>(token) - 1;
  if (i < g_records.size()) (void)hipEventRecord(g_records[i].stop, stream);
}

}  // namespace prof
}  // namespace cfa

extern "C" int cfa_profile_enable(int on) {
  cfa::abi::clear_error();
  cfa::prof::g_enabled.store(on ? 1 : 0);
  return CFA_OK;
}

extern "C" int cfa_profile_reset(void) {
  using namespace cfa::prof;
  cfa::abi::clear_error();
  std::lock_guard<std::mutex> lock(g_mu);
  for (Record &r : g_records) {
    (void)hipEventSynchronize(r.stop);
    g_pool.push_back(r.start);
    g_pool.push_back(r.stop);
  }
  g_records.clear();
  return CFA_OK;
}

extern "C" int cfa_profile_query(const char *kernel, int *count, double *total_ms) {
  using namespace cfa::prof;
  cfa::abi::clear_error();
  if (!kernel || !count || !total_ms) return cfa::abi::fail_arg("cfa_profile_query: null argument");
  std::lock_guard<std::mutex> lock(g_mu);
  int n = 0;
  double ms = 0.0;
  for (Record &r : g_records) {
    if (std::strcmp(r.name, kernel) != 0) continue;
    if (hipError_t e = hipEventSynchronize(r.stop)) return cfa::abi::fail_hip(e, "cfa_profile_query");
    float t = 0.0f;
    if (hipError_t e = hipEventElapsedTime(&t, r.start, r.stop))
      return cfa::abi::fail_hip(e, "cfa_profile_query");
    ms += t;
    ++n;
  }
  *count = n;
  *total_ms = ms;
  return CFA_OK;
}
