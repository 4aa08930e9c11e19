// Optional per-kernel timing: when enabled, every kernel launch of the library
// is bracketed by two HIP events recorded on the launch stream.  Collection
// waits on the recorded events and aggregates elapsed time by kernel name.
#include <mutex>
#include <string>
#include <vector>

#include "kf_common.h"
#include "kf_internal.h"

namespace kf {
namespace prof {

namespace {
struct Rec {
  const char* name;
  hipEvent_t start, stop;
};
std::mutex g_mu;
bool g_on = false;
std::vector<Rec> g_recs;
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

bool enabled() { return g_on; }

void begin(const char* name, hipStream_t s) {
  std::lock_guard<std::mutex> lk(g_mu);
  Rec r{name, take_event(), take_event()};
  if (r.start) (void)hipEventRecord(r.start, s);
  g_recs.push_back(r);
}

void end(hipStream_t s) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_recs.empty() && g_recs.back().stop) (void)hipEventRecord(g_recs.back().stop, s);
}

}  // namespace prof
}  // namespace kf

extern "C" {

int kf_prof_enable(int on) {
  std::lock_guard<std::mutex> lk(kf::prof::g_mu);
  kf::prof::g_on = on != 0;
  return KF_OK;
}

int kf_prof_collect(char* names, float* total_ms, int* counts, int cap) {
  using namespace kf::prof;
  std::lock_guard<std::mutex> lk(g_mu);
  std::vector<std::string> keys;
  std::vector<float> tot;
  std::vector<int> cnt;
  for (Rec& r : g_recs) {
    float ms = 0.f;
    if (r.start && r.stop && hipEventSynchronize(r.stop) == hipSuccess)
      (void)hipEventElapsedTime(&ms, r.start, r.stop);
    size_t i = 0;
    while (i < keys.size() && keys[i] != r.name) ++i;
    if (i == keys.size()) {
      keys.emplace_back(r.name);
      tot.push_back(0.f);
      cnt.push_back(0);
    }
    tot[i] += ms;
    cnt[i] += 1;
    if (r.start) g_pool.push_back(r.start);
    if (r.stop) g_pool.push_back(r.stop);
  }
  g_recs.clear();
  const int n = (int)keys.size();
  for (int i = 0; i < n && i < cap; ++i) {
    if (names) {
      char* dst = names + 64 * i;
      snprintf(dst, 64, "%s", keys[i].c_str());
    }
    if (total_ms) total_ms[i] = tot[i];
    if (counts) counts[i] = cnt[i];
  }
  return n;
}

}  // extern "C"
