// Per-kernel timing (off by default): every kernel of the library is
// launched with hipExtLaunchKernel, which stamps a start / stop event pair
// with the dispatch's own begin and end times on the launch stream.  bench.py
// reads the average duration of the dominant kernel from here; rocprofv3
// kernel traces of the same run agree with it.
#include <cstring>
#include <map>
#include <string>
#include <utility>
#include <vector>

#include "common.h"

namespace {
bool g_on = false;
std::map<std::string, std::vector<std::pair<hipEvent_t, hipEvent_t>>> g_rec;

void clear_all() {
  for (auto& kv : g_rec)
    for (auto& p : kv.second) {
      (void)hipEventDestroy(p.first);
      (void)hipEventDestroy(p.second);
    }
  g_rec.clear();
}
}  // namespace

namespace mi {
void prof_events(const char* name, hipEvent_t* start, hipEvent_t* stop) {
  *start = *stop = nullptr;
  if (!g_on) return;
  hipEvent_t a, b;
  if (hipEventCreate(&a) != hipSuccess) return;
  if (hipEventCreate(&b) != hipSuccess) {
    (void)hipEventDestroy(a);
    return;
  }
  g_rec[name].emplace_back(a, b);
  *start = a;
  *stop = b;
}
}  // namespace mi

extern "C" void mi_prof_enable(int on) {
  (void)hipDeviceSynchronize();
  clear_all();
  g_on = on != 0;
}

extern "C" mi_status mi_prof_read(const char* kernel, double* avg_us, int64_t* count) {
  mi::clear_error();
  if (!kernel || !avg_us || !count) return mi::fail(MI_ERR_INVALID_ARG, "null argument");
  *avg_us = 0.0;
  *count = 0;
  auto it = g_rec.find(kernel);
  if (it == g_rec.end()) return MI_OK;
  double total_ms = 0.0;
  for (auto& p : it->second) {
    MI_HIP(hipEventSynchronize(p.second));
    float ms = 0.f;
    MI_HIP(hipEventElapsedTime(&ms, p.first, p.second));
    total_ms += ms;
  }
  *count = (int64_t)it->second.size();
  if (*count) *avg_us = total_ms * 1000.0 / (double)*count;
  return MI_OK;
}
