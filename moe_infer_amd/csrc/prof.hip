// Per-kernel timing with HIP events recorded on the launch stream around
// each kernel of the library (off by default).  bench.py reads the average
// duration of the dominant kernel from here; rocprofv3 kernel traces of the
// same run must agree with it.
#include <cstring>
#include <map>
#include <string>
#include <utility>
#include <vector>

#include "common.h"

namespace {
bool g_on = false;
std::map<std::string, std::vector<std::pair<hipEvent_t, hipEvent_t>>> g_rec;
std::map<std::string, hipEvent_t> g_open;

void clear_all() {
  for (auto& kv : g_rec)
    for (auto& p : kv.second) {
      (void)hipEventDestroy(p.first);
      (void)hipEventDestroy(p.second);
    }
  g_rec.clear();
  for (auto& kv : g_open) (void)hipEventDestroy(kv.second);
  g_open.clear();
}
}  // namespace

namespace mi {
void prof_begin(const char* name, hipStream_t s) {
  if (!g_on) return;
  hipEvent_t e;
  if (hipEventCreate(&e) != hipSuccess) return;
  (void)hipEventRecord(e, s);
  g_open[name] = e;
}

void prof_end(const char* name, hipStream_t s) {
  if (!g_on) return;
  auto it = g_open.find(name);
  if (it == g_open.end()) return;
  hipEvent_t e;
  if (hipEventCreate(&e) != hipSuccess) return;
  (void)hipEventRecord(e, s);
  g_rec[name].emplace_back(it->second, e);
  g_open.erase(it);
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
