// Library metadata, error names and optional per-kernel event timing.
#include <string.h>

#include <vector>

#include "common.h"

namespace bdh {

namespace {
struct ProfRec {
  const char* name;
  hipEvent_t start, stop;
};
bool g_prof_on = false;
std::vector<ProfRec> g_recs;          // recorded, not yet collected
std::vector<hipEvent_t> g_free;       // reusable events
constexpr size_t kMaxRecs = 1 << 16;  // drop records beyond this until collected

hipEvent_t take_event() {
  if (!g_free.empty()) {
    hipEvent_t e = g_free.back();
    g_free.pop_back();
    return e;
  }
  // Timing-only events: no system-scope fence when they are recorded (the
  // records are read after the caller has synchronised the stream).
  hipEvent_t e = nullptr;
  if (hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess) return nullptr;
  return e;
}
}  // namespace

int prof_begin(const char* name, hipEvent_t* start, hipEvent_t* stop) {
  if (!g_prof_on || g_recs.size() >= kMaxRecs) return -1;
  ProfRec r{name, take_event(), take_event()};
  if (!r.start || !r.stop) return -1;
  g_recs.push_back(r);
  *start = r.start;
  *stop = r.stop;
  return int(g_recs.size()) - 1;
}

}  // namespace bdh

extern "C" const char* bdh_version(void) { return "bdh-hip 0.1 gfx950"; }

extern "C" const char* bdh_error_string(int code) {
  switch (code) {
    case BDH_OK: return "ok";
    case BDH_ERR_SHAPE: return "inconsistent or unsupported shapes";
    case BDH_ERR_DTYPE: return "unsupported dtype or dtype combination";
    case BDH_ERR_STRIDE: return "last dimension must have unit stride";
    case BDH_ERR_WORKSPACE: return "workspace missing or too small";
    case BDH_ERR_LAUNCH: return "HIP kernel launch failed";
    case BDH_ERR_ARG: return "invalid argument";
    case BDH_ERR_ALIAS: return "output overlaps an input";
    case BDH_ERR_SCRATCH: return "input needs more scratch than the no-allocation entry point holds";
    default: return "unknown error";
  }
}

extern "C" void bdh_profile_enable(int32_t on) { bdh::g_prof_on = on != 0; }

extern "C" int bdh_profile_collect(char* names, int32_t name_len, float* ms, int32_t max) {
  using namespace bdh;
  int n = 0;
  for (auto& r : g_recs) {
    if (n < max) {
      float t = -1.f;
      if (hipEventSynchronize(r.stop) == hipSuccess) (void)hipEventElapsedTime(&t, r.start, r.stop);
      if (ms) ms[n] = t;
      if (names && name_len > 0) {
        strncpy(names + size_t(n) * name_len, r.name, size_t(name_len) - 1);
        names[size_t(n) * name_len + name_len - 1] = 0;
      }
      ++n;
    }
    g_free.push_back(r.start);
    g_free.push_back(r.stop);
  }
  g_recs.clear();
  return n;
}
