// C-ABI plumbing shared by every entry point: the per-thread error message,
// the ABI version and the gfx950 device check.
#include <stdarg.h>
#include <stdio.h>

#include "dsa_common.hpp"

namespace dsa {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(DSA_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return DSA_OK;
}

}  // namespace dsa

extern "C" const char *dsa_last_error(void) { return dsa::g_last_error; }

extern "C" int dsa_abi_version(void) { return 201; }

extern "C" int dsa_device_check(int device) {
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess)
    return dsa::set_error(DSA_ERR_HIP, "hipGetDeviceProperties(%d): %s", device, hipGetErrorString(e));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return dsa::set_error(DSA_ERR_UNSUPPORTED,
                          "device %d is %s; this library is built for gfx950 (MI355X) only",
                          device, prop.gcnArchName);
  return DSA_OK;
}

// ---------------------------------------------------------------------------
// Stage timing: a ring of HIP events per thread.  When enabled, each call of a
// multi-kernel entry point takes the next ring record and marks its stage
// boundaries on its own stream; nothing waits until dsa_stage_times() reads a
// record back.
// ---------------------------------------------------------------------------
namespace dsa {

constexpr int kStageRing = 256;
constexpr int kStageMarks = 8;

struct StageRecord {
  int n = 0;
  int device = -1;
  hipEvent_t ev[kStageMarks] = {};
};

static thread_local bool g_stage_on = false;
static thread_local long long g_stage_calls = 0;
static thread_local StageRecord g_stage_ring[kStageRing];
static thread_local StageRecord *g_stage_cur = nullptr;

void stage_begin(hipStream_t st) {
  g_stage_cur = nullptr;
  if (!g_stage_on) return;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return;
  StageRecord &r = g_stage_ring[g_stage_calls % kStageRing];
  if (r.device != dev) {
    for (int i = 0; i < kStageMarks; ++i) {
      if (r.ev[i]) (void)hipEventDestroy(r.ev[i]);
      r.ev[i] = nullptr;
    }
    for (int i = 0; i < kStageMarks; ++i)
      if (hipEventCreate(&r.ev[i]) != hipSuccess) return;
    r.device = dev;
  }
  ++g_stage_calls;
  r.n = 0;
  g_stage_cur = &r;
  stage_mark(st);
}

void stage_mark(hipStream_t st) {
  StageRecord *r = g_stage_cur;
  if (!r || r->n >= kStageMarks) return;
  if (hipEventRecord(r->ev[r->n], st) == hipSuccess) ++r->n;
}

}  // namespace dsa

extern "C" int dsa_stage_timing(int enable) {
  dsa::g_stage_on = enable != 0;
  dsa::g_stage_cur = nullptr;
  return DSA_OK;
}

extern "C" int dsa_stage_times(int back, float *ms, int max_stages) {
  using namespace dsa;
  DSA_REQUIRE(ms && max_stages > 0, "dsa_stage_times: null output");
  DSA_REQUIRE(back >= 0 && back < kStageRing && back < g_stage_calls,
              "dsa_stage_times: no timed call %d back (timed calls so far: %lld, ring %d)", back, g_stage_calls,
              kStageRing);
  const StageRecord &r = g_stage_ring[(g_stage_calls - 1 - back) % kStageRing];
  DSA_REQUIRE(r.n >= 2, "dsa_stage_times: record holds %d marks", r.n);
  hipError_t e = hipEventSynchronize(r.ev[r.n - 1]);
  if (e != hipSuccess) return set_error(DSA_ERR_HIP, "dsa_stage_times: %s", hipGetErrorString(e));
  const int n = r.n - 1 < max_stages ? r.n - 1 : max_stages;
  for (int i = 0; i < n; ++i) {
    e = hipEventElapsedTime(&ms[i], r.ev[i], r.ev[i + 1]);
    if (e != hipSuccess) return set_error(DSA_ERR_HIP, "dsa_stage_times: %s", hipGetErrorString(e));
  }
  return n;
}
