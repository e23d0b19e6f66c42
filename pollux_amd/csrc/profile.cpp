// HIP-event timing of one selected kernel (plx_profile_select: the quantizer's
// scoring kernel by default, or pack / unpack / dequant / the optimiser
// update) for bench.py.
//
// Events come from a pool created at plx_profile_begin(), so nothing is
// allocated inside the timed region; recording stops silently when the pool
// is exhausted.

#include <mutex>
#include <vector>

#include "plx_internal.h"

namespace plx {
namespace {

constexpr int kMaxLaunches = 4096;

struct Profile {
  std::mutex mu;
  bool enabled = false;
  std::vector<hipEvent_t> start, stop;
  int used = 0;
  bool open = false;  // a start event has been recorded without its stop
  int kernel = PLX_PROF_NN;
};

Profile &prof() {
  static Profile p;
  return p;
}

}  // namespace

void profile_before(hipStream_t s, int kernel) {
  Profile &p = prof();
  std::lock_guard<std::mutex> lock(p.mu);
  if (!p.enabled || kernel != p.kernel || p.used >= static_cast<int>(p.start.size())) return;
  if (hipEventRecord(p.start[p.used], s) == hipSuccess) p.open = true;
}

void profile_after(hipStream_t s, int kernel) {
  Profile &p = prof();
  std::lock_guard<std::mutex> lock(p.mu);
  if (!p.enabled || kernel != p.kernel || !p.open) return;
  if (hipEventRecord(p.stop[p.used], s) == hipSuccess) ++p.used;
  p.open = false;
}

}  // namespace plx

using namespace plx;

extern "C" {

int plx_profile_select(int kernel) {
  if (kernel < PLX_PROF_NN || kernel > PLX_PROF_T12)
    return fail(PLX_EINVAL, "plx_profile_select: unknown kernel id %d", kernel);
  Profile &p = prof();
  std::lock_guard<std::mutex> lock(p.mu);
  if (p.enabled) return fail(PLX_EINVAL, "plx_profile_select: recording is on (call it before plx_profile_begin)");
  p.kernel = kernel;
  return PLX_OK;
}

int plx_profile_begin(void) {
  Profile &p = prof();
  std::lock_guard<std::mutex> lock(p.mu);
  if (p.start.empty()) {
    p.start.resize(kMaxLaunches);
    p.stop.resize(kMaxLaunches);
    for (int i = 0; i < kMaxLaunches; ++i) {
      int st = check_hip(hipEventCreate(&p.start[i]), "hipEventCreate");
      if (st == PLX_OK) st = check_hip(hipEventCreate(&p.stop[i]), "hipEventCreate");
      if (st != PLX_OK) {
        p.start.resize(i);
        p.stop.resize(i);
        return st;
      }
    }
  }
  p.used = 0;
  p.open = false;
  p.enabled = true;
  return PLX_OK;
}

int plx_profile_end(double *total_ms, int64_t *launches) {
  Profile &p = prof();
  std::lock_guard<std::mutex> lock(p.mu);
  p.enabled = false;
  double sum = 0.0;
  for (int i = 0; i < p.used; ++i) {
    int st = check_hip(hipEventSynchronize(p.stop[i]), "hipEventSynchronize");
    if (st != PLX_OK) return st;
    float ms = 0.f;
    st = check_hip(hipEventElapsedTime(&ms, p.start[i], p.stop[i]), "hipEventElapsedTime");
    if (st != PLX_OK) return st;
    sum += ms;
  }
  if (total_ms) *total_ms = sum;
  if (launches) *launches = p.used;
  return PLX_OK;
}

}  // extern "C"
