// Library-wide C-ABI plumbing: error reporting and version query.
#include "akt_host.hpp"

#include <string.h>

#include <mutex>
#include <utility>
#include <vector>

namespace akt {

static thread_local char g_error[1024] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_error[0] = '\0'; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(AKT_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return AKT_OK;
}

// Opt-in kernel timer: while enabled, every entry point's dominant kernel is
// launched with an event pair stamped by the runtime at the dispatch's start
// and end; akt_kernel_timer_read() waits for the recorded pairs and returns
// their summed elapsed time.
namespace {
std::mutex g_timer_mu;
bool g_timer_on = false;
std::vector<std::pair<hipEvent_t, hipEvent_t>> g_timer_pairs;
}  // namespace

KernelTimer::KernelTimer() {
  std::lock_guard<std::mutex> lk(g_timer_mu);
  if (!g_timer_on) return;
  // No system-scope fence at the event: the stamps need no cache write-back,
  // which would otherwise be charged to the timed kernel.
  if (hipEventCreateWithFlags(&start_, hipEventDisableSystemFence) != hipSuccess ||
      hipEventCreateWithFlags(&stop_, hipEventDisableSystemFence) != hipSuccess)
    return;
  armed_ = true;
}

void KernelTimer::commit() {
  armed_ = false;
  std::lock_guard<std::mutex> lk(g_timer_mu);
  g_timer_pairs.emplace_back(start_, stop_);
  start_ = stop_ = nullptr;  // owned by g_timer_pairs now
}

KernelTimer::~KernelTimer() {
  if (start_) (void)hipEventDestroy(start_);
  if (stop_) (void)hipEventDestroy(stop_);
}

}  // namespace akt

extern "C" int akt_kernel_timer_enable(int enable) {
  std::lock_guard<std::mutex> lk(akt::g_timer_mu);
  for (auto& pr : akt::g_timer_pairs) {
    (void)hipEventDestroy(pr.first);
    (void)hipEventDestroy(pr.second);
  }
  akt::g_timer_pairs.clear();
  akt::g_timer_on = enable != 0;
  return AKT_OK;
}

extern "C" int akt_kernel_timer_read(double* total_ms, int64_t* launches) {
  std::lock_guard<std::mutex> lk(akt::g_timer_mu);
  double sum = 0.0;
  for (auto& pr : akt::g_timer_pairs) {
    if (hipEventSynchronize(pr.second) != hipSuccess)
      return akt::set_error(AKT_ERR_HIP, "hipEventSynchronize failed");
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, pr.first, pr.second) != hipSuccess)
      return akt::set_error(AKT_ERR_HIP, "hipEventElapsedTime failed");
    sum += ms;
  }
  if (total_ms) *total_ms = sum;
  if (launches) *launches = (int64_t)akt::g_timer_pairs.size();
  return AKT_OK;
}

extern "C" const char* akt_last_error(void) { return akt::g_error; }

extern "C" int akt_abi_version(void) { return AKT_ABI_VERSION; }
