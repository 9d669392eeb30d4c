// Host-side helpers shared by the C-ABI entry points: per-thread error
// message, argument checks and launch-status translation.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <atomic>

#include "../../include/akt_amd.h"

namespace akt {

// Sets the calling thread's error message and returns `code`.
int set_error(int code, const char* fmt, ...);
// Clears the calling thread's error message.
void clear_error();

// Returns AKT_ERR_HIP with a message if the last launch on this thread failed.
int check_launch(const char* what);

// Launches a kernel; while the kernel timer is enabled
// (akt_kernel_timer_enable) the launch goes through hipExtLaunchKernel with an
// event pair that the runtime stamps with the dispatch's own start and end
// times, so the timer sees kernel execution only (no queueing or launch gaps).
class KernelTimer {
 public:
  KernelTimer();
  ~KernelTimer();
  KernelTimer(const KernelTimer&) = delete;
  KernelTimer& operator=(const KernelTimer&) = delete;

  template <typename... Args, typename F = void (*)(Args...)>
  void launch(F kernel, dim3 grid, dim3 block, uint32_t lds_bytes, hipStream_t stream,
              Args... args) {
    if (armed_) {
      hipExtLaunchKernelGGL(kernel, grid, block, lds_bytes, stream, start_, stop_, 0, args...);
      commit();
    } else {
      hipLaunchKernelGGL(kernel, grid, block, lds_bytes, stream, args...);
    }
  }

 private:
  void commit();
  hipEvent_t start_ = nullptr, stop_ = nullptr;
  bool armed_ = false;
};

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

// True when every row that starts at `base + i * strides[j]` (element strides,
// fp16 elements) is 16-byte aligned.
inline bool rows_aligned16(const void* base, const int64_t* strides, int n) {
  if (!aligned16(base)) return false;
  for (int i = 0; i < n; ++i)
    if ((strides[i] * 2) % 16 != 0) return false;
  return true;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

constexpr int kMaxResidentDevices = 64;

// Workgroups of `kernel` (blocks of `threads`) that fit the current device at
// once (occupancy x CUs), cached per kernel instance and device; 0 if the
// queries fail.
template <typename Kernel>
int resident_blocks(Kernel kernel, int threads) {
  static std::atomic<int> cache[kMaxResidentDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxResidentDevices) return 0;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)kernel, threads, 0) !=
          hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  v = (per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
  cache[dev].store(v, std::memory_order_relaxed);
  return v;
}

}  // namespace akt

#define AKT_CHECK(cond, ...)                                         \
  do {                                                               \
    if (!(cond)) return ::akt::set_error(AKT_ERR_INVALID_ARGUMENT, __VA_ARGS__); \
  } while (0)
