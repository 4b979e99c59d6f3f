#pragma once
// Launch bracketing for nbhs_kernel_timing_* (see nibble_hip_shim.h): when timing is enabled, a KernelTimer
// records a HIP event on the launch stream at construction and another at destruction, so the pair spans exactly
// the kernel launched in between.
#include <hip/hip_runtime.h>

namespace nbhs_timing {

bool enabled();
void record_begin(int kernel, hipStream_t s);
void record_end(int kernel, hipStream_t s);

class KernelTimer {
 public:
  KernelTimer(int kernel, hipStream_t s) : kernel_(kernel), s_(s), on_(enabled()) {
    if (on_) record_begin(kernel_, s_);
  }
  ~KernelTimer() {
    if (on_) record_end(kernel_, s_);
  }
  KernelTimer(const KernelTimer&) = delete;
  KernelTimer& operator=(const KernelTimer&) = delete;

 private:
  int kernel_;
  hipStream_t s_;
  bool on_;
};

}  // namespace nbhs_timing
