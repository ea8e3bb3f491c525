// Opt-in kernel timing: while enabled, each launch site wrapped in a Scope
// records a hipEvent pair on the launch stream, tagged with the kernel class
// and the launch's algorithmic FLOPs and HBM bytes. Disabled, a Scope costs
// one relaxed atomic load.
#pragma once

#include <hip/hip_runtime.h>

namespace mc {
namespace prof {

enum Kind { kGemm = 0, kLowRank = 1, kRmsNorm = 2, kSoftmax = 3, kAttention = 4, kAdamW = 5, kRowOps = 6, kNumKinds = 7 };

bool enabled();
void set_enabled(bool on);
// Waits for every recorded event pair and folds it into the per-kind totals.
hipError_t collect();
void read(int kind, double* ms, long long* launches, double* flops, double* bytes);
void reset();

class Scope {
  public:
    Scope(Kind kind, hipStream_t stream, double flops, double bytes);
    ~Scope();
    Scope(const Scope&) = delete;
    Scope& operator=(const Scope&) = delete;

  private:
    int slot_ = -1;
    hipStream_t stream_;
};

}  // namespace prof
}  // namespace mc
