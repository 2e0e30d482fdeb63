// Compensated (Kahan) accumulation, shared by the column sums of the
// library and of its runtime-compiled expression kernels (device only).
#pragma once

namespace tjh {

// Compensated (Kahan) accumulation: s + c carries the running sum with the
// low-order bits lost by each fp32 addition kept in c, so a long sum of
// cancelling terms stays within a few ulp of its exact value.
struct Kahan {
  float s = 0.f, c = 0.f;
  __device__ __forceinline__ void add(float x) {
#pragma clang fp contract(off)
    const float y = x - c;
    const float t = s + y;
    c = (t - s) - y;
    s = t;
  }
};

}  // namespace tjh
