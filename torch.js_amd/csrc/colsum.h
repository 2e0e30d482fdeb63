// Deterministic column sums of per-workgroup partial rows.
//
// A kernel whose workgroups each produce one partial row per output
// (part[b][0..cols)) hands the rows to colsum_final, which sums them in
// increasing b with compensated (Kahan) accumulation in one more launch.
// The sum order never depends on scheduling, so results are bitwise
// reproducible; the kernel boundary between the two launches makes every
// partial row visible without cross-workgroup fences (on MI355X an
// agent-scope fence writes back the XCD's L2).
#pragma once

#include "common.h"

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

constexpr int kFinalMax = 64;  // outputs one colsum_final launch can finish
constexpr int kBatch = 8;     // rows fetched before they are accumulated

// out[i][c] (=|+=) scale * sum_b part[i][b][c] for i < np (out[i] may be
// nullptr: skipped), np <= kFinalMax.  One launch on the library stream.
int colsum_final(float* const* part, float* const* out, int np, int64_t nb, int64_t cols,
                 int accumulate, float scale);

}  // namespace tjh
