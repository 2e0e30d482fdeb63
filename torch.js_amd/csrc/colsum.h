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
#include "kahan.h"

namespace tjh {

constexpr int kFinalMax = 64;  // outputs one colsum_final launch can finish
constexpr int kBatch = 8;     // rows fetched before they are accumulated

// out[i][c] (=|+=) scale * sum_b part[i][b][c] for i < np (out[i] may be
// nullptr: skipped), np <= kFinalMax.  One launch on the library stream.
int colsum_final(float* const* part, float* const* out, int np, int64_t nb, int64_t cols,
                 int accumulate, float scale);
// The same with a row length per output (outputs of different widths in
// one launch).
int colsum_final_cols(float* const* part, float* const* out, const int64_t* cols, int np,
                      int64_t nb, int accumulate, float scale);

// Row partition of a column sum over r of [outer][r][inner] (about two
// workgroups per CU, >= 16 rows each): nb slices of rchunk rows.  `vec`:
// the column blocks hold 4 columns per lane.
void colsum_plan(int64_t outer, int64_t r, int64_t inner, bool vec, int64_t* nb,
                 int64_t* rchunk);

}  // namespace tjh
