// Sampling from categorical distributions on the device: Tensor.multinomial
// (src/tensor/Tensor.ts:271-359), which torch.js evaluates on the host
// after a readback, with Math.random.
//
// Semantics kept from the reference (Tensor.ts:308-359): the weights of a
// row are p_i = max(0, x_i) (negative weights and -inf weigh 0),
// normalised by their sum; a row whose sum is not positive samples
// uniformly.  With replacement, a draw u in [0, 1) picks the first index
// whose running sum of p / sum exceeds u (the last index when rounding
// leaves u above the total).  Without replacement each draw renormalises
// over the indices not taken yet (the distribution of the reference's
// redraw-until-new loop): the first untaken index whose running sum of p
// exceeds u times the untaken mass.
//
// Where the reference is undefined this file states its own contract:
// - a row holding NaN or +inf is an error (PyTorch raises; the reference's
//   Math.max(0, NaN) is NaN, so its cumulative probabilities are NaN and it
//   returns the last index with replacement or loops forever without).
//   The kernel writes -1 for every draw of such a row and a status word
//   per row, which tjh_multinomial reads back (the call synchronises) to
//   return TJH_ERR_INVALID;
// - without replacement, once every positive-weight category is taken,
//   each further draw takes the last untaken index (the reference falls
//   back to index 0 and redraws until it finds a new one, which never
//   ends when 0 is taken; PyTorch raises).
//
// The uniforms are the library's seeded stream, not Math.random: draw s of
// row r uses element e = r * num_samples + s of tjh_random's uniform
// generator with the call's seed (xorshift32 of seed ^ (e*1664525 +
// 1013904223), over 2^32, as float32), so a caller can reproduce every
// draw.
//
// One workgroup per row; thread t owns a contiguous segment of the row, so
// a running sum is a per-segment sequential sum plus the exclusive scan of
// the segment totals (double precision throughout).

#include <vector>

#include "common.h"

namespace tjh {
namespace {

constexpr int kThreads = 256;
constexpr int64_t kTakenBits = 262144;  // LDS bitmap: rows of at most 2^18 categories
constexpr int32_t kNone = 0x7fffffff;   // no segment claimed the draw

__device__ __forceinline__ uint32_t xs32(uint32_t x) {
  x ^= x << 13;
  x ^= x >> 17;
  x ^= x << 5;
  return x;
}

// the float32 uniform of tjh_random's element e
__device__ __forceinline__ double uniform_at(uint32_t seed, uint64_t e) {
  const uint32_t s1 = xs32(seed ^ ((uint32_t)e * 1664525u + 1013904223u));
  return (double)((float)s1 / 4294967296.0f);
}

__device__ __forceinline__ double block_sum_d(double v, double* sm) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) sm[w] = v;
  __syncthreads();
  double r = 0.0;
  for (int i = 0; i < kThreads / 64; ++i) r += sm[i];
  return r;
}

// exclusive prefix of v over the block's threads (thread order)
__device__ __forceinline__ double block_exclusive_d(double v, double* sm) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  double incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const double o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  __syncthreads();
  if (lane == 63) sm[w] = incl;
  __syncthreads();
  double base = 0.0;
  for (int i = 0; i < w; ++i) base += sm[i];
  return base + incl - v;
}

template <bool REPL>
__global__ __launch_bounds__(kThreads) void k_multinomial(const float* __restrict__ probs,
                                                          int64_t cols, int64_t ns,
                                                          uint32_t seed,
                                                          int32_t* __restrict__ out,
                                                          int32_t* __restrict__ status) {
  __shared__ double sm[kThreads / 64];
  __shared__ int32_t pick;
  __shared__ uint32_t taken[REPL ? 1 : kTakenBits / 32];
  const int64_t r = blockIdx.x;
  const float* x = probs + r * cols;
  const int t = threadIdx.x;
  const int64_t seg = (cols + kThreads - 1) / kThreads;
  const int64_t lo = (int64_t)t * seg < cols ? (int64_t)t * seg : cols;
  const int64_t hi = lo + seg < cols ? lo + seg : cols;
  auto weight = [&](int64_t i) -> double {
    const float v = x[i];
    return v > 0.f ? (double)v : 0.0;  // negatives and -inf weigh 0
  };
  double local = 0.0;
  int bad = 0;
  for (int64_t i = lo; i < hi; ++i) {
    const float v = x[i];
    bad |= (v != v) | (v == __builtin_huge_valf());
    local += v > 0.f ? (double)v : 0.0;
  }
  if (__syncthreads_or(bad)) {  // the same value in every thread of the row
    for (int64_t s = t; s < ns; s += kThreads) out[r * ns + s] = -1;
    if (t == 0) status[r] = 1;
    return;
  }
  if (t == 0) status[r] = 0;
  const double total = block_sum_d(local, sm);
  const bool uniform = !(total > 0.0);
  auto w_of = [&](int64_t i) -> double { return uniform ? 1.0 : weight(i); };
  if (!REPL) {
    for (int64_t i = t; i < (cols + 31) / 32; i += kThreads) taken[i] = 0u;
    __syncthreads();  // every word cleared before the first draw reads it
  }
  const double norm = uniform ? (double)cols : total;
  for (int64_t s = 0; s < ns; ++s) {
    const double u = uniform_at(seed, (uint64_t)r * (uint64_t)ns + (uint64_t)s);
    // this thread's segment sum of the weights still in play
    double seg_sum = 0.0;
    for (int64_t i = lo; i < hi; ++i) {
      if (!REPL && ((taken[i >> 5] >> (i & 31)) & 1u)) continue;
      seg_sum += REPL ? w_of(i) / norm : w_of(i);
    }
    const double mass = REPL ? 1.0 : block_sum_d(seg_sum, sm);
    const double target = REPL ? u : u * mass;
    const double before = block_exclusive_d(seg_sum, sm);
    if (t == 0) pick = kNone;
    __syncthreads();
    // the segment holding the target (scan rounding can make two adjacent
    // segments claim it: the smaller index wins, so the pick is the same on
    // every run)
    if (seg_sum > 0.0 && before <= target && target < before + seg_sum) {
      double c = before;
      int64_t last = -1, found = -1;
      for (int64_t i = lo; i < hi; ++i) {
        if (!REPL && ((taken[i >> 5] >> (i & 31)) & 1u)) continue;
        const double wi = REPL ? w_of(i) / norm : w_of(i);
        if (wi <= 0.0) continue;
        last = i;
        c += wi;
        if (target < c) {
          found = i;
          break;
        }
      }
      atomicMin(&pick, (int32_t)(found >= 0 ? found : last));
    }
    __syncthreads();
    int32_t idx = pick == kNone ? -1 : pick;
    if (idx < 0) {
      // rounding left the target at or past the total: the last index in
      // play (the reference's default is the last index)
      if (REPL) {
        idx = (int32_t)(cols - 1);
      } else {
        int64_t best = -1;
        for (int64_t i = hi - 1; i >= lo && best < 0; --i)
          if (!((taken[i >> 5] >> (i & 31)) & 1u)) best = i;
        __syncthreads();
        if (t == 0) pick = -1;
        __syncthreads();
        if (best >= 0) atomicMax(&pick, (int32_t)best);
        __syncthreads();
        idx = pick;
      }
    }
    if (t == 0) out[r * ns + s] = idx;
    if (!REPL) {
      if (t == 0 && idx >= 0) taken[idx >> 5] |= 1u << (idx & 31);
    }
    __syncthreads();
  }
}

}  // namespace
}  // namespace tjh

using namespace tjh;

extern "C" {

int tjh_multinomial(const float* probs, int64_t rows, int64_t cols, int64_t num_samples,
                    int replacement, uint32_t seed, int32_t* out) {
  TJH_REQUIRE_INIT();
  TJH_ARG(rows >= 0 && cols > 0 && num_samples >= 0, "tjh_multinomial: bad sizes");
  TJH_ARG(replacement || num_samples <= cols,
          "tjh_multinomial: cannot sample %lld values from %lld categories without replacement",
          (long long)num_samples, (long long)cols);
  TJH_ARG(replacement || cols <= kTakenBits,
          "tjh_multinomial: rows of more than %lld categories need replacement",
          (long long)kTakenBits);
  TJH_ARG(rows < (int64_t(1) << 31), "tjh_multinomial: too many rows");
  if (rows == 0 || num_samples == 0) return TJH_OK;
  TJH_ARG(probs && out, "tjh_multinomial: NULL pointer");
  if (capturing())  // the per-row status is read back to the host
    return set_error(TJH_ERR_UNSUPPORTED,
                     "tjh_multinomial: not allowed while a graph is being captured");
  Scratch st((size_t)rows * sizeof(int32_t));
  if (!st.ok()) return set_error(TJH_ERR_OOM, "tjh_multinomial: no scratch");
  {
    KernelScope ks("multinomial");
    if (replacement)
      tjh_launch(k_multinomial<true>, dim3((unsigned)rows), dim3(kThreads), 0, stream(), probs,
                 cols, num_samples, seed, out, st.as<int32_t>());
    else
      tjh_launch(k_multinomial<false>, dim3((unsigned)rows), dim3(kThreads), 0, stream(), probs,
                 cols, num_samples, seed, out, st.as<int32_t>());
    const int rc = check_launch("multinomial");
    if (rc != TJH_OK) return rc;
  }
  std::vector<int32_t> hs((size_t)rows);
  hipError_t e = hipMemcpyAsync(hs.data(), st.p, (size_t)rows * sizeof(int32_t),
                                hipMemcpyDeviceToHost, stream());
  if (e == hipSuccess) e = hipStreamSynchronize(stream());
  if (e != hipSuccess) return hip_fail(e, "multinomial status readback");
  for (int64_t r = 0; r < rows; ++r)
    if (hs[(size_t)r])
      return set_error(TJH_ERR_INVALID,
                       "tjh_multinomial: probability row %lld contains NaN or inf", (long long)r);
  return TJH_OK;
}

}  // extern "C"
