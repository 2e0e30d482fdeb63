// Fused multi-tensor Adam / AdamW step.
//
// Replaces, per parameter, the ~9 tensor dispatches, 3-4 blocking
// device->host readbacks, JS update loop and writeBuffer of torch.js's
// Adam.step / AdamW.step (src/optim/adam.ts:46-133,
// src/optim/adamw.ts:46-154) with ONE streaming pass per batch of up to
// kMaxTensors parameters: read p, g, m, v; write p, m, v (28 bytes per
// parameter, HBM-bound).
//
// Rounding follows the reference exactly: the moment updates and the
// denominator are separate fp32 tensor ops there (each rounded), so they
// are rounded after every operation here too (contraction disabled); the
// final parameter update is the reference's JS double-precision loop,
// rounded once to fp32.

#include "common.h"

namespace tjh {
namespace {

constexpr int kBlock = 256;
constexpr int kMaxTensors = 56;  // keeps the kernel argument block under 4 KiB
// Elements per workgroup: one float4 of each of the four streams per lane.
// Small chunks (many workgroups, few registers) measured fastest on
// MI355X: 1024 -> 6.0 TB/s, 2048 -> 5.6, 4096 -> 5.4 over GPT-2's 124M
// parameters.
constexpr int64_t kChunk = kBlock * 4;

struct AdamTensor {
  float* p;
  const float* g;
  float* m;
  float* v;
  int64_t n;
  int64_t first_block;  // prefix sum of blocks
  double step_size;     // lr / bc1
  float bc2;            // f32(1 - beta2^step)
  int vec;
};

struct AdamBatch {  // passed by value: must stay within the 4 KiB kernel argument block
  AdamTensor t[kMaxTensors];
  int count;
  float b1, omb1, b2, omb2, eps, wd;  // fp32 scalars as torch.js's tensor ops see them
  double decay;                        // 1 - lr*wd (AdamW)
  int decoupled;
};
static_assert(sizeof(AdamBatch) <= 4000, "AdamBatch exceeds the kernel argument block");


// Every fp32 operation is rounded on its own (contraction off; IEEE
// division and the correctly rounded llvm.sqrt), as the reference's
// separate tensor ops round them.
__device__ __forceinline__ void adam_elem(float& p, float g, float& m, float& v,
                                          const AdamBatch& B, const AdamTensor& T) {
#pragma clang fp contract(off)
  if (!B.decoupled && B.wd != 0.f) g = g + p * B.wd;
  m = m * B.b1 + g * B.omb1;
  v = v * B.b2 + (g * g) * B.omb2;
  float denom = __builtin_sqrtf(v / T.bc2) + B.eps;
  double pd = (double)p;
  if (B.decoupled) pd = pd * B.decay;
  pd = pd - T.step_size * ((double)m / (double)denom);
  p = (float)pd;
}

__global__ __launch_bounds__(kBlock) void k_adam(AdamBatch B) {
  int b = blockIdx.x;
  // the tensor whose block range holds b: binary search over first_block
  int lo = 0, hi = B.count - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (B.t[mid].first_block <= b) lo = mid;
    else hi = mid - 1;
  }
  const int ti = lo;
  const AdamTensor& T = B.t[ti];
  int64_t beg = (int64_t)(b - T.first_block) * kChunk;
  int64_t end = beg + kChunk < T.n ? beg + kChunk : T.n;
  if (T.vec) {
    // every load of the chunk is issued before the first update
    constexpr int kSteps = kChunk / (4 * kBlock);
    float4 p[kSteps], g[kSteps], m[kSteps], v[kSteps];
#pragma unroll
    for (int u = 0; u < kSteps; ++u) {
      const int64_t i = beg + 4 * (threadIdx.x + (int64_t)u * kBlock);
      if (i < end) {
        p[u] = ld_nt(T.p + i);
        g[u] = ld_nt(T.g + i);
        m[u] = ld_nt(T.m + i);
        v[u] = ld_nt(T.v + i);
      }
    }
#pragma unroll
    for (int u = 0; u < kSteps; ++u) {
      const int64_t i = beg + 4 * (threadIdx.x + (int64_t)u * kBlock);
      if (i < end) {
        adam_elem(p[u].x, g[u].x, m[u].x, v[u].x, B, T);
        adam_elem(p[u].y, g[u].y, m[u].y, v[u].y, B, T);
        adam_elem(p[u].z, g[u].z, m[u].z, v[u].z, B, T);
        adam_elem(p[u].w, g[u].w, m[u].w, v[u].w, B, T);
        st_nt(T.p + i, p[u]);
        st_nt(T.m + i, m[u]);
        st_nt(T.v + i, v[u]);
      }
    }
  } else {
    for (int64_t i = beg + threadIdx.x; i < end; i += kBlock) {
      float p = T.p[i], m = T.m[i], v = T.v[i];
      adam_elem(p, T.g[i], m, v, B, T);
      T.p[i] = p;
      T.m[i] = m;
      T.v[i] = v;
    }
  }
}

}  // namespace
}  // namespace tjh

using namespace tjh;

extern "C" int tjh_adam_step(int n_tensors, float* const* params, const float* const* grads,
                             float* const* exp_avg, float* const* exp_avg_sq,
                             const int64_t* numels, const int64_t* steps, double lr, double beta1,
                             double beta2, double eps, double weight_decay, int decoupled) {
  TJH_REQUIRE_INIT();
  TJH_ARG(n_tensors >= 0, "tjh_adam_step: negative tensor count");
  if (n_tensors == 0) return TJH_OK;
  TJH_ARG(params && grads && exp_avg && exp_avg_sq && numels && steps,
          "tjh_adam_step: NULL array");
  AdamBatch B;
  B.b1 = (float)beta1;
  B.omb1 = (float)(1.0 - beta1);
  B.b2 = (float)beta2;
  B.omb2 = (float)(1.0 - beta2);
  B.eps = (float)eps;
  B.wd = (float)weight_decay;
  B.decay = 1.0 - lr * weight_decay;
  B.decoupled = decoupled ? 1 : 0;
  KernelScope ks("adam");
  int i = 0;
  while (i < n_tensors) {
    B.count = 0;
    int64_t blocks = 0;
    while (i < n_tensors && B.count < kMaxTensors) {
      TJH_ARG(numels[i] >= 0 && steps[i] >= 1, "tjh_adam_step: bad numel/step for tensor %d", i);
      if (numels[i] == 0) { ++i; continue; }
      AdamTensor& T = B.t[B.count];
      T.p = params[i];
      T.g = grads[i];
      T.m = exp_avg[i];
      T.v = exp_avg_sq[i];
      T.n = numels[i];
      T.first_block = blocks;
      double bc1 = 1.0 - pow(beta1, (double)steps[i]);
      double bc2 = 1.0 - pow(beta2, (double)steps[i]);
      T.step_size = lr / bc1;
      T.bc2 = (float)bc2;
      T.vec = (T.n % 4 == 0) && aligned16(T.p) && aligned16(T.g) && aligned16(T.m) &&
              aligned16(T.v);
      blocks += cdiv(T.n, kChunk);
      ++B.count;
      ++i;
    }
    if (B.count == 0) break;
    TJH_ARG(blocks < (int64_t(1) << 31), "tjh_adam_step: tensors too large");
    tjh_launch(k_adam, dim3((unsigned)blocks), dim3(kBlock), 0, stream(), B);
    int rc = check_launch("adam_step");
    if (rc != TJH_OK) return rc;
  }
  return TJH_OK;
}
