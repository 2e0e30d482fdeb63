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

#include <math.h>
#include <string.h>

#include <map>
#include <mutex>
#include <tuple>
#include <vector>

namespace tjh {
namespace {

constexpr int kBlock = 256;
constexpr int kMaxTensors = 48;  // keeps the kernel argument block under 4 KiB
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
  int64_t* step;        // device step counter (capturable steps), else null
};

struct AdamBatch {  // passed by value: must stay within the 4 KiB kernel argument block
  AdamTensor t[kMaxTensors];
  int count;
  float b1, omb1, b2, omb2, eps, wd;  // fp32 scalars as torch.js's tensor ops see them
  double decay;                        // 1 - lr*wd (AdamW)
  int decoupled;
  // capturable steps: per-step lr/bc1 and f32(bc2), from the host's pow,
  // for steps 1..tlen; later steps have bc1 = bc2 = 1 exactly
  const double* sz_table;
  const float* bc2_table;
  int64_t tlen;
  double lr;
};
static_assert(sizeof(AdamBatch) <= 4000, "AdamBatch exceeds the kernel argument block");


// Every fp32 operation is rounded on its own (contraction off; IEEE
// division and the correctly rounded llvm.sqrt), as the reference's
// separate tensor ops round them.
__device__ __forceinline__ void adam_elem(float& p, float g, float& m, float& v,
                                          const AdamBatch& B, double step_size, float bc2) {
#pragma clang fp contract(off)
  if (!B.decoupled && B.wd != 0.f) g = g + p * B.wd;
  m = m * B.b1 + g * B.omb1;
  v = v * B.b2 + (g * g) * B.omb2;
  float denom = __builtin_sqrtf(v / bc2) + B.eps;
  double pd = (double)p;
  if (B.decoupled) pd = pd * B.decay;
  pd = pd - step_size * ((double)m / (double)denom);
  p = (float)pd;
}

// Capturable steps: every tensor's device step counter advances by one
// before the update reads it (one lane per tensor of the batch).
__global__ __launch_bounds__(64) void k_adam_tick(AdamBatch B) {
  const int i = threadIdx.x;
  if (i < B.count && B.t[i].step) B.t[i].step[0] += 1;
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
  double step_size = T.step_size;
  float bc2 = T.bc2;
  if (T.step) {
    const int64_t s = T.step[0];
    step_size = s <= B.tlen ? B.sz_table[s - 1] : B.lr;
    bc2 = s <= B.tlen ? B.bc2_table[s - 1] : 1.0f;
  }
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
        adam_elem(p[u].x, g[u].x, m[u].x, v[u].x, B, step_size, bc2);
        adam_elem(p[u].y, g[u].y, m[u].y, v[u].y, B, step_size, bc2);
        adam_elem(p[u].z, g[u].z, m[u].z, v[u].z, B, step_size, bc2);
        adam_elem(p[u].w, g[u].w, m[u].w, v[u].w, B, step_size, bc2);
        st_nt(T.p + i, p[u]);
        st_nt(T.m + i, m[u]);
        st_nt(T.v + i, v[u]);
      }
    }
  } else {
    for (int64_t i = beg + threadIdx.x; i < end; i += kBlock) {
      float p = T.p[i], m = T.m[i], v = T.v[i];
      adam_elem(p, T.g[i], m, v, B, step_size, bc2);
      T.p[i] = p;
      T.m[i] = m;
      T.v[i] = v;
    }
  }
}

}  // namespace
}  // namespace tjh

using namespace tjh;

namespace {

struct AdamTable {
  double* sz = nullptr;
  float* bc2 = nullptr;
  int64_t len = 0;
};

std::mutex g_table_mu;
std::map<std::tuple<uint64_t, uint64_t, uint64_t>, AdamTable>& adam_tables() {
  static auto* t = new std::map<std::tuple<uint64_t, uint64_t, uint64_t>, AdamTable>();
  return *t;
}

uint64_t bits_of(double d) {
  uint64_t u;
  memcpy(&u, &d, sizeof u);
  return u;
}

// Steps after which 1 - beta^step is 1.0 in double (beta^step < 2^-54).
int64_t table_len(double b) {
  if (!(b > 0.0 && b < 1.0)) return 1;
  return (int64_t)ceil(56.0 / -log2(b)) + 1;
}

// The bias-correction table for (lr, beta1, beta2), made on first use with
// the same host arithmetic as the host-stepped path.
int get_table(double lr, double beta1, double beta2, AdamTable* out) {
  const auto key = std::make_tuple(bits_of(lr), bits_of(beta1), bits_of(beta2));
  std::lock_guard<std::mutex> lk(g_table_mu);
  auto it = adam_tables().find(key);
  if (it != adam_tables().end()) {
    *out = it->second;
    return TJH_OK;
  }
  if (capturing())
    return set_error(TJH_ERR_UNSUPPORTED,
                     "tjh_adam_step_dev: take one step before capturing a graph (its tables are "
                     "uploaded on first use)");
  int64_t len = table_len(beta1);
  if (table_len(beta2) > len) len = table_len(beta2);
  TJH_ARG(len <= (int64_t(1) << 24), "tjh_adam_step_dev: betas too close to 1");
  std::vector<double> sz((size_t)len);
  std::vector<float> bc((size_t)len);
  for (int64_t s = 1; s <= len; ++s) {
    const double bc1 = 1.0 - pow(beta1, (double)s);
    const double bc2 = 1.0 - pow(beta2, (double)s);
    sz[(size_t)(s - 1)] = lr / bc1;
    bc[(size_t)(s - 1)] = (float)bc2;
  }
  AdamTable t;
  t.len = len;
  void* a = nullptr;
  void* b = nullptr;
  int rc = tjh_malloc((size_t)len * sizeof(double), &a);
  if (rc == TJH_OK) rc = tjh_malloc((size_t)len * sizeof(float), &b);
  if (rc == TJH_OK) rc = tjh_h2d(a, sz.data(), (size_t)len * sizeof(double));
  if (rc == TJH_OK) rc = tjh_h2d(b, bc.data(), (size_t)len * sizeof(float));
  if (rc != TJH_OK) return rc;
  t.sz = (double*)a;
  t.bc2 = (float*)b;
  adam_tables()[key] = t;
  *out = t;
  return TJH_OK;
}

int adam_impl(int n_tensors, float* const* params, const float* const* grads,
              float* const* exp_avg, float* const* exp_avg_sq, const int64_t* numels,
              const int64_t* steps, int64_t* const* dev_steps, double lr, double beta1,
              double beta2, double eps, double weight_decay, int decoupled) {
  AdamBatch B;
  B.b1 = (float)beta1;
  B.omb1 = (float)(1.0 - beta1);
  B.b2 = (float)beta2;
  B.omb2 = (float)(1.0 - beta2);
  B.eps = (float)eps;
  B.wd = (float)weight_decay;
  B.decay = 1.0 - lr * weight_decay;
  B.decoupled = decoupled ? 1 : 0;
  B.lr = lr;
  B.sz_table = nullptr;
  B.bc2_table = nullptr;
  B.tlen = 0;
  if (dev_steps) {
    AdamTable t;
    const int rc = get_table(lr, beta1, beta2, &t);
    if (rc != TJH_OK) return rc;
    B.sz_table = t.sz;
    B.bc2_table = t.bc2;
    B.tlen = t.len;
  }
  KernelScope ks("adam");
  int i = 0;
  while (i < n_tensors) {
    B.count = 0;
    int64_t blocks = 0;
    while (i < n_tensors && B.count < kMaxTensors) {
      TJH_ARG(numels[i] >= 0, "tjh_adam_step: bad numel for tensor %d", i);
      TJH_ARG(dev_steps ? dev_steps[i] != nullptr : steps[i] >= 1,
              "tjh_adam_step: bad step for tensor %d", i);
      if (numels[i] == 0) { ++i; continue; }
      AdamTensor& T = B.t[B.count];
      T.p = params[i];
      T.g = grads[i];
      T.m = exp_avg[i];
      T.v = exp_avg_sq[i];
      T.n = numels[i];
      T.first_block = blocks;
      T.step = dev_steps ? dev_steps[i] : nullptr;
      if (!dev_steps) {
        double bc1 = 1.0 - pow(beta1, (double)steps[i]);
        double bc2 = 1.0 - pow(beta2, (double)steps[i]);
        T.step_size = lr / bc1;
        T.bc2 = (float)bc2;
      } else {
        T.step_size = 0.0;
        T.bc2 = 1.0f;
      }
      T.vec = (T.n % 4 == 0) && aligned16(T.p) && aligned16(T.g) && aligned16(T.m) &&
              aligned16(T.v);
      blocks += cdiv(T.n, kChunk);
      ++B.count;
      ++i;
    }
    if (B.count == 0) break;
    TJH_ARG(blocks < (int64_t(1) << 31), "tjh_adam_step: tensors too large");
    if (dev_steps) {
      tjh_launch(k_adam_tick, dim3(1), dim3(64), 0, stream(), B);
      int rc = check_launch("adam_tick");
      if (rc != TJH_OK) return rc;
    }
    tjh_launch(k_adam, dim3((unsigned)blocks), dim3(kBlock), 0, stream(), B);
    int rc = check_launch("adam_step");
    if (rc != TJH_OK) return rc;
  }
  return TJH_OK;
}

}  // namespace

extern "C" int tjh_adam_step(int n_tensors, float* const* params, const float* const* grads,
                             float* const* exp_avg, float* const* exp_avg_sq,
                             const int64_t* numels, const int64_t* steps, double lr, double beta1,
                             double beta2, double eps, double weight_decay, int decoupled) {
  TJH_REQUIRE_INIT();
  TJH_ARG(n_tensors >= 0, "tjh_adam_step: negative tensor count");
  if (n_tensors == 0) return TJH_OK;
  TJH_ARG(params && grads && exp_avg && exp_avg_sq && numels && steps,
          "tjh_adam_step: NULL array");
  return adam_impl(n_tensors, params, grads, exp_avg, exp_avg_sq, numels, steps, nullptr, lr,
                   beta1, beta2, eps, weight_decay, decoupled);
}

extern "C" int tjh_adam_step_dev(int n_tensors, float* const* params, const float* const* grads,
                                 float* const* exp_avg, float* const* exp_avg_sq,
                                 const int64_t* numels, int64_t* const* steps, double lr,
                                 double beta1, double beta2, double eps, double weight_decay,
                                 int decoupled) {
  TJH_REQUIRE_INIT();
  TJH_ARG(n_tensors >= 0, "tjh_adam_step_dev: negative tensor count");
  if (n_tensors == 0) return TJH_OK;
  TJH_ARG(params && grads && exp_avg && exp_avg_sq && numels && steps,
          "tjh_adam_step_dev: NULL array");
  return adam_impl(n_tensors, params, grads, exp_avg, exp_avg_sq, numels, nullptr, steps, lr,
                   beta1, beta2, eps, weight_decay, decoupled);
}
