// Scaled dot-product attention forward / backward.
//
// Reference: F.scaled_dot_product_attention (src/nn/functional.ts:866-890:
// softmax(Q K^T * scale) V, with is_causal ignored there) and
// MultiheadAttention.forward (src/nn/attention.ts:112-271).  The contract
// implemented is torch's: optional causal mask (key j > query i masked,
// top-left aligned), lse saved for the backward.
//
// Head dims up to 128 that are multiples of 4, with D-contiguous, 16-byte
// aligned rows, run the flash kernels of flash.hip.  Any other shape takes
// the GEMM-composed path below, per batch item: S = scale * Q K^T on the
// MFMA GEMM (all heads of one batch item in one batched launch), a fused
// masked softmax that also writes lse, then O = P V.  The backward
// recomputes P from lse and issues dV = P^T dO, dP = dO V^T,
// dS = P * (dP - rowsum(dO * O)) * scale, dQ = dS K, dK = dS^T Q.
// Scratch holds [H, Tq, Tk] scores for ONE batch item at a time.

#include "common.h"
#include "wave.h"

#include <float.h>

namespace tjh {
namespace {

constexpr int kBlock = 256;


// In place: S (already scaled) -> P, lse[row] written.  Row r of [H*Tq]
// has query index i = r % Tq; with causal only cols j <= i are valid.
// One wave per row.
__global__ __launch_bounds__(kBlock) void k_attn_softmax(float* __restrict__ S, int64_t rows,
                                                         int64_t Tq, int64_t Tk, int causal,
                                                         float* __restrict__ lse) {
  int64_t r = (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (r >= rows) return;
  int64_t i = r % Tq;
  int64_t valid = causal ? (i + 1 < Tk ? i + 1 : Tk) : Tk;
  float* row = S + r * Tk;
  float m = -FLT_MAX;
  for (int64_t j = lane; j < valid; j += 64) m = fmaxf(m, row[j]);
  m = wave_max(m);
  float s = 0.f;
  for (int64_t j = lane; j < valid; j += 64) s += __expf(row[j] - m);
  s = wave_sum(s);
  float inv = 1.0f / s;
  for (int64_t j = lane; j < Tk; j += 64) row[j] = j < valid ? __expf(row[j] - m) * inv : 0.f;
  if (lane == 0) lse[r] = m + logf(s);
}

// In place: S (scaled scores) -> P = exp(S - lse), 0 where masked.
__global__ __launch_bounds__(kBlock) void k_attn_p(float* __restrict__ S, int64_t rows, int64_t Tq,
                                                   int64_t Tk, int causal,
                                                   const float* __restrict__ lse) {
  int64_t r = (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (r >= rows) return;
  int64_t i = r % Tq;
  int64_t valid = causal ? (i + 1 < Tk ? i + 1 : Tk) : Tk;
  float* row = S + r * Tk;
  float l = lse[r];
  for (int64_t j = lane; j < Tk; j += 64) row[j] = j < valid ? __expf(row[j] - l) : 0.f;
}

// D[h, i] = sum_d dO[h,i,d] * O[h,i,d] for one batch item (strided heads).
__global__ __launch_bounds__(kBlock) void k_attn_rowdot(const float* __restrict__ dO,
                                                        const float* __restrict__ O, int64_t H,
                                                        int64_t Tq, int64_t D, int64_t g_sh,
                                                        int64_t g_st, int64_t o_sh, int64_t o_st,
                                                        float* __restrict__ Dout) {
  int64_t r = (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (r >= H * Tq) return;
  int64_t h = r / Tq, i = r % Tq;
  const float* a = dO + h * g_sh + i * g_st;
  const float* b = O + h * o_sh + i * o_st;
  float s = 0.f;
  for (int64_t d = lane; d < D; d += 64) s += a[d] * b[d];
  s = wave_sum(s);
  if (lane == 0) Dout[r] = s;
}

// In place: dP -> dS = P * (dP - D[row]) * scale.
__global__ __launch_bounds__(kBlock) void k_attn_ds(const float* __restrict__ P,
                                                    float* __restrict__ dP, int64_t rows,
                                                    int64_t Tk, const float* __restrict__ Drow,
                                                    float scale) {
  int64_t r = (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (r >= rows) return;
  float dd = Drow[r];
  const float* p = P + r * Tk;
  float* g = dP + r * Tk;
  for (int64_t j = lane; j < Tk; j += 64) g[j] = p[j] * (g[j] - dd) * scale;
}

}  // namespace
}  // namespace tjh

using namespace tjh;

extern "C" {

int tjh_sdpa_forward(const float* q, const float* k, const float* v, float* o, float* lse,
                     int64_t B, int64_t H, int64_t Tq, int64_t Tk, int64_t D,
                     const int64_t* qs, const int64_t* ks, const int64_t* vs, const int64_t* os,
                     float scale, int causal) {
  TJH_REQUIRE_INIT();
  TJH_ARG(B >= 0 && H >= 0 && Tq >= 0 && Tk >= 0 && D > 0, "tjh_sdpa_forward: bad sizes");
  TJH_ARG(qs && ks && vs && os, "tjh_sdpa_forward: NULL strides");
  if (B == 0 || H == 0 || Tq == 0) return TJH_OK;
  TJH_ARG(Tk > 0, "tjh_sdpa_forward: empty key sequence");
  {
    const void* ptrs[4] = {q, k, v, o};
    const int64_t* sts[4] = {qs, ks, vs, os};
    if (flash_supported(D, ptrs, sts, 4))
      return flash_forward(q, k, v, o, lse, B, H, Tq, Tk, D, qs, ks, vs, os, scale, causal);
  }
  Scratch S((size_t)(H * Tq * Tk) * sizeof(float));
  if (!S.ok()) return set_error(TJH_ERR_OOM, "sdpa_forward: no scratch for scores");
  float* s = S.as<float>();
  KernelScope kscope("sdpa_fwd_composite");
  for (int64_t b = 0; b < B; ++b) {
    int rc = gemm("sdpa.gemm", 0, 1, Tq, Tk, D, scale, q + b * qs[0], qs[2], qs[1], k + b * ks[0], ks[2],
                      ks[1], 0.f, s, Tk, Tq * Tk, H, nullptr, 0);
    if (rc != TJH_OK) return rc;
    tjh_launch(k_attn_softmax, dim3((unsigned)cdiv(H * Tq, 4)), dim3(kBlock), 0, stream(),
                       s, H * Tq, Tq, Tk, causal, lse + b * H * Tq);
    rc = check_launch("sdpa_softmax");
    if (rc != TJH_OK) return rc;
    rc = gemm("sdpa.gemm", 0, 0, Tq, D, Tk, 1.f, s, Tk, Tq * Tk, v + b * vs[0], vs[2], vs[1], 0.f,
                  o + b * os[0], os[2], os[1], H, nullptr, 0);
    if (rc != TJH_OK) return rc;
  }
  return TJH_OK;
}

int tjh_sdpa_backward(const float* q, const float* k, const float* v, const float* o,
                      const float* do_, const float* lse, float* dq, float* dk, float* dv,
                      int64_t B, int64_t H, int64_t Tq, int64_t Tk, int64_t D,
                      const int64_t* const* strides, float scale, int causal) {
  TJH_REQUIRE_INIT();
  TJH_ARG(B >= 0 && H >= 0 && Tq >= 0 && Tk >= 0 && D > 0, "tjh_sdpa_backward: bad sizes");
  TJH_ARG(strides, "tjh_sdpa_backward: NULL strides");
  for (int i = 0; i < 8; ++i) TJH_ARG(strides[i], "tjh_sdpa_backward: NULL strides[%d]", i);
  const int64_t *qs = strides[0], *ks = strides[1], *vs = strides[2], *os = strides[3],
                *gs = strides[4], *dqs = strides[5], *dks = strides[6], *dvs = strides[7];
  if (B == 0 || H == 0) return TJH_OK;
  if (Tq == 0 || Tk == 0) return TJH_OK;
  {
    const void* ptrs[8] = {q, k, v, o, do_, dq, dk, dv};
    if (flash_supported(D, ptrs, strides, 8))
      return flash_backward(q, k, v, o, do_, lse, dq, dk, dv, B, H, Tq, Tk, D, strides, scale,
                            causal);
  }
  Scratch Ps((size_t)(H * Tq * Tk) * sizeof(float));
  Scratch dPs((size_t)(H * Tq * Tk) * sizeof(float));
  Scratch Ds((size_t)(H * Tq) * sizeof(float));
  if (!Ps.ok() || !dPs.ok() || !Ds.ok()) return set_error(TJH_ERR_OOM, "sdpa_backward: no scratch");
  float* P = Ps.as<float>();
  float* dP = dPs.as<float>();
  float* Dr = Ds.as<float>();
  KernelScope kscope("sdpa_bwd_composite");
  unsigned grows = (unsigned)cdiv(H * Tq, 4);
  for (int64_t b = 0; b < B; ++b) {
    const float* qb = q + b * qs[0];
    const float* kb = k + b * ks[0];
    const float* vb = v + b * vs[0];
    const float* ob = o + b * os[0];
    const float* gb = do_ + b * gs[0];
    // P = exp(scale * Q K^T - lse)
    int rc = gemm("sdpa.gemm", 0, 1, Tq, Tk, D, scale, qb, qs[2], qs[1], kb, ks[2], ks[1], 0.f, P, Tk,
                      Tq * Tk, H, nullptr, 0);
    if (rc != TJH_OK) return rc;
    tjh_launch(k_attn_p, dim3(grows), dim3(kBlock), 0, stream(), P, H * Tq, Tq, Tk, causal,
                       lse + b * H * Tq);
    if ((rc = check_launch("sdpa_p")) != TJH_OK) return rc;
    // dV = P^T dO
    rc = gemm("sdpa.gemm", 1, 0, Tk, D, Tq, 1.f, P, Tk, Tq * Tk, gb, gs[2], gs[1], 0.f, dv + b * dvs[0],
                  dvs[2], dvs[1], H, nullptr, 0);
    if (rc != TJH_OK) return rc;
    // dP = dO V^T
    rc = gemm("sdpa.gemm", 0, 1, Tq, Tk, D, 1.f, gb, gs[2], gs[1], vb, vs[2], vs[1], 0.f, dP, Tk, Tq * Tk, H,
                  nullptr, 0);
    if (rc != TJH_OK) return rc;
    // D = rowsum(dO * O); dS = P * (dP - D) * scale
    tjh_launch(k_attn_rowdot, dim3(grows), dim3(kBlock), 0, stream(), gb, ob, H, Tq, D,
                       gs[1], gs[2], os[1], os[2], Dr);
    tjh_launch(k_attn_ds, dim3(grows), dim3(kBlock), 0, stream(), P, dP, H * Tq, Tk, Dr,
                       scale);
    if ((rc = check_launch("sdpa_ds")) != TJH_OK) return rc;
    // dQ = dS K ; dK = dS^T Q
    rc = gemm("sdpa.gemm", 0, 0, Tq, D, Tk, 1.f, dP, Tk, Tq * Tk, kb, ks[2], ks[1], 0.f, dq + b * dqs[0],
                  dqs[2], dqs[1], H, nullptr, 0);
    if (rc != TJH_OK) return rc;
    rc = gemm("sdpa.gemm", 1, 0, Tk, D, Tq, 1.f, dP, Tk, Tq * Tk, qb, qs[2], qs[1], 0.f, dk + b * dks[0],
                  dks[2], dks[1], H, nullptr, 0);
    if (rc != TJH_OK) return rc;
  }
  return TJH_OK;
}

}  // extern "C"
