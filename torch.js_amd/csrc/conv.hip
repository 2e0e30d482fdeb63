// conv2d forward / input-gradient / weight-gradient, NCHW, with stride,
// padding, dilation and groups.
//
// Reference: F.conv2d (src/nn/functional.ts:438-660) over conv.wgsl:25-60
// (one thread per output, 27- or 288-deep serial dot products) and
// conv_backward.wgsl:24-119 (never reached, the grad_fn is dropped by the
// autograd walk).  The reference ignores dilation (written into the pad
// slot); the contract implemented here is torch's.
//
// All three products run on the MFMA GEMM over an im2col matrix
// col[(c*KH + kh)*KW + kw][n*OH*OW + p] (one column per output pixel of
// every image, so the weight gradient is ONE GEMM with K = N*OH*OW that
// the GEMM splits over workgroups):
//   forward : y[n]  = W_g . col_g[:, n]          (batched over images)
//   dgrad   : dcol  = W_g^T . dy[n]   then col2im gathers (deterministic)
//   wgrad   : dW_g  = dy_g^T-layout . col_g^T    (dy permuted to [OC, N*P])

#include "common.h"

namespace tjh {
namespace {

constexpr int kBlock = 256;

struct ConvGeo {
  int64_t n, c, h, w, oc, kh, kw, sh, sw, ph, pw, dh, dw, groups, oh, ow;
};

ConvGeo geo(const tjh_conv2d_desc* d) {
  return ConvGeo{d->n, d->c, d->h, d->w, d->oc, d->kh, d->kw, d->stride_h, d->stride_w,
                 d->pad_h, d->pad_w, d->dil_h, d->dil_w, d->groups, d->oh, d->ow};
}

// col[(c*KH+kh)*KW+kw][n*P + p] = x[n][c][oh*sh - ph + kh*dh][ow*sw - pw + kw*dw]
__global__ __launch_bounds__(kBlock) void k_im2col(const float* __restrict__ x, ConvGeo g,
                                                   float* __restrict__ col) {
  const int64_t P = g.oh * g.ow;
  const int64_t ncol = g.n * P;
  const int64_t total = g.c * g.kh * g.kw * ncol;
  int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x; e < total; e += stride) {
    int64_t j = e % ncol;
    int64_t row = e / ncol;
    int64_t kw = row % g.kw;
    int64_t kh = (row / g.kw) % g.kh;
    int64_t c = row / (g.kw * g.kh);
    int64_t n = j / P, p = j % P;
    int64_t oy = p / g.ow, ox = p % g.ow;
    int64_t iy = oy * g.sh - g.ph + kh * g.dh;
    int64_t ix = ox * g.sw - g.pw + kw * g.dw;
    float v = 0.f;
    if (iy >= 0 && iy < g.h && ix >= 0 && ix < g.w) v = x[((n * g.c + c) * g.h + iy) * g.w + ix];
    col[e] = v;
  }
}

// dx[n][c][iy][ix] = sum over (kh, kw) hitting an output pixel of dcol.
__global__ __launch_bounds__(kBlock) void k_col2im(const float* __restrict__ dcol, ConvGeo g,
                                                   float* __restrict__ dx) {
  const int64_t P = g.oh * g.ow;
  const int64_t ncol = g.n * P;
  const int64_t total = g.n * g.c * g.h * g.w;
  int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x; e < total; e += stride) {
    int64_t ix = e % g.w;
    int64_t iy = (e / g.w) % g.h;
    int64_t c = (e / (g.w * g.h)) % g.c;
    int64_t n = e / (g.w * g.h * g.c);
    float acc = 0.f;
    for (int64_t kh = 0; kh < g.kh; ++kh) {
      int64_t ty = iy + g.ph - kh * g.dh;
      if (ty < 0 || ty % g.sh) continue;
      int64_t oy = ty / g.sh;
      if (oy >= g.oh) continue;
      for (int64_t kw = 0; kw < g.kw; ++kw) {
        int64_t tx = ix + g.pw - kw * g.dw;
        if (tx < 0 || tx % g.sw) continue;
        int64_t ox = tx / g.sw;
        if (ox >= g.ow) continue;
        int64_t row = (c * g.kh + kh) * g.kw + kw;
        acc += dcol[row * ncol + n * P + oy * g.ow + ox];
      }
    }
    dx[e] = acc;
  }
}

int grid_for(int64_t n) {
  int64_t g = cdiv(n, kBlock);
  int64_t cap = (int64_t)(num_cus() > 0 ? num_cus() : 256) * 16;
  if (g > cap) g = cap;
  return (int)(g < 1 ? 1 : g);
}

int check_desc(const tjh_conv2d_desc* d) {
  TJH_ARG(d, "conv2d: NULL descriptor");
  TJH_ARG(d->n >= 0 && d->c > 0 && d->h >= 0 && d->w >= 0 && d->oc > 0 && d->kh > 0 && d->kw > 0,
          "conv2d: bad sizes");
  TJH_ARG(d->stride_h > 0 && d->stride_w > 0 && d->dil_h > 0 && d->dil_w > 0 && d->pad_h >= 0 &&
              d->pad_w >= 0 && d->groups > 0,
          "conv2d: bad stride/dilation/padding/groups");
  TJH_ARG(d->c % d->groups == 0 && d->oc % d->groups == 0,
          "conv2d: channels (%lld in, %lld out) not divisible by groups %lld", (long long)d->c,
          (long long)d->oc, (long long)d->groups);
  int64_t oh = (d->h + 2 * d->pad_h - d->dil_h * (d->kh - 1) - 1) / d->stride_h + 1;
  int64_t ow = (d->w + 2 * d->pad_w - d->dil_w * (d->kw - 1) - 1) / d->stride_w + 1;
  TJH_ARG(oh == d->oh && ow == d->ow, "conv2d: output size %lldx%lld does not match %lldx%lld",
          (long long)d->oh, (long long)d->ow, (long long)oh, (long long)ow);
  TJH_ARG(oh > 0 && ow > 0, "conv2d: empty output");
  return TJH_OK;
}

}  // namespace
}  // namespace tjh

using namespace tjh;

extern "C" {

int tjh_conv2d_forward(const tjh_conv2d_desc* d, const float* x, const float* w,
                       const float* bias, float* y) {
  TJH_REQUIRE_INIT();
  int rc = check_desc(d);
  if (rc != TJH_OK) return rc;
  ConvGeo g = geo(d);
  if (g.n == 0) return TJH_OK;
  const int64_t P = g.oh * g.ow, ncol = g.n * P;
  const int64_t cg = g.c / g.groups, ocg = g.oc / g.groups, kk = g.kh * g.kw;
  Scratch col((size_t)(g.c * kk * ncol) * sizeof(float));
  if (!col.ok()) return set_error(TJH_ERR_OOM, "conv2d_forward: no im2col scratch");
  KernelScope ks("conv2d_fwd");
  int64_t total = g.c * kk * ncol;
  hipLaunchKernelGGL(k_im2col, dim3(grid_for(total)), dim3(kBlock), 0, stream(), x, g,
                     col.as<float>());
  if ((rc = check_launch("im2col")) != TJH_OK) return rc;
  for (int64_t gi = 0; gi < g.groups; ++gi) {
    // y[n][gi*ocg + o][p] = sum_r W[gi*ocg + o][r] * col[gi*cg*kk + r][n*P + p]
    rc = gemm("conv.gemm", 0, 0, ocg, P, cg * kk, 1.f, w + gi * ocg * cg * kk, cg * kk, 0,
                  col.as<float>() + gi * cg * kk * ncol, ncol, P, 0.f, y + gi * ocg * P, P,
                  g.oc * P, g.n, bias ? bias + gi * ocg : nullptr, bias ? 2 : 0);
    if (rc != TJH_OK) return rc;
  }
  return TJH_OK;
}

int tjh_conv2d_backward_input(const tjh_conv2d_desc* d, const float* dy, const float* w,
                              float* dx) {
  TJH_REQUIRE_INIT();
  int rc = check_desc(d);
  if (rc != TJH_OK) return rc;
  ConvGeo g = geo(d);
  if (g.n == 0) return TJH_OK;
  const int64_t P = g.oh * g.ow, ncol = g.n * P;
  const int64_t cg = g.c / g.groups, ocg = g.oc / g.groups, kk = g.kh * g.kw;
  Scratch dcol((size_t)(g.c * kk * ncol) * sizeof(float));
  if (!dcol.ok()) return set_error(TJH_ERR_OOM, "conv2d_backward_input: no scratch");
  KernelScope ks("conv2d_dgrad");
  for (int64_t gi = 0; gi < g.groups; ++gi) {
    // dcol[gi*cg*kk + r][n*P + p] = sum_o W[gi*ocg + o][r] * dy[n][gi*ocg + o][p]
    rc = gemm("conv.gemm", 1, 0, cg * kk, P, ocg, 1.f, w + gi * ocg * cg * kk, cg * kk, 0,
                  dy + gi * ocg * P, P, g.oc * P, 0.f, dcol.as<float>() + gi * cg * kk * ncol,
                  ncol, P, g.n, nullptr, 0);
    if (rc != TJH_OK) return rc;
  }
  int64_t total = g.n * g.c * g.h * g.w;
  hipLaunchKernelGGL(k_col2im, dim3(grid_for(total)), dim3(kBlock), 0, stream(), dcol.as<float>(),
                     g, dx);
  return check_launch("col2im");
}

int tjh_conv2d_backward_weight(const tjh_conv2d_desc* d, const float* dy, const float* x,
                               float* dw, int accumulate) {
  TJH_REQUIRE_INIT();
  int rc = check_desc(d);
  if (rc != TJH_OK) return rc;
  ConvGeo g = geo(d);
  const int64_t cg = g.c / g.groups, ocg = g.oc / g.groups, kk = g.kh * g.kw;
  if (g.n == 0) {
    if (!accumulate) return tjh_fill_f32(dw, g.oc * cg * kk, 0.f);
    return TJH_OK;
  }
  const int64_t P = g.oh * g.ow, ncol = g.n * P;
  Scratch col((size_t)(g.c * kk * ncol) * sizeof(float));
  Scratch dyt((size_t)(g.oc * ncol) * sizeof(float));
  if (!col.ok() || !dyt.ok()) return set_error(TJH_ERR_OOM, "conv2d_backward_weight: no scratch");
  KernelScope ks("conv2d_wgrad");
  int64_t total = g.c * kk * ncol;
  hipLaunchKernelGGL(k_im2col, dim3(grid_for(total)), dim3(kBlock), 0, stream(), x, g,
                     col.as<float>());
  if ((rc = check_launch("im2col")) != TJH_OK) return rc;
  // dyt[o][n][p] = dy[n][o][p]
  int64_t shape[3] = {g.oc, g.n, P};
  int64_t sst[3] = {P, g.oc * P, 1};
  int64_t dst[3] = {g.n * P, P, 1};
  rc = tjh_copy_strided(3, shape, dy, sst, dyt.as<float>(), dst);
  if (rc != TJH_OK) return rc;
  for (int64_t gi = 0; gi < g.groups; ++gi) {
    // dW[gi*ocg + o][r] (+)= sum_j dyt[gi*ocg + o][j] * col[gi*cg*kk + r][j]
    rc = gemm("conv.gemm", 0, 1, ocg, cg * kk, ncol, 1.f, dyt.as<float>() + gi * ocg * ncol, ncol, 0,
                  col.as<float>() + gi * cg * kk * ncol, ncol, 0, accumulate ? 1.f : 0.f,
                  dw + gi * ocg * cg * kk, cg * kk, 0, 1, nullptr, 0);
    if (rc != TJH_OK) return rc;
  }
  return TJH_OK;
}

}  // extern "C"
