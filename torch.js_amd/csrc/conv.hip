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
// Grid (ceil(P/256), C*KH*KW, N): the patch row (c, kh, kw) and the image
// are per-workgroup constants, threads walk output pixels p (coalesced
// writes; coalesced reads along ox for unit stride).
__global__ __launch_bounds__(kBlock) void k_im2col(const float* __restrict__ x, ConvGeo g,
                                                   float* __restrict__ col) {
  const int P = (int)(g.oh * g.ow);
  const int p = blockIdx.x * kBlock + threadIdx.x;
  if (p >= P) return;
  const int row = blockIdx.y, n = blockIdx.z;
  const int kw = row % (int)g.kw;
  const int kh = (row / (int)g.kw) % (int)g.kh;
  const int c = row / (int)(g.kw * g.kh);
  const int oy = p / (int)g.ow, ox = p - oy * (int)g.ow;
  const int iy = oy * (int)g.sh - (int)g.ph + kh * (int)g.dh;
  const int ix = ox * (int)g.sw - (int)g.pw + kw * (int)g.dw;
  float v = 0.f;
  if (iy >= 0 && iy < g.h && ix >= 0 && ix < g.w)
    v = x[(((int64_t)n * g.c + c) * g.h + iy) * g.w + ix];
  col[(int64_t)row * (g.n * P) + (int64_t)n * P + p] = v;
}

// dx[n][c][iy][ix] = sum over (kh, kw) hitting an output pixel of dcol.
// Grid (ceil(H*W/256), C, N).
__global__ __launch_bounds__(kBlock) void k_col2im(const float* __restrict__ dcol, ConvGeo g,
                                                   float* __restrict__ dx) {
  const int HW = (int)(g.h * g.w);
  const int e = blockIdx.x * kBlock + threadIdx.x;
  if (e >= HW) return;
  const int c = blockIdx.y, n = blockIdx.z;
  const int iy = e / (int)g.w, ix = e - iy * (int)g.w;
  const int64_t P = g.oh * g.ow, ncol = g.n * P;
  const float* __restrict__ base = dcol + (int64_t)n * P;
  float acc = 0.f;
  for (int kh = 0; kh < (int)g.kh; ++kh) {
    const int ty = iy + (int)g.ph - kh * (int)g.dh;
    if (ty < 0 || ty % (int)g.sh) continue;
    const int oy = ty / (int)g.sh;
    if (oy >= g.oh) continue;
    for (int kw = 0; kw < (int)g.kw; ++kw) {
      const int tx = ix + (int)g.pw - kw * (int)g.dw;
      if (tx < 0 || tx % (int)g.sw) continue;
      const int ox = tx / (int)g.sw;
      if (ox >= g.ow) continue;
      const int64_t row = ((int64_t)c * g.kh + kh) * g.kw + kw;
      acc += base[row * ncol + (int64_t)oy * g.ow + ox];
    }
  }
  dx[((int64_t)n * g.c + c) * HW + e] = acc;
}

int launch_im2col(const float* x, const ConvGeo& g, float* col) {
  hipLaunchKernelGGL(k_im2col, dim3((unsigned)cdiv(g.oh * g.ow, kBlock),
                                    (unsigned)(g.c * g.kh * g.kw), (unsigned)g.n),
                     dim3(kBlock), 0, stream(), x, g, col);
  return check_launch("im2col");
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
  TJH_ARG(d->h * d->w < (int64_t(1) << 30) && oh * ow < (int64_t(1) << 30) &&
              d->c * d->kh * d->kw <= 65535 && d->n <= 65535 && d->c <= 65535,
          "conv2d: sizes beyond this implementation's grid (C*KH*KW, N, C <= 65535)");
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
  rc = launch_im2col(x, g, col.as<float>());
  if (rc != TJH_OK) return rc;
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
  hipLaunchKernelGGL(k_col2im, dim3((unsigned)cdiv(g.h * g.w, kBlock), (unsigned)g.c,
                                     (unsigned)g.n), dim3(kBlock), 0, stream(), dcol.as<float>(), g, dx);
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
  rc = launch_im2col(x, g, col.as<float>());
  if (rc != TJH_OK) return rc;
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
