// Row-wise kernels over the last dimension: softmax / log_softmax forward
// and backward, fused cross-entropy forward and backward, nll_loss, and
// LayerNorm forward and backward.
//
// Reference semantics: log_softmax.wgsl:8-36 (max-subtracted),
// log_softmax_backward.wgsl:17-34, nll_loss(_backward).wgsl,
// src/nn/losses.ts:18-145 (cross_entropy = nll_loss(log_softmax)),
// layernorm.wgsl:14-42 (biased variance, eps inside the sqrt) and
// src/nn/layernorm.ts:25-119.  The reference evaluates a row with ONE
// thread; here a row is owned by a wave (short rows) or a workgroup (long
// rows such as the 50257-wide vocabulary) and combined with wave shuffles.
//
// Row access is 128-bit wherever the row start is 16-byte aligned; rows
// whose stride is odd (ld = 50257) peel a scalar prefix up to the next
// 16-byte boundary, stream float4s, and finish with a scalar tail.

#include "colsum.h"
#include "wave.h"

#include <vector>

#include <float.h>

namespace tjh {
namespace {

constexpr int kBlock = 256;
constexpr int kLnBwdWaves = 8;  // waves per k_ln_bwd_wave workgroup

// Online (max, sum-of-exp) pair.
struct MS {
  float m, s;
};
__device__ __forceinline__ MS ms_comb(MS a, MS b) {
  float m = fmaxf(a.m, b.m);
  if (m == -INFINITY) return MS{m, 0.f};
  return MS{m, a.s * __expf(a.m - m) + b.s * __expf(b.m - m)};
}
__device__ __forceinline__ MS ms_add(MS a, float x) {
  if (x > a.m) return MS{x, a.s * __expf(a.m - x) + 1.0f};
  // a -inf element adds exp(-inf) = 0 (with a.m = -inf too, x - a.m would
  // be NaN); NaN still propagates through the last line
  if (x == -INFINITY) return a;
  return MS{a.m, a.s + __expf(x - a.m)};
}
template <int CTRL>
__device__ __forceinline__ MS ms_dpp(MS v) {
  return ms_comb(v, MS{dpp_f<CTRL>(v.m), dpp_f<CTRL>(v.s)});
}
// The pair over the wave through the DPP network (wave.h), every lane.
__device__ __forceinline__ MS wave_ms(MS v) {
  v = ms_dpp<kDppXor1>(v);
  v = ms_dpp<kDppXor2>(v);
  v = ms_dpp<kDppRor4>(v);
  v = ms_dpp<kDppRor8>(v);
  const MS a = ms_comb(MS{lane_f(v.m, 0), lane_f(v.s, 0)}, MS{lane_f(v.m, 16), lane_f(v.s, 16)});
  const MS b = ms_comb(MS{lane_f(v.m, 32), lane_f(v.s, 32)}, MS{lane_f(v.m, 48), lane_f(v.s, 48)});
  return ms_comb(a, b);
}

// Calls f(index, value) for every element of row[0..n) with 128-bit loads
// in the aligned middle.  `lane`/`nl` describe the participating lanes.
constexpr int kRowUnroll = 4;

template <class F>
__device__ __forceinline__ void row_scan(const float* __restrict__ row, int64_t n, int lane,
                                         int nl, F&& f) {
  int64_t pre = (int64_t)((16 - ((uintptr_t)row & 15)) & 15) / 4;
  if (((uintptr_t)row & 3) != 0) pre = n;  // not even float aligned: scalar
  if (pre > n) pre = n;
  for (int64_t i = lane; i < pre; i += nl) f(i, row[i]);
  int64_t n4 = (n - pre) / 4;
  const float4* p4 = reinterpret_cast<const float4*>(row + pre);
  // kRowUnroll float4 per lane are loaded before any is consumed
  for (int64_t i0 = lane; i0 < n4; i0 += (int64_t)nl * kRowUnroll) {
    float4 v[kRowUnroll];
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) {
      const int64_t i = i0 + (int64_t)u * nl;
      if (i < n4) v[u] = p4[i];
    }
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) {
      const int64_t i = i0 + (int64_t)u * nl;
      if (i < n4) {
        const int64_t b = pre + 4 * i;
        f(b, v[u].x);
        f(b + 1, v[u].y);
        f(b + 2, v[u].z);
        f(b + 3, v[u].w);
      }
    }
  }
  for (int64_t i = pre + 4 * n4 + lane; i < n; i += nl) f(i, row[i]);
}

// Block-wide MS reduce (every lane gets the result).
__device__ __forceinline__ MS block_ms(MS v, float* sm) {
  v = wave_ms(v);
  int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) { sm[2 * wid] = v.m; sm[2 * wid + 1] = v.s; }
  __syncthreads();
  MS r{sm[0], sm[1]};
  for (int w = 1; w < kBlock / 64; ++w) r = ms_comb(r, MS{sm[2 * w], sm[2 * w + 1]});
  __syncthreads();
  return r;
}
__device__ __forceinline__ float block_sum(float v, float* sm) {
  v = wave_sum(v);
  int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) sm[wid] = v;
  __syncthreads();
  float r = 0.f;
  for (int w = 0; w < kBlock / 64; ++w) r += sm[w];
  __syncthreads();
  return r;
}

// ------------------------------------------------------------- softmax

// One row per wave (WAVE) or per block.  y = softmax or log_softmax.
template <bool WAVE>
__global__ __launch_bounds__(kBlock) void k_softmax_fwd(const float* __restrict__ x, int64_t ldx,
                                                        float* __restrict__ y, int64_t ldy,
                                                        int64_t rows, int64_t cols, int log) {
  __shared__ float sm[2 * kBlock / 64];
  int64_t r = WAVE ? (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6) : blockIdx.x;
  int lane = WAVE ? (threadIdx.x & 63) : threadIdx.x;
  int nl = WAVE ? 64 : kBlock;
  if (r >= rows) return;
  const float* xr = x + r * ldx;
  float* yr = y + r * ldy;
  MS ms{-INFINITY, 0.f};
  row_scan(xr, cols, lane, nl, [&](int64_t, float v) { ms = ms_add(ms, v); });
  ms = WAVE ? wave_ms(ms) : block_ms(ms, sm);
  float lse = ms.m + logf(ms.s);
  float inv = 1.0f / ms.s;
  for (int64_t i = lane; i < cols; i += nl) {
    float v = xr[i];
    yr[i] = log ? v - lse : __expf(v - ms.m) * inv;
  }
}

template <bool WAVE>
__global__ __launch_bounds__(kBlock) void k_softmax_bwd(const float* __restrict__ dy,
                                                        const float* __restrict__ y,
                                                        float* __restrict__ dx, int64_t rows,
                                                        int64_t cols, int log) {
  __shared__ float sm[kBlock / 64];
  int64_t r = WAVE ? (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6) : blockIdx.x;
  int lane = WAVE ? (threadIdx.x & 63) : threadIdx.x;
  int nl = WAVE ? 64 : kBlock;
  if (r >= rows) return;
  const float* g = dy + r * cols;
  const float* yr = y + r * cols;
  float* o = dx + r * cols;
  float s = 0.f;
  for (int64_t i = lane; i < cols; i += nl) s += log ? g[i] : g[i] * yr[i];
  s = WAVE ? wave_sum(s) : block_sum(s, sm);
  for (int64_t i = lane; i < cols; i += nl) {
    o[i] = log ? g[i] - __expf(yr[i]) * s : yr[i] * (g[i] - s);
  }
}

// ------------------------------------------------------------- cross entropy

// One row per block (vocabulary-wide rows) or per wave (short rows).
template <bool WAVE>
__global__ __launch_bounds__(kBlock) void k_ce_fwd(const float* __restrict__ x, int64_t ld,
                                                   const int32_t* __restrict__ t, int64_t rows,
                                                   int64_t cols, int32_t ignore,
                                                   float* __restrict__ lse_out,
                                                   float* __restrict__ loss_rows) {
  __shared__ float sm[2 * kBlock / 64];
  int64_t r = WAVE ? (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6) : blockIdx.x;
  int lane = WAVE ? (threadIdx.x & 63) : threadIdx.x;
  int nl = WAVE ? 64 : kBlock;
  if (r >= rows) return;
  const float* xr = x + r * ld;
  MS ms{-INFINITY, 0.f};
  row_scan(xr, cols, lane, nl, [&](int64_t, float v) { ms = ms_add(ms, v); });
  ms = WAVE ? wave_ms(ms) : block_ms(ms, sm);
  if (lane == 0) {
    float lse = ms.m + logf(ms.s);
    int32_t tr = t[r];
    lse_out[r] = lse;
    loss_rows[r] = (tr == ignore || tr < 0 || tr >= cols) ? 0.f : lse - xr[tr];
  }
}

// Cross-entropy forward and the logits' gradient of the reduced loss for
// a unit upstream gradient (what loss.backward() seeds), in one pass over
// wide rows: a block of kBlock lanes keeps its row in registers between the
// two, so the logits are read once instead of once per pass.  lse and the
// per-row loss come out bit for bit as k_ce_fwd<false> computes them (the
// same per-lane element order and reductions: lane l takes float4 l,
// l + kBlock, ..., then the tail element l), the gradient as k_ce_bwd_flat
// writes it with grad_out = 1.  Rows 16-byte aligned, cols <= kBlock*4*NV.
template <int NV>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(2))) void k_ce_fwd_grad(
    const float* __restrict__ x, int64_t ld, const int32_t* __restrict__ t, int64_t cols,
    int32_t ignore, const float* __restrict__ count, int reduction,
    float* __restrict__ lse_out, float* __restrict__ loss_rows, float* __restrict__ d,
    int64_t ldd) {
  __shared__ float sm[2 * kBlock / 64];
  const int64_t r = blockIdx.x;
  const int lane = threadIdx.x;
  const float* xr = x + r * ld;
  const int nc = (int)cols;
  const int n4 = nc >> 2;  // >= 1: rows are wider than 2048
  // every load in bounds and unconditional (a lane past the row re-reads
  // the last chunk), so all NV are in flight together; what lies past the
  // row enters the reduction as -inf, which ms_add leaves out exactly
  float4 v[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) v[k] = ld_nt(xr + 4 * min(lane + kBlock * k, n4 - 1));
  const int ti = 4 * n4 + lane;  // the tail (cols % 4 < kBlock elements)
  const float tv = xr[min(ti, nc - 1)];
  MS ms{-INFINITY, 0.f};
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const bool in = lane + kBlock * k < n4;
    ms = ms_add(ms, in ? v[k].x : -INFINITY);
    ms = ms_add(ms, in ? v[k].y : -INFINITY);
    ms = ms_add(ms, in ? v[k].z : -INFINITY);
    ms = ms_add(ms, in ? v[k].w : -INFINITY);
  }
  ms = ms_add(ms, ti < nc ? tv : -INFINITY);
  ms = block_ms(ms, sm);
  const float l = ms.m + logf(ms.s);
  const int32_t tr = t[r];
  const bool valid = !(tr == ignore || tr < 0 || tr >= cols);
  if (lane == 0) {
    lse_out[r] = l;
    loss_rows[r] = valid ? l - xr[tr] : 0.f;
  }
  // ce_scale with grad_out[0] = 1
  const float inv = count ? 1.0f / count[0] : 1.0f;
  const float sc = valid ? ((reduction == 1 || reduction == 3) ? 1.0f * inv : 1.0f) : 0.f;
  float* dr = d + r * ldd;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = lane + kBlock * k;
    if (i < n4) {
      const int c = 4 * i;
      float4 o;
      o.x = (__expf(v[k].x - l) - (c == tr ? 1.f : 0.f)) * sc;
      o.y = (__expf(v[k].y - l) - (c + 1 == tr ? 1.f : 0.f)) * sc;
      o.z = (__expf(v[k].z - l) - (c + 2 == tr ? 1.f : 0.f)) * sc;
      o.w = (__expf(v[k].w - l) - (c + 3 == tr ? 1.f : 0.f)) * sc;
      st_nt(dr + c, o);
    }
  }
  if (ti < nc) dr[ti] = (__expf(tv - l) - (ti == tr ? 1.f : 0.f)) * sc;
  else if ((nc & 3) && ti < 4 * n4 + 4) dr[ti] = 0.f;  // the last chunk's padding, as there
}
constexpr int kCeFusedNV = 50;  // rows up to 51200 classes (GPT-2's 50257)

constexpr int kRowBatch = 16;  // rows per lane whose loads are in flight together

// Final reduction of per-row losses.  reduction 1: sum / (sum over valid
// rows of the target's class weight, 1 without weights), 2: sum,
// 3 ('batchmean', losses.ts:27-28): sum / rows.  One block.
__global__ __launch_bounds__(kBlock) void k_loss_reduce(const float* __restrict__ loss_rows,
                                                        const int32_t* __restrict__ t,
                                                        const float* __restrict__ w,
                                                        int64_t rows, int64_t cols,
                                                        int32_t ignore, int reduction,
                                                        float* __restrict__ out) {
  __shared__ float sm[kBlock / 64];
  float s = 0.f, c = 0.f;
  // each lane adds rows lane, lane + kBlock, ... in that order, with
  // kRowBatch rows' loads issued before their adds (one round trip per
  // batch instead of per row)
  for (int64_t i0 = threadIdx.x; i0 < rows; i0 += (int64_t)kBlock * kRowBatch) {
    float lv[kRowBatch];
    int32_t tv[kRowBatch];
#pragma unroll
    for (int u = 0; u < kRowBatch; ++u) {
      const int64_t i = i0 + (int64_t)u * kBlock;
      lv[u] = i < rows ? loss_rows[i] : 0.f;
      tv[u] = i < rows ? t[i] : 0;
    }
#pragma unroll
    for (int u = 0; u < kRowBatch; ++u) {
      if (i0 + (int64_t)u * kBlock < rows) {
        s += lv[u];
        const int32_t tr = tv[u];
        c += (tr == ignore || tr < 0 || tr >= cols) ? 0.f : (w ? w[tr] : 1.f);
      }
    }
  }
  s = block_sum(s, sm);
  c = block_sum(c, sm);
  if (threadIdx.x == 0) out[0] = reduction == 1 ? s / c : reduction == 3 ? s / (float)rows : s;
}

// Gradient scale of row r: grad_out[r] (none), grad_out[0] / denominator
// (mean, batchmean: the denominator k_count_valid wrote), grad_out[0] (sum).
__device__ __forceinline__ float ce_scale(const float* __restrict__ gout, int reduction,
                                          int64_t r, float inv_count) {
  if (reduction == 0) return gout[r];
  if (reduction == 1 || reduction == 3) return gout[0] * inv_count;
  return gout[0];
}

// Row r's factor of the cross-entropy gradient, (softmax - onehot) * sc[r]
// (0 for a row whose target is ignored or out of range), as the backward
// kernels form it: for GEMMs that build the gradient while loading it.
__global__ __launch_bounds__(kBlock) void k_ce_row_scale(const int32_t* __restrict__ t,
                                                         const float* __restrict__ gout,
                                                         const float* __restrict__ count,
                                                         int64_t rows, int64_t cols,
                                                         int32_t ignore, int reduction,
                                                         float* __restrict__ sc) {
  const int64_t r = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (r >= rows) return;
  const int32_t tr = t[r];
  const bool valid = !(tr == ignore || tr < 0 || tr >= cols);
  sc[r] = valid ? ce_scale(gout, reduction, r, count ? 1.0f / count[0] : 1.0f) : 0.f;
}

// dlogits = (softmax - onehot) * scale.  One row per block/wave.
template <bool WAVE>
__global__ __launch_bounds__(kBlock) void k_ce_bwd(const float* __restrict__ x, int64_t ld,
                                                   const int32_t* __restrict__ t,
                                                   const float* __restrict__ lse,
                                                   const float* __restrict__ gout,
                                                   const float* __restrict__ count,
                                                   int64_t rows, int64_t cols, int32_t ignore,
                                                   int reduction, float* __restrict__ d,
                                                   int64_t ldd, int accumulate) {
  int64_t r = WAVE ? (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6) : blockIdx.x;
  int lane = WAVE ? (threadIdx.x & 63) : threadIdx.x;
  int nl = WAVE ? 64 : kBlock;
  if (r >= rows) return;
  const float* xr = x + r * ld;
  float* dr = d + r * ldd;
  int32_t tr = t[r];
  bool valid = !(tr == ignore || tr < 0 || tr >= cols);
  float sc = valid ? ce_scale(gout, reduction, r, count ? 1.0f / count[0] : 1.0f) : 0.f;
  float l = lse[r];
  // write-aligned streaming: the output row decides the vector alignment
  int64_t pre = (int64_t)((16 - ((uintptr_t)dr & 15)) & 15) / 4;
  if (((uintptr_t)dr & 3) != 0) pre = cols;
  if (pre > cols) pre = cols;
  auto val = [&](int64_t i, float xv) {
    float p = __expf(xv - l);
    return (p - (i == tr ? 1.f : 0.f)) * sc;
  };
  for (int64_t i = lane; i < pre; i += nl) {
    float v = val(i, xr[i]);
    dr[i] = accumulate ? dr[i] + v : v;
  }
  int64_t n4 = (cols - pre) / 4;
  float4* d4 = reinterpret_cast<float4*>(dr + pre);
  bool xal = (((uintptr_t)(xr + pre)) & 15) == 0;
  for (int64_t i0 = lane; i0 < n4; i0 += (int64_t)nl * kRowUnroll) {
    float4 xv[kRowUnroll];
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) {
      const int64_t i = i0 + (int64_t)u * nl, b = pre + 4 * i;
      if (i < n4) {
        if (xal) xv[u] = ld_nt(xr + b);
        else xv[u] = make_float4(xr[b], xr[b + 1], xr[b + 2], xr[b + 3]);
      }
    }
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) {
      const int64_t i = i0 + (int64_t)u * nl, b = pre + 4 * i;
      if (i < n4) {
        float4 o = make_float4(val(b, xv[u].x), val(b + 1, xv[u].y), val(b + 2, xv[u].z),
                               val(b + 3, xv[u].w));
        if (accumulate) {
          float4 q = d4[i];
          o.x += q.x; o.y += q.y; o.z += q.z; o.w += q.w;
        }
        d4[i] = o;
      }
    }
  }
  for (int64_t i = pre + 4 * n4 + lane; i < cols; i += nl) {
    float v = val(i, xr[i]);
    dr[i] = accumulate ? dr[i] + v : v;
  }
}

// Wide rows, flat: the padded matrix is one stream of rows * ld/4 float4;
// a lane takes 4 at a time (loads issued first), the row comes from one
// 32-bit division, columns past `cols` (row padding) are skipped.
__global__ __launch_bounds__(kBlock) void k_ce_bwd_flat(
    const float* __restrict__ x, uint32_t ld4, uint32_t total4, const int32_t* __restrict__ t,
    const float* __restrict__ lse, const float* __restrict__ gout,
    const float* __restrict__ count, int64_t cols, int32_t ignore, int reduction,
    float* __restrict__ d, int accumulate) {
  const float inv = count ? 1.0f / count[0] : 1.0f;
  const uint32_t stride = gridDim.x * kBlock * 4;
  for (uint32_t v0 = blockIdx.x * kBlock * 4 + threadIdx.x; v0 < total4; v0 += stride) {
    // loads first: whole in-bounds chunks as one 128-bit access, a chunk
    // crossing `cols` element-wise (nothing past `cols` is read)
    float4 xv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t v = v0 + u * kBlock;
      if (v >= total4) continue;
      const uint32_t r = v / ld4;
      const int64_t c = 4 * (int64_t)(v - r * ld4);
      if (c + 4 <= cols) {
        xv[u] = ld_nt(x + 4 * (size_t)v);
      } else if (c < cols) {
        const float* xp = x + 4 * (size_t)v;
        xv[u] = make_float4(xp[0], c + 1 < cols ? xp[1] : 0.f, c + 2 < cols ? xp[2] : 0.f, 0.f);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t v = v0 + u * kBlock;
      if (v >= total4) continue;
      const uint32_t r = v / ld4;
      const int64_t c = 4 * (int64_t)(v - r * ld4);
      if (c >= cols) continue;
      const int32_t tr = t[r];
      const bool valid = !(tr == ignore || tr < 0 || tr >= cols);
      const float sc = valid ? ce_scale(gout, reduction, r, inv) : 0.f;
      const float l = lse[r];
      float e[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
      float o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = (c + j < cols) ? (__expf(e[j] - l) - (c + j == tr ? 1.f : 0.f)) * sc : 0.f;
      float* dp = d + 4 * (size_t)v;
      if (c + 4 <= cols) {
        float4 ov = make_float4(o[0], o[1], o[2], o[3]);
        if (accumulate) {
          const float4 q = *reinterpret_cast<const float4*>(dp);
          ov.x += q.x; ov.y += q.y; ov.z += q.z; ov.w += q.w;
          *reinterpret_cast<float4*>(dp) = ov;
        } else {
          st_nt(dp, ov);
        }
      } else {
        for (int j = 0; j < 4 && c + j < cols; ++j) dp[j] = accumulate ? dp[j] + o[j] : o[j];
      }
    }
  }
}

// Denominator of the mean reductions into one float: the number of valid
// targets, or the sum of their class weights (reduction 1), or the row
// count ('batchmean', reduction 3).  When `wsum` is given, also the sum of
// every class weight (C without weights), which label smoothing needs.
__global__ __launch_bounds__(kBlock) void k_count_valid(const int32_t* __restrict__ t, int64_t rows,
                                                        int64_t cols, int32_t ignore,
                                                        const float* __restrict__ w, int reduction,
                                                        float* __restrict__ out,
                                                        float* __restrict__ wsum) {
  __shared__ float sm[kBlock / 64];
  float c = 0.f;
  // per lane in row order, kRowBatch targets loaded before their adds
  for (int64_t i0 = threadIdx.x; i0 < rows; i0 += (int64_t)kBlock * kRowBatch) {
    int32_t tv[kRowBatch];
#pragma unroll
    for (int u = 0; u < kRowBatch; ++u) {
      const int64_t i = i0 + (int64_t)u * kBlock;
      tv[u] = i < rows ? t[i] : 0;
    }
#pragma unroll
    for (int u = 0; u < kRowBatch; ++u) {
      if (i0 + (int64_t)u * kBlock < rows) {
        const int32_t tr = tv[u];
        c += (tr == ignore || tr < 0 || tr >= cols) ? 0.f : (w ? w[tr] : 1.f);
      }
    }
  }
  c = block_sum(c, sm);
  if (wsum) {
    float ws = 0.f;
    for (int64_t i = threadIdx.x; i < cols; i += kBlock) ws += w ? w[i] : 1.f;
    ws = block_sum(ws, sm);
    if (threadIdx.x == 0) wsum[0] = ws;
  }
  if (threadIdx.x == 0 && out) out[0] = reduction == 3 ? (float)rows : c;
}

// ---- cross entropy with class weights and / or label smoothing
// (losses.ts:129-168 under PyTorch's contract, which its @pytorch tag
// declares).  Row i with a valid target t, W = sum_c w_c (C without weights),
// eps the smoothing:
//   loss_i = (1-eps) w_t (lse - x_t) + (eps/C) sum_c w_c (lse - x_c)
//   dx_ic  = s_i [ ((1-eps) w_t + (eps/C) W) p_c - (1-eps) w_t [c == t]
//                  - (eps/C) w_c ]
// with p = softmax(x_i) and s_i the row's gradient scale.  An ignored row
// has loss 0 and gradient 0.  The plain case (no weights, eps 0) runs on
// k_ce_fwd / k_ce_bwd(_flat) instead.
template <bool WAVE>
__global__ __launch_bounds__(kBlock) void k_ce_fwd_gen(const float* __restrict__ x, int64_t ld,
                                                       const int32_t* __restrict__ t, int64_t rows,
                                                       int64_t cols, int32_t ignore,
                                                       const float* __restrict__ w, float eps,
                                                       float* __restrict__ lse_out,
                                                       float* __restrict__ loss_rows) {
  __shared__ float sm[2 * kBlock / 64];
  int64_t r = WAVE ? (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6) : blockIdx.x;
  int lane = WAVE ? (threadIdx.x & 63) : threadIdx.x;
  int nl = WAVE ? 64 : kBlock;
  if (r >= rows) return;
  const float* xr = x + r * ld;
  MS ms{-INFINITY, 0.f};
  row_scan(xr, cols, lane, nl, [&](int64_t, float v) { ms = ms_add(ms, v); });
  ms = WAVE ? wave_ms(ms) : block_ms(ms, sm);
  const float lse = ms.m + logf(ms.s);
  // smoothing term: sum_c w_c (lse - x_c), every term >= 0 (no cancellation)
  float sm_term = 0.f;
  if (eps != 0.f) {
    row_scan(xr, cols, lane, nl,
             [&](int64_t i, float v) { sm_term += (w ? w[i] : 1.f) * (lse - v); });
    sm_term = WAVE ? wave_sum(sm_term) : block_sum(sm_term, sm);
  }
  if (lane == 0) {
    int32_t tr = t[r];
    lse_out[r] = lse;
    float l = 0.f;
    if (!(tr == ignore || tr < 0 || tr >= cols)) {
      const float wt = w ? w[tr] : 1.f;
      l = (1.f - eps) * wt * (lse - xr[tr]);
      if (eps != 0.f) l += eps / (float)cols * sm_term;
    }
    loss_rows[r] = l;
  }
}

template <bool WAVE>
__global__ __launch_bounds__(kBlock) void k_ce_bwd_gen(
    const float* __restrict__ x, int64_t ld, const int32_t* __restrict__ t,
    const float* __restrict__ w, float eps, const float* __restrict__ lse,
    const float* __restrict__ gout, const float* __restrict__ count,
    const float* __restrict__ wsum, int64_t rows, int64_t cols, int32_t ignore, int reduction,
    float* __restrict__ d, int64_t ldd, int accumulate) {
  int64_t r = WAVE ? (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6) : blockIdx.x;
  int lane = WAVE ? (threadIdx.x & 63) : threadIdx.x;
  int nl = WAVE ? 64 : kBlock;
  if (r >= rows) return;
  const float* xr = x + r * ld;
  float* dr = d + r * ldd;
  const int32_t tr = t[r];
  const bool valid = !(tr == ignore || tr < 0 || tr >= cols);
  const float sc = valid ? ce_scale(gout, reduction, r, count ? 1.0f / count[0] : 1.0f) : 0.f;
  const float wt = valid ? (w ? w[tr] : 1.f) : 0.f;
  const float ec = eps / (float)cols;
  const float a = ((1.f - eps) * wt + ec * wsum[0]) * sc;  // coefficient of p_c
  const float b = (1.f - eps) * wt * sc;                   // of [c == t]
  const float e = ec * sc;                                 // of w_c
  const float l = lse[r];
  for (int64_t i = lane; i < cols; i += nl) {
    const float p = __expf(xr[i] - l);
    const float v = a * p - (i == tr ? b : 0.f) - e * (w ? w[i] : 1.f);
    dr[i] = accumulate ? dr[i] + v : v;
  }
}

__global__ __launch_bounds__(kBlock) void k_nll_fwd(const float* __restrict__ lp, int64_t ld,
                                                    const int32_t* __restrict__ t, int64_t rows,
                                                    int64_t cols, int32_t ignore,
                                                    const float* __restrict__ w,
                                                    float* __restrict__ loss_rows) {
  int64_t r = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (r >= rows) return;
  int32_t tr = t[r];
  loss_rows[r] = (tr == ignore || tr < 0 || tr >= cols) ? 0.f
                                                        : -(w ? w[tr] : 1.f) * lp[r * ld + tr];
}

__global__ __launch_bounds__(kBlock) void k_nll_bwd(const int32_t* __restrict__ t,
                                                    const float* __restrict__ w,
                                                    const float* __restrict__ gout,
                                                    const float* __restrict__ count,
                                                    int64_t rows, int64_t cols, int32_t ignore,
                                                    int reduction, float* __restrict__ d) {
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= rows * cols) return;
  int64_t r = i / cols, c = i % cols;
  int32_t tr = t[r];
  bool valid = !(tr == ignore || tr < 0 || tr >= cols);
  float v = 0.f;
  if (valid && c == tr)
    v = -(w ? w[tr] : 1.f) * ce_scale(gout, reduction, r, count ? 1.0f / count[0] : 1.0f);
  d[i] = v;
}

// ------------------------------------------------------------- layer norm

// Wave per row, the row kept in registers: cols % 4 == 0, cols <= 64*4*V4.
// EXACT: cols == 256 * V4, so every lane owns V4 whole float4 and no lane
// guard is needed (the guards otherwise split the loads across branches).
template <int V4, bool EXACT>
__global__ __launch_bounds__(kBlock) void k_ln_fwd_wave(const float* __restrict__ x,
                                                        const float* __restrict__ gamma,
                                                        const float* __restrict__ beta,
                                                        float* __restrict__ y,
                                                        float* __restrict__ mean_out,
                                                        float* __restrict__ rstd_out, int64_t rows,
                                                        int64_t cols, float eps) {
  int64_t r = (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const int c4 = (int)(cols >> 2);
  const float4* xr = reinterpret_cast<const float4*>(x + r * cols);
  const float4* g4 = reinterpret_cast<const float4*>(gamma);
  const float4* b4 = reinterpret_cast<const float4*>(beta);
  float4 v[V4], gv[V4], bv[V4];
  // gamma and beta go out with the row's loads, not after the reductions
#pragma unroll
  for (int j = 0; j < V4; ++j) {
    int i = lane + 64 * j;
    if (EXACT || i < c4) {
      v[j] = xr[i];
      gv[j] = gamma ? g4[i] : make_float4(1.f, 1.f, 1.f, 1.f);
      bv[j] = beta ? b4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
      v[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < V4; ++j) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
  float mean = wave_sum(s) / (float)cols;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < V4; ++j) {
    int i = lane + 64 * j;
    if (EXACT || i < c4) {
      float a = v[j].x - mean, b = v[j].y - mean, c = v[j].z - mean, d = v[j].w - mean;
      q += (a * a + b * b) + (c * c + d * d);
    }
  }
  float var = wave_sum(q) / (float)cols;
  float rstd = 1.0f / sqrtf(var + eps);
  float4* yr = reinterpret_cast<float4*>(y + r * cols);
#pragma unroll
  for (int j = 0; j < V4; ++j) {
    int i = lane + 64 * j;
    if (EXACT || i < c4) {
      float4 o;
      o.x = (v[j].x - mean) * rstd;
      o.y = (v[j].y - mean) * rstd;
      o.z = (v[j].z - mean) * rstd;
      o.w = (v[j].w - mean) * rstd;
      if (gamma) {
        const float4 gg = gv[j];
        o.x *= gg.x; o.y *= gg.y; o.z *= gg.z; o.w *= gg.w;
      }
      if (beta) {
        const float4 bb = bv[j];
        o.x += bb.x; o.y += bb.y; o.z += bb.z; o.w += bb.w;
      }
      yr[i] = o;
    }
  }
  if (lane == 0) {
    mean_out[r] = mean;
    rstd_out[r] = rstd;
  }
}

// General LayerNorm forward: one block per row, scalar, re-reads the row.
__global__ __launch_bounds__(kBlock) void k_ln_fwd_block(const float* __restrict__ x,
                                                         const float* __restrict__ gamma,
                                                         const float* __restrict__ beta,
                                                         float* __restrict__ y,
                                                         float* __restrict__ mean_out,
                                                         float* __restrict__ rstd_out,
                                                         int64_t cols, float eps) {
  __shared__ float sm[kBlock / 64];
  int64_t r = blockIdx.x;
  const float* xr = x + r * cols;
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < cols; i += kBlock) s += xr[i];
  float mean = block_sum(s, sm) / (float)cols;
  float q = 0.f;
  for (int64_t i = threadIdx.x; i < cols; i += kBlock) {
    float a = xr[i] - mean;
    q += a * a;
  }
  float var = block_sum(q, sm) / (float)cols;
  float rstd = 1.0f / sqrtf(var + eps);
  float* yr = y + r * cols;
  for (int64_t i = threadIdx.x; i < cols; i += kBlock) {
    float o = (xr[i] - mean) * rstd;
    if (gamma) o *= gamma[i];
    if (beta) o += beta[i];
    yr[i] = o;
  }
  if (threadIdx.x == 0) {
    mean_out[r] = mean;
    rstd_out[r] = rstd;
  }
}

// LayerNorm backward, dx part + per-block partial dgamma/dbeta.  With res,
// dx = res + the LayerNorm input gradient (a residual stream's gradient).
// Block b (NW waves) owns rows [b*rpb, (b+1)*rpb); wave w takes rows
// b*rpb + w + NW*k.
// Lane owns columns 4*(lane + 64*j) .. +3 (cols % 4 == 0, cols <= 256*V4).
// Partials: pg/pb [nblocks, cols].
// EXACT as for k_ln_fwd_wave.
template <int V4, bool EXACT>
__global__ __launch_bounds__(64 * kLnBwdWaves) void k_ln_bwd_wave(const float* __restrict__ dy,
                                                        const float* __restrict__ x,
                                                        const float* __restrict__ gamma,
                                                        const float* __restrict__ mean,
                                                        const float* __restrict__ rstd,
                                                        const float* __restrict__ res,
                                                        float* __restrict__ dx,
                                                        float* __restrict__ pg,
                                                        float* __restrict__ pb, int64_t rows,
                                                        int64_t cols, int64_t rpb) {
  // no implicit contraction: the compiler versions the row loop on res,
  // and the folded and unfolded residual paths must round alike (the only
  // fused multiply-adds are the explicit ones below)
#pragma clang fp contract(off)
  constexpr int NW = kLnBwdWaves;
  __shared__ float4 red[2][NW][64 * 3];  // partial combine across waves
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c4 = (int)(cols >> 2);
  // Rows of up to 1536 keep gamma in registers and load a residual row
  // before its reductions; wider rows (up to 3072: the dgamma / dbeta
  // partials alone take 96 registers) read gamma at each use (an L1-resident
  // row) and the residual as they write, so nothing spills.
  constexpr bool kWide = V4 > 6;
  float4 ag[V4], ab[V4];
  float4 gm[kWide ? 1 : V4];
  auto gam = [&](int j) {
    const int i = lane + 64 * j;
    return (gamma && (EXACT || i < c4)) ? reinterpret_cast<const float4*>(gamma)[i]
                                        : make_float4(1.f, 1.f, 1.f, 1.f);
  };
#pragma unroll
  for (int j = 0; j < V4; ++j) {
    ag[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    ab[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (!kWide) gm[kWide ? 0 : j] = gam(j);
  }
  const float inv_n = 1.0f / (float)cols;
  int64_t r_beg = (int64_t)blockIdx.x * rpb;
  int64_t r_end = r_beg + rpb < rows ? r_beg + rpb : rows;
  // rows per wave per step (four at GPT-2's 768-wide rows, fewer for wider
  // rows so the registers hold them): every row's loads are issued before
  // any row's reductions
  constexpr int kPair = V4 <= 3 ? 4 : (V4 <= 6 ? 2 : 1);
  constexpr int kStep = NW;
  for (int64_t r0 = r_beg + w; r0 < r_end; r0 += kStep * kPair) {
    float4 gv[kPair][V4], xh[kPair][V4];
    float mu[kPair], rs[kPair];
#pragma unroll
    for (int q = 0; q < kPair; ++q) {
      const int64_t r = r0 + q * kStep;
      if (r < r_end) {
        const float4* g4 = reinterpret_cast<const float4*>(dy + r * cols);
        const float4* x4 = reinterpret_cast<const float4*>(x + r * cols);
        mu[q] = mean[r];
        rs[q] = rstd[r];
#pragma unroll
        for (int j = 0; j < V4; ++j) {
          const int i = lane + 64 * j;
          if (EXACT || i < c4) {
            gv[q][j] = ld_nt(reinterpret_cast<const float*>(g4 + i));
            xh[q][j] = ld_nt(reinterpret_cast<const float*>(x4 + i));
          }
        }
      }
    }
#pragma unroll
    for (int q = 0; q < kPair; ++q) {
      const int64_t r = r0 + q * kStep;
      if (r >= r_end) continue;  // wave-uniform
      float s1 = 0.f, s2 = 0.f;
#pragma unroll
      for (int j = 0; j < V4; ++j) {
        const int i = lane + 64 * j;
        if (EXACT || i < c4) {
          const float4 g = gv[q][j], xv = xh[q][j];
          xh[q][j] = make_float4((xv.x - mu[q]) * rs[q], (xv.y - mu[q]) * rs[q],
                                 (xv.z - mu[q]) * rs[q], (xv.w - mu[q]) * rs[q]);
          const float4 gmj = kWide ? gam(j) : gm[kWide ? 0 : j];
          const float4 gg = make_float4(g.x * gmj.x, g.y * gmj.y, g.z * gmj.z, g.w * gmj.w);
          s1 += (gg.x + gg.y) + (gg.z + gg.w);
          s2 += (gg.x * xh[q][j].x + gg.y * xh[q][j].y) + (gg.z * xh[q][j].z + gg.w * xh[q][j].w);
          ag[j].x += g.x * xh[q][j].x; ag[j].y += g.y * xh[q][j].y;
          ag[j].z += g.z * xh[q][j].z; ag[j].w += g.w * xh[q][j].w;
          ab[j].x += g.x; ab[j].y += g.y; ab[j].z += g.z; ab[j].w += g.w;
        }
      }
      // the residual row's loads go out before the row reductions
      float4 rv[kWide ? 1 : V4];
      if (!kWide && dx && res) {
        const float4* r4 = reinterpret_cast<const float4*>(res + r * cols);
#pragma unroll
        for (int j = 0; j < V4; ++j) {
          const int i = lane + 64 * j;
          if (EXACT || i < c4) rv[kWide ? 0 : j] = ld_nt(reinterpret_cast<const float*>(r4 + i));
        }
      }
      s1 = wave_sum(s1) * inv_n;
      s2 = wave_sum(s2) * inv_n;
      if (dx) {
        float4* d4 = reinterpret_cast<float4*>(dx + r * cols);
#pragma unroll
        for (int j = 0; j < V4; ++j) {
          const int i = lane + 64 * j;
          if (EXACT || i < c4) {
            float4 o;
            const float4 gmj = kWide ? gam(j) : gm[kWide ? 0 : j];
            o.x = rs[q] * fmaf(-xh[q][j].x, s2, fmaf(gv[q][j].x, gmj.x, -s1));
            o.y = rs[q] * fmaf(-xh[q][j].y, s2, fmaf(gv[q][j].y, gmj.y, -s1));
            o.z = rs[q] * fmaf(-xh[q][j].z, s2, fmaf(gv[q][j].z, gmj.z, -s1));
            o.w = rs[q] * fmaf(-xh[q][j].w, s2, fmaf(gv[q][j].w, gmj.w, -s1));
            if (res) {
              const float4 rr =
                  kWide ? ld_nt(res + r * cols + 4 * (int64_t)i) : rv[kWide ? 0 : j];
              o.x = rr.x + o.x; o.y = rr.y + o.y;
              o.z = rr.z + o.z; o.w = rr.w + o.w;
            }
            d4[i] = o;
          }
        }
      }
    }
  }
  // combine the NW waves' column partials (fixed order) and write
  if (pg) {
    for (int j0 = 0; j0 < V4; j0 += 3) {
#pragma unroll
      for (int jj = 0; jj < 3; ++jj) {
        int j = j0 + jj;
        if (j < V4) {
          red[0][w][lane + 64 * jj] = ag[j];
          red[1][w][lane + 64 * jj] = ab[j];
        }
      }
      __syncthreads();
      // wave 0 sums for gamma, wave 1 for beta
      if (w < 2) {
#pragma unroll
        for (int jj = 0; jj < 3; ++jj) {
          int j = j0 + jj;
          int i = lane + 64 * j;
          if (j < V4 && i < c4) {
            float4 s = red[w][0][lane + 64 * jj];
            for (int q = 1; q < NW; ++q) {
              float4 t = red[w][q][lane + 64 * jj];
              s.x += t.x; s.y += t.y; s.z += t.z; s.w += t.w;
            }
            float* dst = (w == 0 ? pg : pb) + (int64_t)blockIdx.x * cols;
            reinterpret_cast<float4*>(dst)[i] = s;
          }
        }
      }
      __syncthreads();
    }
  }
}

// General LayerNorm backward: one block per row (dx) + partials per row.
__global__ __launch_bounds__(kBlock) void k_ln_bwd_block(const float* __restrict__ dy,
                                                         const float* __restrict__ x,
                                                         const float* __restrict__ gamma,
                                                         const float* __restrict__ mean,
                                                         const float* __restrict__ rstd,
                                                         const float* __restrict__ res,
                                                         float* __restrict__ dx,
                                                         float* __restrict__ pg,
                                                         float* __restrict__ pb, int64_t cols) {
  __shared__ float sm[kBlock / 64];
  int64_t r = blockIdx.x;
  const float* g = dy + r * cols;
  const float* xr = x + r * cols;
  float mu = mean[r], rs = rstd[r];
  float s1 = 0.f, s2 = 0.f;
  for (int64_t i = threadIdx.x; i < cols; i += kBlock) {
    float gg = g[i] * (gamma ? gamma[i] : 1.f);
    float xh = (xr[i] - mu) * rs;
    s1 += gg;
    s2 += gg * xh;
    if (pg) pg[r * cols + i] = g[i] * xh;
    if (pb) pb[r * cols + i] = g[i];
  }
  s1 = block_sum(s1, sm) / (float)cols;
  s2 = block_sum(s2, sm) / (float)cols;
  if (dx) {
    for (int64_t i = threadIdx.x; i < cols; i += kBlock) {
      float gg = g[i] * (gamma ? gamma[i] : 1.f);
      float xh = (xr[i] - mu) * rs;
      const float o = rs * (gg - s1 - xh * s2);
      dx[r * cols + i] = res ? res[r * cols + i] + o : o;
    }
  }
}

// dgamma / dbeta from per-block partials [nb, cols]: the split column
// reduction of tjh_reduce (deterministic), added into the outputs when
// accumulating.
int sum_partials(const float* pg, const float* pb, int64_t nb, int64_t cols, float* dgamma,
                 float* dbeta, int accumulate) {
  const float* parts[2] = {pg, pb};
  float* outs[2] = {dgamma, dbeta};
  for (int i = 0; i < 2; ++i) {
    if (!outs[i]) continue;
    if (!accumulate) {
      int rc = tjh_reduce(TJH_REDUCE_SUM, parts[i], 1, nb, cols, outs[i]);
      if (rc != TJH_OK) return rc;
    } else {
      Scratch tmp((size_t)cols * sizeof(float));
      if (!tmp.ok()) return set_error(TJH_ERR_OOM, "layer_norm_backward: no scratch");
      int rc = tjh_reduce(TJH_REDUCE_SUM, parts[i], 1, nb, cols, tmp.as<float>());
      if (rc == TJH_OK) rc = tjh_axpy(1.0f, tmp.as<float>(), outs[i], outs[i], cols);
      if (rc != TJH_OK) return rc;
    }
  }
  return TJH_OK;
}

}  // namespace
}  // namespace tjh

using namespace tjh;

namespace tjh {
namespace {

// The register-resident LayerNorm backward (k_ln_bwd_wave) takes rows
// whose length is a multiple of 4 and at most 3072, with 16-byte aligned
// operands; returns its V4 (float4 per lane), or 0 for the general path.
int ln_bwd_v4(const float* dy, const float* x, const float* gamma, const float* res,
              const float* dx, int64_t cols) {
  const bool vec = cols % 4 == 0 && aligned16(x) && aligned16(dy) && (!dx || aligned16(dx)) &&
                   (!gamma || aligned16(gamma)) && (!res || aligned16(res));
  if (!vec) return 0;
  return cols <= 64 * 4 * 3 ? 3 : (cols <= 64 * 4 * 6 ? 6 : (cols <= 64 * 4 * 12 ? 12 : 0));
}

// Rows per workgroup: one 8-wave workgroup per CU, >= 32 rows each (four
// per wave: the same waves in flight as two 4-wave workgroups of 16 rows,
// half the partial rows for the dgamma/dbeta pass, and measured 3% faster).
// So nb <= max(CUs, ...) and nb <= 256 on a 256-CU MI355X.
void ln_bwd_blocks(int64_t rows, int64_t& rpb, int64_t& nb) {
  const int cus = num_cus() > 0 ? num_cus() : 256;
  rpb = cdiv(rows, 1LL * cus);
  if (rpb < 32) rpb = 32;
  nb = cdiv(rows, rpb);
}

// Launches k_ln_bwd_wave: dx (optionally plus res) and, with pg / pb, the
// per-workgroup partial rows [nb, cols] of dgamma / dbeta (every row
// written whole).
int ln_bwd_wave_launch(int v4, const float* dy, const float* x, const float* gamma,
                       const float* mean, const float* rstd, const float* res, float* dx,
                       float* pg, float* pb, int64_t rows, int64_t cols, int64_t rpb,
                       int64_t nb) {
  if (v4 == 3 && cols == 64 * 4 * 3)
    tjh_launch((k_ln_bwd_wave<3, true>), dim3((unsigned)nb), dim3(64 * kLnBwdWaves), 0, stream(),
                       dy, x, gamma, mean, rstd, res, dx, pg, pb, rows, cols, rpb);
  else if (v4 == 3)
    tjh_launch((k_ln_bwd_wave<3, false>), dim3((unsigned)nb), dim3(64 * kLnBwdWaves), 0, stream(),
                       dy, x, gamma, mean, rstd, res, dx, pg, pb, rows, cols, rpb);
  else if (v4 == 6)
    tjh_launch((k_ln_bwd_wave<6, false>), dim3((unsigned)nb), dim3(64 * kLnBwdWaves), 0, stream(),
                       dy, x, gamma, mean, rstd, res, dx, pg, pb, rows, cols, rpb);
  else
    tjh_launch((k_ln_bwd_wave<12, false>), dim3((unsigned)nb), dim3(64 * kLnBwdWaves), 0, stream(),
                       dy, x, gamma, mean, rstd, res, dx, pg, pb, rows, cols, rpb);
  return check_launch("layer_norm_backward");
}

// LayerNorm backwards whose dgamma/dbeta finishing pass waits for
// tjh_flush_deferred: the partial-row scratch block and the outputs.
struct DeferredSums {
  void* part;  // [2][nb][cols]: dgamma rows, then dbeta rows
  float* outs[2];
  int64_t nb, cols;
  int accumulate;
};

std::vector<DeferredSums>& deferred_sums() {
  static std::vector<DeferredSums> q;
  return q;
}

}  // namespace
}  // namespace tjh

extern "C" {

int tjh_softmax_forward(const float* x, int64_t ldx, float* y, int64_t ldy, int64_t rows,
                        int64_t cols, int log) {
  TJH_REQUIRE_INIT();
  TJH_ARG(rows >= 0 && cols >= 0 && ldx >= cols && ldy >= cols, "tjh_softmax_forward: bad sizes");
  if (rows == 0 || cols == 0) return TJH_OK;
  KernelScope ks(log ? "log_softmax_fwd" : "softmax_fwd");
  if (cols <= 2048) {
    tjh_launch(k_softmax_fwd<true>, dim3((unsigned)cdiv(rows, 4)), dim3(kBlock), 0,
                       stream(), x, ldx, y, ldy, rows, cols, log);
  } else {
    tjh_launch(k_softmax_fwd<false>, dim3((unsigned)rows), dim3(kBlock), 0, stream(), x,
                       ldx, y, ldy, rows, cols, log);
  }
  return check_launch("softmax_forward");
}

int tjh_softmax_backward(const float* dy, const float* y, float* dx, int64_t rows, int64_t cols,
                         int log) {
  TJH_REQUIRE_INIT();
  TJH_ARG(rows >= 0 && cols >= 0, "tjh_softmax_backward: bad sizes");
  if (rows == 0 || cols == 0) return TJH_OK;
  KernelScope ks(log ? "log_softmax_bwd" : "softmax_bwd");
  if (cols <= 2048) {
    tjh_launch(k_softmax_bwd<true>, dim3((unsigned)cdiv(rows, 4)), dim3(kBlock), 0,
                       stream(), dy, y, dx, rows, cols, log);
  } else {
    tjh_launch(k_softmax_bwd<false>, dim3((unsigned)rows), dim3(kBlock), 0, stream(), dy,
                       y, dx, rows, cols, log);
  }
  return check_launch("softmax_backward");
}

int tjh_cross_entropy_forward(const float* logits, int64_t ld, const int32_t* targets,
                              int64_t rows, int64_t cols, int32_t ignore_index,
                              const float* weight, float label_smoothing, float* lse,
                              float* loss_rows, int reduction, float* out) {
  TJH_REQUIRE_INIT();
  TJH_ARG(rows >= 0 && cols > 0 && ld >= cols, "tjh_cross_entropy_forward: bad sizes");
  TJH_ARG(reduction >= 0 && reduction <= 3, "tjh_cross_entropy_forward: bad reduction");
  TJH_ARG(reduction == 0 || out, "tjh_cross_entropy_forward: reduction needs `out`");
  TJH_ARG(label_smoothing >= 0.f && label_smoothing <= 1.f,
          "tjh_cross_entropy_forward: label_smoothing must lie in [0, 1]");
  if (rows == 0) {
    if (reduction) return tjh_fill_f32(out, 1, reduction == 2 ? 0.f : __builtin_nanf(""));
    return TJH_OK;
  }
  const bool gen = weight != nullptr || label_smoothing != 0.f;
  {
    KernelScope ks("cross_entropy_fwd");
    if (gen && cols <= 2048)
      tjh_launch(k_ce_fwd_gen<true>, dim3((unsigned)cdiv(rows, 4)), dim3(kBlock), 0,
                         stream(), logits, ld, targets, rows, cols, ignore_index, weight,
                         label_smoothing, lse, loss_rows);
    else if (gen)
      tjh_launch(k_ce_fwd_gen<false>, dim3((unsigned)rows), dim3(kBlock), 0, stream(),
                         logits, ld, targets, rows, cols, ignore_index, weight, label_smoothing,
                         lse, loss_rows);
    else if (cols <= 2048)
      tjh_launch(k_ce_fwd<true>, dim3((unsigned)cdiv(rows, 4)), dim3(kBlock), 0, stream(),
                         logits, ld, targets, rows, cols, ignore_index, lse, loss_rows);
    else
      tjh_launch(k_ce_fwd<false>, dim3((unsigned)rows), dim3(kBlock), 0, stream(), logits,
                         ld, targets, rows, cols, ignore_index, lse, loss_rows);
    int rc = check_launch("cross_entropy_forward");
    if (rc != TJH_OK) return rc;
  }
  if (reduction) {
    KernelScope ks("loss_reduce");
    tjh_launch(k_loss_reduce, dim3(1), dim3(kBlock), 0, stream(), loss_rows, targets,
                       weight, rows, cols, ignore_index, reduction, out);
    return check_launch("loss_reduce");
  }
  return TJH_OK;
}

int tjh_cross_entropy_backward(const float* logits, int64_t ld, const int32_t* targets,
                               const float* weight, float label_smoothing, const float* lse,
                               const float* grad_out, int64_t rows, int64_t cols,
                               int32_t ignore_index, int reduction, float* dlogits, int64_t ldd,
                               int accumulate) {
  TJH_REQUIRE_INIT();
  TJH_ARG(rows >= 0 && cols > 0 && ld >= cols && ldd >= cols,
          "tjh_cross_entropy_backward: bad sizes");
  TJH_ARG(reduction >= 0 && reduction <= 3, "tjh_cross_entropy_backward: bad reduction");
  TJH_ARG(label_smoothing >= 0.f && label_smoothing <= 1.f,
          "tjh_cross_entropy_backward: label_smoothing must lie in [0, 1]");
  if (rows == 0) return TJH_OK;
  const bool gen = weight != nullptr || label_smoothing != 0.f;
  const bool mean = reduction == 1 || reduction == 3;
  // [0]: the mean's denominator, [1]: the sum of the class weights
  Scratch cnt(mean || gen ? 2 * sizeof(float) : 0);
  if (mean || gen) {
    if (!cnt.ok()) return set_error(TJH_ERR_OOM, "cross_entropy_backward: no scratch");
    KernelScope ks("loss_reduce");
    tjh_launch(k_count_valid, dim3(1), dim3(kBlock), 0, stream(), targets, rows, cols,
                       ignore_index, weight, reduction, mean ? cnt.as<float>() : nullptr,
                       gen ? cnt.as<float>() + 1 : nullptr);
    int rc = check_launch("count_valid");
    if (rc != TJH_OK) return rc;
  }
  const float* count = mean ? cnt.as<float>() : nullptr;
  KernelScope ks("cross_entropy_bwd");
  if (gen && cols <= 2048)
    tjh_launch(k_ce_bwd_gen<true>, dim3((unsigned)cdiv(rows, 4)), dim3(kBlock), 0,
                       stream(), logits, ld, targets, weight, label_smoothing, lse, grad_out,
                       count, cnt.as<float>() + 1, rows, cols, ignore_index, reduction, dlogits,
                       ldd, accumulate);
  else if (gen)
    tjh_launch(k_ce_bwd_gen<false>, dim3((unsigned)rows), dim3(kBlock), 0, stream(),
                       logits, ld, targets, weight, label_smoothing, lse, grad_out, count,
                       cnt.as<float>() + 1, rows, cols, ignore_index, reduction, dlogits, ldd,
                       accumulate);
  else if (cols <= 2048)
    tjh_launch(k_ce_bwd<true>, dim3((unsigned)cdiv(rows, 4)), dim3(kBlock), 0, stream(),
                       logits, ld, targets, lse, grad_out, count, rows, cols, ignore_index,
                       reduction, dlogits, ldd, accumulate);
  else if (ld == ldd && ld % 4 == 0 && aligned16(logits) && aligned16(dlogits) &&
           rows * (ld / 4) < (int64_t(1) << 31)) {
    const int64_t total4 = rows * (ld / 4);
    const int64_t grid = cdiv(total4, (int64_t)kBlock * 4) < 16384 ? cdiv(total4, (int64_t)kBlock * 4)
                                                                   : 16384;
    tjh_launch(k_ce_bwd_flat, dim3((unsigned)grid), dim3(kBlock), 0, stream(), logits,
                       (uint32_t)(ld / 4), (uint32_t)total4, targets, lse, grad_out, count, cols,
                       ignore_index, reduction, dlogits, accumulate);
  } else
    tjh_launch(k_ce_bwd<false>, dim3((unsigned)rows), dim3(kBlock), 0, stream(), logits,
                       ld, targets, lse, grad_out, count, rows, cols, ignore_index, reduction,
                       dlogits, ldd, accumulate);
  return check_launch("cross_entropy_backward");
}

int tjh_cross_entropy_row_scale(const int32_t* targets, const float* grad_out, int64_t rows,
                                int64_t cols, int32_t ignore_index, int reduction,
                                float* row_scale) {
  TJH_REQUIRE_INIT();
  TJH_ARG(rows >= 0 && cols > 0, "tjh_cross_entropy_row_scale: bad sizes");
  TJH_ARG(reduction >= 0 && reduction <= 3, "tjh_cross_entropy_row_scale: bad reduction");
  TJH_ARG(rows == 0 || (targets && grad_out && row_scale),
          "tjh_cross_entropy_row_scale: NULL operand");
  if (rows == 0) return TJH_OK;
  const bool mean = reduction == 1 || reduction == 3;
  Scratch cnt(mean ? 2 * sizeof(float) : 0);
  if (mean) {
    if (!cnt.ok()) return set_error(TJH_ERR_OOM, "cross_entropy_row_scale: no scratch");
    KernelScope ks("loss_reduce");
    tjh_launch(k_count_valid, dim3(1), dim3(kBlock), 0, stream(), targets, rows, cols,
               ignore_index, nullptr, reduction, cnt.as<float>(), nullptr);
    int rc = check_launch("count_valid");
    if (rc != TJH_OK) return rc;
  }
  KernelScope ks("cross_entropy_bwd");
  tjh_launch(k_ce_row_scale, dim3((unsigned)cdiv(rows, kBlock)), dim3(kBlock), 0, stream(),
             targets, grad_out, mean ? cnt.as<float>() : nullptr, rows, cols, ignore_index,
             reduction, row_scale);
  return check_launch("cross_entropy_row_scale");
}

int tjh_cross_entropy_forward_grad(const float* logits, int64_t ld, const int32_t* targets,
                                   int64_t rows, int64_t cols, int32_t ignore_index, float* lse,
                                   float* loss_rows, int reduction, float* out, float* dlogits,
                                   int64_t ldd) {
  TJH_REQUIRE_INIT();
  TJH_ARG(rows >= 0 && cols > 0 && ld >= cols && ldd >= cols,
          "tjh_cross_entropy_forward_grad: bad sizes");
  TJH_ARG(reduction >= 1 && reduction <= 3,
          "tjh_cross_entropy_forward_grad: the reduction must give a scalar loss (1, 2 or 3)");
  TJH_ARG(out && lse && loss_rows && dlogits && targets && logits,
          "tjh_cross_entropy_forward_grad: NULL operand");
  if (rows == 0) return tjh_fill_f32(out, 1, reduction == 2 ? 0.f : __builtin_nanf(""));
  const bool fused = cols > 2048 && cols <= (int64_t)kBlock * 4 * kCeFusedNV && ld % 4 == 0 &&
                     ldd % 4 == 0 && aligned16(logits) && aligned16(dlogits);
  if (!fused) {
    // the two passes, with a unit upstream gradient
    int rc = tjh_cross_entropy_forward(logits, ld, targets, rows, cols, ignore_index, nullptr,
                                       0.f, lse, loss_rows, reduction, out);
    if (rc != TJH_OK) return rc;
    Scratch one(sizeof(float));
    if (!one.ok()) return set_error(TJH_ERR_OOM, "cross_entropy_forward_grad: no scratch");
    rc = tjh_fill_f32(one.as<float>(), 1, 1.0f);
    if (rc != TJH_OK) return rc;
    return tjh_cross_entropy_backward(logits, ld, targets, nullptr, 0.f, lse, one.as<float>(),
                                      rows, cols, ignore_index, reduction, dlogits, ldd, 0);
  }
  const bool mean = reduction == 1 || reduction == 3;
  Scratch cnt(mean ? 2 * sizeof(float) : 0);
  if (mean) {
    if (!cnt.ok()) return set_error(TJH_ERR_OOM, "cross_entropy_forward_grad: no scratch");
    KernelScope ks("loss_reduce");
    tjh_launch(k_count_valid, dim3(1), dim3(kBlock), 0, stream(), targets, rows, cols,
               ignore_index, nullptr, reduction, cnt.as<float>(), nullptr);
    int rc = check_launch("count_valid");
    if (rc != TJH_OK) return rc;
  }
  {
    KernelScope ks("cross_entropy_fwd_grad");
    tjh_launch(k_ce_fwd_grad<kCeFusedNV>, dim3((unsigned)rows), dim3(kBlock), 0, stream(),
               logits, ld, targets, cols, ignore_index, mean ? cnt.as<float>() : nullptr,
               reduction, lse, loss_rows, dlogits, ldd);
    int rc = check_launch("cross_entropy_forward_grad");
    if (rc != TJH_OK) return rc;
  }
  KernelScope ks("loss_reduce");
  tjh_launch(k_loss_reduce, dim3(1), dim3(kBlock), 0, stream(), loss_rows, targets, nullptr,
             rows, cols, ignore_index, reduction, out);
  return check_launch("loss_reduce");
}

int tjh_nll_loss_forward(const float* logp, int64_t ld, const int32_t* targets, int64_t rows,
                         int64_t cols, int32_t ignore_index, const float* weight,
                         float* loss_rows, int reduction, float* out) {
  TJH_REQUIRE_INIT();
  TJH_ARG(rows >= 0 && cols > 0 && ld >= cols, "tjh_nll_loss_forward: bad sizes");
  TJH_ARG(reduction >= 0 && reduction <= 3, "tjh_nll_loss_forward: bad reduction");
  TJH_ARG(reduction == 0 || out, "tjh_nll_loss_forward: reduction needs `out`");
  if (rows == 0) {
    if (reduction) return tjh_fill_f32(out, 1, reduction == 2 ? 0.f : __builtin_nanf(""));
    return TJH_OK;
  }
  KernelScope ks("nll_loss_fwd");
  tjh_launch(k_nll_fwd, dim3((unsigned)cdiv(rows, kBlock)), dim3(kBlock), 0, stream(),
                     logp, ld, targets, rows, cols, ignore_index, weight, loss_rows);
  int rc = check_launch("nll_loss_forward");
  if (rc != TJH_OK || !reduction) return rc;
  tjh_launch(k_loss_reduce, dim3(1), dim3(kBlock), 0, stream(), loss_rows, targets,
                     weight, rows, cols, ignore_index, reduction, out);
  return check_launch("loss_reduce");
}

int tjh_nll_loss_backward(const int32_t* targets, const float* weight, const float* grad_out,
                          int64_t rows, int64_t cols, int32_t ignore_index, int reduction,
                          float* dlogp) {
  TJH_REQUIRE_INIT();
  TJH_ARG(rows >= 0 && cols > 0, "tjh_nll_loss_backward: bad sizes");
  TJH_ARG(reduction >= 0 && reduction <= 3, "tjh_nll_loss_backward: bad reduction");
  if (rows == 0) return TJH_OK;
  const bool mean = reduction == 1 || reduction == 3;
  Scratch cnt(mean ? sizeof(float) : 0);
  if (mean) {
    if (!cnt.ok()) return set_error(TJH_ERR_OOM, "nll_loss_backward: no scratch");
    tjh_launch(k_count_valid, dim3(1), dim3(kBlock), 0, stream(), targets, rows, cols,
                       ignore_index, weight, reduction, cnt.as<float>(), nullptr);
  }
  KernelScope ks("nll_loss_bwd");
  tjh_launch(k_nll_bwd, dim3((unsigned)cdiv(rows * cols, kBlock)), dim3(kBlock), 0,
                     stream(), targets, weight, grad_out, cnt.as<float>(), rows, cols,
                     ignore_index, reduction, dlogp);
  return check_launch("nll_loss_backward");
}

int tjh_layer_norm_forward(const float* x, const float* gamma, const float* beta, float* y,
                           float* mean, float* rstd, int64_t rows, int64_t cols, float eps) {
  TJH_REQUIRE_INIT();
  TJH_ARG(rows >= 0 && cols > 0, "tjh_layer_norm_forward: bad sizes");
  TJH_ARG(mean && rstd, "tjh_layer_norm_forward: mean/rstd outputs required");
  if (rows == 0) return TJH_OK;
  KernelScope ks("layer_norm_fwd");
  bool vec = cols % 4 == 0 && aligned16(x) && aligned16(y) && (!gamma || aligned16(gamma)) &&
             (!beta || aligned16(beta));
  unsigned g = (unsigned)cdiv(rows, 4);
  if (vec && cols == 64 * 4 * 3) {
    tjh_launch((k_ln_fwd_wave<3, true>), dim3(g), dim3(kBlock), 0, stream(), x, gamma,
                       beta, y, mean, rstd, rows, cols, eps);
  } else if (vec && cols <= 64 * 4 * 4) {
    tjh_launch((k_ln_fwd_wave<4, false>), dim3(g), dim3(kBlock), 0, stream(), x, gamma,
                       beta, y, mean, rstd, rows, cols, eps);
  } else if (vec && cols <= 64 * 4 * 16) {
    tjh_launch((k_ln_fwd_wave<16, false>), dim3(g), dim3(kBlock), 0, stream(), x, gamma,
                       beta, y, mean, rstd, rows, cols, eps);
  } else {
    tjh_launch(k_ln_fwd_block, dim3((unsigned)rows), dim3(kBlock), 0, stream(), x, gamma,
                       beta, y, mean, rstd, cols, eps);
  }
  return check_launch("layer_norm_forward");
}

int tjh_layer_norm_backward(const float* dy, const float* x, const float* gamma,
                            const float* mean, const float* rstd, float* dx, float* dgamma,
                            float* dbeta, int64_t rows, int64_t cols, int accumulate) {
  return tjh_layer_norm_backward_res(dy, x, gamma, mean, rstd, nullptr, dx, dgamma, dbeta, rows,
                                     cols, accumulate ? 1 : 0);
}

int tjh_layer_norm_backward_res(const float* dy, const float* x, const float* gamma,
                                const float* mean, const float* rstd, const float* res,
                                float* dx, float* dgamma, float* dbeta, int64_t rows,
                                int64_t cols, int flags) {
  TJH_REQUIRE_INIT();
  TJH_ARG(rows >= 0 && cols > 0, "tjh_layer_norm_backward: bad sizes");
  TJH_ARG(!res || dx, "tjh_layer_norm_backward_res: res needs dx");
  TJH_ARG((flags & ~3) == 0, "tjh_layer_norm_backward: bad flags %d", flags);
  const int accumulate = flags & 1;
  const bool defer = (flags & TJH_LN_DEFER) != 0;
  if (rows == 0) {
    if (!accumulate) {
      if (dgamma) { int rc = tjh_fill_f32(dgamma, cols, 0.f); if (rc) return rc; }
      if (dbeta) { int rc = tjh_fill_f32(dbeta, cols, 0.f); if (rc) return rc; }
    }
    return TJH_OK;
  }
  bool want_p = dgamma || dbeta;
  const int v4 = ln_bwd_v4(dy, x, gamma, res, dx, cols);
  if (v4) {
    int64_t rpb, nb;
    ln_bwd_blocks(rows, rpb, nb);
    Scratch part(want_p ? (size_t)(2 * nb * cols) * sizeof(float) : 0);
    if (want_p && !part.ok()) return set_error(TJH_ERR_OOM, "layer_norm_backward: no scratch");
    float* pg = want_p ? part.as<float>() : nullptr;
    float* pb = want_p ? part.as<float>() + nb * cols : nullptr;
    {
      KernelScope ks("layer_norm_bwd");
      int rc = ln_bwd_wave_launch(v4, dy, x, gamma, mean, rstd, res, dx, pg, pb, rows, cols, rpb,
                                  nb);
      if (rc != TJH_OK) return rc;
      if (want_p && defer) {
        // dgamma and dbeta wait for tjh_flush_deferred, which finishes
        // every queued LayerNorm in one launch
        deferred_sums().push_back(DeferredSums{part.release(), {dgamma, dbeta}, nb, cols,
                                               accumulate});
      } else if (want_p) {
        // dgamma and dbeta from the per-workgroup partial rows, one launch
        float* parts[2] = {pg, pb};
        float* outs[2] = {dgamma, dbeta};
        rc = colsum_final(parts, outs, 2, nb, cols, accumulate, 1.0f);
        if (rc != TJH_OK) return rc;
      }
    }
    return TJH_OK;
  }
  // general path: partials per row, then column sums
  Scratch part(want_p ? (size_t)(2 * rows * cols) * sizeof(float) : 0);
  if (want_p && !part.ok()) return set_error(TJH_ERR_OOM, "layer_norm_backward: no scratch");
  float* pg = want_p ? part.as<float>() : nullptr;
  float* pb = want_p ? part.as<float>() + rows * cols : nullptr;
  {
    KernelScope ks("layer_norm_bwd");
    tjh_launch(k_ln_bwd_block, dim3((unsigned)rows), dim3(kBlock), 0, stream(), dy, x,
                       gamma, mean, rstd, res, dx, pg, pb, cols);
    int rc = check_launch("layer_norm_backward");
    if (rc != TJH_OK) return rc;
  }
  if (want_p) return sum_partials(pg, pb, rows, cols, dgamma, dbeta, accumulate);
  return TJH_OK;
}

}  // extern "C"

// ---------------------------------------------------------------- no-alloc
//
// tjh_layer_norm_backward_noalloc keeps the dgamma / dbeta partial rows in
// this file-scope device array instead of the caching allocator: 2 x 256
// partial rows of up to 3072 floats, the most k_ln_bwd_wave writes on a
// 256-CU MI355X (one partial row per CU; 6 MiB, held by every GPU the
// library runs on until the process ends).  Host code never passes `scratch` itself to a kernel: its
// name is a host-side stand-in there.  Its device address comes from
// hipGetSymbolAddress, taken once per device by tjh_init.

static constexpr int64_t kNoAllocFloats = 2 * 256 * 3072;
static __device__ __align__(256) float scratch[kNoAllocFloats];

namespace tjh {
namespace {
constexpr int kMaxDevices = 64;
float* g_noalloc_scratch[kMaxDevices] = {};  // device address of `scratch`, per device
}  // namespace

int noalloc_setup(int ordinal) {
  if (ordinal < 0 || ordinal >= kMaxDevices)
    return set_error(TJH_ERR_UNSUPPORTED, "device ordinal %d beyond %d", ordinal, kMaxDevices);
  if (g_noalloc_scratch[ordinal]) return TJH_OK;
  void* p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) {
    (void)hipGetLastError();
    return hip_fail(e, "hipGetSymbolAddress(scratch)");
  }
  g_noalloc_scratch[ordinal] = static_cast<float*>(p);
  return TJH_OK;
}
}  // namespace tjh

extern "C" {

int tjh_layer_norm_backward_noalloc(const float* dy, const float* x, const float* gamma,
                                    const float* mean, const float* rstd, const float* res,
                                    float* dx, float* dgamma, float* dbeta, int64_t rows,
                                    int64_t cols, int accumulate) {
  TJH_REQUIRE_INIT();
  TJH_ARG(rows >= 0 && cols > 0, "tjh_layer_norm_backward_noalloc: bad sizes");
  TJH_ARG(!res || dx, "tjh_layer_norm_backward_noalloc: res needs dx");
  TJH_ARG(mean && rstd && dy && x, "tjh_layer_norm_backward_noalloc: NULL input");
  const int dev = device_ordinal();
  float* sp = (dev >= 0 && dev < kMaxDevices) ? g_noalloc_scratch[dev] : nullptr;
  if (!sp)
    return set_error(TJH_ERR_NOT_INITIALIZED,
                     "tjh_layer_norm_backward_noalloc: no scratch address for device %d", dev);
  if (rows == 0) {
    if (!accumulate) {
      if (dgamma) { int rc = tjh_fill_f32(dgamma, cols, 0.f); if (rc) return rc; }
      if (dbeta) { int rc = tjh_fill_f32(dbeta, cols, 0.f); if (rc) return rc; }
    }
    return TJH_OK;
  }
  const int v4 = ln_bwd_v4(dy, x, gamma, res, dx, cols);
  if (!v4)
    return set_error(TJH_ERR_UNSUPPORTED,
                     "tjh_layer_norm_backward_noalloc: rows of %lld floats need a multiple of 4 "
                     "up to 3072 and 16-byte aligned operands (tjh_layer_norm_backward takes "
                     "any layout)", (long long)cols);
  const bool want_p = dgamma || dbeta;
  int64_t rpb, nb;
  ln_bwd_blocks(rows, rpb, nb);
  if (want_p && 2 * nb * cols > kNoAllocFloats)
    return set_error(TJH_ERR_INVALID,
                     "tjh_layer_norm_backward_noalloc: %lld partial floats exceed the %lld-float "
                     "scratch", (long long)(2 * nb * cols), (long long)kNoAllocFloats);
  // the kernel overwrites every partial row it owns: nothing to clear
  float* pg = want_p ? sp : nullptr;
  float* pb = want_p ? sp + nb * cols : nullptr;
  int rc = ln_bwd_wave_launch(v4, dy, x, gamma, mean, rstd, res, dx, pg, pb, rows, cols, rpb, nb);
  if (rc != TJH_OK || !want_p) return rc;
  float* parts[2] = {pg, pb};
  float* outs[2] = {dgamma, dbeta};
  return colsum_final(parts, outs, 2, nb, cols, accumulate ? 1 : 0, 1.0f);
}

int tjh_flush_deferred(void) {
  TJH_REQUIRE_INIT();
  std::vector<DeferredSums>& q = deferred_sums();
  int rc = TJH_OK;
  {
    KernelScope ks("layer_norm_bwd");
    // one colsum_final launch per run of entries with the same shape
    size_t i = 0;
    while (i < q.size() && rc == TJH_OK) {
      float* parts[kFinalMax];
      float* outs[kFinalMax];
      int np = 0;
      size_t j = i;
      while (j < q.size() && np + 2 <= kFinalMax && q[j].nb == q[i].nb &&
             q[j].cols == q[i].cols && q[j].accumulate == q[i].accumulate) {
        float* base = static_cast<float*>(q[j].part);
        parts[np] = base;
        outs[np++] = q[j].outs[0];
        parts[np] = base + q[j].nb * q[j].cols;
        outs[np++] = q[j].outs[1];
        ++j;
      }
      rc = colsum_final(parts, outs, np, q[i].nb, q[i].cols, q[i].accumulate, 1.0f);
      i = j;
    }
  }
  for (DeferredSums& e : q) scratch_free(e.part);
  q.clear();
  return rc;
}

}  // extern "C"
