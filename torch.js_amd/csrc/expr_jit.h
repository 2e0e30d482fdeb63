// Device prelude of the runtime-compiled expression kernels (expr.hip).
//
// A generated kernel defines one functor that computes the value of an
// element group from its leaves in static single assignment form, one
// statement per program instruction, and hands it to eval_body or
// colsum_body below.  Each op is the ABI's scalar definition (ew_ops.h),
// and every result passes an empty asm barrier, so the compiler cannot
// contract a multiply of one op with an add of the next into a fused
// multiply-add: a fused value rounds exactly like the op-by-op kernels.
#pragma once

#include "ew_ops.h"
#include "kahan.h"

namespace tjh {
namespace jit {

constexpr int kBlock = 256;

// Kernel argument block (by value).
struct Args {
  const float* leaf[TJH_EXPR_MAX_LEAVES];
  long long period[TJH_EXPR_MAX_LEAVES];
  float f[TJH_EXPR_MAX_INS];
  float* out;     // eval: the value; colsum: the partial rows
  float* values;  // colsum: the value too (may be null)
  float* values2; // colsum: the program's second value (may be null)
  float* out3;    // colsum3: the partial rows of the third value's column sums
  long long n;    // eval: elements
  long long r, inner, rchunk;
};

template <int W>
struct V {
  float x[W];
};

__device__ __forceinline__ float opaque(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

template <int W>
__device__ __forceinline__ V<W> splat(float s) {
  V<W> v;
#pragma unroll
  for (int j = 0; j < W; ++j) v.x[j] = s;
  return v;
}

// Leaf k of kind K at element e (e % W == 0; ROW / COL periods % W == 0).
template <int W, int K>
__device__ __forceinline__ V<W> leaf(const Args& a, int k, long long e) {
  const float* __restrict__ p = a.leaf[k];
  if constexpr (K == TJH_LEAF_CONTIG || K == TJH_LEAF_ROW) {
    const long long i = K == TJH_LEAF_CONTIG ? e : e % a.period[k];
    V<W> v;
    if constexpr (W == 4) {
      const float4 q = *reinterpret_cast<const float4*>(p + i);
      v.x[0] = q.x;
      v.x[1] = q.y;
      v.x[2] = q.z;
      v.x[3] = q.w;
    } else {
#pragma unroll
      for (int j = 0; j < W; ++j) v.x[j] = p[i + j];
    }
    return v;
  } else if constexpr (K == TJH_LEAF_COL) {
    return splat<W>(p[e / a.period[k]]);
  } else {
    return splat<W>(p[0]);
  }
}

template <int W, int OP>
__device__ __forceinline__ V<W> vunary(const V<W>& x, float alpha) {
  V<W> r;
#pragma unroll
  for (int j = 0; j < W; ++j) r.x[j] = opaque(unary_f(OP, x.x[j], alpha));
  return r;
}
template <int W, int OP>
__device__ __forceinline__ V<W> vunary_bwd(const V<W>& g, const V<W>& x, const V<W>& y,
                                           float alpha) {
  V<W> r;
#pragma unroll
  for (int j = 0; j < W; ++j) r.x[j] = opaque(unary_bwd_f(OP, g.x[j], x.x[j], y.x[j], alpha));
  return r;
}
template <int W, int OP>
__device__ __forceinline__ V<W> vbinary(const V<W>& a, const V<W>& b) {
  V<W> r;
#pragma unroll
  for (int j = 0; j < W; ++j) r.x[j] = opaque(binary_f(OP, a.x[j], b.x[j]));
  return r;
}
template <int W, int OP>
__device__ __forceinline__ V<W> vternary(const V<W>& g, const V<W>& a, const V<W>& b) {
  V<W> r;
#pragma unroll
  for (int j = 0; j < W; ++j) r.x[j] = opaque(ternary_f(OP, g.x[j], a.x[j], b.x[j]));
  return r;
}
template <int W, int OP, bool REV>
__device__ __forceinline__ V<W> vscalar(const V<W>& x, float s) {
  V<W> r;
#pragma unroll
  for (int j = 0; j < W; ++j)
    r.x[j] = opaque(REV ? scalar_rev_f(OP, x.x[j], s) : scalar_f(OP, x.x[j], s));
  return r;
}
template <int W>
__device__ __forceinline__ V<W> vaxpy(float alpha, const V<W>& x, const V<W>& y) {
  V<W> r;
#pragma unroll
  for (int j = 0; j < W; ++j) r.x[j] = opaque(axpy_f(alpha, x.x[j], y.x[j]));
  return r;
}

template <int W>
__device__ __forceinline__ void store(float* __restrict__ p, const V<W>& v) {
  if constexpr (W == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(v.x[0], v.x[1], v.x[2], v.x[3]);
  } else {
#pragma unroll
    for (int j = 0; j < W; ++j) p[j] = v.x[j];
  }
}

// out[0, n) = value: U element groups of W per lane and step (all loads of
// the U groups are issued before the first store), grid-stride.
template <int W, class F>
__device__ __forceinline__ void eval_body(const F& f, const Args& a) {
  constexpr int U = 4;
  const long long groups = a.n / W;
  const long long stride = (long long)gridDim.x * kBlock;
  for (long long g0 = (long long)blockIdx.x * kBlock + threadIdx.x; g0 < groups;
       g0 += stride * U) {
    V<W> v[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (g0 + u * stride < groups) v[u] = f(a, (g0 + u * stride) * W);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (g0 + u * stride < groups) store<W>(a.out + (g0 + u * stride) * W, v[u]);
  }
}

// Column sums over r of the value viewed [outer][r][inner]: workgroup
// (b, cb, o) sums rows [b*rchunk, (b+1)*rchunk) of the W columns of lane
// cb*256 + t, compensated in increasing row order (the order of the
// library's unfused column sum), into the partial row out[o][b]; the
// value goes to `values` too when that is set.
template <int W, class F>
__device__ __forceinline__ void colsum_body(const F& f, const Args& a) {
  const long long o = blockIdx.z;
  const long long nb = gridDim.x, b = blockIdx.x;
  const long long r0 = b * a.rchunk, r1 = r0 + a.rchunk < a.r ? r0 + a.rchunk : a.r;
  const long long c = ((long long)blockIdx.y * kBlock + threadIdx.x) * W;
  if (c >= a.inner) return;
  Kahan acc[W];
  constexpr int U = 4;  // rows whose loads are in flight together
  for (long long k = r0; k < r1; k += U) {
    V<W> v[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (k + u < r1) v[u] = f(a, ((o * a.r + k + u) * a.inner) + c);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (k + u < r1) {
        if (a.values) store<W>(a.values + (o * a.r + k + u) * a.inner + c, v[u]);
#pragma unroll
        for (int j = 0; j < W; ++j) acc[j].add(v[u].x[j]);
      }
    }
  }
  V<W> s;
#pragma unroll
  for (int j = 0; j < W; ++j) s.x[j] = acc[j].s;
  store<W>(a.out + (o * nb + b) * a.inner + c, s);
}

// colsum_body for two column sums from one pass: f(a, e, &third) returns
// the first value and sets the third; both are summed over the same rows
// in the same order into out and out3 (the first value written to
// `values` too when that is set).
template <int W, class F>
__device__ __forceinline__ void colsum3_body(const F& f, const Args& a) {
  const long long o = blockIdx.z;
  const long long nb = gridDim.x, b = blockIdx.x;
  const long long r0 = b * a.rchunk, r1 = r0 + a.rchunk < a.r ? r0 + a.rchunk : a.r;
  const long long c = ((long long)blockIdx.y * kBlock + threadIdx.x) * W;
  if (c >= a.inner) return;
  Kahan acc[W], acc3[W];
  constexpr int U = 4;  // rows whose loads are in flight together (8 measured slower)
  for (long long k = r0; k < r1; k += U) {
    V<W> v[U], v3[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (k + u < r1) v[u] = f(a, ((o * a.r + k + u) * a.inner) + c, &v3[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (k + u < r1) {
        if (a.values) store<W>(a.values + (o * a.r + k + u) * a.inner + c, v[u]);
#pragma unroll
        for (int j = 0; j < W; ++j) {
          acc[j].add(v[u].x[j]);
          acc3[j].add(v3[u].x[j]);
        }
      }
    }
  }
  V<W> s, s3;
#pragma unroll
  for (int j = 0; j < W; ++j) {
    s.x[j] = acc[j].s;
    s3.x[j] = acc3[j].s;
  }
  store<W>(a.out + (o * nb + b) * a.inner + c, s);
  store<W>(a.out3 + (o * nb + b) * a.inner + c, s3);
}

}  // namespace jit
}  // namespace tjh
