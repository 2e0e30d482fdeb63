// Elementwise kernels: fill, RNG, strided copies, unary / binary / ternary /
// scalar ops and their backward helpers, masked_fill and comparisons.
//
// Layout strategy.  Every call is first reduced on the host to the fewest
// dimensions (size-1 dims dropped, adjacent dims merged when every operand
// is contiguous across them).  Then:
//   * 1-D or 2-D [R, C] layouts where each input is contiguous, a row
//     vector (stride [0,1]), a column vector ([1,0]) or a scalar take a
//     128-bit vectorised grid-stride kernel (one float4 per lane per step);
//   * anything else takes a generic strided kernel (<= 8 dims).
// The reference's counterparts are elementwise.wgsl:5-31,
// broadcast.wgsl:28-175, scalar.wgsl:10-67, unary.wgsl:5-252,
// expand.wgsl, transpose(_nd).wgsl, slice(_backward).wgsl,
// masked_fill.wgsl, fill.wgsl and random.wgsl.

#include "common.h"
#include "ew_ops.h"

#include <string.h>

namespace tjh {
namespace {

constexpr int kBlock = 256;

// ------------------------------------------------------------ layouts

constexpr int kMaxOps = 4;  // out + up to 3 inputs

struct Layout {
  int ndim;
  int64_t shape[TJH_MAX_DIMS];
  int64_t st[kMaxOps][TJH_MAX_DIMS];
};

// Builds a coalesced layout for `nops` operands.  Returns numel.
int64_t make_layout(Layout& L, int ndim, const int64_t* shape, int nops,
                    const int64_t* const* strides) {
  int64_t n = 1;
  int k = 0;
  for (int d = 0; d < ndim; ++d) {
    n *= shape[d];
    if (shape[d] == 1) continue;
    L.shape[k] = shape[d];
    for (int o = 0; o < nops; ++o) L.st[o][k] = strides[o][d];
    ++k;
  }
  if (k == 0) {
    L.shape[0] = 1;
    for (int o = 0; o < nops; ++o) L.st[o][0] = 1;
    k = 1;
  }
  // merge dim d into d+1 when contiguous across them for every operand
  int m = 0;
  for (int d = 1; d < k; ++d) {
    bool ok = true;
    for (int o = 0; o < nops; ++o)
      if (L.st[o][m] != L.st[o][d] * L.shape[d]) { ok = false; break; }
    if (ok) {
      L.shape[m] *= L.shape[d];
      for (int o = 0; o < nops; ++o) L.st[o][m] = L.st[o][d];
    } else {
      ++m;
      L.shape[m] = L.shape[d];
      for (int o = 0; o < nops; ++o) L.st[o][m] = L.st[o][d];
    }
  }
  L.ndim = m + 1;
  return n;
}

// Operand kinds for the vectorised 2-D path.
enum Kind { K_CONTIG = 0, K_ROW = 1, K_COL = 2, K_SCALAR = 3, K_NONE = 4 };

// Classifies operand `o` of a layout with <= 2 dims whose output (operand
// 0) is contiguous.  Returns K_NONE when not one of the simple kinds.
int classify(const Layout& L, int o) {
  if (L.ndim == 1) {
    if (L.st[o][0] == 1) return K_CONTIG;
    if (L.st[o][0] == 0) return K_SCALAR;
    return K_NONE;
  }
  if (L.ndim != 2) return K_NONE;
  int64_t C = L.shape[1];
  int64_t s0 = L.st[o][0], s1 = L.st[o][1];
  if (s0 == C && s1 == 1) return K_CONTIG;
  if (s0 == 0 && s1 == 1) return K_ROW;
  if (s0 == 1 && s1 == 0) return K_COL;
  if (s0 == 0 && s1 == 0) return K_SCALAR;
  return K_NONE;
}

bool out_contiguous(const Layout& L) {
  int64_t s = 1;
  for (int d = L.ndim - 1; d >= 0; --d) {
    if (L.st[0][d] != s) return false;
    s *= L.shape[d];
  }
  return true;
}

int grid_for(int64_t work_items) {
  int64_t g = cdiv(work_items, kBlock);
  int64_t cap = (int64_t)num_cus() * 32;
  if (cap < 1) cap = 1024;
  if (g > cap) g = cap;
  if (g < 1) g = 1;
  return (int)g;
}

// ------------------------------------------------------------ op tables

// Ops whose backward reads the saved output y.
bool unary_bwd_needs_y(int op) {
  return op == TJH_UNARY_EXP || op == TJH_UNARY_SQRT || op == TJH_UNARY_RSQRT ||
         op == TJH_UNARY_TANH || op == TJH_UNARY_SIGMOID ||
         op == TJH_UNARY_RECIPROCAL;
}
bool unary_bwd_needs_x(int op) {
  return !(op == TJH_UNARY_NEG || unary_bwd_needs_y(op));
}

// ------------------------------------------------------------ loaders

template <int K>
__device__ __forceinline__ float4 ld4(const float* __restrict__ p, uint32_t i,
                                      uint32_t C) {
  if constexpr (K == K_CONTIG) {
    return *reinterpret_cast<const float4*>(p + i);
  } else if constexpr (K == K_ROW) {
    return *reinterpret_cast<const float4*>(p + (i % C));
  } else if constexpr (K == K_COL) {
    float v = p[i / C];
    return make_float4(v, v, v, v);
  } else {
    float v = p[0];
    return make_float4(v, v, v, v);
  }
}

template <int K>
__device__ __forceinline__ float ld1(const float* __restrict__ p, uint32_t i,
                                     uint32_t C) {
  if constexpr (K == K_CONTIG) return p[i];
  else if constexpr (K == K_ROW) return p[i % C];
  else if constexpr (K == K_COL) return p[i / C];
  else return p[0];
}

// ------------------------------------------------------------ kernels

// Functor-style element op over up to three inputs.
struct UnaryOp {
  int op; float alpha;
  __device__ float operator()(float x, float, float) const { return unary_f(op, x, alpha); }
};
template <int OP>
struct UnaryOpT {
  float alpha;
  __device__ float operator()(float x, float, float) const { return unary_f(OP, x, alpha); }
};
template <int OP>
struct UnaryBwdT {  // inputs: g, x, y
  float alpha;
  __device__ float operator()(float g, float x, float y) const {
    return unary_bwd_f(OP, g, x, y, alpha);
  }
};
template <int OP>
struct BinaryT {
  __device__ float operator()(float a, float b, float) const { return binary_f(OP, a, b); }
};
template <int OP>
struct CmpT {
  __device__ float operator()(float a, float b, float) const { return cmp_f(OP, a, b); }
};
template <int OP>
struct TernaryT {
  __device__ float operator()(float g, float a, float b) const { return ternary_f(OP, g, a, b); }
};
template <int OP, bool REV>
struct ScalarT {
  float s;
  __device__ float operator()(float x, float, float) const {
    return REV ? scalar_rev_f(OP, x, s) : scalar_f(OP, x, s);
  }
};
struct PowScalarBwd {
  float s;
  __device__ float operator()(float g, float x, float) const {
    return g * s * pow_js(x, s - 1.0f);
  }
};
struct Axpy {
  float alpha;
  __device__ float operator()(float x, float y, float) const { return axpy_f(alpha, x, y); }
};
struct CopyOp {
  __device__ float operator()(float x, float, float) const { return x; }
};

// Vectorised kernel over a 1-D/2-D layout with contiguous output.
// NIN inputs of kinds KA, KB, KC; n elements, C = row length (2-D kinds).
// Each lane handles kUnroll float4 per step, all loads issued before any
// store, so a workgroup keeps kUnroll x 4 KiB per input in flight.
constexpr int kUnroll = 4;

template <int NIN, int KA, int KB, int KC, class F>
__global__ __launch_bounds__(kBlock) void k_vec(
    const float* __restrict__ a, const float* __restrict__ b,
    const float* __restrict__ c, float* __restrict__ out, uint32_t n,
    uint32_t C, F f) {
  const uint32_t n4 = n >> 2;
  const uint32_t stride = gridDim.x * blockDim.x * kUnroll;
  for (uint32_t v0 = blockIdx.x * blockDim.x * kUnroll + threadIdx.x; v0 < n4; v0 += stride) {
    float4 xa[kUnroll], xb[kUnroll], xc[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t v = v0 + u * blockDim.x;
      if (v < n4) {
        const uint32_t i = v << 2;
        xa[u] = ld4<KA>(a, i, C);
        xb[u] = NIN > 1 ? ld4<KB>(b, i, C) : xa[u];
        xc[u] = NIN > 2 ? ld4<KC>(c, i, C) : xa[u];
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t v = v0 + u * blockDim.x;
      if (v < n4) {
        float4 r;
        r.x = f(xa[u].x, xb[u].x, xc[u].x);
        r.y = f(xa[u].y, xb[u].y, xc[u].y);
        r.z = f(xa[u].z, xb[u].z, xc[u].z);
        r.w = f(xa[u].w, xb[u].w, xc[u].w);
        *reinterpret_cast<float4*>(out + (v << 2)) = r;
      }
    }
  }
  const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t tail = n - (n4 << 2);
  if (gid < tail) {
    uint32_t i = (n4 << 2) + gid;
    float xa = ld1<KA>(a, i, C);
    float xb = NIN > 1 ? ld1<KB>(b, i, C) : xa;
    float xc = NIN > 2 ? ld1<KC>(c, i, C) : xa;
    out[i] = f(xa, xb, xc);
  }
}

// Scalar (non-vector) version of the same, for unaligned pointers or 2-D
// layouts whose row length is not a multiple of 4.
template <int NIN, int KA, int KB, int KC, class F>
__global__ __launch_bounds__(kBlock) void k_scalar1(
    const float* __restrict__ a, const float* __restrict__ b,
    const float* __restrict__ c, float* __restrict__ out, uint32_t n,
    uint32_t C, F f) {
  uint32_t stride = gridDim.x * blockDim.x;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    float xa = ld1<KA>(a, i, C);
    float xb = NIN > 1 ? ld1<KB>(b, i, C) : xa;
    float xc = NIN > 2 ? ld1<KC>(c, i, C) : xa;
    out[i] = f(xa, xb, xc);
  }
}

// Generic strided kernel: operand 0 is the output.
template <int NIN, typename I, class F>
__global__ __launch_bounds__(kBlock) void k_strided(
    const float* __restrict__ a, const float* __restrict__ b,
    const float* __restrict__ c, float* __restrict__ out, Layout L, I n, F f) {
  I stride = (I)gridDim.x * blockDim.x;
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    I rem = i;
    I off[kMaxOps] = {0, 0, 0, 0};
    for (int d = L.ndim - 1; d >= 0; --d) {
      I s = (I)L.shape[d];
      I coord = rem % s;
      rem /= s;
#pragma unroll
      for (int o = 0; o <= NIN; ++o) off[o] += coord * (I)L.st[o][d];
    }
    float xa = a[off[1]];
    float xb = NIN > 1 ? b[off[2]] : xa;
    float xc = NIN > 2 ? c[off[3]] : xa;
    out[off[0]] = f(xa, xb, xc);
  }
}

// Maximum |offset| reachable by operand o.
int64_t max_offset(const Layout& L, int o) {
  int64_t m = 0;
  for (int d = 0; d < L.ndim; ++d) m += (L.shape[d] - 1) * (L.st[o][d] < 0 ? -L.st[o][d] : L.st[o][d]);
  return m;
}

template <int NIN, int KA, int KB, int KC, class F>
void launch_vec_kinds(const float* a, const float* b, const float* c, float* out,
                      int64_t n, int64_t C, bool vec, F f) {
  if (vec) {
    int g = grid_for(cdiv(n, 4 * kUnroll));
    tjh_launch((k_vec<NIN, KA, KB, KC, F>), dim3(g), dim3(kBlock), 0,
                       stream(), a, b, c, out, (uint32_t)n, (uint32_t)C, f);
  } else {
    int g = grid_for(n);
    tjh_launch((k_scalar1<NIN, KA, KB, KC, F>), dim3(g), dim3(kBlock), 0,
                       stream(), a, b, c, out, (uint32_t)n, (uint32_t)C, f);
  }
}

// Dispatch on operand kinds (each input one of 4 kinds).
template <int NIN, class F>
bool launch_fast(const Layout& L, const float* a, const float* b, const float* c,
                 float* out, int64_t n, F f) {
  if (n >= (int64_t(1) << 31)) return false;
  if (!out_contiguous(L)) return false;
  int ka = classify(L, 1);
  int kb = NIN > 1 ? classify(L, 2) : K_CONTIG;
  int kc = NIN > 2 ? classify(L, 3) : K_CONTIG;
  if (ka == K_NONE || kb == K_NONE || kc == K_NONE) return false;
  int64_t C = L.ndim == 2 ? L.shape[1] : n;
  bool rowish = (ka == K_ROW || ka == K_COL || kb == K_ROW || kb == K_COL ||
                 kc == K_ROW || kc == K_COL);
  bool vec = aligned16(out) && aligned16(a) && (NIN < 2 || aligned16(b)) &&
             (NIN < 3 || aligned16(c)) && (!rowish || (C % 4) == 0);
  // scalar-kind operands need no alignment
  if (ka == K_SCALAR || kb == K_SCALAR || kc == K_SCALAR) {
    vec = aligned16(out) && (ka == K_SCALAR || aligned16(a)) &&
          (NIN < 2 || kb == K_SCALAR || aligned16(b)) &&
          (NIN < 3 || kc == K_SCALAR || aligned16(c)) && (!rowish || (C % 4) == 0);
  }
#define TJH_KB(KA_, KB_, KC_)                                                        \
  if (ka == KA_ && kb == KB_ && kc == KC_) {                                         \
    launch_vec_kinds<NIN, KA_, KB_, KC_>(a, b, c, out, n, C, vec, f);                \
    return true;                                                                     \
  }
  if constexpr (NIN == 1) {
    TJH_KB(K_CONTIG, K_CONTIG, K_CONTIG)
    TJH_KB(K_ROW, K_CONTIG, K_CONTIG)
    TJH_KB(K_COL, K_CONTIG, K_CONTIG)
    TJH_KB(K_SCALAR, K_CONTIG, K_CONTIG)
  } else if constexpr (NIN == 2) {
    TJH_KB(K_CONTIG, K_CONTIG, K_CONTIG)
    TJH_KB(K_CONTIG, K_ROW, K_CONTIG)
    TJH_KB(K_ROW, K_CONTIG, K_CONTIG)
    TJH_KB(K_CONTIG, K_COL, K_CONTIG)
    TJH_KB(K_COL, K_CONTIG, K_CONTIG)
    TJH_KB(K_CONTIG, K_SCALAR, K_CONTIG)
    TJH_KB(K_SCALAR, K_CONTIG, K_CONTIG)
    TJH_KB(K_ROW, K_COL, K_CONTIG)
    TJH_KB(K_COL, K_ROW, K_CONTIG)
  } else {
    TJH_KB(K_CONTIG, K_CONTIG, K_CONTIG)
    TJH_KB(K_ROW, K_CONTIG, K_CONTIG)
    TJH_KB(K_CONTIG, K_ROW, K_CONTIG)
    TJH_KB(K_CONTIG, K_CONTIG, K_ROW)
    TJH_KB(K_COL, K_CONTIG, K_CONTIG)
    TJH_KB(K_CONTIG, K_COL, K_CONTIG)
    TJH_KB(K_CONTIG, K_CONTIG, K_COL)
  }
#undef TJH_KB
  return false;
}

template <int NIN, class F>
void launch_strided(const Layout& L, const float* a, const float* b,
                    const float* c, float* out, int64_t n, F f) {
  bool small = n < (int64_t(1) << 31);
  for (int o = 0; o <= NIN && small; ++o) small = max_offset(L, o) < (int64_t(1) << 31);
  int g = grid_for(n);
  if (small) {
    tjh_launch((k_strided<NIN, uint32_t, F>), dim3(g), dim3(kBlock), 0,
                       stream(), a, b, c, out, L, (uint32_t)n, f);
  } else {
    tjh_launch((k_strided<NIN, int64_t, F>), dim3(g), dim3(kBlock), 0,
                       stream(), a, b, c, out, L, n, f);
  }
}

// Full elementwise launch: layout build, fast path or strided path.
template <int NIN, class F>
int run_elementwise(const char* name, int ndim, const int64_t* shape,
                    const int64_t* out_strides, const float* a,
                    const int64_t* a_st, const float* b, const int64_t* b_st,
                    const float* c, const int64_t* c_st, float* out, F f) {
  TJH_ARG(ndim >= 0 && ndim <= TJH_MAX_DIMS, "%s: ndim %d out of range", name, ndim);
  int64_t zero_shape[1] = {1};
  int64_t unit[1] = {1};
  const int64_t* strides[kMaxOps] = {out_strides, a_st, b_st, c_st};
  if (ndim == 0) {
    shape = zero_shape;
    for (int o = 0; o <= NIN; ++o) strides[o] = unit;
    ndim = 1;
  }
  for (int d = 0; d < ndim; ++d)
    TJH_ARG(shape[d] >= 0, "%s: negative dimension", name);
  Layout L;
  int64_t n = make_layout(L, ndim, shape, NIN + 1, strides);
  if (n == 0) return TJH_OK;
  KernelScope ks(name);
  if (!launch_fast<NIN>(L, a, b, c, out, n, f)) launch_strided<NIN>(L, a, b, c, out, n, f);
  return check_launch(name);
}

void contiguous_strides(int ndim, const int64_t* shape, int64_t* st) {
  int64_t s = 1;
  for (int d = ndim - 1; d >= 0; --d) {
    st[d] = s;
    s *= shape[d];
  }
}

// 1-D contiguous helper.
template <int NIN, class F>
int run_contig(const char* name, const float* a, const float* b, const float* c,
               float* out, int64_t n, F f) {
  TJH_ARG(n >= 0, "%s: negative length", name);
  if (n == 0) return TJH_OK;
  int64_t st[1] = {1};
  return run_elementwise<NIN>(name, 1, &n, st, a, st, b, st, c, st, out, f);
}

// ------------------------------------------------------------ fill / rng

template <typename T>
__global__ __launch_bounds__(kBlock) void k_fill(T* __restrict__ out, int64_t n, T v) {
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = v;
}

__global__ __launch_bounds__(kBlock) void k_fill4(float4* __restrict__ out, int64_t n4, float v) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x * kUnroll;
  const float4 q = make_float4(v, v, v, v);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x * kUnroll + threadIdx.x; i < n4; i += stride)
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (i + u * blockDim.x < n4) out[i + u * blockDim.x] = q;
}

__device__ __forceinline__ uint32_t xorshift32(uint32_t x) {
  x ^= x << 13;
  x ^= x >> 17;
  x ^= x << 5;
  return x;
}

// random.wgsl:9-46: state = seed ^ (idx*1664525 + 1013904223) (mod 2^32),
// one xorshift step; uniform = u / 2^32; normal = Box-Muller (cos branch)
// of two successive states with u1 clamped to >= 1e-7.
__global__ __launch_bounds__(kBlock) void k_random(float* __restrict__ out, int64_t n,
                                                   uint32_t seed, int normal) {
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    uint32_t idx = (uint32_t)i;
    uint32_t s1 = xorshift32(seed ^ (idx * 1664525u + 1013904223u));
    float u1 = (float)s1 / 4294967296.0f;
    if (!normal) {
      out[i] = u1;
    } else {
      uint32_t s2 = xorshift32(s1);
      float u2 = (float)s2 / 4294967296.0f;
      float r = sqrtf(-2.0f * logf(fmaxf(u1, 1e-7f)));
      out[i] = r * cosf(6.283185307179586f * u2);
    }
  }
}

// ------------------------------------------------------------ int32 / uint8 copies

template <typename T>
__global__ __launch_bounds__(kBlock) void k_copy_t(const T* __restrict__ src, T* __restrict__ dst,
                                                   Layout L, int64_t n) {
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    int64_t rem = i, so = 0, dof = 0;
    for (int d = L.ndim - 1; d >= 0; --d) {
      int64_t coord = rem % L.shape[d];
      rem /= L.shape[d];
      dof += coord * L.st[0][d];
      so += coord * L.st[1][d];
    }
    dst[dof] = src[so];
  }
}

// dtype conversions between float32, int32, uint8 and bool (stored as
// uint8): to bool is `!= 0`; float to integer truncates toward zero; to
// uint8 keeps the low 8 bits of that integer.
template <typename S, typename D, bool TO_BOOL>
__global__ __launch_bounds__(kBlock) void k_cast(const S* __restrict__ s, D* __restrict__ d,
                                                 int64_t n) {
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const S v = s[i];
    if (TO_BOOL) d[i] = (D)(v != (S)0 ? 1 : 0);
    else if (sizeof(D) == 1 && sizeof(S) == 4) d[i] = (D)(uint32_t)(int32_t)v;
    else d[i] = (D)v;
  }
}

// triu / tril of a batch of [rows, cols] matrices (contiguous): element
// (r, c) is kept when c - r >= diagonal (upper) or c - r <= diagonal.
__global__ __launch_bounds__(kBlock) void k_triangle(const float* __restrict__ x,
                                                     float* __restrict__ out, int64_t n,
                                                     int64_t rows, int64_t cols,
                                                     int64_t diagonal, int upper) {
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const int64_t c = i % cols, r = (i / cols) % rows;
    const bool keep = upper ? (c - r >= diagonal) : (c - r <= diagonal);
    out[i] = keep ? x[i] : 0.f;
  }
}

__global__ __launch_bounds__(kBlock) void k_f2i(const float* __restrict__ s, int32_t* __restrict__ d,
                                                int64_t n) {
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    d[i] = (int32_t)s[i];
}
__global__ __launch_bounds__(kBlock) void k_i2f(const int32_t* __restrict__ s, float* __restrict__ d,
                                                int64_t n) {
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    d[i] = (float)s[i];
}

// ------------------------------------------------------------ masked fill

__global__ __launch_bounds__(kBlock) void k_masked_fill(const float* __restrict__ x,
                                                        const uint8_t* __restrict__ m,
                                                        float* __restrict__ out, Layout L,
                                                        int64_t n, float value) {
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    int64_t rem = i, oo = 0, xo = 0, mo = 0;
    for (int d = L.ndim - 1; d >= 0; --d) {
      int64_t coord = rem % L.shape[d];
      rem /= L.shape[d];
      oo += coord * L.st[0][d];
      xo += coord * L.st[1][d];
      mo += coord * L.st[2][d];
    }
    out[oo] = m[mo] ? value : x[xo];
  }
}

}  // namespace
}  // namespace tjh

using namespace tjh;

// ====================================================================== C ABI

#define TJH_UNARY_CASES(X)                                                      \
  X(TJH_UNARY_NEG) X(TJH_UNARY_EXP) X(TJH_UNARY_LOG) X(TJH_UNARY_SQRT)          \
  X(TJH_UNARY_RSQRT) X(TJH_UNARY_TANH) X(TJH_UNARY_SIGMOID) X(TJH_UNARY_RELU)   \
  X(TJH_UNARY_GELU) X(TJH_UNARY_SQUARE) X(TJH_UNARY_RECIPROCAL) X(TJH_UNARY_ERF)\
  X(TJH_UNARY_ABS) X(TJH_UNARY_SIN) X(TJH_UNARY_COS) X(TJH_UNARY_SILU)          \
  X(TJH_UNARY_LEAKY_RELU) X(TJH_UNARY_ELU) X(TJH_UNARY_SOFTPLUS) X(TJH_UNARY_SIGN)

extern "C" {

int tjh_fill_f32(float* out, int64_t n, float value) {
  TJH_REQUIRE_INIT();
  TJH_ARG(n >= 0 && (out || n == 0), "tjh_fill_f32: bad arguments");
  if (n == 0) return TJH_OK;
  KernelScope ks("fill");
  if (aligned16(out) && n % 4 == 0) {
    tjh_launch(k_fill4, dim3(grid_for(cdiv(n / 4, kUnroll))), dim3(kBlock), 0, stream(),
                       reinterpret_cast<float4*>(out), n / 4, value);
  } else {
    tjh_launch(k_fill<float>, dim3(grid_for(n)), dim3(kBlock), 0, stream(), out, n, value);
  }
  return check_launch("fill");
}

int tjh_fill_i32(int32_t* out, int64_t n, int32_t value) {
  TJH_REQUIRE_INIT();
  TJH_ARG(n >= 0 && (out || n == 0), "tjh_fill_i32: bad arguments");
  if (n == 0) return TJH_OK;
  KernelScope ks("fill");
  tjh_launch(k_fill<int32_t>, dim3(grid_for(n)), dim3(kBlock), 0, stream(), out, n, value);
  return check_launch("fill_i32");
}

int tjh_random(float* out, int64_t n, uint32_t seed, int normal) {
  TJH_REQUIRE_INIT();
  TJH_ARG(n >= 0 && (out || n == 0), "tjh_random: bad arguments");
  if (n == 0) return TJH_OK;
  KernelScope ks("random");
  tjh_launch(k_random, dim3(grid_for(n)), dim3(kBlock), 0, stream(), out, n, seed, normal);
  return check_launch("random");
}

int tjh_copy_strided(int ndim, const int64_t* shape, const float* src,
                     const int64_t* src_strides, float* dst, const int64_t* dst_strides) {
  TJH_REQUIRE_INIT();
  TJH_ARG(ndim == 0 || (shape && src_strides && dst_strides), "tjh_copy_strided: NULL shape/strides");
  return run_elementwise<1>("copy_strided", ndim, shape, dst_strides, src, src_strides,
                            nullptr, nullptr, nullptr, nullptr, dst, CopyOp{});
}

int tjh_copy_strided_i32(int ndim, const int64_t* shape, const int32_t* src,
                         const int64_t* src_strides, int32_t* dst, const int64_t* dst_strides) {
  TJH_REQUIRE_INIT();
  TJH_ARG(ndim >= 0 && ndim <= TJH_MAX_DIMS, "tjh_copy_strided_i32: ndim out of range");
  int64_t one = 1, unit = 1;
  if (ndim == 0) { shape = &one; src_strides = &unit; dst_strides = &unit; ndim = 1; }
  const int64_t* st[2] = {dst_strides, src_strides};
  Layout L;
  int64_t n = make_layout(L, ndim, shape, 2, st);
  if (n == 0) return TJH_OK;
  KernelScope ks("copy_strided_i32");
  tjh_launch(k_copy_t<int32_t>, dim3(grid_for(n)), dim3(kBlock), 0, stream(), src, dst, L, n);
  return check_launch("copy_strided_i32");
}

int tjh_copy_strided_u8(int ndim, const int64_t* shape, const uint8_t* src,
                        const int64_t* src_strides, uint8_t* dst, const int64_t* dst_strides) {
  TJH_REQUIRE_INIT();
  TJH_ARG(ndim >= 0 && ndim <= TJH_MAX_DIMS, "tjh_copy_strided_u8: ndim out of range");
  int64_t one = 1, unit = 1;
  if (ndim == 0) { shape = &one; src_strides = &unit; dst_strides = &unit; ndim = 1; }
  const int64_t* st[2] = {dst_strides, src_strides};
  Layout L;
  int64_t n = make_layout(L, ndim, shape, 2, st);
  if (n == 0) return TJH_OK;
  KernelScope ks("copy_strided_u8");
  tjh_launch(k_copy_t<uint8_t>, dim3(grid_for(n)), dim3(kBlock), 0, stream(), src, dst, L, n);
  return check_launch("copy_strided_u8");
}

int tjh_fill_u8(uint8_t* out, int64_t n, uint8_t value) {
  TJH_REQUIRE_INIT();
  TJH_ARG(n >= 0 && (out || n == 0), "tjh_fill_u8: bad arguments");
  if (n == 0) return TJH_OK;
  KernelScope ks("fill");
  tjh_launch(k_fill<uint8_t>, dim3(grid_for(n)), dim3(kBlock), 0, stream(), out, n, value);
  return check_launch("fill_u8");
}

int tjh_cast(int src_dtype, int dst_dtype, const void* src, void* dst, int64_t n) {
  TJH_REQUIRE_INIT();
  TJH_ARG(src_dtype >= 0 && src_dtype < TJH_DTYPE_COUNT && dst_dtype >= 0 &&
              dst_dtype < TJH_DTYPE_COUNT, "tjh_cast: unknown dtype %d -> %d", src_dtype,
          dst_dtype);
  TJH_ARG(n >= 0 && ((src && dst) || n == 0), "tjh_cast: bad arguments");
  if (n == 0) return TJH_OK;
  KernelScope ks("cast");
  const dim3 g(grid_for(n)), b(kBlock);
  const bool to_bool = dst_dtype == TJH_DTYPE_BOOL;
  const int sk = src_dtype == TJH_DTYPE_BOOL ? TJH_DTYPE_U8 : src_dtype;
  const int dk = to_bool ? TJH_DTYPE_U8 : dst_dtype;
  const float* sf = static_cast<const float*>(src);
  const int32_t* si = static_cast<const int32_t*>(src);
  const uint8_t* su = static_cast<const uint8_t*>(src);
  float* df = static_cast<float*>(dst);
  int32_t* di = static_cast<int32_t*>(dst);
  uint8_t* du = static_cast<uint8_t*>(dst);
  if (sk == TJH_DTYPE_F32 && dk == TJH_DTYPE_F32) tjh_launch(k_cast<float, float, false>, g, b, 0, stream(), sf, df, n);
  else if (sk == TJH_DTYPE_F32 && dk == TJH_DTYPE_I32) tjh_launch(k_cast<float, int32_t, false>, g, b, 0, stream(), sf, di, n);
  else if (sk == TJH_DTYPE_F32 && to_bool) tjh_launch(k_cast<float, uint8_t, true>, g, b, 0, stream(), sf, du, n);
  else if (sk == TJH_DTYPE_F32) tjh_launch(k_cast<float, uint8_t, false>, g, b, 0, stream(), sf, du, n);
  else if (sk == TJH_DTYPE_I32 && dk == TJH_DTYPE_F32) tjh_launch(k_cast<int32_t, float, false>, g, b, 0, stream(), si, df, n);
  else if (sk == TJH_DTYPE_I32 && dk == TJH_DTYPE_I32) tjh_launch(k_cast<int32_t, int32_t, false>, g, b, 0, stream(), si, di, n);
  else if (sk == TJH_DTYPE_I32 && to_bool) tjh_launch(k_cast<int32_t, uint8_t, true>, g, b, 0, stream(), si, du, n);
  else if (sk == TJH_DTYPE_I32) tjh_launch(k_cast<int32_t, uint8_t, false>, g, b, 0, stream(), si, du, n);
  else if (dk == TJH_DTYPE_F32) tjh_launch(k_cast<uint8_t, float, false>, g, b, 0, stream(), su, df, n);
  else if (dk == TJH_DTYPE_I32) tjh_launch(k_cast<uint8_t, int32_t, false>, g, b, 0, stream(), su, di, n);
  else if (to_bool) tjh_launch(k_cast<uint8_t, uint8_t, true>, g, b, 0, stream(), su, du, n);
  else tjh_launch(k_cast<uint8_t, uint8_t, false>, g, b, 0, stream(), su, du, n);
  return check_launch("cast");
}

int tjh_triangle(const float* x, float* out, int64_t batch, int64_t rows, int64_t cols,
                 int64_t diagonal, int upper) {
  TJH_REQUIRE_INIT();
  TJH_ARG(batch >= 0 && rows >= 0 && cols >= 0, "tjh_triangle: bad sizes");
  const int64_t n = batch * rows * cols;
  if (n == 0) return TJH_OK;
  TJH_ARG(x && out, "tjh_triangle: NULL pointer");
  KernelScope ks("triangle");
  tjh_launch(k_triangle, dim3(grid_for(n)), dim3(kBlock), 0, stream(), x, out, n, rows, cols,
             diagonal, upper);
  return check_launch("triangle");
}

int tjh_cast_f32_i32(const float* src, int32_t* dst, int64_t n) {
  TJH_REQUIRE_INIT();
  if (n <= 0) return TJH_OK;
  KernelScope ks("cast");
  tjh_launch(k_f2i, dim3(grid_for(n)), dim3(kBlock), 0, stream(), src, dst, n);
  return check_launch("cast_f32_i32");
}

int tjh_cast_i32_f32(const int32_t* src, float* dst, int64_t n) {
  TJH_REQUIRE_INIT();
  if (n <= 0) return TJH_OK;
  KernelScope ks("cast");
  tjh_launch(k_i2f, dim3(grid_for(n)), dim3(kBlock), 0, stream(), src, dst, n);
  return check_launch("cast_i32_f32");
}

int tjh_unary(int op, const float* x, float* out, int64_t n, float alpha) {
  TJH_REQUIRE_INIT();
  TJH_ARG(op >= 0 && op < TJH_UNARY_COUNT, "tjh_unary: unknown op %d", op);
  switch (op) {
#define X(OPC) case OPC: return run_contig<1>("unary", x, nullptr, nullptr, out, n, UnaryOpT<OPC>{alpha});
    TJH_UNARY_CASES(X)
#undef X
  }
  return set_error(TJH_ERR_INVALID, "tjh_unary: unknown op %d", op);
}

int tjh_unary_backward(int op, const float* g, const float* x, const float* y, float* out,
                       int64_t n, float alpha) {
  TJH_REQUIRE_INIT();
  TJH_ARG(op >= 0 && op < TJH_UNARY_COUNT, "tjh_unary_backward: unknown op %d", op);
  TJH_ARG(!unary_bwd_needs_y(op) || y, "tjh_unary_backward: op %d needs the saved output", op);
  TJH_ARG(!unary_bwd_needs_x(op) || x, "tjh_unary_backward: op %d needs the saved input", op);
  // unused operands alias g so the loaders read valid memory
  const float* xx = x ? x : g;
  const float* yy = y ? y : g;
  switch (op) {
#define X(OPC) case OPC: return run_contig<3>("unary_backward", g, xx, yy, out, n, UnaryBwdT<OPC>{alpha});
    TJH_UNARY_CASES(X)
#undef X
  }
  return set_error(TJH_ERR_INVALID, "tjh_unary_backward: unknown op %d", op);
}

int tjh_binary(int op, int ndim, const int64_t* shape, const float* a, const int64_t* a_strides,
               const float* b, const int64_t* b_strides, float* out) {
  TJH_REQUIRE_INIT();
  TJH_ARG(ndim >= 0 && ndim <= TJH_MAX_DIMS, "tjh_binary: ndim %d out of range", ndim);
  int64_t ost[TJH_MAX_DIMS];
  contiguous_strides(ndim, shape, ost);
  switch (op) {
#define B(OPC) case OPC: return run_elementwise<2>("binary", ndim, shape, ost, a, a_strides, b, b_strides, nullptr, nullptr, out, BinaryT<OPC>{});
    B(TJH_BINARY_ADD) B(TJH_BINARY_SUB) B(TJH_BINARY_MUL) B(TJH_BINARY_DIV)
    B(TJH_BINARY_POW) B(TJH_BINARY_MAXIMUM) B(TJH_BINARY_MINIMUM)
#undef B
  }
  return set_error(TJH_ERR_INVALID, "tjh_binary: unknown op %d", op);
}

int tjh_compare(int op, int ndim, const int64_t* shape, const float* a, const int64_t* a_strides,
                const float* b, const int64_t* b_strides, float* out) {
  TJH_REQUIRE_INIT();
  TJH_ARG(ndim >= 0 && ndim <= TJH_MAX_DIMS, "tjh_compare: ndim %d out of range", ndim);
  int64_t ost[TJH_MAX_DIMS];
  contiguous_strides(ndim, shape, ost);
  switch (op) {
#define C(OPC) case OPC: return run_elementwise<2>("compare", ndim, shape, ost, a, a_strides, b, b_strides, nullptr, nullptr, out, CmpT<OPC>{});
    C(0) C(1) C(2) C(3) C(4) C(5)
#undef C
  }
  return set_error(TJH_ERR_INVALID, "tjh_compare: unknown op %d", op);
}

int tjh_ternary(int op, int ndim, const int64_t* shape, const float* g, const int64_t* g_strides,
                const float* a, const int64_t* a_strides, const float* b,
                const int64_t* b_strides, float* out) {
  TJH_REQUIRE_INIT();
  TJH_ARG(ndim >= 0 && ndim <= TJH_MAX_DIMS, "tjh_ternary: ndim %d out of range", ndim);
  int64_t ost[TJH_MAX_DIMS];
  contiguous_strides(ndim, shape, ost);
  switch (op) {
#define T(OPC) case OPC: return run_elementwise<3>("ternary", ndim, shape, ost, g, g_strides, a, a_strides, b, b_strides, out, TernaryT<OPC>{});
    T(TJH_TERNARY_DIV_B) T(TJH_TERNARY_POW_A) T(TJH_TERNARY_POW_B) T(TJH_TERNARY_MUL3)
#undef T
  }
  return set_error(TJH_ERR_INVALID, "tjh_ternary: unknown op %d", op);
}

int tjh_scalar(int op, const float* x, float s, int reverse, float* out, int64_t n) {
  TJH_REQUIRE_INIT();
  switch (op) {
#define S(OPC)                                                                                  \
  case OPC:                                                                                     \
    return reverse ? run_contig<1>("scalar", x, nullptr, nullptr, out, n, ScalarT<OPC, true>{s}) \
                   : run_contig<1>("scalar", x, nullptr, nullptr, out, n, ScalarT<OPC, false>{s});
    S(TJH_SCALAR_ADD) S(TJH_SCALAR_SUB) S(TJH_SCALAR_MUL) S(TJH_SCALAR_DIV)
    S(TJH_SCALAR_POW) S(TJH_SCALAR_MAXIMUM) S(TJH_SCALAR_MINIMUM)
#undef S
  }
  return set_error(TJH_ERR_INVALID, "tjh_scalar: unknown op %d", op);
}

int tjh_pow_scalar_backward(const float* g, const float* x, float s, float* out, int64_t n) {
  TJH_REQUIRE_INIT();
  return run_contig<2>("pow_scalar_backward", g, x, nullptr, out, n, PowScalarBwd{s});
}

int tjh_axpy(float alpha, const float* x, const float* y, float* out, int64_t n) {
  TJH_REQUIRE_INIT();
  return run_contig<2>("axpy", x, y, nullptr, out, n, Axpy{alpha});
}

int tjh_masked_fill(int ndim, const int64_t* shape, const float* x, const int64_t* x_strides,
                    const uint8_t* mask, const int64_t* mask_strides, float value, float* out) {
  TJH_REQUIRE_INIT();
  TJH_ARG(ndim >= 0 && ndim <= TJH_MAX_DIMS, "tjh_masked_fill: ndim out of range");
  int64_t one = 1, unit = 1;
  int64_t ost[TJH_MAX_DIMS];
  if (ndim == 0) { shape = &one; x_strides = &unit; mask_strides = &unit; ndim = 1; }
  contiguous_strides(ndim, shape, ost);
  const int64_t* st[3] = {ost, x_strides, mask_strides};
  Layout L;
  int64_t n = make_layout(L, ndim, shape, 3, st);
  if (n == 0) return TJH_OK;
  KernelScope ks("masked_fill");
  tjh_launch(k_masked_fill, dim3(grid_for(n)), dim3(kBlock), 0, stream(), x, mask, out, L,
                     n, value);
  return check_launch("masked_fill");
}

}  // extern "C"
