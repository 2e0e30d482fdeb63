// Reductions over the middle axis of a contiguous [outer, r, inner] view:
// sum / mean / max / min / prod, and argmax / argmin.
//
// Replaces reduce_sum.wgsl (+max/min/prod), reduce_dim.wgsl and the
// broadcast-grad column sum reduce_broadcast_grad.wgsl:10-20 (torch.js
// Tensor._reduce / _reduceDim / _sumAlongDim0, Tensor.ts:2359-2425,
// 3560-3591, 3794-3906).
//
// Two shapes of work:
//  * inner == 1 ("row" reduction, e.g. a full sum or a softmax-like row):
//    a row is split over `splits` workgroups when it is long, each lane
//    accumulates float4 loads, then a wave shuffle + LDS tree combine.
//  * inner > 1 ("column" reduction, e.g. the bias gradient sum over
//    tokens): lanes own 4 adjacent columns (float4, coalesced along inner)
//    and walk a slice of r; long r is split over workgroups.
// Split reductions write partials and finish with a second pass.  Every
// split point and combine order is fixed, so results are deterministic.

#include "colsum.h"
#include "wave.h"

#include <float.h>

namespace tjh {
namespace {

constexpr int kBlock = 256;

template <int OP>
__device__ __forceinline__ float rinit() {
  if constexpr (OP == TJH_REDUCE_MAX) return -FLT_MAX;
  else if constexpr (OP == TJH_REDUCE_MIN) return FLT_MAX;
  else if constexpr (OP == TJH_REDUCE_PROD) return 1.0f;
  else return 0.0f;
}

template <int OP>
__device__ __forceinline__ float rcomb(float a, float b) {
  if constexpr (OP == TJH_REDUCE_MAX) return fmaxf(a, b);
  else if constexpr (OP == TJH_REDUCE_MIN) return fminf(a, b);
  else if constexpr (OP == TJH_REDUCE_PROD) return a * b;
  else return a + b;
}

template <int OP>
struct RComb {
  __device__ __forceinline__ float operator()(float a, float b) const { return rcomb<OP>(a, b); }
};

// The combination over the wave through the DPP network (wave.h).
template <int OP>
__device__ __forceinline__ float wave_reduce(float v) {
  return wave_reduce_dpp(v, RComb<OP>{});
}

// Block-wide reduce of one value per lane; result valid in every lane.
template <int OP>
__device__ __forceinline__ float block_reduce(float v, float* sm) {
  v = wave_reduce<OP>(v);
  int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) sm[wid] = v;
  __syncthreads();
  float r = sm[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = rcomb<OP>(r, sm[w]);
  __syncthreads();
  return r;
}

// Row reduction: grid (outer, splits). Block (o, b) reduces elements
// [b*chunk, min(r, (b+1)*chunk)) of row o.  out[o*splits + b] = result*scale.
template <int OP, bool VEC>
__global__ __launch_bounds__(kBlock) void k_reduce_rows(const float* __restrict__ x,
                                                        int64_t r, int64_t chunk,
                                                        float* __restrict__ out,
                                                        float scale) {
  __shared__ float sm[kBlock / 64];
  int64_t o = blockIdx.x;
  int64_t beg = (int64_t)blockIdx.y * chunk;
  int64_t end = beg + chunk < r ? beg + chunk : r;
  const float* row = x + o * r;
  float acc = rinit<OP>();
  if (VEC) {
    // beg and chunk are multiples of 4 and the row base is 16B aligned
    int64_t n4 = (end - beg) >> 2;
    const float4* p4 = reinterpret_cast<const float4*>(row + beg);
    for (int64_t i = threadIdx.x; i < n4; i += kBlock) {
      float4 v = p4[i];
      acc = rcomb<OP>(acc, rcomb<OP>(rcomb<OP>(v.x, v.y), rcomb<OP>(v.z, v.w)));
    }
    for (int64_t i = beg + (n4 << 2) + threadIdx.x; i < end; i += kBlock) acc = rcomb<OP>(acc, row[i]);
  } else {
    for (int64_t i = beg + threadIdx.x; i < end; i += kBlock) acc = rcomb<OP>(acc, row[i]);
  }
  float t = block_reduce<OP>(acc, sm);
  if (threadIdx.x == 0) out[o * gridDim.y + blockIdx.y] = t * scale;
}

// Short rows: one wave per row, 4 rows per block.
template <int OP>
__global__ __launch_bounds__(kBlock) void k_reduce_rows_wave(const float* __restrict__ x,
                                                             int64_t outer, int64_t r,
                                                             float* __restrict__ out,
                                                             float scale) {
  int64_t o = (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (o >= outer) return;
  const float* row = x + o * r;
  float acc = rinit<OP>();
  for (int64_t i = lane; i < r; i += 64) acc = rcomb<OP>(acc, row[i]);
  acc = wave_reduce<OP>(acc);
  if (lane == 0) out[o] = acc * scale;
}

// Column reduction: grid (gx*outer, splits) with gx = ceil(lanes/256);
// a lane owns 4 columns (VEC) or 1.  out[(o*splits + s)*inner + i] =
// reduce over r-slice s.
template <int OP, bool VEC>
__global__ __launch_bounds__(kBlock) void k_reduce_cols(const float* __restrict__ x,
                                                        int64_t r, int64_t inner,
                                                        int64_t rchunk, int64_t gx,
                                                        float* __restrict__ out,
                                                        float scale) {
  int64_t o = blockIdx.x / gx;
  int64_t bx = blockIdx.x % gx;
  int64_t s = blockIdx.y;
  int64_t splits = gridDim.y;
  int64_t r0 = s * rchunk;
  int64_t r1 = r0 + rchunk < r ? r0 + rchunk : r;
  const float* base = x + o * r * inner;
  float* dst = out + (o * splits + s) * inner;
  if (VEC) {
    int64_t c4 = bx * kBlock + threadIdx.x;
    if (c4 * 4 >= inner) return;
    float4 acc = make_float4(rinit<OP>(), rinit<OP>(), rinit<OP>(), rinit<OP>());
    for (int64_t k = r0; k < r1; ++k) {
      float4 v = *reinterpret_cast<const float4*>(base + k * inner + c4 * 4);
      acc.x = rcomb<OP>(acc.x, v.x);
      acc.y = rcomb<OP>(acc.y, v.y);
      acc.z = rcomb<OP>(acc.z, v.z);
      acc.w = rcomb<OP>(acc.w, v.w);
    }
    acc.x *= scale; acc.y *= scale; acc.z *= scale; acc.w *= scale;
    *reinterpret_cast<float4*>(dst + c4 * 4) = acc;
  } else {
    int64_t c = bx * kBlock + threadIdx.x;
    if (c >= inner) return;
    float acc = rinit<OP>();
    for (int64_t k = r0; k < r1; ++k) acc = rcomb<OP>(acc, base[k * inner + c]);
    dst[c] = acc * scale;
  }
}

// Column sums of x viewed [outer][r][inner]: workgroup (b, cb, o) sums
// rows [b*rchunk, (b+1)*rchunk) of column block cb (256 lanes of 4 or 1
// columns) of o, compensated, into the partial row part[o][b]; colsum_final
// adds the partial rows.
template <bool VEC>
__global__ __launch_bounds__(kBlock) void k_colsum(const float* __restrict__ x, int64_t r,
                                                   int64_t inner, int64_t rchunk,
                                                   float* __restrict__ part) {
  const int64_t o = blockIdx.z;
  const int64_t nb = gridDim.x, b = blockIdx.x;
  const float* __restrict__ base = x + o * r * inner;
  const int64_t r0 = b * rchunk, r1 = r0 + rchunk < r ? r0 + rchunk : r;
  float* __restrict__ prow = part + (o * nb + b) * inner;
  // rows are fetched kBatch at a time before they are accumulated, so the
  // loads of a batch are in flight together
  if (VEC) {
    const int64_t c4 = (int64_t)blockIdx.y * kBlock + threadIdx.x;
    if (c4 * 4 < inner) {
      Kahan kx, ky, kz, kw;
      const float4* __restrict__ col = reinterpret_cast<const float4*>(base + c4 * 4);
      const int64_t st = inner / 4;
      for (int64_t k = r0; k < r1; k += kBatch) {
        float4 v[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
          v[u] = k + u < r1 ? col[(k + u) * st] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          kx.add(v[u].x); ky.add(v[u].y); kz.add(v[u].z); kw.add(v[u].w);
        }
      }
      *reinterpret_cast<float4*>(prow + c4 * 4) = make_float4(kx.s, ky.s, kz.s, kw.s);
    }
  } else {
    const int64_t cc = (int64_t)blockIdx.y * kBlock + threadIdx.x;
    if (cc < inner) {
      Kahan kc;
      for (int64_t k = r0; k < r1; k += kBatch) {
        float v[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) v[u] = k + u < r1 ? base[(k + u) * inner + cc] : 0.f;
#pragma unroll
        for (int u = 0; u < kBatch; ++u) kc.add(v[u]);
      }
      prow[cc] = kc.s;
    }
  }
}

// Final pass: workgroup (x, i) owns 64 columns of output i; wave w of 16
// sums partial rows w, w+16, ... (compensated, fetched kFinalBatch at a time)
// and the 16 wave sums are added in wave order.
constexpr int kFinalWaves = 16;
// partial rows per wave fetched together: 256 partial rows (one per CU) in
// one round trip per wave
constexpr int kFinalBatch = 16;

struct FinalArgs {
  const float* part[kFinalMax];
  float* out[kFinalMax];
  int64_t cols[kFinalMax];  // row length of each output
};

__global__ __launch_bounds__(64 * kFinalWaves) void k_colsum_final(FinalArgs fa, int64_t nb,
                                                                   int accumulate, float scale) {
  __shared__ float red[kFinalWaves][64];
  const int i = blockIdx.y;
  const int64_t cols = fa.cols[i];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + lane;
  float* __restrict__ out = fa.out[i];
  const float* __restrict__ p = fa.part[i];
  Kahan k;
  if (c < cols) {
    for (int64_t b = w; b < nb; b += kFinalWaves * kFinalBatch) {
      float v[kFinalBatch];
#pragma unroll
      for (int u = 0; u < kFinalBatch; ++u) {
        const int64_t bb = b + (int64_t)u * kFinalWaves;
        v[u] = bb < nb ? p[bb * cols + c] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < kFinalBatch; ++u)
        if (b + (int64_t)u * kFinalWaves < nb) k.add(v[u]);  // rows past nb add nothing
    }
  }
  red[w][lane] = k.s;
  __syncthreads();
  if (w == 0 && c < cols) {
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < kFinalWaves; ++q) s += red[q][lane];
    s *= scale;
    out[c] = accumulate ? out[c] + s : s;
  }
}

template <int OP>
int reduce_rows(const float* x, int64_t outer, int64_t r, float* out, float scale) {
  // a single reduction level: split long rows over several workgroups
  int cus = num_cus() > 0 ? num_cus() : 256;
  if (r <= 4096 && outer >= 4) {
    int64_t g = cdiv(outer, kBlock / 64);
    tjh_launch(k_reduce_rows_wave<OP>, dim3((unsigned)g), dim3(kBlock), 0, stream(), x,
                       outer, r, out, scale);
    return check_launch("reduce_rows_wave");
  }
  int64_t splits = 1;
  if (outer < 4LL * cus) {
    int64_t want = cdiv(4LL * cus, outer);
    int64_t by_len = r / 16384;  // keep >= 16K elements per workgroup
    splits = want < by_len ? want : by_len;
    if (splits < 1) splits = 1;
    if (splits > 2048) splits = 2048;
  }
  int64_t chunk = cdiv(r, splits);
  chunk = cdiv(chunk, 4) * 4;
  splits = cdiv(r, chunk);
  bool vec = aligned16(x) && (r % 4) == 0;
  float* part = out;
  Scratch scratch(splits > 1 ? (size_t)(outer * splits) * sizeof(float) : 0);
  if (splits > 1) {
    if (!scratch.ok()) return set_error(TJH_ERR_OOM, "reduce: no scratch memory");
    part = scratch.as<float>();
  }
  dim3 grid((unsigned)outer, (unsigned)splits);
  float s1 = splits > 1 ? 1.0f : scale;
  if (vec)
    tjh_launch((k_reduce_rows<OP, true>), grid, dim3(kBlock), 0, stream(), x, r, chunk, part, s1);
  else
    tjh_launch((k_reduce_rows<OP, false>), grid, dim3(kBlock), 0, stream(), x, r, chunk, part, s1);
  int rc = check_launch("reduce_rows");
  if (rc != TJH_OK || splits == 1) return rc;
  return reduce_rows<OP>(part, outer, splits, out, scale);
}

}  // namespace

void colsum_plan(int64_t outer, int64_t r, int64_t inner, bool vec, int64_t* nb_out,
                 int64_t* rchunk_out) {
  const int cus = num_cus() > 0 ? num_cus() : 256;
  const int64_t col_waves = cdiv(vec ? inner / 4 : inner, kBlock);
  // ~4 workgroups per CU in total, >= 16 rows each
  int64_t nb = cdiv(4LL * cus, outer * col_waves);
  if (nb > cdiv(r, 16)) nb = cdiv(r, 16);
  if (nb < 1) nb = 1;
  const int64_t rchunk = cdiv(r, nb);
  *nb_out = cdiv(r, rchunk);
  *rchunk_out = rchunk;
}

namespace {

// SUM / MEAN over the middle axis: partial rows (k_colsum), then their
// fixed-order sum (colsum_final).
int colsum_launch(const float* x, int64_t outer, int64_t r, int64_t inner, float* out,
                  float scale) {
  const bool vec = aligned16(x) && (inner % 4) == 0;
  const int64_t col_waves = cdiv(vec ? inner / 4 : inner, kBlock);
  int64_t nb = 0, rchunk = 0;
  colsum_plan(outer, r, inner, vec, &nb, &rchunk);
  Scratch part((size_t)(outer * nb * inner) * sizeof(float));
  if (!part.ok()) return set_error(TJH_ERR_OOM, "reduce: no scratch memory");
  dim3 grid((unsigned)nb, (unsigned)col_waves, (unsigned)outer);
  if (vec)
    tjh_launch(k_colsum<true>, grid, dim3(kBlock), 0, stream(), x, r, inner, rchunk,
                       part.as<float>());
  else
    tjh_launch(k_colsum<false>, grid, dim3(kBlock), 0, stream(), x, r, inner, rchunk,
                       part.as<float>());
  int rc = check_launch("reduce_colsum");
  if (rc != TJH_OK) return rc;
  // the [outer][nb][inner] partials are outer*inner columns of nb rows only
  // when outer == 1; otherwise finish each o separately
  for (int64_t o = 0; o < outer && rc == TJH_OK; o += kFinalMax) {
    float* parts[kFinalMax];
    float* outs[kFinalMax];
    const int np = (int)(outer - o < kFinalMax ? outer - o : kFinalMax);
    for (int i = 0; i < np; ++i) {
      parts[i] = part.as<float>() + (o + i) * nb * inner;
      outs[i] = out + (o + i) * inner;
    }
    rc = colsum_final(parts, outs, np, nb, inner, 0, scale);
  }
  return rc;
}

template <int OP>
int reduce_cols(const float* x, int64_t outer, int64_t r, int64_t inner, float* out,
                float scale) {
  if ((OP == TJH_REDUCE_SUM || OP == TJH_REDUCE_MEAN) && outer <= 64 && r >= 64)
    return colsum_launch(x, outer, r, inner, out, scale);
  int cus = num_cus() > 0 ? num_cus() : 256;
  bool vec = aligned16(x) && aligned16(out) && (inner % 4) == 0;
  int64_t lanes = vec ? inner / 4 : inner;
  int64_t gx = cdiv(lanes, kBlock);
  int64_t splits = 1;
  int64_t blocks = gx * outer;
  if (blocks < 4LL * cus && r >= 16) {
    int64_t want = cdiv(4LL * cus, blocks);
    int64_t by_len = r / 8;  // keep >= 8 rows per slice
    splits = want < by_len ? want : by_len;
    if (splits < 1) splits = 1;
    if (splits > 65535) splits = 65535;
  }
  int64_t rchunk = cdiv(r, splits);
  splits = cdiv(r, rchunk);
  Scratch scratch(splits > 1 ? (size_t)(outer * splits * inner) * sizeof(float) : 0);
  float* part = out;
  if (splits > 1) {
    if (!scratch.ok()) return set_error(TJH_ERR_OOM, "reduce: no scratch memory");
    part = scratch.as<float>();
  }
  dim3 grid((unsigned)(gx * outer), (unsigned)splits);
  float s1 = splits > 1 ? 1.0f : scale;
  if (vec)
    tjh_launch((k_reduce_cols<OP, true>), grid, dim3(kBlock), 0, stream(), x, r, inner,
                       rchunk, gx, part, s1);
  else
    tjh_launch((k_reduce_cols<OP, false>), grid, dim3(kBlock), 0, stream(), x, r, inner,
                       rchunk, gx, part, s1);
  int rc = check_launch("reduce_cols");
  if (rc != TJH_OK || splits == 1) return rc;
  return reduce_cols<OP>(part, outer, splits, inner, out, scale);
}

template <int OP>
int reduce_any(const float* x, int64_t outer, int64_t r, int64_t inner, float* out, float scale) {
  if (inner == 1) return reduce_rows<OP>(x, outer, r, out, scale);
  return reduce_cols<OP>(x, outer, r, inner, out, scale);
}

// ------------------------------------------------------------- argmax

template <bool MIN>
__device__ __forceinline__ bool better(float v, int64_t i, float bv, int64_t bi) {
  // strictly better value wins; equal values keep the lower index
  if (MIN ? (v < bv) : (v > bv)) return true;
  if (v == bv && i < bi) return true;
  return false;
}

template <bool MIN>
__global__ __launch_bounds__(kBlock) void k_argmax_rows(const float* __restrict__ x, int64_t r,
                                                        int32_t* __restrict__ out) {
  __shared__ float sv[kBlock];
  __shared__ int64_t si[kBlock];
  int64_t o = blockIdx.x;
  const float* row = x + o * r;
  float bv = MIN ? FLT_MAX : -FLT_MAX;
  int64_t bi = r;  // sentinel larger than any index
  for (int64_t i = threadIdx.x; i < r; i += kBlock) {
    float v = row[i];
    if (bi == r || better<MIN>(v, i, bv, bi)) { bv = v; bi = i; }
  }
  sv[threadIdx.x] = bv;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int s = kBlock / 2; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) {
      float v = sv[threadIdx.x + s];
      int64_t i = si[threadIdx.x + s];
      if (i < r && (si[threadIdx.x] == r || better<MIN>(v, i, sv[threadIdx.x], si[threadIdx.x]))) {
        sv[threadIdx.x] = v;
        si[threadIdx.x] = i;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) out[o] = (int32_t)si[0];
}

template <bool MIN>
__global__ __launch_bounds__(kBlock) void k_argmax_cols(const float* __restrict__ x, int64_t outer,
                                                        int64_t r, int64_t inner,
                                                        int32_t* __restrict__ out) {
  int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (t >= outer * inner) return;
  int64_t o = t / inner, c = t % inner;
  const float* base = x + o * r * inner + c;
  float bv = base[0];
  int64_t bi = 0;
  for (int64_t k = 1; k < r; ++k) {
    float v = base[k * inner];
    if (MIN ? (v < bv) : (v > bv)) { bv = v; bi = k; }
  }
  out[t] = (int32_t)bi;
}

}  // namespace

int colsum_final_cols(float* const* part, float* const* out, const int64_t* cols, int np,
                      int64_t nb, int accumulate, float scale) {
  TJH_ARG(np >= 1 && np <= kFinalMax, "colsum_final: %d outputs", np);
  FinalArgs fa{};
  int used = 0;
  int64_t maxc = 0;
  for (int i = 0; i < np; ++i) {
    if (!out[i]) continue;
    fa.part[used] = part[i];
    fa.out[used] = out[i];
    fa.cols[used] = cols[i];
    if (cols[i] > maxc) maxc = cols[i];
    ++used;
  }
  if (used == 0 || maxc == 0) return TJH_OK;
  tjh_launch(k_colsum_final, dim3((unsigned)cdiv(maxc, 64), (unsigned)used),
             dim3(64 * kFinalWaves), 0, stream(), fa, nb, accumulate, scale);
  return check_launch("colsum_final");
}

int colsum_final(float* const* part, float* const* out, int np, int64_t nb, int64_t cols,
                 int accumulate, float scale) {
  int64_t cs[kFinalMax];
  for (int i = 0; i < np && i < kFinalMax; ++i) cs[i] = cols;
  return colsum_final_cols(part, out, cs, np, nb, accumulate, scale);
}

}  // namespace tjh

using namespace tjh;

extern "C" {

int tjh_reduce(int op, const float* x, int64_t outer, int64_t r, int64_t inner, float* out) {
  TJH_REQUIRE_INIT();
  TJH_ARG(outer >= 0 && r >= 0 && inner >= 0, "tjh_reduce: negative size");
  TJH_ARG(op >= 0 && op < TJH_REDUCE_COUNT, "tjh_reduce: unknown op %d", op);
  if (outer == 0 || inner == 0) return TJH_OK;
  KernelScope ks(inner == 1 ? "reduce_rows" : "reduce_cols");
  if (r == 0) {
    // empty reduction: identity (sum/mean -> 0 / nan like torch, prod -> 1)
    float v = op == TJH_REDUCE_PROD ? 1.0f : (op == TJH_REDUCE_MEAN ? __builtin_nanf("") : 0.0f);
    if (op == TJH_REDUCE_MAX || op == TJH_REDUCE_MIN)
      return set_error(TJH_ERR_INVALID, "tjh_reduce: max/min of an empty dimension");
    return tjh_fill_f32(out, outer * inner, v);
  }
  float scale = op == TJH_REDUCE_MEAN ? (float)(1.0 / (double)r) : 1.0f;
  switch (op) {
    case TJH_REDUCE_SUM:
    case TJH_REDUCE_MEAN: return reduce_any<TJH_REDUCE_SUM>(x, outer, r, inner, out, scale);
    case TJH_REDUCE_MAX: return reduce_any<TJH_REDUCE_MAX>(x, outer, r, inner, out, 1.0f);
    case TJH_REDUCE_MIN: return reduce_any<TJH_REDUCE_MIN>(x, outer, r, inner, out, 1.0f);
    case TJH_REDUCE_PROD: return reduce_any<TJH_REDUCE_PROD>(x, outer, r, inner, out, 1.0f);
  }
  return set_error(TJH_ERR_INVALID, "tjh_reduce: unknown op %d", op);
}

int tjh_argmax(const float* x, int64_t outer, int64_t r, int64_t inner, int is_min, int32_t* out) {
  TJH_REQUIRE_INIT();
  TJH_ARG(outer >= 0 && r > 0 && inner >= 0, "tjh_argmax: empty reduction dimension");
  if (outer == 0 || inner == 0) return TJH_OK;
  KernelScope ks("argmax");
  if (inner == 1) {
    if (is_min)
      tjh_launch(k_argmax_rows<true>, dim3((unsigned)outer), dim3(kBlock), 0, stream(), x, r, out);
    else
      tjh_launch(k_argmax_rows<false>, dim3((unsigned)outer), dim3(kBlock), 0, stream(), x, r, out);
  } else {
    unsigned g = (unsigned)cdiv(outer * inner, kBlock);
    if (is_min)
      tjh_launch(k_argmax_cols<true>, dim3(g), dim3(kBlock), 0, stream(), x, outer, r, inner, out);
    else
      tjh_launch(k_argmax_cols<false>, dim3(g), dim3(kBlock), 0, stream(), x, outer, r, inner, out);
  }
  return check_launch("argmax");
}

}  // extern "C"
