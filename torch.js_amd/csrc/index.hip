// Embedding and indexing kernels: embedding forward / deterministic
// backward, index_select / index_add, gather / scatter_add, one_hot and
// nonzero.
//
// Reference semantics: embedding.wgsl:13-27 (ids clamped to the table),
// src/nn/embedding.ts:25-101 (the backward is a TODO there),
// index_select.wgsl:20-55, Tensor.gather (Tensor.ts:2651-2705, negative
// indices wrap), F.one_hot (src/nn/functional.ts:764-796: Math.round,
// out-of-range values leave the row zero) and Tensor.nonzero
// (Tensor.ts:1323-1345: row-major coordinates).  The reference runs
// gather / one_hot / nonzero on the host after a readback.
//
// Embedding backward is deterministic: (id, position) pairs are sorted as
// 64-bit keys with a bitonic network (LDS-resident 2048-element stages and
// global merge stages), then each run of equal ids is summed by one wave
// in increasing position order.

#include "common.h"

namespace tjh {
namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ int64_t clamp_id(int32_t id, int64_t num) {
  return id < 0 ? 0 : (id >= num ? num - 1 : id);
}

// ------------------------------------------------------------ embedding fwd

// One wave per token row; float4 copies when dim % 4 == 0.
template <bool VEC>
__global__ __launch_bounds__(kBlock) void k_emb_fwd(const float* __restrict__ w, int64_t num,
                                                    int64_t dim, const int32_t* __restrict__ ids,
                                                    int64_t n, float* __restrict__ out) {
  int64_t t = (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (t >= n) return;
  int64_t row = clamp_id(ids[t], num);
  const float* src = w + row * dim;
  float* dst = out + t * dim;
  if (VEC) {
    const float4* s4 = reinterpret_cast<const float4*>(src);
    float4* d4 = reinterpret_cast<float4*>(dst);
    for (int64_t i = lane; i < dim / 4; i += 64) d4[i] = s4[i];
  } else {
    for (int64_t i = lane; i < dim; i += 64) dst[i] = src[i];
  }
}

// ------------------------------------------------------------ bitonic sort

__global__ __launch_bounds__(kBlock) void k_make_keys(const int32_t* __restrict__ ids, int64_t n,
                                                      int64_t num, int64_t npad,
                                                      uint64_t* __restrict__ keys) {
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= npad) return;
  keys[i] = i < n ? (((uint64_t)clamp_id(ids[i], num)) << 32) | (uint64_t)i : ~0ull;
}

// Sorting a short index list in one workgroup: an LSD radix sort of
// 32-bit keys clamp(id) << pos_bits | position, held in LDS, over the id
// bits only, 8 bits per pass.  A pass is stable: each of the 16 waves owns
// a contiguous block of positions; per-wave digit histograms are scanned in
// (digit, wave) order, and each wave scatters its block in position order,
// 64 keys at a time, a key's rank among same-digit lanes coming from
// ballots.  So equal ids keep increasing positions (the summation order of
// the backward) and the result is the same on every run.  n <= 16384 and
// pos_bits + id bits <= 32 (vocabularies up to 2^18 at n = 16384).
constexpr int kLdsSortMax = 16384;
constexpr int kLdsSortThreads = 1024;
constexpr int kLdsSortWaves = kLdsSortThreads / 64;

__global__ __launch_bounds__(kLdsSortThreads) void k_sort_ids_lds(
    const int32_t* __restrict__ ids, int n, int64_t num, int pos_bits, int passes,
    uint64_t* __restrict__ keys_out) {
  __shared__ uint32_t buf[2][kLdsSortMax];
  __shared__ uint32_t hist[kLdsSortWaves][256];
  __shared__ uint32_t wsum[kLdsSortWaves];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int i = tid; i < n; i += kLdsSortThreads)
    buf[0][i] = ((uint32_t)clamp_id(ids[i], num) << pos_bits) | (uint32_t)i;
  // wave w owns positions [beg, end), a multiple of 64 long
  const int per = ((n + kLdsSortWaves - 1) / kLdsSortWaves + 63) & ~63;
  const int beg = w * per < n ? w * per : n;
  const int end = beg + per < n ? beg + per : n;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int src = 0;
  __syncthreads();
  for (int p = 0; p < passes; ++p) {
    const int shift = pos_bits + 8 * p;
    const uint32_t* a = buf[src];
    uint32_t* b = buf[src ^ 1];
    for (int d = lane; d < 256; d += 64) hist[w][d] = 0;
    __syncthreads();
    for (int e = beg + lane; e < end; e += 64) atomicAdd(&hist[w][(a[e] >> shift) & 255u], 1u);
    __syncthreads();
    // exclusive scan in (digit, wave) order: entry q = d * 16 + wave
    uint32_t v[4], t = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int q = 4 * tid + k;
      v[k] = hist[q & (kLdsSortWaves - 1)][q >> 4];
      t += v[k];
    }
    uint32_t incl = t;  // inclusive scan of the thread totals within the wave
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t o = __shfl_up(incl, off, 64);
      if (lane >= off) incl += o;
    }
    if (lane == 63) wsum[w] = incl;
    __syncthreads();
    uint32_t wbase = 0;
    for (int k = 0; k < w; ++k) wbase += wsum[k];
    uint32_t run = wbase + incl - t;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int q = 4 * tid + k;
      hist[q & (kLdsSortWaves - 1)][q >> 4] = run;
      run += v[k];
    }
    __syncthreads();
    // stable scatter of the wave's block, 64 keys at a time, in order
    for (int c = beg; c < end; c += 64) {
      const int e = c + lane;
      const bool valid = e < end;
      const uint32_t key = valid ? a[e] : 0u;
      const uint32_t d = (key >> shift) & 255u;
      uint64_t peers = __ballot(valid);
#pragma unroll
      for (int bit = 0; bit < 8; ++bit) {
        const uint64_t m = __ballot(valid && ((d >> bit) & 1u));
        peers &= ((d >> bit) & 1u) ? m : ~m;
      }
      const uint32_t rank = (uint32_t)__popcll(peers & lt_mask);
      const uint32_t base = valid ? hist[w][d] : 0u;
      if (valid) b[base + rank] = key;
      // the lowest peer advances the digit's cursor (every peer has read it)
      if (valid && (peers & lt_mask) == 0) hist[w][d] = base + (uint32_t)__popcll(peers);
    }
    __syncthreads();
    src ^= 1;
  }
  const uint32_t pmask = (1u << pos_bits) - 1u;
  for (int i = tid; i < n; i += kLdsSortThreads) {
    const uint32_t k = buf[src][i];
    keys_out[i] = ((uint64_t)(k >> pos_bits) << 32) | (uint64_t)(k & pmask);
  }
}

constexpr int kSortChunk = 2048;  // elements per LDS stage (1024 lanes x 2)
constexpr int kSortThreads = 1024;

__device__ __forceinline__ void cmp_swap(uint64_t& a, uint64_t& b, bool up) {
  if ((a > b) == up) {
    uint64_t t = a;
    a = b;
    b = t;
  }
}

// FULL: sort each 2048-chunk for all k <= min(npad, 2048).
// !FULL: finish merge stage k for j = 1024 .. 1 inside each chunk.
template <bool FULL>
__global__ __launch_bounds__(kSortThreads) void k_bitonic_local(uint64_t* __restrict__ keys,
                                                                int64_t npad, int64_t kstage) {
  __shared__ uint64_t s[kSortChunk];
  int64_t base = (int64_t)blockIdx.x * kSortChunk;
  int64_t len = npad - base < kSortChunk ? npad - base : kSortChunk;
  for (int i = threadIdx.x; i < len; i += kSortThreads) s[i] = keys[base + i];
  __syncthreads();
  int64_t kmax = FULL ? (len < kSortChunk ? len : kSortChunk) : kstage;
  int64_t kmin = FULL ? 2 : kstage;
  for (int64_t k = kmin; k <= kmax; k <<= 1) {
    int64_t jstart = FULL ? (k >> 1) : (kSortChunk >> 1);
    if (jstart > (len >> 1)) jstart = len >> 1;
    for (int64_t j = jstart; j > 0; j >>= 1) {
      for (int t = threadIdx.x; t < (len >> 1); t += kSortThreads) {
        // pair (i, i+j) with i having bit j clear
        int64_t i = ((t / j) * 2 * j) + (t % j);
        int64_t gi = base + i;
        bool up = (gi & k) == 0;
        cmp_swap(s[i], s[i + j], up);
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < len; i += kSortThreads) keys[base + i] = s[i];
}

__global__ __launch_bounds__(kBlock) void k_bitonic_global(uint64_t* __restrict__ keys,
                                                           int64_t npad, int64_t k, int64_t j) {
  int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (t >= (npad >> 1)) return;
  int64_t i = ((t / j) * 2 * j) + (t % j);
  bool up = (i & k) == 0;
  uint64_t a = keys[i], b = keys[i + j];
  if ((a > b) == up) {
    keys[i] = b;
    keys[i + j] = a;
  }
}

// One wave per sorted entry; only run heads do work.
template <bool VEC>
__global__ __launch_bounds__(kBlock) void k_emb_bwd_runs(const uint64_t* __restrict__ keys,
                                                         int64_t n, const float* __restrict__ dout,
                                                         int64_t dim, float* __restrict__ dw,
                                                         int accumulate) {
  int64_t s = (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (s >= n) return;
  uint32_t id = (uint32_t)(keys[s] >> 32);
  if (s > 0 && (uint32_t)(keys[s - 1] >> 32) == id) return;
  float* dst = dw + (int64_t)id * dim;
  if (VEC) {
    int64_t d4n = dim / 4;
    for (int64_t c = lane; c < d4n; c += 64) {
      float4 acc = accumulate ? reinterpret_cast<float4*>(dst)[c] : make_float4(0.f, 0.f, 0.f, 0.f);
      for (int64_t q = s; q < n && (uint32_t)(keys[q] >> 32) == id; ++q) {
        int64_t pos = (int64_t)(keys[q] & 0xffffffffull);
        float4 v = reinterpret_cast<const float4*>(dout + pos * dim)[c];
        acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
      }
      reinterpret_cast<float4*>(dst)[c] = acc;
    }
  } else {
    for (int64_t c = lane; c < dim; c += 64) {
      float acc = accumulate ? dst[c] : 0.f;
      for (int64_t q = s; q < n && (uint32_t)(keys[q] >> 32) == id; ++q) {
        int64_t pos = (int64_t)(keys[q] & 0xffffffffull);
        acc += dout[pos * dim + c];
      }
      dst[c] = acc;
    }
  }
}

// ------------------------------------------------------------ index ops

__device__ __forceinline__ int64_t wrap_idx(int32_t v, int64_t len) {
  int64_t i = v;
  if (i < 0) i += len;
  return i;
}

__global__ __launch_bounds__(kBlock) void k_index_select(const float* __restrict__ x, int64_t outer,
                                                         int64_t src_len, int64_t inner,
                                                         const int32_t* __restrict__ idx,
                                                         int64_t n_idx, float* __restrict__ out) {
  int64_t total = outer * n_idx * inner;
  int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x; e < total; e += stride) {
    int64_t i = e % inner;
    int64_t j = (e / inner) % n_idx;
    int64_t o = e / (inner * n_idx);
    int64_t s = idx[j];  // no wrap: the host rejects indices outside [0, src_len)
    out[e] = (s >= 0 && s < src_len) ? x[(o * src_len + s) * inner + i] : 0.f;
  }
}

// dx[o, s, i] += sum_{j : idx[j] == s} dout[o, j, i]  (j increasing)
__global__ __launch_bounds__(kBlock) void k_index_add(float* __restrict__ dx, int64_t outer,
                                                      int64_t src_len, int64_t inner,
                                                      const int32_t* __restrict__ idx,
                                                      int64_t n_idx,
                                                      const float* __restrict__ dout) {
  int64_t total = outer * src_len * inner;
  int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x; e < total; e += stride) {
    int64_t i = e % inner;
    int64_t s = (e / inner) % src_len;
    int64_t o = e / (inner * src_len);
    float acc = dx[e];
    for (int64_t j = 0; j < n_idx; ++j)
      if ((int64_t)idx[j] == s) acc += dout[(o * n_idx + j) * inner + i];
    dx[e] = acc;
  }
}

__global__ __launch_bounds__(kBlock) void k_gather(const float* __restrict__ x, int64_t outer,
                                                   int64_t src_len, int64_t inner,
                                                   const int32_t* __restrict__ idx,
                                                   int64_t idx_len, float* __restrict__ out) {
  int64_t total = outer * idx_len * inner;
  int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x; e < total; e += stride) {
    int64_t i = e % inner;
    int64_t o = e / (inner * idx_len);
    int64_t s = wrap_idx(idx[e], src_len);
    out[e] = (s >= 0 && s < src_len) ? x[(o * src_len + s) * inner + i] : 0.f;
  }
}

// One lane per (o, i) column: walks j in order, so no two lanes collide.
__global__ __launch_bounds__(kBlock) void k_scatter_add(float* __restrict__ dx, int64_t outer,
                                                        int64_t dst_len, int64_t inner,
                                                        const int32_t* __restrict__ idx,
                                                        int64_t idx_len,
                                                        const float* __restrict__ src) {
  int64_t col = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (col >= outer * inner) return;
  int64_t o = col / inner, i = col % inner;
  for (int64_t j = 0; j < idx_len; ++j) {
    int64_t e = (o * idx_len + j) * inner + i;
    int64_t s = wrap_idx(idx[e], dst_len);
    if (s >= 0 && s < dst_len) dx[(o * dst_len + s) * inner + i] += src[e];
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void k_one_hot(const T* __restrict__ x, int64_t n,
                                                    int64_t classes, float* __restrict__ out) {
  int64_t total = n * classes;
  int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x; e < total; e += stride) {
    int64_t i = e / classes, c = e % classes;
    int64_t v;
    if constexpr (sizeof(T) == 4 && T(0.5) != T(0)) v = (int64_t)floor((double)x[i] + 0.5);
    else v = (int64_t)x[i];
    out[e] = (v == c) ? 1.f : 0.f;
  }
}

// nonzero: per-chunk counts, then ordered writes.
constexpr int kNzChunk = 1024;
__global__ __launch_bounds__(kBlock) void k_nz_count(const float* __restrict__ x, int64_t n,
                                                     int64_t* __restrict__ counts) {
  __shared__ int sm[kBlock / 64];
  int64_t base = (int64_t)blockIdx.x * kNzChunk;
  int c = 0;
  for (int i = threadIdx.x; i < kNzChunk; i += kBlock) {
    int64_t e = base + i;
    if (e < n && x[e] != 0.f) ++c;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) c += __shfl_xor(c, off, 64);
  if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    int t = 0;
    for (int w = 0; w < kBlock / 64; ++w) t += sm[w];
    counts[blockIdx.x] = t;
  }
}

struct Shape8 {
  int64_t d[TJH_MAX_DIMS];
};

// One block per chunk; a single lane writes the chunk's coordinates in
// order (chunks are small, offsets come from the exclusive scan).
__global__ __launch_bounds__(64) void k_nz_write(const float* __restrict__ x, int64_t n, int ndim,
                                                 Shape8 shape, const int64_t* __restrict__ offs,
                                                 int32_t* __restrict__ out, int64_t max_out) {
  if (threadIdx.x != 0) return;
  int64_t base = (int64_t)blockIdx.x * kNzChunk;
  int64_t o = offs[blockIdx.x];
  for (int i = 0; i < kNzChunk; ++i) {
    int64_t e = base + i;
    if (e >= n) break;
    if (x[e] == 0.f) continue;
    if (o >= max_out) return;
    int64_t rem = e;
    for (int d = ndim - 1; d >= 0; --d) {
      out[o * ndim + d] = (int32_t)(rem % shape.d[d]);
      rem /= shape.d[d];
    }
    ++o;
  }
}

}  // namespace
}  // namespace tjh

using namespace tjh;

extern "C" {

int tjh_embedding_forward(const float* weight, int64_t num, int64_t dim, const int32_t* ids,
                          int64_t n, float* out) {
  TJH_REQUIRE_INIT();
  TJH_ARG(num > 0 && dim >= 0 && n >= 0, "tjh_embedding_forward: bad sizes");
  if (n == 0 || dim == 0) return TJH_OK;
  KernelScope ks("embedding_fwd");
  unsigned g = (unsigned)cdiv(n, kBlock / 64);
  bool vec = dim % 4 == 0 && ((uintptr_t)weight & 15) == 0 && ((uintptr_t)out & 15) == 0;
  if (vec)
    tjh_launch(k_emb_fwd<true>, dim3(g), dim3(kBlock), 0, stream(), weight, num, dim, ids,
                       n, out);
  else
    tjh_launch(k_emb_fwd<false>, dim3(g), dim3(kBlock), 0, stream(), weight, num, dim, ids,
                       n, out);
  return check_launch("embedding_forward");
}

int tjh_embedding_backward(const float* dout, const int32_t* ids, int64_t n, int64_t dim,
                           float* dweight, int64_t num, int accumulate) {
  TJH_REQUIRE_INIT();
  TJH_ARG(num > 0 && dim >= 0 && n >= 0, "tjh_embedding_backward: bad sizes");
  TJH_ARG(n < (int64_t(1) << 32), "tjh_embedding_backward: too many indices");
  if (!accumulate) {
    int rc = tjh_fill_f32(dweight, num * dim, 0.f);
    if (rc != TJH_OK) return rc;
  }
  if (n == 0 || dim == 0) return TJH_OK;
  // short lists (a batch of token positions) are radix-sorted in LDS by one
  // workgroup; longer ones (or ids too wide to pack) by the bitonic network
  int pos_bits = 1, id_bits = 1;
  while ((int64_t(1) << pos_bits) < n) ++pos_bits;
  while ((int64_t(1) << id_bits) < num) ++id_bits;
  const bool lds_sort = n <= kLdsSortMax && pos_bits + id_bits <= 32;
  int64_t npad = 1;
  while (npad < n) npad <<= 1;
  if (npad < 2) npad = 2;
  Scratch keys_s((size_t)(lds_sort ? n : npad) * sizeof(uint64_t));
  if (!keys_s.ok()) return set_error(TJH_ERR_OOM, "embedding_backward: no scratch");
  uint64_t* keys = keys_s.as<uint64_t>();
  KernelScope ks("embedding_bwd");
  if (lds_sort) {
    tjh_launch(k_sort_ids_lds, dim3(1), dim3(kLdsSortThreads), 0, stream(), ids, (int)n, num,
               pos_bits, (id_bits + 7) / 8, keys);
  } else {
    tjh_launch(k_make_keys, dim3((unsigned)cdiv(npad, kBlock)), dim3(kBlock), 0, stream(),
                       ids, n, num, npad, keys);
    unsigned chunks = (unsigned)cdiv(npad, kSortChunk);
    tjh_launch(k_bitonic_local<true>, dim3(chunks), dim3(kSortThreads), 0, stream(), keys,
                       npad, (int64_t)0);
    for (int64_t k = 2 * kSortChunk; k <= npad; k <<= 1) {
      for (int64_t j = k >> 1; j >= kSortChunk; j >>= 1)
        tjh_launch(k_bitonic_global, dim3((unsigned)cdiv(npad / 2, kBlock)), dim3(kBlock),
                           0, stream(), keys, npad, k, j);
      tjh_launch(k_bitonic_local<false>, dim3(chunks), dim3(kSortThreads), 0, stream(),
                         keys, npad, k);
    }
  }
  int rc = check_launch("embedding_backward_sort");
  if (rc != TJH_OK) return rc;
  bool vec = dim % 4 == 0 && ((uintptr_t)dout & 15) == 0 && ((uintptr_t)dweight & 15) == 0;
  unsigned g = (unsigned)cdiv(n, kBlock / 64);
  if (vec)
    tjh_launch(k_emb_bwd_runs<true>, dim3(g), dim3(kBlock), 0, stream(), keys, n, dout, dim,
                       dweight, 1);
  else
    tjh_launch(k_emb_bwd_runs<false>, dim3(g), dim3(kBlock), 0, stream(), keys, n, dout,
                       dim, dweight, 1);
  return check_launch("embedding_backward");
}

int tjh_index_select(const float* x, int64_t outer, int64_t src_len, int64_t inner,
                     const int32_t* idx, int64_t n_idx, float* out) {
  TJH_REQUIRE_INIT();
  TJH_ARG(outer >= 0 && src_len >= 0 && inner >= 0 && n_idx >= 0, "tjh_index_select: bad sizes");
  int64_t total = outer * n_idx * inner;
  if (total == 0) return TJH_OK;
  KernelScope ks("index_select");
  int64_t g = cdiv(total, kBlock);
  if (g > 65536) g = 65536;
  tjh_launch(k_index_select, dim3((unsigned)g), dim3(kBlock), 0, stream(), x, outer,
                     src_len, inner, idx, n_idx, out);
  return check_launch("index_select");
}

int tjh_index_add(float* dx, int64_t outer, int64_t src_len, int64_t inner, const int32_t* idx,
                  int64_t n_idx, const float* dout) {
  TJH_REQUIRE_INIT();
  TJH_ARG(outer >= 0 && src_len >= 0 && inner >= 0 && n_idx >= 0, "tjh_index_add: bad sizes");
  int64_t total = outer * src_len * inner;
  if (total == 0 || n_idx == 0) return TJH_OK;
  KernelScope ks("index_add");
  int64_t g = cdiv(total, kBlock);
  if (g > 65536) g = 65536;
  tjh_launch(k_index_add, dim3((unsigned)g), dim3(kBlock), 0, stream(), dx, outer, src_len,
                     inner, idx, n_idx, dout);
  return check_launch("index_add");
}

int tjh_gather(const float* x, int64_t outer, int64_t src_len, int64_t inner, const int32_t* idx,
               int64_t idx_len, float* out) {
  TJH_REQUIRE_INIT();
  TJH_ARG(outer >= 0 && src_len >= 0 && inner >= 0 && idx_len >= 0, "tjh_gather: bad sizes");
  int64_t total = outer * idx_len * inner;
  if (total == 0) return TJH_OK;
  KernelScope ks("gather");
  int64_t g = cdiv(total, kBlock);
  if (g > 65536) g = 65536;
  tjh_launch(k_gather, dim3((unsigned)g), dim3(kBlock), 0, stream(), x, outer, src_len,
                     inner, idx, idx_len, out);
  return check_launch("gather");
}

int tjh_scatter_add(float* dx, int64_t outer, int64_t dst_len, int64_t inner, const int32_t* idx,
                    int64_t idx_len, const float* src) {
  TJH_REQUIRE_INIT();
  TJH_ARG(outer >= 0 && dst_len >= 0 && inner >= 0 && idx_len >= 0, "tjh_scatter_add: bad sizes");
  if (outer * inner == 0 || idx_len == 0) return TJH_OK;
  KernelScope ks("scatter_add");
  tjh_launch(k_scatter_add, dim3((unsigned)cdiv(outer * inner, kBlock)), dim3(kBlock), 0,
                     stream(), dx, outer, dst_len, inner, idx, idx_len, src);
  return check_launch("scatter_add");
}

int tjh_one_hot(const float* x, int64_t n, int64_t classes, float* out) {
  TJH_REQUIRE_INIT();
  TJH_ARG(n >= 0 && classes > 0, "tjh_one_hot: bad sizes");
  if (n == 0) return TJH_OK;
  KernelScope ks("one_hot");
  int64_t g = cdiv(n * classes, kBlock);
  if (g > 65536) g = 65536;
  tjh_launch(k_one_hot<float>, dim3((unsigned)g), dim3(kBlock), 0, stream(), x, n, classes,
                     out);
  return check_launch("one_hot");
}

int tjh_one_hot_i32(const int32_t* x, int64_t n, int64_t classes, float* out) {
  TJH_REQUIRE_INIT();
  TJH_ARG(n >= 0 && classes > 0, "tjh_one_hot_i32: bad sizes");
  if (n == 0) return TJH_OK;
  KernelScope ks("one_hot");
  int64_t g = cdiv(n * classes, kBlock);
  if (g > 65536) g = 65536;
  tjh_launch(k_one_hot<int32_t>, dim3((unsigned)g), dim3(kBlock), 0, stream(), x, n,
                     classes, out);
  return check_launch("one_hot_i32");
}

int tjh_nonzero(const float* x, int ndim, const int64_t* shape, int32_t* out, int64_t max_out,
                int64_t* count) {
  TJH_REQUIRE_INIT();
  TJH_ARG(ndim >= 1 && ndim <= TJH_MAX_DIMS && shape && count, "tjh_nonzero: bad arguments");
  int64_t n = 1;
  Shape8 sh;
  for (int d = 0; d < ndim; ++d) {
    TJH_ARG(shape[d] >= 0, "tjh_nonzero: negative dimension");
    n *= shape[d];
    sh.d[d] = shape[d];
  }
  *count = 0;
  if (n == 0) return TJH_OK;
  if (capturing())  // the count is read back to the host
    return set_error(TJH_ERR_UNSUPPORTED, "tjh_nonzero: not allowed while a graph is being captured");
  int64_t chunks = cdiv(n, kNzChunk);
  Scratch cs((size_t)chunks * sizeof(int64_t));
  if (!cs.ok()) return set_error(TJH_ERR_OOM, "nonzero: no scratch");
  KernelScope ks("nonzero");
  tjh_launch(k_nz_count, dim3((unsigned)chunks), dim3(kBlock), 0, stream(), x, n,
                     cs.as<int64_t>());
  int rc = check_launch("nonzero_count");
  if (rc != TJH_OK) return rc;
  int64_t* hc = new int64_t[chunks];
  hipError_t e = hipMemcpyAsync(hc, cs.p, chunks * sizeof(int64_t), hipMemcpyDeviceToHost, stream());
  if (e == hipSuccess) e = hipStreamSynchronize(stream());
  if (e != hipSuccess) {
    delete[] hc;
    return hip_fail(e, "nonzero readback");
  }
  int64_t tot = 0;
  for (int64_t c = 0; c < chunks; ++c) {
    int64_t v = hc[c];
    hc[c] = tot;
    tot += v;
  }
  *count = tot;
  if (tot > 0 && out) {
    e = hipMemcpyAsync(cs.p, hc, chunks * sizeof(int64_t), hipMemcpyHostToDevice, stream());
    if (e == hipSuccess) e = hipStreamSynchronize(stream());
    delete[] hc;
    if (e != hipSuccess) return hip_fail(e, "nonzero offsets upload");
    tjh_launch(k_nz_write, dim3((unsigned)chunks), dim3(64), 0, stream(), x, n, ndim, sh,
                       cs.as<int64_t>(), out, max_out);
    return check_launch("nonzero_write");
  }
  delete[] hc;
  return TJH_OK;
}

}  // extern "C"
