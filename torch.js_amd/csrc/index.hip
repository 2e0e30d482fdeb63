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
// Embedding backward is deterministic: every table row is the sum of its
// dout rows in increasing position order.  Short index lists are handled by
// workgroups that each own a range of table rows (k_emb_bwd_owned); long
// ones sort (id, position) pairs as 64-bit keys with a bitonic network
// (LDS-resident 2048-element stages and global merge stages) and sum each
// run of equal ids with one wave.

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

// out[p] = w[ids[p]] + wp[pos0 + p mod T]: the sum of a token and a
// position embedding, one wave per token row.
template <bool VEC>
__global__ __launch_bounds__(kBlock) void k_emb_pos_fwd(const float* __restrict__ w, int64_t num,
                                                        int64_t dim,
                                                        const int32_t* __restrict__ ids, int64_t n,
                                                        const float* __restrict__ wp,
                                                        int64_t num_pos, int64_t pos0, int64_t T,
                                                        float* __restrict__ out) {
  int64_t t = (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (t >= n) return;
  const float* src = w + clamp_id(ids[t], num) * dim;
  const float* psrc = wp + clamp_id((int32_t)(pos0 + t % T), num_pos) * dim;
  float* dst = out + t * dim;
  if (VEC) {
    const float4* s4 = reinterpret_cast<const float4*>(src);
    const float4* p4 = reinterpret_cast<const float4*>(psrc);
    float4* d4 = reinterpret_cast<float4*>(dst);
    for (int64_t i = lane; i < dim / 4; i += 64) {
      const float4 a = s4[i], b = p4[i];
      d4[i] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
    }
  } else {
    for (int64_t i = lane; i < dim; i += 64) dst[i] = src[i] + psrc[i];
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

// Embedding backward over owned row ranges, for index lists up to
// kOwnMaxN: workgroup g owns the table rows [g*span, (g+1)*span).  It reads
// the whole id list (from L2 after the first workgroups), collects the
// positions that hit its rows in position order into an LDS list (ballot
// ranks: hits are rare, so a round costs a few instructions per id), orders
// the list by row with a stable counting sort, and then spreads the (row,
// column) work of the rows that have entries over all threads: each output
// element is its prior value (accumulate) or zero plus the row's dout
// elements in increasing position order.  When not accumulating, rows
// without entries are written as zeros, so no separate fill runs.  A list
// longer than the LDS holds is processed in consecutive position chunks,
// each adding into what the previous chunk stored; a float32 store and
// reload is exact, so every sum is the one of a single pass in increasing
// position order, and the result is the same on every run.
constexpr int kOwnThreads = 256;
constexpr int kOwnWaves = kOwnThreads / 64;
constexpr int kOwnCap = 1024;       // list entries per chunk (>= one round's hits)
constexpr int kOwnMaxSpan = 1024;   // rows per workgroup
constexpr int kOwnGroups = 1024;    // workgroups while span <= kOwnMaxSpan
constexpr int64_t kOwnMaxN = 65536;
constexpr int64_t kOwnMaxScan = int64_t(1) << 25;  // id reads over all workgroups
constexpr int kOwnRound = 4 * kOwnThreads;          // positions per compaction round
constexpr int kOwnSub = 8;                          // rounds loaded together
constexpr int kOwnBatch = 8;                        // output elements per thread in flight

// ids[p .. p+3] (entries at or past n read as 0, unused); one 128-bit load
// when the list is 16-byte aligned (p is a multiple of 4)
__device__ __forceinline__ void load_ids4(const int32_t* __restrict__ ids, int n, int p,
                                          int vec, int (&v)[4]) {
  if (vec && p + 3 < n) {
    const int4 q = *reinterpret_cast<const int4*>(ids + p);
    v[0] = q.x;
    v[1] = q.y;
    v[2] = q.z;
    v[3] = q.w;
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = p + k < n ? ids[p + k] : 0;
  }
}

// Lanes below this one whose bit is set in a wave-wide mask.
__device__ __forceinline__ int lanes_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                        __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

template <bool VEC>
struct EmbUnit;
template <>
struct EmbUnit<true> {
  typedef float4 T;
  static __device__ __forceinline__ T zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }
  static __device__ __forceinline__ void add(T& a, const T& b) {
    a.x += b.x;
    a.y += b.y;
    a.z += b.z;
    a.w += b.w;
  }
};
template <>
struct EmbUnit<false> {
  typedef float T;
  static __device__ __forceinline__ T zero() { return 0.f; }
  static __device__ __forceinline__ void add(T& a, const T& b) { a += b; }
};

// The rows [blk * span, ...) of the table, owned by one workgroup.
template <bool VEC>
__device__ __forceinline__ void emb_owned_body(
    int blk, const int32_t* __restrict__ ids, int n, int ids_vec, int num, int span,
    int span_bits, const float* __restrict__ dout, int units, float* __restrict__ dw,
    int accumulate) {
  typedef EmbUnit<VEC> U;
  typedef typename U::T T;
  __shared__ uint32_t lpos[kOwnCap];     // list: positions, in position order
  __shared__ uint32_t lrow[kOwnCap];     // list: row within the range
  __shared__ uint32_t spos[kOwnCap];     // positions ordered by (row, position)
  __shared__ uint32_t cur[kOwnMaxSpan];  // per row: start, then end, of its entries
  __shared__ uint32_t rows[kOwnMaxSpan]; // the rows to write, in order
  __shared__ uint32_t wcnt[kOwnSub * kOwnWaves];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int lo = blk * span;
  const int nrows = num - lo < span ? num - lo : span;  // >= 1 by the grid
  const T* __restrict__ src = reinterpret_cast<const T*>(dout);
  T* __restrict__ dst = reinterpret_cast<T*>(dw);
  int scan = 0;
  for (int chunk = 0;; ++chunk) {
    // 1. the positions from `scan` on that hit rows [lo, lo + nrows), in
    // order.  A super-round covers kOwnSub rounds of 1024 positions (four
    // consecutive ones per thread per round), all loaded at once so the
    // workgroup waits for one memory latency, and appends them after one
    // barrier: the rounds whose hits still fit in the list are appended, the
    // rest are read again by the next chunk (a round has at most kOwnCap
    // hits, so every chunk makes progress)
    int L = 0;
    bool full = false;
    while (scan < n && !full) {
      int idv[kOwnSub][4];
#pragma unroll
      for (int j = 0; j < kOwnSub; ++j)
        load_ids4(ids, n, scan + j * kOwnRound + 4 * tid, ids_vec, idv[j]);
      uint32_t hitm[kOwnSub];
      int pre[kOwnSub];
#pragma unroll
      for (int j = 0; j < kOwnSub; ++j) {
        const int p0 = scan + j * kOwnRound + 4 * tid;
        uint32_t m = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int r = min(max(idv[j][k], 0), num - 1) - lo;
          idv[j][k] = r;
          m |= (p0 + k < n && (uint32_t)r < (uint32_t)nrows) ? (1u << k) : 0u;
        }
        // rank of this thread's first hit: hits of the lower lanes
        int below = 0, tot = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint64_t b = __ballot((m >> k) & 1u);
          below += lanes_below(b);
          tot += (int)__popcll(b);
        }
        hitm[j] = m;
        pre[j] = below;
        if (lane == 0) wcnt[j * kOwnWaves + w] = (uint32_t)tot;
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < kOwnSub; ++j) {
        if (scan >= n) break;  // uniform over the workgroup
        int before = 0, total = 0;
#pragma unroll
        for (int k = 0; k < kOwnWaves; ++k) {
          const int t = (int)wcnt[j * kOwnWaves + k];
          before += k < w ? t : 0;
          total += t;
        }
        if (L + total > kOwnCap) {
          full = true;
          break;
        }
        if (hitm[j]) {
          const int p0 = scan + 4 * tid;
          int at = L + before + pre[j];
#pragma unroll
          for (int k = 0; k < 4; ++k)
            if ((hitm[j] >> k) & 1u) {
              lpos[at] = (uint32_t)(p0 + k);
              lrow[at] = (uint32_t)idv[j][k];
              ++at;
            }
        }
        L += total;
        scan += kOwnRound;
      }
      __syncthreads();  // wcnt is written again by the next super-round
    }
    const bool acc = accumulate || chunk > 0;
    if (L == 0 && acc) break;  // nothing (more) hits these rows
    // 2. stable counting sort of the list by row: counts, then one scan that
    // gives each row's start and the list of rows to write (rows with
    // entries; every row when zero rows are written too)
    for (int i = tid; i < nrows; i += kOwnThreads) cur[i] = 0u;
    __syncthreads();
    for (int e = tid; e < L; e += kOwnThreads) atomicAdd(&cur[lrow[e]], 1u);
    __syncthreads();
    int nwrite;
    {
      const int per = (nrows + kOwnThreads - 1) / kOwnThreads;  // <= 4
      const int b0 = tid * per;
      uint32_t v = 0;  // entries (low 16 bits) and rows to write (high 16)
      for (int i = 0; i < per; ++i)
        if (b0 + i < nrows) {
          const uint32_t c = cur[b0 + i];
          v += c + ((c || !acc) ? 0x10000u : 0u);
        }
      uint32_t incl = v;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = __shfl_up(incl, off, 64);
        if (lane >= off) incl += o;
      }
      if (lane == 63) wcnt[w] = incl;
      __syncthreads();
      uint32_t run = incl - v, all = 0;
      for (int k = 0; k < kOwnWaves; ++k) {
        run += k < w ? wcnt[k] : 0u;
        all += wcnt[k];
      }
      nwrite = (int)(all >> 16);
      for (int i = 0; i < per; ++i)
        if (b0 + i < nrows) {
          const uint32_t c = cur[b0 + i];
          cur[b0 + i] = run & 0xffffu;
          if (c || !acc) rows[run >> 16] = (uint32_t)(b0 + i);
          run += c + ((c || !acc) ? 0x10000u : 0u);
        }
    }
    __syncthreads();
    // scatter by one wave, 64 entries at a time in list order; a lane's rank
    // among the lanes of the same row comes from ballots over the row bits,
    // and the lowest such lane advances the row's cursor after every lane
    // has read it (one wave's LDS accesses execute in program order)
    if (w == 0) {
      for (int c = 0; c < L; c += 64) {
        const int e = c + lane;
        const bool valid = e < L;
        const uint32_t r = valid ? lrow[e] : 0u;
        uint64_t peers = __ballot(valid);
        for (int bit = 0; bit < span_bits; ++bit) {
          const uint64_t m = __ballot(valid && ((r >> bit) & 1u));
          peers &= ((r >> bit) & 1u) ? m : ~m;
        }
        const int rank = lanes_below(peers);
        const uint32_t base = valid ? cur[r] : 0u;
        if (valid) spos[base + rank] = lpos[e];
        if (valid && rank == 0) cur[r] = base + (uint32_t)__popcll(peers);
      }
    }
    __syncthreads();
    // 3. element (row slot, column) of the rows to write, kOwnBatch per
    // thread in flight; row r's entries are spos[cur[r-1] .. cur[r])
    const int items = nwrite * units;
    for (int i0 = tid; i0 < items; i0 += kOwnThreads * kOwnBatch) {
      T s[kOwnBatch];
      int beg[kOwnBatch], cnt[kOwnBatch], col[kOwnBatch], row[kOwnBatch];
      int maxc = 0;
#pragma unroll
      for (int b = 0; b < kOwnBatch; ++b) {
        const int i = i0 + b * kOwnThreads;
        cnt[b] = -1;
        s[b] = U::zero();
        if (i < items) {
          const int slot = i / units;
          col[b] = i - slot * units;
          row[b] = (int)rows[slot];
          beg[b] = row[b] ? (int)cur[row[b] - 1] : 0;
          cnt[b] = (int)cur[row[b]] - beg[b];
          if (acc) s[b] = dst[(int64_t)(lo + row[b]) * units + col[b]];
          maxc = max(maxc, cnt[b]);
        }
      }
      for (int k = 0; k < maxc; ++k) {
#pragma unroll
        for (int b = 0; b < kOwnBatch; ++b)
          if (k < cnt[b]) U::add(s[b], src[(int64_t)spos[beg[b] + k] * units + col[b]]);
      }
#pragma unroll
      for (int b = 0; b < kOwnBatch; ++b)
        if (cnt[b] >= 0) dst[(int64_t)(lo + row[b]) * units + col[b]] = s[b];
    }
    __syncthreads();  // the LDS lists are rebuilt by the next chunk
    if (scan >= n) break;
  }
}

template <bool VEC>
__global__ __launch_bounds__(kOwnThreads) void k_emb_bwd_owned(
    const int32_t* __restrict__ ids, int n, int ids_vec, int num, int span, int span_bits,
    const float* __restrict__ dout, int units, float* __restrict__ dw, int accumulate) {
  emb_owned_body<VEC>((int)blockIdx.x, ids, n, ids_vec, num, span, span_bits, dout, units, dw,
                      accumulate);
}

// Rows of a position table [num_pos, units] whose ids are pos0 + t for the
// positions t of a [batch, T] gradient: row pos0 + t is its prior value (or
// zero) plus dout[b][t] for b = 0, 1, ... in that order -- the embedding
// backward's rule (rows summed in increasing position order) for the ids
// pos0 + (p mod T).  Rows outside [pos0, pos0 + T) are zeroed when not
// accumulating.  Work item i = (row, unit); four items per thread with the
// loads of all four issued before their sums.
template <bool VEC>
__device__ __forceinline__ void emb_pos_body(int pg, int npg, const float* __restrict__ dout,
                                             int batch, int T, int units,
                                             float* __restrict__ dwp, int num_pos, int pos0,
                                             int accumulate) {
  typedef EmbUnit<VEC> U;
  typedef typename U::T E;
  const E* __restrict__ src = reinterpret_cast<const E*>(dout);
  E* __restrict__ dst = reinterpret_cast<E*>(dwp);
  const int64_t items = (int64_t)num_pos * units;
  const int64_t stride = (int64_t)npg * kOwnThreads;
  const int64_t bstride = (int64_t)T * units;
  constexpr int kPer = 4;
  for (int64_t i0 = (int64_t)pg * kOwnThreads + threadIdx.x; i0 < items; i0 += stride * kPer) {
    E s[kPer];
    int64_t base[kPer];
    bool in[kPer], live[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int64_t i = i0 + u * stride;
      live[u] = i < items;
      const int64_t r = live[u] ? i / units : 0;
      const int64_t t = r - pos0;
      in[u] = live[u] && t >= 0 && t < T;
      base[u] = in[u] ? t * units + (i - r * units) : 0;
      s[u] = (live[u] && accumulate) ? dst[i] : U::zero();
    }
    for (int b = 0; b < batch; ++b) {
      E v[kPer];
#pragma unroll
      for (int u = 0; u < kPer; ++u) v[u] = in[u] ? src[b * bstride + base[u]] : U::zero();
#pragma unroll
      for (int u = 0; u < kPer; ++u)
        if (in[u]) U::add(s[u], v[u]);
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u)
      if (live[u] && (in[u] || !accumulate)) dst[i0 + u * stride] = s[u];
  }
}

// One launch for the gradients of x = wte[ids] + wpe[pos0 + t]: workgroups
// [0, tok_groups) own row ranges of wte (emb_owned_body), the rest write
// wpe (emb_pos_body).
template <bool VEC>
__global__ __launch_bounds__(kOwnThreads) void k_emb_bwd_tok_pos(
    const int32_t* __restrict__ ids, int n, int ids_vec, int num, int span, int span_bits,
    const float* __restrict__ dout, int units, float* __restrict__ dw, int accumulate,
    int tok_groups, int batch, int T, float* __restrict__ dwp, int num_pos, int pos0,
    int acc_pos) {
  if ((int)blockIdx.x < tok_groups)
    emb_owned_body<VEC>((int)blockIdx.x, ids, n, ids_vec, num, span, span_bits, dout, units, dw,
                        accumulate);
  else
    emb_pos_body<VEC>((int)blockIdx.x - tok_groups, (int)gridDim.x - tok_groups, dout, batch, T,
                      units, dwp, num_pos, pos0, acc_pos);
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
  if (dim == 0) return TJH_OK;
  const bool vec = dim % 4 == 0 && ((uintptr_t)dout & 15) == 0 && ((uintptr_t)dweight & 15) == 0;
  // short lists (a batch of token positions): each workgroup sums the rows
  // it owns in one launch, zero rows included
  int64_t span = cdiv(num, (int64_t)kOwnGroups);
  if (span > kOwnMaxSpan) span = kOwnMaxSpan;
  const int64_t groups = cdiv(num, span);
  const int64_t units = vec ? dim / 4 : dim;
  if (n > 0 && n <= kOwnMaxN && groups * n <= kOwnMaxScan && num < (int64_t(1) << 31) &&
      span * units < (int64_t(1) << 31)) {
    int span_bits = 0;
    while ((int64_t(1) << span_bits) < span) ++span_bits;
    const int ids_vec = ((uintptr_t)ids & 15) == 0;
    KernelScope ks("embedding_bwd");
    if (vec)
      tjh_launch(k_emb_bwd_owned<true>, dim3((unsigned)groups), dim3(kOwnThreads), 0, stream(),
                 ids, (int)n, ids_vec, (int)num, (int)span, span_bits, dout, (int)units, dweight,
                 accumulate);
    else
      tjh_launch(k_emb_bwd_owned<false>, dim3((unsigned)groups), dim3(kOwnThreads), 0,
                 stream(), ids, (int)n, ids_vec, (int)num, (int)span, span_bits, dout,
                 (int)units, dweight, accumulate);
    return check_launch("embedding_backward");
  }
  if (!accumulate) {
    int rc = tjh_fill_f32(dweight, num * dim, 0.f);
    if (rc != TJH_OK) return rc;
  }
  if (n == 0) return TJH_OK;
  // long lists: (id, position) keys sorted by the bitonic network, then one
  // wave per run of equal ids
  int64_t npad = 1;
  while (npad < n) npad <<= 1;
  if (npad < 2) npad = 2;
  Scratch keys_s((size_t)npad * sizeof(uint64_t));
  if (!keys_s.ok()) return set_error(TJH_ERR_OOM, "embedding_backward: no scratch");
  uint64_t* keys = keys_s.as<uint64_t>();
  KernelScope ks("embedding_bwd");
  tjh_launch(k_make_keys, dim3((unsigned)cdiv(npad, kBlock)), dim3(kBlock), 0, stream(), ids, n,
             num, npad, keys);
  unsigned chunks = (unsigned)cdiv(npad, kSortChunk);
  tjh_launch(k_bitonic_local<true>, dim3(chunks), dim3(kSortThreads), 0, stream(), keys, npad,
             (int64_t)0);
  for (int64_t k = 2 * kSortChunk; k <= npad; k <<= 1) {
    for (int64_t j = k >> 1; j >= kSortChunk; j >>= 1)
      tjh_launch(k_bitonic_global, dim3((unsigned)cdiv(npad / 2, kBlock)), dim3(kBlock), 0,
                 stream(), keys, npad, k, j);
    tjh_launch(k_bitonic_local<false>, dim3(chunks), dim3(kSortThreads), 0, stream(), keys, npad,
               k);
  }
  int rc = check_launch("embedding_backward_sort");
  if (rc != TJH_OK) return rc;
  unsigned g = (unsigned)cdiv(n, kBlock / 64);
  if (vec)
    tjh_launch(k_emb_bwd_runs<true>, dim3(g), dim3(kBlock), 0, stream(), keys, n, dout, dim,
               dweight, 1);
  else
    tjh_launch(k_emb_bwd_runs<false>, dim3(g), dim3(kBlock), 0, stream(), keys, n, dout, dim,
               dweight, 1);
  return check_launch("embedding_backward");
}

int tjh_embedding_pos_forward(const float* weight, int64_t num, int64_t dim, const int32_t* ids,
                              int64_t batch, int64_t T, const float* pos_weight,
                              int64_t num_pos, int64_t pos0, float* out) {
  TJH_REQUIRE_INIT();
  TJH_ARG(num > 0 && num_pos > 0 && dim >= 0 && batch >= 0 && T >= 0 && pos0 >= 0,
          "tjh_embedding_pos_forward: bad sizes");
  TJH_ARG(pos0 + T <= num_pos, "tjh_embedding_pos_forward: positions [%lld, %lld) past the "
          "%lld-row position table", (long long)pos0, (long long)(pos0 + T), (long long)num_pos);
  const int64_t n = batch * T;
  if (n == 0 || dim == 0) return TJH_OK;
  TJH_ARG(weight && pos_weight && ids && out, "tjh_embedding_pos_forward: NULL pointer");
  KernelScope ks("embedding_fwd");
  const unsigned g = (unsigned)cdiv(n, kBlock / 64);
  const bool vec = dim % 4 == 0 && aligned16(weight) && aligned16(pos_weight) && aligned16(out);
  if (vec)
    tjh_launch(k_emb_pos_fwd<true>, dim3(g), dim3(kBlock), 0, stream(), weight, num, dim, ids, n,
               pos_weight, num_pos, pos0, T, out);
  else
    tjh_launch(k_emb_pos_fwd<false>, dim3(g), dim3(kBlock), 0, stream(), weight, num, dim, ids,
               n, pos_weight, num_pos, pos0, T, out);
  return check_launch("embedding_pos_forward");
}

int tjh_embedding_pos_backward(const float* dout, const int32_t* ids, int64_t batch, int64_t T,
                               int64_t dim, float* dweight, int64_t num, int accumulate,
                               float* dpos, int64_t num_pos, int64_t pos0, int acc_pos) {
  TJH_REQUIRE_INIT();
  TJH_ARG(num > 0 && num_pos > 0 && dim >= 0 && batch >= 0 && T >= 0 && pos0 >= 0,
          "tjh_embedding_pos_backward: bad sizes");
  TJH_ARG(pos0 + T <= num_pos, "tjh_embedding_pos_backward: positions past the table");
  const int64_t n = batch * T;
  TJH_ARG(n < (int64_t(1) << 31) && num_pos * dim < (int64_t(1) << 31),
          "tjh_embedding_pos_backward: too many elements");
  if (dim == 0) return TJH_OK;
  const bool vec = dim % 4 == 0 && aligned16(dout) && (!dweight || aligned16(dweight)) &&
                   (!dpos || aligned16(dpos));
  const int64_t units = vec ? dim / 4 : dim;
  int64_t span = cdiv(num, (int64_t)kOwnGroups);
  if (span > kOwnMaxSpan) span = kOwnMaxSpan;
  int64_t tok_groups = cdiv(num, span);
  const bool owned = n > 0 && n <= kOwnMaxN && tok_groups * n <= kOwnMaxScan &&
                     num < (int64_t(1) << 31) && span * units < (int64_t(1) << 31);
  if (dweight && !owned) {
    // a long id list: the sorting path for the token table, then the
    // position rows alone
    const int rc = tjh_embedding_backward(dout, ids, n, dim, dweight, num, accumulate);
    if (rc != TJH_OK) return rc;
  }
  if (!dweight || !owned) tok_groups = 0;
  int64_t pos_groups = 0;
  if (dpos) pos_groups = cdiv(num_pos * units, (int64_t)kOwnThreads * 4);
  if (pos_groups > 1024) pos_groups = 1024;
  if (tok_groups + pos_groups == 0) return TJH_OK;
  TJH_ARG(!tok_groups || ids, "tjh_embedding_pos_backward: NULL ids");
  int span_bits = 0;
  while ((int64_t(1) << span_bits) < span) ++span_bits;
  const int ids_vec = ((uintptr_t)ids & 15) == 0;
  KernelScope ks("embedding_bwd");
  const dim3 grid((unsigned)(tok_groups + pos_groups));
  if (vec)
    tjh_launch(k_emb_bwd_tok_pos<true>, grid, dim3(kOwnThreads), 0, stream(), ids, (int)n,
               ids_vec, (int)num, (int)span, span_bits, dout, (int)units, dweight, accumulate,
               (int)tok_groups, (int)batch, (int)T, dpos, (int)num_pos, (int)pos0, acc_pos);
  else
    tjh_launch(k_emb_bwd_tok_pos<false>, grid, dim3(kOwnThreads), 0, stream(), ids, (int)n,
               ids_vec, (int)num, (int)span, span_bits, dout, (int)units, dweight, accumulate,
               (int)tok_groups, (int)batch, (int)T, dpos, (int)num_pos, (int)pos0, acc_pos);
  return check_launch("embedding_pos_backward");
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
