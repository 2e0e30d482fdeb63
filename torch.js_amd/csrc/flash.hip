// Flash-style scaled dot-product attention for head dim 64, fp32 on the
// CDNA4 matrix cores (v_mfma_f32_32x32x2_f32), O(T) extra memory.
//
// Replaces the materialised-scores SDPA of torch.js
// (src/nn/functional.ts:866-890: Q K^T, log_softmax(...).exp(), @ V; the
// [B,H,T,T] score tensor is 403 MB per layer at T=1024) with tiles that
// never leave LDS / registers.
//
// Register layouts (one wave64 per 32 rows; lane l, l32 = l%32, h = l/32):
//   * contraction over the head dim d uses, in MFMA step s (0..31), the
//     pair d = s (lanes h=0) and d = 32 + s (lanes h=1): each lane's 32
//     operand values are one contiguous run of a row, read as float4s;
//   * a 32x32 accumulator register j of lane l holds C[8(j/4)+4h+j%4][l32],
//     so contracting over that accumulator's row index in step s pairs the
//     rows kappa(s,h) = 8(s/4)+4h+s%4 — exactly the lane's own register
//     j = s.  Probabilities computed in an accumulator therefore feed the
//     next product straight from registers, with no LDS round trip.
// Forward: S^T = K Q^T per 32-key block (lane <-> query), online softmax
//   per query in base 2, O^T += V^T P^T; lse written for the backward.
// Backward (deterministic, no atomics): D = rowsum(dO*O); a key-block
//   kernel accumulates dV^T = dO^T P and dK^T = Q^T dS (lane <-> key); a
//   query-block kernel accumulates dQ^T = K^T dS^T (lane <-> query).
// Causal masking (key > query masked, top-left aligned) skips every
// 32x32 tile that is entirely masked.

#include "common.h"

#include <float.h>

namespace tjh {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int HD = 64;        // head dim handled here
constexpr int TILE = 32;      // rows per wave and per streamed block
constexpr int WAVES = 4;      // waves per workgroup
constexpr int ROWS = WAVES * TILE;  // 128 rows (queries or keys) per workgroup
constexpr int LDSW = HD + 4;  // padded LDS row length (floats)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct Strides3 {
  int64_t b, h, t;
};

struct FlashArgs {
  const float* q;
  const float* k;
  const float* v;
  const float* o;
  const float* dout;
  const float* lse;   // [B,H,Tq] natural log
  const float* dsum;  // [B,H,Tq] rowsum(dO*O)
  float* out;         // o (forward) or dq / dk (backward)
  float* out2;        // dv (key kernel)
  float* lse_out;
  Strides3 qs, ks, vs, os, gs, o1s, o2s;
  int64_t H, Tq, Tk;
  float scale;        // softmax scale
  int causal;
  int nblk;           // row blocks per (b, h)
};

__device__ __forceinline__ int kappa(int s, int h) { return 8 * (s >> 2) + 4 * h + (s & 3); }

__device__ __forceinline__ floatx16 zero16() {
  floatx16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Loads rows [r0, r0+32) x 64 of a strided [T, 64] matrix into two float4
// registers per lane of a 256-lane workgroup (rows >= T read as zero).
__device__ __forceinline__ void load_tile(const float* __restrict__ base, int64_t st, int64_t r0,
                                          int64_t T, float4 (&reg)[2]) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    int f = threadIdx.x + 256 * i;
    int row = f >> 4, c4 = f & 15;
    int64_t r = r0 + row;
    reg[i] = r < T ? *reinterpret_cast<const float4*>(base + r * st + c4 * 4)
                   : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

__device__ __forceinline__ void store_tile(float* __restrict__ S, const float4 (&reg)[2]) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    int f = threadIdx.x + 256 * i;
    int row = f >> 4, c4 = f & 15;
    *reinterpret_cast<float4*>(S + row * LDSW + c4 * 4) = reg[i];
  }
}

// 32 operand values of a row: row[h*32 .. h*32+31] from LDS.
__device__ __forceinline__ void lds_row32(const float* __restrict__ S, int row, int h,
                                          float (&x)[32]) {
  const float4* p = reinterpret_cast<const float4*>(S + row * LDSW + h * 32);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float4 v = p[i];
    x[4 * i] = v.x;
    x[4 * i + 1] = v.y;
    x[4 * i + 2] = v.z;
    x[4 * i + 3] = v.w;
  }
}

// Same from global memory (rows >= T are zero), times `mul`.
__device__ __forceinline__ void gl_row32(const float* __restrict__ base, int64_t st, int64_t r,
                                         int64_t T, int h, float mul, float (&x)[32]) {
  if (r < T) {
    const float4* p = reinterpret_cast<const float4*>(base + r * st + h * 32);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float4 v = p[i];
      x[4 * i] = v.x * mul;
      x[4 * i + 1] = v.y * mul;
      x[4 * i + 2] = v.z * mul;
      x[4 * i + 3] = v.w * mul;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) x[i] = 0.f;
  }
}

// acc = A[32 x 64] . B[64 x 32] with A rows from LDS (row l32) and B
// columns from registers (b[s] pairs d = s / 32+s).
__device__ __forceinline__ floatx16 dot64_lds_reg(const float* __restrict__ S, int l32, int h,
                                                  const float (&b)[32]) {
  float a[32];
  lds_row32(S, l32, h, a);
  floatx16 acc = zero16();
#pragma unroll
  for (int s = 0; s < 32; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], b[s], acc, 0, 0, 0);
  return acc;
}

// acc[blk] += X^T[d x r] . P[r x 32] where X is a 32x64 LDS tile indexed
// [r][d] and P comes from the lane's accumulator registers.
__device__ __forceinline__ void accum_t(floatx16 (&acc)[2], const float* __restrict__ S,
                                        const floatx16& p, int l32, int h) {
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      float a = S[kappa(s, h) * LDSW + blk * 32 + l32];
      acc[blk] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, p[s], acc[blk], 0, 0, 0);
    }
  }
}

// Writes a transposed accumulator pair acc[blk][j] = X[row = l32][d] (d =
// blk*32 + 8(j/4)+4h+j%4) for the wave's 32 rows through LDS (buf, 32 x
// LDSW floats) into dst rows r0.. (stride st), scaled by mul[l32-row].
__device__ __forceinline__ void write_rows(float* __restrict__ buf, const floatx16 (&acc)[2],
                                           float mul, float* __restrict__ dst, int64_t st,
                                           int64_t r0, int64_t T, int l32, int h, int lane) {
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int j = 0; j < 16; ++j)
      buf[l32 * LDSW + blk * 32 + 8 * (j >> 2) + 4 * h + (j & 3)] = acc[blk][j] * mul;
  __syncthreads();  // every wave of the workgroup calls this the same number of times
  // 32 rows x 16 float4: 8 float4 per lane
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int f = lane + 64 * i;
    int row = f >> 4, c4 = f & 15;
    int64_t r = r0 + row;
    if (r < T)
      *reinterpret_cast<float4*>(dst + r * st + c4 * 4) =
          *reinterpret_cast<const float4*>(buf + row * LDSW + c4 * 4);
  }
}

// ------------------------------------------------------------ forward

__global__ __launch_bounds__(256) void k_flash_fwd(FlashArgs a) {
  __shared__ __attribute__((aligned(16))) float Ks[2][TILE * LDSW];
  __shared__ __attribute__((aligned(16))) float Vs[2][TILE * LDSW];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const int64_t bh = blockIdx.x / a.nblk;
  const int qb = a.nblk - 1 - (int)(blockIdx.x % a.nblk);  // heavy (causal) blocks first
  const int64_t b = bh / a.H, hh = bh % a.H;
  const float* Q = a.q + b * a.qs.b + hh * a.qs.h;
  const float* K = a.k + b * a.ks.b + hh * a.ks.h;
  const float* V = a.v + b * a.vs.b + hh * a.vs.h;
  const int64_t q0 = (int64_t)qb * ROWS + w * TILE;  // this wave's first query
  const int64_t myq = q0 + l32;

  float qf[32];
  gl_row32(Q, a.qs.t, myq, a.Tq, h, a.scale * kLog2e, qf);
  floatx16 acc[2] = {zero16(), zero16()};
  float m = -INFINITY, lsum = 0.f;

  int64_t kend = a.Tk;
  if (a.causal) {
    int64_t lim = (int64_t)qb * ROWS + ROWS;
    kend = lim < kend ? lim : kend;
  }
  const int nkb = (int)cdiv(kend, TILE);
  float4 rk[2], rv[2];
  load_tile(K, a.ks.t, 0, a.Tk, rk);
  load_tile(V, a.vs.t, 0, a.Tk, rv);
  store_tile(Ks[0], rk);
  store_tile(Vs[0], rv);
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const int cur = kb & 1;
    const bool more = kb + 1 < nkb;
    if (more) {
      load_tile(K, a.ks.t, (int64_t)(kb + 1) * TILE, a.Tk, rk);
      load_tile(V, a.vs.t, (int64_t)(kb + 1) * TILE, a.Tk, rv);
    }
    const int64_t k0 = (int64_t)kb * TILE;
    const bool skip = (a.causal && k0 > q0 + TILE - 1) || q0 >= a.Tq;
    if (!skip) {
      floatx16 st = dot64_lds_reg(Ks[cur], l32, h, qf);  // S^T[key][query], base-2 units
      float bm = -INFINITY;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        int64_t key = k0 + 8 * (j >> 2) + 4 * h + (j & 3);
        bool ok = key < a.Tk && (!a.causal || key <= myq);
        st[j] = ok ? st[j] : -INFINITY;
        bm = fmaxf(bm, st[j]);
      }
      bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
      const float mn = fmaxf(m, bm);
      if (mn != -INFINITY) {
        const float alpha = exp2f(m - mn);  // m = -inf -> 0
        float rs = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          st[j] = exp2f(st[j] - mn);
          rs += st[j];
        }
        rs += __shfl_xor(rs, 32, 64);
        lsum = lsum * alpha + rs;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          acc[0][j] *= alpha;
          acc[1][j] *= alpha;
        }
        m = mn;
        accum_t(acc, Vs[cur], st, l32, h);  // O^T += V^T P^T
      }
    }
    if (more) {
      store_tile(Ks[cur ^ 1], rk);
      store_tile(Vs[cur ^ 1], rv);
    }
    __syncthreads();
  }
  // normalise and write O (via LDS) and lse
  // every accumulator of a lane belongs to its query column: scale by 1/l
  const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
  float* obase = a.out + b * a.os.b + hh * a.os.h;
  float* buf = (w < 2 ? Ks[w] : Vs[w - 2]);
  write_rows(buf, acc, inv, obase, a.os.t, q0, a.Tq, l32, h, lane);
  if (h == 0 && myq < a.Tq) a.lse_out[bh * a.Tq + myq] = (m + log2f(lsum)) * kLn2;
}

// ------------------------------------------------------------ backward

// D[b,h,q] = sum_d dO*O  (one wave per query row of 64)
__global__ __launch_bounds__(256) void k_flash_dsum(FlashArgs a, float* __restrict__ dsum,
                                                    int64_t rows) {
  int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (r >= rows) return;
  int64_t bh = r / a.Tq, q = r % a.Tq;
  int64_t b = bh / a.H, hh = bh % a.H;
  float x = a.dout[b * a.gs.b + hh * a.gs.h + q * a.gs.t + lane] *
            a.o[b * a.os.b + hh * a.os.h + q * a.os.t + lane];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  if (lane == 0) dsum[r] = x;
}

// Key-block kernel: dK, dV for 128 keys per workgroup (32 per wave).
__global__ __launch_bounds__(256) void k_flash_dkv(FlashArgs a) {
  __shared__ __attribute__((aligned(16))) float Qs[2][TILE * LDSW];
  __shared__ __attribute__((aligned(16))) float Gs[2][TILE * LDSW];
  __shared__ float Ls[2][TILE];
  __shared__ float Ds[2][TILE];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const int64_t bh = blockIdx.x / a.nblk;
  const int kblk = (int)(blockIdx.x % a.nblk);
  const int64_t b = bh / a.H, hh = bh % a.H;
  const float* Q = a.q + b * a.qs.b + hh * a.qs.h;
  const float* K = a.k + b * a.ks.b + hh * a.ks.h;
  const float* V = a.v + b * a.vs.b + hh * a.vs.h;
  const float* G = a.dout + b * a.gs.b + hh * a.gs.h;
  const float* L = a.lse + bh * a.Tq;
  const float* Dd = a.dsum + bh * a.Tq;
  const int64_t k0 = (int64_t)kblk * ROWS + w * TILE;  // this wave's first key
  const int64_t mykey = k0 + l32;

  float kf[32], vf[32];
  gl_row32(K, a.ks.t, mykey, a.Tk, h, a.scale * kLog2e, kf);
  gl_row32(V, a.vs.t, mykey, a.Tk, h, 1.0f, vf);
  floatx16 dv[2] = {zero16(), zero16()};
  floatx16 dk[2] = {zero16(), zero16()};

  const int64_t qstart = a.causal ? (int64_t)kblk * ROWS : 0;
  const int nqb = (int)(qstart < a.Tq ? cdiv(a.Tq - qstart, TILE) : 0);
  auto load_ld = [&](int i, int buf) {
    if (threadIdx.x < TILE) {
      int64_t q = qstart + (int64_t)i * TILE + threadIdx.x;
      Ls[buf][threadIdx.x] = q < a.Tq ? L[q] * kLog2e : 0.f;
      Ds[buf][threadIdx.x] = q < a.Tq ? Dd[q] : 0.f;
    }
  };
  float4 rq[2], rg[2];
  if (nqb > 0) {
    load_tile(Q, a.qs.t, qstart, a.Tq, rq);
    load_tile(G, a.gs.t, qstart, a.Tq, rg);
    store_tile(Qs[0], rq);
    store_tile(Gs[0], rg);
    load_ld(0, 0);
  }
  __syncthreads();
  for (int qi = 0; qi < nqb; ++qi) {
    const int cur = qi & 1;
    const bool more = qi + 1 < nqb;
    const int64_t qq0 = qstart + (int64_t)qi * TILE;
    if (more) {
      load_tile(Q, a.qs.t, qq0 + TILE, a.Tq, rq);
      load_tile(G, a.gs.t, qq0 + TILE, a.Tq, rg);
    }
    const bool skip = (a.causal && qq0 + TILE - 1 < k0) || k0 >= a.Tk;
    if (!skip) {
      // S[q][key] (base 2): A = Q rows from LDS, B = K^T from registers
      floatx16 p = dot64_lds_reg(Qs[cur], l32, h, kf);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        int r = 8 * (j >> 2) + 4 * h + (j & 3);
        int64_t q = qq0 + r;
        bool ok = q < a.Tq && mykey < a.Tk && (!a.causal || mykey <= q);
        p[j] = ok ? exp2f(p[j] - Ls[cur][r]) : 0.f;
      }
      accum_t(dv, Gs[cur], p, l32, h);  // dV^T += dO^T P
      // dP[q][key] = dO . V^T
      floatx16 dp = dot64_lds_reg(Gs[cur], l32, h, vf);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        int r = 8 * (j >> 2) + 4 * h + (j & 3);
        dp[j] = p[j] * (dp[j] - Ds[cur][r]);  // dS
      }
      accum_t(dk, Qs[cur], dp, l32, h);  // dK^T += Q^T dS
    }
    if (more) {
      store_tile(Qs[cur ^ 1], rq);
      store_tile(Gs[cur ^ 1], rg);
      load_ld(qi + 1, cur ^ 1);
    }
    __syncthreads();
  }
  float* dkb = a.out + b * a.o1s.b + hh * a.o1s.h;
  float* dvb = a.out2 + b * a.o2s.b + hh * a.o2s.h;
  float* buf = (w < 2 ? Qs[w] : Gs[w - 2]);
  write_rows(buf, dk, a.scale, dkb, a.o1s.t, k0, a.Tk, l32, h, lane);
  __syncthreads();
  write_rows(buf, dv, 1.0f, dvb, a.o2s.t, k0, a.Tk, l32, h, lane);
}

// Query-block kernel: dQ for 128 queries per workgroup (32 per wave).
__global__ __launch_bounds__(256) void k_flash_dq(FlashArgs a) {
  __shared__ __attribute__((aligned(16))) float Ks[2][TILE * LDSW];
  __shared__ __attribute__((aligned(16))) float Vs[2][TILE * LDSW];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const int64_t bh = blockIdx.x / a.nblk;
  const int qb = a.nblk - 1 - (int)(blockIdx.x % a.nblk);
  const int64_t b = bh / a.H, hh = bh % a.H;
  const float* Q = a.q + b * a.qs.b + hh * a.qs.h;
  const float* K = a.k + b * a.ks.b + hh * a.ks.h;
  const float* V = a.v + b * a.vs.b + hh * a.vs.h;
  const float* G = a.dout + b * a.gs.b + hh * a.gs.h;
  const int64_t q0 = (int64_t)qb * ROWS + w * TILE;
  const int64_t myq = q0 + l32;

  float qf[32], gf[32];
  gl_row32(Q, a.qs.t, myq, a.Tq, h, a.scale * kLog2e, qf);
  gl_row32(G, a.gs.t, myq, a.Tq, h, 1.0f, gf);
  const float lq = myq < a.Tq ? a.lse[bh * a.Tq + myq] * kLog2e : 0.f;
  const float dq_ = myq < a.Tq ? a.dsum[bh * a.Tq + myq] : 0.f;
  floatx16 dq[2] = {zero16(), zero16()};

  int64_t kend = a.Tk;
  if (a.causal) {
    int64_t lim = (int64_t)qb * ROWS + ROWS;
    kend = lim < kend ? lim : kend;
  }
  const int nkb = (int)cdiv(kend, TILE);
  float4 rk[2], rv[2];
  load_tile(K, a.ks.t, 0, a.Tk, rk);
  load_tile(V, a.vs.t, 0, a.Tk, rv);
  store_tile(Ks[0], rk);
  store_tile(Vs[0], rv);
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const int cur = kb & 1;
    const bool more = kb + 1 < nkb;
    if (more) {
      load_tile(K, a.ks.t, (int64_t)(kb + 1) * TILE, a.Tk, rk);
      load_tile(V, a.vs.t, (int64_t)(kb + 1) * TILE, a.Tk, rv);
    }
    const int64_t k0 = (int64_t)kb * TILE;
    const bool skip = (a.causal && k0 > q0 + TILE - 1) || q0 >= a.Tq;
    if (!skip) {
      floatx16 p = dot64_lds_reg(Ks[cur], l32, h, qf);   // S^T[key][q]
      floatx16 dp = dot64_lds_reg(Vs[cur], l32, h, gf);  // dP^T[key][q]
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        int64_t key = k0 + 8 * (j >> 2) + 4 * h + (j & 3);
        bool ok = key < a.Tk && myq < a.Tq && (!a.causal || key <= myq);
        float pj = ok ? exp2f(p[j] - lq) : 0.f;
        dp[j] = pj * (dp[j] - dq_);  // dS^T
      }
      accum_t(dq, Ks[cur], dp, l32, h);  // dQ^T += K^T dS^T
    }
    if (more) {
      store_tile(Ks[cur ^ 1], rk);
      store_tile(Vs[cur ^ 1], rv);
    }
    __syncthreads();
  }
  float* dqb = a.out + b * a.o1s.b + hh * a.o1s.h;
  float* buf = (w < 2 ? Ks[w] : Vs[w - 2]);
  write_rows(buf, dq, a.scale, dqb, a.o1s.t, q0, a.Tq, l32, h, lane);
}

bool rows_ok(const int64_t* s, const void* p) {
  // D contiguous, 16-byte aligned rows
  return ((uintptr_t)p & 15) == 0 && (s[0] % 4) == 0 && (s[1] % 4) == 0 && (s[2] % 4) == 0;
}

Strides3 s3(const int64_t* s) { return Strides3{s[0], s[1], s[2]}; }

}  // namespace

bool flash_supported(int64_t D, const void* const* ptrs, const int64_t* const* strides, int n) {
  if (D != HD) return false;
  for (int i = 0; i < n; ++i)
    if (!rows_ok(strides[i], ptrs[i])) return false;
  return true;
}

int flash_forward(const float* q, const float* k, const float* v, float* o, float* lse, int64_t B,
                  int64_t H, int64_t Tq, int64_t Tk, const int64_t* qs, const int64_t* ks,
                  const int64_t* vs, const int64_t* os, float scale, int causal) {
  FlashArgs a{};
  a.q = q; a.k = k; a.v = v; a.out = o; a.lse_out = lse;
  a.qs = s3(qs); a.ks = s3(ks); a.vs = s3(vs); a.os = s3(os);
  a.H = H; a.Tq = Tq; a.Tk = Tk; a.scale = scale; a.causal = causal;
  a.nblk = (int)cdiv(Tq, ROWS);
  int64_t grid = B * H * a.nblk;
  TJH_ARG(grid < (int64_t(1) << 31), "sdpa: grid too large");
  KernelScope ks_("sdpa_fwd");
  hipLaunchKernelGGL(k_flash_fwd, dim3((unsigned)grid), dim3(256), 0, stream(), a);
  return check_launch("flash_forward");
}

int flash_backward(const float* q, const float* k, const float* v, const float* o,
                   const float* dout, const float* lse, float* dq, float* dk, float* dv,
                   int64_t B, int64_t H, int64_t Tq, int64_t Tk, const int64_t* const* st,
                   float scale, int causal) {
  FlashArgs a{};
  a.q = q; a.k = k; a.v = v; a.o = o; a.dout = dout; a.lse = lse;
  a.qs = s3(st[0]); a.ks = s3(st[1]); a.vs = s3(st[2]); a.os = s3(st[3]); a.gs = s3(st[4]);
  a.H = H; a.Tq = Tq; a.Tk = Tk; a.scale = scale; a.causal = causal;
  Scratch ds((size_t)(B * H * Tq) * sizeof(float));
  if (!ds.ok()) return set_error(TJH_ERR_OOM, "sdpa_backward: no scratch");
  a.dsum = ds.as<float>();
  KernelScope ks_("sdpa_bwd");
  int64_t rows = B * H * Tq;
  hipLaunchKernelGGL(k_flash_dsum, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, stream(), a,
                     ds.as<float>(), rows);
  int rc = check_launch("flash_dsum");
  if (rc != TJH_OK) return rc;
  // keys: dK, dV
  a.nblk = (int)cdiv(Tk, ROWS);
  a.out = dk; a.out2 = dv; a.o1s = s3(st[6]); a.o2s = s3(st[7]);
  hipLaunchKernelGGL(k_flash_dkv, dim3((unsigned)(B * H * a.nblk)), dim3(256), 0, stream(), a);
  rc = check_launch("flash_dkv");
  if (rc != TJH_OK) return rc;
  // queries: dQ
  a.nblk = (int)cdiv(Tq, ROWS);
  a.out = dq; a.out2 = nullptr; a.o1s = s3(st[5]);
  hipLaunchKernelGGL(k_flash_dq, dim3((unsigned)(B * H * a.nblk)), dim3(256), 0, stream(), a);
  return check_launch("flash_dq");
}

}  // namespace tjh
