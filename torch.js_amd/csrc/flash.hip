// Flash-style scaled dot-product attention, fp32 on the CDNA4 matrix cores
// (v_mfma_f32_32x32x2_f32), O(T) extra memory, for head dims D <= 128 with
// D % 4 == 0.  Each kernel is compiled for a padded head dim HD in
// {32, 64, 96, 128} (D rounded up to a multiple of 32); columns D..HD-1 are
// read as zero and never written, so they add exact zeros to every product.
//
// Replaces the materialised-scores SDPA of torch.js
// (src/nn/functional.ts:866-890: Q K^T, log_softmax(...).exp(), @ V; the
// [B,H,T,T] score tensor is 403 MB per layer at T=1024) with tiles that
// never leave LDS / registers.
//
// Register layouts (one wave64 per 32 rows; lane l, l32 = l%32, h = l/32):
//   * contraction over the head dim d uses, in MFMA step s (0..HD/2-1), the
//     pair d = s (lanes h=0) and d = HD/2 + s (lanes h=1): each lane's HD/2
//     operand values are one contiguous run of a row, read as 128-bit LDS
//     loads;
//   * a 32x32 accumulator register j of lane l holds C[8(j/4)+4h+j%4][l32],
//     so contracting over that accumulator's row index in step s pairs the
//     rows kappa(s,h) = 8(s/4)+4h+s%4 — exactly the lane's own register
//     j = s.  Probabilities computed in an accumulator therefore feed the
//     next product straight from registers, with no LDS round trip;
//   * a transposed [HD, 32] result (O^T, dK^T, ...) is HD/32 accumulators,
//     one per 32-column block of the head dim;
//   * a per-row offset (-lse, -rowsum(dO*O)) is folded into a product as
//     one extra MFMA step whose operands are (offset, 1) on the h = 0 lanes
//     and zero on the others, so it costs no per-element VALU work.
// Forward: S^T = K Q^T per 32-key block (lane <-> query), online softmax
//   per query in base 2, O^T += V^T P^T; lse written for the backward.
// Backward (deterministic, no atomics): D = rowsum(dO*O); a key-block
//   kernel accumulates dV^T = dO^T P and dK^T = Q^T dS (lane <-> key) and
//   stores each 32x32 block of dS, the products of each 32-key group split
//   over a pair of waves (P and dV / dS and dK); a query-block kernel
//   accumulates dQ^T = K^T dS^T (lane <-> query) from those blocks, so S
//   and dP are computed once (when the blocks cannot be allocated, a
//   four-product key-block kernel runs and the query kernel recomputes S
//   and dP instead).
// Causal masking (key > query masked, top-left aligned) skips every
// 32x32 tile that is entirely masked and masks element-wise only on tiles
// that cross the diagonal or the end of the sequence.
// exp2 runs on the hardware unit (v_exp_f32); arguments are <= 0 after the
// max / lse subtraction, and results below 2^-126 flush to zero.
// Workgroups are mapped to (batch*head, block) items by cost rank so that
// every XCD, and every CU inside it, holds the same mix of long and short
// causal blocks (balanced_rank).

#include "common.h"
#include "wave.h"

#include <float.h>
#include <stdlib.h>

namespace tjh {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int HD_MAX = 128;   // largest head dim handled here
constexpr int TILE = 32;      // rows per wave and per streamed block
constexpr int WAVES = 4;      // waves per workgroup
constexpr int ROWS = WAVES * TILE;  // 128 rows (queries or keys) per workgroup
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kXcds = 8;

// Shape constants of a padded head dim HD.
template <int HD>
struct Hd {
  static_assert(HD % 32 == 0 && HD >= 32 && HD <= HD_MAX, "head dim");
  static constexpr int NC = HD / 32;   // 32-column blocks (accumulators of a [HD,32] result)
  static constexpr int RUN = HD / 2;   // contraction values per lane
  static constexpr int W = HD + 4;     // padded LDS row length (floats)
  static constexpr int F4 = HD / 4;    // float4 per row
};

// Workgroups per CU each kernel is compiled for: the LDS tiles grow with
// HD (the paired key kernel's 43 KB at HD 64 allows three per CU, 76 KB at
// HD 128 two), and so do the register-resident rows (the forward at HD 128
// and the four-product kernels above HD 64 would spill at two).
template <int HD> constexpr int occ_fwd() { return HD <= 96 ? 2 : 1; }
template <int HD> constexpr int occ_main() { return HD <= 64 ? 2 : 1; }
template <int HD> constexpr int occ_pair() { return HD <= 64 ? 3 : 2; }

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
  int64_t H;
  int Tq, Tk;
  int D;              // head dim (columns D.. of the padded tiles are zero)
  float scale;        // softmax scale
  int causal;
  int nblk;           // row blocks per (b, h)
  int cus;            // compute units per XCD
  // dS blocks written by the key-block kernel for the query-block kernel:
  // [b*H + h][query tile][key tile][32 x 32], or null (dQ recomputes dS)
  float* dsblk;
  int nqt, nkt;       // 32-row query / key tiles per (b, h)
  int64_t spare_blk;  // index of the spare block after the last one
};

// Column of key offset ko (0..31) inside a dS block row: the query-block
// kernel's lane (query row, h) reads its 16 keys kappa(j, h), j = 0..15, as
// one contiguous run at h*16, so key kappa(j, h) sits at h*16 + j.
__device__ __forceinline__ int ds_col(int ko) {
  return ((ko >> 2) & 1) * 16 + (((ko >> 3) << 2) | (ko & 3));
}

// Cost rank of the item a workgroup processes (rank 0 = most expensive).
// Workgroup w runs on XCD w % 8, and the j-th workgroup an XCD receives
// lands on its CU j % cus (one "round" per cus workgroups; the rounds are
// co-resident when the kernel's occupancy allows).  Ranks go round-robin
// over the XCDs, and within an XCD each round is laid over the CUs in
// alternating direction, so every CU holds one long, one middle and one
// short causal block instead of three of the same length.
__device__ __forceinline__ int balanced_rank(int bid, int n, int cus) {
  const int x = bid % kXcds, j = bid / kXcds;
  const int cnt = (n - x + kXcds - 1) / kXcds;  // items on this XCD
  const int round = j / cus, c = j % cus;
  const int in_round = min(cus, cnt - round * cus);
  const int p = round * cus + ((round & 1) ? in_round - 1 - c : c);
  return p * kXcds + x;
}

__device__ __forceinline__ int kappa(int s, int h) { return 8 * (s >> 2) + 4 * h + (s & 3); }

__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ floatx16 mfma(float a, float b, const floatx16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ floatx16 zero16() {
  floatx16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Loads rows [r0, r0+32) x HD of a strided [T, D] matrix, HD/32 float4 per
// lane of a 256-lane workgroup.  GUARD: rows >= T and columns >= D read as
// zero.
template <int HD, bool GUARD>
__device__ __forceinline__ void load_tile(const float* __restrict__ base, int64_t st, int r0, int T,
                                          int D, floatx4 (&reg)[Hd<HD>::NC], int tid = -1) {
  if (tid < 0) tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < Hd<HD>::NC; ++i) {
    const int f = tid + 256 * i;
    const int row = f / Hd<HD>::F4, c4 = f % Hd<HD>::F4;
    const int r = r0 + row;
    if (!GUARD || (r < T && c4 * 4 < D))
      reg[i] = *reinterpret_cast<const floatx4*>(base + (int64_t)r * st + c4 * 4);
    else
      reg[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
}

template <int HD>
__device__ __forceinline__ void store_tile(float* __restrict__ S, const floatx4 (&reg)[Hd<HD>::NC],
                                           int tid = -1) {
  if (tid < 0) tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < Hd<HD>::NC; ++i) {
    const int f = tid + 256 * i;
    const int row = f / Hd<HD>::F4, c4 = f % Hd<HD>::F4;
    *reinterpret_cast<floatx4*>(S + row * Hd<HD>::W + c4 * 4) = reg[i];
  }
}

// The HD/2 operand values row[h*HD/2 ..] of an LDS tile row.
template <int HD>
__device__ __forceinline__ void lds_run(const float* __restrict__ S, int row, int h,
                                        float (&x)[Hd<HD>::RUN]) {
  const floatx4* p = reinterpret_cast<const floatx4*>(S + row * Hd<HD>::W + h * Hd<HD>::RUN);
#pragma unroll
  for (int i = 0; i < Hd<HD>::RUN / 4; ++i) {
    const floatx4 v = p[i];
    x[4 * i] = v.x;
    x[4 * i + 1] = v.y;
    x[4 * i + 2] = v.z;
    x[4 * i + 3] = v.w;
  }
}

// The same run from global memory (rows >= T are zero; with GUARD, columns
// >= D too), times `mul`.
template <int HD, bool GUARD>
__device__ __forceinline__ void gl_run(const float* __restrict__ base, int64_t st, int r, int T,
                                       int D, int h, float mul, float (&x)[Hd<HD>::RUN]) {
  if (r < T) {
    const floatx4* p =
        reinterpret_cast<const floatx4*>(base + (int64_t)r * st + h * Hd<HD>::RUN);
#pragma unroll
    for (int i = 0; i < Hd<HD>::RUN / 4; ++i) {
      floatx4 v = floatx4{0.f, 0.f, 0.f, 0.f};
      if (!GUARD || h * Hd<HD>::RUN + 4 * i < D) v = p[i];
      x[4 * i] = v.x * mul;
      x[4 * i + 1] = v.y * mul;
      x[4 * i + 2] = v.z * mul;
      x[4 * i + 3] = v.w * mul;
    }
  } else {
#pragma unroll
    for (int i = 0; i < Hd<HD>::RUN; ++i) x[i] = 0.f;
  }
}

// Operands of a transposed product X^T . P for a 32-row LDS tile X [r][d]:
// in step s the lane contributes X[kappa(s,h)][c*32 + l32] to block c.
template <int HD>
__device__ __forceinline__ void lds_cols(const float* __restrict__ S, int l32, int h,
                                         float (&x)[Hd<HD>::NC][16]) {
#pragma unroll
  for (int s = 0; s < 16; ++s)
#pragma unroll
    for (int c = 0; c < Hd<HD>::NC; ++c) x[c][s] = S[kappa(s, h) * Hd<HD>::W + c * 32 + l32];
}

// acc = offset-step + sum over HD/2 steps of a[s] * b[s].  The offset step
// adds off_a[m] * off_b[n] through the h = 0 lanes (a rank-1 update).
template <int HD>
__device__ __forceinline__ floatx16 chain(float off_a, float off_b,
                                          const float (&a)[Hd<HD>::RUN],
                                          const float (&b)[Hd<HD>::RUN]) {
  floatx16 acc = mfma(off_a, off_b, zero16());
#pragma unroll
  for (int s = 0; s < Hd<HD>::RUN; ++s) acc = mfma(a[s], b[s], acc);
  return acc;
}

template <int HD>
__device__ __forceinline__ floatx16 chain0(const float (&a)[Hd<HD>::RUN],
                                           const float (&b)[Hd<HD>::RUN]) {
  floatx16 acc = mfma(a[0], b[0], zero16());
#pragma unroll
  for (int s = 1; s < Hd<HD>::RUN; ++s) acc = mfma(a[s], b[s], acc);
  return acc;
}

// Writes transposed accumulators acc[c][j] = X[row = l32][d] (d = c*32 +
// 8(j/4)+4h+j%4) for the wave's 32 rows through LDS (buf, 32 x W floats)
// into dst rows r0.. (stride st, columns < D), times `mul`.
template <int HD>
__device__ __forceinline__ void write_rows(float* __restrict__ buf,
                                           const floatx16 (&acc)[Hd<HD>::NC], float mul,
                                           float* __restrict__ dst, int64_t st, int r0, int T,
                                           int D, int l32, int h, int lane) {
#pragma unroll
  for (int j = 0; j < 16; ++j)
#pragma unroll
    for (int c = 0; c < Hd<HD>::NC; ++c)
      buf[l32 * Hd<HD>::W + c * 32 + 8 * (j >> 2) + 4 * h + (j & 3)] = acc[c][j] * mul;
  __syncthreads();  // every wave of the workgroup calls this the same number of times
  // 32 rows x HD/4 float4: HD/8 float4 per lane
#pragma unroll
  for (int i = 0; i < HD / 8; ++i) {
    const int f = lane + 64 * i;
    const int row = f / Hd<HD>::F4, c4 = f % Hd<HD>::F4;
    const int r = r0 + row;
    if (r < T && c4 * 4 < D)
      *reinterpret_cast<floatx4*>(dst + (int64_t)r * st + c4 * 4) =
          *reinterpret_cast<const floatx4*>(buf + row * Hd<HD>::W + c4 * 4);
  }
}

template <int NC>
__device__ __forceinline__ void zero_acc(floatx16 (&acc)[NC]) {
#pragma unroll
  for (int c = 0; c < NC; ++c) acc[c] = zero16();
}

// ------------------------------------------------------------ forward

// GUARD: Tk is not a multiple of 32 (the last key tile is partial), or D <
// HD (padded columns).
template <int HD, bool GUARD>
__global__ __launch_bounds__(256, occ_fwd<HD>()) void k_flash_fwd(FlashArgs a) {
  using S_ = Hd<HD>;
  __shared__ __attribute__((aligned(16))) float Ks[2][TILE * S_::W];
  __shared__ __attribute__((aligned(16))) float Vs[2][TILE * S_::W];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const int64_t nbh = (int64_t)gridDim.x / a.nblk;
  const int g = balanced_rank(blockIdx.x, gridDim.x, a.cus);
  const int64_t bh = g % nbh;
  const int qb = a.nblk - 1 - (int)(g / nbh);  // long (causal) blocks rank first
  const int64_t b = bh / a.H, hh = bh % a.H;
  const float* Q = a.q + b * a.qs.b + hh * a.qs.h;
  const float* K = a.k + b * a.ks.b + hh * a.ks.h;
  const float* V = a.v + b * a.vs.b + hh * a.vs.h;
  const int q0 = qb * ROWS + w * TILE;  // this wave's first query
  const int myq = q0 + l32;

  float qf[S_::RUN];
  gl_run<HD, GUARD>(Q, a.qs.t, myq, a.Tq, a.D, h, a.scale * kLog2e, qf);
  floatx16 acc[S_::NC];
  zero_acc(acc);
  float m = -INFINITY, lsum = 0.f;

  int kend = a.Tk;
  if (a.causal) kend = min(kend, qb * ROWS + ROWS);
  const int nkb = (kend + TILE - 1) / TILE;
  floatx4 rk[S_::NC], rv[S_::NC];
  load_tile<HD, GUARD>(K, a.ks.t, 0, a.Tk, a.D, rk);
  load_tile<HD, GUARD>(V, a.vs.t, 0, a.Tk, a.D, rv);
  store_tile<HD>(Ks[0], rk);
  store_tile<HD>(Vs[0], rv);
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const int cur = kb & 1;
    const bool more = kb + 1 < nkb;
    if (more) {
      load_tile<HD, GUARD>(K, a.ks.t, (kb + 1) * TILE, a.Tk, a.D, rk);
      load_tile<HD, GUARD>(V, a.vs.t, (kb + 1) * TILE, a.Tk, a.D, rv);
    }
    const int k0 = kb * TILE;
    const bool skip = (a.causal && k0 > q0 + TILE - 1) || q0 >= a.Tq;
    if (!skip) {
      float ka[S_::RUN];
      lds_run<HD>(Ks[cur], l32, h, ka);
      floatx16 st = chain0<HD>(ka, qf);  // S^T[key][query], base-2 units
      float va[S_::NC][16];
      lds_cols<HD>(Vs[cur], l32, h, va);
      const bool edge = (a.causal && k0 + TILE - 1 > q0) || (GUARD && k0 + TILE > a.Tk);
      if (edge) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int key = k0 + kappa(j, h);
          const bool ok = key < a.Tk && (!a.causal || key <= myq);
          st[j] = ok ? st[j] : -INFINITY;
        }
      }
      float bm = st[0];
#pragma unroll
      for (int j = 1; j < 16; ++j) bm = fmaxf(bm, st[j]);
      bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
      const float mn = fmaxf(m, bm);
      const float ms = mn == -INFINITY ? 0.f : mn;  // every key so far masked
      const float alpha = exp2_hw(m - ms);          // m = -inf -> 0
      float rs = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        st[j] = exp2_hw(st[j] - ms);
        rs += st[j];
      }
      rs += __shfl_xor(rs, 32, 64);
      lsum = lsum * alpha + rs;
      m = mn;
#pragma unroll
      for (int c = 0; c < S_::NC; ++c) acc[c] *= alpha;
#pragma unroll
      for (int s = 0; s < 16; ++s)  // O^T += V^T P^T
#pragma unroll
        for (int c = 0; c < S_::NC; ++c) acc[c] = mfma(va[c][s], st[s], acc[c]);
    }
    if (more) {
      store_tile<HD>(Ks[cur ^ 1], rk);
      store_tile<HD>(Vs[cur ^ 1], rv);
    }
    __syncthreads();
  }
  // every accumulator of a lane belongs to its query column: scale by 1/l
  const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
  float* obase = a.out + b * a.os.b + hh * a.os.h;
  float* buf = (w < 2 ? Ks[w] : Vs[w - 2]);
  write_rows<HD>(buf, acc, inv, obase, a.os.t, q0, a.Tq, a.D, l32, h, lane);
  if (h == 0 && myq < a.Tq) a.lse_out[bh * a.Tq + myq] = (m + __log2f(lsum)) * kLn2;
}

// ------------------------------------------------------------ backward

// D[b,h,q] = sum_d dO*O  (one wave per query row, lanes striding the row)
__global__ __launch_bounds__(256) void k_flash_dsum(FlashArgs a, float* __restrict__ dsum,
                                                    int64_t rows) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const int64_t bh = r / a.Tq, q = r % a.Tq;
  const int64_t b = bh / a.H, hh = bh % a.H;
  float x = 0.f;
  for (int c = lane; c < a.D; c += 64)
    x += a.dout[b * a.gs.b + hh * a.gs.h + q * a.gs.t + c] *
         a.o[b * a.os.b + hh * a.os.h + q * a.os.t + c];
  x = wave_sum(x);
  if (lane == 0) dsum[r] = x;
}

// The same with 128-bit loads: 16 lanes per row (each taking the float4s
// sub, sub + 16, ... of its row), four rows per 16-lane group with all
// loads issued first (64 rows per workgroup; 9% faster than one row per
// group at D = 64); O is read here only (non-temporal), dO stays cached for
// the two kernels that follow.  Needs 16-byte aligned rows.
template <int HD>
__global__ __launch_bounds__(256) void k_flash_dsum4(FlashArgs a, float* __restrict__ dsum,
                                                     int64_t rows) {
  constexpr int R = 4;                       // rows per 16-lane group, all loads issued first
  constexpr int CH = (HD / 4 + 15) / 16;     // float4 per lane and row
  const int64_t r0 = ((int64_t)blockIdx.x * 16 + (threadIdx.x >> 4)) * R;
  const int sub = threadIdx.x & 15;
  float4 g[R][CH], o[R][CH];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int64_t r = min(r0 + i, rows - 1);
    const int64_t bh = r / a.Tq, q = r % a.Tq;
    const int64_t b = bh / a.H, hh = bh % a.H;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int col = 4 * (sub + 16 * c);
      if (col < a.D) {
        g[i][c] = *reinterpret_cast<const float4*>(a.dout + b * a.gs.b + hh * a.gs.h +
                                                   q * a.gs.t + col);
        o[i][c] = ld_nt(a.o + b * a.os.b + hh * a.os.h + q * a.os.t + col);
      } else {
        g[i][c] = make_float4(0.f, 0.f, 0.f, 0.f);
        o[i][c] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < R; ++i) {
    float x = (g[i][0].x * o[i][0].x + g[i][0].y * o[i][0].y) +
              (g[i][0].z * o[i][0].z + g[i][0].w * o[i][0].w);
#pragma unroll
    for (int c = 1; c < CH; ++c)
      x += (g[i][c].x * o[i][c].x + g[i][c].y * o[i][c].y) +
           (g[i][c].z * o[i][c].z + g[i][c].w * o[i][c].w);
    x = row16_sum(x);  // the 16-lane group is one DPP row
    if (sub == 0 && r0 + i < rows) dsum[r0 + i] = x;
  }
}

// Key-block kernel: dK, dV for 128 keys per workgroup (32 per wave), each
// wave forming all four products; the path taken when the dS blocks cannot
// be allocated (the query-block kernel then recomputes S and dP).
// GUARD: Tq or Tk is not a multiple of 32, or D < HD.
template <int HD, bool GUARD>
__global__ __launch_bounds__(256, occ_main<HD>()) void k_flash_dkv(FlashArgs a) {
  using S_ = Hd<HD>;
  __shared__ __attribute__((aligned(16))) float Qs[2][TILE * S_::W];
  __shared__ __attribute__((aligned(16))) float Gs[2][TILE * S_::W];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const int64_t nbh = (int64_t)gridDim.x / a.nblk;
  const int g = balanced_rank(blockIdx.x, gridDim.x, a.cus);
  const int64_t bh = g % nbh;
  const int kblk = (int)(g / nbh);  // long (causal) blocks rank first
  const int64_t b = bh / a.H, hh = bh % a.H;
  const float* Q = a.q + b * a.qs.b + hh * a.qs.h;
  const float* K = a.k + b * a.ks.b + hh * a.ks.h;
  const float* V = a.v + b * a.vs.b + hh * a.vs.h;
  const float* G = a.dout + b * a.gs.b + hh * a.gs.h;
  const float* L = a.lse + bh * a.Tq;
  const float* Dd = a.dsum + bh * a.Tq;
  const int k0 = kblk * ROWS + w * TILE;  // this wave's first key
  const int mykey = k0 + l32;

  float kf[S_::RUN], vf[S_::RUN];
  gl_run<HD, GUARD>(K, a.ks.t, mykey, a.Tk, a.D, h, a.scale * kLog2e, kf);
  gl_run<HD, GUARD>(V, a.vs.t, mykey, a.Tk, a.D, h, 1.0f, vf);
  floatx16 dv[S_::NC], dk[S_::NC];
  zero_acc(dv);
  zero_acc(dk);
  const float one = h == 0 ? 1.f : 0.f;

  const int qstart = a.causal ? kblk * ROWS : 0;
  const int nqb = qstart < a.Tq ? (a.Tq - qstart + TILE - 1) / TILE : 0;
  // per-lane row offsets of the current / next query tile (query qq0 + l32)
  auto row_off = [&](int qq0, float& lo, float& dof) {
    const int q = qq0 + l32;
    const bool in = !GUARD || q < a.Tq;
    lo = (h == 0 && in) ? -L[q] * kLog2e : 0.f;
    dof = (h == 0 && in) ? -Dd[q] : 0.f;
  };
  floatx4 rq[S_::NC], rg[S_::NC];
  float lo = 0.f, dof = 0.f, lo_n = 0.f, dof_n = 0.f;
  if (nqb > 0) {
    load_tile<HD, GUARD>(Q, a.qs.t, qstart, a.Tq, a.D, rq);
    load_tile<HD, GUARD>(G, a.gs.t, qstart, a.Tq, a.D, rg);
    store_tile<HD>(Qs[0], rq);
    store_tile<HD>(Gs[0], rg);
    row_off(qstart, lo, dof);
  }
  __syncthreads();
  for (int qi = 0; qi < nqb; ++qi) {
    const int cur = qi & 1;
    const bool more = qi + 1 < nqb;
    const int qq0 = qstart + qi * TILE;
    if (more) {
      load_tile<HD, GUARD>(Q, a.qs.t, qq0 + TILE, a.Tq, a.D, rq);
      load_tile<HD, GUARD>(G, a.gs.t, qq0 + TILE, a.Tq, a.D, rg);
      row_off(qq0 + TILE, lo_n, dof_n);
    }
    const bool skip = (a.causal && qq0 + TILE - 1 < k0) || k0 >= a.Tk;
    if (!skip) {
      float xa[S_::RUN];
      // S[q][key] - lse[q] (base 2): A = Q rows, B = K^T from registers
      lds_run<HD>(Qs[cur], l32, h, xa);
      floatx16 p = chain<HD>(lo, one, xa, kf);
      // dP[q][key] - D[q] = dO . V^T - D
      lds_run<HD>(Gs[cur], l32, h, xa);
      floatx16 dp = chain<HD>(dof, one, xa, vf);
      float ct[S_::NC][16];
      lds_cols<HD>(Gs[cur], l32, h, ct);
      const bool edge = (a.causal && qq0 < k0 + TILE - 1) || (GUARD && qq0 + TILE > a.Tq);
      if (edge) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int q = qq0 + kappa(j, h);
          const bool ok = (!GUARD || q < a.Tq) && (!a.causal || mykey <= q);
          p[j] = ok ? exp2_hw(p[j]) : 0.f;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) p[j] = exp2_hw(p[j]);
      }
#pragma unroll
      for (int s = 0; s < 16; ++s)  // dV^T += dO^T P
#pragma unroll
        for (int c = 0; c < S_::NC; ++c) dv[c] = mfma(ct[c][s], p[s], dv[c]);
      lds_cols<HD>(Qs[cur], l32, h, ct);
#pragma unroll
      for (int j = 0; j < 16; ++j) dp[j] *= p[j];  // dS
#pragma unroll
      for (int s = 0; s < 16; ++s)  // dK^T += Q^T dS
#pragma unroll
        for (int c = 0; c < S_::NC; ++c) dk[c] = mfma(ct[c][s], dp[s], dk[c]);
    }
    if (more) {
      store_tile<HD>(Qs[cur ^ 1], rq);
      store_tile<HD>(Gs[cur ^ 1], rg);
      lo = lo_n;
      dof = dof_n;
    }
    __syncthreads();
  }
  float* dkb = a.out + b * a.o1s.b + hh * a.o1s.h;
  float* dvb = a.out2 + b * a.o2s.b + hh * a.o2s.h;
  float* buf = (w < 2 ? Qs[w] : Gs[w - 2]);
  write_rows<HD>(buf, dk, a.scale, dkb, a.o1s.t, k0, a.Tk, a.D, l32, h, lane);
  __syncthreads();
  write_rows<HD>(buf, dv, 1.0f, dvb, a.o2s.t, k0, a.Tk, a.D, l32, h, lane);
}

// Query-block kernel: dQ for 128 queries per workgroup (32 per wave).
// GUARD: Tk is not a multiple of 32, or D < HD.
template <int HD, bool GUARD>
__global__ __launch_bounds__(256, occ_main<HD>()) void k_flash_dq(FlashArgs a) {
  using S_ = Hd<HD>;
  __shared__ __attribute__((aligned(16))) float Ks[2][TILE * S_::W];
  __shared__ __attribute__((aligned(16))) float Vs[2][TILE * S_::W];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const int64_t nbh = (int64_t)gridDim.x / a.nblk;
  const int g = balanced_rank(blockIdx.x, gridDim.x, a.cus);
  const int64_t bh = g % nbh;
  const int qb = a.nblk - 1 - (int)(g / nbh);
  const int64_t b = bh / a.H, hh = bh % a.H;
  const float* Q = a.q + b * a.qs.b + hh * a.qs.h;
  const float* K = a.k + b * a.ks.b + hh * a.ks.h;
  const float* V = a.v + b * a.vs.b + hh * a.vs.h;
  const float* G = a.dout + b * a.gs.b + hh * a.gs.h;
  const int q0 = qb * ROWS + w * TILE;
  const int myq = q0 + l32;

  float qf[S_::RUN], gf[S_::RUN];
  gl_run<HD, GUARD>(Q, a.qs.t, myq, a.Tq, a.D, h, a.scale * kLog2e, qf);
  gl_run<HD, GUARD>(G, a.gs.t, myq, a.Tq, a.D, h, 1.0f, gf);
  const bool qin = myq < a.Tq;
  const float lo = (h == 0 && qin) ? -a.lse[bh * a.Tq + myq] * kLog2e : 0.f;
  const float dof = (h == 0 && qin) ? -a.dsum[bh * a.Tq + myq] : 0.f;
  const float one = h == 0 ? 1.f : 0.f;
  floatx16 dq[S_::NC];
  zero_acc(dq);

  int kend = a.Tk;
  if (a.causal) kend = min(kend, qb * ROWS + ROWS);
  const int nkb = (kend + TILE - 1) / TILE;
  floatx4 rk[S_::NC], rv[S_::NC];
  load_tile<HD, GUARD>(K, a.ks.t, 0, a.Tk, a.D, rk);
  load_tile<HD, GUARD>(V, a.vs.t, 0, a.Tk, a.D, rv);
  store_tile<HD>(Ks[0], rk);
  store_tile<HD>(Vs[0], rv);
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const int cur = kb & 1;
    const bool more = kb + 1 < nkb;
    if (more) {
      load_tile<HD, GUARD>(K, a.ks.t, (kb + 1) * TILE, a.Tk, a.D, rk);
      load_tile<HD, GUARD>(V, a.vs.t, (kb + 1) * TILE, a.Tk, a.D, rv);
    }
    const int k0 = kb * TILE;
    const bool skip = (a.causal && k0 > q0 + TILE - 1) || q0 >= a.Tq;
    if (!skip) {
      float xa[S_::RUN];
      lds_run<HD>(Ks[cur], l32, h, xa);
      floatx16 p = chain<HD>(one, lo, xa, qf);    // S^T[key][q] - lse[q]
      lds_run<HD>(Vs[cur], l32, h, xa);
      floatx16 dp = chain<HD>(one, dof, xa, gf);  // dP^T[key][q] - D[q]
      float ct[S_::NC][16];
      lds_cols<HD>(Ks[cur], l32, h, ct);
      const bool edge = (a.causal && k0 + TILE - 1 > q0) || (GUARD && k0 + TILE > a.Tk);
      if (edge) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int key = k0 + kappa(j, h);
          const bool ok = (!GUARD || key < a.Tk) && (!a.causal || key <= myq);
          dp[j] = ok ? exp2_hw(p[j]) * dp[j] : 0.f;  // dS^T
        }
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) dp[j] *= exp2_hw(p[j]);
      }
#pragma unroll
      for (int s = 0; s < 16; ++s)  // dQ^T += K^T dS^T
#pragma unroll
        for (int c = 0; c < S_::NC; ++c) dq[c] = mfma(ct[c][s], dp[s], dq[c]);
    }
    if (more) {
      store_tile<HD>(Ks[cur ^ 1], rk);
      store_tile<HD>(Vs[cur ^ 1], rv);
    }
    __syncthreads();
  }
  float* dqb = a.out + b * a.o1s.b + hh * a.o1s.h;
  float* buf = (w < 2 ? Ks[w] : Vs[w - 2]);
  write_rows<HD>(buf, dq, a.scale, dqb, a.o1s.t, q0, a.Tq, a.D, l32, h, lane);
}

// Query-block kernel from stored dS: dQ^T = K^T dS^T for 128 queries per
// workgroup, reading the 32x32 dS blocks the key-block kernel wrote (each
// lane's 16 values are one contiguous run) instead of recomputing S and dP.
// 8 waves: two groups of four take the even and the odd key tiles of the
// 128 queries, so the longest (causal) query block runs half as many steps
// (measured faster than 4 waves over all tiles); the groups' dQ
// accumulators are added through LDS in a fixed order (even + odd), so the
// result is deterministic.  GUARD: Tk is not a multiple of 32, or D < HD.
template <int HD, bool GUARD>
__global__ __launch_bounds__(512, 1) void k_flash_dq_ds8(FlashArgs a) {
  using S_ = Hd<HD>;
  // group g stages its K tiles in Ks[2g], Ks[2g+1]; the combine and the
  // dQ row staging reuse all four
  __shared__ __attribute__((aligned(16))) float Ks[WAVES][TILE * S_::W];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int grp = wv >> 2, w = wv & 3, gt = threadIdx.x & 255;
  const int l32 = lane & 31, h = lane >> 5;
  const int64_t nbh = (int64_t)gridDim.x / a.nblk;
  const int g = balanced_rank(blockIdx.x, gridDim.x, a.cus);
  const int64_t bh = g % nbh;
  const int qb = a.nblk - 1 - (int)(g / nbh);
  const int64_t b = bh / a.H, hh = bh % a.H;
  const float* K = a.k + b * a.ks.b + hh * a.ks.h;
  const int q0 = qb * ROWS + w * TILE;
  const bool wave_in = q0 < a.Tq;
  const float* dsrow = a.dsblk +
                       ((int64_t)bh * a.nqt + (wave_in ? q0 / TILE : 0)) * a.nkt * (TILE * TILE) +
                       l32 * TILE + h * 16;
  floatx16 dq[S_::NC];
  zero_acc(dq);

  int kend = a.Tk;
  if (a.causal) kend = min(kend, qb * ROWS + ROWS);
  const int nkb = (kend + TILE - 1) / TILE;
  int nmine = wave_in ? nkb : 0;
  if (a.causal && wave_in) nmine = min(nkb, (q0 + TILE - 1) / TILE + 1);
  // this group's key tiles: kb = grp + 2t; both groups run nst0 steps (the
  // odd group's last one may be empty) so their barriers pair up
  const int nst0 = (nkb + 1) / 2;
  auto kb_of = [&](int t) { return grp + 2 * t; };
  // Every prefetch is issued, from a block clamped into this wave's range
  // when it would be past it (its values are then never used): loads on
  // conditional paths leave the compiler unable to count the loads in
  // flight, and its in-order vmcnt waits then wait for the newest
  // prefetch before the current tile's MFMAs.
  auto fetch_ds = [&](int t, floatx4 (&d)[4]) {
    int kb = kb_of(t);
    if (kb >= nmine) kb = nmine > 0 ? nmine - 1 : 0;
    const floatx4* src = reinterpret_cast<const floatx4*>(dsrow + (int64_t)kb * (TILE * TILE));
#pragma unroll
    for (int i = 0; i < 4; ++i) d[i] = src[i];
  };
  floatx4 d0[4], d1[4], d2[4];
  fetch_ds(0, d0);
  fetch_ds(1, d1);
  floatx4 rk[S_::NC];
  if (kb_of(0) < nkb) load_tile<HD, GUARD>(K, a.ks.t, kb_of(0) * TILE, a.Tk, a.D, rk, gt);
  if (kb_of(0) < nkb) store_tile<HD>(Ks[2 * grp], rk, gt);
  __syncthreads();
  auto step = [&](int t, const floatx4 (&use)[4], floatx4 (&into)[4]) {
    const int cur = 2 * grp + (t & 1);
    const int kb = kb_of(t);
    const bool more = kb + 2 < nkb;
    load_tile<HD, GUARD>(K, a.ks.t, (more ? kb + 2 : nkb - 1) * TILE, a.Tk, a.D, rk, gt);
    fetch_ds(t + 2, into);
    if (kb < nmine) {
      float ct[S_::NC][16];
      lds_cols<HD>(Ks[cur], l32, h, ct);
#pragma unroll
      for (int s = 0; s < 16; ++s) {  // dQ^T += K^T dS^T
        const float d = use[s >> 2][s & 3];
#pragma unroll
        for (int c = 0; c < S_::NC; ++c) dq[c] = mfma(ct[c][s], d, dq[c]);
      }
    }
    if (more) store_tile<HD>(Ks[2 * grp + ((t + 1) & 1)], rk, gt);
    __syncthreads();
  };
  for (int t = 0; t < nst0; t += 3) {
    step(t, d0, d2);
    if (t + 1 >= nst0) break;
    step(t + 1, d1, d0);
    if (t + 2 >= nst0) break;
    step(t + 2, d2, d1);
  }
  // dQ = even-group sum + odd-group sum (wave w's NC x 16 x 64 floats fit
  // in its own 32 x W tile)
  float* red = &Ks[0][0] + w * (S_::NC * 16 * 64);
  if (grp == 1) {
#pragma unroll
    for (int c = 0; c < S_::NC; ++c)
#pragma unroll
      for (int j = 0; j < 16; ++j) red[(c * 16 + j) * 64 + lane] = dq[c][j];
  }
  __syncthreads();
  if (grp == 0) {
#pragma unroll
    for (int c = 0; c < S_::NC; ++c)
#pragma unroll
      for (int j = 0; j < 16; ++j) dq[c][j] = dq[c][j] + red[(c * 16 + j) * 64 + lane];
  }
  __syncthreads();
  float* dqb = a.out + b * a.o1s.b + hh * a.o1s.h;
  if (grp == 0)
    write_rows<HD>(Ks[w], dq, a.scale, dqb, a.o1s.t, q0, a.Tq, a.D, l32, h, lane);
  else
    __syncthreads();  // the one barrier inside write_rows
}

// Key-block kernel with the work of each 32-key group split over a pair of
// waves: wave A holds the group's K rows and forms P = exp2(S - lse) (S =
// Q K^T), hands P over through LDS and accumulates dV^T += dO^T P; wave B
// holds the V rows, forms dP - D = dO V^T - D, then dS = P * (dP - D),
// stores the dS block and accumulates dK^T += Q^T dS.  A workgroup of four
// waves covers 64 keys (two pairs).  Each wave holds half the registers of
// a wave that does all four products, so three workgroups fit on a CU at
// HD 64 (three waves per SIMD).  Each query tile takes two barriers: P is
// written before the middle one and read after it.  B stores its dS block
// at the end of the step, after the wait for the next tile's prefetch, so
// that wait never waits for the stores.  GUARD: Tq or Tk is not a multiple
// of 32, or D < HD.
constexpr int PROWS = 64;  // keys per workgroup
template <int HD, bool GUARD, bool STORE>
__global__ __launch_bounds__(256, occ_pair<HD>()) void k_flash_dkv_pair(FlashArgs a) {
  using S_ = Hd<HD>;
  __shared__ __attribute__((aligned(16))) float Qs[2][TILE * S_::W];
  __shared__ __attribute__((aligned(16))) float Gs[2][TILE * S_::W];
  __shared__ __attribute__((aligned(16))) float Ps[2][16 * 64];
  // the workgroups of a CU run at different wave priorities, so they do
  // not fall into step (identical workgroups sharing the matrix pipe
  // fairly finish their MFMA phases together and then leave it idle
  // together): measured 5% faster than equal priorities
  if (blockIdx.x % 3 == 0) __builtin_amdgcn_s_setprio(2);
  else if (blockIdx.x % 3 == 1) __builtin_amdgcn_s_setprio(1);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int role = wv >> 1, pr = wv & 1;  // role 0: A (P, dV), 1: B (dS, dK)
  const int l32 = lane & 31, h = lane >> 5;
  const int64_t nbh = (int64_t)gridDim.x / a.nblk;
  const int g = balanced_rank(blockIdx.x, gridDim.x, a.cus);
  const int64_t bh = g % nbh;
  const int kblk = (int)(g / nbh);  // long (causal) blocks rank first
  const int64_t b = bh / a.H, hh = bh % a.H;
  const float* Q = a.q + b * a.qs.b + hh * a.qs.h;
  const float* K = a.k + b * a.ks.b + hh * a.ks.h;
  const float* V = a.v + b * a.vs.b + hh * a.vs.h;
  const float* G = a.dout + b * a.gs.b + hh * a.gs.h;
  const float* L = role == 0 ? a.lse + bh * a.Tq : a.dsum + bh * a.Tq;
  const int k0 = kblk * PROWS + pr * TILE;  // the pair's first key
  const int mykey = k0 + l32;

  // A: K rows (scaled to base-2 logits); B: V rows
  float kv[S_::RUN];
  if (role == 0)
    gl_run<HD, GUARD>(K, a.ks.t, mykey, a.Tk, a.D, h, a.scale * kLog2e, kv);
  else
    gl_run<HD, GUARD>(V, a.vs.t, mykey, a.Tk, a.D, h, 1.0f, kv);
  // complete the loads here: a wait for them inside the loop would also
  // wait for every step's prefetch
#pragma unroll
  for (int i = 0; i < S_::RUN; ++i) asm volatile("" : "+v"(kv[i]));
  floatx16 acc[S_::NC];  // A: dV^T, B: dK^T
  zero_acc(acc);
  const float one = h == 0 ? 1.f : 0.f;
  // row offset of a query tile: A -lse*log2e, B -D (loaded by every lane,
  // the index clamped into range, with the tile; formed after the step)
  const float omul = role == 0 ? -kLog2e : -1.f;
  auto row_raw = [&](int qq0) { return L[min(qq0 + l32, a.Tq - 1)]; };
  auto row_fix = [&](int qq0, float raw) {
    const bool in = !GUARD || qq0 + l32 < a.Tq;
    return (h == 0 && in) ? raw * omul : 0.f;
  };

  const int qstart = a.causal ? kblk * PROWS : 0;
  const int nqb = qstart < a.Tq ? (a.Tq - qstart + TILE - 1) / TILE : 0;
  floatx4 rq[S_::NC], rg[S_::NC];
  float off = 0.f, raw_n = 0.f;
  if (nqb > 0) {
    load_tile<HD, GUARD>(Q, a.qs.t, qstart, a.Tq, a.D, rq);
    load_tile<HD, GUARD>(G, a.gs.t, qstart, a.Tq, a.D, rg);
    raw_n = row_raw(qstart);
    store_tile<HD>(Qs[0], rq);
    store_tile<HD>(Gs[0], rg);
    off = row_fix(qstart, raw_n);
  }
  __syncthreads();
  float* pbuf = Ps[pr];
  for (int qi = 0; qi < nqb; ++qi) {
    const int cur = qi & 1;
    const bool more = qi + 1 < nqb;
    const int qq0 = qstart + qi * TILE;
    if (more) {
      load_tile<HD, GUARD>(Q, a.qs.t, qq0 + TILE, a.Tq, a.D, rq);
      load_tile<HD, GUARD>(G, a.gs.t, qq0 + TILE, a.Tq, a.D, rg);
      raw_n = row_raw(qq0 + TILE);
    }
    const bool skip = (a.causal && qq0 + TILE - 1 < k0) || k0 >= a.Tk;
    const bool edge = (a.causal && qq0 < k0 + TILE - 1) || (GUARD && qq0 + TILE > a.Tq);
    floatx16 x = zero16();  // A: P; B: dP - D, then dS
    if (!skip) {
      float xa[S_::RUN];
      // A: S[q][key] - lse[q] from Q rows; B: dP[q][key] - D[q] from dO rows
      lds_run<HD>(role == 0 ? Qs[cur] : Gs[cur], l32, h, xa);
      x = chain<HD>(off, one, xa, kv);
      if (role == 0) {
        if (edge) {
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int q = qq0 + kappa(j, h);
            const bool ok = (!GUARD || q < a.Tq) && (!a.causal || mykey <= q);
            x[j] = ok ? exp2_hw(x[j]) : 0.f;
          }
        } else {
#pragma unroll
          for (int j = 0; j < 16; ++j) x[j] = exp2_hw(x[j]);
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) pbuf[j * 64 + lane] = x[j];
      }
    }
    __syncthreads();
    if (!skip) {
      float ct[S_::NC][16];
      if (role == 0) {
        lds_cols<HD>(Gs[cur], l32, h, ct);
#pragma unroll
        for (int s = 0; s < 16; ++s)  // dV^T += dO^T P
#pragma unroll
          for (int c = 0; c < S_::NC; ++c) acc[c] = mfma(ct[c][s], x[s], acc[c]);
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) x[j] *= pbuf[j * 64 + lane];  // dS (0 where masked)
        lds_cols<HD>(Qs[cur], l32, h, ct);
#pragma unroll
        for (int s = 0; s < 16; ++s)  // dK^T += Q^T dS
#pragma unroll
          for (int c = 0; c < S_::NC; ++c) acc[c] = mfma(ct[c][s], x[s], acc[c]);
      }
    }
    if (more) {
      store_tile<HD>(Qs[cur ^ 1], rq);
      store_tile<HD>(Gs[cur ^ 1], rg);
      off = row_fix(qq0 + TILE, raw_n);
    }
    if (STORE && role == 1) {
      // this lane's key column of the (query tile, key tile) dS block, on
      // every step (masked blocks hold zeros; a pair past the last key
      // writes the spare block).  Non-temporal: read once, by the
      // query-block kernel
      const int64_t blk_id = k0 < a.Tk ? ((int64_t)bh * a.nqt + qq0 / TILE) * a.nkt + k0 / TILE
                                       : a.spare_blk;
      float* blk = a.dsblk + blk_id * (TILE * TILE) + ds_col(l32);
#pragma unroll
      for (int j = 0; j < 16; ++j) __builtin_nontemporal_store(x[j], blk + kappa(j, h) * TILE);
    }
    __syncthreads();
  }
  float* buf = (wv < 2 ? Qs[wv] : Gs[wv - 2]);
  if (role == 0) {
    float* dvb = a.out2 + b * a.o2s.b + hh * a.o2s.h;
    write_rows<HD>(buf, acc, 1.0f, dvb, a.o2s.t, k0, a.Tk, a.D, l32, h, lane);
  } else {
    float* dkb = a.out + b * a.o1s.b + hh * a.o1s.h;
    write_rows<HD>(buf, acc, a.scale, dkb, a.o1s.t, k0, a.Tk, a.D, l32, h, lane);
  }
}

bool rows_ok(const int64_t* s, const void* p) {
  // D contiguous, 16-byte aligned rows
  return ((uintptr_t)p & 15) == 0 && (s[0] % 4) == 0 && (s[1] % 4) == 0 && (s[2] % 4) == 0;
}

Strides3 s3(const int64_t* s) { return Strides3{s[0], s[1], s[2]}; }

int cus_per_xcd() {
  const int c = num_cus() / kXcds;
  return c > 0 ? c : 1;
}

int padded_hd(int64_t D) { return (int)((D + 31) / 32 * 32); }

template <int HD>
void launch_forward(const FlashArgs& a, unsigned grid) {
  if ((a.Tk % TILE) || a.D != HD)
    tjh_launch(k_flash_fwd<HD, true>, dim3(grid), dim3(256), 0, stream(), a);
  else
    tjh_launch(k_flash_fwd<HD, false>, dim3(grid), dim3(256), 0, stream(), a);
}

// The key kernel (dK, dV) then the query kernel (dQ) of the backward; a.out
// / a.o1s and a.nblk are set here for each.
template <int HD>
int launch_backward(FlashArgs a, int64_t BH, const int64_t* dq_st, float* dq) {
  const bool ragged = (a.Tq % TILE) || (a.Tk % TILE) || a.D != HD;
  if (a.dsblk) {
    a.nblk = (int)cdiv(a.Tk, PROWS);
    const unsigned gk = (unsigned)(BH * a.nblk);
    if (ragged)
      tjh_launch(k_flash_dkv_pair<HD, true, true>, dim3(gk), dim3(256), 0, stream(), a);
    else
      tjh_launch(k_flash_dkv_pair<HD, false, true>, dim3(gk), dim3(256), 0, stream(), a);
  } else {
    a.nblk = (int)cdiv(a.Tk, ROWS);
    const unsigned gk = (unsigned)(BH * a.nblk);
    if (ragged)
      tjh_launch(k_flash_dkv<HD, true>, dim3(gk), dim3(256), 0, stream(), a);
    else
      tjh_launch(k_flash_dkv<HD, false>, dim3(gk), dim3(256), 0, stream(), a);
  }
  const int rc = check_launch("flash_dkv");
  if (rc != TJH_OK) return rc;
  // queries: dQ from the stored dS blocks, or recomputed when the blocks
  // could not be allocated
  a.nblk = (int)cdiv(a.Tq, ROWS);
  a.out = dq; a.out2 = nullptr; a.o1s = s3(dq_st);
  const unsigned gq = (unsigned)(BH * a.nblk);
  const bool kguard = (a.Tk % TILE) || a.D != HD;
  if (a.dsblk) {
    if (kguard)
      tjh_launch(k_flash_dq_ds8<HD, true>, dim3(gq), dim3(512), 0, stream(), a);
    else
      tjh_launch(k_flash_dq_ds8<HD, false>, dim3(gq), dim3(512), 0, stream(), a);
  } else if (kguard) {
    tjh_launch(k_flash_dq<HD, true>, dim3(gq), dim3(256), 0, stream(), a);
  } else {
    tjh_launch(k_flash_dq<HD, false>, dim3(gq), dim3(256), 0, stream(), a);
  }
  return check_launch("flash_dq");
}

}  // namespace

bool flash_supported(int64_t D, const void* const* ptrs, const int64_t* const* strides, int n) {
  if (D <= 0 || D > HD_MAX || D % 4) return false;
  for (int i = 0; i < n; ++i)
    if (!rows_ok(strides[i], ptrs[i])) return false;
  return true;
}

int flash_forward(const float* q, const float* k, const float* v, float* o, float* lse, int64_t B,
                  int64_t H, int64_t Tq, int64_t Tk, int64_t D, const int64_t* qs,
                  const int64_t* ks, const int64_t* vs, const int64_t* os, float scale,
                  int causal) {
  TJH_ARG(Tq < (int64_t(1) << 30) && Tk < (int64_t(1) << 30), "sdpa: sequence too long");
  TJH_ARG(D > 0 && D <= HD_MAX && D % 4 == 0, "sdpa: flash head dim %lld", (long long)D);
  FlashArgs a{};
  a.q = q; a.k = k; a.v = v; a.out = o; a.lse_out = lse;
  a.qs = s3(qs); a.ks = s3(ks); a.vs = s3(vs); a.os = s3(os);
  a.H = H; a.Tq = (int)Tq; a.Tk = (int)Tk; a.D = (int)D; a.scale = scale; a.causal = causal;
  a.nblk = (int)cdiv(Tq, ROWS);
  a.cus = cus_per_xcd();
  const int64_t grid = B * H * a.nblk;
  TJH_ARG(grid < (int64_t(1) << 31), "sdpa: grid too large");
  KernelScope ks_("sdpa_fwd");
  switch (padded_hd(D)) {
    case 32: launch_forward<32>(a, (unsigned)grid); break;
    case 64: launch_forward<64>(a, (unsigned)grid); break;
    case 96: launch_forward<96>(a, (unsigned)grid); break;
    default: launch_forward<128>(a, (unsigned)grid); break;
  }
  return check_launch("flash_forward");
}

int flash_backward(const float* q, const float* k, const float* v, const float* o,
                   const float* dout, const float* lse, float* dq, float* dk, float* dv,
                   int64_t B, int64_t H, int64_t Tq, int64_t Tk, int64_t D,
                   const int64_t* const* st, float scale, int causal) {
  TJH_ARG(Tq < (int64_t(1) << 30) && Tk < (int64_t(1) << 30), "sdpa: sequence too long");
  TJH_ARG(D > 0 && D <= HD_MAX && D % 4 == 0, "sdpa: flash head dim %lld", (long long)D);
  FlashArgs a{};
  a.q = q; a.k = k; a.v = v; a.o = o; a.dout = dout; a.lse = lse;
  a.qs = s3(st[0]); a.ks = s3(st[1]); a.vs = s3(st[2]); a.os = s3(st[3]); a.gs = s3(st[4]);
  a.H = H; a.Tq = (int)Tq; a.Tk = (int)Tk; a.D = (int)D; a.scale = scale; a.causal = causal;
  a.cus = cus_per_xcd();
  Scratch ds((size_t)(B * H * Tq) * sizeof(float));
  if (!ds.ok()) return set_error(TJH_ERR_OOM, "sdpa_backward: no scratch");
  a.dsum = ds.as<float>();
  KernelScope ks_("sdpa_bwd");
  const int64_t rows = B * H * Tq;
  const bool v4 = aligned16(dout) && aligned16(o) && a.gs.b % 4 == 0 && a.gs.h % 4 == 0 &&
                  a.gs.t % 4 == 0 && a.os.b % 4 == 0 && a.os.h % 4 == 0 && a.os.t % 4 == 0;
  const int HDp = padded_hd(D);
  const unsigned g4 = (unsigned)cdiv(rows, 64);
  if (v4 && HDp <= 64)
    tjh_launch(k_flash_dsum4<64>, dim3(g4), dim3(256), 0, stream(), a, ds.as<float>(), rows);
  else if (v4)
    tjh_launch(k_flash_dsum4<128>, dim3(g4), dim3(256), 0, stream(), a, ds.as<float>(), rows);
  else
    tjh_launch(k_flash_dsum, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, stream(), a,
               ds.as<float>(), rows);
  int rc = check_launch("flash_dsum");
  if (rc != TJH_OK) return rc;
  // dS blocks for the query-block kernel (about 403 MB for 96 heads of
  // T = 1024; released once the query kernel is queued)
  a.nqt = (int)cdiv(Tq, TILE);
  a.nkt = (int)cdiv(Tk, TILE);
  // TJH_SDPA_RECOMPUTE=1 (read on every call) forces the recomputing path
  const char* rec = getenv("TJH_SDPA_RECOMPUTE");
  const bool want_blocks = !(rec && rec[0] == '1');
  a.spare_blk = (int64_t)(B * H) * a.nqt * a.nkt;
  Scratch dsb(want_blocks ? (size_t)(a.spare_blk + 1) * (TILE * TILE) * sizeof(float) : 0);
  a.dsblk = dsb.ok() ? dsb.as<float>() : nullptr;
  // keys: dK, dV (the paired-wave kernel, which also stores the dS blocks;
  // without blocks, the four-product kernel)
  a.out = dk; a.out2 = dv; a.o1s = s3(st[6]); a.o2s = s3(st[7]);
  switch (HDp) {
    case 32: return launch_backward<32>(a, B * H, st[5], dq);
    case 64: return launch_backward<64>(a, B * H, st[5], dq);
    case 96: return launch_backward<96>(a, B * H, st[5], dq);
    default: return launch_backward<128>(a, B * H, st[5], dq);
  }
}

}  // namespace tjh
