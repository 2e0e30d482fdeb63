// fp32 GEMM on the CDNA4 matrix cores (v_mfma_f32_32x32x2_f32).
//
// Replaces matmul.wgsl:17-50 (a 16x16 scalar tile kernel) behind torch.js's
// Tensor.matmul / mm / bmm and nn.Linear (Tensor.ts:2132-2331,
// src/nn/linear.ts:43-66), and supplies the dgrad / wgrad products the
// reference's autograd never issues (Tensor.ts:2212-2221).
//
// C[b] = alpha * op(A[b]) op(B[b]) + beta * C[b] (+ bias), row-major.
//
// Tiling (one workgroup = 4 wave64 arranged 2 x 2, or 8 arranged 4 x 2 for
// 256-row tiles):
//   block tile BM x BN in {256x128, 128x128, 128x64, 64x64, 256x256}, K
//   step 16; each wave owns a (BM/2 or 64) x (BN/2) sub-tile of 32x32 MFMA
//   blocks; the 8-wave 256x128 tile shares each B tile among four row waves
//   (a quarter fewer global loads and LDS stores per FLOP than 128x128);
//   the 8-wave 256x256 tile (64x128 per wave, two waves per SIMD) serves
//   only A . B with a very long K, where it halves the re-reads of A.  Tiles
//   are double-buffered in LDS: the next K tile is fetched from HBM into
//   registers while the MFMAs consume the current LDS tile.  A stored
//   [M][K] (k contiguous) is staged As[m][k] and read as 128-bit fragments
//   under a K-step permutation (below); every other operand is staged
//   k-major (As[k][m], Bs[k][n]) with a 4-float pad.
// The tile is chosen per call from M, N and the CU count so that the
// number of workgroups divides evenly over the 256 CUs (an 8192 x 768
// product has 384 tiles of 128x128 — 1.5 per CU — but 768 of 128x64).
// Small M x N with long K (weight gradients: K = tokens) is split over K;
// partials are summed by a second pass in a fixed order (deterministic).
// MFMA operand layout (32x32x2 f32): lane l feeds A[m = l%32][k = l/32] and
//   B[k = l/32][n = l%32]; accumulator register r of lane l holds
//   C[8*(r/4) + 4*(l/32) + r%4][l%32].
// Operand loads are 128-bit at any 4-byte alignment (HSA runs the GPU in
// unaligned-access mode; the compiler itself emits such loads for packed
// data), so an odd row stride — the 50257-wide logits — still loads a
// float4 per access; only runs that cross the problem's edge go
// element-wise.
// Workgroup order: tiles are grouped 8 M-tiles at a time so neighbouring
// tiles share B columns, and each XCD receives a contiguous run of that
// order so the sharing happens inside one L2.

#include "colsum.h"
#include "common.h"
#include "ops_math.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

namespace tjh {
namespace {

constexpr int BK = 16;

typedef float floatx16 __attribute__((ext_vector_type(16)));
// Staging registers are native 4-wide vectors: a struct float4 copied out
// of a reinterpret_cast load is not always split into registers by the
// compiler and then lives in scratch memory.
typedef float floatx4 __attribute__((ext_vector_type(4)));
// The same vector at 4-byte alignment: operand rows start wherever the row
// stride puts them.
typedef float floatx4u __attribute__((ext_vector_type(4), aligned(4)));

struct GemmArgs {
  const float* A;
  const float* B;
  float* C;
  const float* bias;
  int64_t M, N, K;
  int64_t lda, ldb, ldc;
  int64_t sA, sB, sC;
  float alpha, beta;
  int bias_mode;
  int vecA, vecB;  // 128-bit loads allowed for the operand
  int tiles_m, tiles_n;
  int64_t kchunk;  // K range per split (multiple of BK); splits = gridDim.y
  float* ws;       // split-K partials [batch][split][M][N] (nullptr: none)
  float* rsw;      // split-K partials of the row sums (bias_mode 3/4) [split][M]
  // epilogue activation on the final C values (after alpha, beta, bias):
  // 1: aux <- v, C <- GELU(v);  2: C <- v * GELU'(aux);  3: C <- aux + v
  float* aux;
  int64_t ldaux;
  int act;
  // A formed on load from logits (k_gemm<..., XF>): A's element at logits
  // row r, class c is (exp(logits[r][c] - lse_r) - (c == t_r)) * s_r, the
  // cross-entropy gradient, with xrow[r] = {lse_r, s_r, t_r (int bits), 0};
  // xm0 / xk0 locate this (sub-)product in the logits (rows = m without
  // TA, k with TA)
  const floatx4* xrow;
  int64_t xm0, xk0;
};

// A compile-time int carried by a value (dispatch into generic lambdas).
template <int V>
struct IConst {
  static constexpr int value = V;
};

// The activation epilogue, shared by the GEMM and the split-K sum.
__device__ __forceinline__ float epilogue_act(const GemmArgs& g, int64_t row, int64_t col,
                                              float v) {
  if (g.act == 1) {
    g.aux[row * g.ldaux + col] = v;
    return gelu_f(v);
  }
  if (g.act == 2) return v * gelu_grad(g.aux[row * g.ldaux + col]);
  if (g.act == 3) return g.aux[row * g.ldaux + col] + v;
  return v;
}

// Loads a logical OUTER x BK tile (outer = m for A, n for B) for this lane:
// V float4 per lane.  !TRANS: storage [outer][k] (k contiguous, 4 float4
// per outer row); TRANS: storage [k][outer] (outer contiguous).
// EDGE == false: the caller guarantees the tile is in bounds, so every load
// is an unconditional 128-bit load.  EDGE == true: every 4-run is
// bounds-checked (tiles on the problem's edge); `vec` (the operand is
// 4-byte aligned) lets runs that are wholly in bounds load as one 128-bit
// access.
template <bool TRANS, int OUTER, int V, bool EDGE, int T>
__device__ __forceinline__ void load_tile(const float* __restrict__ P, int64_t ld, int64_t rows,
                                          int64_t cols, int64_t r0, int64_t c0, bool vec,
                                          floatx4 (&reg)[V]) {
  const int t = threadIdx.x;
  constexpr int NF = OUTER * BK / 4;  // float4s in the tile (the last pass may be partial)
#pragma unroll
  for (int i = 0; i < V; ++i) {
    int f = t + T * i;
    if (NF % T != 0 && f >= NF) {
      reg[i] = floatx4{0.f, 0.f, 0.f, 0.f};
      continue;
    }
    if (!EDGE) {
      if (!TRANS) {
        int o = f >> 2, kq = f & 3;
        reg[i] = *reinterpret_cast<const floatx4u*>(P + (r0 + o) * ld + c0 + kq * 4);
      } else {
        constexpr int Q = OUTER / 4;
        int k = f / Q, oq = f % Q;
        reg[i] = *reinterpret_cast<const floatx4u*>(P + (c0 + k) * ld + r0 + oq * 4);
      }
    } else {
      // guarded: a 4-run wholly in bounds of an aligned operand is still
      // one 128-bit load; only runs that cross an edge go element-wise
      float v[4];
      if (!TRANS) {
        int o = f >> 2, kq = f & 3;
        int64_t go = r0 + o, gk = c0 + kq * 4;
        if (vec && go < rows && gk + 3 < cols) {
          reg[i] = *reinterpret_cast<const floatx4u*>(P + go * ld + gk);
          continue;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
          v[j] = (go < rows && gk + j < cols) ? P[go * ld + gk + j] : 0.f;
      } else {
        constexpr int Q = OUTER / 4;
        int k = f / Q, oq = f % Q;
        int64_t gk = c0 + k, go = r0 + oq * 4;
        if (vec && gk < cols && go + 3 < rows) {
          reg[i] = *reinterpret_cast<const floatx4u*>(P + gk * ld + go);
          continue;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
          v[j] = (gk < cols && go + j < rows) ? P[gk * ld + go + j] : 0.f;
      }
      reg[i] = floatx4{v[0], v[1], v[2], v[3]};
    }
  }
}

// Stores a loaded tile into LDS.  TRANS (outer contiguous in memory):
// S[k][outer], row length W, one 128-bit store per float4.  !TRANS (k
// contiguous): KC ? S[outer][k] with row length KS, one 128-bit store per
// float4 : S[k][outer] (transposed, four 32-bit stores per float4).
constexpr int KS = BK + 4;  // [outer][k] row length: 16-lane groups of 128-bit reads are conflict free
template <bool TRANS, bool KC, int OUTER, int V, int W, int T>
__device__ __forceinline__ void store_tile(float* __restrict__ S, const floatx4 (&reg)[V]) {
  const int t = threadIdx.x;
  constexpr int NF = OUTER * BK / 4;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    int f = t + T * i;
    if (NF % T != 0 && f >= NF) continue;
    if (!TRANS && KC) {
      int o = f >> 2, kq = f & 3;
      *reinterpret_cast<floatx4*>(S + o * KS + kq * 4) = reg[i];
    } else if (!TRANS) {
      int o = f >> 2, kq = f & 3;
      S[(kq * 4 + 0) * W + o] = reg[i].x;
      S[(kq * 4 + 1) * W + o] = reg[i].y;
      S[(kq * 4 + 2) * W + o] = reg[i].z;
      S[(kq * 4 + 3) * W + o] = reg[i].w;
    } else {
      constexpr int Q = OUTER / 4;
      int k = f / Q, oq = f % Q;
      *reinterpret_cast<floatx4*>(S + k * W + oq * 4) = reg[i];
    }
  }
}

// The logits row (and class offset) of float4 i of this lane's A tile
// load, and whether that row lies inside the product.
template <bool TRANS, int OUTER, bool EDGE, int T>
__device__ __forceinline__ bool ce_row(const GemmArgs& g, int64_t rows, int64_t cols, int64_t r0,
                                       int64_t c0, int i, int64_t& lr, int64_t& rel) {
  const int f = threadIdx.x + T * i;
  if (!TRANS) {
    const int64_t go = r0 + (f >> 2), gk = c0 + (f & 3) * 4;
    lr = g.xm0 + go;
    rel = g.xk0 + gk;
    return !EDGE || go < rows;
  }
  constexpr int Q = OUTER / 4;
  const int64_t gk = c0 + f / Q, go = r0 + (f % Q) * 4;
  lr = g.xk0 + gk;
  rel = g.xm0 + go;
  return !EDGE || gk < cols;
}

// The per-row records the A tile's float4s need (lse, scale, target),
// issued with the tile's own loads.  Without TA a lane's rows are the same
// for every K tile, so they are fetched once.
template <bool TRANS, int OUTER, int V, bool EDGE, int T>
__device__ __forceinline__ void ce_fetch(const GemmArgs& g, int64_t rows, int64_t cols,
                                         int64_t r0, int64_t c0, float (&cl)[V], float (&cs)[V],
                                         int (&ct)[V]) {
#pragma unroll
  for (int i = 0; i < V; ++i) {
    int64_t lr, rel;
    if (ce_row<TRANS, OUTER, EDGE, T>(g, rows, cols, r0, c0, i, lr, rel)) {
      const floatx4 v = g.xrow[lr];
      cl[i] = v.x;
      cs[i] = v.y;
      ct[i] = __float_as_int(v.z);
    } else {
      cl[i] = cs[i] = 0.f;
      ct[i] = -1;
    }
  }
}

// Turns a loaded A tile of logits into the cross-entropy gradient, element
// for element the expression of the cross-entropy backward kernel, so the
// product equals the one over the stored gradient bit for bit.  Elements
// outside the product stay zero.
template <bool TRANS, int OUTER, int V, bool EDGE, int T>
__device__ __forceinline__ void ce_apply(const GemmArgs& g, int64_t rows, int64_t cols,
                                         int64_t r0, int64_t c0, const float (&cl)[V],
                                         const float (&cs)[V], const int (&ct)[V],
                                         floatx4 (&reg)[V]) {
#pragma unroll
  for (int i = 0; i < V; ++i) {
    int64_t lr, rel;
    if (!ce_row<TRANS, OUTER, EDGE, T>(g, rows, cols, r0, c0, i, lr, rel)) continue;
    const int tc = ct[i] - (int)rel;  // classes are int32
    const int f = threadIdx.x + T * i;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bool in = true;
      if (EDGE) {
        if (!TRANS) in = c0 + (f & 3) * 4 + j < cols;
        else in = r0 + (f % (OUTER / 4)) * 4 + j < rows;
      }
      reg[i][j] = in ? (__expf(reg[i][j] - cl[i]) - (tc == j ? 1.f : 0.f)) * cs[i] : 0.f;
    }
  }
}

// xrow[r] = {lse[r], scale[r], targets[r] (int bits), 0} for k_gemm<..., XF>.
__global__ __launch_bounds__(256) void k_ce_rows(const float* __restrict__ lse,
                                                 const int32_t* __restrict__ t,
                                                 const float* __restrict__ sc, int64_t rows,
                                                 floatx4* __restrict__ xrow) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r < rows) xrow[r] = floatx4{lse[r], sc[r], __int_as_float(t[r]), 0.f};
}

// Reads this lane's MFMA operand values for K steps 4q .. 4q+3 of a tile: F
// blocks of 32 outer indices, 4 k values each.  K-step permutation: at MFMA
// step j the lanes of half h (lane / 32) feed k = 8h + j, so a lane's k
// values are contiguous in an [outer][k] tile (one 128-bit read per block).
template <bool KC, int F, int W>
__device__ __forceinline__ void read_frags(const float* __restrict__ S, int outer0, int l32, int h,
                                           int q, floatx4 (&fr)[F]) {
#pragma unroll
  for (int i = 0; i < F; ++i) {
    const int o = outer0 + i * 32 + l32;
    if (KC) {
      fr[i] = *reinterpret_cast<const floatx4*>(S + o * KS + 8 * h + 4 * q);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) fr[i][j] = S[(8 * h + 4 * q + j) * W + o];
    }
  }
}

// Workgroups are dispatched to the 8 XCDs round-robin (workgroup w runs on
// XCD w % 8), and each XCD has its own L2.  Renumbering so that XCD x
// receives the contiguous run [x*n/8, (x+1)*n/8) of the grouped tile order
// keeps the tiles that share A rows and B columns on one L2.  A bijection on
// [0, n): ids past the last multiple of 8 keep their number.
// Waves per workgroup: WR rows x 2 columns, each wave keeping a
// (BM / WR) x (BN / 2) sub-tile: 2 x 2 waves, or 4 x 2 for the 8-wave
// 256-row tiles (B shared by four waves).
constexpr int gemm_threads(int wr) { return wr * 128; }
// Wave tiles of 64 x 96 or more run two waves per SIMD (their
// accumulators alone take 96 registers or more), smaller ones four.
constexpr int gemm_waves_per_simd(int bm, int bn, int wr) {
  return (bm / wr) * (bn / 2) >= 64 * 96 ? 2 : 4;
}

constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_tile(int bid, int n) {
  const int full = n - n % kXcds;
  if (bid >= full) return bid;
  return (bid % kXcds) * (full / kXcds) + bid / kXcds;
}

template <int BM, int BN, int WR, bool TA, bool TB, bool EDGE, bool XF = false>
__global__ __launch_bounds__(gemm_threads(WR), gemm_waves_per_simd(BM, BN, WR)) void k_gemm(
    GemmArgs g) {
  constexpr int LA = BM + 4, LB = BN + 4;       // LDS row lengths
  constexpr int WM = BM / WR, WN = BN / 2;      // wave tile: WR x 2 waves
  constexpr int FM = WM / 32, FN = WN / 32;     // MFMA blocks per wave
  constexpr int T = gemm_threads(WR);
  constexpr int VA = (BM * BK / 4 + T - 1) / T;  // float4 loads per lane (last pass may be partial)
  constexpr int VB = (BN * BK / 4 + T - 1) / T;
  static_assert(FM >= 1 && FN >= 1 && VA >= 1 && VB >= 1, "tile too small");
  // A with k contiguous is staged [m][k] (128-bit stores and reads).  B
  // stays k-major: staging a k-contiguous B as [n][k] measured slower on
  // the forward products (A . B^T) of GPT-2's shapes (on the 4-wave
  // 256 x 128 tile too: 470 against 378 us for 8192 x 3072 x 768).
  constexpr bool AKC = !TA, BKC = false;
  constexpr int SA = AKC ? BM * KS : BK * LA, SB = BKC ? BN * KS : BK * LB;
  __shared__ __attribute__((aligned(16))) float As[2][SA];
  __shared__ __attribute__((aligned(16))) float Bs[2][SB];

  // Wave priority: the prologue and the epilogue run at raised priority.
  // Two workgroups share a CU, and at equal priority the one in its
  // epilogue (address arithmetic and stores) barely advances while the
  // other issues MFMAs: its stores drained only when the other's main loop
  // ended, ~40 us per launch for GPT-2's 8192 x 3072 products, and its
  // successor could not start.
  __builtin_amdgcn_s_setprio(3);
  // ---- tile coordinates (grouped ordering for L2 reuse)
  const int tiles_m = g.tiles_m, tiles_n = g.tiles_n;
  int bid = xcd_tile(blockIdx.x, gridDim.x);
  constexpr int GROUP = 8;
  int group_size = GROUP * tiles_n;
  int group = bid / group_size;
  int first_m = group * GROUP;
  int gm = tiles_m - first_m < GROUP ? tiles_m - first_m : GROUP;
  int in_group = bid % group_size;
  int tm = first_m + in_group % gm;
  int tn = in_group / gm;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

  const int64_t b = blockIdx.z;
  const float* __restrict__ A = g.A + b * g.sA;
  const float* __restrict__ B = g.B + b * g.sB;
  float* __restrict__ C = g.C + b * g.sC;
  // split-K: this workgroup covers K range [kbeg, kend)
  const int64_t kbeg = (int64_t)blockIdx.y * g.kchunk;
  const int64_t kend = kbeg + g.kchunk < g.K ? kbeg + g.kchunk : g.K;

  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int wm = wid >> 1, wn = wid & 1;
  const int l32 = lane & 31, h = lane >> 5;

  floatx16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // A: logical [M][K]; stored [M][K] (!TA) or [K][M] (TA)
  // B: logical [K][N]; as an "outer = n" tile it is stored [N][K] when TB
  //    (k contiguous, like !TA) and [K][N] when !TB (n contiguous, like TA).
  const int64_t ktiles = kend > kbeg ? cdiv(kend - kbeg, BK) : 0;
  // bias_mode 3/4: the workgroups of the first column tile also sum the
  // rows of op(A) over their K range (the bias gradient of a weight
  // gradient), compensated, RKPT k values per lane and K step
  constexpr int RKPT = BK * BM / T;
  const bool row_sums = g.bias_mode >= 3 && tn == 0;
  Kahan rsum;
  floatx4 ra[VA], rb[VB];
  // XF: lse, scale and target of the logits row of each A float4
  float cl[XF ? VA : 1], cs[XF ? VA : 1];
  int ct[XF ? VA : 1];
  // PF2: two register sets in flight (tile t + 2 is fetched while tile t's
  // MFMAs run, and tile t + 1, fetched one K step earlier, is stored after
  // them), for the tiles at two waves per SIMD, where few other waves cover
  // the fetch of the next tile; not for the A . B and A . B^T forms of the
  // 4-wave 256 x 128 tile, whose second set leaves its 128 x 64 wave tiles
  // too few registers to read fragments ahead (measured slower)
  constexpr bool PF2 = gemm_waves_per_simd(BM, BN, WR) == 2 && !XF && (WR == 4 || TA);
  floatx4 ra2[VA], rb2[VB];
  auto fetch = [&](int64_t k0, floatx4 (&xa)[VA], floatx4 (&xb)[VB]) {
    load_tile<TA, BM, VA, EDGE, T>(A, g.lda, g.M, kend, m0, k0, g.vecA, xa);
    load_tile<!TB, BN, VB, EDGE, T>(B, g.ldb, g.N, kend, n0, k0, g.vecB, xb);
  };
  auto stage = [&](int buf, const floatx4 (&xa)[VA], const floatx4 (&xb)[VB]) {
    store_tile<TA, AKC, BM, VA, LA, T>(As[buf], xa);
    store_tile<!TB, BKC, BN, VB, LB, T>(Bs[buf], xb);
  };
  // MID: the two-deep loop stages the other buffer halfway through the
  // MFMAs instead of after them.  It pays where fragments are read a K step
  // ahead as single floats (A^T . B: 4.84 against 5.01 ms for the LM head's
  // weight gradient); with 128-bit fragment reads the stores delay the
  // second half's reads and staging after the MFMAs is faster (4.59
  // against 4.68 ms for its input gradient).
  constexpr bool MID = PF2 && !(AKC || BKC);
  // the MFMAs of the K tile in LDS buffer `cur` (and its row sums); with
  // MID, `mid` runs halfway through them, pinned there
  auto compute = [&](int cur, auto&& mid) {
    auto half = [&]() {
      if constexpr (MID) {
        __builtin_amdgcn_sched_barrier(0);
        mid();
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    if (AKC || BKC) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        floatx4 a[FM], bv[FN];
        read_frags<AKC, FM, LA>(As[cur], wm * WM, l32, h, q, a);
        read_frags<BKC, FN, LB>(Bs[cur], wn * WN, l32, h, q, bv);
        if (q == 1) half();  // after the reads its MFMAs need
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int jn = 0; jn < FN; ++jn)
              acc[i][jn] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][j], bv[jn][j], acc[i][jn], 0, 0, 0);
      }
    } else {
      const float* __restrict__ as = As[cur] + wm * WM + l32;
      const float* __restrict__ bs = Bs[cur] + wn * WN + l32;
      // fragments of step kk+2 are read from LDS before the MFMAs of step kk
      float a[2][FM], bv[2][FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) a[0][i] = as[h * LA + i * 32];
#pragma unroll
      for (int j = 0; j < FN; ++j) bv[0][j] = bs[h * LB + j * 32];
#pragma unroll
      for (int kk = 0; kk < BK; kk += 2) {
        const int c = (kk >> 1) & 1;
        if (kk == BK / 2) half();
        if (kk + 2 < BK) {
#pragma unroll
          for (int i = 0; i < FM; ++i) a[c ^ 1][i] = as[(kk + 2 + h) * LA + i * 32];
#pragma unroll
          for (int j = 0; j < FN; ++j) bv[c ^ 1][j] = bs[(kk + 2 + h) * LB + j * 32];
        }
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[c][i], bv[c][j], acc[i][j], 0, 0, 0);
      }
    }
    if (row_sums) {
      // this lane's k slice of row t % BM of the current A tile
      const int rm = threadIdx.x % BM, rk = (threadIdx.x / BM) * RKPT;
#pragma unroll
      for (int i = 0; i < RKPT; ++i)
        rsum.add(AKC ? As[cur][rm * KS + rk + i] : As[cur][(rk + i) * LA + rm]);
    }
  };

  // K offset of tile t, clamped to the last tile: the two-deep loop fetches
  // unconditionally (a fetch under a condition keeps the register set's old
  // value live beside the new one), re-reading the last tile past the end
  auto kof = [&](int64_t t) { return kbeg + (t < ktiles ? t : (ktiles > 0 ? ktiles - 1 : 0)) * BK; };
  fetch(kbeg, ra, rb);
  if (PF2) fetch(kof(1), ra2, rb2);
  if constexpr (XF) {
    ce_fetch<TA, BM, VA, EDGE, T>(g, g.M, kend, m0, kbeg, cl, cs, ct);
    ce_apply<TA, BM, VA, EDGE, T>(g, g.M, kend, m0, kbeg, cl, cs, ct, ra);
  }
  stage(0, ra, rb);
  __syncthreads();
  __builtin_amdgcn_s_setprio(0);

  if constexpr (PF2) {
    // tile t sits in LDS buffer t % 2 and, until staged, in register set
    // t % 2 (ra/rb even, ra2/rb2 odd); two steps per pass keep the sets static
    int64_t kt = 0;
    for (; kt + 1 < ktiles; kt += 2) {
      fetch(kof(kt + 2), ra, rb);
      // keeps the loads ahead of the MFMAs (the scheduler sinks them to
      // shorten their registers' lifetimes)
      __builtin_amdgcn_sched_barrier(0);
      compute(0, [&]() { stage(1, ra2, rb2); });
      if constexpr (!MID) stage(1, ra2, rb2);
      __syncthreads();
      fetch(kof(kt + 3), ra2, rb2);
      __builtin_amdgcn_sched_barrier(0);
      // unconditional: past the last tile this stages the clamped re-read,
      // and buffer 0 is not read again
      compute(1, [&]() { stage(0, ra, rb); });
      if constexpr (!MID) stage(0, ra, rb);
      __syncthreads();
    }
    if (kt < ktiles) {  // an odd count: the last tile is in buffer 0
      compute(0, [] {});
      __syncthreads();
    }
  } else {
    for (int64_t kt = 0; kt < ktiles; ++kt) {
      const int cur = kt & 1;
      const bool more = kt + 1 < ktiles;
      if (more) {
        const int64_t k0 = kbeg + (kt + 1) * BK;
        fetch(k0, ra, rb);
        if constexpr (XF && TA) ce_fetch<TA, BM, VA, EDGE, T>(g, g.M, kend, m0, k0, cl, cs, ct);
      }
      compute(cur, [] {});
      if (more) {
        if constexpr (XF)
          ce_apply<TA, BM, VA, EDGE, T>(g, g.M, kend, m0, kbeg + (kt + 1) * BK, cl, cs, ct, ra);
        stage(cur ^ 1, ra, rb);
      }
      __syncthreads();
    }
  }

  __builtin_amdgcn_s_setprio(3);
  if (row_sums) {
    // lanes t, t + BM, ... hold slices of row t: combined in that order.
    // The staging tiles are free here (the K loop ended on a barrier).
    float* rpart = As[0];
    rpart[threadIdx.x] = rsum.s;
    __syncthreads();
    const int64_t row = m0 + threadIdx.x;
    if (threadIdx.x < BM && row < g.M) {
      float v = 0.f;
#pragma unroll
      for (int q = 0; q < T / BM; ++q) v += rpart[threadIdx.x + q * BM];
      float* out = const_cast<float*>(g.bias);
      if (g.rsw) g.rsw[(int64_t)blockIdx.y * g.M + row] = v;
      else if (g.bias_mode == 3) out[row] = v;
      else out[row] += v;
    }
  }

  // ---- epilogue
  // Element (i, j, r) of this wave sits at row r0 + ro(i, r), column
  // c0 + 32 j, with ro = 32 i + 8 (r / 4) + r % 4.  Addresses are one base
  // per lane plus a uniform row offset (ro x ld, scalar arithmetic), and
  // the beta / bias / activation choice is made once, not per element:
  // the epilogue runs beside the other workgroup's MFMAs, where every
  // vector instruction it issues is slow.
  const int64_t r0 = m0 + wm * WM + 4 * h, c0 = n0 + wn * WN + l32;
  auto each = [&](auto&& put) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        if (EDGE && c0 + j * 32 >= g.N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int ro = i * 32 + 8 * (r >> 2) + (r & 3);
          if (!EDGE || r0 + ro < g.M) put(acc[i][j][r], ro, j * 32);
        }
      }
  };
  if (g.ws) {
    // raw partial sums; the reduce kernel applies alpha / beta / bias
    float* __restrict__ W =
        g.ws + ((int64_t)b * gridDim.y + blockIdx.y) * g.M * g.N + r0 * g.N + c0;
    const int64_t ld = g.N;
    each([&](float a, int ro, int co) { W[ro * ld + co] = a; });
    return;
  }
  float* __restrict__ Cb = C + r0 * g.ldc + c0;
  const int64_t ldc = g.ldc, ldx = g.ldaux;
  float* __restrict__ Xb = g.aux ? g.aux + r0 * ldx + c0 : nullptr;
  const float alpha = g.alpha;
  const bool nobias = g.bias_mode == 0 || g.bias_mode >= 3;  // 3, 4: row sums, no add
  if (g.beta == 0.f && nobias && g.act == 0) {
    each([&](float a, int ro, int co) { Cb[ro * ldc + co] = alpha * a; });
  } else if (g.beta == 0.f && g.bias_mode == 1 && (g.act == 0 || g.act == 1 || g.act == 3)) {
    // bias per column (+ GELU with its input kept, or + residual)
    const float* __restrict__ bb = g.bias + c0;
    const int act = g.act;
    auto run = [&](auto ACT) {
      constexpr int A = decltype(ACT)::value;
      each([&](float a, int ro, int co) {
        float v = alpha * a + bb[co];
        if (A == 1) {
          Xb[ro * ldx + co] = v;
          v = gelu_f(v);
        } else if (A == 3) {
          v += Xb[ro * ldx + co];
        }
        Cb[ro * ldc + co] = v;
      });
    };
    if (act == 0) run(IConst<0>());
    else if (act == 1) run(IConst<1>());
    else run(IConst<3>());
  } else if (g.beta == 0.f && nobias && g.act == 2) {
    // the GELU gradient of the kept input
    each([&](float a, int ro, int co) {
      Cb[ro * ldc + co] = alpha * a * gelu_grad(Xb[ro * ldx + co]);
    });
  } else {
    each([&](float a, int ro, int co) {
      const int64_t row = r0 + ro, col = c0 + co;
      float v = alpha * a;
      float* cp = Cb + ro * ldc + co;
      if (g.beta != 0.f) v += g.beta * *cp;
      if (g.bias_mode == 1) v += g.bias[col];
      else if (g.bias_mode == 2) v += g.bias[row];
      *cp = epilogue_act(g, row, col, v);
    });
  }
}

// C = alpha * sum_s ws[b][s] + beta*C + bias, in a fixed split order.
// VEC: N, ldc and C are 16-byte aligned, so a lane sums 4 columns with
// 128-bit accesses.  Partials are dead after this read (non-temporal).
template <bool VEC>
__global__ __launch_bounds__(256) void k_splitk_reduce(GemmArgs g, int splits) {
  const int64_t mn = g.M * g.N;
  const int64_t b = blockIdx.y;
  float* __restrict__ C = g.C + b * g.sC;
  const float* __restrict__ W = g.ws + b * splits * mn;
  const uint32_t w = VEC ? (uint32_t)(g.N / 4) : (uint32_t)g.N;  // items per row
  const uint32_t items = (uint32_t)g.M * w;
  for (uint32_t e = blockIdx.x * 256 + threadIdx.x; e < items; e += gridDim.x * 256) {
    const uint32_t row = e / w, c0 = (e - row * w) * (VEC ? 4 : 1);
    const int64_t off = (int64_t)row * g.N + c0;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    // four splits' loads in flight before their adds (the same order of adds)
    int q = 0;
    if (VEC) {
      for (; q + 4 <= splits; q += 4) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = ld_nt(W + (q + u) * mn + off);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          s[0] += v[u].x; s[1] += v[u].y; s[2] += v[u].z; s[3] += v[u].w;
        }
      }
    }
    for (; q < splits; ++q) {
      if (VEC) {
        const float4 v = ld_nt(W + q * mn + off);
        s[0] += v.x; s[1] += v.y; s[2] += v.z; s[3] += v.w;
      } else {
        s[0] += W[q * mn + off];
      }
    }
    float* cp = C + (int64_t)row * g.ldc + c0;
#pragma unroll
    for (int j = 0; j < (VEC ? 4 : 1); ++j) {
      float v = g.alpha * s[j];
      if (g.beta != 0.f) v += g.beta * cp[j];
      if (g.bias_mode == 1) v += g.bias[c0 + j];
      else if (g.bias_mode == 2) v += g.bias[row];
      s[j] = epilogue_act(g, row, c0 + j, v);
    }
    if (VEC) *reinterpret_cast<float4*>(cp) = make_float4(s[0], s[1], s[2], s[3]);
    else cp[0] = s[0];
  }
  if (g.rsw && b == 0) {
    // row sums of op(A) (bias_mode 3/4), splits summed in order
    float* out = const_cast<float*>(g.bias);
    for (int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x; r < g.M; r += (int64_t)gridDim.x * 256) {
      float t = 0.f;
      for (int q = 0; q < splits; ++q) t += g.rsw[q * g.M + r];
      out[r] = g.bias_mode == 3 ? t : out[r] + t;
    }
  }
}

// ------------------------------------------------------------ tile choice

struct TileCfg {
  int bm, bn, wr;  // block tile, wave rows (2 wave columns)
};
constexpr TileCfg kTiles[] = {{256, 128, 4}, {128, 128, 2}, {128, 64, 2}, {64, 64, 2},
                              {256, 256, 4}, {256, 128, 2}, {256, 192, 4}};
constexpr int kNumTiles = sizeof(kTiles) / sizeof(kTiles[0]);

// Measured relative per-FLOP throughput of each tile with the CUs full, by
// operand layout (GPT-2 products on MI355X, every tile forced in turn): the
// 8-wave 256x128 tile is 3-8% faster than 128x128 on products that fill the
// CUs with it (the LM head's three, the 3072-wide ones); 128x64 is 3-5%
// slower per FLOP and wins only where the larger tiles leave CUs idle.
float tile_speed(int ti, int ta, int tb) {
  static const float nt[kNumTiles] = {1.04f, 1.00f, 0.95f, 0.85f, 0.0f, 0.0f, 1.08f};
  static const float nn[kNumTiles] = {1.03f, 1.00f, 0.97f, 0.85f, 1.10f, 0.0f, 1.08f};
  static const float tn[kNumTiles] = {1.03f, 1.00f, 0.97f, 0.85f, 1.10f, 1.04f, 0.0f};
  if (!ta && tb) return nt[ti];
  if (!ta && !tb) return nn[ti];
  if (ta && !tb) return tn[ti];
  return nt[ti];
}

struct Plan {
  int tile;
  int64_t splits;
};

// Work per CU is balanced when the workgroup count is a multiple of the
// CU count: fill = (wgs / cus) / ceil(wgs / cus).
double fill_of(int64_t wgs, int cus) {
  double r = (double)wgs / cus;
  return r / (double)cdiv(wgs, cus);
}

// Split-K factor for `tiles` output tiles: K slices of >= 256 (>= 64 when
// the tiles would occupy fewer than half the CUs), at most 64, chosen for
// the best fill once the tiles alone cannot fill the CUs twice.
int64_t choose_splits(int64_t tiles, int64_t K, int cus) {
  if (tiles >= 2LL * cus) return 1;
  const int64_t slice = 2 * tiles < cus ? 64 : 256;
  if (K < 4 * slice) return 1;
  int64_t smax = K / slice;
  if (smax > 64) smax = 64;
  int64_t best = 1;
  double best_f = -1.0;
  for (int64_t s = 1; s <= smax; ++s) {
    if (tiles * s < cus && s < smax) continue;
    // partial traffic grows with s: prefer fewer splits on near ties
    double f = fill_of(tiles * s, cus) * (1.0 - 0.004 * (double)s);
    if (tiles * s < cus) f *= (double)(tiles * s) / cus;
    if (f > best_f + 1e-9) {
      best_f = f;
      best = s;
    }
  }
  return best;
}

// K slices for the 256 x 256 tile when its tiles alone leave the last
// round of workgroups part-empty (one workgroup per CU): the best fill,
// each slice charged 2% for its [M, N] partials (written, then summed).
int64_t wide_splits(int64_t tiles, int64_t K, int cus) {
  int64_t best = 1;
  double best_f = -1.0;
  for (int64_t s = 1; s <= 8 && K / s >= 1024; ++s) {
    const double f = fill_of(tiles * s, cus) * (1.0 - 0.02 * (double)s);
    if (f > best_f + 1e-9) {
      best_f = f;
      best = s;
    }
  }
  return best;
}

// Picks tile and split maximising (useful fraction of padded work) x
// (CU fill) x tile speed.  TJH_GEMM_TILE=BMxBN forces a tile (read on every
// call, so a test can sweep the tiles in one process; the 4-wave 256 x 128
// tile is 256x128w4).  The 8-wave 256x128
// tile needs more K splits than 128x128 for the same fill, which doubles
// the split-sum traffic: it is taken only with no K split (measured on the
// GPT-2 products, the best of three interleaved runs each: the split
// weight gradients and 768-wide input gradients run 3-8% slower with it,
// the LM head's K-split input gradient (K = 50257) 3.4% slower, 6.45
// against 6.23 ms; the MLP's 3072-wide GEMMs 2-5% faster).
Plan choose_plan(int64_t M, int64_t N, int64_t K, int64_t batch, int cus, int ta, int tb,
                 int act) {
  int forced = -1;
  if (const char* e = getenv("TJH_GEMM_TILE")) {
    for (int i = 0; i < kNumTiles; ++i) {
      char buf[32];
      // the 4-wave 256 x 128 tile is named 256x128w4
      snprintf(buf, sizeof(buf), "%dx%d%s", kTiles[i].bm, kTiles[i].bn,
               kTiles[i].bm / kTiles[i].wr > 64 ? "w4" : "");
      if (strcmp(buf, e) == 0) forced = i;
    }
  }
  Plan best{1, 1};
  double best_score = -1.0;
  for (int i = 0; i < kNumTiles; ++i) {
    if (forced >= 0 && i != forced) continue;
    const TileCfg& t = kTiles[i];
    // 256 x 256 (two waves per SIMD, 64 x 128 per wave): only for A . B
    // with a very long K (the LM head's input gradient, K = vocab: 5.68
    // against 6.27 ms) and for A^T . B with vocabulary-sized M (its weight
    // gradient, over three K slices: 5.31 against 5.86 ms), where halving
    // the column tiles halves the re-reads of the [vocab, tokens] operand;
    // slower on every other GPT-2 product
    const bool wide = t.bn >= 256;
    const bool wide_ok = tb == 0 && ((!ta && K >= 32768) || (ta && M >= 32768));
    if (wide && forced < 0 && !wide_ok) continue;
    int64_t tm = cdiv(M, t.bm), tn = cdiv(N, t.bn);
    double useful = (double)(M * N) / (double)(tm * t.bm * tn * t.bn);
    int64_t tiles = tm * tn * batch;
    int64_t s = choose_splits(tiles, K, cus);
    if (wide && ta && s == 1) s = wide_splits(tiles, K, cus);
    // 4-wave 256 x 128 (128 x 64 per wave, two workgroups per CU): only for
    // A^T . B over K slices of >= 1024 (GPT-2's 3072 x 768 weight
    // gradients over 7 slices: 351 against 363 us; 3-4% slower over the 14
    // and 28 slices of the smaller ones, and on every A . B and A . B^T)
    if (i == 5 && forced < 0 && (!ta || tb || K / s < 1024)) continue;
    // 256 x 192 (8 waves of 64 x 96, one workgroup per CU): for A . B and
    // A . B^T split over K into at most two rounds of the CUs (GPT-2's
    // 8192 x 768 products over K = 2304 or 3072 in two slices: 3-5% faster
    // than 128 x 128).  Unsplit, or with the GELU-gradient epilogue (which
    // reads the kept input; nothing else on the CU hides it), the tiles that
    // share a CU at four waves per SIMD are as fast or faster (8192 x 3072 x
    // 768 with GELU': 350 against 323 us on 256 x 128), and with more rounds
    // they hide each other's fetch and epilogue better (LM head: 4.81
    // against 5.00 ms).
    if (i == 6 && forced < 0 && (ta || act == 2 || s < 2 || tiles * s > 2LL * cus)) continue;
    if (t.bm >= 256 && t.wr == 4 && t.bn == 128 && forced < 0 && s > 1) continue;
    double score = useful * fill_of(tiles * s, cus) * tile_speed(i, ta, tb);
    if (tiles * s < cus) score *= (double)(tiles * s) / cus;
    if (score > best_score + 1e-9) {
      best_score = score;
      best = Plan{i, s};
    }
  }
  return best;
}

template <int BM, int BN, int WR, bool EDGE>
void launch_e(const GemmArgs& g, dim3 grid, int ta, int tb) {
  const dim3 block(gemm_threads(WR));
  if (g.xrow) {  // A formed from logits: B is never transposed here
    if (ta)
      tjh_launch((k_gemm<BM, BN, WR, true, false, EDGE, true>), grid, block, 0, stream(), g);
    else
      tjh_launch((k_gemm<BM, BN, WR, false, false, EDGE, true>), grid, block, 0, stream(), g);
    return;
  }
  if (!ta && !tb)
    tjh_launch((k_gemm<BM, BN, WR, false, false, EDGE>), grid, block, 0, stream(), g);
  else if (!ta && tb)
    tjh_launch((k_gemm<BM, BN, WR, false, true, EDGE>), grid, block, 0, stream(), g);
  else if (ta && !tb)
    tjh_launch((k_gemm<BM, BN, WR, true, false, EDGE>), grid, block, 0, stream(), g);
  else
    tjh_launch((k_gemm<BM, BN, WR, true, true, EDGE>), grid, block, 0, stream(), g);
}

template <int BM, int BN, int WR>
void launch(const GemmArgs& g, dim3 grid, int ta, int tb, bool edge) {
  if (edge) launch_e<BM, BN, WR, true>(g, grid, ta, tb);
  else launch_e<BM, BN, WR, false>(g, grid, ta, tb);
}

void launch_tile(int ti, const GemmArgs& g, dim3 grid, int ta, int tb, bool edge) {
  switch (ti) {
    case 0: launch<256, 128, 4>(g, grid, ta, tb, edge); break;
    case 1: launch<128, 128, 2>(g, grid, ta, tb, edge); break;
    case 2: launch<128, 64, 2>(g, grid, ta, tb, edge); break;
    case 4: launch<256, 256, 4>(g, grid, ta, tb, edge); break;
    case 5: launch<256, 128, 2>(g, grid, ta, tb, edge); break;
    case 6: launch<256, 192, 4>(g, grid, ta, tb, edge); break;
    default: launch<64, 64, 2>(g, grid, ta, tb, edge); break;
  }
}

// One launch of tile `ti` over the whole of g (plus the split-K pass).
int run_block(int ti, GemmArgs g, int ta, int tb, int64_t splits, int64_t batch, bool edge,
              int cus) {
  const TileCfg& tc = kTiles[ti];
  g.tiles_m = (int)cdiv(g.M, tc.bm);
  g.tiles_n = (int)cdiv(g.N, tc.bn);
  TJH_ARG((int64_t)g.tiles_m * g.tiles_n < (int64_t(1) << 31), "tjh_gemm: too many tiles");
  g.kchunk = cdiv(cdiv(g.K, splits), BK) * BK;
  if (g.kchunk < BK) g.kchunk = BK;
  splits = cdiv(g.K, g.kchunk) > 0 ? cdiv(g.K, g.kchunk) : 1;
  if (g.M * g.N >= (int64_t(1) << 32)) {  // the split-K sum indexes elements in 32 bits
    splits = 1;
    g.kchunk = g.K > 0 ? cdiv(g.K, BK) * BK : BK;
  }
  g.ws = nullptr;
  g.rsw = nullptr;
  const int64_t rs_len = g.bias_mode >= 3 ? splits * g.M : 0;
  Scratch ws(splits > 1 ? (size_t)(batch * splits * g.M * g.N + rs_len) * sizeof(float) : 0);
  if (splits > 1) {
    if (!ws.ok()) {
      splits = 1;
      g.kchunk = g.K > 0 ? cdiv(g.K, BK) * BK : BK;
    } else {
      g.ws = ws.as<float>();
      if (rs_len) g.rsw = g.ws + batch * splits * g.M * g.N;
    }
  }
  dim3 grid((unsigned)(g.tiles_m * g.tiles_n), (unsigned)splits, (unsigned)batch);
  launch_tile(ti, g, grid, ta, tb, edge);
  int rc = check_launch("gemm");
  if (rc != TJH_OK || splits == 1) return rc;
  const bool vec = g.N % 4 == 0 && g.ldc % 4 == 0 && g.sC % 4 == 0 && aligned16(g.C);
  int64_t blocks = cdiv(g.M * g.N / (vec ? 4 : 1), 256);
  if (blocks > 16LL * cus) blocks = 16LL * cus;
  if (vec)
    tjh_launch(k_splitk_reduce<true>, dim3((unsigned)blocks, (unsigned)batch), dim3(256),
                       0, stream(), g, (int)splits);
  else
    tjh_launch(k_splitk_reduce<false>, dim3((unsigned)blocks, (unsigned)batch), dim3(256),
                       0, stream(), g, (int)splits);
  return check_launch("gemm_splitk_reduce");
}

// Sub-problem of g: rows [m0, m0+M), cols [n0, n0+N), k [k0, k0+K).
GemmArgs sub(const GemmArgs& g, int ta, int tb, int64_t m0, int64_t M, int64_t n0, int64_t N,
             int64_t k0, int64_t K) {
  GemmArgs s = g;
  s.M = M; s.N = N; s.K = K;
  s.A = g.A + (ta ? k0 * g.lda + m0 : m0 * g.lda + k0);
  s.B = g.B + (tb ? n0 * g.ldb + k0 : k0 * g.ldb + n0);
  s.C = g.C + m0 * g.ldc + n0;
  if (g.aux) s.aux = g.aux + m0 * g.ldaux + n0;
  s.xm0 = g.xm0 + m0;
  s.xk0 = g.xk0 + k0;
  if (g.bias_mode == 1) s.bias = g.bias + n0;
  else if (g.bias_mode >= 2) s.bias = g.bias + m0;
  return s;
}

}  // namespace
}  // namespace tjh

using namespace tjh;

int tjh::gemm(const char* family, int transA, int transB, int64_t M, int64_t N, int64_t K,
              float alpha, const float* A, int64_t lda, int64_t strideA, const float* B,
              int64_t ldb, int64_t strideB, float beta, float* C, int64_t ldc, int64_t strideC,
              int64_t batch, const float* bias, int bias_mode, float* aux, int64_t ldaux, int act,
              const float* ce_rows) {
  TJH_REQUIRE_INIT();
  TJH_ARG(M >= 0 && N >= 0 && K >= 0 && batch >= 0, "tjh_gemm: negative size");
  TJH_ARG(bias_mode >= 0 && bias_mode <= 3, "tjh_gemm: bad bias_mode %d", bias_mode);
  TJH_ARG(bias_mode == 0 || bias, "tjh_gemm: bias_mode %d needs a bias pointer", bias_mode);
  TJH_ARG(bias_mode != 3 || batch <= 1, "tjh_gemm: bias_mode 3 needs batch 1");
  TJH_ARG(act >= 0 && act <= 3, "tjh_gemm_act: bad activation %d", act);
  TJH_ARG(act == 0 || (aux && ldaux >= N && batch <= 1),
          "tjh_gemm_act: activation %d needs aux (ld >= N) and batch 1", act);
  TJH_ARG(!ce_rows || (!transB && batch <= 1 && bias_mode == 0 && act == 0),
          "tjh_gemm_ce: B not transposed, no batch, bias or activation");
  if (M == 0 || N == 0 || batch == 0) return TJH_OK;
  TJH_ARG(batch <= 65535, "tjh_gemm: batch %lld exceeds 65535", (long long)batch);
  // row strides must cover the contiguous extent
  TJH_ARG(lda >= (transA ? M : K) || (transA ? M : K) <= 1, "tjh_gemm: lda too small");
  TJH_ARG(ldb >= (transB ? K : N) || (transB ? K : N) <= 1, "tjh_gemm: ldb too small");
  TJH_ARG(ldc >= N, "tjh_gemm: ldc too small");
  const int cus = num_cus() > 0 ? num_cus() : 256;
  GemmArgs g;
  g.A = A; g.B = B; g.C = C; g.bias = bias;
  g.M = M; g.N = N; g.K = K;
  g.lda = lda; g.ldb = ldb; g.ldc = ldc;
  g.sA = strideA; g.sB = strideB; g.sC = strideC;
  g.alpha = alpha; g.beta = beta; g.bias_mode = bias_mode;
  g.vecA = ((uintptr_t)A & 3) == 0;
  g.vecB = ((uintptr_t)B & 3) == 0;
  g.tiles_m = g.tiles_n = 0;
  g.kchunk = BK;
  g.ws = nullptr;
  g.rsw = nullptr;
  g.aux = act ? aux : nullptr;
  g.ldaux = ldaux;
  g.act = act;
  g.xrow = reinterpret_cast<const floatx4*>(ce_rows);
  g.xm0 = g.xk0 = 0;
  KernelScope ks(family);
  const Plan plan = choose_plan(M, N, K, batch, cus, transA, transB, act);
  const TileCfg& tc = kTiles[plan.tile];
  if (!(g.vecA && g.vecB)) {
    // operands not 4-byte aligned: guarded scalar loads everywhere
    return run_block(plan.tile, g, transA, transB, plan.splits, batch, true, cus);
  }
  // Interior block [0,Mm) x [0,Nm) x [0,Km) runs the unguarded kernel; the
  // row / column strips beyond it run the guarded one; a K remainder is
  // added by one more guarded pass with beta = 1.
  const int64_t Mm = M / tc.bm * tc.bm, Nm = N / tc.bn * tc.bn, Km = K / BK * BK;
  const int64_t Kr = K - Km;
  GemmArgs gk = g;
  gk.K = Km;
  if (Kr > 0) gk.act = 0;  // the K remainder pass applies the activation
  int rc = TJH_OK;
  if (Km == 0) {
    // K < 16: one guarded pass does it all
    return run_block(plan.tile, g, transA, transB, 1, batch, true, cus);
  }
  if (Mm > 0 && Nm > 0)
    rc = run_block(plan.tile, sub(gk, transA, transB, 0, Mm, 0, Nm, 0, Km), transA, transB,
                   plan.splits, batch, false, cus);
  // Edge strips pick their own tile and K split: a thin strip of a long-K
  // product (the 81 leftover rows of a 50257-row weight gradient) would
  // otherwise run on a dozen workgroups for the whole K range.
  if (rc == TJH_OK && Nm < N) {  // right strip (all rows)
    const Plan ps = choose_plan(M, N - Nm, Km, batch, cus, transA, transB, act);
    GemmArgs gs = sub(gk, transA, transB, 0, M, Nm, N - Nm, 0, Km);
    if (gs.bias_mode == 3 && Nm > 0) gs.bias_mode = 0;  // row sums come from column 0's tiles
    rc = run_block(ps.tile, gs, transA, transB, ps.splits, batch, true, cus);
  }
  if (rc == TJH_OK && Mm < M && Nm > 0) {  // bottom strip (interior columns)
    const Plan ps = choose_plan(M - Mm, Nm, Km, batch, cus, transA, transB, act);
    rc = run_block(ps.tile, sub(gk, transA, transB, Mm, M - Mm, 0, Nm, 0, Km), transA, transB,
                   ps.splits, batch, true, cus);
  }
  if (rc == TJH_OK && Kr > 0) {
    GemmArgs gr = sub(g, transA, transB, 0, M, 0, N, Km, Kr);
    gr.beta = 1.0f;
    if (g.bias_mode == 3) {
      gr.bias_mode = 4;  // add this K range's row sums
    } else {
      gr.bias_mode = 0;
      gr.bias = nullptr;
    }
    // its own tile: a few K steps over the whole of C is a pass over C,
    // which wants every CU (the LM head's 17-deep remainder on the 256 x 256
    // tile ran on 96 workgroups)
    const Plan pr = choose_plan(M, N, Kr, batch, cus, transA, transB, act);
    rc = run_block(pr.tile, gr, transA, transB, 1, batch, true, cus);
  }
  return rc;
}

extern "C" int tjh_gemm(int transA, int transB, int64_t M, int64_t N, int64_t K, float alpha,
                        const float* A, int64_t lda, int64_t strideA, const float* B, int64_t ldb,
                        int64_t strideB, float beta, float* C, int64_t ldc, int64_t strideC,
                        int64_t batch, const float* bias, int bias_mode) {
  return tjh::gemm("gemm", transA, transB, M, N, K, alpha, A, lda, strideA, B, ldb, strideB, beta,
                   C, ldc, strideC, batch, bias, bias_mode);
}

extern "C" int tjh_gemm_act(int transA, int transB, int64_t M, int64_t N, int64_t K, float alpha,
                            const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                            float* C, int64_t ldc, const float* bias, int bias_mode, float* aux,
                            int64_t ldaux, int act) {
  return tjh::gemm("gemm", transA, transB, M, N, K, alpha, A, lda, 0, B, ldb, 0, beta, C, ldc, 0,
                   1, bias, bias_mode, aux, ldaux, act);
}

extern "C" int tjh_gemm_ce(int transA, int64_t M, int64_t N, int64_t K, const float* logits,
                           int64_t ld, const float* lse, const int32_t* targets,
                           const float* row_scale, const float* B, int64_t ldb, float* C,
                           int64_t ldc) {
  TJH_REQUIRE_INIT();
  TJH_ARG(lse && targets && row_scale && logits, "tjh_gemm_ce: NULL operand");
  TJH_ARG(M >= 0 && N >= 0 && K >= 0, "tjh_gemm_ce: negative size");
  const int64_t rows = transA ? K : M;  // logits rows
  if (M == 0 || N == 0) return TJH_OK;
  Scratch xrow((size_t)(rows > 0 ? rows : 1) * 4 * sizeof(float));
  if (!xrow.ok()) return set_error(TJH_ERR_OOM, "tjh_gemm_ce: no scratch");
  if (rows > 0) {
    KernelScope ks("gemm");
    tjh_launch(k_ce_rows, dim3((unsigned)cdiv(rows, 256)), dim3(256), 0, stream(), lse, targets,
               row_scale, rows, xrow.as<floatx4>());
    int rc = check_launch("gemm_ce_rows");
    if (rc != TJH_OK) return rc;
  }
  return tjh::gemm("gemm", transA, 0, M, N, K, 1.0f, logits, ld, 0, B, ldb, 0, 0.0f, C, ldc, 0, 1,
                   nullptr, 0, nullptr, 0, 0, xrow.as<float>());
}
