// fp32 GEMM on the CDNA4 matrix cores (v_mfma_f32_32x32x2_f32).
//
// Replaces matmul.wgsl:17-50 (a 16x16 scalar tile kernel) behind torch.js's
// Tensor.matmul / mm / bmm and nn.Linear (Tensor.ts:2132-2331,
// src/nn/linear.ts:43-66), and supplies the dgrad / wgrad products the
// reference's autograd never issues (Tensor.ts:2212-2221).
//
// C[b] = alpha * op(A[b]) op(B[b]) + beta * C[b] (+ bias), row-major.
//
// Tiling (one workgroup = 256 lanes = 4 wave64):
//   block tile 128 x 128, K step 16, waves arranged 2 x 2, each wave owns a
//   64 x 64 sub-tile = 2 x 2 MFMA 32x32 blocks (64 accumulator registers).
//   A and B tiles are staged in LDS k-major (As[k][m], Bs[k][n]) with a
//   4-float pad, double-buffered: the next K tile is fetched from HBM into
//   registers while the MFMAs consume the current LDS tile.
// MFMA operand layout (32x32x2 f32): lane l feeds A[m = l%32][k = l/32] and
//   B[k = l/32][n = l%32]; accumulator register r of lane l holds
//   C[8*(r/4) + 4*(l/32) + r%4][l%32].
// Global loads are 128-bit when the operand's contiguous dimension and row
// stride allow it; edge tiles fall back to guarded scalar loads.
// Workgroup order: tiles are grouped 8 M-tiles at a time so neighbouring
// workgroups share B columns in L2.

#include "common.h"

namespace tjh {
namespace {

constexpr int BM = 128, BN = 128, BK = 16;
constexpr int kThreads = 256;
constexpr int PAD = 4;
constexpr int LDA_S = BM + PAD;  // LDS row length of As[k][*]
constexpr int LDB_S = BN + PAD;

typedef float floatx16 __attribute__((ext_vector_type(16)));

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
};

// Loads the A tile (BM x BK, rows m0.., cols k0..) for lane t into regs.
// Non-transposed A ([M][K], k contiguous): 2 float4 along k per lane.
// Transposed A ([K][M], m contiguous): 2 float4 along m per lane.
template <bool TRANS>
__device__ __forceinline__ void load_tile(const float* __restrict__ P, int64_t ld,
                                          int64_t rows, int64_t cols, int64_t r0,
                                          int64_t c0, bool vec, float4 (&reg)[2]) {
  // Logical tile: R = 128 "outer" indices (m or n), BK k indices.
  // For !TRANS the storage is [outer][k]: element (o, k) at P[o*ld + k].
  // For TRANS the storage is [k][outer]: element (o, k) at P[k*ld + o].
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    int f = t + kThreads * i;
    if (!TRANS) {
      int o = f >> 2, kq = f & 3;
      int64_t go = r0 + o, gk = c0 + kq * 4;
      if (vec && go < rows && gk + 3 < cols) {
        reg[i] = *reinterpret_cast<const float4*>(P + go * ld + gk);
      } else {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          v[j] = (go < rows && gk + j < cols) ? P[go * ld + gk + j] : 0.f;
        reg[i] = make_float4(v[0], v[1], v[2], v[3]);
      }
    } else {
      int k = f >> 5, oq = f & 31;
      int64_t gk = c0 + k, go = r0 + oq * 4;
      if (vec && gk < cols && go + 3 < rows) {
        reg[i] = *reinterpret_cast<const float4*>(P + gk * ld + go);
      } else {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          v[j] = (gk < cols && go + j < rows) ? P[gk * ld + go + j] : 0.f;
        reg[i] = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
  }
}

// Stores a loaded tile into LDS laid out S[k][outer] (row length LDS_W).
template <bool TRANS, int LDS_W>
__device__ __forceinline__ void store_tile(float* __restrict__ S, const float4 (&reg)[2]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    int f = t + kThreads * i;
    if (!TRANS) {
      int o = f >> 2, kq = f & 3;
      S[(kq * 4 + 0) * LDS_W + o] = reg[i].x;
      S[(kq * 4 + 1) * LDS_W + o] = reg[i].y;
      S[(kq * 4 + 2) * LDS_W + o] = reg[i].z;
      S[(kq * 4 + 3) * LDS_W + o] = reg[i].w;
    } else {
      int k = f >> 5, oq = f & 31;
      *reinterpret_cast<float4*>(S + k * LDS_W + oq * 4) = reg[i];
    }
  }
}

template <bool TA, bool TB>
__global__ __launch_bounds__(kThreads, 2) void k_gemm(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) float As[2][BK * LDA_S];
  __shared__ __attribute__((aligned(16))) float Bs[2][BK * LDB_S];

  // ---- tile coordinates (grouped ordering for L2 reuse)
  const int tiles_m = g.tiles_m, tiles_n = g.tiles_n;
  int bid = blockIdx.x;
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

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // A: logical [M][K]; stored [M][K] (!TA) or [K][M] (TA)
  // B: logical [K][N]; as an "outer = n" tile it is stored [N][K] when TB
  //    (k contiguous, like !TA) and [K][N] when !TB (n contiguous, like TA).
  const int64_t ktiles = kend > kbeg ? cdiv(kend - kbeg, BK) : 0;
  float4 ra[2], rb[2];
  load_tile<TA>(A, g.lda, g.M, kend, m0, kbeg, g.vecA, ra);
  load_tile<!TB>(B, g.ldb, g.N, kend, n0, kbeg, g.vecB, rb);
  store_tile<TA, LDA_S>(As[0], ra);
  store_tile<!TB, LDB_S>(Bs[0], rb);
  __syncthreads();

  for (int64_t kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < ktiles;
    if (more) {
      load_tile<TA>(A, g.lda, g.M, kend, m0, kbeg + (kt + 1) * BK, g.vecA, ra);
      load_tile<!TB>(B, g.ldb, g.N, kend, n0, kbeg + (kt + 1) * BK, g.vecB, rb);
    }
    const float* __restrict__ as = As[cur];
    const float* __restrict__ bs = Bs[cur];
#pragma unroll
    for (int kk = 0; kk < BK; kk += 2) {
      float a0 = as[(kk + h) * LDA_S + wm * 64 + l32];
      float a1 = as[(kk + h) * LDA_S + wm * 64 + 32 + l32];
      float b0 = bs[(kk + h) * LDB_S + wn * 64 + l32];
      float b1 = bs[(kk + h) * LDB_S + wn * 64 + 32 + l32];
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc[1][1], 0, 0, 0);
    }
    if (more) {
      store_tile<TA, LDA_S>(As[cur ^ 1], ra);
      store_tile<!TB, LDB_S>(Bs[cur ^ 1], rb);
    }
    __syncthreads();
  }

  // ---- epilogue
  if (g.ws) {
    // raw partial sums; the reduce kernel applies alpha / beta / bias
    float* __restrict__ W = g.ws + ((int64_t)b * gridDim.y + blockIdx.y) * g.M * g.N;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int64_t col = n0 + wn * 64 + j * 32 + l32;
        if (col >= g.N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          if (row < g.M) W[row * g.N + col] = acc[i][j][r];
        }
      }
    return;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = n0 + wn * 64 + j * 32 + l32;
      if (col >= g.N) continue;
      float bn = (g.bias_mode == 1) ? g.bias[col] : 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (row < g.M) {
          float v = g.alpha * acc[i][j][r];
          float* cp = C + row * g.ldc + col;
          if (g.beta != 0.f) v += g.beta * *cp;
          if (g.bias_mode == 1) v += bn;
          else if (g.bias_mode == 2) v += g.bias[row];
          *cp = v;
        }
      }
    }
  }
}

// C = alpha * sum_s ws[b][s] + beta*C + bias, in a fixed split order.
__global__ __launch_bounds__(256) void k_splitk_reduce(GemmArgs g, int splits) {
  const int64_t mn = g.M * g.N;
  const int64_t b = blockIdx.y;
  float* __restrict__ C = g.C + b * g.sC;
  const float* __restrict__ W = g.ws + b * splits * mn;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < mn; e += (int64_t)gridDim.x * 256) {
    float s = 0.f;
    for (int q = 0; q < splits; ++q) s += W[q * mn + e];
    const int64_t row = e / g.N, col = e % g.N;
    float v = g.alpha * s;
    float* cp = C + row * g.ldc + col;
    if (g.beta != 0.f) v += g.beta * *cp;
    if (g.bias_mode == 1) v += g.bias[col];
    else if (g.bias_mode == 2) v += g.bias[row];
    *cp = v;
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace
}  // namespace tjh

using namespace tjh;

int tjh::gemm(const char* family, int transA, int transB, int64_t M, int64_t N, int64_t K,
              float alpha, const float* A, int64_t lda, int64_t strideA, const float* B,
              int64_t ldb, int64_t strideB, float beta, float* C, int64_t ldc, int64_t strideC,
              int64_t batch, const float* bias, int bias_mode) {
  TJH_REQUIRE_INIT();
  TJH_ARG(M >= 0 && N >= 0 && K >= 0 && batch >= 0, "tjh_gemm: negative size");
  TJH_ARG(bias_mode >= 0 && bias_mode <= 2, "tjh_gemm: bad bias_mode %d", bias_mode);
  TJH_ARG(bias_mode == 0 || bias, "tjh_gemm: bias_mode %d needs a bias pointer", bias_mode);
  if (M == 0 || N == 0 || batch == 0) return TJH_OK;
  TJH_ARG(batch <= 65535, "tjh_gemm: batch %lld exceeds 65535", (long long)batch);
  // row strides must cover the contiguous extent
  TJH_ARG(lda >= (transA ? M : K) || (transA ? M : K) <= 1, "tjh_gemm: lda too small");
  TJH_ARG(ldb >= (transB ? K : N) || (transB ? K : N) <= 1, "tjh_gemm: ldb too small");
  TJH_ARG(ldc >= N, "tjh_gemm: ldc too small");
  GemmArgs g;
  g.A = A; g.B = B; g.C = C; g.bias = bias;
  g.M = M; g.N = N; g.K = K;
  g.lda = lda; g.ldb = ldb; g.ldc = ldc;
  g.sA = strideA; g.sB = strideB; g.sC = strideC;
  g.alpha = alpha; g.beta = beta; g.bias_mode = bias_mode;
  g.vecA = aligned16(A) && (lda % 4 == 0) && (strideA % 4 == 0);
  g.vecB = aligned16(B) && (ldb % 4 == 0) && (strideB % 4 == 0);
  g.tiles_m = (int)cdiv(M, BM);
  g.tiles_n = (int)cdiv(N, BN);
  TJH_ARG((int64_t)g.tiles_m * g.tiles_n < (int64_t(1) << 31), "tjh_gemm: too many tiles");
  // Split K when the output tiles alone cannot fill the machine (weight
  // gradients: small M x N, K = tokens).  Partials go to scratch and a
  // second pass sums them in a fixed order.
  int cus = num_cus() > 0 ? num_cus() : 256;
  int64_t tiles = (int64_t)g.tiles_m * g.tiles_n * batch;
  int64_t splits = 1;
  if (tiles < 2LL * cus && K >= 4 * 256) {
    splits = cdiv(2LL * cus, tiles);
    int64_t by_k = K / 256;  // >= 256 of K per split
    if (splits > by_k) splits = by_k;
    if (splits > 64) splits = 64;
    if (splits < 1) splits = 1;
  }
  g.kchunk = cdiv(cdiv(K, splits), BK) * BK;
  if (g.kchunk < BK) g.kchunk = BK;
  splits = cdiv(K, g.kchunk) > 0 ? cdiv(K, g.kchunk) : 1;
  g.ws = nullptr;
  Scratch ws(splits > 1 ? (size_t)(batch * splits * M * N) * sizeof(float) : 0);
  if (splits > 1) {
    if (!ws.ok()) {
      splits = 1;
      g.kchunk = K > 0 ? cdiv(K, BK) * BK : BK;
    } else {
      g.ws = ws.as<float>();
    }
  }
  dim3 grid((unsigned)(g.tiles_m * g.tiles_n), (unsigned)splits, (unsigned)batch);
  KernelScope ks(family);
  if (!transA && !transB)
    hipLaunchKernelGGL((k_gemm<false, false>), grid, dim3(kThreads), 0, stream(), g);
  else if (!transA && transB)
    hipLaunchKernelGGL((k_gemm<false, true>), grid, dim3(kThreads), 0, stream(), g);
  else if (transA && !transB)
    hipLaunchKernelGGL((k_gemm<true, false>), grid, dim3(kThreads), 0, stream(), g);
  else
    hipLaunchKernelGGL((k_gemm<true, true>), grid, dim3(kThreads), 0, stream(), g);
  int rc = check_launch("gemm");
  if (rc != TJH_OK || splits == 1) return rc;
  int64_t blocks = cdiv(M * N, 256);
  if (blocks > 4LL * cus) blocks = 4LL * cus;
  hipLaunchKernelGGL(k_splitk_reduce, dim3((unsigned)blocks, (unsigned)batch), dim3(256), 0,
                     stream(), g, (int)splits);
  return check_launch("gemm_splitk_reduce");
}

extern "C" int tjh_gemm(int transA, int transB, int64_t M, int64_t N, int64_t K, float alpha,
                        const float* A, int64_t lda, int64_t strideA, const float* B, int64_t ldb,
                        int64_t strideB, float beta, float* C, int64_t ldc, int64_t strideC,
                        int64_t batch, const float* bias, int bias_mode) {
  return tjh::gemm("gemm", transA, transB, M, N, K, alpha, A, lda, strideA, B, ldb, strideB, beta,
                   C, ldc, strideC, batch, bias, bias_mode);
}
