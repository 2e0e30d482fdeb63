// conv2d forward / input-gradient / weight-gradient, NCHW, with stride,
// padding, dilation and groups, as implicit GEMMs on the matrix cores
// (v_mfma_f32_32x32x2_f32).
//
// Reference: F.conv2d (src/nn/functional.ts:438-660) over conv.wgsl:25-60
// (one thread per output, 27- or 288-deep serial dot products) and
// conv_backward.wgsl:24-119 (never reached, the grad_fn is dropped by the
// autograd walk).  The reference ignores dilation (written into the pad
// slot); the contract implemented here is torch's.
//
// No patch matrix is materialised.  Each product is a GEMM per group
// whose operand tiles are gathered straight from the NCHW tensors while
// they are staged into LDS (zero outside the image, or where a stride
// skips an input pixel), and whose epilogue writes NCHW directly:
//   forward : y [n][oc][p]     = sum_r  W[oc][r]                * x(r; n,p)
//             M = OC/g, N = images * OH*OW, K = C/g * KH*KW
//   dgrad   : dx[n][c][e]      = sum_k  W[oc][c][kh][kw]        * dy(k; n,e)
//             M = C/g,  N = images * H*W,   K = OC/g * KH*KW,
//             dy(k; n,e) = dy[n][oc][oy][ox] where iy + ph - kh*dh = oy*sh
//             and ix + pw - kw*dw = ox*sw, else 0.  With dilation 1 the
//             input pixels are split into sh*sw stride classes (iy mod sh,
//             ix mod sw); within a class only every sh-th kh (sw-th kw)
//             contributes, so each class is an exact GEMM with
//             K = OC/g * ceil(KH/sh) * ceil(KW/sw) and no skipped taps
//   wgrad   : dW[oc][r]        = sum_j  dy[n][oc][p]            * x(r; n,p)
//             M = OC/g, N = C/g * KH*KW, K = images * OH*OW (split over
//             workgroups, partials summed in split order by colsum_final);
//             the bias gradient db[oc] = sum_j dy[n][oc][p] is the row sum
//             of that A operand, taken by the first column tile's
//             workgroups while they stage it
// with r = (c*KH + kh)*KW + kw, p = oy*OW + ox, e = iy*W + ix and
// x(r; n,p) = x[n][c][oy*sh - ph + kh*dh][ox*sw - pw + kw*dw] (0 outside).
//
// Tiling: 256 lanes = 4 waves, each owning a 32x32 accumulator block; the
// workgroup tile is 32x128, 64x64 or 128x32 (waves 1x4, 2x2, 4x1), chosen
// per call for the least padded work.  K steps of 16 through LDS stored
// k-major, double-buffered, with gathers issued two steps ahead (the
// grids are small, so latency is hidden within a workgroup, not by
// occupancy).  Index arithmetic uses 32-bit
// division by run-time constants through multiply-high (all tensors here
// are below 2^31 elements, checked on the host).

#include "colsum.h"
#include "common.h"
#include "kahan.h"

namespace tjh {
namespace {

constexpr int kThreads = 256;
constexpr int BK = 16;
typedef float floatx16 __attribute__((ext_vector_type(16)));

// Unsigned 32-bit division by a run-time constant d: the round-up method of
// Granlund & Montgomery, "Division by invariant integers using
// multiplication" (PLDI 1994), fig. 4.1, with s = ceil(log2 d) and
// m = floor(2^32 (2^s - d) / d) + 1.  Exact for dividends below 2^31.
struct FastDiv {
  uint32_t d, m, s;
};

FastDiv make_fastdiv(uint32_t d) {
  FastDiv f{d, 0, 0};
  if (d <= 1) return f;
  uint32_t s = 0;
  while ((uint64_t(1) << s) < d) ++s;
  f.s = s;
  f.m = (uint32_t)(((uint64_t(1) << 32) * ((uint64_t(1) << s) - d)) / d + 1);
  return f;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t x, const FastDiv& f) {
  if (f.d <= 1) return x;  // 1; 0 only for divisors of empty extents, never used
  const uint32_t t = __umulhi(x, f.m);
  return (t + ((x - t) >> 1)) >> (f.s - 1);
}

enum Mode { kFwd = 0, kDgrad = 1, kWgrad = 2, kDgradClass = 3 };

struct ConvArgs {
  const float* x;     // input (forward, wgrad)
  const float* wt;    // weights (forward, dgrad)
  const float* dy;    // output gradient (dgrad, wgrad)
  const float* bias;  // forward only, may be null
  float* out;         // y, dx or dW
  float* ws;          // wgrad split partials [groups][splits][M][N], or null
  float* db;          // wgrad: the bias gradient (row sums of dy), or null
  float* rsw;         // wgrad split partials of db [groups][splits][M], or null
  int accumulate;     // wgrad without split: dW (and db) += instead of =
  int relu;           // forward: the output is ReLU(conv + bias)
  uint32_t n, c, h, w, oc, kh, kw, sh, sw, ph, pw, dh, dw, oh, ow;
  uint32_t cg, ocg, kk;      // channels per group, KH*KW
  uint32_t M, N, K;          // GEMM sizes per group
  uint32_t tiles_m, kchunk;  // M tiles; K range of one split (multiple of BK)
  FastDiv f_kk, f_kw, f_p, f_ow, f_hw, f_w, f_sh, f_sw;
  // BK written in the mixed radices the cursors step through:
  // BK = s_c*KK + s_kh*KW + s_kw (digits (c|oc, kh, kw)) and
  // BK = s_oy*OW + s_ox (digits (oy, ox) of an output pixel)
  uint32_t s_c, s_kh, s_kw, s_oy, s_ox;
  // dgrad by stride class (dilation 1): input pixels iy = ry + sh*qy,
  // ix = rx + sw*qx (qy < qh, qx < qw) take taps kh = rkh + sh*ta,
  // kw = rkw + sw*tb (ta < th, tb < tw) from dy[oy = qy + oyc - ta][ox =
  // qx + oxc - tb]; BK = c_oc*th*tw + c_a*tw + c_b.  The fields describe
  // one class; a launch over several classes carries them in `cls`, one
  // class per grid row (blockIdx.y), and the kernel reads its own
  uint32_t ry, rx, rkh, rkw, th, tw, oyc, oxc, qh, qw, c_oc, c_a, c_b;
  FastDiv f_tt, f_tw, f_qq, f_qw;
};

constexpr int kMaxClasses = 4;  // stride classes per dgrad launch
struct ClassArgs {
  uint32_t ry, rx, rkh, rkw, th, tw, oyc, oxc, qh, qw, c_oc, c_a, c_b, N, K;
  FastDiv f_tt, f_tw, f_qq, f_qw;
};
struct ClassSet {
  ClassArgs c[kMaxClasses];
};

// Operand cursors.  A lane stages the same (o, k - k0) positions of every
// K step, so each position gets a cursor: init() decomposes its first k
// (and its fixed o) with divisions once, next() advances k by BK with
// mixed-radix carries, get() reads the element (0 outside [0, M|N) x
// [kbeg, kend), outside the image, or on a stride-skipped pixel).

// (c|oc, kh, kw) += BK
__device__ __forceinline__ void step_taps(const ConvArgs& a, uint32_t& c, uint32_t& kh,
                                          uint32_t& kw) {
  kw += a.s_kw;
  if (kw >= a.kw) { kw -= a.kw; ++kh; }
  kh += a.s_kh;
  if (kh >= a.kh) { kh -= a.kh; ++c; }
  c += a.s_c;
}

// (n, oy, ox) += BK
__device__ __forceinline__ void step_pixel(const ConvArgs& a, uint32_t& n, uint32_t& oy,
                                           uint32_t& ox) {
  ox += a.s_ox;
  if (ox >= a.ow) { ox -= a.ow; ++oy; }
  oy += a.s_oy;
  while (oy >= a.oh) { oy -= a.oh; ++n; }
}

// forward A / wgrad-free weights: W[g*ocg + o][k], k contiguous
struct CurW {
  uint32_t off, k;
  bool ok;
  __device__ void init(const ConvArgs& a, uint32_t g, uint32_t o, uint32_t k0) {
    ok = o < a.M;
    k = k0;
    off = (g * a.ocg + (ok ? o : 0)) * (a.cg * a.kk) + k0;
  }
  __device__ float get(const ConvArgs& a, uint32_t kend) const {
    return (ok && k < kend) ? a.wt[off] : 0.f;
  }
  __device__ void next(const ConvArgs&) { off += BK; k += BK; }
};

// dgrad A: W[g*ocg + oc][o][kh][kw] for k = oc*KK + t
struct CurWt {
  uint32_t oc, t, o, k;
  bool ok;
  __device__ void init(const ConvArgs& a, uint32_t, uint32_t o_, uint32_t k0) {
    ok = o_ < a.M;
    o = ok ? o_ : 0;
    k = k0;
    oc = fdiv(k0, a.f_kk);
    t = k0 - oc * a.kk;
  }
  __device__ float get(const ConvArgs& a, uint32_t kend, uint32_t g) const {
    return (ok && k < kend) ? a.wt[((g * a.ocg + oc) * a.cg + o) * a.kk + t] : 0.f;
  }
  __device__ void next(const ConvArgs& a) {
    k += BK;
    t += a.s_kh * a.kw + a.s_kw;
    if (t >= a.kk) { t -= a.kk; ++oc; }
    oc += a.s_c;
  }
};

// forward B: x(k; j) for a fixed output pixel j and taps k = (c, kh, kw)
struct CurXf {
  uint32_t base, c, kh, kw, k;
  int iy0, ix0;
  bool ok;
  __device__ void init(const ConvArgs& a, uint32_t g, uint32_t j, uint32_t k0) {
    ok = j < a.N;
    const uint32_t jj = ok ? j : 0;
    const uint32_t n = fdiv(jj, a.f_p), p = jj - n * (a.oh * a.ow);
    const uint32_t oy = fdiv(p, a.f_ow), ox = p - oy * a.ow;
    base = (n * a.c + g * a.cg) * a.h * a.w;
    iy0 = (int)(oy * a.sh) - (int)a.ph;
    ix0 = (int)(ox * a.sw) - (int)a.pw;
    k = k0;
    c = fdiv(k0, a.f_kk);
    const uint32_t t = k0 - c * a.kk;
    kh = fdiv(t, a.f_kw);
    kw = t - kh * a.kw;
  }
  __device__ float get(const ConvArgs& a, uint32_t kend) const {
    if (!ok || k >= kend) return 0.f;
    const int iy = iy0 + (int)(kh * a.dh), ix = ix0 + (int)(kw * a.dw);
    if (iy < 0 || iy >= (int)a.h || ix < 0 || ix >= (int)a.w) return 0.f;
    return a.x[base + (c * a.h + (uint32_t)iy) * a.w + (uint32_t)ix];
  }
  __device__ void next(const ConvArgs& a) { k += BK; step_taps(a, c, kh, kw); }
};

// dgrad B: dy(k; j) for a fixed input pixel j and taps k = (oc, kh, kw)
struct CurDy {
  uint32_t base, oc, kh, kw, k;
  int ty0, tx0;
  bool ok;
  __device__ void init(const ConvArgs& a, uint32_t g, uint32_t j, uint32_t k0) {
    ok = j < a.N;
    const uint32_t jj = ok ? j : 0;
    const uint32_t n = fdiv(jj, a.f_hw), e = jj - n * (a.h * a.w);
    const uint32_t iy = fdiv(e, a.f_w), ix = e - iy * a.w;
    base = (n * a.oc + g * a.ocg) * a.oh * a.ow;
    ty0 = (int)(iy + a.ph);
    tx0 = (int)(ix + a.pw);
    k = k0;
    oc = fdiv(k0, a.f_kk);
    const uint32_t t = k0 - oc * a.kk;
    kh = fdiv(t, a.f_kw);
    kw = t - kh * a.kw;
  }
  __device__ float get(const ConvArgs& a, uint32_t kend) const {
    if (!ok || k >= kend) return 0.f;
    const int ty = ty0 - (int)(kh * a.dh), tx = tx0 - (int)(kw * a.dw);
    if (ty < 0 || tx < 0) return 0.f;
    const uint32_t oy = fdiv((uint32_t)ty, a.f_sh), ox = fdiv((uint32_t)tx, a.f_sw);
    if (oy * a.sh != (uint32_t)ty || ox * a.sw != (uint32_t)tx || oy >= a.oh || ox >= a.ow)
      return 0.f;
    return a.dy[base + (oc * a.oh + oy) * a.ow + ox];
  }
  __device__ void next(const ConvArgs& a) { k += BK; step_taps(a, oc, kh, kw); }
};

// wgrad A: dy[n][g*ocg + o][p] for k = j = n*P + p
struct CurDyRow {
  uint32_t n, oy, ox, o, k;
  bool ok;
  __device__ void init(const ConvArgs& a, uint32_t, uint32_t o_, uint32_t k0) {
    ok = o_ < a.M;
    o = ok ? o_ : 0;
    k = k0;
    n = fdiv(k0, a.f_p);
    const uint32_t p = k0 - n * (a.oh * a.ow);
    oy = fdiv(p, a.f_ow);
    ox = p - oy * a.ow;
  }
  __device__ float get(const ConvArgs& a, uint32_t kend, uint32_t g) const {
    if (!ok || k >= kend) return 0.f;
    return a.dy[((n * a.oc + g * a.ocg + o) * a.oh + oy) * a.ow + ox];
  }
  __device__ void next(const ConvArgs& a) { k += BK; step_pixel(a, n, oy, ox); }
};

// wgrad B: x(r; j) for a fixed tap r = (c, kh, kw) and pixels k = j
struct CurXw {
  uint32_t coff, n, oy, ox, k;
  int dy0, dx0;
  bool ok;
  __device__ void init(const ConvArgs& a, uint32_t g, uint32_t r, uint32_t k0) {
    ok = r < a.N;
    const uint32_t rr = ok ? r : 0;
    const uint32_t c = fdiv(rr, a.f_kk), t = rr - c * a.kk;
    const uint32_t kh = fdiv(t, a.f_kw), kw = t - kh * a.kw;
    coff = (g * a.cg + c) * a.h * a.w;
    dy0 = (int)(kh * a.dh) - (int)a.ph;
    dx0 = (int)(kw * a.dw) - (int)a.pw;
    k = k0;
    n = fdiv(k0, a.f_p);
    const uint32_t p = k0 - n * (a.oh * a.ow);
    oy = fdiv(p, a.f_ow);
    ox = p - oy * a.ow;
  }
  __device__ float get(const ConvArgs& a, uint32_t kend) const {
    if (!ok || k >= kend) return 0.f;
    const int iy = (int)(oy * a.sh) + dy0, ix = (int)(ox * a.sw) + dx0;
    if (iy < 0 || iy >= (int)a.h || ix < 0 || ix >= (int)a.w) return 0.f;
    return a.x[n * a.c * a.h * a.w + coff + (uint32_t)iy * a.w + (uint32_t)ix];
  }
  __device__ void next(const ConvArgs& a) { k += BK; step_pixel(a, n, oy, ox); }
};

// (oc, ta, tb) += BK in radices (th, tw)
__device__ __forceinline__ void step_class_taps(const ConvArgs& a, uint32_t& oc, uint32_t& ta,
                                                uint32_t& tb) {
  tb += a.c_b;
  if (tb >= a.tw) { tb -= a.tw; ++ta; }
  ta += a.c_a;
  if (ta >= a.th) { ta -= a.th; ++oc; }
  oc += a.c_oc;
}

// class dgrad A: W[g*ocg + oc][o][rkh + sh*ta][rkw + sw*tb], k = (oc, ta, tb)
struct CurWc {
  uint32_t oc, ta, tb, o, k;
  bool ok;
  __device__ void init(const ConvArgs& a, uint32_t, uint32_t o_, uint32_t k0) {
    ok = o_ < a.M;
    o = ok ? o_ : 0;
    k = k0;
    oc = fdiv(k0, a.f_tt);
    const uint32_t t = k0 - oc * (a.th * a.tw);
    ta = fdiv(t, a.f_tw);
    tb = t - ta * a.tw;
  }
  __device__ float get(const ConvArgs& a, uint32_t kend, uint32_t g) const {
    if (!ok || k >= kend) return 0.f;
    const uint32_t khi = a.rkh + a.sh * ta, kwi = a.rkw + a.sw * tb;
    return a.wt[((g * a.ocg + oc) * a.cg + o) * a.kk + khi * a.kw + kwi];
  }
  __device__ void next(const ConvArgs& a) { k += BK; step_class_taps(a, oc, ta, tb); }
};

// class dgrad B: dy[n][g*ocg + oc][qy + oyc - ta][qx + oxc - tb] for the
// class pixel j = (n*qh + qy)*qw + qx
struct CurDyc {
  uint32_t base, oc, ta, tb, k;
  int oy0, ox0;
  bool ok;
  __device__ void init(const ConvArgs& a, uint32_t g, uint32_t j, uint32_t k0) {
    ok = j < a.N;
    const uint32_t jj = ok ? j : 0;
    const uint32_t n = fdiv(jj, a.f_qq), q = jj - n * (a.qh * a.qw);
    const uint32_t qy = fdiv(q, a.f_qw), qx = q - qy * a.qw;
    base = (n * a.oc + g * a.ocg) * a.oh * a.ow;
    oy0 = (int)(qy + a.oyc);
    ox0 = (int)(qx + a.oxc);
    k = k0;
    oc = fdiv(k0, a.f_tt);
    const uint32_t t = k0 - oc * (a.th * a.tw);
    ta = fdiv(t, a.f_tw);
    tb = t - ta * a.tw;
  }
  __device__ float get(const ConvArgs& a, uint32_t kend) const {
    if (!ok || k >= kend) return 0.f;
    const int oy = oy0 - (int)ta, ox = ox0 - (int)tb;
    if (oy < 0 || oy >= (int)a.oh || ox < 0 || ox >= (int)a.ow) return 0.f;
    return a.dy[base + (oc * a.oh + (uint32_t)oy) * a.ow + (uint32_t)ox];
  }
  __device__ void next(const ConvArgs& a) { k += BK; step_class_taps(a, oc, ta, tb); }
};

// Uniform access to the cursors of each product.
template <int MODE> struct Ops;
template <> struct Ops<kFwd> {
  typedef CurW A;
  typedef CurXf B;
  __device__ static float ga(const A& c, const ConvArgs& a, uint32_t kend, uint32_t) { return c.get(a, kend); }
  __device__ static float gb(const B& c, const ConvArgs& a, uint32_t kend) { return c.get(a, kend); }
};
template <> struct Ops<kDgrad> {
  typedef CurWt A;
  typedef CurDy B;
  __device__ static float ga(const A& c, const ConvArgs& a, uint32_t kend, uint32_t g) { return c.get(a, kend, g); }
  __device__ static float gb(const B& c, const ConvArgs& a, uint32_t kend) { return c.get(a, kend); }
};
template <> struct Ops<kDgradClass> {
  typedef CurWc A;
  typedef CurDyc B;
  __device__ static float ga(const A& c, const ConvArgs& a, uint32_t kend, uint32_t g) { return c.get(a, kend, g); }
  __device__ static float gb(const B& c, const ConvArgs& a, uint32_t kend) { return c.get(a, kend); }
};
template <> struct Ops<kWgrad> {
  typedef CurDyRow A;
  typedef CurXw B;
  __device__ static float ga(const A& c, const ConvArgs& a, uint32_t kend, uint32_t g) { return c.get(a, kend, g); }
  __device__ static float gb(const B& c, const ConvArgs& a, uint32_t kend) { return c.get(a, kend); }
};

// Lane -> (o, k) of an OUTER x BK operand tile.  K_FAST: consecutive lanes
// take consecutive k (operands contiguous along k); otherwise consecutive o.
template <bool K_FAST, int OUTER>
__device__ __forceinline__ void tile_pos(int idx, uint32_t& o, uint32_t& k) {
  if (K_FAST) {
    o = idx / BK;
    k = idx % BK;
  } else {
    o = idx % OUTER;
    k = idx / OUTER;
  }
}

// The fields of one stride class written into a.
__device__ __forceinline__ void apply_class(ConvArgs& a, const ClassArgs& c) {
  a.ry = c.ry; a.rx = c.rx; a.rkh = c.rkh; a.rkw = c.rkw; a.th = c.th; a.tw = c.tw;
  a.oyc = c.oyc; a.oxc = c.oxc; a.qh = c.qh; a.qw = c.qw;
  a.c_oc = c.c_oc; a.c_a = c.c_a; a.c_b = c.c_b; a.N = c.N; a.K = c.K;
  a.f_tt = c.f_tt; a.f_tw = c.f_tw; a.f_qq = c.f_qq; a.f_qw = c.f_qw;
}

template <int MODE, int BM, int BN>
__global__ __launch_bounds__(kThreads, 2) void k_conv_igemm(ConvArgs a0, ClassSet cs) {
  // class dgrad: grid row y is a stride class (these launches never split K)
  ConvArgs a = a0;
  if (MODE == kDgradClass) apply_class(a, cs.c[blockIdx.y]);
  constexpr int WGM = BM / 32, WGN = BN / 32;  // wave grid
  static_assert(WGM * WGN == 4, "four waves of 32x32");
  constexpr int LA = BM + 4, LB = BN + 4;
  constexpr int EA = BM * BK / kThreads, EB = BN * BK / kThreads;  // elements per lane
  constexpr bool A_KFAST = true, B_KFAST = (MODE == kWgrad);
  __shared__ float As[2][BK * LA];
  __shared__ float Bs[2][BK * LB];

  const uint32_t g = blockIdx.z;
  const uint32_t tile = blockIdx.x;
  const uint32_t tm = tile % a.tiles_m, tn = tile / a.tiles_m;
  const uint32_t m0 = tm * BM, n0 = tn * BN;
  if (MODE == kDgradClass && n0 >= a.N) return;  // a smaller class's grid row
  const uint32_t kbeg = MODE == kDgradClass ? 0u : blockIdx.y * a.kchunk;
  const uint32_t kend = kbeg + a.kchunk < a.K ? kbeg + a.kchunk : a.K;
  const uint32_t ktiles = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;

  const int t = threadIdx.x;
  const int lane = t & 63, wid = t >> 6;
  const int wm = wid / WGN, wn = wid % WGN;
  const int l32 = lane & 31, h = lane >> 5;

  floatx16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;

  // cursors of the positions this lane stages, and their LDS slots
  typename Ops<MODE>::A ca[EA];
  typename Ops<MODE>::B cb[EB];
  uint32_t sa[EA], sb[EB];
#pragma unroll
  for (int i = 0; i < EA; ++i) {
    uint32_t o, k;
    tile_pos<A_KFAST, BM>(t + kThreads * i, o, k);
    ca[i].init(a, g, m0 + o, kbeg + k);
    sa[i] = k * LA + o;
  }
#pragma unroll
  for (int i = 0; i < EB; ++i) {
    uint32_t o, k;
    tile_pos<B_KFAST, BN>(t + kThreads * i, o, k);
    cb[i].init(a, g, n0 + o, kbeg + k);
    sb[i] = k * LB + o;
  }
  // two register sets, so a step's gathers are issued two steps before its
  // elements are written to LDS (the cursors always hold the next step)
  float ra0[EA], rb0[EB], ra1[EA], rb1[EB];
  auto fetch = [&](float (&ra)[EA], float (&rb)[EB]) {
#pragma unroll
    for (int i = 0; i < EA; ++i) {
      ra[i] = Ops<MODE>::ga(ca[i], a, kend, g);
      ca[i].next(a);
    }
#pragma unroll
    for (int i = 0; i < EB; ++i) {
      rb[i] = Ops<MODE>::gb(cb[i], a, kend);
      cb[i].next(a);
    }
  };
  auto stage = [&](int s, const float (&ra)[EA], const float (&rb)[EB]) {
#pragma unroll
    for (int i = 0; i < EA; ++i) As[s][sa[i]] = ra[i];
#pragma unroll
    for (int i = 0; i < EB; ++i) Bs[s][sb[i]] = rb[i];
  };
  auto compute = [&](int cur) {
    const float* as = As[cur] + wm * 32 + l32;
    const float* bs = Bs[cur] + wn * 32 + l32;
#pragma unroll
    for (int kk = 0; kk < BK; kk += 2)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(as[(kk + h) * LA], bs[(kk + h) * LB], acc, 0, 0, 0);
  };

  if (ktiles > 0) {
    fetch(ra0, rb0);
    stage(0, ra0, rb0);
  }
  __syncthreads();
  // wgrad with a bias gradient: the first column tile's workgroups also sum
  // the rows of their dy tiles (db[oc] = sum over images and pixels of dy),
  // compensated, RKPT k values per lane and K step
  constexpr int RKPT = BK * BM / kThreads;
  const bool row_sums = MODE == kWgrad && a.db != nullptr && tn == 0;
  Kahan rsum;
  for (uint32_t kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < ktiles;
    if (more) fetch(ra0, rb0);
    compute(cur);
    if (row_sums) {
      const int rm = t % BM, rk = (t / BM) * RKPT;
#pragma unroll
      for (int i = 0; i < RKPT; ++i) rsum.add(As[cur][(rk + i) * LA + rm]);
    }
    if (more) stage(cur ^ 1, ra0, rb0);
    __syncthreads();
  }
  if (MODE == kWgrad && row_sums) {
    // lanes t, t + BM, ... hold slices of row t: combined in that order (the
    // staging tiles are free: the K loop ended on a barrier)
    float* rpart = As[0];
    rpart[t] = rsum.s;
    __syncthreads();
    const uint32_t row = m0 + (uint32_t)t;
    if (t < BM && row < a.M) {
      float v = 0.f;
#pragma unroll
      for (int q = 0; q < kThreads / BM; ++q) v += rpart[t + q * BM];
      if (a.rsw) {
        a.rsw[((size_t)g * gridDim.y + blockIdx.y) * a.M + row] = v;
      } else {
        float* o = a.db + g * a.ocg + row;
        *o = a.accumulate ? *o + v : v;
      }
    }
  }

  // epilogue: accumulator register r of lane (l32, h) holds tile row
  // 8*(r/4) + 4*h + r%4 and column l32 of this wave's 32x32 block
  const uint32_t col = n0 + wn * 32 + l32;
  if (col >= a.N) return;
  const uint32_t P = a.oh * a.ow, HW = a.h * a.w;
  uint32_t n_img = 0, pix = 0;
  if (MODE == kFwd) {
    n_img = fdiv(col, a.f_p);
    pix = col - n_img * P;
  } else if (MODE == kDgrad) {
    n_img = fdiv(col, a.f_hw);
    pix = col - n_img * HW;
  } else if (MODE == kDgradClass) {
    n_img = fdiv(col, a.f_qq);
    const uint32_t q = col - n_img * (a.qh * a.qw);
    const uint32_t qy = fdiv(q, a.f_qw), qx = q - qy * a.qw;
    pix = (a.ry + a.sh * qy) * a.w + a.rx + a.sw * qx;
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const uint32_t row = m0 + wm * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
    if (row >= a.M) continue;
    const float v = acc[r];
    if (MODE == kFwd) {
      const uint32_t oc = g * a.ocg + row;
      const float o = a.bias ? v + a.bias[oc] : v;
      a.out[(n_img * a.oc + oc) * P + pix] = a.relu ? fmaxf(o, 0.0f) : o;  // the library's ReLU
    } else if (MODE == kDgrad || MODE == kDgradClass) {
      a.out[(n_img * a.c + g * a.cg + row) * HW + pix] = v;
    } else if (a.ws) {
      a.ws[(((size_t)g * gridDim.y + blockIdx.y) * a.M + row) * a.N + col] = v;
    } else {
      float* o = a.out + (g * a.ocg + row) * a.N + col;
      *o = a.accumulate ? *o + v : v;
    }
  }
}

struct TileCfg {
  int bm, bn;
};
constexpr TileCfg kCfgs[3] = {{32, 128}, {64, 64}, {128, 32}};

// The tile with the least padded M x N work (64x64 on ties).
int choose_cfg(uint32_t M, uint32_t N) {
  int best = 1;
  uint64_t best_area = ~0ull;
  for (int i : {1, 0, 2}) {
    const uint64_t area = (uint64_t)cdiv(M, kCfgs[i].bm) * kCfgs[i].bm *
                          ((uint64_t)cdiv(N, kCfgs[i].bn) * kCfgs[i].bn);
    if (area < best_area) {
      best_area = area;
      best = i;
    }
  }
  return best;
}

template <int MODE>
void launch_cfg(int cfg, const ConvArgs& a, const ClassSet& cs, dim3 grid) {
  if (cfg == 0)
    tjh_launch((k_conv_igemm<MODE, 32, 128>), grid, dim3(kThreads), 0, stream(), a, cs);
  else if (cfg == 1)
    tjh_launch((k_conv_igemm<MODE, 64, 64>), grid, dim3(kThreads), 0, stream(), a, cs);
  else
    tjh_launch((k_conv_igemm<MODE, 128, 32>), grid, dim3(kThreads), 0, stream(), a, cs);
}

ConvArgs make_args(const tjh_conv2d_desc* d) {
  ConvArgs a{};
  a.n = (uint32_t)d->n; a.c = (uint32_t)d->c; a.h = (uint32_t)d->h; a.w = (uint32_t)d->w;
  a.oc = (uint32_t)d->oc; a.kh = (uint32_t)d->kh; a.kw = (uint32_t)d->kw;
  a.sh = (uint32_t)d->stride_h; a.sw = (uint32_t)d->stride_w;
  a.ph = (uint32_t)d->pad_h; a.pw = (uint32_t)d->pad_w;
  a.dh = (uint32_t)d->dil_h; a.dw = (uint32_t)d->dil_w;
  a.oh = (uint32_t)d->oh; a.ow = (uint32_t)d->ow;
  a.cg = (uint32_t)(d->c / d->groups); a.ocg = (uint32_t)(d->oc / d->groups);
  a.kk = a.kh * a.kw;
  a.f_kk = make_fastdiv(a.kk); a.f_kw = make_fastdiv(a.kw);
  a.f_p = make_fastdiv(a.oh * a.ow); a.f_ow = make_fastdiv(a.ow);
  a.f_hw = make_fastdiv(a.h * a.w); a.f_w = make_fastdiv(a.w);
  a.f_sh = make_fastdiv(a.sh); a.f_sw = make_fastdiv(a.sw);
  a.s_c = BK / a.kk;
  a.s_kh = (BK % a.kk) / a.kw;
  a.s_kw = (BK % a.kk) % a.kw;
  a.s_oy = BK / a.ow;
  a.s_ox = BK % a.ow;
  return a;
}

// One implicit-GEMM launch of `mode` over all groups; wgrad splits K when
// the output tiles alone cannot fill the CUs.
int run_conv(int mode, ConvArgs a, int64_t groups, const ClassSet* cs = nullptr,
             int nclass = 1) {
  if (a.M == 0 || a.N == 0) return TJH_OK;
  const int cfg = choose_cfg(a.M, a.N);
  a.tiles_m = (uint32_t)cdiv(a.M, kCfgs[cfg].bm);
  const int64_t tiles = (int64_t)a.tiles_m * cdiv(a.N, kCfgs[cfg].bn);
  int64_t splits = 1;
  if (mode == kWgrad) {
    const int cus = num_cus() > 0 ? num_cus() : 256;
    const int64_t want = cdiv(4LL * cus, tiles * groups);
    const int64_t by_k = a.K / 128;  // at least 128 of K per split
    splits = want < by_k ? want : by_k;
    if (splits < 1) splits = 1;
    if (splits > 1024) splits = 1024;
  }
  a.kchunk = a.K > 0 ? (uint32_t)(cdiv(cdiv(a.K, splits), BK) * BK) : BK;
  splits = a.K > 0 ? cdiv(a.K, a.kchunk) : 1;  // K = 0: one pass writes zeros
  const int64_t rs_len = (mode == kWgrad && a.db) ? groups * splits * a.M : 0;
  Scratch ws(splits > 1 ? (size_t)(groups * splits * a.M * a.N + rs_len) * sizeof(float) : 0);
  if (splits > 1 && !ws.ok()) return set_error(TJH_ERR_OOM, "conv2d: no split-K scratch");
  a.ws = splits > 1 ? ws.as<float>() : nullptr;
  a.rsw = (splits > 1 && rs_len) ? ws.as<float>() + groups * splits * a.M * a.N : nullptr;
  TJH_ARG(tiles < (int64_t(1) << 31) && groups <= 65535, "conv2d: grid too large");
  const dim3 grid((unsigned)tiles, (unsigned)(mode == kDgradClass ? nclass : splits),
                  (unsigned)groups);
  const ClassSet none{};
  if (mode == kFwd) launch_cfg<kFwd>(cfg, a, none, grid);
  else if (mode == kDgrad) launch_cfg<kDgrad>(cfg, a, none, grid);
  else if (mode == kDgradClass) launch_cfg<kDgradClass>(cfg, a, *cs, grid);
  else launch_cfg<kWgrad>(cfg, a, none, grid);
  int rc = check_launch("conv2d_igemm");
  if (rc != TJH_OK || splits == 1) return rc;
  // dW[g] (+)= the splits' partial rows summed in split order (compensated),
  // and db[g] (+)= the splits' partial row sums, in one launch
  const int64_t mn = (int64_t)a.M * a.N;
  const int per = a.rsw ? 2 : 1;
  for (int64_t g0 = 0; g0 < groups; g0 += kFinalMax / per) {
    float* parts[kFinalMax];
    float* outs[kFinalMax];
    int64_t cols[kFinalMax];
    const int64_t ng = groups - g0 < kFinalMax / per ? groups - g0 : kFinalMax / per;
    int np = 0;
    for (int64_t i = 0; i < ng; ++i) {
      parts[np] = a.ws + (g0 + i) * splits * mn;
      outs[np] = a.out + (g0 + i) * mn;
      cols[np++] = mn;
      if (a.rsw) {
        parts[np] = a.rsw + (g0 + i) * splits * a.M;
        outs[np] = a.db + (g0 + i) * a.ocg;
        cols[np++] = a.M;
      }
    }
    rc = colsum_final_cols(parts, outs, cols, np, splits, a.accumulate, 1.0f);
    if (rc != TJH_OK) return rc;
  }
  return TJH_OK;
}

int check_desc(const tjh_conv2d_desc* d) {
  TJH_ARG(d, "conv2d: NULL descriptor");
  TJH_ARG(d->n >= 0 && d->c > 0 && d->h >= 0 && d->w >= 0 && d->oc > 0 && d->kh > 0 && d->kw > 0,
          "conv2d: bad sizes");
  TJH_ARG(d->stride_h > 0 && d->stride_w > 0 && d->dil_h > 0 && d->dil_w > 0 && d->pad_h >= 0 &&
              d->pad_w >= 0 && d->groups > 0,
          "conv2d: bad stride/dilation/padding/groups");
  TJH_ARG(d->c % d->groups == 0 && d->oc % d->groups == 0,
          "conv2d: channels (%lld in, %lld out) not divisible by groups %lld", (long long)d->c,
          (long long)d->oc, (long long)d->groups);
  int64_t oh = (d->h + 2 * d->pad_h - d->dil_h * (d->kh - 1) - 1) / d->stride_h + 1;
  int64_t ow = (d->w + 2 * d->pad_w - d->dil_w * (d->kw - 1) - 1) / d->stride_w + 1;
  TJH_ARG(oh == d->oh && ow == d->ow, "conv2d: output size %lldx%lld does not match %lldx%lld",
          (long long)d->oh, (long long)d->ow, (long long)oh, (long long)ow);
  TJH_ARG(oh > 0 && ow > 0, "conv2d: empty output");
  // 32-bit index arithmetic inside the kernels: every tensor and every
  // GEMM extent below 2^31 elements, padded coordinates below 2^31
  const int64_t lim = int64_t(1) << 31;
  const int64_t kk = d->kh * d->kw;
  TJH_ARG(d->n * d->c * d->h * d->w < lim && d->n * d->oc * oh * ow < lim &&
              d->oc * (d->c / d->groups) * kk < lim && d->n * oh * ow < lim &&
              d->n * d->h * d->w < lim && d->h + d->pad_h < lim / 2 && d->w + d->pad_w < lim / 2 &&
              oh * d->stride_h + d->kh * d->dil_h < lim / 2 &&
              ow * d->stride_w + d->kw * d->dil_w < lim / 2,
          "conv2d: sizes beyond this implementation's 32-bit indexing");
  return TJH_OK;
}

}  // namespace
}  // namespace tjh

using namespace tjh;

extern "C" {

int tjh_conv2d_forward(const tjh_conv2d_desc* d, const float* x, const float* w,
                       const float* bias, float* y) {
  return tjh_conv2d_forward_act(d, x, w, bias, y, 0);
}

int tjh_conv2d_forward_act(const tjh_conv2d_desc* d, const float* x, const float* w,
                           const float* bias, float* y, int act) {
  TJH_REQUIRE_INIT();
  TJH_ARG(act == 0 || act == 1, "tjh_conv2d_forward_act: bad activation %d", act);
  int rc = check_desc(d);
  if (rc != TJH_OK) return rc;
  if (d->n == 0) return TJH_OK;
  ConvArgs a = make_args(d);
  a.x = x; a.wt = w; a.bias = bias; a.out = y;
  a.relu = act;
  a.M = a.ocg;
  a.N = (uint32_t)(d->n * d->oh * d->ow);
  a.K = a.cg * a.kk;
  KernelScope ks("conv2d_fwd");
  return run_conv(kFwd, a, d->groups);
}

int tjh_conv2d_backward_input(const tjh_conv2d_desc* d, const float* dy, const float* w,
                              float* dx) {
  TJH_REQUIRE_INIT();
  int rc = check_desc(d);
  if (rc != TJH_OK) return rc;
  if (d->n == 0) return TJH_OK;
  ConvArgs a = make_args(d);
  a.dy = dy; a.wt = w; a.out = dx;
  a.M = a.cg;
  KernelScope ks("conv2d_dgrad");
  if (a.dh != 1 || a.dw != 1) {
    // dilated: every tap is a candidate, stride-skipped ones read as 0
    a.N = (uint32_t)(d->n * d->h * d->w);
    a.K = a.ocg * a.kk;
    return run_conv(kDgrad, a, d->groups);
  }
  // one exact GEMM per stride class of input pixels, up to kMaxClasses
  // classes per launch (one per grid row; the grid is sized for the
  // largest, the others' extra workgroups return at once)
  ClassSet cs{};
  int nc = 0;
  uint32_t maxN = 0, maxK = 0;
  auto flush = [&]() -> int {
    if (nc == 0) return TJH_OK;
    ConvArgs b = a;
    b.N = maxN;
    b.K = maxK;
    const int r = run_conv(kDgradClass, b, d->groups, &cs, nc);
    nc = 0;
    maxN = maxK = 0;
    return r;
  };
  for (uint32_t ry = 0; ry < a.sh && ry < a.h; ++ry) {
    for (uint32_t rx = 0; rx < a.sw && rx < a.w; ++rx) {
      ClassArgs& b = cs.c[nc];
      b = ClassArgs{};
      b.ry = ry; b.rx = rx;
      b.rkh = (ry + a.ph) % a.sh;
      b.rkw = (rx + a.pw) % a.sw;
      b.th = a.kh > b.rkh ? (a.kh - b.rkh + a.sh - 1) / a.sh : 0;
      b.tw = a.kw > b.rkw ? (a.kw - b.rkw + a.sw - 1) / a.sw : 0;
      b.oyc = (ry + a.ph - b.rkh) / a.sh;
      b.oxc = (rx + a.pw - b.rkw) / a.sw;
      b.qh = (a.h - ry + a.sh - 1) / a.sh;
      b.qw = (a.w - rx + a.sw - 1) / a.sw;
      const uint32_t tt = b.th * b.tw;
      b.f_tt = make_fastdiv(tt > 0 ? tt : 1);
      b.f_tw = make_fastdiv(b.tw > 0 ? b.tw : 1);
      b.f_qq = make_fastdiv(b.qh * b.qw);
      b.f_qw = make_fastdiv(b.qw);
      if (tt > 0) {
        b.c_oc = BK / tt;
        b.c_a = (BK % tt) / b.tw;
        b.c_b = (BK % tt) % b.tw;
      }
      b.N = (uint32_t)d->n * b.qh * b.qw;
      b.K = a.ocg * tt;
      if (b.N > maxN) maxN = b.N;
      if (b.K > maxK) maxK = b.K;
      if (++nc == kMaxClasses) {
        rc = flush();
        if (rc != TJH_OK) return rc;
      }
    }
  }
  return flush();
}

int tjh_conv2d_backward_weight_bias(const tjh_conv2d_desc* d, const float* dy, const float* x,
                                    float* dw, float* db, int accumulate) {
  TJH_REQUIRE_INIT();
  int rc = check_desc(d);
  if (rc != TJH_OK) return rc;
  const int64_t cg = d->c / d->groups, kk = d->kh * d->kw;
  if (d->n == 0) {
    if (accumulate) return TJH_OK;
    rc = tjh_fill_f32(dw, d->oc * cg * kk, 0.f);
    if (rc == TJH_OK && db) rc = tjh_fill_f32(db, d->oc, 0.f);
    return rc;
  }
  ConvArgs a = make_args(d);
  a.dy = dy; a.x = x; a.out = dw; a.db = db; a.accumulate = accumulate ? 1 : 0;
  a.M = a.ocg;
  a.N = a.cg * a.kk;
  a.K = (uint32_t)(d->n * d->oh * d->ow);
  KernelScope ks("conv2d_wgrad");
  return run_conv(kWgrad, a, d->groups);
}

int tjh_conv2d_backward_weight(const tjh_conv2d_desc* d, const float* dy, const float* x,
                               float* dw, int accumulate) {
  return tjh_conv2d_backward_weight_bias(d, dy, x, dw, nullptr, accumulate);
}

}  // extern "C"
