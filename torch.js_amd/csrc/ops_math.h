// Device-side scalar math shared by the elementwise, loss and optimizer
// kernels.
#pragma once

// Runtime-compiled kernels (hipRTC) have the HIP device API built in.
#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>
#endif

namespace tjh {

// Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7), the erf used by
// torch.js's WGSL (unary.wgsl:230-236): 1 - erf(a) = P(t) exp(-a^2) for
// a >= 0, t = 1 / (1 + p a).  The reciprocal and the exponential use the
// hardware's v_rcp_f32 and v_exp_f32 (about 1 ulp each, far below the
// approximation's own error): the GEMM epilogues that apply GELU and GELU'
// to every output spend most of their time here.
__device__ __forceinline__ float erfc_poly(float a) {
  const float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * a);
  return ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t - 0.284496736f) * t +
          0.254829592f) * t;
}
// exp(-a^2) as 2^(-a^2 log2 e)
__device__ __forceinline__ float exp_neg_sq(float a) {
  return __builtin_amdgcn_exp2f(-(a * a) * 1.4426950408889634f);
}

// 1 - erf(a) for a >= 0.  The complement is formed directly, so
// erf(x) = sign(x)*(1 - erfc_as(|x|)) and 1 + erf(-a) = erfc_as(a) carry no
// cancellation.
__device__ __forceinline__ float erfc_as(float a) { return erfc_poly(a) * exp_neg_sq(a); }

__device__ __forceinline__ float erf_as(float x) {
  float y = 1.0f - erfc_as(fabsf(x));
  return x < 0.f ? -y : y;
}

// Phi(x) = 0.5 * (1 + erf(x / sqrt(2))) with the A&S erf above.
__device__ __forceinline__ float phi_cdf(float x) {
  float c = 0.5f * erfc_as(fabsf(x) * 0.7071067811865475f);
  return x < 0.f ? c : 1.0f - c;
}

// GELU(x) = 0.5*x*(1+erf(x/sqrt 2)) = x*Phi(x)   (unary.wgsl:246-252)
__device__ __forceinline__ float gelu_f(float x) { return x * phi_cdf(x); }

// d/dx GELU = Phi(x) + x*phi(x), phi the standard normal density; phi(x)
// and the erf term share e = exp(-x^2 / 2) (a = |x| / sqrt 2).
__device__ __forceinline__ float gelu_grad(float x) {
  const float a = fabsf(x) * 0.7071067811865475f;
  const float e = exp_neg_sq(a);
  const float c = 0.5f * erfc_poly(a) * e;
  const float cdf = x < 0.f ? c : 1.0f - c;
  return cdf + x * 0.3989422804014327f * e;
}

__device__ __forceinline__ float sigmoid_f(float x) {
  return 1.0f / (1.0f + expf(-x));
}

// pow with torch.js's rule for small non-negative integer exponents:
// repeated multiplication for exponents 0..10 (scalar.wgsl:53-66).
__device__ __forceinline__ float pow_js(float base, float e) {
  float r = rintf(e);
  if (fabsf(e - r) < 1e-6f && r >= 0.f && r <= 10.f) {
    int n = (int)r;
    float acc = 1.0f;
    for (int i = 0; i < n; ++i) acc *= base;
    return acc;
  }
  return powf(base, e);
}

}  // namespace tjh
