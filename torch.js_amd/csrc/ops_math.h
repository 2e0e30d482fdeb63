// Device-side scalar math shared by the elementwise, loss and optimizer
// kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace tjh {

// 1 - erf(a) for a >= 0 by Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7),
// the erf used by torch.js's WGSL (unary.wgsl:230-236).  The complement is
// formed directly as P(t)*exp(-a^2), so erf(x) = sign(x)*(1 - erfc_as(|x|))
// and 1 + erf(-a) = erfc_as(a) carry no cancellation.
__device__ __forceinline__ float erfc_as(float a) {
  float t = 1.0f / (1.0f + 0.3275911f * a);
  float p = ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t -
              0.284496736f) * t + 0.254829592f) * t;
  return p * expf(-a * a);
}

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

// d/dx GELU = Phi(x) + x*phi(x), phi the standard normal density.
__device__ __forceinline__ float gelu_grad(float x) {
  return phi_cdf(x) + x * 0.3989422804014327f * expf(-0.5f * x * x);
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
