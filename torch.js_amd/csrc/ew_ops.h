// Scalar definitions of the elementwise op codes of the ABI (TJH_UNARY_*,
// TJH_BINARY_*, TJH_SCALAR_*, TJH_TERNARY_*, comparisons), shared by the
// elementwise kernels and the fused expression evaluator so that both
// compute every op with the same instructions.
#pragma once

#include "ops_math.h"
#include "torchjs_hip.h"

namespace tjh {

__device__ __forceinline__ float unary_f(int op, float x, float alpha) {
  switch (op) {
    case TJH_UNARY_NEG: return -x;
    case TJH_UNARY_EXP: return expf(x);
    case TJH_UNARY_LOG: return logf(x);
    case TJH_UNARY_SQRT: return sqrtf(x);
    case TJH_UNARY_RSQRT: return 1.0f / sqrtf(x);
    case TJH_UNARY_TANH: return tanhf(x);
    case TJH_UNARY_SIGMOID: return sigmoid_f(x);
    case TJH_UNARY_RELU: return fmaxf(x, 0.0f);
    case TJH_UNARY_GELU: return gelu_f(x);
    case TJH_UNARY_SQUARE: return x * x;
    case TJH_UNARY_RECIPROCAL: return 1.0f / x;
    case TJH_UNARY_ERF: return erf_as(x);
    case TJH_UNARY_ABS: return fabsf(x);
    case TJH_UNARY_SIN: return sinf(x);
    case TJH_UNARY_COS: return cosf(x);
    case TJH_UNARY_SILU: return x * sigmoid_f(x);
    case TJH_UNARY_LEAKY_RELU: return x > 0.f ? x : alpha * x;
    case TJH_UNARY_ELU: return x > 0.f ? x : alpha * (expf(x) - 1.0f);
    case TJH_UNARY_SOFTPLUS: return x > 20.f ? x : log1pf(expf(x));
    case TJH_UNARY_SIGN: return (float)((x > 0.f) - (x < 0.f));
    default: return 0.f;
  }
}

// g * d op(x)/dx, using the saved output y where that is cheaper.
__device__ __forceinline__ float unary_bwd_f(int op, float g, float x, float y,
                                             float alpha) {
  switch (op) {
    case TJH_UNARY_NEG: return -g;
    case TJH_UNARY_EXP: return g * y;
    case TJH_UNARY_LOG: return g / x;
    case TJH_UNARY_SQRT: return g * 0.5f / y;
    case TJH_UNARY_RSQRT: return g * -0.5f * y * y * y;
    case TJH_UNARY_TANH: return g * (1.0f - y * y);
    case TJH_UNARY_SIGMOID: return g * y * (1.0f - y);
    case TJH_UNARY_RELU: return x > 0.f ? g : 0.0f;
    case TJH_UNARY_GELU: return g * gelu_grad(x);
    case TJH_UNARY_SQUARE: return g * 2.0f * x;
    case TJH_UNARY_RECIPROCAL: return -g * y * y;
    case TJH_UNARY_ERF: return g * 1.1283791670955126f * expf(-x * x);
    case TJH_UNARY_ABS: return g * (float)((x > 0.f) - (x < 0.f));
    case TJH_UNARY_SIN: return g * cosf(x);
    case TJH_UNARY_COS: return -g * sinf(x);
    case TJH_UNARY_SILU: {
      float s = sigmoid_f(x);
      return g * s * (1.0f + x * (1.0f - s));
    }
    case TJH_UNARY_LEAKY_RELU: return x > 0.f ? g : alpha * g;
    case TJH_UNARY_ELU: return x > 0.f ? g : g * alpha * expf(x);
    case TJH_UNARY_SOFTPLUS: return x > 20.f ? g : g * sigmoid_f(x);
    case TJH_UNARY_SIGN: return 0.0f;
    default: return 0.f;
  }
}

__device__ __forceinline__ float binary_f(int op, float a, float b) {
  switch (op) {
    case TJH_BINARY_ADD: return a + b;
    case TJH_BINARY_SUB: return a - b;
    case TJH_BINARY_MUL: return a * b;
    case TJH_BINARY_DIV: return a / b;
    case TJH_BINARY_POW: return powf(a, b);
    case TJH_BINARY_MAXIMUM: return (a != a || b != b) ? __builtin_nanf("") : fmaxf(a, b);
    case TJH_BINARY_MINIMUM: return (a != a || b != b) ? __builtin_nanf("") : fminf(a, b);
    default: return 0.f;
  }
}

// comparison ops: 0 eq 1 ne 2 lt 3 le 4 gt 5 ge
constexpr int kCmpBase = 100;
__device__ __forceinline__ float cmp_f(int op, float a, float b) {
  switch (op) {
    case 0: return a == b ? 1.f : 0.f;
    case 1: return a != b ? 1.f : 0.f;
    case 2: return a < b ? 1.f : 0.f;
    case 3: return a <= b ? 1.f : 0.f;
    case 4: return a > b ? 1.f : 0.f;
    case 5: return a >= b ? 1.f : 0.f;
    default: return 0.f;
  }
}

__device__ __forceinline__ float ternary_f(int op, float g, float a, float b) {
  switch (op) {
    case TJH_TERNARY_DIV_B: return -g * a / (b * b);
    case TJH_TERNARY_POW_A: return g * b * powf(a, b - 1.0f);
    case TJH_TERNARY_POW_B: return g * powf(a, b) * logf(a);
    case TJH_TERNARY_MUL3: return g * a * b;
    default: return 0.f;
  }
}

// alpha * x + y (tjh_axpy)
__device__ __forceinline__ float axpy_f(float alpha, float x, float y) { return alpha * x + y; }

__device__ __forceinline__ float scalar_f(int op, float x, float s) {
  switch (op) {
    case TJH_SCALAR_ADD: return x + s;
    case TJH_SCALAR_SUB: return x - s;
    case TJH_SCALAR_MUL: return x * s;
    case TJH_SCALAR_DIV: return x / s;
    case TJH_SCALAR_POW: return pow_js(x, s);
    case TJH_SCALAR_MAXIMUM: return fmaxf(x, s);
    case TJH_SCALAR_MINIMUM: return fminf(x, s);
    default: return 0.f;
  }
}
__device__ __forceinline__ float scalar_rev_f(int op, float x, float s) {
  switch (op) {
    case TJH_SCALAR_ADD: return s + x;
    case TJH_SCALAR_SUB: return s - x;
    case TJH_SCALAR_MUL: return s * x;
    case TJH_SCALAR_DIV: return s / x;
    case TJH_SCALAR_POW: return powf(s, x);
    case TJH_SCALAR_MAXIMUM: return fmaxf(s, x);
    case TJH_SCALAR_MINIMUM: return fminf(s, x);
    default: return 0.f;
  }
}

}  // namespace tjh
