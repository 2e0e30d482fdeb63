// Wavefront-64 reductions through the DPP network (no LDS traffic): xor 1
// and xor 2 within quads, rotations by 4 and 8 within 16-lane rows (after
// which every lane of a row holds the row's result), and the four row
// results read as scalars.  readlane moves 32-bit words, so floats are
// bit-cast, never converted.  Every lane gets the same value, combined in
// a fixed order, so a result is the same on every run.
#pragma once

#include <hip/hip_runtime.h>

namespace tjh {

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

constexpr int kDppXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppRor4 = 0x124; // row_ror:4
constexpr int kDppRor8 = 0x128; // row_ror:8

// Combination of v over each 16-lane row (lanes 16k .. 16k + 15), in every
// lane of the row.
template <class C>
__device__ __forceinline__ float row16_reduce(float v, C comb) {
  v = comb(v, dpp_f<kDppXor1>(v));
  v = comb(v, dpp_f<kDppXor2>(v));
  v = comb(v, dpp_f<kDppRor4>(v));
  v = comb(v, dpp_f<kDppRor8>(v));
  return v;
}

// Combination of v over the wave, in every lane.
template <class C>
__device__ __forceinline__ float wave_reduce_dpp(float v, C comb) {
  v = row16_reduce(v, comb);
  return comb(comb(lane_f(v, 0), lane_f(v, 16)), comb(lane_f(v, 32), lane_f(v, 48)));
}

struct AddOp {
  __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};
struct MaxOp {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

__device__ __forceinline__ float wave_sum(float v) { return wave_reduce_dpp(v, AddOp{}); }
__device__ __forceinline__ float wave_max(float v) { return wave_reduce_dpp(v, MaxOp{}); }
__device__ __forceinline__ float row16_sum(float v) { return row16_reduce(v, AddOp{}); }

}  // namespace tjh
