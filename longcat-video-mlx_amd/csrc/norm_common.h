// Row-normalisation helpers shared by the fused pre-BSA pass and the DiT
// block's row kernels: exact sums across lane groups, products rounded once,
// and the two-step rounding (fp32, then the tensor dtype) of the reference's
// fp32 op followed by a cast.  Including this header turns off floating-point
// contraction for the rest of the translation unit: every product and sum is
// rounded on its own, as the reference's separate tensor operations are.
#pragma once

#include "bsa_common.h"

#pragma clang fp contract(off)

namespace lcv {

// Lane exchange inside a row of 16 lanes (DPP): quad_perm [1,0,3,2] and
// [2,3,0,1] swap neighbours and pairs, row_half_mirror (0x141) maps lane i of
// each 8 to 7-i, row_mirror (0x140) lane i of each 16 to 15-i.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}

// Sum over aligned groups of L lanes (8 or 16), every lane getting the same
// bits: each step adds a value from a lane of the partner group whose sums
// already agree, so the additions pair the same operands in every lane.
template <int L>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp<0xb1>(v);
  v += dpp<0x4e>(v);
  v += dpp<0x141>(v);
  if constexpr (L == 16) v += dpp<0x140>(v);
  return v;
}

// a * b rounded once, written as fma(a, b, -0) so a 16-bit operand widened
// just before feeds the mixed-precision FMA (v_fma_mix_f32) with no separate
// conversion; -0 keeps the sign of a zero product.  The -0 (and the 1 of
// acc + o as fma(o, 1, acc)) come from the kernel arguments: as literals the
// compiler would fold the FMA back into a plain multiply or add.
__device__ __forceinline__ float mul1(float a, float b, float neg_zero) { return __builtin_fmaf(a, b, neg_zero); }

// Round an fp32 result to T in two steps, as the reference's fp32 op followed
// by a cast does: the empty asm pins the fp32 value, so the compiler cannot
// fold the conversion into the producing FMA (v_fma_mixlo_f16 rounds the
// exact result to f16 once, which differs when the fp32 value is a tie).
template <typename T>
__device__ __forceinline__ T round_from_f32(float v) {
  asm("" : "+v"(v));
  return from_f32<T>(v);
}

// RMSNorm_FP32's output: round(x * rs) to T, times the weight, rounded to T
// (an exact product of two T values rounded once, so fp16 uses the packed
// fp16 multiply).
template <typename T>
__device__ __forceinline__ void norm_scale(const float* x, float rs, u32x4 wr, float nz, float* y);

template <>
__device__ __forceinline__ void norm_scale<f16>(const float* x, float rs, u32x4 wr, float nz, float* y) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t wm = wr[m];  // bit-cast a scalar copy, not the vector element
    const h2 xn = {round_from_f32<f16>(mul1(x[2 * m], rs, nz)), round_from_f32<f16>(mul1(x[2 * m + 1], rs, nz))};
    const h2 p = xn * __builtin_bit_cast(h2, wm);
    y[2 * m] = (float)p[0];
    y[2 * m + 1] = (float)p[1];
  }
}

template <>
__device__ __forceinline__ void norm_scale<bf16>(const float* x, float rs, u32x4 wr, float nz, float* y) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t wm = wr[m];
    const float w0 = __builtin_bit_cast(float, wm << 16), w1 = __builtin_bit_cast(float, wm & 0xffff0000u);
    y[2 * m] = to_f32(round_from_f32<bf16>(mul1(to_f32(round_from_f32<bf16>(mul1(x[2 * m], rs, nz))), w0, nz)));
    y[2 * m + 1] =
        to_f32(round_from_f32<bf16>(mul1(to_f32(round_from_f32<bf16>(mul1(x[2 * m + 1], rs, nz))), w1, nz)));
  }
}

// Sum over the 64 lanes of a wave (butterfly; every lane gets the same bits).
__device__ __forceinline__ float wave_sum(float v) {
  v = group_sum<16>(v);
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

}  // namespace lcv
