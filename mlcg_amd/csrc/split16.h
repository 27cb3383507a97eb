// Helpers for fp32-accurate products on the fp16 MFMA and for lane
// reductions, shared by the filter and node kernels (gfx950).
//
// An fp32 operand x is carried as fp16 parts hi = fp16(x) and
// lo = fp16((x - hi) S), S = 2^e, which together hold about 22 significant
// bits.  A product is accumulated in fp32 as
//     S A B ~ (hi_A S) hi_B + hi_A lo_B + lo_A hi_B      (three MFMAs)
// so one side carries three planes (hi, hi S, lo S) and the other two
// (hi, lo S).  Operands of unknown size are first brought into [-4, 4) by a
// power of two (x3_norm), which is undone exactly on the fp32 result.
#pragma once

#include <hip/hip_runtime.h>

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef _Float16 halfx4 __attribute__((ext_vector_type(4)));

// The two fp16 parts of an fp32 operand, hi = fp16(v) and lo = fp16((v - hi)
// S), taken from one rounded fp32 value.  v is first made opaque to the
// optimiser: hipcc contracts floating-point expressions by default and has
// been seen to fold the product that computed v into one of the conversions
// only (a mixed-precision fma rounds the exact product straight to fp16, which
// can differ in the last bit from fp16 of the fp32-rounded product), and a hi
// that differs from the one lo was formed against leaves an uncompensated
// error of one fp16 ulp.  The empty asm emits no instruction.
struct f16split {
  _Float16 hi, lo;
};
__device__ __forceinline__ f16split split2(float v, float S) {
  asm("" : "+v"(v));
  const _Float16 hi = (_Float16)v;
  return f16split{hi, (_Float16)((v - (float)hi) * S)};
}

// sigma = 2^k with m sigma < 4: brings values of magnitude <= m into the
// range the split planes of an operand expect (sigma = 4 for m = 0).
__device__ __forceinline__ float x3_norm(float m) {
  int ex = 0;
  (void)frexpf(m, &ex);  // m < 2^ex (ex = 0 for 0)
  return ldexpf(1.0f, 2 - ex);
}

// 1 / x3_norm(m), exactly
__device__ __forceinline__ float x3_norm_inv(float m) {
  int ex = 0;
  (void)frexpf(m, &ex);
  return ldexpf(1.0f, ex - 2);
}

// Maxima across lanes without the LDS crossbar: DPP inside a row of 16
// lanes, v_permlane16_swap / v_permlane32_swap across the four rows.
template <int kCtrl>
__device__ __forceinline__ float dpp_fmax(float v) {
  return fmaxf(v, __int_as_float(
                      __builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, false)));
}
// max over the 16 lanes of each row, in every lane of the row
__device__ __forceinline__ float row16_max(float v) {
  v = dpp_fmax<0xB1>(v);      // quad_perm [1, 0, 3, 2]
  v = dpp_fmax<0x4E>(v);      // quad_perm [2, 3, 0, 1]
  v = dpp_fmax<0x141>(v);     // row_half_mirror
  return dpp_fmax<0x140>(v);  // row_mirror
}
// max over lanes l and l ^ 16, in both
__device__ __forceinline__ float pair_row_max(float v) {
  const auto a =
      __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
}
// max over lanes l, l ^ 16, l ^ 32, l ^ 48, in each of them
__device__ __forceinline__ float cross_row_max(float v) {
  v = pair_row_max(v);
  const auto b =
      __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Sums across lanes in the same fixed patterns (the result is the same on
// every run).
template <int kCtrl>
__device__ __forceinline__ float dpp_fadd(float v) {
  return v + __int_as_float(
                 __builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, false));
}
// sum over the 16 lanes of each row, in every lane of the row
__device__ __forceinline__ float row16_sum(float v) {
  v = dpp_fadd<0xB1>(v);      // quad_perm [1, 0, 3, 2]
  v = dpp_fadd<0x4E>(v);      // quad_perm [2, 3, 0, 1]
  v = dpp_fadd<0x141>(v);     // row_half_mirror
  return dpp_fadd<0x140>(v);  // row_mirror
}
// sum over the 32 lanes of each half-wave, in every lane of the half
__device__ __forceinline__ float half32_sum(float v) {
  v = row16_sum(v);
  const auto a =
      __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}
