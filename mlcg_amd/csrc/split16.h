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

typedef _Float16 halfx2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

// split2 of two values at once: both hi parts from one packed round-to-
// nearest-even conversion, and each lo part as fma(-hi, S, v S) rounded to
// fp16 once.  v S is exact (S is a power of two) and so is the fma's exact
// result (v - hi) S, so lo equals split2's fp16((v - hi) S) bit for bit; the
// fma takes hi straight from its fp16 half (a mixed-precision fma), which
// makes the pair cost five instructions instead of ten.
__device__ __forceinline__ void split2x2(float v0, float v1, float S, halfx2& hi, halfx2& lo) {
  asm("" : "+v"(v0), "+v"(v1));
  hi = __builtin_convertvector(floatx2{v0, v1}, halfx2);
  lo[0] = (_Float16)__builtin_fmaf(-(float)hi[0], S, v0 * S);
  lo[1] = (_Float16)__builtin_fmaf(-(float)hi[1], S, v1 * S);
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
// lanes, v_permlane16_swap / v_permlane32_swap across the four rows.  The
// arguments are magnitudes (non-negative floats, or NaN): their bit patterns
// order as unsigned integers, so the maxima are taken as v_max_u32 (one
// instruction per step with the DPP operand folded in; a float max would
// first quiet the moved operand), and a NaN, being the largest pattern,
// propagates instead of being dropped.
template <int kCtrl>
__device__ __forceinline__ unsigned dpp_umax(unsigned v) {
  return max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, kCtrl, 0xF, 0xF, false));
}
// max over the 16 lanes of each row, in every lane of the row
__device__ __forceinline__ float row16_max(float v) {
  unsigned u = __float_as_uint(v);
  u = dpp_umax<0xB1>(u);      // quad_perm [1, 0, 3, 2]
  u = dpp_umax<0x4E>(u);      // quad_perm [2, 3, 0, 1]
  u = dpp_umax<0x141>(u);     // row_half_mirror
  u = dpp_umax<0x140>(u);     // row_mirror
  return __uint_as_float(u);
}
// max over lanes l and l ^ 16, in both
__device__ __forceinline__ float pair_row_max(float v) {
  const unsigned u = __float_as_uint(v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __uint_as_float(max(a[0], a[1]));
}
// max over lanes l, l ^ 16, l ^ 32, l ^ 48, in each of them
__device__ __forceinline__ float cross_row_max(float v) {
  const unsigned u = __float_as_uint(pair_row_max(v));
  const auto b = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(max(b[0], b[1]));
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
