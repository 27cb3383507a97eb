// Shared helpers for the gfx950 kernels of libmlcg_hip.so.
//
// Every exported entry point is `extern "C"`, takes raw device pointers,
// sizes and a stream (passed as `void*`), launches on that stream and
// returns an mlcg_status code (see include/mlcg_hip.h).  No entry point
// allocates device memory or synchronises with the host.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mlcg_hip.h"

#define MLCG_WAVE 64

#define MLCG_REQUIRE(cond)                                                     \
  do {                                                                         \
    if (!(cond)) return MLCG_ERR_ARGUMENT;                                     \
  } while (0)

static inline int mlcg_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? MLCG_OK : MLCG_ERR_LAUNCH;
}

static inline hipStream_t mlcg_stream(void* s) {
  return reinterpret_cast<hipStream_t>(s);
}

static inline unsigned mlcg_div_up(int64_t a, int64_t b) {
  return (unsigned)((a + b - 1) / b);
}

// Number of workgroups that fills the chip several times for grid-stride
// loops: 256 CUs x `per_cu` resident groups.
static inline unsigned mlcg_persistent_groups(int64_t work_groups, int per_cu) {
  int64_t cap = 256LL * per_cu;
  if (work_groups < 1) work_groups = 1;
  return (unsigned)(work_groups < cap ? work_groups : cap);
}

__device__ __forceinline__ int mlcg_lane() { return threadIdx.x & (MLCG_WAVE - 1); }

// Device address of the library's numerics flag word on the current device
// (defined in filter.hip, read by mlcg_numerics_flags), or nullptr.
unsigned* mlcg_numerics_word_ptr();
constexpr unsigned kFlagTypeRange = 4u;  // bit 2: an atom type outside the table

// Sum across the 64 lanes of a wave (butterfly through ds_swizzle/dpp via
// __shfl_xor); every lane receives the total.
__device__ __forceinline__ float mlcg_wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, MLCG_WAVE);
  return v;
}

// Activation ids shared by the filter network, the interaction block and the
// output network (they are one module instance in StandardSchNet).
enum { MLCG_ACT_TANH = 0, MLCG_ACT_SSP = 1 };
// Cutoff ids for the RBF envelope and the CFConv envelope.
enum { MLCG_CUT_IDENTITY = 0, MLCG_CUT_COSINE = 1 };

// Elementary functions used per pair and per feature, written for this
// library on the hardware's exp2 / log2 / reciprocal instructions with
// polynomial parts fitted by weighted least squares (iterated towards equal
// ripple) to the target on the stated interval.  Measured in fp32 against
// fp64 over dense grids: tanh relative error <= 1.7e-7, sin(pi u) and
// cos(pi u) absolute error <= 2e-7 -- the size of fp32 rounding, far below
// the tolerances the filters and forces are held to.

// sin(pi u) and cos(pi u): u = k + f with k = rint(u), |f| <= 1/2, then
// sin(pi f) = f S(f^2), cos(pi f) = C(f^2) and the sign (-1)^k.
__device__ __forceinline__ void mlcg_sincospi(float u, float& s, float& c) {
  const float k = rintf(u);
  const float f = u - k;
  const float z = f * f;
  float ps = 0.07765979656518615f;
  ps = fmaf(ps, z, -0.5982923788083212f);
  ps = fmaf(ps, z, 2.550077700968031f);
  ps = fmaf(ps, z, -5.167710093195969f);
  ps = fmaf(ps, z, 3.1415926402373544f);
  float pc = -0.0243968021245328f;
  pc = fmaf(pc, z, 0.23493761798519963f);
  pc = fmaf(pc, z, -1.3352120714704687f);
  pc = fmaf(pc, z, 4.058709165964045f);
  pc = fmaf(pc, z, -4.934802137300611f);
  pc = fmaf(pc, z, 0.9999999997815456f);
  const float h = 0.5f * k;
  const float sg = h == rintf(h) ? 1.0f : -1.0f;  // (-1)^k, exact for any k
  s = f * ps * sg;
  c = pc * sg;
}

// tanh(x): x + x^3 T(x^2) for |x| < 0.625, else sign(x) (1 - 2 / (e^2|x| + 1)).
__device__ __forceinline__ float mlcg_tanh(float x) {
  const float ax = fabsf(x);
  const float z = x * x;
  float p = -0.00587577945524298f;
  p = fmaf(p, z, 0.02080220662361536f);
  p = fmaf(p, z, -0.05379347673240063f);
  p = fmaf(p, z, 0.13332141745110193f);
  p = fmaf(p, z, -0.33333310329858473f);
  const float small = fmaf(x * z, p, x);
  const float e = __builtin_amdgcn_exp2f(ax * 2.8853900817779268f);  // 2 / ln 2
  const float big = copysignf(fmaf(-2.0f, __builtin_amdgcn_rcpf(e + 1.0f), 1.0f), x);
  return ax < 0.625f ? small : big;
}

// 1 / (1 + e^-x)
__device__ __forceinline__ float mlcg_sigmoid(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

// log(1 + e^x) with torch's threshold (x above 20 returns x):
// max(x, 0) + log1p(y), y = e^-|x|, and log1p(y) = log(u) y / (u - 1) with
// u = 1 + y (exact for y below half an ulp of 1, where u - 1 = 0).
__device__ __forceinline__ float mlcg_softplus(float x) {
  const float y = __builtin_amdgcn_exp2f(-1.4426950408889634f * fabsf(x));
  const float u = 1.0f + y;
  const float d = u - 1.0f;
  const float l1p = d == 0.0f ? y : 0.6931471805599453f * __builtin_amdgcn_logf(u) * (y * __builtin_amdgcn_rcpf(d));
  return x > 20.0f ? x : fmaxf(x, 0.0f) + l1p;
}

// Activation value, first and second derivative.  Shifted softplus is
// softplus(x) - ln 2 with torch's threshold of 20 (softplus(x) = x above it).
__device__ __forceinline__ void mlcg_act(int act, float x, float& s, float& d1,
                                         float& d2) {
  if (act == MLCG_ACT_TANH) {
    s = mlcg_tanh(x);
    d1 = 1.0f - s * s;
    d2 = -2.0f * s * d1;
  } else {
    s = mlcg_softplus(x) - 0.69314718055994530942f;
    const float sg = mlcg_sigmoid(x);
    d1 = sg;
    d2 = sg * (1.0f - sg);
  }
}

__device__ __forceinline__ float mlcg_act_value(int act, float x) {
  if (act == MLCG_ACT_TANH) return mlcg_tanh(x);
  return mlcg_softplus(x) - 0.69314718055994530942f;
}

// Cutoff envelope and its derivative with respect to the distance.
// Cosine with lower == 0:  0.5 (cos(pi d / hi) + 1) [d < hi]
// Cosine with lower  > 0:  0.5 (cos(pi (2 (d - lo)/(hi - lo) + 1)) + 1) [lo < d < hi]
// (mlcg/nn/cutoff.py:110-153).
__device__ __forceinline__ void mlcg_cutoff(int kind, float lo, float hi, float d,
                                            float& c, float& dc) {
  const float pi = 3.14159265358979323846f;
  if (kind == MLCG_CUT_IDENTITY) {
    c = 1.0f;
    dc = 0.0f;
  } else if (lo > 0.0f) {
    const float iw = 1.0f / (hi - lo);
    float sn, cs;
    mlcg_sincospi(2.0f * (d - lo) * iw + 1.0f, sn, cs);
    const float m = (d < hi && d > lo) ? 1.0f : 0.0f;
    c = 0.5f * (cs + 1.0f) * m;
    dc = -sn * (pi * iw) * m;
  } else {
    const float ih = 1.0f / hi;
    float sn, cs;
    mlcg_sincospi(d * ih, sn, cs);
    const float m = d < hi ? 1.0f : 0.0f;
    c = 0.5f * (cs + 1.0f) * m;
    dc = -0.5f * sn * (pi * ih) * m;
  }
}
