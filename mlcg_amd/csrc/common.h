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

// Activation value, first and second derivative.  Shifted softplus is
// softplus(x) - ln 2 with torch's threshold of 20 (softplus(x) = x above it).
__device__ __forceinline__ void mlcg_act(int act, float x, float& s, float& d1,
                                         float& d2) {
  if (act == MLCG_ACT_TANH) {
    s = tanhf(x);
    d1 = 1.0f - s * s;
    d2 = -2.0f * s * d1;
  } else {
    float sp = x > 20.0f ? x : log1pf(expf(x));
    s = sp - 0.69314718055994530942f;
    float sg = 1.0f / (1.0f + expf(-x));
    d1 = sg;
    d2 = sg * (1.0f - sg);
  }
}

__device__ __forceinline__ float mlcg_act_value(int act, float x) {
  if (act == MLCG_ACT_TANH) return tanhf(x);
  float sp = x > 20.0f ? x : log1pf(expf(x));
  return sp - 0.69314718055994530942f;
}

// Cutoff envelope and its derivative with respect to the distance.
// Cosine with lower == 0:  0.5 (cos(pi d / hi) + 1) [d < hi]
// Cosine with lower  > 0:  0.5 (cos(pi (2 (d - lo)/(hi - lo) + 1)) + 1) [lo < d < hi]
// (mlcg/nn/cutoff.py:110-153).  cos(pi u) and sin(pi u) come from sincospif,
// whose argument reduction is exact and cheap (no large-argument path).
__device__ __forceinline__ void mlcg_cutoff(int kind, float lo, float hi, float d,
                                            float& c, float& dc) {
  const float pi = 3.14159265358979323846f;
  if (kind == MLCG_CUT_IDENTITY) {
    c = 1.0f;
    dc = 0.0f;
  } else if (lo > 0.0f) {
    float w = hi - lo;
    float sn, cs;
    sincospif(2.0f * (d - lo) / w + 1.0f, &sn, &cs);
    float m = (d < hi && d > lo) ? 1.0f : 0.0f;
    c = 0.5f * (cs + 1.0f) * m;
    dc = -0.5f * sn * (2.0f * pi / w) * m;
  } else {
    float sn, cs;
    sincospif(d / hi, &sn, &cs);
    float m = d < hi ? 1.0f : 0.0f;
    c = 0.5f * (cs + 1.0f) * m;
    dc = -0.5f * sn * (pi / hi) * m;
  }
}
