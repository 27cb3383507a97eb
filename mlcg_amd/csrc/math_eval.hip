// Evaluation of the library's own elementary functions (common.h) on an
// array, so that their accuracy can be measured against fp64 on dense grids.
// The same inline functions run inside the filter, node and output kernels.
#include "common.h"

namespace {

__global__ void math_eval_kernel(int fn, const float* __restrict__ x, int64_t n,
                                 float* __restrict__ y) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float v = x[i];
    float out = 0.0f, s, c;
    switch (fn) {
      case MLCG_MATH_TANH: out = mlcg_tanh(v); break;
      case MLCG_MATH_SIGMOID: out = mlcg_sigmoid(v); break;
      case MLCG_MATH_SOFTPLUS: out = mlcg_softplus(v); break;
      case MLCG_MATH_SINPI: mlcg_sincospi(v, s, c); out = s; break;
      default: mlcg_sincospi(v, s, c); out = c; break;
    }
    y[i] = out;
  }
}

}  // namespace

extern "C" int mlcg_math_eval(int fn, const float* x, int64_t n, float* y, void* stream) {
  MLCG_REQUIRE(n >= 0 && fn >= MLCG_MATH_TANH && fn <= MLCG_MATH_COSPI);
  if (n == 0) return MLCG_OK;
  MLCG_REQUIRE(x && y);
  hipLaunchKernelGGL(math_eval_kernel, dim3(mlcg_persistent_groups(mlcg_div_up(n, 256), 8)),
                     dim3(256), 0, mlcg_stream(stream), fn, x, n, y);
  return mlcg_launch_status();
}
