// The force-matching loss of the training step: mean squared error of two
// fp32 arrays (mlcg/nn/losses.py ForceMSE, torch's mse_loss with reduction
// "mean") and its gradient with respect to the prediction.
//
// Forward: each workgroup sums (x - y)^2 over one chunk of 64 Ki elements
// (every thread a strided part, float4 loads eight in flight when the arrays
// are 16-byte aligned, then a fixed butterfly over the wave and the waves in
// order); with one chunk the workgroup writes the mean itself, otherwise
// its partial sum, which mse_final_kernel adds in workgroup order.  Backward: grad_x = (norm (x - y)) g with norm = 2 / n as
// a float, the same expression and order as torch's mse_loss backward, so
// the gradient is the same bit for bit.
#include "common.h"

namespace {

constexpr int kMseThreads = 512;
constexpr int64_t kMseChunk = 65536;  // elements per workgroup

__device__ __forceinline__ float sq4(float4 a, float4 b) {
  const float dx = a.x - b.x, dy = a.y - b.y, dz = a.z - b.z, dw = a.w - b.w;
  return fmaf(dx, dx, dy * dy) + fmaf(dz, dz, dw * dw);
}

// vec4: x and y 16-byte aligned and the chunk a multiple of 4 elements, so
// that each thread reads float4s (eight in flight): one workgroup then has
// 64 KiB of loads outstanding instead of 8 KiB.
__global__ __launch_bounds__(kMseThreads) void mse_partial_kernel(
    const float* __restrict__ x, const float* __restrict__ y, int64_t n, int vec4,
    float* __restrict__ partial, float* __restrict__ loss) {
  const int64_t base = (int64_t)blockIdx.x * kMseChunk;
  const int64_t end = base + kMseChunk < n ? base + kMseChunk : n;
  constexpr int kU = 8;
  float acc[kU] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int64_t k = base;
  if (vec4) {
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const float4* y4 = reinterpret_cast<const float4*>(y);
    const int64_t e4 = base / 4 + (end - base) / 4;
    int64_t q = base / 4 + threadIdx.x;
    for (; q + (kU - 1) * kMseThreads < e4; q += kU * kMseThreads) {
      float4 a[kU], c[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        a[u] = x4[q + u * kMseThreads];
        c[u] = y4[q + u * kMseThreads];
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) acc[u] += sq4(a[u], c[u]);
    }
    for (; q < e4; q += kMseThreads) acc[0] += sq4(x4[q], y4[q]);
    k = 4 * e4;  // the chunk's last n mod 4 elements, if any, below
  }
  for (k += threadIdx.x; k < end; k += kMseThreads) {
    const float d = x[k] - y[k];
    acc[1] = fmaf(d, d, acc[1]);
  }
  float s = mlcg_wave_sum(((acc[0] + acc[1]) + (acc[2] + acc[3])) +
                          ((acc[4] + acc[5]) + (acc[6] + acc[7])));
  __shared__ float part[kMseThreads / MLCG_WAVE];
  if (mlcg_lane() == 0) part[threadIdx.x / MLCG_WAVE] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < kMseThreads / MLCG_WAVE; ++w) t += part[w];
    if (gridDim.x == 1)
      *loss = t / (float)n;
    else
      partial[blockIdx.x] = t;
  }
}

__global__ __launch_bounds__(MLCG_WAVE) void mse_final_kernel(const float* __restrict__ partial,
                                                              int groups, int64_t n,
                                                              float* __restrict__ loss) {
  // lane l adds the partials l, l + 64, ... in order, then a fixed butterfly
  float t = 0.f;
  for (int g = threadIdx.x; g < groups; g += MLCG_WAVE) t += partial[g];
  t = mlcg_wave_sum(t);
  if (threadIdx.x == 0) *loss = t / (float)n;
}

__global__ __launch_bounds__(256) void mse_backward_kernel(const float* __restrict__ x,
                                                           const float* __restrict__ y,
                                                           const float* __restrict__ g,
                                                           int64_t n, float norm,
                                                           float* __restrict__ out) {
  const float gv = *g;
  for (int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x; k < n;
       k += (int64_t)gridDim.x * 256)
    out[k] = norm * (x[k] - y[k]) * gv;
}

int mse_groups(int64_t n) { return (int)((n + kMseChunk - 1) / kMseChunk); }

}  // namespace

extern "C" int64_t mlcg_mse_workspace_floats(int64_t n) {
  if (n < 0) return -1;
  const int g = mse_groups(n);
  return g > 1 ? g : 0;
}

extern "C" int mlcg_mse_mean(const float* x, const float* y, int64_t n, float* loss,
                             float* workspace, int64_t workspace_floats, void* stream) {
  MLCG_REQUIRE(n >= 1 && n <= (int64_t(1) << 40) && x && y && loss);
  const int groups = mse_groups(n);
  MLCG_REQUIRE(groups == 1 || (workspace && workspace_floats >= groups));
  hipStream_t s = mlcg_stream(stream);
  const int vec4 = reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(y) % 16 == 0;  // kMseChunk is a multiple of 4
  hipLaunchKernelGGL(mse_partial_kernel, dim3((unsigned)groups), dim3(kMseThreads), 0, s, x, y,
                     n, vec4, workspace, loss);
  if (groups > 1)
    hipLaunchKernelGGL(mse_final_kernel, dim3(1), dim3(MLCG_WAVE), 0, s, workspace, groups, n,
                       loss);
  return mlcg_launch_status();
}

extern "C" int mlcg_mse_mean_backward(const float* x, const float* y, const float* grad_loss,
                                      int64_t n, float* grad_x, void* stream) {
  MLCG_REQUIRE(n >= 0 && (n == 0 || (x && y && grad_loss && grad_x)));
  if (n == 0) return MLCG_OK;
  const float norm = (float)(2.0 / (double)n);
  const unsigned groups = mlcg_persistent_groups(mlcg_div_up(n, 256), 8);
  hipLaunchKernelGGL(mse_backward_kernel, dim3(groups), dim3(256), 0, mlcg_stream(stream), x, y,
                     grad_loss, n, norm, grad_x);
  return mlcg_launch_status();
}
