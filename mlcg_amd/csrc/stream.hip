// Streaming read and copy kernels: the HBM ceiling the memory-bound kernels
// of this library are measured against (a STREAM-style probe on this part,
// not part of the SchNet path).
//
// Each thread of a grid-stride loop keeps kUnroll 16-byte loads in flight:
// an iteration of thread t starting at float4 i reads i + u G for u <
// kUnroll (G threads in the grid), so consecutive lanes read consecutive
// 16-byte chunks and every wave reads a whole 1 KiB run per load.  The read
// kernel folds what it loads into one float per workgroup so that no load is
// dead; the copy kernel writes every chunk back to the destination.
#include "common.h"

namespace {

constexpr int kStreamThreads = 256;

template <int kUnroll>
__global__ __launch_bounds__(kStreamThreads) void stream_read_kernel(
    const float4* __restrict__ src, int64_t n4, float* __restrict__ partial) {
  const int64_t G = (int64_t)gridDim.x * kStreamThreads;
  const int64_t t = (int64_t)blockIdx.x * kStreamThreads + threadIdx.x;
  float acc = 0.f;
  int64_t i = t;
  for (; i + (kUnroll - 1) * G < n4; i += kUnroll * G) {
    float4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = src[i + u * G];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc += (v[u].x + v[u].y) + (v[u].z + v[u].w);
  }
  for (; i < n4; i += G) {
    const float4 v = src[i];
    acc += (v.x + v.y) + (v.z + v.w);
  }
  __shared__ float part[kStreamThreads / MLCG_WAVE];
  acc = mlcg_wave_sum(acc);
  if (mlcg_lane() == 0) part[threadIdx.x / MLCG_WAVE] = acc;
  __syncthreads();
  if (threadIdx.x == 0) partial[blockIdx.x] = (part[0] + part[1]) + (part[2] + part[3]);
}

template <int kUnroll>
__global__ __launch_bounds__(kStreamThreads) void stream_copy_kernel(
    const float4* __restrict__ src, float4* __restrict__ dst, int64_t n4) {
  const int64_t G = (int64_t)gridDim.x * kStreamThreads;
  const int64_t t = (int64_t)blockIdx.x * kStreamThreads + threadIdx.x;
  int64_t i = t;
  for (; i + (kUnroll - 1) * G < n4; i += kUnroll * G) {
    float4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = src[i + u * G];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) dst[i + u * G] = v[u];
  }
  for (; i < n4; i += G) dst[i] = src[i];
}

// One launch for a batch of device-to-device copies (a training batch's
// tensors into the inputs of a recorded step): the jobs' 16-byte units are
// numbered consecutively and a grid-stride loop copies them; the last unit of
// a job whose size is not a multiple of 16 is copied byte by byte.
constexpr int kCopyJobs = 8;
struct CopyBatch {
  const char* src[kCopyJobs];
  char* dst[kCopyJobs];
  int64_t bytes[kCopyJobs];
  int64_t first[kCopyJobs + 1];  // first unit of each job; first[count] = total
  int count;
};

__global__ __launch_bounds__(kStreamThreads) void copy_batch_kernel(CopyBatch b) {
  const int64_t G = (int64_t)gridDim.x * kStreamThreads;
  const int64_t total = b.first[b.count];
  int k = 0;
  for (int64_t u = (int64_t)blockIdx.x * kStreamThreads + threadIdx.x; u < total; u += G) {
    while (u >= b.first[k + 1]) ++k;  // units only grow along a thread's loop
    const int64_t off = (u - b.first[k]) * 16;
    const int64_t rem = b.bytes[k] - off;
    if (rem >= 16) {
      *reinterpret_cast<float4*>(b.dst[k] + off) =
          *reinterpret_cast<const float4*>(b.src[k] + off);
    } else {
      for (int64_t c = 0; c < rem; ++c) b.dst[k][off + c] = b.src[k][off + c];
    }
  }
}

// out = ((0 + a_0) + a_1) + ... + a_{count-1} elementwise, the order in
// which SumOut's running sum adds its models' outputs (mlcg/nn/gradients.py
// SumOut), so the result is that loop's bit for bit, in one launch.
constexpr int kSumMax = 8;
struct SumBatch {
  const float* a[kSumMax];
  int count;
};

__global__ __launch_bounds__(kStreamThreads) void sum_arrays_kernel(SumBatch b, int64_t n,
                                                                    float* __restrict__ out) {
  const int64_t G = (int64_t)gridDim.x * kStreamThreads;
  for (int64_t k = (int64_t)blockIdx.x * kStreamThreads + threadIdx.x; k < n; k += G) {
    float acc = 0.0f;
    for (int m = 0; m < b.count; ++m) acc = acc + b.a[m][k];
    out[k] = acc;
  }
}

}  // namespace

extern "C" int mlcg_sum_arrays(const float* const* arrays, int count, int64_t n, float* out,
                               void* stream) {
  MLCG_REQUIRE(count >= 1 && n >= 0 && arrays && (n == 0 || out));
  if (count > kSumMax) return MLCG_ERR_UNSUPPORTED;
  if (n == 0) return MLCG_OK;
  SumBatch b{};
  b.count = count;
  for (int m = 0; m < count; ++m) {
    MLCG_REQUIRE(arrays[m] != nullptr);
    b.a[m] = arrays[m];
  }
  const unsigned groups = mlcg_persistent_groups(mlcg_div_up(n, kStreamThreads), 8);
  hipLaunchKernelGGL(sum_arrays_kernel, dim3(groups), dim3(kStreamThreads), 0,
                     mlcg_stream(stream), b, n, out);
  return mlcg_launch_status();
}

extern "C" int mlcg_copy_batch(const void* const* srcs, void* const* dsts, const int64_t* bytes,
                               int count, void* stream) {
  MLCG_REQUIRE(count >= 0 && srcs && dsts && bytes);
  if (count > kCopyJobs) return MLCG_ERR_UNSUPPORTED;
  CopyBatch b{};
  b.count = count;
  b.first[0] = 0;
  for (int k = 0; k < count; ++k) {
    MLCG_REQUIRE(bytes[k] >= 0 && (bytes[k] == 0 || (srcs[k] && dsts[k])));
    MLCG_REQUIRE(reinterpret_cast<uintptr_t>(srcs[k]) % 16 == 0 &&
                 reinterpret_cast<uintptr_t>(dsts[k]) % 16 == 0);
    b.src[k] = static_cast<const char*>(srcs[k]);
    b.dst[k] = static_cast<char*>(dsts[k]);
    b.bytes[k] = bytes[k];
    b.first[k + 1] = b.first[k] + (bytes[k] + 15) / 16;
  }
  const int64_t total = b.first[count];
  if (total == 0) return MLCG_OK;
  const unsigned groups = mlcg_persistent_groups(mlcg_div_up(total, kStreamThreads), 8);
  hipLaunchKernelGGL(copy_batch_kernel, dim3(groups), dim3(kStreamThreads), 0,
                     mlcg_stream(stream), b);
  return mlcg_launch_status();
}

extern "C" int mlcg_stream_read(const float* src, int64_t n, int groups, int unroll,
                                float* partial, void* stream) {
  MLCG_REQUIRE(src && partial && n >= 0 && n % 4 == 0 && groups >= 1 && groups <= 65536);
  MLCG_REQUIRE(unroll == 1 || unroll == 4 || unroll == 8 || unroll == 16);
  MLCG_REQUIRE(reinterpret_cast<uintptr_t>(src) % 16 == 0);
  const auto s = mlcg_stream(stream);
  const auto* s4 = reinterpret_cast<const float4*>(src);
  if (unroll == 1)
    stream_read_kernel<1><<<groups, kStreamThreads, 0, s>>>(s4, n / 4, partial);
  else if (unroll == 4)
    stream_read_kernel<4><<<groups, kStreamThreads, 0, s>>>(s4, n / 4, partial);
  else if (unroll == 8)
    stream_read_kernel<8><<<groups, kStreamThreads, 0, s>>>(s4, n / 4, partial);
  else
    stream_read_kernel<16><<<groups, kStreamThreads, 0, s>>>(s4, n / 4, partial);
  return mlcg_launch_status();
}

extern "C" int mlcg_stream_copy(const float* src, float* dst, int64_t n, int groups, int unroll,
                                void* stream) {
  MLCG_REQUIRE(src && dst && n >= 0 && n % 4 == 0 && groups >= 1 && groups <= 65536);
  MLCG_REQUIRE(unroll == 1 || unroll == 4 || unroll == 8 || unroll == 16);
  MLCG_REQUIRE(reinterpret_cast<uintptr_t>(src) % 16 == 0 &&
               reinterpret_cast<uintptr_t>(dst) % 16 == 0);
  const auto s = mlcg_stream(stream);
  const auto* s4 = reinterpret_cast<const float4*>(src);
  auto* d4 = reinterpret_cast<float4*>(dst);
  if (unroll == 1)
    stream_copy_kernel<1><<<groups, kStreamThreads, 0, s>>>(s4, d4, n / 4);
  else if (unroll == 4)
    stream_copy_kernel<4><<<groups, kStreamThreads, 0, s>>>(s4, d4, n / 4);
  else if (unroll == 8)
    stream_copy_kernel<8><<<groups, kStreamThreads, 0, s>>>(s4, d4, n / 4);
  else
    stream_copy_kernel<16><<<groups, kStreamThreads, 0, s>>>(s4, d4, n / 4);
  return mlcg_launch_status();
}
