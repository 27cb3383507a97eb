// Weight gradients of the node-level linears of the interaction blocks
// (gfx950, MFMA fp32).
//
// The CFConv and interaction-block linears of SchNet (conv.lin1, conv.lin2,
// lin: mlcg/nn/schnet.py:259-261,343,347) act on [N, 128] node features with
// 128 x 128 weights; their weight gradients are transposed products a^T b
// with the reduction over the N ~ 10^4-10^5 rows, a shape (M = N = 128,
// huge K) that a general GEMM library tiles poorly.  They run here on
// v_mfma_f32_16x16x4f32:
//
//   node_tmm      out = a1^T b1 [+ a2^T b2] ([128, 128]): up to 128 workgroups
//                 each reduce a fixed set of 64-row chunks (staged in LDS)
//                 with the row index as the MFMA reduction axis (wave w owns
//                 output rows 16w..16w+15) and write their partial; a second
//                 kernel adds the partials in a fixed order -- deterministic
//                 for a given row count.
#include "common.h"

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kF = 128;
constexpr int kFT = kF / 16;
// ---------------------------------------------------------------------------
constexpr int kTmmWaves = 8;
constexpr int kTmmThreads = kTmmWaves * MLCG_WAVE;
constexpr int kTmmRows = 64;                     // rows per workgroup slice
constexpr int kTRow = kF + 4;                    // padded LDS row

// Loads rows r0..r0+63 of a and b into LDS (zero past `rows`): 8 float4 per
// thread, all issued before the stores.
__device__ __forceinline__ void tmm_stage(float* la, float* lb, const float* __restrict__ a,
                                          const float* __restrict__ b, int64_t r0,
                                          int64_t rows) {
  constexpr int kChunks = kTmmRows * kF / 4;       // float4 chunks per matrix
  constexpr int kPer = kChunks / kTmmThreads;      // 4
  float4 va[kPer], vb[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int c = threadIdx.x + k * kTmmThreads;
    const int64_t r = r0 + c / (kF / 4);
    const int col = 4 * (c % (kF / 4));
    const bool ok = r < rows;
    va[k] = ok ? *reinterpret_cast<const float4*>(a + r * kF + col) : float4{0.f, 0.f, 0.f, 0.f};
    vb[k] = ok ? *reinterpret_cast<const float4*>(b + r * kF + col) : float4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int c = threadIdx.x + k * kTmmThreads;
    const int rr = c / (kF / 4), col = 4 * (c % (kF / 4));
    *reinterpret_cast<float4*>(la + rr * kTRow + col) = va[k];
    *reinterpret_cast<float4*>(lb + rr * kTRow + col) = vb[k];
  }
}

__device__ __forceinline__ void tmm_accumulate(const float* la, const float* lb, int w, int q,
                                               int n, floatx4* acc) {
#pragma unroll 4
  for (int kk = 0; kk < kTmmRows / 4; ++kk) {
    const float av = la[(4 * kk + q) * kTRow + 16 * w + n];
    float bv[kFT];
#pragma unroll
    for (int u = 0; u < kFT; ++u) bv[u] = lb[(4 * kk + q) * kTRow + 16 * u + n];
#pragma unroll
    for (int u = 0; u < kFT; ++u)
      acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv[u], acc[u], 0, 0, 0);
  }
}

__global__ __launch_bounds__(kTmmThreads) void node_tmm_kernel(
    const float* __restrict__ a1, const float* __restrict__ b1,
    const float* __restrict__ a2, const float* __restrict__ b2, int64_t rows,
    float* __restrict__ partial) {
  __shared__ float lds[4 * kTmmRows * kTRow];
  float* la1 = lds;
  float* lb1 = la1 + kTmmRows * kTRow;
  float* la2 = lb1 + kTmmRows * kTRow;
  float* lb2 = la2 + kTmmRows * kTRow;
  const int w = threadIdx.x / MLCG_WAVE;
  const int l = mlcg_lane();
  const int q = l >> 4, n = l & 15;
  floatx4 acc[kFT];
#pragma unroll
  for (int u = 0; u < kFT; ++u) acc[u] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int64_t chunks = (rows + kTmmRows - 1) / kTmmRows;
  for (int64_t c = blockIdx.x; c < chunks; c += gridDim.x) {
    const int64_t r0 = c * kTmmRows;
    tmm_stage(la1, lb1, a1, b1, r0, rows);
    if (a2) tmm_stage(la2, lb2, a2, b2, r0, rows);
    __syncthreads();
    tmm_accumulate(la1, lb1, w, q, n, acc);
    if (a2) tmm_accumulate(la2, lb2, w, q, n, acc);
    __syncthreads();
  }
  float* o = partial + (int64_t)blockIdx.x * kF * kF;
#pragma unroll
  for (int u = 0; u < kFT; ++u)
#pragma unroll
    for (int i = 0; i < 4; ++i) o[(16 * w + 4 * q + i) * kF + 16 * u + n] = acc[u][i];
}

// out (+)= sum of the `slices` partials.  A block covers 64 outputs with 8
// waves, wave g summing the partials s = g (mod 8) (two interleaved
// accumulators); the 8 wave sums are combined in a fixed order.
__global__ __launch_bounds__(512) void node_tmm_reduce_kernel(const float* __restrict__ partial,
                                                              int slices, int accumulate,
                                                              float* __restrict__ out) {
  __shared__ float part[8][64];
  const int o = threadIdx.x & 63, g = threadIdx.x >> 6;
  const int j = blockIdx.x * 64 + o;
  float a0 = 0.f, a1 = 0.f;
  int s = g;
  for (; s + 8 < slices; s += 16) {
    a0 += partial[(int64_t)s * kF * kF + j];
    a1 += partial[(int64_t)(s + 8) * kF * kF + j];
  }
  if (s < slices) a0 += partial[(int64_t)s * kF * kF + j];
  part[g][o] = a0 + a1;
  __syncthreads();
  if (g == 0) {
    const float v = ((part[0][o] + part[1][o]) + (part[2][o] + part[3][o])) +
                    ((part[4][o] + part[5][o]) + (part[6][o] + part[7][o]));
    out[j] = accumulate ? out[j] + v : v;
  }
}

int tmm_groups(int64_t rows) {
  const int64_t chunks = rows == 0 ? 1 : (rows + kTmmRows - 1) / kTmmRows;
  return (int)(chunks < 128 ? chunks : 128);
}

}  // namespace

extern "C" int64_t mlcg_node_tmm_workspace_floats(int64_t rows) {
  if (rows < 0) return -1;
  return (int64_t)tmm_groups(rows) * kF * kF;
}

extern "C" int mlcg_node_tmm(const float* a1, const float* b1, const float* a2,
                             const float* b2, int64_t rows, int features, int accumulate,
                             float* out, float* workspace, int64_t workspace_floats,
                             void* stream) {
  if (features != kF) return MLCG_ERR_UNSUPPORTED;
  MLCG_REQUIRE(rows >= 0 && out && workspace);
  MLCG_REQUIRE(rows == 0 || (a1 && b1));
  MLCG_REQUIRE((a2 == nullptr) == (b2 == nullptr));
  const int groups = tmm_groups(rows);
  MLCG_REQUIRE(workspace_floats >= (int64_t)groups * kF * kF);
  hipStream_t s = mlcg_stream(stream);
  hipLaunchKernelGGL(node_tmm_kernel, dim3((unsigned)groups), dim3(kTmmThreads), 0, s, a1, b1,
                     rows == 0 ? nullptr : a2, b2, rows, workspace);
  hipLaunchKernelGGL(node_tmm_reduce_kernel, dim3(kF * kF / 64), dim3(512), 0, s, workspace,
                     groups, accumulate, out);
  return mlcg_launch_status();
}
