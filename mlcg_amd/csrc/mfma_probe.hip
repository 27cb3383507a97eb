// MFMA-loop probe: the sustained matrix-core rate of this part for the MFMA
// shapes the filter and node kernels use (a measurement probe, not part of
// the SchNet path).
//
// Every wave runs `iters` iterations of kChains independent MFMAs of one
// shape (kChains accumulator chains, so no MFMA waits for the previous one's
// result) on operands held in registers.  The accumulators are added and
// stored per lane at the end, so no product is dead.  The rate is
// groups * (threads / 64) * iters * kChains * flops(shape) / time.
#include "common.h"
#include "split16.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kProbeThreads = 256;
constexpr int kChains = 8;

enum ProbeKind {
  kF16_16x16x32 = 0,   // v_mfma_f32_16x16x32_f16   (filter, node products)
  kF16_16x16x16 = 1,   // v_mfma_f32_16x16x16_f16   (filter backward, step 1)
  kF32_16x16x4 = 2,    // v_mfma_f32_16x16x4_f32    (strict fp32 filters)
  kBF16_16x16x32 = 3,  // v_mfma_f32_16x16x32_bf16  (weight-gradient reductions)
  kF16_32x32x16 = 4,   // v_mfma_f32_32x32x16_f16   (the larger fp16 shape)
};

template <int KIND>
__global__ __launch_bounds__(kProbeThreads) void mfma_loop_kernel(int64_t iters,
                                                                   float* __restrict__ out) {
  const int l = mlcg_lane();
  // small operands that differ per lane and chain (values stay finite over
  // any iteration count used here)
  const float base = 1.0f / 1024.0f * (float)((l & 15) + 1);
  float sum = 0.f;
  if constexpr (KIND == kF16_32x32x16) {
    floatx16 acc[kChains];
    halfx8 a[kChains], b;
#pragma unroll
    for (int c = 0; c < kChains; ++c) {
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[c][j] = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) a[c][j] = (_Float16)(base * (float)(c + j + 1));
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) b[j] = (_Float16)(base * (float)(j + 2));
    for (int64_t it = 0; it < iters; ++it)
#pragma unroll
      for (int c = 0; c < kChains; ++c)
        acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[c], b, acc[c], 0, 0, 0);
#pragma unroll
    for (int c = 0; c < kChains; ++c)
#pragma unroll
      for (int j = 0; j < 16; ++j) sum += acc[c][j];
  } else {
    floatx4 acc[kChains];
#pragma unroll
    for (int c = 0; c < kChains; ++c) acc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
    if constexpr (KIND == kF16_16x16x32) {
      halfx8 a[kChains], b;
#pragma unroll
      for (int c = 0; c < kChains; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) a[c][j] = (_Float16)(base * (float)(c + j + 1));
#pragma unroll
      for (int j = 0; j < 8; ++j) b[j] = (_Float16)(base * (float)(j + 2));
      for (int64_t it = 0; it < iters; ++it)
#pragma unroll
        for (int c = 0; c < kChains; ++c)
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[c], b, acc[c], 0, 0, 0);
    } else if constexpr (KIND == kF16_16x16x16) {
      halfx4 a[kChains], b;
#pragma unroll
      for (int c = 0; c < kChains; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) a[c][j] = (_Float16)(base * (float)(c + j + 1));
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = (_Float16)(base * (float)(j + 2));
      for (int64_t it = 0; it < iters; ++it)
#pragma unroll
        for (int c = 0; c < kChains; ++c)
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x16f16(a[c], b, acc[c], 0, 0, 0);
    } else if constexpr (KIND == kF32_16x16x4) {
      float a[kChains];
      const float b = base * 2.0f;
#pragma unroll
      for (int c = 0; c < kChains; ++c) a[c] = base * (float)(c + 1);
      for (int64_t it = 0; it < iters; ++it)
#pragma unroll
        for (int c = 0; c < kChains; ++c)
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[c], b, acc[c], 0, 0, 0);
    } else {
      bf16x8 a[kChains], b;
#pragma unroll
      for (int c = 0; c < kChains; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) a[c][j] = (__bf16)(base * (float)(c + j + 1));
#pragma unroll
      for (int j = 0; j < 8; ++j) b[j] = (__bf16)(base * (float)(j + 2));
      for (int64_t it = 0; it < iters; ++it)
#pragma unroll
        for (int c = 0; c < kChains; ++c)
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[c], b, acc[c], 0, 0, 0);
    }
#pragma unroll
    for (int c = 0; c < kChains; ++c) sum += (acc[c][0] + acc[c][1]) + (acc[c][2] + acc[c][3]);
  }
  out[(int64_t)blockIdx.x * kProbeThreads + threadIdx.x] = sum;
}

}  // namespace

extern "C" int64_t mlcg_mfma_loop_flops_per_wave_iter(int kind) {
  switch (kind) {
    case kF16_16x16x32:
    case kBF16_16x16x32:
      return (int64_t)kChains * 2 * 16 * 16 * 32;
    case kF16_16x16x16:
      return (int64_t)kChains * 2 * 16 * 16 * 16;
    case kF32_16x16x4:
      return (int64_t)kChains * 2 * 16 * 16 * 4;
    case kF16_32x32x16:
      return (int64_t)kChains * 2 * 32 * 32 * 16;
    default:
      return -1;
  }
}

extern "C" int mlcg_mfma_loop(int kind, int64_t iters, int groups, float* out, void* stream) {
  MLCG_REQUIRE(out && iters >= 1 && groups >= 1 && groups <= 65536);
  MLCG_REQUIRE(kind >= 0 && kind <= 4);
  const auto s = mlcg_stream(stream);
  switch (kind) {
    case kF16_16x16x32:
      mfma_loop_kernel<kF16_16x16x32><<<groups, kProbeThreads, 0, s>>>(iters, out);
      break;
    case kF16_16x16x16:
      mfma_loop_kernel<kF16_16x16x16><<<groups, kProbeThreads, 0, s>>>(iters, out);
      break;
    case kF32_16x16x4:
      mfma_loop_kernel<kF32_16x16x4><<<groups, kProbeThreads, 0, s>>>(iters, out);
      break;
    case kBF16_16x16x32:
      mfma_loop_kernel<kBF16_16x16x32><<<groups, kProbeThreads, 0, s>>>(iters, out);
      break;
    default:
      mfma_loop_kernel<kF16_32x32x16><<<groups, kProbeThreads, 0, s>>>(iters, out);
      break;
  }
  return mlcg_launch_status();
}
