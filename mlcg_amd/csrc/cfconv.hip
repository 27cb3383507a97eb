// CFConv gather/scatter over the receiver CSR, with the hand-derived force
// backward, tangent and second-order reverse (gfx950).
//
// Reference: CFConv.forward/propagate/message (mlcg/nn/schnet.py:312-368) with
// PyG's SumAggregation: agg[t] = sum_e x[s_e] * W_e over edges e = (s, t).
// The neighbour list is symmetric and W depends only on |r_ij|, so the same
// sum is agg[i] = sum_{j in N(i)} y[j] * W_{p(i,j)}.  With rows sorted by
// receiver and each row sorted by neighbour, a sequential sum along the row
// reproduces the CPU reference's accumulation order (ascending sender) and
// needs no atomics.
//
// Mapping: one wave per receiver row; every lane owns 2 of the 128 features
// (float2), so one W row (512 B) or node row is one coalesced wave load.  The
// row's (col, pair) indices are fetched 64 at a time by the lanes and
// broadcast with readlane, and loads for several edges are issued before
// their products are accumulated (in order) to keep HBM busy.
#include "common.h"

#include <hip/hip_fp16.h>

namespace {

constexpr int kF = 128;
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * MLCG_WAVE;
constexpr int kUnroll = 4;

struct F2 {
  float x, y;
};

__device__ __forceinline__ F2 ld2(const float* __restrict__ p, int64_t row, int lane) {
  float2 v = *reinterpret_cast<const float2*>(p + row * kF + 2 * lane);
  return F2{v.x, v.y};
}

__device__ __forceinline__ F2 ldw(const void* __restrict__ W, bool f16, int64_t row, int lane) {
  if (f16) {
    __half2 h = *reinterpret_cast<const __half2*>(static_cast<const __half*>(W) + row * kF +
                                                  2 * lane);
    float2 v = __half22float2(h);
    return F2{v.x, v.y};
  }
  return ld2(static_cast<const float*>(W), row, lane);
}

__device__ __forceinline__ void st2(float* __restrict__ p, int64_t row, int lane, F2 v) {
  *reinterpret_cast<float2*>(p + row * kF + 2 * lane) = float2{v.x, v.y};
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Iterate the row of wave-uniform receiver i in chunks of 64 edges: lane k
// holds col/pair of edge chunk_start + k.
#define MLCG_ROW_LOOP_BEGIN(i)                                                  \
  const int e_begin = uniform(rowptr[i]);                                       \
  const int e_end = uniform(rowptr[(i) + 1]);                                   \
  for (int c0 = e_begin; c0 < e_end; c0 += MLCG_WAVE) {                         \
    const int cn = min(MLCG_WAVE, e_end - c0);                                  \
    const int my_col = lane < cn ? col[c0 + lane] : 0;                          \
    const int my_pair = lane < cn ? eid2pair[c0 + lane] : 0;

#define MLCG_ROW_LOOP_END }

__global__ __launch_bounds__(kThreads) void gather_kernel(
    const float* __restrict__ src, const void* __restrict__ W, int w_f16,
    const int32_t* __restrict__ rowptr, const int32_t* __restrict__ col,
    const int32_t* __restrict__ eid2pair, int64_t n, float* __restrict__ out) {
  const int lane = mlcg_lane();
  const bool f16 = w_f16 != 0;
  for (int64_t i = (int64_t)blockIdx.x * kWaves + threadIdx.x / MLCG_WAVE; i < n;
       i += (int64_t)gridDim.x * kWaves) {
    F2 acc{0.f, 0.f};
    MLCG_ROW_LOOP_BEGIN(i)
    int k = 0;
    for (; k + kUnroll <= cn; k += kUnroll) {
      F2 s[kUnroll], w[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int j = __builtin_amdgcn_readlane(my_col, k + u);
        const int p = __builtin_amdgcn_readlane(my_pair, k + u);
        s[u] = ld2(src, j, lane);
        w[u] = ldw(W, f16, p, lane);
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        acc.x += s[u].x * w[u].x;
        acc.y += s[u].y * w[u].y;
      }
    }
    for (; k < cn; ++k) {
      const int j = __builtin_amdgcn_readlane(my_col, k);
      const int p = __builtin_amdgcn_readlane(my_pair, k);
      F2 s = ld2(src, j, lane), w = ldw(W, f16, p, lane);
      acc.x += s.x * w.x;
      acc.y += s.y * w.y;
    }
    MLCG_ROW_LOOP_END
    st2(out, i, lane, acc);
  }
}

__global__ __launch_bounds__(kThreads) void gather_bwd_kernel(
    const float* __restrict__ gagg, const float* __restrict__ y, const void* __restrict__ W,
    const void* __restrict__ Wd, int w_f16, const int32_t* __restrict__ rowptr,
    const int32_t* __restrict__ col, const int32_t* __restrict__ eid2pair, int64_t n,
    float* __restrict__ ybar, float* __restrict__ dbar) {
  const int lane = mlcg_lane();
  const bool f16 = w_f16 != 0;
  for (int64_t i = (int64_t)blockIdx.x * kWaves + threadIdx.x / MLCG_WAVE; i < n;
       i += (int64_t)gridDim.x * kWaves) {
    const F2 gi = ld2(gagg, i, lane);
    const F2 yi = ld2(y, i, lane);
    F2 acc{0.f, 0.f};
    MLCG_ROW_LOOP_BEGIN(i)
    for (int k = 0; k < cn; ++k) {
      const int j = __builtin_amdgcn_readlane(my_col, k);
      const int p = __builtin_amdgcn_readlane(my_pair, k);
      const F2 gj = ld2(gagg, j, lane);
      const F2 w = ldw(W, f16, p, lane);
      acc.x += gj.x * w.x;
      acc.y += gj.y * w.y;
      if (j > i) {
        const F2 yj = ld2(y, j, lane);
        const F2 wd = ldw(Wd, f16, p, lane);
        float part = wd.x * (gi.x * yj.x + gj.x * yi.x) + wd.y * (gi.y * yj.y + gj.y * yi.y);
        part = mlcg_wave_sum(part);
        if (lane == 0) dbar[p] += part;
      }
    }
    MLCG_ROW_LOOP_END
    st2(ybar, i, lane, acc);
  }
}

__global__ __launch_bounds__(kThreads) void gather_tangent_kernel(
    const float* __restrict__ ydot, const float* __restrict__ y, const float* __restrict__ W,
    const float* __restrict__ Wd, const float* __restrict__ ddot,
    const int32_t* __restrict__ rowptr, const int32_t* __restrict__ col,
    const int32_t* __restrict__ eid2pair, int64_t n, float* __restrict__ out) {
  const int lane = mlcg_lane();
  for (int64_t i = (int64_t)blockIdx.x * kWaves + threadIdx.x / MLCG_WAVE; i < n;
       i += (int64_t)gridDim.x * kWaves) {
    F2 acc{0.f, 0.f};
    MLCG_ROW_LOOP_BEGIN(i)
    const float my_dd = lane < cn ? ddot[my_pair] : 0.f;
    for (int k = 0; k < cn; ++k) {
      const int j = __builtin_amdgcn_readlane(my_col, k);
      const int p = __builtin_amdgcn_readlane(my_pair, k);
      const float dd = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_dd), k));
      const F2 yj = ld2(y, j, lane);
      const F2 wd = ld2(Wd, p, lane);
      if (ydot) {
        const F2 yd = ld2(ydot, j, lane);
        const F2 w = ld2(W, p, lane);
        acc.x += yd.x * w.x + yj.x * (wd.x * dd);
        acc.y += yd.y * w.y + yj.y * (wd.y * dd);
      } else {
        acc.x += yj.x * (wd.x * dd);
        acc.y += yj.y * (wd.y * dd);
      }
    }
    MLCG_ROW_LOOP_END
    st2(out, i, lane, acc);
  }
}

__global__ __launch_bounds__(kThreads) void gather_rev2_kernel(
    const float* __restrict__ gagg2, const float* __restrict__ gagg1,
    const float* __restrict__ y, const float* __restrict__ ydot, const float* __restrict__ W,
    const float* __restrict__ Wd, const float* __restrict__ ddot,
    const int32_t* __restrict__ rowptr, const int32_t* __restrict__ col,
    const int32_t* __restrict__ eid2pair, int64_t n, float* __restrict__ ybar2,
    float* __restrict__ Wbar, float* __restrict__ Wdbar) {
  const int lane = mlcg_lane();
  const bool tangent = gagg1 != nullptr;
  for (int64_t i = (int64_t)blockIdx.x * kWaves + threadIdx.x / MLCG_WAVE; i < n;
       i += (int64_t)gridDim.x * kWaves) {
    const F2 g2i = ld2(gagg2, i, lane);
    const F2 yi = ld2(y, i, lane);
    const F2 g1i = tangent ? ld2(gagg1, i, lane) : F2{0.f, 0.f};
    const F2 ydi = (tangent && ydot) ? ld2(ydot, i, lane) : F2{0.f, 0.f};
    F2 acc{0.f, 0.f};
    MLCG_ROW_LOOP_BEGIN(i)
    const float my_dd = (tangent && lane < cn) ? ddot[my_pair] : 0.f;
    for (int k = 0; k < cn; ++k) {
      const int j = __builtin_amdgcn_readlane(my_col, k);
      const int p = __builtin_amdgcn_readlane(my_pair, k);
      const float dd = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_dd), k));
      const F2 g2j = ld2(gagg2, j, lane);
      const F2 w = ld2(W, p, lane);
      F2 g1j{0.f, 0.f}, wd{0.f, 0.f};
      if (tangent) {
        g1j = ld2(gagg1, j, lane);
        wd = ld2(Wd, p, lane);
      }
      acc.x += g2j.x * w.x + g1j.x * (wd.x * dd);
      acc.y += g2j.y * w.y + g1j.y * (wd.y * dd);
      if (j > i) {
        const F2 yj = ld2(y, j, lane);
        F2 wb, wdb;
        wb.x = g2i.x * yj.x + g2j.x * yi.x;
        wb.y = g2i.y * yj.y + g2j.y * yi.y;
        if (tangent) {
          const F2 ydj = ydot ? ld2(ydot, j, lane) : F2{0.f, 0.f};
          wb.x += g1i.x * ydj.x + g1j.x * ydi.x;
          wb.y += g1i.y * ydj.y + g1j.y * ydi.y;
          wdb.x = dd * (g1i.x * yj.x + g1j.x * yi.x);
          wdb.y = dd * (g1i.y * yj.y + g1j.y * yi.y);
        } else {
          wdb = F2{0.f, 0.f};
        }
        st2(Wbar, p, lane, wb);
        st2(Wdbar, p, lane, wdb);
      }
    }
    MLCG_ROW_LOOP_END
    st2(ybar2, i, lane, acc);
  }
}

__global__ void pair_ddot_kernel(const float* __restrict__ pos, const float* __restrict__ dist,
                                 const int32_t* __restrict__ pi, const int32_t* __restrict__ pj,
                                 const int32_t* __restrict__ n_pairs_dev, int64_t max_pairs,
                                 const float* __restrict__ u, float* __restrict__ ddot) {
  int64_t np = *n_pairs_dev;
  if (np > max_pairs) np = max_pairs;
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < np;
       p += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = pi[p], j = pj[p];
    const float inv = 1.0f / dist[p];
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < 3; ++c) acc += (pos[3 * j + c] - pos[3 * i + c]) * (u[3 * j + c] - u[3 * i + c]);
    ddot[p] = acc * inv;
  }
}

__global__ void pair_forces_kernel(const float* __restrict__ pos, const float* __restrict__ dist,
                                   const float* __restrict__ dbar,
                                   const int32_t* __restrict__ rowptr,
                                   const int32_t* __restrict__ col,
                                   const int32_t* __restrict__ eid2pair, int64_t n,
                                   int accumulate, float* __restrict__ forces) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float xi = pos[3 * i], yi = pos[3 * i + 1], zi = pos[3 * i + 2];
    float fx = 0.f, fy = 0.f, fz = 0.f;
    for (int e = rowptr[i]; e < rowptr[i + 1]; ++e) {
      const int64_t j = col[e];
      const int p = eid2pair[e];
      const float s = dbar[p] / dist[p];
      fx += s * (pos[3 * j] - xi);
      fy += s * (pos[3 * j + 1] - yi);
      fz += s * (pos[3 * j + 2] - zi);
    }
    if (accumulate) {
      forces[3 * i] += fx;
      forces[3 * i + 1] += fy;
      forces[3 * i + 2] += fz;
    } else {
      forces[3 * i] = fx;
      forces[3 * i + 1] = fy;
      forces[3 * i + 2] = fz;
    }
  }
}

// One workgroup per segment: every thread keeps a compensated (Kahan) sum of
// a strided subset, then the partial sums are combined in a fixed tree order
// in LDS.  Deterministic for a given launch shape, and accurate to a few ulp
// even for the ~10^5-term per-frame sums of a pair prior.
constexpr int kSegThreads = 256;

__global__ __launch_bounds__(kSegThreads) void segment_sum_kernel(
    const float* __restrict__ v, int64_t stride, const int64_t* __restrict__ ptr, int64_t nb,
    float* __restrict__ out) {
  __shared__ float part[kSegThreads];
  for (int64_t b = blockIdx.x; b < nb; b += gridDim.x) {
    float s = 0.f, c = 0.f;
    for (int64_t k = ptr[b] + threadIdx.x; k < ptr[b + 1]; k += kSegThreads) {
      const float y = v[k * stride] - c;
      const float t = s + y;
      c = (t - s) - y;
      s = t;
    }
    part[threadIdx.x] = s;
    __syncthreads();
    for (int w = kSegThreads / 2; w > 0; w >>= 1) {
      if (threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
      __syncthreads();
    }
    if (threadIdx.x == 0) out[b] = part[0];
    __syncthreads();
  }
}

unsigned row_groups(int64_t n) { return mlcg_persistent_groups(mlcg_div_up(n, kWaves), 16); }

}  // namespace

extern "C" int mlcg_cfconv_gather(const float* src, const void* W, int w_f16,
                                  const int32_t* rowptr, const int32_t* col,
                                  const int32_t* eid2pair, int64_t n_nodes, int num_filters,
                                  float* out, void* stream) {
  if (num_filters != kF) return MLCG_ERR_UNSUPPORTED;
  MLCG_REQUIRE(n_nodes >= 0);
  if (n_nodes == 0) return MLCG_OK;
  MLCG_REQUIRE(src && W && rowptr && col && eid2pair && out);
  hipLaunchKernelGGL(gather_kernel, dim3(row_groups(n_nodes)), dim3(kThreads), 0,
                     mlcg_stream(stream), src, W, w_f16, rowptr, col, eid2pair, n_nodes, out);
  return mlcg_launch_status();
}

extern "C" int mlcg_cfconv_gather_bwd(const float* gagg, const float* y, const void* W,
                                      const void* Wd, int w_f16, const int32_t* rowptr,
                                      const int32_t* col, const int32_t* eid2pair,
                                      int64_t n_nodes, int num_filters, float* ybar,
                                      float* dbar, void* stream) {
  if (num_filters != kF) return MLCG_ERR_UNSUPPORTED;
  MLCG_REQUIRE(n_nodes >= 0);
  if (n_nodes == 0) return MLCG_OK;
  MLCG_REQUIRE(gagg && y && W && Wd && rowptr && col && eid2pair && ybar && dbar);
  hipLaunchKernelGGL(gather_bwd_kernel, dim3(row_groups(n_nodes)), dim3(kThreads), 0,
                     mlcg_stream(stream), gagg, y, W, Wd, w_f16, rowptr, col, eid2pair,
                     n_nodes, ybar, dbar);
  return mlcg_launch_status();
}

extern "C" int mlcg_cfconv_gather_tangent(const float* ydot, const float* y, const float* W,
                                          const float* Wd, const float* ddot,
                                          const int32_t* rowptr, const int32_t* col,
                                          const int32_t* eid2pair, int64_t n_nodes,
                                          int num_filters, float* out, void* stream) {
  if (num_filters != kF) return MLCG_ERR_UNSUPPORTED;
  MLCG_REQUIRE(n_nodes >= 0);
  if (n_nodes == 0) return MLCG_OK;
  MLCG_REQUIRE(y && W && Wd && ddot && rowptr && col && eid2pair && out);
  hipLaunchKernelGGL(gather_tangent_kernel, dim3(row_groups(n_nodes)), dim3(kThreads), 0,
                     mlcg_stream(stream), ydot, y, W, Wd, ddot, rowptr, col, eid2pair,
                     n_nodes, out);
  return mlcg_launch_status();
}

extern "C" int mlcg_cfconv_gather_rev2(const float* gagg2, const float* gagg1, const float* y,
                                       const float* ydot, const float* W, const float* Wd,
                                       const float* ddot, const int32_t* rowptr,
                                       const int32_t* col, const int32_t* eid2pair,
                                       int64_t n_nodes, int num_filters, float* ybar2,
                                       float* Wbar, float* Wdbar, void* stream) {
  if (num_filters != kF) return MLCG_ERR_UNSUPPORTED;
  MLCG_REQUIRE(n_nodes >= 0);
  if (n_nodes == 0) return MLCG_OK;
  MLCG_REQUIRE(gagg2 && y && W && rowptr && col && eid2pair && ybar2 && Wbar && Wdbar);
  MLCG_REQUIRE(!gagg1 || (Wd && ddot));
  hipLaunchKernelGGL(gather_rev2_kernel, dim3(row_groups(n_nodes)), dim3(kThreads), 0,
                     mlcg_stream(stream), gagg2, gagg1, y, ydot, W, Wd, ddot, rowptr, col,
                     eid2pair, n_nodes, ybar2, Wbar, Wdbar);
  return mlcg_launch_status();
}

extern "C" int mlcg_pair_ddot(const float* pos, const float* dist, const int32_t* pair_ij,
                              int64_t pair_stride, const int32_t* n_pairs_dev,
                              int64_t max_pairs, const float* u, float* ddot, void* stream) {
  MLCG_REQUIRE(max_pairs >= 0 && pair_stride >= max_pairs);
  if (max_pairs == 0) return MLCG_OK;
  MLCG_REQUIRE(pos && dist && pair_ij && n_pairs_dev && u && ddot);
  hipLaunchKernelGGL(pair_ddot_kernel, dim3(mlcg_persistent_groups(mlcg_div_up(max_pairs, 256), 8)),
                     dim3(256), 0, mlcg_stream(stream), pos, dist, pair_ij,
                     pair_ij + pair_stride, n_pairs_dev, max_pairs, u, ddot);
  return mlcg_launch_status();
}

extern "C" int mlcg_pair_forces(const float* pos, const float* dist, const float* dbar,
                                const int32_t* rowptr, const int32_t* col,
                                const int32_t* eid2pair, int64_t n_nodes, int accumulate,
                                float* forces, void* stream) {
  MLCG_REQUIRE(n_nodes >= 0);
  if (n_nodes == 0) return MLCG_OK;
  MLCG_REQUIRE(pos && dist && dbar && rowptr && col && eid2pair && forces);
  hipLaunchKernelGGL(pair_forces_kernel, dim3(mlcg_div_up(n_nodes, 256)), dim3(256), 0,
                     mlcg_stream(stream), pos, dist, dbar, rowptr, col, eid2pair, n_nodes,
                     accumulate, forces);
  return mlcg_launch_status();
}

extern "C" int mlcg_segment_sum(const float* values, int64_t stride, const int64_t* frame_ptr,
                                int64_t n_frames, float* out, void* stream) {
  MLCG_REQUIRE(n_frames >= 0 && stride >= 1);
  if (n_frames == 0) return MLCG_OK;
  MLCG_REQUIRE(values && frame_ptr && out);
  hipLaunchKernelGGL(segment_sum_kernel, dim3(mlcg_persistent_groups(n_frames, 8)),
                     dim3(kSegThreads), 0, mlcg_stream(stream), values, stride, frame_ptr,
                     n_frames, out);
  return mlcg_launch_status();
}
