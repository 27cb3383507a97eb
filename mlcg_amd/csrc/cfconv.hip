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

__device__ __forceinline__ float lanef(float v, int k) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), k));
}

// XCD-aware receiver row of this wave.  Workgroups are dispatched round-robin
// over the 8 XCDs of the chip; the logical block index below gives every XCD
// one contiguous range of rows, so the rows of a frame run together on one
// XCD and the second read of each pair's filter row (once from row i, once
// from row j) hits that XCD's L2 instead of HBM.
constexpr int kXcds = 8;

__device__ __forceinline__ int64_t xcd_row() {
  const int nb = gridDim.x, b = blockIdx.x;
  const int x = b % kXcds, local = b / kXcds;
  const int base = nb / kXcds, rem = nb % kXcds;
  const int lb = x * base + min(x, rem) + local;
  return (int64_t)lb * kWaves + threadIdx.x / MLCG_WAVE;
}

// Iterate the row of wave-uniform receiver i in chunks of 64 edges: lane k
// holds col/pair of edge chunk_start + k; `split` is the first edge of the
// chunk whose neighbour j exceeds i (rows are sorted by j, so edges before it
// are lower edges j < i and edges from it on are upper edges j > i).
#define MLCG_ROW_LOOP_BEGIN(i)                                                  \
  const int e_begin = uniform(rowptr[i]);                                       \
  const int e_end = uniform(rowptr[(i) + 1]);                                   \
  for (int c0 = e_begin; c0 < e_end; c0 += MLCG_WAVE) {                         \
    const int cn = min(MLCG_WAVE, e_end - c0);                                  \
    const int my_col = lane < cn ? col[c0 + lane] : 0;                          \
    const int my_pair = lane < cn ? eid2pair[c0 + lane] : 0;                    \
    const uint64_t up_mask = __ballot(lane < cn && my_col > (int)(i));          \
    const int split = up_mask ? (int)__builtin_ctzll(up_mask) : cn;

#define MLCG_ROW_LOOP_END }

__global__ __launch_bounds__(kThreads) void gather_kernel(
    const float* __restrict__ src, const void* __restrict__ W, int w_f16,
    const int32_t* __restrict__ rowptr, const int32_t* __restrict__ col,
    const int32_t* __restrict__ eid2pair, int64_t n, float* __restrict__ out) {
  const int lane = mlcg_lane();
  const bool f16 = w_f16 != 0;
  const int64_t i = xcd_row();
  if (i >= n) return;
  F2 acc{0.f, 0.f};
  MLCG_ROW_LOOP_BEGIN(i)
  (void)split;
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

// ybar[i] = sum_j gagg[j] W_ij (all edges, ascending j) and, on the upper
// edges (i < j) that own pair p, dbar[p] += <Wd_p, gagg_i y_j + gagg_j y_i>.
__global__ __launch_bounds__(kThreads) void gather_bwd_kernel(
    const float* __restrict__ gagg, const float* __restrict__ y, const void* __restrict__ W,
    const void* __restrict__ Wd, int w_f16, const int32_t* __restrict__ rowptr,
    const int32_t* __restrict__ col, const int32_t* __restrict__ eid2pair, int64_t n,
    float* __restrict__ ybar, float* __restrict__ dbar) {
  const int lane = mlcg_lane();
  const bool f16 = w_f16 != 0;
  const int64_t i = xcd_row();
  if (i >= n) return;
  const F2 gi = ld2(gagg, i, lane);
  const F2 yi = ld2(y, i, lane);
  F2 acc{0.f, 0.f};
  MLCG_ROW_LOOP_BEGIN(i)
  int k = 0;
  // lower edges: gather only
  for (; k + kUnroll <= split; k += kUnroll) {
    F2 g[kUnroll], w[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int j = __builtin_amdgcn_readlane(my_col, k + u);
      const int p = __builtin_amdgcn_readlane(my_pair, k + u);
      g[u] = ld2(gagg, j, lane);
      w[u] = ldw(W, f16, p, lane);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      acc.x += g[u].x * w[u].x;
      acc.y += g[u].y * w[u].y;
    }
  }
  for (; k < split; ++k) {
    const int j = __builtin_amdgcn_readlane(my_col, k);
    const int p = __builtin_amdgcn_readlane(my_pair, k);
    const F2 g = ld2(gagg, j, lane), w = ldw(W, f16, p, lane);
    acc.x += g.x * w.x;
    acc.y += g.y * w.y;
  }
  // upper edges: gather plus the pair's distance adjoint
  for (; k + kUnroll <= cn; k += kUnroll) {
    F2 g[kUnroll], w[kUnroll], yj[kUnroll], wd[kUnroll];
    int p[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int j = __builtin_amdgcn_readlane(my_col, k + u);
      p[u] = __builtin_amdgcn_readlane(my_pair, k + u);
      g[u] = ld2(gagg, j, lane);
      w[u] = ldw(W, f16, p[u], lane);
      yj[u] = ld2(y, j, lane);
      wd[u] = ldw(Wd, f16, p[u], lane);
    }
    float part[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      acc.x += g[u].x * w[u].x;
      acc.y += g[u].y * w[u].y;
      part[u] = wd[u].x * (gi.x * yj[u].x + g[u].x * yi.x) +
                wd[u].y * (gi.y * yj[u].y + g[u].y * yi.y);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) part[u] += __shfl_xor(part[u], o, MLCG_WAVE);
    if (lane == 0)
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) dbar[p[u]] += part[u];
  }
  for (; k < cn; ++k) {
    const int j = __builtin_amdgcn_readlane(my_col, k);
    const int p = __builtin_amdgcn_readlane(my_pair, k);
    const F2 g = ld2(gagg, j, lane), w = ldw(W, f16, p, lane);
    const F2 yj = ld2(y, j, lane), wd = ldw(Wd, f16, p, lane);
    acc.x += g.x * w.x;
    acc.y += g.y * w.y;
    float part = wd.x * (gi.x * yj.x + g.x * yi.x) + wd.y * (gi.y * yj.y + g.y * yi.y);
    part = mlcg_wave_sum(part);
    if (lane == 0) dbar[p] += part;
  }
  MLCG_ROW_LOOP_END
  st2(ybar, i, lane, acc);
}

// out[i] = sum_j ydot[j] W_ij + y[j] Wd_ij ddot_p (ydot may be null).
__global__ __launch_bounds__(kThreads) void gather_tangent_kernel(
    const float* __restrict__ ydot, const float* __restrict__ y, const float* __restrict__ W,
    const float* __restrict__ Wd, const float* __restrict__ ddot,
    const int32_t* __restrict__ rowptr, const int32_t* __restrict__ col,
    const int32_t* __restrict__ eid2pair, int64_t n, float* __restrict__ out) {
  const int lane = mlcg_lane();
  const int64_t i = xcd_row();
  if (i >= n) return;
  const bool has_ydot = ydot != nullptr;
  F2 acc{0.f, 0.f};
  MLCG_ROW_LOOP_BEGIN(i)
  (void)split;
  const float my_dd = lane < cn ? ddot[my_pair] : 0.f;
  int k = 0;
  for (; k + kUnroll <= cn; k += kUnroll) {
    F2 yj[kUnroll], wd[kUnroll], yd[kUnroll], w[kUnroll];
    float dd[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int j = __builtin_amdgcn_readlane(my_col, k + u);
      const int p = __builtin_amdgcn_readlane(my_pair, k + u);
      dd[u] = lanef(my_dd, k + u);
      yj[u] = ld2(y, j, lane);
      wd[u] = ld2(Wd, p, lane);
      if (has_ydot) {
        yd[u] = ld2(ydot, j, lane);
        w[u] = ld2(W, p, lane);
      } else {
        yd[u] = F2{0.f, 0.f};
        w[u] = F2{0.f, 0.f};
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      acc.x += yd[u].x * w[u].x + yj[u].x * (wd[u].x * dd[u]);
      acc.y += yd[u].y * w[u].y + yj[u].y * (wd[u].y * dd[u]);
    }
  }
  for (; k < cn; ++k) {
    const int j = __builtin_amdgcn_readlane(my_col, k);
    const int p = __builtin_amdgcn_readlane(my_pair, k);
    const float dd = lanef(my_dd, k);
    const F2 yj = ld2(y, j, lane), wd = ld2(Wd, p, lane);
    F2 yd{0.f, 0.f}, w{0.f, 0.f};
    if (has_ydot) {
      yd = ld2(ydot, j, lane);
      w = ld2(W, p, lane);
    }
    acc.x += yd.x * w.x + yj.x * (wd.x * dd);
    acc.y += yd.y * w.y + yj.y * (wd.y * dd);
  }
  MLCG_ROW_LOOP_END
  st2(out, i, lane, acc);
}

// Reverse over (primal, tangent) of the aggregation (see mlcg_hip.h):
//   ybar2[i] = sum_j gagg2[j] W_ij + gagg1[j] Wd_ij ddot_p
// and on the upper edges of pair p:
//   Wbar[p]  = gagg2_i y_j + gagg2_j y_i + gagg1_i ydot_j + gagg1_j ydot_i
//   Wdbar[p] = ddot_p (gagg1_i y_j + gagg1_j y_i)
template <bool kTangent>
__device__ __forceinline__ void rev2_edge(int lane, int64_t p, float dd, F2 g2j, F2 w, F2 g1j,
                                          F2 wd, F2& acc) {
  if (kTangent) {
    acc.x += g2j.x * w.x + g1j.x * (wd.x * dd);
    acc.y += g2j.y * w.y + g1j.y * (wd.y * dd);
  } else {
    acc.x += g2j.x * w.x;
    acc.y += g2j.y * w.y;
  }
}

template <bool kTangent>
__global__ __launch_bounds__(kThreads) void gather_rev2_kernel(
    const float* __restrict__ gagg2, const float* __restrict__ gagg1,
    const float* __restrict__ y, const float* __restrict__ ydot, const float* __restrict__ W,
    const float* __restrict__ Wd, const float* __restrict__ ddot,
    const int32_t* __restrict__ rowptr, const int32_t* __restrict__ col,
    const int32_t* __restrict__ eid2pair, int64_t n, float* __restrict__ ybar2,
    float* __restrict__ Wbar, float* __restrict__ Wdbar) {
  const int lane = mlcg_lane();
  const int64_t i = xcd_row();
  if (i >= n) return;
  const bool has_ydot = ydot != nullptr;
  const F2 g2i = ld2(gagg2, i, lane);
  const F2 yi = ld2(y, i, lane);
  const F2 g1i = kTangent ? ld2(gagg1, i, lane) : F2{0.f, 0.f};
  const F2 ydi = (kTangent && has_ydot) ? ld2(ydot, i, lane) : F2{0.f, 0.f};
  F2 acc{0.f, 0.f};
  const bool want_adj = Wbar != nullptr;
  MLCG_ROW_LOOP_BEGIN(i)
  const float my_dd = (kTangent && lane < cn) ? ddot[my_pair] : 0.f;
  // without pair-adjoint outputs every edge is a plain gather edge
  const int lo_end = want_adj ? split : cn;
  int k = 0;
  // lower edges: only the gather into ybar2
  for (; k + kUnroll <= lo_end; k += kUnroll) {
    F2 g2j[kUnroll], w[kUnroll], g1j[kUnroll], wd[kUnroll];
    float dd[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int j = __builtin_amdgcn_readlane(my_col, k + u);
      const int p = __builtin_amdgcn_readlane(my_pair, k + u);
      dd[u] = lanef(my_dd, k + u);
      g2j[u] = ld2(gagg2, j, lane);
      w[u] = ld2(W, p, lane);
      g1j[u] = kTangent ? ld2(gagg1, j, lane) : F2{0.f, 0.f};
      wd[u] = kTangent ? ld2(Wd, p, lane) : F2{0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      rev2_edge<kTangent>(lane, 0, dd[u], g2j[u], w[u], g1j[u], wd[u], acc);
  }
  for (; k < lo_end; ++k) {
    const int j = __builtin_amdgcn_readlane(my_col, k);
    const int p = __builtin_amdgcn_readlane(my_pair, k);
    const F2 g2j = ld2(gagg2, j, lane), w = ld2(W, p, lane);
    const F2 g1j = kTangent ? ld2(gagg1, j, lane) : F2{0.f, 0.f};
    const F2 wd = kTangent ? ld2(Wd, p, lane) : F2{0.f, 0.f};
    rev2_edge<kTangent>(lane, 0, lanef(my_dd, k), g2j, w, g1j, wd, acc);
  }
  // upper edges: gather plus the pair adjoints of W and Wd
  for (; k < cn; ++k) {
    const int j = __builtin_amdgcn_readlane(my_col, k);
    const int p = __builtin_amdgcn_readlane(my_pair, k);
    const float dd = lanef(my_dd, k);
    const F2 g2j = ld2(gagg2, j, lane), w = ld2(W, p, lane);
    const F2 g1j = kTangent ? ld2(gagg1, j, lane) : F2{0.f, 0.f};
    const F2 wd = kTangent ? ld2(Wd, p, lane) : F2{0.f, 0.f};
    const F2 yj = ld2(y, j, lane);
    const F2 ydj = (kTangent && has_ydot) ? ld2(ydot, j, lane) : F2{0.f, 0.f};
    rev2_edge<kTangent>(lane, p, dd, g2j, w, g1j, wd, acc);
    F2 wb, wdb{0.f, 0.f};
    wb.x = g2i.x * yj.x + g2j.x * yi.x;
    wb.y = g2i.y * yj.y + g2j.y * yi.y;
    if (kTangent) {
      wb.x += g1i.x * ydj.x + g1j.x * ydi.x;
      wb.y += g1i.y * ydj.y + g1j.y * ydi.y;
      wdb.x = dd * (g1i.x * yj.x + g1j.x * yi.x);
      wdb.y = dd * (g1i.y * yj.y + g1j.y * yi.y);
    }
    st2(Wbar, p, lane, wb);
    st2(Wdbar, p, lane, wdb);
  }
  MLCG_ROW_LOOP_END
  st2(ybar2, i, lane, acc);
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

// one wave per receiver row, kWaves rows per workgroup (see xcd_row)
unsigned row_groups(int64_t n) { return mlcg_div_up(n, kWaves); }

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
  MLCG_REQUIRE(gagg2 && y && W && rowptr && col && eid2pair && ybar2);
  MLCG_REQUIRE((Wbar == nullptr) == (Wdbar == nullptr));
  MLCG_REQUIRE(!gagg1 || (Wd && ddot));
  if (gagg1)
    hipLaunchKernelGGL(gather_rev2_kernel<true>, dim3(row_groups(n_nodes)), dim3(kThreads), 0,
                       mlcg_stream(stream), gagg2, gagg1, y, ydot, W, Wd, ddot, rowptr, col,
                       eid2pair, n_nodes, ybar2, Wbar, Wdbar);
  else
    hipLaunchKernelGGL(gather_rev2_kernel<false>, dim3(row_groups(n_nodes)), dim3(kThreads), 0,
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
