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
// Mapping: one wave per receiver row.  The two half-waves take consecutive
// edges of the row (edges 2t and 2t + 1), and every lane of a half owns 4 of
// the 128 features (float4), so one step moves two W rows and two node rows
// (2 x 512 B each) with one 16-byte load per lane and tensor.  The row's
// (col, pair) indices are fetched 64 at a time by the lanes and broadcast
// with readlane; the loads of several steps are issued before their
// products are accumulated.  Each half accumulates its edges in ascending
// order and the two halves are added at the end, so the result does not
// depend on timing.
#include "common.h"
#include "split16.h"

#include <hip/hip_fp16.h>

namespace {

constexpr int kF = 128;
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * MLCG_WAVE;
#ifndef MLCG_GATHER_STEPS
#define MLCG_GATHER_STEPS 4
#endif
constexpr int kSteps = MLCG_GATHER_STEPS;  // steps (2 edges each) with loads in flight together

__device__ __forceinline__ float4 f4zero() { return float4{0.f, 0.f, 0.f, 0.f}; }

// Row `row` of a [*, 128] fp32 tensor, features 4m .. 4m + 3.
__device__ __forceinline__ float4 ld4(const float* __restrict__ p, int64_t row, int m) {
  return *reinterpret_cast<const float4*>(p + row * kF + 4 * m);
}

__device__ __forceinline__ float4 ldw4(const void* __restrict__ W, bool f16, int64_t row, int m) {
  if (f16) {
    const __half2* h = reinterpret_cast<const __half2*>(static_cast<const __half*>(W) + row * kF +
                                                        4 * m);
    const float2 a = __half22float2(h[0]), b = __half22float2(h[1]);
    return float4{a.x, a.y, b.x, b.y};
  }
  return ld4(static_cast<const float*>(W), row, m);
}

__device__ __forceinline__ void st4(float* __restrict__ p, int64_t row, int m, float4 v) {
  *reinterpret_cast<float4*>(p + row * kF + 4 * m) = v;
}

__device__ __forceinline__ void fma4(float4& acc, float4 a, float4 b) {
  acc.x += a.x * b.x;
  acc.y += a.y * b.y;
  acc.z += a.z * b.z;
  acc.w += a.w * b.w;
}

__device__ __forceinline__ float dot4(float4 a, float4 b) {
  return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ float lanef(float v, int k) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), k));
}

// Sum over the 32 lanes of a half-wave, returned to all of them (DPP and
// v_permlane16_swap: no LDS round trips).
__device__ __forceinline__ float half_sum(float v) { return half32_sum(v); }

// Adds the other half-wave's accumulator (lanes l and l ^ 32 hold the same
// features): lower half first, then upper half, on both.
__device__ __forceinline__ float4 combine_halves(float4 a, int h) {
  float4 o;
  o.x = __shfl_xor(a.x, 32, MLCG_WAVE);
  o.y = __shfl_xor(a.y, 32, MLCG_WAVE);
  o.z = __shfl_xor(a.z, 32, MLCG_WAVE);
  o.w = __shfl_xor(a.w, 32, MLCG_WAVE);
  return h == 0 ? float4{a.x + o.x, a.y + o.y, a.z + o.z, a.w + o.w}
                : float4{o.x + a.x, o.y + a.y, o.z + a.z, o.w + a.w};
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

// Edge of half h at step base k (k even, so k + 1 <= 63): its neighbour,
// pair, the per-edge scalar `sv` (lane k / k + 1 of v) and whether it exists.
struct Edge {
  int j, p;
  float sv;
  bool ok;
};

__device__ __forceinline__ Edge edge_at(int k, int h, int cn, int my_col, int my_pair,
                                        float v) {
  const int ja = __builtin_amdgcn_readlane(my_col, k);
  const int jb = __builtin_amdgcn_readlane(my_col, k + 1);
  const int pa = __builtin_amdgcn_readlane(my_pair, k);
  const int pb = __builtin_amdgcn_readlane(my_pair, k + 1);
  const float va = lanef(v, k), vb = lanef(v, k + 1);
  Edge e;
  e.j = h ? jb : ja;
  e.p = h ? pb : pa;
  e.sv = h ? vb : va;
  e.ok = k + h < cn;
  return e;
}

__global__ __launch_bounds__(kThreads) void gather_kernel(
    const float* __restrict__ src, const void* __restrict__ W, int w_f16,
    const int32_t* __restrict__ rowptr, const int32_t* __restrict__ col,
    const int32_t* __restrict__ eid2pair, int64_t n, float* __restrict__ out) {
  const int lane = mlcg_lane();
  const int h = lane >> 5, m = lane & 31;
  const bool f16 = w_f16 != 0;
  const int64_t i = xcd_row();
  if (i >= n) return;
  float4 acc = f4zero();
  MLCG_ROW_LOOP_BEGIN(i)
  (void)split;
  int k = 0;
  for (; k + 2 * kSteps <= cn; k += 2 * kSteps) {
    float4 sv[kSteps], wv[kSteps];
#pragma unroll
    for (int u = 0; u < kSteps; ++u) {
      const Edge e = edge_at(k + 2 * u, h, cn, my_col, my_pair, 0.f);
      sv[u] = ld4(src, e.j, m);
      wv[u] = ldw4(W, f16, e.p, m);
    }
#pragma unroll
    for (int u = 0; u < kSteps; ++u) fma4(acc, sv[u], wv[u]);
  }
  for (; k < cn; k += 2) {
    const Edge e = edge_at(k, h, cn, my_col, my_pair, 0.f);
    if (e.ok) fma4(acc, ld4(src, e.j, m), ldw4(W, f16, e.p, m));
  }
  MLCG_ROW_LOOP_END
  acc = combine_halves(acc, h);
  if (h == 0) st4(out, i, m, acc);
}

// ybar[i] = sum_j gagg[j] W_ij (all edges) and, on the upper edges (i < j)
// that own pair p, dbar[p] += <Wd_p, gagg_i y_j + gagg_j y_i> (dbar[p] = ...
// with accumulate == 0, so the first of a model's blocks needs no zeroed
// dbar).  The steps of
// upper edges keep kUp steps (four loads per edge) in flight: its registers
// set the kernel's occupancy, lower-edge steps included.
// <Wd, gi yj + gj yi> of one lane's four features, in a fixed fma order
// (the backend would otherwise contract the products differently in each
// instantiation of the kernel, and the two gather_bwd forms must agree).
__device__ __forceinline__ float dbar_term(float4 wd, float4 gi, float4 yj, float4 gj,
                                           float4 yi) {
  const float tx = __builtin_fmaf(gi.x, yj.x, __fmul_rn(gj.x, yi.x));
  const float ty = __builtin_fmaf(gi.y, yj.y, __fmul_rn(gj.y, yi.y));
  const float tz = __builtin_fmaf(gi.z, yj.z, __fmul_rn(gj.z, yi.z));
  const float tw = __builtin_fmaf(gi.w, yj.w, __fmul_rn(gj.w, yi.w));
  return __builtin_fmaf(wd.w, tw, __builtin_fmaf(wd.z, tz,
                                                 __builtin_fmaf(wd.y, ty, __fmul_rn(wd.x, tx))));
}

// kYbar = false: dbar only (no ybar): the lower edges, which add to ybar
// alone, are skipped, and the upper edges load no filter rows W; their dbar
// terms are formed by the same code, so they equal the full kernel's bit for
// bit.  (A model's first block needs no ybar on the force sweep: its input
// is the embedding, which does not depend on the positions.)
template <int kUp, bool kYbar>
__global__ __launch_bounds__(kThreads) void gather_bwd_kernel(
    const float* __restrict__ gagg, const float* __restrict__ y, const void* __restrict__ W,
    const void* __restrict__ Wd, int w_f16, const int32_t* __restrict__ rowptr,
    const int32_t* __restrict__ col, const int32_t* __restrict__ eid2pair, int64_t n,
    float* __restrict__ ybar, float* __restrict__ dbar, int accumulate) {
  const int lane = mlcg_lane();
  const int h = lane >> 5, m = lane & 31;
  const bool f16 = w_f16 != 0;
  const int64_t i = xcd_row();
  if (i >= n) return;
  const float4 gi = ld4(gagg, i, m);
  const float4 yi = ld4(y, i, m);
  float4 acc = f4zero();
  MLCG_ROW_LOOP_BEGIN(i)
  // steps before the first step that holds an upper edge: gather only
  const int lo_steps_end = split & ~1;
  int k = 0;
  if constexpr (kYbar) {
    for (; k + 2 * kSteps <= lo_steps_end; k += 2 * kSteps) {
      float4 g[kSteps], w[kSteps];
#pragma unroll
      for (int u = 0; u < kSteps; ++u) {
        const Edge e = edge_at(k + 2 * u, h, cn, my_col, my_pair, 0.f);
        g[u] = ld4(gagg, e.j, m);
        w[u] = ldw4(W, f16, e.p, m);
      }
#pragma unroll
      for (int u = 0; u < kSteps; ++u) fma4(acc, g[u], w[u]);
    }
    for (; k < lo_steps_end; k += 2) {
      const Edge e = edge_at(k, h, cn, my_col, my_pair, 0.f);
      fma4(acc, ld4(gagg, e.j, m), ldw4(W, f16, e.p, m));
    }
  } else {
    k = lo_steps_end;
  }
  // remaining steps: gather, plus the distance adjoint on upper edges
  for (; k < cn; k += 2 * kUp) {
    float4 g[kUp], w[kUp], yj[kUp], wd[kUp];
    int p[kUp];
    bool ok[kUp], up[kUp];
#pragma unroll
    for (int u = 0; u < kUp; ++u) {
      const Edge e = edge_at(k + 2 * u < 62 ? k + 2 * u : 62, h, cn, my_col, my_pair, 0.f);
      const int ke = k + 2 * u + h;
      ok[u] = k + 2 * u < cn && ke < cn;
      up[u] = ok[u] && ke >= split;
      p[u] = e.p;
      g[u] = (kYbar ? ok[u] : up[u]) ? ld4(gagg, e.j, m) : f4zero();
      w[u] = kYbar && ok[u] ? ldw4(W, f16, e.p, m) : f4zero();
      yj[u] = up[u] ? ld4(y, e.j, m) : f4zero();
      wd[u] = up[u] ? ldw4(Wd, f16, e.p, m) : f4zero();
    }
    float part[kUp];
#pragma unroll
    for (int u = 0; u < kUp; ++u) {
      if constexpr (kYbar) fma4(acc, g[u], w[u]);
      part[u] = dbar_term(wd[u], gi, yj[u], g[u], yi);
    }
#pragma unroll
    for (int u = 0; u < kUp; ++u) part[u] = half_sum(part[u]);
    // each pair has exactly one upper edge, so one write per address and
    // launch: a plain store, or a returnless float atomic (performed in the
    // L2) that adds without the dependent load of a read-modify-write holding
    // up the next step
    if (m == 0) {
      if (accumulate) {
#pragma unroll
        for (int u = 0; u < kUp; ++u)
          if (up[u]) unsafeAtomicAdd(dbar + p[u], part[u]);
      } else {
#pragma unroll
        for (int u = 0; u < kUp; ++u)
          if (up[u]) dbar[p[u]] = part[u];
      }
    }
  }
  MLCG_ROW_LOOP_END
  if constexpr (kYbar) {
    acc = combine_halves(acc, h);
    if (h == 0) st4(ybar, i, m, acc);
  }
}

// out[i] = sum_j ydot[j] W_ij + y[j] Wd_ij ddot_p (ydot may be null).
__global__ __launch_bounds__(kThreads) void gather_tangent_kernel(
    const float* __restrict__ ydot, const float* __restrict__ y, const float* __restrict__ W,
    const float* __restrict__ Wd, const float* __restrict__ ddot,
    const int32_t* __restrict__ rowptr, const int32_t* __restrict__ col,
    const int32_t* __restrict__ eid2pair, int64_t n, float* __restrict__ out) {
  const int lane = mlcg_lane();
  const int h = lane >> 5, m = lane & 31;
  const int64_t i = xcd_row();
  if (i >= n) return;
  const bool has_ydot = ydot != nullptr;
  float4 acc = f4zero();
  MLCG_ROW_LOOP_BEGIN(i)
  (void)split;
  const float my_dd = lane < cn ? ddot[my_pair] : 0.f;
  for (int k = 0; k < cn; k += 2 * kSteps) {
    float4 yj[kSteps], wd[kSteps], yd[kSteps], w[kSteps];
    float dd[kSteps];
#pragma unroll
    for (int u = 0; u < kSteps; ++u) {
      const int kb = k + 2 * u < 62 ? k + 2 * u : 62;
      const Edge e = edge_at(kb, h, cn, my_col, my_pair, my_dd);
      const bool ok = k + 2 * u + h < cn;
      dd[u] = ok ? e.sv : 0.f;
      yj[u] = ok ? ld4(y, e.j, m) : f4zero();
      wd[u] = ok ? ld4(Wd, e.p, m) : f4zero();
      yd[u] = (ok && has_ydot) ? ld4(ydot, e.j, m) : f4zero();
      w[u] = (ok && has_ydot) ? ld4(W, e.p, m) : f4zero();
    }
#pragma unroll
    for (int u = 0; u < kSteps; ++u) {
      acc.x += yd[u].x * w[u].x + yj[u].x * (wd[u].x * dd[u]);
      acc.y += yd[u].y * w[u].y + yj[u].y * (wd[u].y * dd[u]);
      acc.z += yd[u].z * w[u].z + yj[u].z * (wd[u].z * dd[u]);
      acc.w += yd[u].w * w[u].w + yj[u].w * (wd[u].w * dd[u]);
    }
  }
  MLCG_ROW_LOOP_END
  acc = combine_halves(acc, h);
  if (h == 0) st4(out, i, m, acc);
}

// Reverse over (primal, tangent) of the aggregation (see mlcg_hip.h):
//   ybar2[i] = sum_j gagg2[j] W_ij + gagg1[j] Wd_ij ddot_p
// and on the upper edges of pair p (when Wbar is given):
//   Wbar[p]  = gagg2_i y_j + gagg2_j y_i + gagg1_i ydot_j + gagg1_j ydot_i
//   Wdbar[p] = ddot_p (gagg1_i y_j + gagg1_j y_i)
// The pair-adjoint path is a template parameter: compiled in, its node rows of
// i and edge state hold 140 VGPRs (3 waves per SIMD); without it the kernel
// needs about 90 (5 waves per SIMD), as the tangent gather does.
template <bool kTangent, bool kAdj>
__global__ __launch_bounds__(kThreads) void gather_rev2_kernel(
    const float* __restrict__ gagg2, const float* __restrict__ gagg1,
    const float* __restrict__ y, const float* __restrict__ ydot, const float* __restrict__ W,
    const float* __restrict__ Wd, const float* __restrict__ ddot,
    const int32_t* __restrict__ rowptr, const int32_t* __restrict__ col,
    const int32_t* __restrict__ eid2pair, int64_t n, float* __restrict__ ybar2,
    float* __restrict__ Wbar, float* __restrict__ Wdbar) {
  const int lane = mlcg_lane();
  const int h = lane >> 5, m = lane & 31;
  const int64_t i = xcd_row();
  if (i >= n) return;
  const bool has_ydot = ydot != nullptr;
  constexpr bool want_adj = kAdj;
  const float4 g2i = want_adj ? ld4(gagg2, i, m) : f4zero();
  const float4 yi = want_adj ? ld4(y, i, m) : f4zero();
  const float4 g1i = (kTangent && want_adj) ? ld4(gagg1, i, m) : f4zero();
  const float4 ydi = (kTangent && want_adj && has_ydot) ? ld4(ydot, i, m) : f4zero();
  float4 acc = f4zero();
  MLCG_ROW_LOOP_BEGIN(i)
  const float my_dd = (kTangent && lane < cn) ? ddot[my_pair] : 0.f;
  for (int k = 0; k < cn; k += 2 * kSteps) {
    float4 g2j[kSteps], w[kSteps], g1j[kSteps], wd[kSteps];
    float dd[kSteps];
    bool ok[kSteps];
    Edge ed[kSteps];
#pragma unroll
    for (int u = 0; u < kSteps; ++u) {
      const int kb = k + 2 * u < 62 ? k + 2 * u : 62;
      ed[u] = edge_at(kb, h, cn, my_col, my_pair, my_dd);
      ok[u] = k + 2 * u + h < cn;
      dd[u] = ok[u] ? ed[u].sv : 0.f;
      g2j[u] = ok[u] ? ld4(gagg2, ed[u].j, m) : f4zero();
      w[u] = ok[u] ? ld4(W, ed[u].p, m) : f4zero();
      g1j[u] = (kTangent && ok[u]) ? ld4(gagg1, ed[u].j, m) : f4zero();
      wd[u] = (kTangent && ok[u]) ? ld4(Wd, ed[u].p, m) : f4zero();
    }
#pragma unroll
    for (int u = 0; u < kSteps; ++u) {
      fma4(acc, g2j[u], w[u]);
      if (kTangent) {
        acc.x += g1j[u].x * (wd[u].x * dd[u]);
        acc.y += g1j[u].y * (wd[u].y * dd[u]);
        acc.z += g1j[u].z * (wd[u].z * dd[u]);
        acc.w += g1j[u].w * (wd[u].w * dd[u]);
      }
    }
    if constexpr (want_adj) {
#pragma unroll
      for (int u = 0; u < kSteps; ++u) {
        if (!(ok[u] && k + 2 * u + h >= split)) continue;
        const float4 yj = ld4(y, ed[u].j, m);
        const float4 ydj = (kTangent && has_ydot) ? ld4(ydot, ed[u].j, m) : f4zero();
        float4 wb{g2i.x * yj.x + g2j[u].x * yi.x, g2i.y * yj.y + g2j[u].y * yi.y,
                  g2i.z * yj.z + g2j[u].z * yi.z, g2i.w * yj.w + g2j[u].w * yi.w};
        float4 wdb = f4zero();
        if (kTangent) {
          wb.x += g1i.x * ydj.x + g1j[u].x * ydi.x;
          wb.y += g1i.y * ydj.y + g1j[u].y * ydi.y;
          wb.z += g1i.z * ydj.z + g1j[u].z * ydi.z;
          wb.w += g1i.w * ydj.w + g1j[u].w * ydi.w;
          const float d = dd[u];
          wdb = float4{d * (g1i.x * yj.x + g1j[u].x * yi.x), d * (g1i.y * yj.y + g1j[u].y * yi.y),
                       d * (g1i.z * yj.z + g1j[u].z * yi.z), d * (g1i.w * yj.w + g1j[u].w * yi.w)};
        }
        st4(Wbar, ed[u].p, m, wb);
        st4(Wdbar, ed[u].p, m, wdb);
      }
    }
  }
  MLCG_ROW_LOOP_END
  acc = combine_halves(acc, h);
  if (h == 0) st4(ybar2, i, m, acc);
}

__global__ void pair_ddot_kernel(const float* __restrict__ pos, const float* __restrict__ dist,
                                 const int32_t* __restrict__ pi, const int32_t* __restrict__ pj,
                                 const int32_t* __restrict__ n_pairs_dev, int64_t max_pairs,
                                 const float* __restrict__ u, float scale,
                                 float* __restrict__ ddot) {
  int64_t np = *n_pairs_dev;
  if (np > max_pairs) np = max_pairs;
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < np;
       p += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = pi[p], j = pj[p];
    const float inv = 1.0f / dist[p];
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < 3; ++c) acc += (pos[3 * j + c] - pos[3 * i + c]) * (u[3 * j + c] - u[3 * i + c]);
    ddot[p] = (acc * inv) * scale;
  }
}

// 16 lanes per node: lane `sub` takes the node's edges sub, sub + 16, ...,
// and the 16 partial forces are added by a fixed xor butterfly, so the
// result does not depend on timing.
constexpr int kForceLanes = 16;

__global__ __launch_bounds__(256) void pair_forces_kernel(
    const float* __restrict__ pos, const float* __restrict__ dist,
    const float* __restrict__ dbar, const int32_t* __restrict__ rowptr,
    const int32_t* __restrict__ col, const int32_t* __restrict__ eid2pair, int64_t n,
    int accumulate, float* __restrict__ forces) {
  const int sub = threadIdx.x % kForceLanes;
  const int64_t i = (int64_t)blockIdx.x * (256 / kForceLanes) + threadIdx.x / kForceLanes;
  float fx = 0.f, fy = 0.f, fz = 0.f;
  if (i < n) {
    const float xi = pos[3 * i], yi = pos[3 * i + 1], zi = pos[3 * i + 2];
    const int e1 = rowptr[i + 1];
    for (int e = rowptr[i] + sub; e < e1; e += kForceLanes) {
      const int64_t j = col[e];
      const int p = eid2pair[e];
      const float s = dbar[p] / dist[p];
      fx += s * (pos[3 * j] - xi);
      fy += s * (pos[3 * j + 1] - yi);
      fz += s * (pos[3 * j + 2] - zi);
    }
  }
#pragma unroll
  for (int o = kForceLanes / 2; o > 0; o >>= 1) {
    fx += __shfl_xor(fx, o, kForceLanes);
    fy += __shfl_xor(fy, o, kForceLanes);
    fz += __shfl_xor(fz, o, kForceLanes);
  }
  if (i < n && sub == 0) {
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
constexpr int kSegThreads = 1024;
constexpr int kSegWaves = kSegThreads / MLCG_WAVE;
constexpr int kSegLoads = 4;  // 16-byte loads in flight per thread

// Compensated (Kahan) accumulation of y into (s, c).
__device__ __forceinline__ void kahan_add(float& s, float& c, float y) {
  const float yy = y - c;
  const float t = s + yy;
  c = (t - s) - yy;
  s = t;
}

// out[b] = sum of v[k * stride] over the frame's k in [ptr[b], ptr[b+1]).  One
// workgroup per frame (grid-stride over frames); with stride 1 its 1024
// threads read the frame as 16-byte vectors, kSegLoads in flight per thread,
// after a scalar head up to 16-byte alignment and before a scalar tail (a
// prior's per-interaction energies run to 71,556 values a frame).  Each
// thread keeps a compensated sum over a fixed set of elements; the threads'
// sums are added by a fixed butterfly within each wave and the wave sums in
// wave order, so the result does not depend on timing.
__global__ __launch_bounds__(kSegThreads) void segment_sum_kernel(
    const float* __restrict__ v, int64_t stride, const int64_t* __restrict__ ptr, int64_t nb,
    float* __restrict__ out) {
  __shared__ float part[kSegWaves];
  const int tid = threadIdx.x;
  const int lane = mlcg_lane(), wv = tid / MLCG_WAVE;
  for (int64_t b = blockIdx.x; b < nb; b += gridDim.x) {
    const int64_t k0 = ptr[b], k1 = ptr[b + 1];
    float s = 0.f, c = 0.f;
    if (stride == 1) {
      // aligned body [a0, a1) as float4, head [k0, a0) and tail [a1, k1) scalar
      const int64_t a0 = k0 + ((4 - ((reinterpret_cast<uintptr_t>(v + k0) >> 2) & 3)) & 3);
      const int64_t a1 = a0 < k1 ? a0 + ((k1 - a0) & ~int64_t(3)) : a0;
      if (a0 >= k1) {  // no aligned body
        for (int64_t k = k0 + tid; k < k1; k += kSegThreads) kahan_add(s, c, v[k]);
      } else {
        if (k0 + tid < a0) kahan_add(s, c, v[k0 + tid]);
        const float4* v4 = reinterpret_cast<const float4*>(v + a0);
        const int64_t n4 = (a1 - a0) / 4;
        int64_t q = tid;
        for (; q + (kSegLoads - 1) * kSegThreads < n4; q += kSegLoads * kSegThreads) {
          float4 x[kSegLoads];
#pragma unroll
          for (int u = 0; u < kSegLoads; ++u) x[u] = v4[q + u * kSegThreads];
#pragma unroll
          for (int u = 0; u < kSegLoads; ++u) {
            kahan_add(s, c, x[u].x);
            kahan_add(s, c, x[u].y);
            kahan_add(s, c, x[u].z);
            kahan_add(s, c, x[u].w);
          }
        }
        for (; q < n4; q += kSegThreads) {
          const float4 x = v4[q];
          kahan_add(s, c, x.x);
          kahan_add(s, c, x.y);
          kahan_add(s, c, x.z);
          kahan_add(s, c, x.w);
        }
        if (a1 + tid < k1) kahan_add(s, c, v[a1 + tid]);
      }
    } else {
      for (int64_t k = k0 + tid; k < k1; k += kSegThreads) kahan_add(s, c, v[k * stride]);
    }
    const float ws = mlcg_wave_sum(s);
    if (lane == 0) part[wv] = ws;
    __syncthreads();
    if (tid == 0) {
      float t = 0.f;
      for (int w = 0; w < kSegWaves; ++w) t += part[w];
      out[b] = t;
    }
    __syncthreads();
  }
}

// float64 models (the module path of a model moved to double, as the
// reference's simulations do with dtype="double"): out[i] = sum_j src[j] W_p
// for any feature count F, one wave per receiver row (XCD-aware as above),
// lane l holding features l, l + 64, ...; each feature sums the row's edges in
// CSR order (ascending neighbour), the CPU reference's order.
__global__ __launch_bounds__(kThreads) void gather_f64_kernel(
    const double* __restrict__ src, const double* __restrict__ W, int F,
    const int32_t* __restrict__ rowptr, const int32_t* __restrict__ col,
    const int32_t* __restrict__ eid2pair, int64_t n, double* __restrict__ out) {
  const int lane = mlcg_lane();
  const int64_t i = xcd_row();
  if (i >= n) return;
  const int e0 = uniform(rowptr[i]), e1 = uniform(rowptr[i + 1]);
  for (int f = lane; f < F; f += MLCG_WAVE) {
    double acc = 0.0;
    for (int e = e0; e < e1; ++e) {
      const int64_t j = col[e], p = eid2pair[e];
      acc += src[j * F + f] * W[p * F + f];
    }
    out[i * F + f] = acc;
  }
}

// Per-segment sums of a float64 vector: one workgroup per segment, each
// thread a strided part in order, then the waves' sums (fixed butterfly) in
// wave order.
__global__ __launch_bounds__(kSegThreads) void segment_sum_f64_kernel(
    const double* __restrict__ v, const int64_t* __restrict__ ptr, int64_t nb,
    double* __restrict__ out) {
  __shared__ double part[kSegThreads / MLCG_WAVE];
  for (int64_t b = blockIdx.x; b < nb; b += gridDim.x) {
    double s = 0.0;
    for (int64_t k = ptr[b] + threadIdx.x; k < ptr[b + 1]; k += kSegThreads) s += v[k];
    for (int o = MLCG_WAVE / 2; o > 0; o >>= 1) s += __shfl_xor(s, o, MLCG_WAVE);
    if (mlcg_lane() == 0) part[threadIdx.x / MLCG_WAVE] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
      double t = 0.0;
      for (int w = 0; w < kSegThreads / MLCG_WAVE; ++w) t += part[w];
      out[b] = t;
    }
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
                                      float* dbar, int accumulate, void* stream) {
  if (num_filters != kF) return MLCG_ERR_UNSUPPORTED;
  MLCG_REQUIRE(n_nodes >= 0);
  if (n_nodes == 0) return MLCG_OK;
  MLCG_REQUIRE(gagg && y && W && Wd && rowptr && col && eid2pair && dbar);
  // upper steps in flight: 4 with fp32 filter rows (104 VGPRs, 4 waves per
  // SIMD; config 2, 24 edges a row: 48 us against 54 with 2), 2 with fp16
  // rows (68 VGPRs, 7 waves per SIMD; config 4, 47 edges a row: 0.61 ms
  // against 0.89 with 4); ybar == NULL: dbar only
  const dim3 grid(row_groups(n_nodes)), block(kThreads);
  const auto s = mlcg_stream(stream);
  if (w_f16) {
    if (ybar)
      hipLaunchKernelGGL((gather_bwd_kernel<2, true>), grid, block, 0, s, gagg, y, W, Wd, w_f16,
                         rowptr, col, eid2pair, n_nodes, ybar, dbar, accumulate);
    else
      hipLaunchKernelGGL((gather_bwd_kernel<2, false>), grid, block, 0, s, gagg, y, W, Wd, w_f16,
                         rowptr, col, eid2pair, n_nodes, ybar, dbar, accumulate);
  } else {
    if (ybar)
      hipLaunchKernelGGL((gather_bwd_kernel<kSteps, true>), grid, block, 0, s, gagg, y, W, Wd,
                         w_f16, rowptr, col, eid2pair, n_nodes, ybar, dbar, accumulate);
    else
      hipLaunchKernelGGL((gather_bwd_kernel<kSteps, false>), grid, block, 0, s, gagg, y, W, Wd,
                         w_f16, rowptr, col, eid2pair, n_nodes, ybar, dbar, accumulate);
  }
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
  auto kern = gagg1 ? (Wbar ? gather_rev2_kernel<true, true> : gather_rev2_kernel<true, false>)
                    : (Wbar ? gather_rev2_kernel<false, true> : gather_rev2_kernel<false, false>);
  hipLaunchKernelGGL(kern, dim3(row_groups(n_nodes)), dim3(kThreads), 0, mlcg_stream(stream),
                     gagg2, gagg1, y, ydot, W, Wd, ddot, rowptr, col, eid2pair, n_nodes, ybar2,
                     Wbar, Wdbar);
  return mlcg_launch_status();
}

extern "C" int mlcg_pair_ddot(const float* pos, const float* dist, const int32_t* pair_ij,
                              int64_t pair_stride, const int32_t* n_pairs_dev,
                              int64_t max_pairs, const float* u, float scale, float* ddot,
                              void* stream) {
  MLCG_REQUIRE(max_pairs >= 0 && pair_stride >= max_pairs);
  if (max_pairs == 0) return MLCG_OK;
  MLCG_REQUIRE(pos && dist && pair_ij && n_pairs_dev && u && ddot);
  hipLaunchKernelGGL(pair_ddot_kernel, dim3(mlcg_persistent_groups(mlcg_div_up(max_pairs, 256), 8)),
                     dim3(256), 0, mlcg_stream(stream), pos, dist, pair_ij,
                     pair_ij + pair_stride, n_pairs_dev, max_pairs, u, scale, ddot);
  return mlcg_launch_status();
}

extern "C" int mlcg_pair_forces(const float* pos, const float* dist, const float* dbar,
                                const int32_t* rowptr, const int32_t* col,
                                const int32_t* eid2pair, int64_t n_nodes, int accumulate,
                                float* forces, void* stream) {
  MLCG_REQUIRE(n_nodes >= 0);
  if (n_nodes == 0) return MLCG_OK;
  MLCG_REQUIRE(pos && dist && dbar && rowptr && col && eid2pair && forces);
  hipLaunchKernelGGL(pair_forces_kernel, dim3(mlcg_div_up(n_nodes, 256 / kForceLanes)), dim3(256), 0,
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

extern "C" int mlcg_cfconv_gather_f64(const double* src, const double* W,
                                      const int32_t* rowptr, const int32_t* col,
                                      const int32_t* eid2pair, int64_t n_nodes, int num_filters,
                                      double* out, void* stream) {
  MLCG_REQUIRE(n_nodes >= 0 && num_filters >= 1);
  if (n_nodes == 0) return MLCG_OK;
  MLCG_REQUIRE(src && W && rowptr && col && eid2pair && out);
  hipLaunchKernelGGL(gather_f64_kernel, dim3(row_groups(n_nodes)), dim3(kThreads), 0,
                     mlcg_stream(stream), src, W, num_filters, rowptr, col, eid2pair, n_nodes,
                     out);
  return mlcg_launch_status();
}

extern "C" int mlcg_segment_sum_f64(const double* values, const int64_t* frame_ptr,
                                    int64_t n_frames, double* out, void* stream) {
  MLCG_REQUIRE(n_frames >= 0);
  if (n_frames == 0) return MLCG_OK;
  MLCG_REQUIRE(values && frame_ptr && out);
  hipLaunchKernelGGL(segment_sum_f64_kernel, dim3(mlcg_persistent_groups(n_frames, 8)),
                     dim3(kSegThreads), 0, mlcg_stream(stream), values, frame_ptr, n_frames,
                     out);
  return mlcg_launch_status();
}
