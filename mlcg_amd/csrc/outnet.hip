// Output network of SchNet with its force and force-matching sweeps
// (gfx950, MFMA fp32).
//
// StandardSchNet's output network is MLP([H, HH, 1], last_bias=False)
// (mlcg/nn/schnet.py:462-467, mlp.py:31-58):
//     oz = x W0^T + b0 ;  os = act(oz) ;  o = os . w1 (+ b1)
// per node, with x [N, 128] the last block's output and HH its hidden width.
// Every piece is row-local, so each sweep runs as one kernel over 16-row
// tiles instead of a chain of small library GEMMs, GEMVs and elementwise
// passes:
//
//   out_fwd    o (per-node energy), the saved oz/os, and -- when a reverse
//              seed is given -- the adjoint entering the interaction blocks,
//              xbar = ((seed w1) * act'(oz)) W0.
//   out_rev2   the tangent of the network along xdot (ozdot, odot) and the
//              second reverse sweep of the force-matching double backward:
//              xbar2 = zbar2 W0 with
//                zbar2 = (pw w1) act'(oz) + (tw w1) act''(oz) ozdot,
//              and the weight gradients gW0 = zdotbar^T xdot + zbar2^T x,
//              gb0 = sum zbar2, gW1 = sum tw hdot + pw os, gb1 = sum pw,
//              reduced per workgroup (rows as the MFMA reduction axis) and
//              then across workgroups in a fixed order.
//
// Four waves per workgroup.  The 128 -> HH product gives wave w the hidden
// 16-column tiles w, w+4 (B fragments of W0 kept in registers); the HH -> 128
// product gives wave w output columns 32w..32w+31.
#include "common.h"

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kH = 128;        // input width (hidden_channels)
constexpr int kRowsT = 16;     // rows per tile
constexpr int kThreads = 256;  // 4 waves
constexpr int kXR = kH + 4;    // padded LDS row of [16, 128] tiles

template <int HH>
struct OutDims {
  static constexpr int NT = HH / 16;       // hidden 16-column tiles
  static constexpr int TA = (NT + 3) / 4;  // hidden tiles per wave
  static constexpr int ZR = HH + 4;        // padded LDS row of [16, HH] tiles
  static constexpr int KB = HH / 4;        // MFMA k-steps of the HH -> 128 product
  // partial sums per workgroup: gW0 [HH, 128], gb0 [HH], gW1 [HH], gb1
  static constexpr int PART = HH * kH + 2 * HH + 4;
};

__device__ __forceinline__ float4 ld4(const float* __restrict__ p) {
  return *reinterpret_cast<const float4*>(p);
}

// MFMA step kk of lane group q covers k = 16(kk/4) + 4q + kk%4: a lane's four
// consecutive steps read one float4 of its A row.
__device__ __forceinline__ int kperm(int kk, int q) { return 16 * (kk >> 2) + 4 * q + (kk & 3); }

// Stages rows t*16 .. t*16+15 of a [rows, 128] tensor into LDS (zero past rows).
__device__ __forceinline__ void stage_rows(float* dst, const float* __restrict__ src, int64_t r0,
                                           int64_t rows) {
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const int c = threadIdx.x + m * kThreads;
    const int64_t r = r0 + (c >> 5);
    const float4 v = r < rows ? ld4(src + r * kH + 4 * (c & 31)) : float4{0.f, 0.f, 0.f, 0.f};
    *reinterpret_cast<float4*>(dst + (c >> 5) * kXR + 4 * (c & 31)) = v;
  }
}

// B fragments of the 128 -> HH product (B[k][h] = W0[h][k]) for the hidden
// tiles u = w + 4a of this wave.
template <int HH>
__device__ __forceinline__ void load_bA(float (&bA)[OutDims<HH>::TA][32],
                                        const float* __restrict__ W0, int w, int q, int n) {
  using D = OutDims<HH>;
#pragma unroll
  for (int a = 0; a < D::TA; ++a) {
    const int u = w + 4 * a;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const float4 v = u < D::NT ? ld4(W0 + (16 * u + n) * kH + 16 * m + 4 * q)
                                 : float4{0.f, 0.f, 0.f, 0.f};
      bA[a][4 * m + 0] = v.x;
      bA[a][4 * m + 1] = v.y;
      bA[a][4 * m + 2] = v.z;
      bA[a][4 * m + 3] = v.w;
    }
  }
}

// B fragments of the HH -> 128 product (B[k][c] = W0[k][c]), columns
// 32w + 16c + n.
template <int HH>
__device__ __forceinline__ void load_bB(float (&bB)[2][OutDims<HH>::KB],
                                        const float* __restrict__ W0, int w, int q, int n) {
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int kk = 0; kk < OutDims<HH>::KB; ++kk)
      bB[c][kk] = W0[kperm(kk, q) * kH + 32 * w + 16 * c + n];
}

// acc[a] += x_tile (LDS) . W0^T for this wave's hidden tiles.
template <int HH>
__device__ __forceinline__ void gemm_a(floatx4 (&acc)[OutDims<HH>::TA], const float* xs,
                                       const float (&bA)[OutDims<HH>::TA][32], int w, int q,
                                       int n) {
  using D = OutDims<HH>;
#pragma unroll
  for (int a = 0; a < D::TA; ++a) acc[a] = floatx4{0.f, 0.f, 0.f, 0.f};
  if (w >= D::NT) return;  // wave-uniform: waves without a hidden tile
  const float* xa = xs + n * kXR + 4 * q;
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const float4 v = ld4(xa + 16 * m);
    const float av[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int a = 0; a < D::TA; ++a)
        if (w + 4 * a < D::NT)
          acc[a] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j], bA[a][4 * m + j], acc[a], 0, 0, 0);
  }
}

// acc[c] = z_tile (LDS, [16, HH]) . W0 for columns 32w + 16c + n.
template <int HH>
__device__ __forceinline__ void gemm_b(floatx4 (&acc)[2], const float* zs,
                                       const float (&bB)[2][OutDims<HH>::KB], int q, int n) {
  using D = OutDims<HH>;
  acc[0] = acc[1] = floatx4{0.f, 0.f, 0.f, 0.f};
  const float* za = zs + n * D::ZR + 4 * q;
#pragma unroll
  for (int m = 0; m < HH / 16; ++m) {
    const float4 v = ld4(za + 16 * m);
    const float av[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j], bB[0][4 * m + j], acc[0], 0, 0, 0);
      acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j], bB[1][4 * m + j], acc[1], 0, 0, 0);
    }
  }
}

// Sum over the 16 lanes of a lane group (same q), returned to every lane.
__device__ __forceinline__ float group16_sum(float v) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v += __shfl_xor(v, o, MLCG_WAVE);
  return v;
}

// Per-row sum over the hidden units of `part` (rows 4q+i of this wave's
// tiles): partials per wave into opart, then a fixed-order sum of the 4
// waves by threads 0..15.  Contains one barrier.
__device__ __forceinline__ float rows_total(const float (&part)[4], float (*opart)[kRowsT], int w,
                                            int q, int n) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float v = group16_sum(part[i]);
    if (n == 0) opart[w][4 * q + i] = v;
  }
  __syncthreads();
  const int t = threadIdx.x & (kRowsT - 1);
  return (opart[0][t] + opart[1][t]) + (opart[2][t] + opart[3][t]);
}

__device__ __forceinline__ void act_d1d2(int act, float z, float s, float& d1, float& d2) {
  if (act == MLCG_ACT_TANH) {
    d1 = 1.0f - s * s;
    d2 = -2.0f * s * d1;
  } else {
    const float sg = mlcg_sigmoid(z);
    d1 = sg;
    d2 = sg * (1.0f - sg);
  }
}

template <int HH, bool kRev>
__global__ __launch_bounds__(kThreads) void out_fwd_kernel(
    const float* __restrict__ x, int64_t rows, const float* __restrict__ W0,
    const float* __restrict__ b0, const float* __restrict__ w1, const float* __restrict__ b1,
    int act, const float* __restrict__ seed, float* __restrict__ o, float* __restrict__ oz,
    float* __restrict__ os, float* __restrict__ xbar) {
  using D = OutDims<HH>;
  __shared__ float xs[kRowsT * kXR];
  __shared__ float zs[kRowsT * D::ZR];
  __shared__ float opart[4][kRowsT];
  const int w = threadIdx.x / MLCG_WAVE;
  const int l = mlcg_lane();
  const int q = l >> 4, n = l & 15;
  float bA[D::TA][32];
  load_bA<HH>(bA, W0, w, q, n);
  float bB[2][D::KB];
  if (kRev) load_bB<HH>(bB, W0, w, q, n);
  float w1v[D::TA], b0v[D::TA];
#pragma unroll
  for (int a = 0; a < D::TA; ++a) {
    const int u = w + 4 * a;
    w1v[a] = u < D::NT ? w1[16 * u + n] : 0.f;
    b0v[a] = (u < D::NT && b0) ? b0[16 * u + n] : 0.f;
  }
  const float bias1 = b1 ? *b1 : 0.f;
  const int64_t tiles = (rows + kRowsT - 1) / kRowsT;
  for (int64_t t = blockIdx.x; t < tiles; t += gridDim.x) {
    const int64_t r0 = t * kRowsT;
    stage_rows(xs, x, r0, rows);
    __syncthreads();
    floatx4 acc[D::TA];
    gemm_a<HH>(acc, xs, bA, w, q, n);
    float part[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int a = 0; a < D::TA; ++a) {
      const int u = w + 4 * a;
      if (u >= D::NT) continue;
      const int h = 16 * u + n;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t r = r0 + 4 * q + i;
        const float zv = acc[a][i] + b0v[a];
        float s, d1, d2;
        mlcg_act(act, zv, s, d1, d2);
        if (r < rows) {
          if (oz) oz[r * HH + h] = zv;
          if (os) os[r * HH + h] = s;
        }
        part[i] += s * w1v[a];
        if (kRev) {
          const float sd = r < rows ? (seed ? seed[r] : 1.0f) : 0.0f;
          zs[(4 * q + i) * D::ZR + h] = sd * w1v[a] * d1;
        }
      }
    }
    const float ot = rows_total(part, opart, w, q, n);  // barrier inside
    if (o && threadIdx.x < kRowsT && r0 + threadIdx.x < rows) o[r0 + threadIdx.x] = ot + bias1;
    if (kRev) {
      floatx4 yb[2];
      gemm_b<HH>(yb, zs, bB, q, n);
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t r = r0 + 4 * q + i;
          if (r < rows) xbar[r * kH + 32 * w + 16 * c + n] = yb[c][i];
        }
    }
    __syncthreads();
  }
}

template <int HH, bool kTan>
__global__ __launch_bounds__(kThreads) void out_rev2_kernel(
    const float* __restrict__ x, const float* __restrict__ xdot, int64_t rows,
    const float* __restrict__ W0, const float* __restrict__ w1, const float* __restrict__ oz,
    const float* __restrict__ os, int act, const float* __restrict__ tw,
    const float* __restrict__ pw, float* __restrict__ odot, float* __restrict__ xbar2,
    float* __restrict__ partial) {
  using D = OutDims<HH>;
  __shared__ float xs[kRowsT * kXR];
  __shared__ float xds[kTan ? kRowsT * kXR : 4];
  __shared__ float zd[kTan ? kRowsT * D::ZR : 4];
  __shared__ float z2[kRowsT * D::ZR];
  __shared__ float opart[4][kRowsT];
  const int w = threadIdx.x / MLCG_WAVE;
  const int l = mlcg_lane();
  const int q = l >> 4, n = l & 15;
  float bA[D::TA][32];
  if (kTan) load_bA<HH>(bA, W0, w, q, n);
  float bB[2][D::KB];
  load_bB<HH>(bB, W0, w, q, n);
  float w1v[D::TA];
#pragma unroll
  for (int a = 0; a < D::TA; ++a) {
    const int u = w + 4 * a;
    w1v[a] = u < D::NT ? w1[16 * u + n] : 0.f;
  }
  // gW0 tiles: hidden tile u (all), columns 16(2w + cc) + n
  floatx4 g[D::NT][2];
#pragma unroll
  for (int u = 0; u < D::NT; ++u) g[u][0] = g[u][1] = floatx4{0.f, 0.f, 0.f, 0.f};
  float gb0[D::TA], gw1[D::TA];
#pragma unroll
  for (int a = 0; a < D::TA; ++a) gb0[a] = gw1[a] = 0.f;
  float gb1 = 0.f;
  const int64_t tiles = (rows + kRowsT - 1) / kRowsT;
  for (int64_t t = blockIdx.x; t < tiles; t += gridDim.x) {
    const int64_t r0 = t * kRowsT;
    stage_rows(xs, x, r0, rows);
    if (kTan) stage_rows(xds, xdot, r0, rows);
    if (pw && threadIdx.x < kRowsT && r0 + threadIdx.x < rows) gb1 += pw[r0 + threadIdx.x];
    __syncthreads();
    floatx4 zdot[D::TA];
    if (kTan) gemm_a<HH>(zdot, xds, bA, w, q, n);
    float part[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int a = 0; a < D::TA; ++a) {
      const int u = w + 4 * a;
      if (u >= D::NT) continue;
      const int h = 16 * u + n;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t r = r0 + 4 * q + i;
        const bool ok = r < rows;
        const float s = ok ? os[r * HH + h] : 0.f;
        const float zv = (ok && act != MLCG_ACT_TANH) ? oz[r * HH + h] : s;
        float d1, d2;
        act_d1d2(act, zv, s, d1, d2);
        const float twr = (tw && ok) ? tw[r] : 0.f;
        const float pwr = (pw && ok) ? pw[r] : 0.f;
        const float zt = kTan ? zdot[a][i] : 0.f;
        const float hdot = d1 * zt;
        part[i] += hdot * w1v[a];
        gw1[a] += twr * hdot + pwr * s;
        const float hdotbar = twr * w1v[a];
        const float zb2 = pwr * w1v[a] * d1 + hdotbar * d2 * zt;
        gb0[a] += zb2;
        if (kTan) zd[(4 * q + i) * D::ZR + h] = hdotbar * d1;
        z2[(4 * q + i) * D::ZR + h] = zb2;
      }
    }
    const float ot = rows_total(part, opart, w, q, n);  // barrier inside
    if (odot && threadIdx.x < kRowsT && r0 + threadIdx.x < rows) odot[r0 + threadIdx.x] = ot;
    // gW0 += zbar2^T x (+ zdotbar^T xdot): the 16 rows are the reduction axis
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int rr = 4 * kk + q;
      float bx[2], bxd[2];
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        bx[cc] = xs[rr * kXR + 16 * (2 * w + cc) + n];
        bxd[cc] = kTan ? xds[rr * kXR + 16 * (2 * w + cc) + n] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < D::NT; ++u) {
        const float a2 = z2[rr * D::ZR + 16 * u + n];
        const float ad = kTan ? zd[rr * D::ZR + 16 * u + n] : 0.f;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
          g[u][cc] = __builtin_amdgcn_mfma_f32_16x16x4f32(a2, bx[cc], g[u][cc], 0, 0, 0);
          if (kTan) g[u][cc] = __builtin_amdgcn_mfma_f32_16x16x4f32(ad, bxd[cc], g[u][cc], 0, 0, 0);
        }
      }
    }
    floatx4 yb[2];
    gemm_b<HH>(yb, z2, bB, q, n);
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t r = r0 + 4 * q + i;
        if (r < rows) xbar2[r * kH + 32 * w + 16 * c + n] = yb[c][i];
      }
    __syncthreads();
  }
  // this workgroup's partial sums
  float* part_out = partial + (int64_t)blockIdx.x * D::PART;
#pragma unroll
  for (int u = 0; u < D::NT; ++u)
#pragma unroll
    for (int cc = 0; cc < 2; ++cc)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        part_out[(16 * u + 4 * q + i) * kH + 16 * (2 * w + cc) + n] = g[u][cc][i];
#pragma unroll
  for (int a = 0; a < D::TA; ++a) {
    const int u = w + 4 * a;
    float vb = gb0[a], vw = gw1[a];
    vb += __shfl_xor(vb, 16, MLCG_WAVE);
    vb += __shfl_xor(vb, 32, MLCG_WAVE);
    vw += __shfl_xor(vw, 16, MLCG_WAVE);
    vw += __shfl_xor(vw, 32, MLCG_WAVE);
    if (u < D::NT && q == 0) {
      part_out[HH * kH + 16 * u + n] = vb;
      part_out[HH * kH + HH + 16 * u + n] = vw;
    }
  }
  if (w == 0) {
    const float v = group16_sum(gb1);
    if (l == 0) part_out[HH * kH + 2 * HH] = v;
  }
}

// out[j] = sum over groups of partial[g][j] (fixed order: 8 interleaved
// slices, combined pairwise), split into gW0 / gb0 / gW1 / gb1.
template <int HH>
__global__ __launch_bounds__(512) void out_rev2_reduce_kernel(const float* __restrict__ partial,
                                                             int groups, float* __restrict__ gW0,
                                                             float* __restrict__ gb0,
                                                             float* __restrict__ gW1,
                                                             float* __restrict__ gb1) {
  using D = OutDims<HH>;
  __shared__ float part[8][64];
  const int o = threadIdx.x & 63, s0 = threadIdx.x >> 6;
  const int j = blockIdx.x * 64 + o;
  const int total = HH * kH + 2 * HH + 1;
  float a0 = 0.f, a1 = 0.f;
  if (j < total) {
    int s = s0;
    for (; s + 8 < groups; s += 16) {
      a0 += partial[(int64_t)s * D::PART + j];
      a1 += partial[(int64_t)(s + 8) * D::PART + j];
    }
    if (s < groups) a0 += partial[(int64_t)s * D::PART + j];
  }
  part[s0][o] = a0 + a1;
  __syncthreads();
  if (s0 == 0 && j < total) {
    const float v = ((part[0][o] + part[1][o]) + (part[2][o] + part[3][o])) +
                    ((part[4][o] + part[5][o]) + (part[6][o] + part[7][o]));
    if (j < HH * kH) {
      gW0[j] = v;
    } else if (j < HH * kH + HH) {
      if (gb0) gb0[j - HH * kH] = v;
    } else if (j < HH * kH + 2 * HH) {
      gW1[j - HH * kH - HH] = v;
    } else if (gb1) {
      gb1[0] = v;
    }
  }
}

constexpr int kRev2MaxGroups = 512;  // two per CU: about two 16-row tiles each

int rev2_groups(int64_t rows) {
  const int64_t tiles = rows == 0 ? 1 : (rows + kRowsT - 1) / kRowsT;
  return (int)(tiles < kRev2MaxGroups ? tiles : kRev2MaxGroups);
}

int part_floats(int hidden) { return hidden * kH + 2 * hidden + 4; }

template <int HH>
void launch_fwd(bool rev, dim3 grid, hipStream_t s, const float* x, int64_t rows,
                const float* W0, const float* b0, const float* w1, const float* b1, int act,
                const float* seed, float* o, float* oz, float* os, float* xbar) {
  if (rev)
    hipLaunchKernelGGL((out_fwd_kernel<HH, true>), grid, dim3(kThreads), 0, s, x, rows, W0, b0,
                       w1, b1, act, seed, o, oz, os, xbar);
  else
    hipLaunchKernelGGL((out_fwd_kernel<HH, false>), grid, dim3(kThreads), 0, s, x, rows, W0, b0,
                       w1, b1, act, seed, o, oz, os, xbar);
}

template <int HH>
void launch_rev2(bool tan, dim3 grid, hipStream_t s, const float* x, const float* xdot,
                 int64_t rows, const float* W0, const float* w1, const float* oz,
                 const float* os, int act, const float* tw, const float* pw, float* odot,
                 float* xbar2, float* gW0, float* gb0, float* gW1, float* gb1, float* ws) {
  if (tan)
    hipLaunchKernelGGL((out_rev2_kernel<HH, true>), grid, dim3(kThreads), 0, s, x, xdot, rows,
                       W0, w1, oz, os, act, tw, pw, odot, xbar2, ws);
  else
    hipLaunchKernelGGL((out_rev2_kernel<HH, false>), grid, dim3(kThreads), 0, s, x, xdot, rows,
                       W0, w1, oz, os, act, tw, pw, odot, xbar2, ws);
  const int total = HH * kH + 2 * HH + 1;
  hipLaunchKernelGGL((out_rev2_reduce_kernel<HH>), dim3(mlcg_div_up(total, 64)), dim3(512), 0, s,
                     ws, (int)grid.x, gW0, gb0, gW1, gb1);
}

bool hidden_ok(int hidden) { return hidden == 32 || hidden == 64 || hidden == 128; }

}  // namespace

extern "C" int mlcg_out_forward(const float* x, int64_t rows, int in_features, int hidden,
                                const float* W0, const float* b0, const float* w1,
                                const float* b1, int act, int reverse, const float* seed,
                                float* o, float* oz, float* os, float* xbar, void* stream) {
  if (in_features != kH || !hidden_ok(hidden)) return MLCG_ERR_UNSUPPORTED;
  MLCG_REQUIRE(rows >= 0 && (act == MLCG_ACT_TANH || act == MLCG_ACT_SSP));
  MLCG_REQUIRE(!reverse || xbar);
  if (rows == 0) return MLCG_OK;
  MLCG_REQUIRE(x && W0 && w1);
  const int64_t tiles = (rows + kRowsT - 1) / kRowsT;
  const dim3 grid(mlcg_persistent_groups(tiles, 4));
  hipStream_t s = mlcg_stream(stream);
  const bool rev = reverse != 0;
  if (hidden == 32)
    launch_fwd<32>(rev, grid, s, x, rows, W0, b0, w1, b1, act, seed, o, oz, os, xbar);
  else if (hidden == 64)
    launch_fwd<64>(rev, grid, s, x, rows, W0, b0, w1, b1, act, seed, o, oz, os, xbar);
  else
    launch_fwd<128>(rev, grid, s, x, rows, W0, b0, w1, b1, act, seed, o, oz, os, xbar);
  return mlcg_launch_status();
}

extern "C" int64_t mlcg_out_rev2_workspace_floats(int64_t rows, int hidden) {
  if (rows < 0 || !hidden_ok(hidden)) return -1;
  return (int64_t)rev2_groups(rows) * part_floats(hidden);
}

extern "C" int mlcg_out_rev2(const float* x, const float* xdot, int64_t rows, int in_features,
                             int hidden, const float* W0, const float* w1, const float* oz,
                             const float* os, int act, const float* tw, const float* pw,
                             float* odot, float* xbar2, float* gW0, float* gb0, float* gW1,
                             float* gb1, float* workspace, int64_t workspace_floats,
                             void* stream) {
  if (in_features != kH || !hidden_ok(hidden)) return MLCG_ERR_UNSUPPORTED;
  MLCG_REQUIRE(rows >= 0 && (act == MLCG_ACT_TANH || act == MLCG_ACT_SSP));
  MLCG_REQUIRE(xbar2 && gW0 && gW1 && workspace);
  MLCG_REQUIRE(!odot || xdot);
  const int groups = rev2_groups(rows);
  MLCG_REQUIRE(workspace_floats >= (int64_t)groups * part_floats(hidden));
  if (rows > 0) MLCG_REQUIRE(x && W0 && w1 && os && (oz || act == MLCG_ACT_TANH));
  hipStream_t s = mlcg_stream(stream);
  const bool tan = xdot != nullptr;
  const dim3 grid((unsigned)groups);
  if (hidden == 32)
    launch_rev2<32>(tan, grid, s, x, xdot, rows, W0, w1, oz, os, act, tw, pw, odot, xbar2, gW0,
                    gb0, gW1, gb1, workspace);
  else if (hidden == 64)
    launch_rev2<64>(tan, grid, s, x, xdot, rows, W0, w1, oz, os, act, tw, pw, odot, xbar2, gW0,
                    gb0, gW1, gb1, workspace);
  else
    launch_rev2<128>(tan, grid, s, x, xdot, rows, W0, w1, oz, os, act, tw, pw, odot, xbar2,
                     gW0, gb0, gW1, gb1, workspace);
  return mlcg_launch_status();
}
