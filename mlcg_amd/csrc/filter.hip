// Fused Gaussian-RBF -> cutoff -> filter MLP -> cutoff chain (gfx950, MFMA).
//
// Reference: GaussianBasis.forward (mlcg/nn/radial_basis/gaussian.py:83-102),
// CosineCutoff.forward (mlcg/nn/cutoff.py:110-153), MLP([K, F, F],
// last_bias=False) (mlcg/nn/mlp.py:31-58) and CFConv.forward lines 340-341
// (mlcg/nn/schnet.py).  The filter depends only on the pair distance, so it
// is evaluated once per unordered pair (W_ij == W_ji bitwise in the
// reference too, since d_ij == d_ji).
//
// Layout of the work.  One wave owns a tile of 16 pairs and computes the
// transposed products a^T = W1 g^T ([F x 16]) and w^T = W2 h^T with
// v_mfma_f32_16x16x4_f32 (fp32 path) or v_mfma_f32_16x16x32_f16 (fp16 path).
// With pairs on the N axis every lane ends up owning one pair (lane % 16) and
// a strip of features, so
//   * the RBF values g are computed directly in the B-operand layout (no LDS),
//   * the MFMA output of the first product is already the B operand of the
//     second one (the contraction order over features is permuted to match,
//     and the matching permutation is baked into the LDS copy of W2),
//   * the epilogue (x cutoff, d/dd) is per-lane scalar work, and
//   * W rows are written as float4/half4 strips.
// W1 and W2 are staged once per workgroup in LDS in the exact per-lane order
// the MFMA A operand needs (conflict-free ds_read_b32/b128), and workgroups
// loop persistently over pair tiles.  The forward also produces the distance
// derivative Wd = dW/dd by pushing the tangent g' = dg/dd through the same
// chain (a second accumulator set sharing every A fragment).
#include "common.h"
#include "split16.h"

#include <hip/hip_fp16.h>

#include <mutex>

namespace {

// Filter rows are written with non-temporal stores: W and W' (222 MB per
// block at config 2) are read again only by the gathers, after other work,
// and written through the caches they leave dirty lines that the next
// gather's reads must first evict.  Measured on config 2: the forward filter
// 93 -> 98 us, the gather after it 45 -> 39 us and the force gather 72 ->
// 67 us; the config-4 fp16 call 5.71 -> 5.61 ms.
__device__ __forceinline__ void nt_store4(float* p, float4 v) {
  __builtin_nontemporal_store(floatx4{v.x, v.y, v.z, v.w}, reinterpret_cast<floatx4*>(p));
}

#ifndef MLCG_FILTER_FWD_X3
#define MLCG_FILTER_FWD_X3 1  // fp32-accurate forward on the fp16 MFMA (see filter_fwd_x3)
#endif
constexpr int kF = 128;          // number of filters (fixed by the MFMA tiling)
constexpr int kFT = kF / 16;     // feature tiles of 16
constexpr int kWaves = 8;        // waves per workgroup
constexpr int kThreads = kWaves * MLCG_WAVE;
constexpr int kMaxK = 128;

// Radial basis (per basis function k, distance d, envelope C(d)):
//   basis 0, Gaussian (gaussian.py:83-102): g_k = C exp(c (d - centers[k])^2),
//            c = widths[0] (the module's 0-dim `coeff`)
//   basis 1, ExpNormal (exp_normal.py:116-130):
//            g_k = C exp(-widths[k] (exp(alpha (lo - d)) - centers[k])^2)
//            with widths = betas, centers = means, lo = the basis' lower cutoff.
// A cutoff envelope in branch-free form (the kernels evaluate it without a
// data- or kind-dependent branch, so that it schedules freely among the MFMA
// chains): u = (d - lo) s + o, C = 0.5 (cos(pi u) + 1) m, dC/dd = -sin(pi u) k m
// with m = [d < hi] and, when gate, [d > lo]:
//   cosine, lo = 0   s = 1 / hi,        o = 0, k = pi s / 2, gate off
//   cosine, lo > 0   s = 2 / (hi - lo), o = 1, k = pi s / 2, gate on
//   identity         s = o = k = 0, hi = +inf (C = 1, dC = 0)
// The same operations, in the same order, as mlcg_cutoff of common.h.
struct Cut {
  float lo, hi, s, o, k;
  int gate;
};

__host__ Cut make_cut(int kind, float lo, float hi) {
  Cut c{0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0};
  const float pi = 3.14159265358979323846f;
  if (kind == MLCG_CUT_IDENTITY) {
    c.hi = __builtin_huge_valf();
  } else if (lo > 0.0f) {
    const float iw = 1.0f / (hi - lo);
    c.lo = lo;
    c.hi = hi;
    c.s = 2.0f * iw;
    c.o = 1.0f;
    c.k = pi * iw;
    c.gate = 1;
  } else {
    const float ih = 1.0f / hi;
    c.hi = hi;
    c.s = ih;
    c.k = 0.5f * (pi * ih);
  }
  return c;
}

__device__ __forceinline__ void cut_eval(const Cut& c, float d, float& cv, float& dcv) {
  float sn, cs;
  mlcg_sincospi((d - c.lo) * c.s + c.o, sn, cs);
  const float m = (d < c.hi && (!c.gate || d > c.lo)) ? 1.0f : 0.0f;
  cv = 0.5f * (cs + 1.0f) * m;
  dcv = -sn * c.k * m;
}

struct RbfParams {
  const float* centers;
  const float* widths;
  float alpha;
  int basis;
  int K;
  int rbf_kind;
  float rbf_lo, rbf_hi;
  int conv_kind;
  float conv_lo, conv_hi;
  int act;
  int same_cut;  // the CFConv envelope is the RBF envelope: evaluated once
  Cut rcut, ccut;  // the two envelopes in branch-free form
};

// Activation value and first derivative for a compile-time activation id.
template <int ACT>
__device__ __forceinline__ void act_t(float x, float& s, float& d1, float& d2) {
  if constexpr (ACT == MLCG_ACT_TANH) {
    s = mlcg_tanh(x);
    d1 = 1.0f - s * s;
    d2 = -2.0f * s * d1;
  } else {
    s = mlcg_softplus(x) - 0.69314718055994530942f;
    const float sg = mlcg_sigmoid(x);
    d1 = sg;
    d2 = sg * (1.0f - sg);
  }
}

// CFConv envelope of a pair whose RBF envelope (crbf, dcrbf) is known.
__device__ __forceinline__ void conv_cutoff(const RbfParams& rp, float d, float crbf, float dcrbf,
                                            float& cc, float& dcc) {
  if (rp.same_cut) {
    cc = crbf;
    dcc = dcrbf;
  } else {
    mlcg_cutoff(rp.conv_kind, rp.conv_lo, rp.conv_hi, d, cc, dcc);
  }
}

// Pair geometry for the lane's pair; out-of-range tiles use a harmless d.
__device__ __forceinline__ float pair_distance(const float* __restrict__ pos,
                                               const int32_t* __restrict__ pi,
                                               const int32_t* __restrict__ pj, int64_t p,
                                               bool valid) {
  if (!valid) return 1.0f;
  const int64_t i = pi[p], j = pj[p];
  float dx = pos[3 * j + 0] - pos[3 * i + 0];
  float dy = pos[3 * j + 1] - pos[3 * i + 1];
  float dz = pos[3 * j + 2] - pos[3 * i + 2];
  return sqrtf(dx * dx + dy * dy + dz * dz);
}

// g_k and dg_k/dd for one basis function (zero past K).
// g_k and g_k' of one basis function from its centre `cen` and width `wid`
// (the Gaussian's shared coeff, or the exp-normal beta_k); zero when !on.
__device__ __forceinline__ void rbf_eval(const RbfParams& rp, bool on, float cen, float wid,
                                         float d, float crbf, float dcrbf, float& g,
                                         float& gd) {
  if (!on) {
    g = 0.0f;
    gd = 0.0f;
  } else if (rp.basis == 0) {
    const float diff = d - cen;
    const float e = __expf(wid * (diff * diff));  // argument <= 0: no overflow
    g = e * crbf;
    gd = e * (2.0f * wid * diff * crbf + dcrbf);
  } else {
    const float ex = __expf(rp.alpha * (rp.rbf_lo - d));
    const float u = ex - cen;
    const float e = __expf(-wid * (u * u));
    g = e * crbf;
    gd = e * (dcrbf + 2.0f * rp.alpha * wid * u * ex * crbf);
  }
}

// rbf_eval for a compile-time basis kind (no branch on rp.basis).
template <int BASIS>
__device__ __forceinline__ void rbf_eval_t(const RbfParams& rp, bool on, float cen, float wid,
                                           float d, float crbf, float dcrbf, float& g,
                                           float& gd) {
  if constexpr (BASIS == 0) {
    const float diff = d - cen;
    const float e = __expf(wid * (diff * diff));
    g = on ? e * crbf : 0.0f;
    gd = on ? e * (2.0f * wid * diff * crbf + dcrbf) : 0.0f;
  } else {
    const float ex = __expf(rp.alpha * (rp.rbf_lo - d));
    const float u = ex - cen;
    const float e = __expf(-wid * (u * u));
    g = on ? e * crbf : 0.0f;
    gd = on ? e * (dcrbf + 2.0f * rp.alpha * wid * u * ex * crbf) : 0.0f;
  }
}

// Basis, activation and envelopes for a compile-time kind, or (kind -1)
// dispatched at run time on rp.
template <int BASIS>
__device__ __forceinline__ void rbf_any(const RbfParams& rp, bool on, float cen, float wid,
                                        float d, float crbf, float dcrbf, float& g, float& gd) {
  if constexpr (BASIS < 0) {
    rbf_eval(rp, on, cen, wid, d, crbf, dcrbf, g, gd);
  } else {
    rbf_eval_t<BASIS>(rp, on, cen, wid, d, crbf, dcrbf, g, gd);
  }
}
template <int ACT>
__device__ __forceinline__ void act_any(int act, float x, float& s, float& d1, float& d2) {
  if constexpr (ACT < 0) {
    mlcg_act(act, x, s, d1, d2);
  } else {
    act_t<ACT>(x, s, d1, d2);
  }
}
// Both envelopes of a pair from their branch-free forms.
__device__ __forceinline__ void envelopes(const RbfParams& rp, float d, float& crbf,
                                          float& dcrbf, float& cc, float& dcc) {
  cut_eval(rp.rcut, d, crbf, dcrbf);
  if (rp.same_cut) {  // uniform
    cc = crbf;
    dcc = dcrbf;
  } else {
    cut_eval(rp.ccut, d, cc, dcc);
  }
}

// Centre and width of basis function k read from global memory (zero past K).
__device__ __forceinline__ void basis_params(const RbfParams& rp, int k, float& cen,
                                             float& wid) {
  const bool on = k < rp.K;
  cen = on ? rp.centers[k] : 0.0f;
  wid = on ? (rp.basis == 0 ? rp.widths[0] : rp.widths[k]) : 0.0f;
}

// The basis parameters staged in LDS once per workgroup, so that the
// per-tile basis evaluation reads them with LDS latency instead of a global
// load: bc[k], bw[k] for k < kMaxK (zero past K).
__device__ void stage_basis(float* bc, float* bw, const RbfParams& rp) {
  for (int k = threadIdx.x; k < kMaxK; k += blockDim.x) basis_params(rp, k, bc[k], bw[k]);
}

// ---------------------------------------------------------------------------
// LDS staging.
//
// fp32, first product (A = W1, 16x16x4):   w1s[(t*KS + s)*64 + l] =
//     W1[16t + l%16][4s + l/16]
// fp32, second product (A = W2, k order kappa(s, q) = 16(s/4) + 4q + s%4):
//     w2s[((t*8 + u)*64 + l)*4 + i] = W2[16t + l%16][16u + 4(l/16) + i]
// fp32, reverse product (A = W2^T):
//     w2ts[((t*8 + u)*64 + l)*4 + i] = W2[16u + 4(l/16) + i][16t + l%16]
__device__ void stage_w1_f32(float* w1s, const float* __restrict__ W1, int K, int KS) {
  const int total = kFT * KS * MLCG_WAVE;
  for (int x = threadIdx.x; x < total; x += blockDim.x) {
    const int l = x & 63;
    const int ts = x >> 6;
    const int s = ts % KS, t = ts / KS;
    const int k = 4 * s + (l >> 4);
    w1s[x] = k < K ? W1[(16 * t + (l & 15)) * K + k] : 0.0f;
  }
}

__device__ void stage_w2_f32(float* w2s, const float* __restrict__ W2, bool transpose) {
  const int total = kFT * kFT * MLCG_WAVE;  // float4 slots
  for (int x = threadIdx.x; x < total; x += blockDim.x) {
    const int l = x & 63;
    const int tu = x >> 6;
    const int u = tu % kFT, t = tu / kFT;
    const int r = 16 * t + (l & 15);
    const int c0 = 16 * u + 4 * (l >> 4);
    float4 v;
    if (!transpose) {
      v = *reinterpret_cast<const float4*>(W2 + r * kF + c0);
    } else {
      v.x = W2[(c0 + 0) * kF + r];
      v.y = W2[(c0 + 1) * kF + r];
      v.z = W2[(c0 + 2) * kF + r];
      v.w = W2[(c0 + 3) * kF + r];
    }
    reinterpret_cast<float4*>(w2s)[x] = v;
  }
}

// First product for one 16-pair tile: acc_a = W1 g^T, acc_d = W1 g'^T (fp32).
// Also returns the lane's g/g' values when `gout` is non-null (reverse pass).
__device__ __forceinline__ void gemm1_f32(const float* w1s, int KS, const RbfParams& rp,
                                          const float* bc, const float* bw, float d,
                                          float crbf, float dcrbf, floatx4* acc_a,
                                          floatx4* acc_d, float* gout, float* gdout,
                                          float gscale) {
  const int l = mlcg_lane();
  const int q = l >> 4;
#pragma unroll
  for (int t = 0; t < kFT; ++t) {
    acc_a[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    acc_d[t] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  for (int s = 0; s < KS; ++s) {
    float g, gd;
    const int k = 4 * s + q;
    rbf_eval(rp, k < rp.K, bc[k], bw[k], d, crbf, dcrbf, g, gd);
    if (gout) {
      gout[4 * s + q] = g * gscale;
      gdout[4 * s + q] = gd * gscale;
    }
#pragma unroll
    for (int t = 0; t < kFT; ++t) {
      const float w = w1s[(t * KS + s) * MLCG_WAVE + l];
      acc_a[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(w, g, acc_a[t], 0, 0, 0);
      acc_d[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(w, gd, acc_d[t], 0, 0, 0);
    }
  }
}

// Second product: out_x = A2 bx^T, out_y = A2 by^T, with A2 staged by
// stage_w2_f32 and bx/by holding [tile u][i] values of the lane's pair.
__device__ __forceinline__ void gemm2_f32(const float* w2s, const floatx4* bx,
                                          const floatx4* by, floatx4* out_x,
                                          floatx4* out_y) {
  const int l = mlcg_lane();
#pragma unroll
  for (int t = 0; t < kFT; ++t) {
    out_x[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    out_y[t] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  for (int u = 0; u < kFT; ++u) {
#pragma unroll
    for (int t = 0; t < kFT; ++t) {
      const float4 a = reinterpret_cast<const float4*>(w2s)[(t * kFT + u) * MLCG_WAVE + l];
      out_x[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, bx[u][0], out_x[t], 0, 0, 0);
      out_y[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, by[u][0], out_y[t], 0, 0, 0);
      out_x[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, bx[u][1], out_x[t], 0, 0, 0);
      out_y[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, by[u][1], out_y[t], 0, 0, 0);
      out_x[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, bx[u][2], out_x[t], 0, 0, 0);
      out_y[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, by[u][2], out_y[t], 0, 0, 0);
      out_x[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, bx[u][3], out_x[t], 0, 0, 0);
      out_y[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, by[u][3], out_y[t], 0, 0, 0);
    }
  }
}

__global__ __launch_bounds__(kThreads) void filter_fwd_f32_kernel(
    const float* __restrict__ pos, const int32_t* __restrict__ pi,
    const int32_t* __restrict__ pj, const int32_t* __restrict__ n_pairs_dev,
    int64_t max_pairs, RbfParams rp, const float* __restrict__ W1,
    const float* __restrict__ b1, const float* __restrict__ W2, float* __restrict__ Wout,
    float* __restrict__ Wdout, float* __restrict__ dist_out) {
  extern __shared__ float lds[];
  const int KS = (rp.K + 3) / 4;
  float* w1s = lds;
  float* w2s = lds + kFT * KS * MLCG_WAVE;
  float* bc = w2s + kFT * kFT * MLCG_WAVE * 4;
  float* bw = bc + kMaxK;
  stage_w1_f32(w1s, W1, rp.K, KS);
  stage_w2_f32(w2s, W2, false);
  stage_basis(bc, bw, rp);
  __syncthreads();

  int64_t np = *n_pairs_dev;
  if (np > max_pairs) np = max_pairs;
  const int64_t tiles = (np + 15) / 16;
  const int l = mlcg_lane();
  const int q = l >> 4;
  float bias[kFT][4];
#pragma unroll
  for (int t = 0; t < kFT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) bias[t][i] = b1[16 * t + 4 * q + i];

  const int64_t wave = (int64_t)blockIdx.x * kWaves + threadIdx.x / MLCG_WAVE;
  const int64_t nwaves = (int64_t)gridDim.x * kWaves;
  for (int64_t tile = wave; tile < tiles; tile += nwaves) {
    const int64_t p = tile * 16 + (l & 15);
    const bool valid = p < np;
    const float d = pair_distance(pos, pi, pj, p, valid);
    float crbf, dcrbf, cc, dcc;
    mlcg_cutoff(rp.rbf_kind, rp.rbf_lo, rp.rbf_hi, d, crbf, dcrbf);
    conv_cutoff(rp, d, crbf, dcrbf, cc, dcc);

    floatx4 a[kFT], ad[kFT];
    gemm1_f32(w1s, KS, rp, bc, bw, d, crbf, dcrbf, a, ad, nullptr, nullptr, 0.0f);
    // h = act(a + b1), h' = act'(a + b1) * a'
#pragma unroll
    for (int t = 0; t < kFT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float s, d1, d2;
        mlcg_act(rp.act, a[t][i] + bias[t][i], s, d1, d2);
        a[t][i] = s;
        ad[t][i] = d1 * ad[t][i];
      }
    floatx4 w[kFT], wd[kFT];
    gemm2_f32(w2s, a, ad, w, wd);
    if (valid) {
      float* wr = Wout + p * kF + 4 * q;
      float* wdr = Wdout + p * kF + 4 * q;
#pragma unroll
      for (int t = 0; t < kFT; ++t) {
        float4 o, od;
        o.x = w[t][0] * cc;
        o.y = w[t][1] * cc;
        o.z = w[t][2] * cc;
        o.w = w[t][3] * cc;
        od.x = wd[t][0] * cc + w[t][0] * dcc;
        od.y = wd[t][1] * cc + w[t][1] * dcc;
        od.z = wd[t][2] * cc + w[t][2] * dcc;
        od.w = wd[t][3] * cc + w[t][3] * dcc;
        nt_store4(wr + 16 * t, o);
        nt_store4(wdr + 16 * t, od);
      }
      if (dist_out && q == 0) dist_out[p] = d;
    }
  }
}

// ---------------------------------------------------------------------------
// fp16 operands, fp32 accumulation (v_mfma_f32_16x16x32_f16).
//
// First product, k block s (32 basis functions): lane l supplies
//   A[m = l%16][8q + j] = W1[16t + l%16][32s + 8q + j]      (j = 0..7)
//   B[8q + j][n = l%16] = g[pair l%16][32s + 8q + j]
// Second product, k block s covers feature tiles 2s and 2s+1; lane group q
// supplies features 16(2s + j/4) + 4q + j%4 -- exactly the accumulator
// values it owns after the first product.
//   w1h[((t*KS32 + s)*64 + l)*8 + j] = W1[16t + l%16][32s + 8q + j]
//   w2h[((t*4 + s)*64 + l)*8 + j]    = W2[f(t, l%16)][16(2s + j/4) + 4q + j%4]
// with the output-row permutation f(t, m) = 32(t/2) + 8(m/4) + 4(t%2) + m%4.
__device__ void stage_f16(_Float16* w1h, _Float16* w2h, const float* __restrict__ W1,
                          const float* __restrict__ W2, int K, int KS32) {
  const int n1 = kFT * KS32 * MLCG_WAVE * 8;
  for (int x = threadIdx.x; x < n1; x += blockDim.x) {
    const int j = x & 7;
    const int l = (x >> 3) & 63;
    const int ts = x >> 9;
    const int s = ts % KS32, t = ts / KS32;
    const int k = 32 * s + 8 * (l >> 4) + j;
    w1h[x] = (_Float16)(k < K ? W1[(16 * t + (l & 15)) * K + k] : 0.0f);
  }
  const int n2 = kFT * (kFT / 2) * MLCG_WAVE * 8;
  for (int x = threadIdx.x; x < n2; x += blockDim.x) {
    const int j = x & 7;
    const int l = (x >> 3) & 63;
    const int ts = x >> 9;
    const int s = ts % (kFT / 2), t = ts / (kFT / 2);
    const int c = 16 * (2 * s + (j >> 2)) + 4 * (l >> 4) + (j & 3);
    // A row m of output tile t is output feature 32 (t / 2) + 8 (m / 4) +
    // 4 (t % 2) + m % 4, so that after tiles 2u and 2u + 1 lane (n, q) holds
    // the eight consecutive features 32 u + 8 q .. + 7 of its pair
    const int m = l & 15;
    const int f = 32 * (t >> 1) + 8 * (m >> 2) + 4 * (t & 1) + (m & 3);
    w2h[x] = (_Float16)W2[f * kF + c];
  }
}

// tanh for the fp16 filter: 1 - 2 / (e^2x + 1) in fp32 (two hardware
// transcendentals; saturates to exactly +-1).  Its absolute error is a few
// 1e-7 -- relative accuracy is lost only where |tanh x| < 1e-3, and the value
// is rounded to fp16 (relative step 2^-11) right after.
__device__ __forceinline__ float tanh_f16path(float x) {
  const float e = __builtin_amdgcn_exp2f(x * 2.8853900817779268f);  // e^2x
  return fmaf(-2.0f, __builtin_amdgcn_rcpf(e + 1.0f), 1.0f);
}

// 8 waves per workgroup and two workgroups per CU: one wave per 16-pair
// tile, feature tile at a time (as filter_fwd_x3_kernel), so only two
// accumulators are live next to the fp16 operands.  The second linear's
// output rows are permuted at staging (stage_f16) so that each lane ends up
// with eight consecutive features of its pair and stores them as 16 bytes.
#ifndef MLCG_F16_WAVES
#define MLCG_F16_WAVES 8
#endif
#ifndef MLCG_F16_GROUPS_PER_CU
#define MLCG_F16_GROUPS_PER_CU 2
#endif
constexpr int kWaves16 = MLCG_F16_WAVES;  // the second launch bound is waves per SIMD
constexpr int kThreads16 = kWaves16 * MLCG_WAVE;

template <int KS32, int BASIS, int ACT>
__global__ __launch_bounds__(kThreads16, kWaves16 * MLCG_F16_GROUPS_PER_CU / 4) void filter_fwd_f16_kernel(
    const float* __restrict__ pos, const int32_t* __restrict__ pi,
    const int32_t* __restrict__ pj, const int32_t* __restrict__ n_pairs_dev,
    int64_t max_pairs, RbfParams rp, const float* __restrict__ W1,
    const float* __restrict__ b1, const float* __restrict__ W2, __half* __restrict__ Wout,
    __half* __restrict__ Wdout, float* __restrict__ dist_out) {
  extern __shared__ float lds[];
  _Float16* w1h = reinterpret_cast<_Float16*>(lds);
  _Float16* w2h = w1h + kFT * KS32 * MLCG_WAVE * 8;
  float* b1s = reinterpret_cast<float*>(w2h + kFT * (kFT / 2) * MLCG_WAVE * 8);
  float* bc = b1s + kF;
  float* bw = bc + kMaxK;
  stage_f16(w1h, w2h, W1, W2, rp.K, KS32);
  for (int x = threadIdx.x; x < kF; x += blockDim.x) b1s[x] = b1[x];
  stage_basis(bc, bw, rp);  // zeros past K: finite basis values that meet zero weights
  __syncthreads();

  int64_t np = *n_pairs_dev;
  if (np > max_pairs) np = max_pairs;
  const int64_t tiles = (np + 15) / 16;
  const int l = mlcg_lane();
  const int q = l >> 4;

  const halfx8* w1v = reinterpret_cast<const halfx8*>(w1h);
  const halfx8* w2v = reinterpret_cast<const halfx8*>(w2h);
  const int64_t wave = (int64_t)blockIdx.x * kWaves16 + threadIdx.x / MLCG_WAVE;
  const int64_t nwaves = (int64_t)gridDim.x * kWaves16;
  auto pair_at = [&](int64_t t_) -> int64_t {
    const int64_t p_ = (t_ < tiles ? t_ : tiles - 1) * 16 + (l & 15);
    return p_ < np ? p_ : np - 1;
  };
  float3 ri{0.f, 0.f, 0.f}, rj{0.f, 0.f, 0.f};
  int64_t ni = 0, nj = 0;
  if (wave < tiles) {
    const int64_t p0 = pair_at(wave), p1 = pair_at(wave + nwaves);
    const int64_t i0 = pi[p0], j0 = pj[p0];
    ri = float3{pos[3 * i0], pos[3 * i0 + 1], pos[3 * i0 + 2]};
    rj = float3{pos[3 * j0], pos[3 * j0 + 1], pos[3 * j0 + 2]};
    ni = pi[p1];
    nj = pj[p1];
  }
  for (int64_t tile = wave; tile < tiles; tile += nwaves) {
    // the weight fragments are re-read from LDS every tile: without this
    // barrier the compiler hoists all 48 of them into registers and spills
    asm volatile("" ::: "memory");
    const int64_t p = tile * 16 + (l & 15);
    const bool valid = p < np;
    float d = 1.0f;
    if (valid) {
      const float dx = rj.x - ri.x, dy = rj.y - ri.y, dz = rj.z - ri.z;
      d = sqrtf(dx * dx + dy * dy + dz * dz);
    }
    ri = float3{pos[3 * ni], pos[3 * ni + 1], pos[3 * ni + 2]};
    rj = float3{pos[3 * nj], pos[3 * nj + 1], pos[3 * nj + 2]};
    {
      const int64_t p2 = pair_at(tile + 2 * nwaves);
      ni = pi[p2];
      nj = pj[p2];
    }
    float crbf, dcrbf, cc, dcc;
    envelopes(rp, d, crbf, dcrbf, cc, dcc);

    halfx8 g8[KS32], gd8[KS32];
#pragma unroll
    for (int s = 0; s < KS32; ++s)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float g, gd;
        const int k = 32 * s + 8 * q + j;
        rbf_eval_t<BASIS>(rp, true, bc[k], bw[k], d, crbf, dcrbf, g, gd);
        g8[s][j] = (_Float16)g;
        gd8[s][j] = (_Float16)gd;
      }
    halfx8 h8[kFT / 2], hd8[kFT / 2];
#pragma unroll
    for (int t = 0; t < kFT; ++t) {
      floatx4 a = {0.f, 0.f, 0.f, 0.f}, ad = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS32; ++s) {
        const halfx8 w = w1v[(t * KS32 + s) * MLCG_WAVE + l];
        a = __builtin_amdgcn_mfma_f32_16x16x32_f16(w, g8[s], a, 0, 0, 0);
        ad = __builtin_amdgcn_mfma_f32_16x16x32_f16(w, gd8[s], ad, 0, 0, 0);
      }
      const float4 bias = *reinterpret_cast<const float4*>(b1s + 16 * t + 4 * q);
      const float bv[4] = {bias.x, bias.y, bias.z, bias.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float sv, d1;
        if constexpr (ACT == MLCG_ACT_TANH) {
          sv = tanh_f16path(a[i] + bv[i]);
          d1 = fmaf(-sv, sv, 1.0f);
        } else {
          float d2;
          act_t<ACT>(a[i] + bv[i], sv, d1, d2);
        }
        h8[t >> 1][4 * (t & 1) + i] = (_Float16)sv;
        hd8[t >> 1][4 * (t & 1) + i] = (_Float16)(d1 * ad[i]);
      }
    }
    __half* wr = Wout + p * kF + 8 * q;
    __half* wdr = Wdout + p * kF + 8 * q;
#pragma unroll
    for (int u = 0; u < kFT / 2; ++u) {
      halfx8 o, od;
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        const int t = 2 * u + v;
        floatx4 w = {0.f, 0.f, 0.f, 0.f}, wd = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < kFT / 2; ++s) {
          const halfx8 a2 = w2v[(t * (kFT / 2) + s) * MLCG_WAVE + l];
          w = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2, h8[s], w, 0, 0, 0);
          wd = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2, hd8[s], wd, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          o[4 * v + i] = (_Float16)(w[i] * cc);
          od[4 * v + i] = (_Float16)(wd[i] * cc + w[i] * dcc);
        }
      }
      if (valid) {
        __builtin_nontemporal_store(o, reinterpret_cast<halfx8*>(wr + 32 * u));
        __builtin_nontemporal_store(od, reinterpret_cast<halfx8*>(wdr + 32 * u));
      }
    }
    if (valid && dist_out && q == 0) dist_out[p] = d;
  }
}

// ---------------------------------------------------------------------------
// fp32-accurate products on the fp16 MFMA (v_mfma_f32_16x16x32_f16).
//
// An fp32 operand x is carried as two fp16 parts, hi = fp16(x) and
// lo = fp16((x - hi) S) with S = 2^e, which together hold about 22
// significant bits.  A product A B (A = a weight matrix, B = per-pair data)
// is accumulated in fp32 as
//     S A B ~ (hi_A S) hi_B + hi_A lo_B + lo_A hi_B       (three MFMAs)
// dropping only lo_A lo_B / S (2^-22 relative), and the accumulator is
// divided by S afterwards.  The weights' three planes (hi, hi S, lo) are
// staged in LDS once per workgroup, with e <= 11 chosen per workgroup and
// per matrix from its largest entry so that hi S stays inside the fp16
// range.  The per-pair operands (basis values, activations, their distance
// derivatives) are required to stay below 2^15 in magnitude -- basis values
// are at most 1 and the activations and derivatives of a trained filter are
// of order one -- and a lane whose operand overflows yields a non-finite
// filter value rather than a silently wrong one.  On this part the fp16 MFMA
// issues at about 14 times the fp32 rate, so the three products cost about a
// fifth of the fp32 ones.
// waves per workgroup of the split-product forward (a build-time tuning
// constant: the workgroup shares one copy of the staged weights)
#ifndef MLCG_X3_WAVES
#define MLCG_X3_WAVES 12
#endif
constexpr int kWavesX3 = MLCG_X3_WAVES;
constexpr int kThreadsX3 = kWavesX3 * MLCG_WAVE;

// Largest |v| over the workgroup (every thread must call; two barriers).
__device__ float block_absmax(float v, float* red) {
  v = fabsf(v);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, MLCG_WAVE));
  if (mlcg_lane() == 0) red[threadIdx.x / MLCG_WAVE] = v;
  __syncthreads();
  float m = 0.f;
  for (int i = 0; i < (int)(blockDim.x / MLCG_WAVE); ++i) m = fmaxf(m, red[i]);
  __syncthreads();
  return m;
}

// S = 2^e with e <= 11 and maxabs S < 2^14.
__device__ __forceinline__ float x3_scale(float maxabs) {
  int ex = 0;
  (void)frexpf(maxabs, &ex);  // maxabs < 2^ex (ex = 0 for 0)
  const int e = ex > 3 ? 14 - ex : 11;
  return ldexpf(1.0f, e);
}

// acc += S A B over one 32-wide k block from A's planes and B's parts.
__device__ __forceinline__ floatx4 mfma_x3(halfx8 ah, halfx8 ahs, halfx8 al, halfx8 bh,
                                           halfx8 bl, floatx4 acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahs, bh, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, acc, 0, 0, 0);
  return acc;
}

// Numerics flags of the split-product kernels (one word per device, set with
// a vector atomic OR, read and cleared by mlcg_numerics_flags):
//   bit 0 -- the filter backward met an activation value |h| or derivative
//            |h'| of 2^19 or more (or a non-finite one), past the range its
//            split operands hold, so its weight gradients may be non-finite;
//   bit 1 -- a filter weight (W1 or W2) of magnitude 65504 (the fp16
//            maximum) or more, past what the weights' fp16 planes hold
//            (forward and backward);
//   bit 2 -- an atom type outside the embedding table (node.hip's
//            embedding lookup, which finds the word through
//            mlcg_numerics_word_ptr).
// (The split forward needs no flag for large activations: a tile whose
// values pass its bound is recomputed with a power-of-two scale, exactly.)
__device__ unsigned mlcg_numerics_word;
constexpr unsigned kFlagBwdRange = 1u;
constexpr unsigned kFlagWeightRange = 2u;
constexpr float kWeightBound = 65504.0f;

__device__ __forceinline__ void raise_numerics_flag(unsigned bits) {
  atomicOr(&mlcg_numerics_word, bits);
}

constexpr int kFlagDevices = 64;
std::mutex g_flag_mutex;
unsigned* g_flag_ptr[kFlagDevices] = {};

__global__ void numerics_flags_kernel(int* out, int clear) {
  if (threadIdx.x == 0) {
    out[0] = (int)mlcg_numerics_word;
    if (clear) mlcg_numerics_word = 0u;
  }
}

// Filter forward, fp32-accurate, on the fp16 MFMA.  The operand layouts are
// those of filter_fwd_f16_kernel (see stage_f16) with K padded to two 32-wide
// k blocks (K <= 64); W1 and W2 are staged as three planes each.  One wave per
// 16-pair tile, 12 waves per workgroup.  Per tile the wave evaluates the basis
// of its 16 pairs once, then walks the 8 feature tiles: a, a' of tile t
// (6 MFMAs per k block), their activation, and the split h, h' parts, which
// accumulate into the B operands of the second product; then the 8 output
// tiles of W, W' (6 MFMAs per 32-wide feature block).  Taking one feature
// tile at a time keeps only 8 accumulators live next to the operand parts.
// Basis rows k >= K are evaluated with centre and width 0 (finite values)
// and meet zero weights, so they add exact zeros.
constexpr int kX3Blocks = 2;  // 32-wide k blocks of the first product
constexpr int kRedoSlots = 8;  // tiles per wave recorded for the scaled pass

template <int BASIS, int ACT>
__global__ __launch_bounds__(kThreadsX3) void filter_fwd_x3_kernel(
    const float* __restrict__ pos, const int32_t* __restrict__ pi,
    const int32_t* __restrict__ pj, const int32_t* __restrict__ n_pairs_dev,
    int64_t max_pairs, RbfParams rp, const float* __restrict__ W1,
    const float* __restrict__ b1, const float* __restrict__ W2, float* __restrict__ Wout,
    float* __restrict__ Wdout, float* __restrict__ dist_out) {
  extern __shared__ float lds[];
  const int K = rp.K;
  constexpr int KS32 = kX3Blocks;
  constexpr int n1 = kFT * KS32 * MLCG_WAVE * 8;       // halfs per W1 plane
  constexpr int n2 = kFT * (kFT / 2) * MLCG_WAVE * 8;  // halfs per W2 plane
  _Float16* w1p = reinterpret_cast<_Float16*>(lds);
  _Float16* w2p = w1p + 3 * n1;
  float* b1s = reinterpret_cast<float*>(w2p + 3 * n2);
  float* bc = b1s + kF;
  float* bw = bc + kMaxK;
  float* red = bw + kMaxK;
  // The weights are read once, into registers, in chunks of 8 plane
  // elements (one halfx8 of one lane's A fragment; chunk c of a plane is
  // held by thread c mod blockDim), which also gives the per-matrix scales
  // from the largest weights; the three planes are then written as halfx8.
  //   W1 chunk c = (t, s, l): W1[16 t + (l & 15)][32 s + 8 (l >> 4) + 0..7]
  //      (zero for k >= K; K <= 64, rows 8-byte aligned: float2 loads)
  //   W2 chunk c = (t, s, l): W2[16 t + (l & 15)][32 s + 4 (l >> 4) + 0..3]
  //      and the same + 16 (two float4 loads)
  constexpr int nc1 = n1 / 8, nc2 = n2 / 8;
  constexpr int kPer1 = (nc1 + kThreadsX3 - 1) / kThreadsX3;
  constexpr int kPer2 = (nc2 + kThreadsX3 - 1) / kThreadsX3;
  float v1[kPer1][8], v2[kPer2][8];
  float m1 = 0.f, m2 = 0.f;
#pragma unroll
  for (int r = 0; r < kPer1; ++r) {
    const int c = threadIdx.x + r * kThreadsX3;
    const int l = c & 63, ts = c >> 6;
    const int s = ts % KS32, t = ts / KS32;
    const int k0 = 32 * s + 8 * (l >> 4);
    const float* row = W1 + (16 * t + (l & 15)) * K;
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      float2 w = float2{0.f, 0.f};
      if (c < nc1) {
        if (k0 + j + 1 < K && (K & 1) == 0) {
          w = *reinterpret_cast<const float2*>(row + k0 + j);
        } else {
          w.x = k0 + j < K ? row[k0 + j] : 0.0f;
          w.y = k0 + j + 1 < K ? row[k0 + j + 1] : 0.0f;
        }
      }
      v1[r][j] = w.x;
      v1[r][j + 1] = w.y;
      m1 = fmaxf(m1, fmaxf(fabsf(w.x), fabsf(w.y)));
    }
  }
#pragma unroll
  for (int r = 0; r < kPer2; ++r) {
    const int c = threadIdx.x + r * kThreadsX3;
    const int l = c & 63, ts = c >> 6;
    const int s = ts % (kFT / 2), t = ts / (kFT / 2);
    const float* src = W2 + (16 * t + (l & 15)) * kF + 32 * s + 4 * (l >> 4);
    float4 lo4 = float4{0.f, 0.f, 0.f, 0.f}, hi4 = lo4;
    if (c < nc2) {
      lo4 = *reinterpret_cast<const float4*>(src);
      hi4 = *reinterpret_cast<const float4*>(src + 16);
    }
    const float w8[8] = {lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v2[r][j] = w8[j];
      m2 = fmaxf(m2, fabsf(w8[j]));
    }
  }
  const float mw1 = block_absmax(m1, red), mw2 = block_absmax(m2, red);
  const float S1 = x3_scale(mw1);
  const float S2 = x3_scale(mw2);
  if (threadIdx.x == 0 && !(fmaxf(mw1, mw2) < kWeightBound)) raise_numerics_flag(kFlagWeightRange);
  auto store_chunk = [](_Float16* plane, int plane_halfs, int c, const float* v, float S) {
    halfx8 h, hs, lo;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const f16split sp = split2(v[j], S);
      h[j] = sp.hi;
      hs[j] = (_Float16)((float)sp.hi * S);
      lo[j] = sp.lo;
    }
    halfx8* p = reinterpret_cast<halfx8*>(plane) + c;
    p[0] = h;
    p[plane_halfs / 8] = hs;
    p[2 * (plane_halfs / 8)] = lo;
  };
#pragma unroll
  for (int r = 0; r < kPer1; ++r) {
    const int c = threadIdx.x + r * kThreadsX3;
    if (c < nc1) store_chunk(w1p, n1, c, v1[r], S1);
  }
#pragma unroll
  for (int r = 0; r < kPer2; ++r) {
    const int c = threadIdx.x + r * kThreadsX3;
    if (c < nc2) store_chunk(w2p, n2, c, v2[r], S2);
  }
  for (int x = threadIdx.x; x < kF; x += blockDim.x) b1s[x] = b1[x];
  stage_basis(bc, bw, rp);  // zeros past K
  __syncthreads();

  int64_t np = *n_pairs_dev;
  if (np > max_pairs) np = max_pairs;
  const int64_t tiles = (np + 15) / 16;
  const int l = mlcg_lane();
  const int q = l >> 4;
  const float inv1 = 1.0f / S1, inv2 = 1.0f / S2;  // powers of two: exact

  const halfx8* w1v = reinterpret_cast<const halfx8*>(w1p);
  const halfx8* w2v = reinterpret_cast<const halfx8*>(w2p);
  constexpr int n1v = n1 / 8, n2v = n2 / 8;
  const int64_t wave = (int64_t)blockIdx.x * kWavesX3 + threadIdx.x / MLCG_WAVE;
  const int64_t nwaves = (int64_t)gridDim.x * kWavesX3;
  // the pair indices are requested two tiles ahead and the bead positions one
  // tile ahead (clamped to the last pair: valid memory, values unused)
  auto pair_at = [&](int64_t t_) -> int64_t {
    const int64_t p_ = (t_ < tiles ? t_ : tiles - 1) * 16 + (l & 15);
    return p_ < np ? p_ : np - 1;
  };
  float3 ri{0.f, 0.f, 0.f}, rj{0.f, 0.f, 0.f};
  int64_t ni = 0, nj = 0;
  if (wave < tiles) {
    const int64_t p0 = pair_at(wave), p1 = pair_at(wave + nwaves);
    const int64_t i0 = pi[p0], j0 = pj[p0];
    ri = float3{pos[3 * i0], pos[3 * i0 + 1], pos[3 * i0 + 2]};
    rj = float3{pos[3 * j0], pos[3 * j0 + 1], pos[3 * j0 + 2]};
    ni = pi[p1];
    nj = pj[p1];
  }
  // outputs of `tile` (lane's pair p, distance d) with the activations
  // scaled by sig; true (wave-uniform) when an output of the tile is not
  // finite
  auto tile_body = [&](int64_t tile, float d, float sig, float inv_sig) -> bool {
    const int64_t p = tile * 16 + (l & 15);
    const bool valid = p < np;
      float crbf, dcrbf, cc, dcc;
      cut_eval(rp.rcut, d, crbf, dcrbf);
      if (rp.same_cut) {  // uniform
        cc = crbf;
        dcc = dcrbf;
      } else {
        cut_eval(rp.ccut, d, cc, dcc);
      }

      // basis g, g' of the lane's pair, k = 32 s + 8 q + j, as split B parts
      halfx8 gh[KS32], gl[KS32], gdh[KS32], gdl[KS32];
#pragma unroll
      for (int s = 0; s < KS32; ++s)
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          float g0, gd0, g1, gd1;
          const int k = 32 * s + 8 * q + j;
          rbf_eval_t<BASIS>(rp, true, bc[k], bw[k], d, crbf, dcrbf, g0, gd0);
          rbf_eval_t<BASIS>(rp, true, bc[k + 1], bw[k + 1], d, crbf, dcrbf, g1, gd1);
          halfx2 h, lo, hd, lod;
          split2x2(g0, g1, S1, h, lo);
          split2x2(gd0, gd1, S1, hd, lod);
          gh[s][j] = h[0];
          gh[s][j + 1] = h[1];
          gl[s][j] = lo[0];
          gl[s][j + 1] = lo[1];
          gdh[s][j] = hd[0];
          gdh[s][j + 1] = hd[1];
          gdl[s][j] = lod[0];
          gdl[s][j + 1] = lod[1];
        }
      // 1.-2. per feature tile t: a = W1 g, a' = W1 g' (times S1); then
      // h = act(a + b1), h' = act'(a + b1) a', times sig, split for the second
      // product.  The split holds |h sig|, |h' sig| below 65504 (the fp16
      // maximum; hi_h S2 is never formed).  A larger value makes its fp16 hi
      // part infinite, and through every row of W2 every output of its pair
      // non-finite: one output of each pair is checked, and such a tile is
      // done again with sig 2^6, 2^12, ... times smaller (exact, undone on the
      // outputs).
      halfx8 hh[kFT / 2], hl[kFT / 2], hdh[kFT / 2], hdl[kFT / 2];
      auto features = [&](float sig) {
#pragma unroll
        for (int t = 0; t < kFT; ++t) {
          floatx4 a = {0.f, 0.f, 0.f, 0.f}, ad = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < KS32; ++s) {
            const int o = (t * KS32 + s) * MLCG_WAVE + l;
            const halfx8 ah = w1v[o], ahs = w1v[n1v + o], al = w1v[2 * n1v + o];
            a = mfma_x3(ah, ahs, al, gh[s], gl[s], a);
            ad = mfma_x3(ah, ahs, al, gdh[s], gdl[s], ad);
          }
          const float4 bias = *reinterpret_cast<const float4*>(b1s + 16 * t + 4 * q);
          const float bv[4] = {bias.x, bias.y, bias.z, bias.w};
#pragma unroll
          for (int i = 0; i < 4; i += 2) {
            float s0, s1, e0, e1, unused;
            act_t<ACT>(a[i] * inv1 + bv[i], s0, e0, unused);
            act_t<ACT>(a[i + 1] * inv1 + bv[i + 1], s1, e1, unused);
            float hd0 = e0 * (ad[i] * inv1), hd1 = e1 * (ad[i + 1] * inv1);
            s0 *= sig;
            s1 *= sig;
            hd0 *= sig;
            hd1 *= sig;
            halfx2 h, lo, hd, lod;
            split2x2(s0, s1, S2, h, lo);
            split2x2(hd0, hd1, S2, hd, lod);
            const int e = 4 * (t & 1) + i;
            hh[t >> 1][e] = h[0];
            hh[t >> 1][e + 1] = h[1];
            hl[t >> 1][e] = lo[0];
            hl[t >> 1][e + 1] = lo[1];
            hdh[t >> 1][e] = hd[0];
            hdh[t >> 1][e + 1] = hd[1];
            hdl[t >> 1][e] = lod[0];
            hdl[t >> 1][e + 1] = lod[1];
          }
        }
      };
      features(sig);
      // 3. per output tile t: w = W2 h, w' = W2 h' (times S2 sig), enveloped
      const float c2 = cc * (inv2 * inv_sig), dc2 = dcc * (inv2 * inv_sig);  // powers of two
      bool bad = false;
      float* wr = Wout + p * kF + 4 * q;
      float* wdr = Wdout + p * kF + 4 * q;
#pragma unroll
      for (int t = 0; t < kFT; ++t) {
        floatx4 w = {0.f, 0.f, 0.f, 0.f}, wd = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < kFT / 2; ++s) {
          const int o = (t * (kFT / 2) + s) * MLCG_WAVE + l;
          const halfx8 ah = w2v[o], ahs = w2v[n2v + o], al = w2v[2 * n2v + o];
          w = mfma_x3(ah, ahs, al, hh[s], hl[s], w);
          wd = mfma_x3(ah, ahs, al, hdh[s], hdl[s], wd);
        }
        if (t == 0) bad = valid && !(__builtin_isfinite(w[0]) && __builtin_isfinite(wd[0]));
        if (valid) {
          float4 o, od;
          float* op = reinterpret_cast<float*>(&o);
          float* odp = reinterpret_cast<float*>(&od);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            op[i] = w[i] * c2;
            odp[i] = wd[i] * c2 + w[i] * dc2;
          }
          nt_store4(wr + 16 * t, o);
          nt_store4(wdr + 16 * t, od);
        }
      }
    if (valid && dist_out && q == 0) dist_out[p] = d;
    return __builtin_amdgcn_ballot_w64(bad) != 0;
  };
  // tiles of this wave to do again with scaled activations (rare)
  int* redo = reinterpret_cast<int*>(red + kWavesX3) +
              __builtin_amdgcn_readfirstlane(threadIdx.x / MLCG_WAVE) * kRedoSlots;
  int n_redo = 0;
  for (int64_t tile = wave; tile < tiles; tile += nwaves) {
    const int64_t p = tile * 16 + (l & 15);
    const bool valid = p < np;
    float d = 1.0f;
    if (valid) {
      const float dx = rj.x - ri.x, dy = rj.y - ri.y, dz = rj.z - ri.z;
      d = sqrtf(dx * dx + dy * dy + dz * dz);
    }
    ri = float3{pos[3 * ni], pos[3 * ni + 1], pos[3 * ni + 2]};
    rj = float3{pos[3 * nj], pos[3 * nj + 1], pos[3 * nj + 2]};
    {
      const int64_t p2 = pair_at(tile + 2 * nwaves);
      ni = pi[p2];
      nj = pj[p2];
    }
    if (tile_body(tile, d, 1.0f, 1.0f)) {  // rare: recorded, done again below
      if (n_redo < kRedoSlots && l == 0) redo[n_redo] = (int)tile;
      ++n_redo;
    }
  }
  // Tiles with an activation past the fp16 range (or a non-finite input,
  // which no scale repairs) again, with sig = 2^-6, 2^-12, ..., 2^-30, after
  // the main loop so that its registers are not shared with this path; when
  // more tiles overflowed than the slots hold, every tile of the wave is
  // checked again from sig = 1.
  const bool redo_all = n_redo > kRedoSlots;
  const int n_pass = redo_all ? (int)((tiles - wave + nwaves - 1) / nwaves) : n_redo;
  for (int r = 0; r < n_pass; ++r) {
    const int64_t tile =
        redo_all ? wave + (int64_t)r * nwaves : (int64_t)__builtin_amdgcn_readfirstlane(redo[r]);
    const int64_t p = pair_at(tile);
    const int64_t i = pi[p], j = pj[p];
    const float dx = pos[3 * j] - pos[3 * i], dy = pos[3 * j + 1] - pos[3 * i + 1],
                dz = pos[3 * j + 2] - pos[3 * i + 2];
    const float d = tile * 16 + (l & 15) < np ? sqrtf(dx * dx + dy * dy + dz * dz) : 1.0f;
    float sig = redo_all ? 64.0f : 1.0f, inv_sig = redo_all ? 0.015625f : 1.0f;
    for (int pass = 0; pass < 6; ++pass) {
      sig *= 0.015625f;
      inv_sig *= 64.0f;
      if (!tile_body(tile, d, sig, inv_sig)) break;
    }
  }
}

size_t fwd_x3_lds_bytes(int K) {
  if (K > 32 * kX3Blocks) return SIZE_MAX;  // the x3 kernel pads K to 64
  return sizeof(_Float16) * 3 *
             (kFT * kX3Blocks * MLCG_WAVE * 8 + kFT * (kFT / 2) * MLCG_WAVE * 8) +
         sizeof(float) * (kF + 2 * kMaxK + kWavesX3) + sizeof(int) * kWavesX3 * kRedoSlots;
}

// ---------------------------------------------------------------------------
// Reverse of the chain with the weight-gradient reductions fused in (fp32).
//
// For given pair adjoints Wbar = dL/dW and Wdbar = dL/dWd, per pair:
//   t   = Wbar C + Wdbar C'            t'  = Wdbar C
//   hb  = W2^T t                       hb' = W2^T t'
//   ab  = hb act'(a) + hb' act''(a) a' ab' = hb' act'(a)
// and the parameter gradients are pair sums
//   dW2 = sum_p t h^T + t' h'^T,  dW1 = sum_p ab g^T + ab' g'^T,  db1 = sum_p ab.
//
// Work split: a workgroup of 8 waves walks 16-pair tiles; wave w owns feature
// tile w (features 16w..16w+15) in every product.  Its slice of W1 (one A
// fragment per k step) stays in registers; the W2^T A fragments of all eight
// tiles are staged once in LDS.  Per tile:
//   1. a, a' of feature tile w (v_mfma_f32_16x16x4f32, B operand g, g' from
//      LDS; for K <= 64 three v_mfma_f32_16x16x32_f16 per 32-wide k block of
//      split operands, W1's two planes in registers -- the 16x16x16 fp16
//      shape sustains half the rate of the 16x16x32 one on gfx950);
//   2. t, t', h, h' of its features, published in LDS;         -- barrier --
//   3. hb, hb' of its tile (B operands = all 128 t features from LDS);
//   4. dW2 rows of its tile += t^T h over the 16 pairs (the pair index is the
//      MFMA reduction axis);
//   5. ab, ab' published, and the basis g, g' and envelope C, C' of the next
//      tile evaluated (wave w: k steps w, w + 8, ...);        -- barrier --
//   6. dW1 rows of its tile += ab^T g.
// g, g' are double-buffered across tiles, so a tile costs two barriers.  The
// accumulators stay in registers across all tiles of the workgroup; at the
// end each workgroup writes its partial sums, and filter_bwd_reduce adds the
// partials in workgroup order, so the result is deterministic.  Nothing per
// pair is written to HBM (unless the first-layer pair adjoints are asked for).
//
// The global inputs of a tile (bead positions, node vectors) are requested
// one tile ahead and the pair indices two tiles ahead, so no load latency is
// waited for inside a tile.
//
// LDS layouts (fp32 path; the split path's TB, TT and AT layouts and the
// measured lane groups of the LDS are given at tb_swz and tt_at).
//   TB  [pair][feature]: t, t' as the B operand of step 3 (float4 of four
//       features of one pair); rows of 128 floats, float4 group g of pair n
//       stored at g ^ (n & 7).
//   TT, HT, AT, GT  [row][pair] (row = feature, or basis index k for GT): the
//       operands of the pair reductions, steps 4 and 6 (float4 of four pairs
//       of one row), and the B operand of step 1 (scalar); rows of 16 floats,
//       float4 pair group c of row r stored at c ^ ((r >> 1) & 3).
constexpr int kBwdWaves = 8;
constexpr int kBwdXcds = 8;  // XCDs of the chip (workgroups dispatched round-robin)
constexpr int kBwdThreads = kBwdWaves * MLCG_WAVE;

__device__ __forceinline__ int tb_at(int pair, int g) { return pair * kF + ((g ^ (pair & 7)) << 2); }
// Split path: chunk g (16 bytes) of pair n's fp16 row at g ^ tb_swz(n).
// Measured on gfx950 (LDS bank-conflict counter, one wave): a 16-byte-per-lane
// access is served for the lane groups {0-3, 12-15, 20-23, 24-27} and
// {4-11, 16-19, 28-31} (and the same + 32) in one cycle each over 64
// four-byte banks, an 8-byte access for lanes 0-31 and 32-63 over 64 banks,
// a 4-byte access for lanes 0-31 and 32-63 over 32 banks.  The pair row of
// 256 bytes covers the 64 banks once; with this permutation both the step-3
// reads (chunk 4 sb + q of pair n) and the step-2 writes (chunk 2 w + q / 2,
// half q % 2) reach distinct banks in every group.
__device__ __forceinline__ int tb_swz(int n) { return n ^ (n >> 2); }
// Split path: TT and AT [row][pair] (rows of 16 floats): row r at position
// r ^ ((r >> 2) & 3) and pair p at p ^ 4 ((r >> 2) & 1).  The scalar writes
// (lane (n, q) -> row 16 w + 4 q + i, pair n) and the float4 reads (lane
// (n, q) -> row 16 w + n, pairs 8 (q & 1) + 0..3 and + 4..7) are then free of
// bank conflicts under the lane groups above.
__device__ __forceinline__ int tt_at(int r, int pair) {
  return 16 * (r ^ ((r >> 2) & 3)) + (pair ^ (((r >> 2) & 1) << 2));
}
__device__ __forceinline__ int rp_at(int r, int pair) {
  return r * 16 + ((((pair >> 2) ^ ((r >> 1) & 3)) << 2) | (pair & 3));
}

__host__ __device__ constexpr int bwd_kp16(int K) { return 16 * ((K + 15) / 16); }
__host__ __device__ constexpr int bwd_partial_floats(int K) {
  return kF * kF + kF * bwd_kp16(K) + kF;
}
__host__ __device__ constexpr int bwd_krows(int K) { return K <= 64 ? 64 : 128; }
// LDS: W2^T fragments [8][8][64] float4 (or two fp16 planes) | TB [2][16][128]
//      (or two fp16 planes) | TT, HT, AT [2][128][16] (split path: AT in
//      TT's memory) | GT [2 buffers][2][krows][16] (split path: two fp16
//      planes, followed by the pair-major three-plane copy of g, g' for step
//      1, [3][2][16][64] halfs) | per-pair maxima (split path: [2 buffers][2]
//      [16] atomic-max bits; 256 floats reserved, the W2 scale's reduction
//      scratch); 144,384 bytes for K <= 64 and exactly the 160 KiB of a
//      gfx950 CU for K <= 128
__host__ __device__ constexpr int bwd_lds_floats(int K) {
  return K <= 64 ? kFT * kFT * MLCG_WAVE * 4 + 2 * 16 * kF + 2 * 2 * kF * 16 +
                       2 * 2 * bwd_krows(K) * 16 + 3 * 2 * 16 * 64 / 2 + 2 * kBwdWaves * 16
                 : kFT * kFT * MLCG_WAVE * 4 + 2 * 16 * kF + 3 * 2 * kF * 16 +
                       2 * 2 * bwd_krows(K) * 16;
}

// Where the pair adjoints (Wbar, Wdbar) come from: explicit [P, F] arrays, or
// formed on the fly from node vectors of the CFConv aggregation (the reverse
// of agg_i = sum_j y_j W_ij with a tangent stream, see mlcg_hip.h):
//   Wbar_p  = g2_i y_j + g2_j y_i + g1_i yd_j + g1_j yd_i
//   Wdbar_p = dd_p (g1_i y_j + g1_j y_i)
// which saves writing and re-reading two [P, F] arrays.
struct PairAdjoint {
  const float* Wbar;
  const float* Wdbar;
  const float* g2;    // node mode: gagg2 [N, F]
  const float* y;     //            y [N, F]
  const float* g1;    //            gagg1 [N, F] or null (no tangent)
  const float* yd;    //            ydot [N, F] or null
  const float* dd;    //            ddot [P] (with g1)
};

__device__ __forceinline__ float4 ld4(const float* __restrict__ p, int64_t row, int col) {
  return *reinterpret_cast<const float4*>(p + row * kF + col);
}
__device__ __forceinline__ float4 f4(float a, float b, float c, float d) {
  return float4{a, b, c, d};
}

// Global inputs of one lane's pair for one tile.  Every load is issued
// unconditionally (lanes past the last pair read the last pair, and absent
// tangent arrays are replaced by present ones whose values are not used), so
// that no branch joins force a wait for the loads before they are needed.
struct TileIn {
  float xi, yi, zi, xj, yj, zj;  // positions of the pair's beads
  float4 v[8];                   // adjoint sources (explicit: v[0..1])
  float dd;
};

template <bool kNodes>
__device__ __forceinline__ TileIn fetch_tile(const float* __restrict__ pos,
                                             const PairAdjoint& adj, const float* ddp,
                                             const float* g1p, const float* ydp, int64_t p,
                                             int64_t i, int64_t j, int fcol) {
  TileIn t;
  t.xi = pos[3 * i];
  t.yi = pos[3 * i + 1];
  t.zi = pos[3 * i + 2];
  t.xj = pos[3 * j];
  t.yj = pos[3 * j + 1];
  t.zj = pos[3 * j + 2];
  if (!kNodes) {
    t.v[0] = ld4(adj.Wbar, p, fcol);
    t.v[1] = ld4(adj.Wdbar, p, fcol);
#pragma unroll
    for (int k = 2; k < 8; ++k) t.v[k] = float4{0.f, 0.f, 0.f, 0.f};
    t.dd = 0.f;
  } else {
    t.v[0] = ld4(adj.g2, i, fcol);
    t.v[1] = ld4(adj.g2, j, fcol);
    t.v[2] = ld4(adj.y, i, fcol);
    t.v[3] = ld4(adj.y, j, fcol);
    t.v[4] = ld4(g1p, i, fcol);
    t.v[5] = ld4(g1p, j, fcol);
    t.v[6] = ld4(ydp, i, fcol);
    t.v[7] = ld4(ydp, j, fcol);
    t.dd = ddp[p];
  }
  return t;
}

// Wbar, Wdbar of the lane's 4 features from the prefetched sources (zero for
// a lane past the last pair: vm = 0).
template <bool kNodes>
__device__ __forceinline__ void tile_adjoint(const TileIn& t, bool tangent, bool has_yd,
                                             float vm, float4& wb, float4& wdb) {
  if (!kNodes) {
    wb = f4(t.v[0].x * vm, t.v[0].y * vm, t.v[0].z * vm, t.v[0].w * vm);
    wdb = f4(t.v[1].x * vm, t.v[1].y * vm, t.v[1].z * vm, t.v[1].w * vm);
    return;
  }
  const float4 g2i = t.v[0], g2j = t.v[1], yi = t.v[2], yj = t.v[3];
  const float4 g1i = t.v[4], g1j = t.v[5], ydi = t.v[6], ydj = t.v[7];
  wb = f4(g2i.x * yj.x + g2j.x * yi.x, g2i.y * yj.y + g2j.y * yi.y,
          g2i.z * yj.z + g2j.z * yi.z, g2i.w * yj.w + g2j.w * yi.w);
  wdb = f4(0.f, 0.f, 0.f, 0.f);
  if (tangent) {
    if (has_yd) {
      wb.x += g1i.x * ydj.x + g1j.x * ydi.x;
      wb.y += g1i.y * ydj.y + g1j.y * ydi.y;
      wb.z += g1i.z * ydj.z + g1j.z * ydi.z;
      wb.w += g1i.w * ydj.w + g1j.w * ydi.w;
    }
    const float s = t.dd * vm;
    wdb = f4(s * (g1i.x * yj.x + g1j.x * yi.x), s * (g1i.y * yj.y + g1j.y * yi.y),
             s * (g1i.z * yj.z + g1j.z * yi.z), s * (g1i.w * yj.w + g1j.w * yi.w));
  }
  wb = f4(wb.x * vm, wb.y * vm, wb.z * vm, wb.w * vm);
}

template <int KSMAX, bool kNodes, int BASIS, int ACT>
__global__ __launch_bounds__(kBwdThreads) void filter_bwd_fused_kernel(
    const float* __restrict__ pos, const int32_t* __restrict__ pi,
    const int32_t* __restrict__ pj, const int32_t* __restrict__ n_pairs_dev,
    int64_t max_pairs, RbfParams rp, const float* __restrict__ W1,
    const float* __restrict__ b1, const float* __restrict__ W2, PairAdjoint adj,
    float* __restrict__ abar_out, float* __restrict__ adbar_out, float* __restrict__ partial) {
  constexpr int KTMAX = (4 * KSMAX + 15) / 16;
  // basis rows span the compile-time maximum width (rows k >= K hold zeros),
  // so the k loops below run without data-dependent branches
  constexpr int kRows = 16 * KTMAX;
  static_assert(4 * KSMAX == kRows, "every basis row is written for every tile");
  extern __shared__ float lds[];
  const int K = rp.K;
  const int Kp16 = bwd_kp16(K);
  const int KT = Kp16 / 16;
  // step 3 on the fp16 MFMA with split operands (see filter_fwd_x3_kernel)
  // when the LDS allows it (K <= 64); the wide variant keeps it on fp32
  constexpr bool kX3 = KSMAX <= 16;
  // split scales: S4 of every split product; h enters step 4 as h beta_h, and
  // g, g' enter step 1 as g beta_0, g' beta_1 (so hi S4 stays in the fp16
  // range for |h| < 2^20, |g| < 512 and |g'| < 2047)
  constexpr float kS4 = 2048.0f, kBetaH = 0.0625f, kBetaG0 = 0.0625f, kBetaG1 = 0.015625f;
  // fp32: W2^T A fragments [8 t][8 u][64 l] float4; x3: W2^T as two fp16
  // planes (hi, lo S) of [8 t][4 s][64 l][8]
  float* w2ts = lds;
  // fp32: [2][16 pairs][128] t, t'; x3: two fp16 planes (hi, lo S) of
  // [2][16 pairs][128], each t scaled per pair (sigma) into [-4, 4]
  float* TB = w2ts + kFT * kFT * MLCG_WAVE * 4;
  float* TT = TB + 2 * 16 * kF;  // [2][128][16 pairs]  t, t'
  float* HT = TT + 2 * kF * 16;  // [2][128][16 pairs]  h, h'
  // [2][128][16 pairs] ab, ab'.  On the split path AT shares TT's memory: both
  // hold rows of the wave's own features only, and a wave reads TT (step 4)
  // before it writes AT (step 5) and reads AT (step 6) before it writes the
  // next tile's TT (step 2), all in program order.
  float* AT = kX3 ? TT : HT + 2 * kF * 16;
  float* GT0 = kX3 ? HT + 2 * kF * 16 : AT + 2 * kF * 16;  // [2 bufs][2][kRows][16] g, g'
  // split path: GT0 holds the [row][pair] fp16 planes of g, g' (step 6); G1h
  // the pair-major planes (hi, hi S4, lo S4) of g beta_0, g' beta_1 for step
  // 1, [3][2][16 pairs][64 k], 16-byte chunk c of pair n's row stored at
  // c ^ (n & 7) (one buffer: written in step 5 after the barrier that follows
  // step 1).  With this permutation the step-1 reads (lane (q, n): chunk
  // 4b + q of pair n) reach distinct banks in both 16-byte lane groups.
  _Float16* G1h = reinterpret_cast<_Float16*>(GT0 + 2 * 2 * kRows * 16);
  float* PMAX = GT0 + 2 * 2 * kRows * 16 + (kX3 ? 3 * 2 * 16 * 64 / 2 : 0);  // x3: [2][2][16] bits
  unsigned* PMAXu = reinterpret_cast<unsigned*>(PMAX);
  const int w = threadIdx.x / MLCG_WAVE;
  const int l = mlcg_lane();
  const int q = l >> 4, n = l & 15;

  float S = 1.0f, inv_S = 1.0f;  // x3: the split scale of W2 and t
  if constexpr (kX3) {
    // W2 read once into registers, in chunks of 8 plane elements (one halfx8
    // of one lane's A fragment; chunk c held by thread c mod blockDim), which
    // also gives the scale; then both planes written as halfx8.  Chunk
    // c = (t, s, ll): A[m][8 kq + j] of block s for tile t =
    // W2[32 s + 8 kq + j][16 t + m], m = ll & 15, kq = ll >> 4.
    constexpr int kChunks = kF * kF / 8;
    constexpr int kPer = kChunks / kBwdThreads;
    static_assert(kChunks % kBwdThreads == 0, "whole chunks per thread");
    float v2[kPer][8];
    float m2 = 0.f;
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
      const int c = threadIdx.x + r * kBwdThreads;
      const int ll = c & 63, ts = c >> 6;
      const int sb = ts & 3, t = ts >> 2;
      const float* src = W2 + (32 * sb + 8 * (ll >> 4)) * kF + 16 * t + (ll & 15);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        v2[r][j] = src[j * kF];
        m2 = fmaxf(m2, fabsf(v2[r][j]));
      }
    }
    const float mw2 = block_absmax(m2, PMAX);
    S = x3_scale(mw2);
    inv_S = 1.0f / S;
    if (threadIdx.x == 0 && !(mw2 < kWeightBound)) raise_numerics_flag(kFlagWeightRange);
    halfx8* w2h = reinterpret_cast<halfx8*>(w2ts);
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
      const int c = threadIdx.x + r * kBwdThreads;
      halfx8 h, lo;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const f16split sp = split2(v2[r][j], S);
        h[j] = sp.hi;
        lo[j] = sp.lo;
      }
      w2h[c] = h;
      w2h[kChunks + c] = lo;
    }
  } else {
    stage_w2_f32(w2ts, W2, true);
  }

  // W1 fragment of feature tile w stays in registers: W1[16w + n][4s + q]
  // (fp32 path) or, on the split path, the two planes (hi, lo S4) of the
  // v_mfma_f32_16x16x32_f16 A fragments W1[16w + n][32b + 8q + j]
  float w1f[KSMAX];
  halfx8 w1h[KSMAX / 8], w1l[KSMAX / 8];
  if constexpr (kX3) {
    bool w1_big = false;
#pragma unroll
    for (int b = 0; b < KSMAX / 8; ++b)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int k = 32 * b + 8 * q + j;
        const float v = k < K ? W1[(16 * w + n) * K + k] : 0.0f;
        w1_big = w1_big || !(fabsf(v) < kWeightBound);
        const f16split sp = split2(v, kS4);
        w1h[b][j] = sp.hi;
        w1l[b][j] = sp.lo;
      }
    if (w1_big) raise_numerics_flag(kFlagWeightRange);
  } else {
#pragma unroll
    for (int s = 0; s < KSMAX; ++s) {
      const int k = 4 * s + q;
      w1f[s] = k < K ? W1[(16 * w + n) * K + k] : 0.0f;
    }
  }
  float bias[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) bias[i] = b1[16 * w + 4 * q + i];
  // parameters of the basis functions this lane evaluates (k = 4 (8e + w) + q),
  // kept in registers when K <= 64 (the wide variant has no registers to
  // spare and reads them per tile)
  constexpr int kBasisSteps = (KSMAX + kBwdWaves - 1) / kBwdWaves;
  constexpr bool kBasisRegs = KSMAX <= 16;
  float bcen[kBasisSteps], bwid[kBasisSteps];
#pragma unroll
  for (int e = 0; e < kBasisSteps; ++e)
    if (kBasisRegs) basis_params(rp, 4 * (kBwdWaves * e + w) + q, bcen[e], bwid[e]);

  floatx4 acc2[kFT];
#pragma unroll
  for (int u = 0; u < kFT; ++u) acc2[u] = floatx4{0.f, 0.f, 0.f, 0.f};
  floatx4 acc1[KTMAX];
#pragma unroll
  for (int kt = 0; kt < KTMAX; ++kt) acc1[kt] = floatx4{0.f, 0.f, 0.f, 0.f};
  float db[4] = {0.f, 0.f, 0.f, 0.f};

  int64_t np = max_pairs > 0 ? *n_pairs_dev : 0;
  if (np > max_pairs) np = max_pairs;
  const int64_t tiles = (np + 15) / 16;
  const int fcol = 16 * w + 4 * q;  // first of the lane's 4 features
  // LDS offsets: a per-lane base plus a compile-time offset per unrolled step
  const int oTBw = tb_at(n, 4 * w + q);  // step 2: t, t' of (pair n, features fcol..)
  int oTB3[2];                           // step 3: tb_at(n, 4u + q) = oTB3[u & 1] + 32 (u >> 1)
#pragma unroll
  for (int e = 0; e < 2; ++e) oTB3[e] = n * kF + 16 * (e ^ ((n >> 2) & 1)) + 4 * (q ^ (n & 3));
  // steps 4, 6: rp_at(16x + n, 4q) = oR + 256 x (float4 of pairs 4q..4q+3)
  const int oR = n * 16 + 4 * (q ^ ((n >> 1) & 3));
  const int oRw = oR + 256 * w;
  int oG1[2];  // step 1: rp_at(4s + q, n) = oG1[s & 1] + 64 s
#pragma unroll
  for (int e = 0; e < 2; ++e) oG1[e] = 16 * q + 4 * ((n >> 2) ^ ((2 * e) | (q >> 1))) + (n & 3);
  int oW[4];  // steps 2, 5: rp_at(16w + 4q + i, n)
#pragma unroll
  for (int i = 0; i < 4; ++i) oW[i] = kX3 ? tt_at(fcol + i, n) : rp_at(fcol + i, n);
  const float4* w2v = reinterpret_cast<const float4*>(w2ts) + (w * kFT) * MLCG_WAVE + l;
  // step 4 on the split path: A = TT row 16w + n, stream q >> 1, pairs
  // 8 (q & 1) .. + 7 (two float4, the second at offset ^ 4); B = halfx8 of HT
  // plane rows 16u + (n ^ (n >> 2)), same stream and pairs
  // split scales of step 4: t rw (rw = 2^k, with |t| rw < 4 over every tile
  // seen so far), h beta; the accumulators hold S4 rw beta dW2
  float rw = 1.0f, trun = 0.0f;
  float ra = 1.0f, arun = 0.0f;  // the same for ab in step 6 (no beta: |g| <= 1)

  const bool tangent = kNodes && adj.g1 != nullptr;
  const bool has_yd = tangent && adj.yd != nullptr;
  // stand-ins for absent tangent arrays: valid memory, values never used
  const float* g1p = tangent ? adj.g1 : adj.g2;
  const float* ydp = has_yd ? adj.yd : adj.y;
  const float* ddp = tangent ? adj.dd : reinterpret_cast<const float*>(pi);
  auto clamp_pair = [&](int64_t t_) -> int64_t {
    const int64_t p = t_ * 16 + n;
    return p < np ? p : np - 1;
  };
  // Basis of a tile: wave w evaluates k steps w, w + 8, ... for the 16 pairs
  // (into GT), every lane the envelope of its own pair.  In two parts, so that
  // the arithmetic (basis_eval) can be scheduled among the MFMAs of step 4
  // and only the LDS writes (basis_store) come after them.
  // Lanes past the last pair evaluate the (finite) basis and activations of
  // the last pair but carry zero adjoints (tile_adjoint's mask), hence
  // t = t' = 0 and ab = ab' = 0: they add exact zeros to every pair sum.
  struct BasisV {
    float cc, dcc;                        // envelope of the lane's pair
    float g[kBasisSteps], gd[kBasisSteps];  // fp32 path
    halfx2 sh[kBasisSteps], sl[kBasisSteps];  // split path: GT planes (hi, lo S4)
    halfx2 ch[kBasisSteps], chs[kBasisSteps], cl[kBasisSteps];  // step 1's planes
  };
  auto basis_eval = [&](const TileIn& t) -> BasisV {
    BasisV bv;
    const float dx = t.xj - t.xi, dy = t.yj - t.yi, dz = t.zj - t.zi;
    const float d = sqrtf(dx * dx + dy * dy + dz * dz);
    float crbf, dcrbf;
    envelopes(rp, d, crbf, dcrbf, bv.cc, bv.dcc);
#pragma unroll
    for (int e = 0; e < kBasisSteps; ++e) {
      const int s = kBwdWaves * e + w;
      float g = 0.f, gd = 0.f;
      if (s < KSMAX) {
        float cen = bcen[e], wid = bwid[e];
        if (!kBasisRegs) basis_params(rp, 4 * s + q, cen, wid);
        rbf_any<BASIS>(rp, 4 * s + q < K, cen, wid, d, crbf, dcrbf, g, gd);  // zero for k >= K
      }
      bv.g[e] = g;
      bv.gd[e] = gd;
      if constexpr (kX3) {
        split2x2(g, gd, kS4, bv.sh[e], bv.sl[e]);
        split2x2(g * kBetaG0, gd * kBetaG1, kS4, bv.ch[e], bv.cl[e]);
        // hi S4 in fp16: exact (a power of two), one packed multiply
        bv.chs[e] = bv.ch[e] * halfx2{(_Float16)kS4, (_Float16)kS4};
      }
    }
    return bv;
  };
  auto basis_store = [&](const BasisV& bv, int bsel) {
    float* GTb = GT0 + bsel * 2 * kRows * 16;
#pragma unroll
    for (int e = 0; e < kBasisSteps; ++e) {
      const int s = kBwdWaves * e + w;
      if (s < KSMAX) {
        if constexpr (kX3) {
          // two fp16 planes (hi, lo S4) of [2][kRows][16 pairs]
          _Float16* GTh = reinterpret_cast<_Float16*>(GTb);
          const int o = (4 * s + q) * 16 + n;
          GTh[o] = bv.sh[e][0];
          GTh[kRows * 16 + o] = bv.sh[e][1];
          GTh[2 * kRows * 16 + o] = bv.sl[e][0];
          GTh[3 * kRows * 16 + o] = bv.sl[e][1];
          // step 1's copy (k = 4s + q: 16-byte chunk s / 2, element
          // 4 (s & 1) + q)
          const int o1 = n * 64 + 8 * ((s >> 1) ^ (n & 7)) + 4 * (s & 1) + q;
          G1h[o1] = bv.ch[e][0];
          G1h[1024 + o1] = bv.ch[e][1];
          G1h[2048 + o1] = bv.chs[e][0];
          G1h[3072 + o1] = bv.chs[e][1];
          G1h[4096 + o1] = bv.cl[e][0];
          G1h[5120 + o1] = bv.cl[e][1];
        } else {
          const int o = rp_at(4 * s + q, n);
          GTb[o] = bv.g[e];
          GTb[kRows * 16 + o] = bv.gd[e];
        }
      }
    }
  };

  // t, t' of the lane's 4 features of a tile (formed one tile ahead, in the
  // barrier interval of step 5) and, on the split path, the per-pair maxima
  // of |t|, |t'| over the wave's 16 features, published for step 2
  float tbv[4], tdbv[4];
  float tmax_tile = 0.f;  // split path: max |t|, |t'| over the wave's features and pairs
  // in two parts like the basis: the arithmetic, then the LDS atomics
  auto pair_adjoints_eval = [&](float4 wb, float4 wdb, float cc, float dcc, float& m0,
                                float& m1) {
    const float wbv[4] = {wb.x, wb.y, wb.z, wb.w};
    const float wdbv[4] = {wdb.x, wdb.y, wdb.z, wdb.w};
    m0 = 0.f;
    m1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      tbv[i] = wbv[i] * cc + wdbv[i] * dcc;
      tdbv[i] = wdbv[i] * cc;
      m0 = fmaxf(m0, fabsf(tbv[i]));
      m1 = fmaxf(m1, fabsf(tdbv[i]));
    }
    if constexpr (kX3) {
      m0 = cross_row_max(m0);
      m1 = cross_row_max(m1);
      const float mx = row16_max(fmaxf(m0, m1));
      tmax_tile = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(mx)));
    }
  };
  auto pair_adjoints_store = [&](float m0, float m1, int pb) {
    if constexpr (kX3) {
      if (q == 0) {  // non-negative floats order as their bit patterns
        atomicMax(PMAXu + pb * 32 + n, __float_as_uint(m0));
        atomicMax(PMAXu + pb * 32 + 16 + n, __float_as_uint(m1));
      }
    }
  };

  int buf = 0;
  float cc_cur = 0.f, dcc_cur = 0.f;
  int64_t ni = 0, nj = 0;  // bead indices of the next tile's pair
  __syncthreads();  // PMAX served as scratch of the W2 scale
  if constexpr (kX3) {
    if (threadIdx.x < 64) PMAXu[threadIdx.x] = 0u;
    __syncthreads();
  }
  // XCD-aware tile order: workgroups are dispatched round-robin over the
  // XCDs, and the workgroups of one XCD take one contiguous range of tiles
  // (strided among them), so the node rows of a frame's pairs are fetched
  // into that XCD's L2 only, not into every XCD's (config 2: 269.5 -> 265 us).
  const int nx = (int)gridDim.x < kBwdXcds ? (int)gridDim.x : kBwdXcds;
  const int xcd = blockIdx.x % nx, wl = blockIdx.x / nx;
  const int64_t stride = gridDim.x / nx + (xcd < (int)(gridDim.x % nx) ? 1 : 0);
  const int64_t t_start = tiles * xcd / nx + wl, t_end = tiles * (xcd + 1) / nx;
  if (np > 0) {  // uniform across the workgroup
    const int64_t p0 = clamp_pair(t_start);
    const TileIn first = fetch_tile<kNodes>(pos, adj, ddp, g1p, ydp, p0, pi[p0], pj[p0], fcol);
    const int64_t p1 = clamp_pair(t_start + stride);
    ni = pi[p1];
    nj = pj[p1];
    const float vm0 = t_start * 16 + n < np ? 1.0f : 0.0f;
    const BasisV bv0 = basis_eval(first);
    basis_store(bv0, 0);
    cc_cur = bv0.cc;
    dcc_cur = bv0.dcc;
    float4 wb0, wdb0;
    tile_adjoint<kNodes>(first, tangent, has_yd, vm0, wb0, wdb0);
    float pm0, pm1;
    pair_adjoints_eval(wb0, wdb0, cc_cur, dcc_cur, pm0, pm1);
    pair_adjoints_store(pm0, pm1, 0);
  }
  __syncthreads();
  for (int64_t tile = t_start; tile < t_end; tile += stride, buf ^= 1) {
    float* GT = GT0 + buf * 2 * kRows * 16;
    const float vmask = tile * 16 + n < np ? 1.0f : 0.0f;
    // inputs of the next tile and indices of the one after it: consumed in
    // step 5 and one tile later
    const int64_t pn = clamp_pair(tile + stride);
    const TileIn nxt = fetch_tile<kNodes>(pos, adj, ddp, g1p, ydp, pn, ni, nj, fcol);
    {
      const int64_t pnn = clamp_pair(tile + 2 * stride);
      ni = pi[pnn];
      nj = pj[pnn];
    }

    // 1. a, a' of feature tile w (two accumulators each: shorter MFMA chains)
    floatx4 a = {0.f, 0.f, 0.f, 0.f}, ad = {0.f, 0.f, 0.f, 0.f};
    floatx4 a_o = {0.f, 0.f, 0.f, 0.f}, ad_o = {0.f, 0.f, 0.f, 0.f};
    if constexpr (kX3) {
      // 32-wide k blocks; B fragment = halfx8 of pair n, k = 32b + 8q .. + 7;
      // slabs (plane, stream) of 128 halfx8: hi (0, 1), hi S (2, 3), lo S (4, 5)
      const halfx8* g1v = reinterpret_cast<const halfx8*>(G1h);
#pragma unroll
      for (int b = 0; b < KSMAX / 8; ++b) {
        const int c = n * 8 + ((4 * b + q) ^ (n & 7));
        const halfx8 h0 = g1v[c], s0 = g1v[256 + c], l0 = g1v[512 + c];
        const halfx8 h1 = g1v[128 + c], s1 = g1v[384 + c], l1 = g1v[640 + c];
        floatx4& A0 = (b & 1) ? a_o : a;
        floatx4& A1 = (b & 1) ? ad_o : ad;
        A0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(w1h[b], s0, A0, 0, 0, 0);
        A1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(w1h[b], s1, A1, 0, 0, 0);
        A0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(w1h[b], l0, A0, 0, 0, 0);
        A1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(w1h[b], l1, A1, 0, 0, 0);
        A0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(w1l[b], h0, A0, 0, 0, 0);
        A1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(w1l[b], h1, A1, 0, 0, 0);
      }
      a = (a + a_o) * (1.0f / (kS4 * kBetaG0));
      ad = (ad + ad_o) * (1.0f / (kS4 * kBetaG1));
    } else {
#pragma unroll
      for (int s = 0; s < KSMAX; ++s) {
        const int o = oG1[s & 1] + 64 * s;  // rp_at(4s + q, n)
        const float g = GT[o];
        const float gd = GT[kRows * 16 + o];
        if (s & 1) {
          a_o = __builtin_amdgcn_mfma_f32_16x16x4f32(w1f[s], g, a_o, 0, 0, 0);
          ad_o = __builtin_amdgcn_mfma_f32_16x16x4f32(w1f[s], gd, ad_o, 0, 0, 0);
        } else {
          a = __builtin_amdgcn_mfma_f32_16x16x4f32(w1f[s], g, a, 0, 0, 0);
          ad = __builtin_amdgcn_mfma_f32_16x16x4f32(w1f[s], gd, ad, 0, 0, 0);
        }
      }
      a += a_o;
      ad += ad_o;
    }
    // 2. h, h', activation derivatives; publish t, t', h, h'
    float act1[4], act2[4];
    float hv[4], hdv[4];
    const float* tb = tbv;
    const float* tdb = tdbv;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float sv, d1, d2;
      act_any<ACT>(rp.act, a[i] + bias[i], sv, d1, d2);
      act1[i] = d1;
      act2[i] = d2 * ad[i];
      hv[i] = sv;
      hdv[i] = d1 * ad[i];
    }
    if constexpr (kX3) {
      // h, h' enter step 4 as fp16 planes of h beta_h: past 2^19 they leave
      // the planes' range -- report it (rare; the result is not repaired)
      // (written so that a NaN counts as out of range)
      bool out = false;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        out = out || !(fabsf(hv[i]) < 524288.0f) || !(fabsf(hdv[i]) < 524288.0f);
      if (out) raise_numerics_flag(kFlagBwdRange);
    }
    if constexpr (kX3) {
      // h beta, h' beta as two fp16 planes (hi, lo S4) of [2][128 rows][16
      // pairs]; row 4q + i of a 16-row block stored at 4q + (i ^ q)
      _Float16* HTh = reinterpret_cast<_Float16*>(HT);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int o = (16 * w + 4 * q + (i ^ q)) * 16 + n;
        halfx2 sh, sl;
        split2x2(hv[i] * kBetaH, hdv[i] * kBetaH, kS4, sh, sl);
        HTh[o] = sh[0];
        HTh[kF * 16 + o] = sh[1];
        HTh[2 * kF * 16 + o] = sl[0];
        HTh[3 * kF * 16 + o] = sl[1];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        HT[oW[i]] = hv[i];
        HT[kF * 16 + oW[i]] = hdv[i];
      }
    }
    float inv_t = 1.0f, inv_td = 1.0f;  // x3: 1 / (S sigma) of the lane's pair
    if constexpr (kX3) {
      const float m0 = __uint_as_float(PMAXu[buf * 32 + n]);
      const float m1 = __uint_as_float(PMAXu[buf * 32 + 16 + n]);
      // the other buffer collects the next tile's maxima (phase 5, after the
      // barrier below); its last reader was phase 2 of the previous tile
      if (w == 0 && l < 32) PMAXu[(buf ^ 1) * 32 + l] = 0u;
      const float sg0 = x3_norm(m0), sg1 = x3_norm(m1);
      inv_t = x3_norm_inv(m0) * inv_S;
      inv_td = x3_norm_inv(m1) * inv_S;
      // two planes (hi, lo S) of t sigma (step 3 scales W2's hi plane by S
      // instead of reading a third, hi S plane); 16-byte chunk g of pair n's
      // row (8 halfs) at g ^ tb_swz(n)
      _Float16* TBh = reinterpret_cast<_Float16*>(TB);
      const int o = n * kF + 8 * ((2 * w + (q >> 1)) ^ tb_swz(n)) + 4 * (q & 1);
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const float sg = st ? sg1 : sg0;
        const float* src = st ? tdb : tb;
        halfx4 ph, pl;
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
          halfx2 sh, sl;
          split2x2(src[i] * sg, src[i + 1] * sg, S, sh, sl);
          ph[i] = sh[0];
          ph[i + 1] = sh[1];
          pl[i] = sl[0];
          pl[i + 1] = sl[1];
        }
        *reinterpret_cast<halfx4*>(TBh + (0 * 2 + st) * 16 * kF + o) = ph;
        *reinterpret_cast<halfx4*>(TBh + (1 * 2 + st) * 16 * kF + o) = pl;
      }
    } else {
      *reinterpret_cast<float4*>(TB + oTBw) = f4(tb[0], tb[1], tb[2], tb[3]);
      *reinterpret_cast<float4*>(TB + 16 * kF + oTBw) = f4(tdb[0], tdb[1], tdb[2], tdb[3]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      TT[oW[i]] = tb[i];
      TT[kF * 16 + oW[i]] = tdb[i];
    }
    __syncthreads();

    // 3. hb, hb' of feature tile w (all 128 t features from LDS)
    floatx4 hb = {0.f, 0.f, 0.f, 0.f}, hdb = {0.f, 0.f, 0.f, 0.f};
    floatx4 hb_o = {0.f, 0.f, 0.f, 0.f}, hdb_o = {0.f, 0.f, 0.f, 0.f};
    if constexpr (kX3) {
      // S sigma W2^T t in 4 k blocks of 32 features, three fp16 MFMAs each
      const halfx8* w2hv = reinterpret_cast<const halfx8*>(w2ts);
      const halfx8* tbh = reinterpret_cast<const halfx8*>(TB);
#pragma unroll
      for (int sb = 0; sb < 4; ++sb) {
        const int oa = (w * 4 + sb) * MLCG_WAVE + l;
        const halfx8 ah = w2hv[oa], al = w2hv[kF * kF / 8 + oa];
        // hi_A S in fp16: exact (S a power of two, |W2| S < 2^14)
        const halfx8 ahs = ah * (_Float16)S;
        const int ob = (n * kF + 8 * ((4 * sb + q) ^ tb_swz(n))) / 8;
        constexpr int kP = 16 * kF / 8;  // halfx8 per (plane, stream)
        // planes of t: (hi, lo S) at (0, 2) kP, of t' at (1, 3) kP;
        // S sigma A t ~ (hi_A S) hi_t + hi_A (lo_t S) + (lo_A S) hi_t, the
        // first product equal to hi_A (hi_t S) bit for bit
        const halfx8 t0h = tbh[ob], t0l = tbh[2 * kP + ob];
        const halfx8 t1h = tbh[kP + ob], t1l = tbh[3 * kP + ob];
        hb = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahs, t0h, hb, 0, 0, 0);
        hdb = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahs, t1h, hdb, 0, 0, 0);
        hb = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, t0l, hb, 0, 0, 0);
        hdb = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, t1l, hdb, 0, 0, 0);
        hb = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, t0h, hb, 0, 0, 0);
        hdb = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, t1h, hdb, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        hb[i] *= inv_t;
        hdb[i] *= inv_td;
      }
    } else {
#pragma unroll
    for (int u = 0; u < kFT; ++u) {
      const float4 a2 = w2v[u * MLCG_WAVE];
      const int o = oTB3[u & 1] + 32 * (u >> 1);  // tb_at(n, 4u + q)
      const float4 bx = *reinterpret_cast<const float4*>(TB + o);
      const float4 by = *reinterpret_cast<const float4*>(TB + 16 * kF + o);
      hb = __builtin_amdgcn_mfma_f32_16x16x4f32(a2.x, bx.x, hb, 0, 0, 0);
      hdb = __builtin_amdgcn_mfma_f32_16x16x4f32(a2.x, by.x, hdb, 0, 0, 0);
      hb_o = __builtin_amdgcn_mfma_f32_16x16x4f32(a2.y, bx.y, hb_o, 0, 0, 0);
      hdb_o = __builtin_amdgcn_mfma_f32_16x16x4f32(a2.y, by.y, hdb_o, 0, 0, 0);
      hb = __builtin_amdgcn_mfma_f32_16x16x4f32(a2.z, bx.z, hb, 0, 0, 0);
      hdb = __builtin_amdgcn_mfma_f32_16x16x4f32(a2.z, by.z, hdb, 0, 0, 0);
      hb_o = __builtin_amdgcn_mfma_f32_16x16x4f32(a2.w, bx.w, hb_o, 0, 0, 0);
      hdb_o = __builtin_amdgcn_mfma_f32_16x16x4f32(a2.w, by.w, hdb_o, 0, 0, 0);
    }
    hb += hb_o;
    hdb += hdb_o;
    }
    // the next tile's pair adjoints from its node vectors (requested at the
    // start of this tile), early so that their registers are free for step 4
    const float vm_nxt = (tile + stride) * 16 + n < np ? 1.0f : 0.0f;
    float4 wb_nxt, wdb_nxt;
    tile_adjoint<kNodes>(nxt, tangent, has_yd, vm_nxt, wb_nxt, wdb_nxt);
    float abv[4], adbv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      abv[i] = hb[i] * act1[i] + hdb[i] * act2[i];
      adbv[i] = hdb[i] * act1[i];
      db[i] += abv[i];
    }
    float amax_tile = 0.f;  // split path: max |ab|, |ab'| over the wave
    if constexpr (kX3) {
      float mx = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = fmaxf(mx, fmaxf(fabsf(abv[i]), fabsf(adbv[i])));
      mx = cross_row_max(row16_max(mx));
      amax_tile = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(mx)));
    }
    // 4. dW2[16w + m][16u + c] += sum_pairs t[pair][16w + m] h[pair][16u + c]
    if constexpr (kX3) {
      // fp16 MFMA, k = 32 = (stream, pair): lane group q holds stream q >> 1,
      // pairs 8 (q & 1) .. + 7.  A = t rw split when read, B = h beta
      if (tmax_tile > trun) {  // wave-uniform; the running scale only shrinks
        const float rn =
            __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x3_norm(tmax_tile))));
        const float f = rn / rw;
#pragma unroll
        for (int u = 0; u < kFT; ++u) acc2[u] *= f;
        rw = rn;
        trun = tmax_tile;
      }
      const int oA4 = (q >> 1) * kF * 16;
      const int oB4 = (q >> 1) * 2 * kF + 2 * (n ^ (n >> 2)) + (q & 1);
      const float4 x0 = *reinterpret_cast<const float4*>(TT + oA4 + tt_at(16 * w + n, 8 * (q & 1)));
      const float4 x1 =
          *reinterpret_cast<const float4*>(TT + oA4 + tt_at(16 * w + n, 8 * (q & 1) + 4));
      const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      halfx8 ah, al;
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        halfx2 sh, sl;
        split2x2(xv[j] * rw, xv[j + 1] * rw, kS4, sh, sl);
        ah[j] = sh[0];
        ah[j + 1] = sh[1];
        al[j] = sl[0];
        al[j + 1] = sl[1];
      }
      // hi S4 in fp16: exact (a power of two; |hi| < 4), packed multiplies
      const halfx8 ahs = ah * (_Float16)kS4;
      const halfx8* hth = reinterpret_cast<const halfx8*>(HT);
#pragma unroll
      for (int u = 0; u < kFT; ++u) {
        const halfx8 bh = hth[oB4 + 32 * u], bl = hth[oB4 + 2 * kF * 16 / 8 + 32 * u];
        acc2[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahs, bh, acc2[u], 0, 0, 0);
        acc2[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, acc2[u], 0, 0, 0);
        acc2[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, acc2[u], 0, 0, 0);
      }
    } else {
    //    MFMA step kk of lane group q reduces over pair 4q + kk
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const float* T = TT + st * kF * 16;
      const float* H = HT + st * kF * 16;
      const float4 av = *reinterpret_cast<const float4*>(T + oRw);
#pragma unroll
      for (int u = 0; u < kFT; ++u) {
        const float4 bv = *reinterpret_cast<const float4*>(H + oR + 256 * u);
        acc2[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.x, bv.x, acc2[u], 0, 0, 0);
        acc2[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.y, bv.y, acc2[u], 0, 0, 0);
        acc2[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.z, bv.z, acc2[u], 0, 0, 0);
        acc2[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.w, bv.w, acc2[u], 0, 0, 0);
      }
    }
    }
    // the next tile's basis, envelope and pair adjoints t, t': independent of
    // step 4, so their arithmetic can issue among its MFMAs
    const BasisV bv = basis_eval(nxt);
    cc_cur = bv.cc;
    dcc_cur = bv.dcc;
    float pm0, pm1;
    pair_adjoints_eval(wb_nxt, wdb_nxt, cc_cur, dcc_cur, pm0, pm1);
    if constexpr (kX3) {
      // scheduling hint for the region above: the operand loads and splits
      // first, then each MFMA of step 4 followed by a few of the independent
      // VALU instructions of the next tile's basis
      __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);  // DS reads
      __builtin_amdgcn_sched_group_barrier(0x002, 24, 0);  // VALU
#pragma unroll
      for (int i = 0; i < 3 * kFT; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
      }
    }
    // 5. publish ab, ab' (and store them per pair when the basis parameters
    //    need gradients) and the next tile's basis
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      AT[oW[i]] = abv[i];
      AT[kF * 16 + oW[i]] = adbv[i];
    }
    if (abar_out && vmask != 0.0f) {
      const int64_t p = tile * 16 + n;
      *reinterpret_cast<float4*>(abar_out + p * kF + fcol) = f4(abv[0], abv[1], abv[2], abv[3]);
      *reinterpret_cast<float4*>(adbar_out + p * kF + fcol) =
          f4(adbv[0], adbv[1], adbv[2], adbv[3]);
    }
    basis_store(bv, buf ^ 1);
    pair_adjoints_store(pm0, pm1, buf ^ 1);
    __syncthreads();
    // 6. dW1[16w + m][k] += sum_pairs ab[pair][16w + m] g[pair][k]
    if constexpr (kX3) {
      // as step 4: A = ab ra split when read (ra = 2^k, |ab| ra < 4 over every
      // tile seen so far), B = the two planes of g
      if (amax_tile > arun) {  // wave-uniform; the running scale only shrinks
        const float rn =
            __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x3_norm(amax_tile))));
        const float f = rn / ra;
#pragma unroll
        for (int kt = 0; kt < KTMAX; ++kt) acc1[kt] *= f;
        ra = rn;
        arun = amax_tile;
      }
      const int oA6 = (q >> 1) * kF * 16;
      const float4 x0 = *reinterpret_cast<const float4*>(AT + oA6 + tt_at(16 * w + n, 8 * (q & 1)));
      const float4 x1 =
          *reinterpret_cast<const float4*>(AT + oA6 + tt_at(16 * w + n, 8 * (q & 1) + 4));
      const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      halfx8 ah, al;
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        halfx2 sh, sl;
        split2x2(xv[j] * ra, xv[j + 1] * ra, kS4, sh, sl);
        ah[j] = sh[0];
        ah[j + 1] = sh[1];
        al[j] = sl[0];
        al[j + 1] = sl[1];
      }
      // hi S4 in fp16: exact (a power of two; |hi| < 4), packed multiplies
      const halfx8 ahs = ah * (_Float16)kS4;
      // B: halfx8 of plane rows 16kt + n, stream q >> 1, pairs 8 (q & 1) .. + 7
      const halfx8* gth = reinterpret_cast<const halfx8*>(GT);
      const int oB6 = (q >> 1) * 2 * kRows + 2 * n + (q & 1);
#pragma unroll
      for (int kt = 0; kt < KTMAX; ++kt) {
        const halfx8 bh = gth[oB6 + 32 * kt], bl = gth[oB6 + 2 * kRows * 16 / 8 + 32 * kt];
        acc1[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahs, bh, acc1[kt], 0, 0, 0);
        acc1[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, acc1[kt], 0, 0, 0);
        acc1[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, acc1[kt], 0, 0, 0);
      }
    } else {
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const float* A = AT + st * kF * 16;
      const float* G = GT + st * kRows * 16;
      const float4 av = *reinterpret_cast<const float4*>(A + oRw);
#pragma unroll
      for (int kt = 0; kt < KTMAX; ++kt) {
        const float4 bv = *reinterpret_cast<const float4*>(G + oR + 256 * kt);
        acc1[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.x, bv.x, acc1[kt], 0, 0, 0);
        acc1[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.y, bv.y, acc1[kt], 0, 0, 0);
        acc1[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.z, bv.z, acc1[kt], 0, 0, 0);
        acc1[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.w, bv.w, acc1[kt], 0, 0, 0);
      }
    }
    }
  }

  if constexpr (kX3) {
    const float f = 1.0f / (kS4 * rw * kBetaH);
#pragma unroll
    for (int u = 0; u < kFT; ++u) acc2[u] *= f;
    const float f1 = 1.0f / (kS4 * ra);
#pragma unroll
    for (int kt = 0; kt < KTMAX; ++kt) acc1[kt] *= f1;
  }
  // partial sums of this workgroup: [dW2 (F x F) | dW1 (F x Kp16) | db1 (F)]
  float* out = partial + (int64_t)blockIdx.x * bwd_partial_floats(K);
#pragma unroll
  for (int u = 0; u < kFT; ++u)
#pragma unroll
    for (int r = 0; r < 4; ++r) out[(16 * w + 4 * q + r) * kF + 16 * u + n] = acc2[u][r];
  float* o1 = out + kF * kF;
#pragma unroll
  for (int kt = 0; kt < KTMAX; ++kt)
    if (kt < KT)
#pragma unroll
      for (int r = 0; r < 4; ++r) o1[(16 * w + 4 * q + r) * Kp16 + 16 * kt + n] = acc1[kt][r];
  // db1: sum the 16 pair lanes that share q (fixed butterfly order)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float v = db[i];
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) v += __shfl_xor(v, o, MLCG_WAVE);
    db[i] = v;
  }
  if (n == 0) {
    float* o2 = o1 + kF * Kp16;
#pragma unroll
    for (int i = 0; i < 4; ++i) o2[16 * w + 4 * q + i] = db[i];
  }
}

// dW2 [F, F], dW1 [F, K], db1 [F] = sum over the workgroup partials.  A block
// handles 64 outputs; its 4 waves take the groups g = slice (mod 4), each lane
// keeping 4 interleaved accumulators, and the partial sums are combined in a
// fixed order, so the result does not depend on timing.
constexpr int kRedOut = 64;

__global__ __launch_bounds__(256) void filter_bwd_reduce_kernel(
    const float* __restrict__ partial, int groups, int K, float* __restrict__ dW1,
    float* __restrict__ db1, float* __restrict__ dW2) {
  __shared__ float part[4][kRedOut];
  const int Kp16 = bwd_kp16(K);
  const int stride = bwd_partial_floats(K);
  const int total = kF * kF + kF * K + kF;
  const int o = threadIdx.x & (kRedOut - 1);
  const int slice = threadIdx.x / kRedOut;
  const int j = blockIdx.x * kRedOut + o;
  int src = 0;
  float* dst = nullptr;
  if (j < kF * kF) {
    src = j;
    dst = dW2 + j;
  } else if (j < kF * kF + kF * K) {
    const int r = j - kF * kF;
    src = kF * kF + (r / K) * Kp16 + (r % K);
    dst = dW1 + r;
  } else if (j < total) {
    const int r = j - kF * kF - kF * K;
    src = kF * kF + kF * Kp16 + r;
    dst = db1 + r;
  }
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if (dst) {
    int g = slice;
    for (; g + 12 < groups; g += 16) {
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[u] += partial[(int64_t)(g + 4 * u) * stride + src];
    }
    for (int u = 0; g < groups; g += 4, ++u) acc[u & 3] += partial[(int64_t)g * stride + src];
  }
  part[slice][o] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  __syncthreads();
  if (slice == 0 && dst) *dst = (part[0][o] + part[1][o]) + (part[2][o] + part[3][o]);
}

int bwd_groups(int64_t max_pairs) {
  const int64_t tiles = (max_pairs + 15) / 16;
  return (int)(tiles < 256 ? (tiles < 1 ? 1 : tiles) : 256);
}

// Kernels here use more than 64 KiB of dynamic LDS; raise their limit to the
// 160 KiB of a gfx950 CU once per device (not per launch, so launches inside
// a stream capture make no extra runtime calls).
void allow_lds_once() {
  static bool done[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64 || done[dev]) return;
  const int bytes = 160 * 1024;
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(filter_fwd_f32_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(filter_fwd_x3_kernel<0, 0>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(filter_fwd_x3_kernel<0, 1>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(filter_fwd_x3_kernel<1, 0>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(filter_fwd_x3_kernel<1, 1>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  const void* f16[] = {
      reinterpret_cast<const void*>(filter_fwd_f16_kernel<2, 0, 0>),
      reinterpret_cast<const void*>(filter_fwd_f16_kernel<2, 0, 1>),
      reinterpret_cast<const void*>(filter_fwd_f16_kernel<2, 1, 0>),
      reinterpret_cast<const void*>(filter_fwd_f16_kernel<2, 1, 1>),
      reinterpret_cast<const void*>(filter_fwd_f16_kernel<4, 0, 0>),
      reinterpret_cast<const void*>(filter_fwd_f16_kernel<4, 0, 1>),
      reinterpret_cast<const void*>(filter_fwd_f16_kernel<4, 1, 0>),
      reinterpret_cast<const void*>(filter_fwd_f16_kernel<4, 1, 1>)};
  for (const void* f : f16)
    (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  const void* bwd[] = {
      reinterpret_cast<const void*>(filter_bwd_fused_kernel<16, false, 0, 0>),
      reinterpret_cast<const void*>(filter_bwd_fused_kernel<16, false, 0, 1>),
      reinterpret_cast<const void*>(filter_bwd_fused_kernel<16, false, 1, 0>),
      reinterpret_cast<const void*>(filter_bwd_fused_kernel<16, false, 1, 1>),
      reinterpret_cast<const void*>(filter_bwd_fused_kernel<16, true, 0, 0>),
      reinterpret_cast<const void*>(filter_bwd_fused_kernel<16, true, 0, 1>),
      reinterpret_cast<const void*>(filter_bwd_fused_kernel<16, true, 1, 0>),
      reinterpret_cast<const void*>(filter_bwd_fused_kernel<16, true, 1, 1>),
      reinterpret_cast<const void*>(filter_bwd_fused_kernel<32, false, -1, -1>),
      reinterpret_cast<const void*>(filter_bwd_fused_kernel<32, true, -1, -1>)};
  for (const void* f : bwd)
    (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  done[dev] = true;
}

RbfParams make_params(int basis, const float* centers, const float* widths, float alpha, int K,
                      int rk, float rlo, float rhi, int ck, float clo, float chi, int act) {
  RbfParams rp;
  rp.basis = basis;
  rp.centers = centers;
  rp.widths = widths;
  rp.alpha = alpha;
  rp.K = K;
  rp.rbf_kind = rk;
  rp.rbf_lo = rlo;
  rp.rbf_hi = rhi;
  rp.conv_kind = ck;
  rp.conv_lo = clo;
  rp.conv_hi = chi;
  rp.act = act;
  rp.same_cut = rk == ck && rlo == clo && rhi == chi;
  rp.rcut = make_cut(rk, rlo, rhi);
  rp.ccut = make_cut(ck, clo, chi);
  return rp;
}

bool valid_params(int basis, int K, int rk, int ck, int act, int F) {
  return F == kF && K >= 1 && K <= kMaxK && (basis == 0 || basis == 1) && (rk == 0 || rk == 1) &&
         (ck == 0 || ck == 1) && (act == 0 || act == 1);
}

}  // namespace

// Device address of the numerics flag word on the current device (looked up
// once per device with hipGetSymbolAddress; nullptr on failure), for the
// kernels of other translation units that raise its bits.
unsigned* mlcg_numerics_word_ptr() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kFlagDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_flag_mutex);
  if (g_flag_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(mlcg_numerics_word)) != hipSuccess || p == nullptr)
      return nullptr;
    g_flag_ptr[dev] = static_cast<unsigned*>(p);
  }
  return g_flag_ptr[dev];
}

extern "C" int mlcg_numerics_flags(int* out, int clear, void* stream) {
  MLCG_REQUIRE(out != nullptr);
  hipLaunchKernelGGL(numerics_flags_kernel, dim3(1), dim3(64), 0, mlcg_stream(stream), out,
                     clear);
  return mlcg_launch_status();
}

extern "C" int mlcg_filter_fwd(const float* pos, const int32_t* pair_ij, int64_t pair_stride,
                               const int32_t* n_pairs_dev, int64_t max_pairs, int basis,
                               const float* centers, const float* widths, float alpha,
                               int num_rbf, int rbf_cut_kind, float rbf_lo, float rbf_hi,
                               int conv_cut_kind, float conv_lo, float conv_hi, int act,
                               const float* W1, const float* b1, const float* W2,
                               int num_filters, int f16, void* W_out, void* Wd_out,
                               float* dist_out, void* stream) {
  if (!valid_params(basis, num_rbf, rbf_cut_kind, conv_cut_kind, act, num_filters))
    return MLCG_ERR_UNSUPPORTED;
  MLCG_REQUIRE(max_pairs >= 0 && pair_stride >= max_pairs);
  if (max_pairs == 0) return MLCG_OK;
  MLCG_REQUIRE(pos && pair_ij && n_pairs_dev && centers && widths && W1 && b1 && W2 && W_out &&
               Wd_out);
  RbfParams rp = make_params(basis, centers, widths, alpha, num_rbf, rbf_cut_kind, rbf_lo,
                             rbf_hi, conv_cut_kind, conv_lo, conv_hi, act);
  const unsigned groups = mlcg_persistent_groups(mlcg_div_up(max_pairs, 16 * kWaves), 1);
  hipStream_t s = mlcg_stream(stream);
  MLCG_REQUIRE(f16 == MLCG_FILTER_FP32 || f16 == MLCG_FILTER_FP16 ||
               f16 == MLCG_FILTER_FP32_STRICT);
  if (f16 == MLCG_FILTER_FP32 && MLCG_FILTER_FWD_X3 &&
      fwd_x3_lds_bytes(num_rbf) <= 160 * 1024) {  // K <= 64
    const size_t lds = fwd_x3_lds_bytes(num_rbf);
    allow_lds_once();
    const unsigned gx = mlcg_persistent_groups(mlcg_div_up(max_pairs, 16 * kWavesX3), 1);
#define MLCG_X3_LAUNCH(B, A)                                                               \
  hipLaunchKernelGGL((filter_fwd_x3_kernel<B, A>), dim3(gx), dim3(kThreadsX3), lds, s, pos,  \
                     pair_ij, pair_ij + pair_stride, n_pairs_dev, max_pairs, rp, W1, b1, W2, \
                     static_cast<float*>(W_out), static_cast<float*>(Wd_out), dist_out)
    if (basis == 0 && act == 0) MLCG_X3_LAUNCH(0, 0);
    else if (basis == 0) MLCG_X3_LAUNCH(0, 1);
    else if (act == 0) MLCG_X3_LAUNCH(1, 0);
    else MLCG_X3_LAUNCH(1, 1);
#undef MLCG_X3_LAUNCH
  } else if (f16 != MLCG_FILTER_FP16) {
    const int KS = (num_rbf + 3) / 4;
    const size_t lds =
        sizeof(float) * (kFT * KS * MLCG_WAVE + kFT * kFT * MLCG_WAVE * 4 + 2 * kMaxK);
    allow_lds_once();
    hipLaunchKernelGGL(filter_fwd_f32_kernel, dim3(groups), dim3(kThreads), lds, s, pos,
                       pair_ij, pair_ij + pair_stride, n_pairs_dev, max_pairs, rp, W1, b1, W2,
                       static_cast<float*>(W_out), static_cast<float*>(Wd_out), dist_out);
  } else {
    // K padded to 64 or 128 (two or four 32-wide k blocks)
    const int KS32 = num_rbf <= 64 ? 2 : 4;
    const size_t lds =
        sizeof(_Float16) * (kFT * KS32 * MLCG_WAVE * 8 + kFT * (kFT / 2) * MLCG_WAVE * 8) +
        sizeof(float) * (kF + 2 * kMaxK);
    allow_lds_once();
    const unsigned groups16 =
        mlcg_persistent_groups(mlcg_div_up(max_pairs, 16 * kWaves16), MLCG_F16_GROUPS_PER_CU);
#define MLCG_F16_LAUNCH(KB, B, A)                                                             \
  hipLaunchKernelGGL((filter_fwd_f16_kernel<KB, B, A>), dim3(groups16), dim3(kThreads16), lds, \
                     s, pos, pair_ij, pair_ij + pair_stride, n_pairs_dev, max_pairs, rp, W1,   \
                     b1, W2, static_cast<__half*>(W_out), static_cast<__half*>(Wd_out),       \
                     dist_out)
#define MLCG_F16_KB(KB)                                       \
  if (basis == 0 && act == 0) MLCG_F16_LAUNCH(KB, 0, 0);      \
  else if (basis == 0) MLCG_F16_LAUNCH(KB, 0, 1);             \
  else if (act == 0) MLCG_F16_LAUNCH(KB, 1, 0);               \
  else MLCG_F16_LAUNCH(KB, 1, 1)
    if (KS32 == 2) {
      MLCG_F16_KB(2);
    } else {
      MLCG_F16_KB(4);
    }
#undef MLCG_F16_KB
#undef MLCG_F16_LAUNCH
  }
  return mlcg_launch_status();
}

extern "C" int64_t mlcg_filter_bwd_workspace_floats(int64_t max_pairs, int num_rbf) {
  if (max_pairs < 0 || num_rbf < 1 || num_rbf > kMaxK) return -1;
  return (int64_t)bwd_groups(max_pairs) * bwd_partial_floats(num_rbf);
}

namespace {

int launch_filter_bwd(const float* pos, const int32_t* pair_ij, int64_t pair_stride,
                      const int32_t* n_pairs_dev, int64_t max_pairs, int basis,
                      const float* centers, const float* widths, float alpha, int num_rbf,
                      int rbf_cut_kind, float rbf_lo, float rbf_hi, int conv_cut_kind,
                      float conv_lo, float conv_hi, int act, const float* W1, const float* b1,
                      const float* W2, int num_filters, const PairAdjoint& adj, bool nodes,
                      float* dW1, float* db1, float* dW2, float* abar_out, float* adbar_out,
                      float* workspace, int64_t workspace_floats, bool fp32_strict,
                      void* stream) {
  if (!valid_params(basis, num_rbf, rbf_cut_kind, conv_cut_kind, act, num_filters))
    return MLCG_ERR_UNSUPPORTED;
  MLCG_REQUIRE(max_pairs >= 0 && pair_stride >= max_pairs);
  MLCG_REQUIRE(centers && widths && W1 && b1 && W2 && dW1 && db1 && dW2 && workspace);
  MLCG_REQUIRE(max_pairs == 0 || (pos && pair_ij && n_pairs_dev));
  MLCG_REQUIRE((abar_out == nullptr) == (adbar_out == nullptr));
  const int groups = bwd_groups(max_pairs);
  MLCG_REQUIRE(workspace_floats >= (int64_t)groups * bwd_partial_floats(num_rbf));
  RbfParams rp = make_params(basis, centers, widths, alpha, num_rbf, rbf_cut_kind, rbf_lo,
                             rbf_hi, conv_cut_kind, conv_lo, conv_hi, act);
  hipStream_t s = mlcg_stream(stream);
  // the split (fp16 MFMA) form serves K <= 64 unless fp32 products are asked
  // for; the fp32 form (KS = 32, rows up to 128) uses the wide LDS layout
  const bool small_k = num_rbf <= 64 && !fp32_strict;
  const size_t lds = sizeof(float) * bwd_lds_floats(small_k ? num_rbf : kMaxK);
  allow_lds_once();
  const int grid = max_pairs == 0 ? 1 : groups;
#define MLCG_BWD_LAUNCH(KS, NODES, B, A)                                                      \
  hipLaunchKernelGGL((filter_bwd_fused_kernel<KS, NODES, B, A>), dim3(grid),                 \
                     dim3(kBwdThreads), lds, s, pos, pair_ij, pair_ij + pair_stride,         \
                     n_pairs_dev, max_pairs, rp, W1, b1, W2, adj, abar_out, adbar_out,       \
                     workspace)
#define MLCG_BWD_SMALL(NODES)                                   \
  if (basis == 0 && act == 0) MLCG_BWD_LAUNCH(16, NODES, 0, 0); \
  else if (basis == 0) MLCG_BWD_LAUNCH(16, NODES, 0, 1);        \
  else if (act == 0) MLCG_BWD_LAUNCH(16, NODES, 1, 0);          \
  else MLCG_BWD_LAUNCH(16, NODES, 1, 1)
  if (small_k && !nodes) {
    MLCG_BWD_SMALL(false);
  } else if (small_k) {
    MLCG_BWD_SMALL(true);
  } else if (!nodes) {
    MLCG_BWD_LAUNCH(32, false, -1, -1);
  } else {
    MLCG_BWD_LAUNCH(32, true, -1, -1);
  }
#undef MLCG_BWD_SMALL
#undef MLCG_BWD_LAUNCH
  const int total = kF * kF + kF * num_rbf + kF;
  hipLaunchKernelGGL(filter_bwd_reduce_kernel, dim3((total + kRedOut - 1) / kRedOut), dim3(256),
                     0, s, workspace, groups, num_rbf, dW1, db1, dW2);
  return mlcg_launch_status();
}

}  // namespace

extern "C" int mlcg_filter_bwd(const float* pos, const int32_t* pair_ij, int64_t pair_stride,
                               const int32_t* n_pairs_dev, int64_t max_pairs, int basis,
                               const float* centers, const float* widths, float alpha,
                               int num_rbf, int rbf_cut_kind, float rbf_lo, float rbf_hi,
                               int conv_cut_kind, float conv_lo, float conv_hi, int act,
                               const float* W1, const float* b1, const float* W2,
                               int num_filters, const float* Wbar, const float* Wdbar,
                               float* dW1, float* db1, float* dW2, float* abar_out,
                               float* adbar_out, float* workspace, int64_t workspace_floats,
                               int fp32_strict, void* stream) {
  MLCG_REQUIRE(max_pairs == 0 || (Wbar && Wdbar));
  PairAdjoint adj{Wbar, Wdbar, nullptr, nullptr, nullptr, nullptr, nullptr};
  return launch_filter_bwd(pos, pair_ij, pair_stride, n_pairs_dev, max_pairs, basis, centers,
                           widths, alpha, num_rbf, rbf_cut_kind, rbf_lo, rbf_hi, conv_cut_kind,
                           conv_lo, conv_hi, act, W1, b1, W2, num_filters, adj, false, dW1, db1,
                           dW2, abar_out, adbar_out, workspace, workspace_floats,
                           fp32_strict != 0, stream);
}

extern "C" int mlcg_filter_bwd_cfconv(const float* pos, const int32_t* pair_ij,
                                      int64_t pair_stride, const int32_t* n_pairs_dev,
                                      int64_t max_pairs, int basis, const float* centers,
                                      const float* widths, float alpha, int num_rbf,
                                      int rbf_cut_kind, float rbf_lo, float rbf_hi,
                                      int conv_cut_kind, float conv_lo, float conv_hi, int act,
                                      const float* W1, const float* b1, const float* W2,
                                      int num_filters, const float* gagg2, const float* y,
                                      const float* gagg1, const float* ydot,
                                      const float* ddot, float* dW1, float* db1, float* dW2,
                                      float* abar_out, float* adbar_out, float* workspace,
                                      int64_t workspace_floats, int fp32_strict, void* stream) {
  MLCG_REQUIRE(max_pairs == 0 || (gagg2 && y));
  MLCG_REQUIRE(!gagg1 || ddot);
  PairAdjoint adj{nullptr, nullptr, gagg2, y, gagg1, gagg1 ? ydot : nullptr, ddot};
  return launch_filter_bwd(pos, pair_ij, pair_stride, n_pairs_dev, max_pairs, basis, centers,
                           widths, alpha, num_rbf, rbf_cut_kind, rbf_lo, rbf_hi, conv_cut_kind,
                           conv_lo, conv_hi, act, W1, b1, W2, num_filters, adj, true, dW1, db1,
                           dW2, abar_out, adbar_out, workspace, workspace_floats,
                           fp32_strict != 0, stream);
}

// ---------------------------------------------------------------------------
// Gradients of trainable basis parameters.
//
// With the pair adjoints of the first filter layer, abar = dL/da and
// adbar = dL/da' (a = W1 g + b1, a' = W1 g'), the basis adjoints are
// gbar = W1^T abar and gdbar = W1^T adbar, and per basis function k
//   dcenters[k] += sum_p gbar_pk dg_pk/dcenter_k + gdbar_pk dg'_pk/dcenter_k
//   dwidths[k]  += sum_p gbar_pk dg_pk/dwidth_k  + gdbar_pk dg'_pk/dwidth_k
// (for the Gaussian basis dwidths[k] is the share of basis function k in
// d/dcoeff).  One wave per 16-pair tile computes gbar, gdbar with
// v_mfma_f32_16x16x4f32 (A = the pair adjoints, B = W1 from LDS), the
// derivative factors per (pair, k), and keeps per-lane sums; the
// workgroup partials are added in a fixed order by rbf_grad_reduce_kernel.
namespace {

constexpr int kRgWaves = 4;
constexpr int kRgThreads = kRgWaves * MLCG_WAVE;
constexpr int kRgMaxGroups = 512;

__device__ __forceinline__ void basis_param_derivs(const RbfParams& rp, float cen, float wid,
                                                   float d, float C, float dC, float& g_c,
                                                   float& g_w, float& gd_c, float& gd_w) {
  if (rp.basis == 0) {
    const float c = wid;
    const float x = d - cen;
    const float e = __expf(c * x * x);
    const float q = 2.0f * c * x * C + dC;            // g' = e q
    g_c = -2.0f * c * x * C * e;                       // dg/dcenter
    g_w = x * x * C * e;                               // dg/dc
    gd_c = -e * (2.0f * c * x * q + 2.0f * c * C);     // dg'/dcenter
    gd_w = e * (x * x * q + 2.0f * x * C);             // dg'/dc
  } else {
    const float ex = __expf(rp.alpha * (rp.rbf_lo - d));
    const float u = ex - cen;
    const float b = wid;
    const float e = __expf(-b * u * u);
    const float r = dC + 2.0f * rp.alpha * b * u * ex * C;  // g' = e r
    g_c = 2.0f * b * u * C * e;
    g_w = -u * u * C * e;
    gd_c = e * (2.0f * b * u * r - 2.0f * rp.alpha * b * ex * C);
    gd_w = e * (-u * u * r + 2.0f * rp.alpha * u * ex * C);
  }
}

template <int KT>
__global__ __launch_bounds__(kRgThreads) void rbf_grad_kernel(
    const float* __restrict__ dist, const int32_t* __restrict__ n_pairs_dev, int64_t max_pairs,
    RbfParams rp, const float* __restrict__ W1, const float* __restrict__ abar,
    const float* __restrict__ adbar, float* __restrict__ partial) {
  __shared__ float w1s[kF * (16 * KT + 1)];  // W1 as [f][k], zero past K
  const int K = rp.K;
  const int kr = 16 * KT + 1;
  for (int x = threadIdx.x; x < kF * 16 * KT; x += blockDim.x) {
    const int f = x / (16 * KT), k = x % (16 * KT);
    w1s[f * kr + k] = k < K ? W1[f * K + k] : 0.0f;
  }
  __syncthreads();
  const int w = threadIdx.x / MLCG_WAVE, l = mlcg_lane(), q = l >> 4, n = l & 15;
  int64_t np = max_pairs > 0 ? *n_pairs_dev : 0;
  if (np > max_pairs) np = max_pairs;
  const int64_t tiles = (np + 15) / 16;
  float cen[KT], wid[KT];  // basis function 16kt + n of this lane
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) basis_params(rp, 16 * kt + n, cen[kt], wid[kt]);
  float sc[KT], sw[KT];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) sc[kt] = sw[kt] = 0.f;
  for (int64_t tile = (int64_t)blockIdx.x * kRgWaves + w; tile < tiles;
       tile += (int64_t)gridDim.x * kRgWaves) {
    const int64_t pa = tile * 16 + n;  // the pair this lane feeds into the A operand
    const bool va = pa < np;
    floatx4 gb[KT], gdb[KT];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) gb[kt] = gdb[kt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
    for (int m = 0; m < kF / 16; ++m) {
      // MFMA step s = 4m + j covers feature f = 16m + 4q + j of pair pa
      const float4 av = va ? *reinterpret_cast<const float4*>(abar + pa * kF + 16 * m + 4 * q)
                           : float4{0.f, 0.f, 0.f, 0.f};
      const float4 ad = va ? *reinterpret_cast<const float4*>(adbar + pa * kF + 16 * m + 4 * q)
                           : float4{0.f, 0.f, 0.f, 0.f};
      const float a4[4] = {av.x, av.y, av.z, av.w};
      const float d4[4] = {ad.x, ad.y, ad.z, ad.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int f = 16 * m + 4 * q + j;
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
          const float bw = w1s[f * kr + 16 * kt + n];
          gb[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a4[j], bw, gb[kt], 0, 0, 0);
          gdb[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(d4[j], bw, gdb[kt], 0, 0, 0);
        }
      }
    }
    // gb[kt][i]: pair tile*16 + 4q + i, basis function 16kt + n
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t p = tile * 16 + 4 * q + i;
      if (p >= np) continue;
      const float d = dist[p];
      float C, dC;
      mlcg_cutoff(rp.rbf_kind, rp.rbf_lo, rp.rbf_hi, d, C, dC);
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        const int k = 16 * kt + n;
        if (k >= K) continue;
        float g_c, g_w, gd_c, gd_w;
        basis_param_derivs(rp, cen[kt], wid[kt], d, C, dC, g_c, g_w, gd_c, gd_w);
        sc[kt] += gb[kt][i] * g_c + gdb[kt][i] * gd_c;
        sw[kt] += gb[kt][i] * g_w + gdb[kt][i] * gd_w;
      }
    }
  }
  // sum the 4 lane groups, then the waves (fixed order through LDS)
  __shared__ float red[kRgWaves][2][16 * KT];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) {
    float c = sc[kt], v = sw[kt];
    c += __shfl_xor(c, 16, MLCG_WAVE);
    c += __shfl_xor(c, 32, MLCG_WAVE);
    v += __shfl_xor(v, 16, MLCG_WAVE);
    v += __shfl_xor(v, 32, MLCG_WAVE);
    if (q == 0) {
      red[w][0][16 * kt + n] = c;
      red[w][1][16 * kt + n] = v;
    }
  }
  __syncthreads();
  for (int x = threadIdx.x; x < 2 * 16 * KT; x += blockDim.x) {
    const int which = x / (16 * KT), k = x % (16 * KT);
    partial[(int64_t)blockIdx.x * 2 * 16 * KT + x] =
        (red[0][which][k] + red[1][which][k]) + (red[2][which][k] + red[3][which][k]);
  }
}

// out[x] (+)= sum over the groups' partials, in group order.
__global__ void rbf_grad_reduce_kernel(const float* __restrict__ partial, int groups, int kp,
                                       int K, int accumulate, float* __restrict__ dcenters,
                                       float* __restrict__ dwidths) {
  const int x = threadIdx.x;
  if (x >= 2 * kp) return;
  const int which = x / kp, k = x % kp;
  if (k >= K) return;
  float v = 0.f;
  for (int g = 0; g < groups; ++g) v += partial[(int64_t)g * 2 * kp + x];
  float* dst = which == 0 ? dcenters + k : dwidths + k;
  *dst = accumulate ? *dst + v : v;
}

int rg_groups(int64_t max_pairs) {
  const int64_t tiles = (max_pairs + 15) / 16;
  const int64_t g = (tiles + kRgWaves - 1) / kRgWaves;
  return (int)(g < 1 ? 1 : (g < kRgMaxGroups ? g : kRgMaxGroups));
}

}  // namespace

extern "C" int64_t mlcg_rbf_param_grad_workspace_floats(int64_t max_pairs, int num_rbf) {
  if (max_pairs < 0 || num_rbf < 1 || num_rbf > kMaxK) return -1;
  return (int64_t)rg_groups(max_pairs) * 2 * 16 * ((num_rbf + 15) / 16);
}

extern "C" int mlcg_rbf_param_grad(const float* dist, const int32_t* n_pairs_dev,
                                   int64_t max_pairs, int basis, const float* centers,
                                   const float* widths, float alpha, int num_rbf,
                                   int rbf_cut_kind, float rbf_lo, float rbf_hi,
                                   const float* W1, int num_filters, const float* abar,
                                   const float* adbar, int accumulate, float* dcenters,
                                   float* dwidths, float* workspace, int64_t workspace_floats,
                                   void* stream) {
  if (!valid_params(basis, num_rbf, rbf_cut_kind, 0, 0, num_filters))
    return MLCG_ERR_UNSUPPORTED;
  MLCG_REQUIRE(max_pairs >= 0 && centers && widths && W1 && dcenters && dwidths && workspace);
  MLCG_REQUIRE(max_pairs == 0 || (dist && n_pairs_dev && abar && adbar));
  const int groups = rg_groups(max_pairs);
  const int KT = (num_rbf + 15) / 16;
  MLCG_REQUIRE(workspace_floats >= (int64_t)groups * 2 * 16 * KT);
  RbfParams rp = make_params(basis, centers, widths, alpha, num_rbf, rbf_cut_kind, rbf_lo,
                             rbf_hi, 0, 0.f, 1.f, 0);
  hipStream_t s = mlcg_stream(stream);
  switch (KT) {
#define MLCG_RG(KTV)                                                                        \
  case KTV:                                                                                 \
    hipLaunchKernelGGL(rbf_grad_kernel<KTV>, dim3(groups), dim3(kRgThreads), 0, s, dist,   \
                       n_pairs_dev, max_pairs, rp, W1, abar, adbar, workspace);             \
    break;
    MLCG_RG(1)
    MLCG_RG(2)
    MLCG_RG(3)
    MLCG_RG(4)
    MLCG_RG(5)
    MLCG_RG(6)
    MLCG_RG(7)
    MLCG_RG(8)
#undef MLCG_RG
    default:
      return MLCG_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL(rbf_grad_reduce_kernel, dim3(1), dim3(256), 0, s, workspace, groups,
                     16 * KT, num_rbf, accumulate, dcenters, dwidths);
  return mlcg_launch_status();
}
