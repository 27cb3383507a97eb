// Bonded and repulsion prior energies with analytic forces (gfx950).
//
// Reference forms (ClementiGroup/mlcg):
//   bonds      U = k (r - x0)^2 + V0, r = |p1 - p0|
//              (Harmonic.compute, nn/prior/harmonic.py:119-120; features from
//              compute_distances, geometry/internal_coordinates.py:73-100)
//   angles     U = k (cos t - x0)^2 + V0, cos t = (dr1.dr2)/|dr1|/|dr2|,
//              dr1 = p0 - p1, dr2 = p2 - p1 (internal_coordinates.py:146-183)
//   dihedrals  V = sum_n k1_n sin(n t) + k2_n cos(n t) + v0
//              (FourierSeries.compute, nn/prior/fourier_series.py:160-198) with
//              the mdtraj-convention torsion of internal_coordinates.py:187-252
//   repulsion  U = (sigma / r)^6 (Repulsion.compute, nn/prior/repulsion.py:136-140)
// The reference obtains forces by autograd; here each interaction writes its
// energy and the analytic force on each of its beads ("slot forces"), and a
// second kernel sums the slot forces of every bead over a bead -> slot CSR in
// ascending slot order, so the force reduction is deterministic and needs no
// atomics.  Per-frame energies use the segmented sum of cfconv.hip.
//
// The repulsion prior gives every bead a few hundred slots, so its slot
// forces (24 bytes per interaction written, 12 per slot read back) cost more
// than the arithmetic.  Its forces also have a direct form: pair_records_kernel
// lists, in the bead -> slot CSR order, each slot's partner bead, role (bead 0
// or 1 of the interaction) and sigma (once per topology and parameter table),
// and repulsion_forces_kernel evaluates each slot's force from the two
// positions with the operations of prior_terms_kernel and adds them in
// prior_gather_kernel's order, so the forces are the same bit for bit while
// the terms kernel writes energies only.
//
// Torsion: with rij = pi - pj, rkj = pk - pj, rkl = pk - pl, m = rij x rkj,
// n = rkj x rkl, the reference's atan2(-y, x) equals
//   t = atan2(|rkj| (rij . n), m . n),
// and dt/dp follows the Bekker/Blondel-Karplus form:
//   dt/dpi = -|rkj|/|m|^2 m,  dt/dpl = |rkj|/|n|^2 n, and the two inner
//   beads from p = (rij.rkj)/|rkj|^2, q = (rkl.rkj)/|rkj|^2.
#include "common.h"

namespace {

template <typename T>
struct V3T {
  T x, y, z;
};
using V3 = V3T<float>;
using D3 = V3T<double>;
template <typename T = float, typename P>
__device__ __forceinline__ V3T<T> ld3(const P* __restrict__ p, int64_t i) {
  return V3T<T>{(T)p[3 * i], (T)p[3 * i + 1], (T)p[3 * i + 2]};
}
template <typename T>
__device__ __forceinline__ V3T<T> sub(V3T<T> a, V3T<T> b) {
  return V3T<T>{a.x - b.x, a.y - b.y, a.z - b.z};
}
template <typename T>
__device__ __forceinline__ V3T<T> add(V3T<T> a, V3T<T> b) {
  return V3T<T>{a.x + b.x, a.y + b.y, a.z + b.z};
}
template <typename T>
__device__ __forceinline__ V3T<T> scl(T s, V3T<T> a) {
  return V3T<T>{s * a.x, s * a.y, s * a.z};
}
// Fused multiply-adds in a fixed order: left to the compiler, the contraction
// of a sum of products follows the surrounding code, and the repulsion forces
// of prior_terms_kernel and repulsion_forces_kernel must round alike.
template <typename T>
__device__ __forceinline__ T dot(V3T<T> a, V3T<T> b) {
  return fma(a.z, b.z, fma(a.y, b.y, a.x * b.x));
}
template <typename T>
__device__ __forceinline__ V3T<T> cross(V3T<T> a, V3T<T> b) {
  return V3T<T>{a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x};
}
template <typename S, typename T>
__device__ __forceinline__ void st3(S* __restrict__ f, int64_t slot, V3T<T> v) {
  f[3 * slot] = (S)v.x;
  f[3 * slot + 1] = (S)v.y;
  f[3 * slot + 2] = (S)v.z;
}
__device__ __forceinline__ void sin_cos(float x, float* s, float* c) { sincosf(x, s, c); }
__device__ __forceinline__ void sin_cos(double x, double* s, double* c) { sincos(x, s, c); }
__device__ __forceinline__ float sqrt_t(float x) { return sqrtf(x); }
__device__ __forceinline__ double sqrt_t(double x) { return sqrt(x); }
__device__ __forceinline__ float atan2_t(float y, float x) { return atan2f(y, x); }
__device__ __forceinline__ double atan2_t(double y, double x) { return atan2(y, x); }

// S: the storage type of positions, parameters, energies and slot forces
// (float, or double for a model moved to double).  Bonds and angles are
// evaluated in double either way; the repulsion and the dihedrals in S.
template <int KIND, typename S>
__global__ __launch_bounds__(256) void prior_terms_kernel(
    int n_degs, const S* __restrict__ pos, const int64_t* __restrict__ map,
    int64_t stride, int64_t M, const S* __restrict__ params, int n_params,
    S* __restrict__ energy, S* __restrict__ slot_f) {
  using C = S;  // compute type of the repulsion and the dihedrals
  using VC = V3T<C>;
  for (int64_t m = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; m < M;
       m += (int64_t)gridDim.x * blockDim.x) {
    const S* pr = params + m * n_params;
    if (KIND == MLCG_PRIOR_BOND) {
      // Harmonic terms are evaluated in fp64 from the fp32 positions: the
      // force 2 k (r - x0) of a stiff bond (k = 100 at config 5) amplifies the
      // fp32 rounding of r (a few 1e-7 A) into force errors of ~6e-5, which the
      // reference's fp32 arithmetic carries; in fp64 only the final rounding
      // of the force remains.
      const D3 pi = ld3<double>(pos, map[m]);
      const D3 pj = ld3<double>(pos, map[stride + m]);
      const D3 d = sub(pj, pi);
      const double r = sqrt(dot(d, d));
      const double x0 = pr[0], k = pr[1], v0 = pr[2];
      const double dr = r - x0;
      const double dUdr = 2.0 * k * dr;
      const D3 fi = scl(dUdr / r, d);  // force on bead 0; bead 1 gets -fi
      energy[m] = (S)(k * (dr * dr) + v0);
      if (slot_f) {
        st3(slot_f, 2 * m, fi);
        st3(slot_f, 2 * m + 1, scl(-1.0, fi));
      }
    } else if (KIND == MLCG_PRIOR_REPULSION) {
      const VC pi = ld3<C>(pos, map[m]);
      const VC pj = ld3<C>(pos, map[stride + m]);
      const VC d = sub(pj, pi);
      const C r = sqrt_t(dot(d, d));
      const C s = pr[0] / r;
      const C rr = s * s;
      const C e = rr * rr * rr;
      const C dUdr = (C)-6.0 * e / r;
      const VC fi = scl(dUdr / r, d);
      energy[m] = e;
      if (slot_f) {
        st3(slot_f, 2 * m, fi);
        st3(slot_f, 2 * m + 1, scl((C)-1.0, fi));
      }
    } else if (KIND == MLCG_PRIOR_ANGLE) {
      // fp64 for the same reason as the bonds (k (cos t - x0)^2)
      const D3 p0 = ld3<double>(pos, map[m]);
      const D3 p1 = ld3<double>(pos, map[stride + m]);
      const D3 p2 = ld3<double>(pos, map[2 * stride + m]);
      const D3 a = sub(p0, p1), b = sub(p2, p1);
      const double na = sqrt(dot(a, a)), nb = sqrt(dot(b, b));
      const double c = dot(a, b) / na / nb;
      const double x0 = pr[0], k = pr[1], v0 = pr[2];
      const double dc = c - x0;
      energy[m] = (S)(k * (dc * dc) + v0);
      const double g = 2.0 * k * dc;  // dU/dcos
      const double inv = 1.0 / (na * nb);
      const D3 dca = sub(scl(inv, b), scl(c / (na * na), a));
      const D3 dcb = sub(scl(inv, a), scl(c / (nb * nb), b));
      const D3 f0 = scl(-g, dca), f2 = scl(-g, dcb);
      if (slot_f) {
        st3(slot_f, 3 * m, f0);
        st3(slot_f, 3 * m + 1, scl(-1.0, add(f0, f2)));
        st3(slot_f, 3 * m + 2, f2);
      }
    } else {  // MLCG_PRIOR_DIHEDRAL
      const VC pi = ld3<C>(pos, map[m]);
      const VC pj = ld3<C>(pos, map[stride + m]);
      const VC pk = ld3<C>(pos, map[2 * stride + m]);
      const VC pl = ld3<C>(pos, map[3 * stride + m]);
      const VC rij = sub(pi, pj), rkj = sub(pk, pj), rkl = sub(pk, pl);
      const VC mv = cross(rij, rkj), nv = cross(rkj, rkl);
      const C rkj2 = dot(rkj, rkj);
      const C nrkj = sqrt_t(rkj2);
      const C t = atan2_t(nrkj * dot(rij, nv), dot(mv, nv));
      C V = pr[0], dV = 0;
      for (int d = 1; d <= n_degs; ++d) {
        C sn, co;
        sin_cos((C)d * t, &sn, &co);
        const C k1 = pr[d], k2 = pr[n_degs + d];
        V += k1 * sn + k2 * co;
        dV += (C)d * (k1 * co - k2 * sn);
      }
      energy[m] = V;
      const VC fi = scl(-dV * nrkj / dot(mv, mv), mv);
      const VC fl = scl(dV * nrkj / dot(nv, nv), nv);
      const C p = dot(rij, rkj) / rkj2, q = dot(rkl, rkj) / rkj2;
      const VC sv = sub(scl(p, fi), scl(q, fl));
      const VC fj = sub(fi, sv), fk = add(fl, sv);
      if (slot_f) {
        st3(slot_f, 4 * m, fi);
        st3(slot_f, 4 * m + 1, scl((C)-1.0, fj));
        st3(slot_f, 4 * m + 2, scl((C)-1.0, fk));
        st3(slot_f, 4 * m + 3, fl);
      }
    }
  }
}

// forces[a] (+)= sum over the slots of bead a.  A group of kGatherLanes
// lanes serves one bead: lane k sums the bead's slots k, k + kGatherLanes,
// ... in ascending order, and the group then adds its partial sums in a fixed
// butterfly, so the result does not depend on timing (a bead of the
// repulsion prior has hundreds of slots; a lane per bead would walk them one
// dependent load at a time).
constexpr int kGatherLanes = 16;

template <typename S>
__global__ __launch_bounds__(256) void prior_gather_kernel(
    const S* __restrict__ slot_f, const int32_t* __restrict__ bead_ptr,
    const int32_t* __restrict__ bead_slots, int64_t n, int accumulate,
    S* __restrict__ forces) {
  const int sub = threadIdx.x % kGatherLanes;
  const int64_t ngroups = (int64_t)gridDim.x * blockDim.x / kGatherLanes;
  for (int64_t a = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kGatherLanes; a < n;
       a += ngroups) {
    S fx = 0, fy = 0, fz = 0;
    const int32_t s1 = bead_ptr[a + 1];
    for (int32_t s = bead_ptr[a] + sub; s < s1; s += kGatherLanes) {
      const int64_t slot = bead_slots[s];
      fx += slot_f[3 * slot];
      fy += slot_f[3 * slot + 1];
      fz += slot_f[3 * slot + 2];
    }
    // every lane of the group shares a, so the group is active together
#pragma unroll
    for (int o = kGatherLanes / 2; o > 0; o >>= 1) {
      fx += __shfl_xor(fx, o, kGatherLanes);
      fy += __shfl_xor(fy, o, kGatherLanes);
      fz += __shfl_xor(fz, o, kGatherLanes);
    }
    if (sub == 0) {
      if (accumulate) {
        forces[3 * a] += fx;
        forces[3 * a + 1] += fy;
        forces[3 * a + 2] += fz;
      } else {
        forces[3 * a] = fx;
        forces[3 * a + 1] = fy;
        forces[3 * a + 2] = fz;
      }
    }
  }
}

// Bead-major records of an order-2 prior: position s of bead_slots (slot
// 2m + k of interaction m) gets {partner bead | k << 31, params[m][0]}.
__global__ __launch_bounds__(256) void pair_records_kernel(
    const int64_t* __restrict__ map, int64_t stride, const float* __restrict__ params,
    int n_params, const int32_t* __restrict__ bead_slots, int64_t n_slots,
    int2* __restrict__ rec) {
  for (int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; s < n_slots;
       s += (int64_t)gridDim.x * blockDim.x) {
    const int32_t slot = bead_slots[s];
    const int64_t m = slot >> 1;
    const int k = slot & 1;
    const int64_t partner = map[(1 - k) * stride + m];
    rec[s] = int2{(int)((uint32_t)partner | ((uint32_t)k << 31)), __float_as_int(params[m * n_params])};
  }
}

// The repulsion kernels look up a random partner bead per slot; fetched from
// the L2 these lookups (one request each) and not the bytes set their time,
// so each workgroup stages the positions of the bead window its work touches
// in LDS first.  Windows are computed with the records (once per topology):
// for a force block of kRepBeads beads the range of the beads and all their
// partners, for an energy chunk of kRepChunk interactions the range of their
// beads.  A window wider than kRepWin beads is served from global memory.
constexpr int kRepBeads = 256 / kGatherLanes;  // beads per force workgroup
constexpr int kRepU = 4;                       // interactions per energy thread
constexpr int kRepChunk = 256 * kRepU;         // interactions per energy workgroup
constexpr int kRepWin = 1024;                  // LDS window, beads (16 KiB)

__device__ __forceinline__ int2 block_minmax(int lo, int hi, int* red) {
  for (int o = 32; o > 0; o >>= 1) {
    lo = min(lo, __shfl_xor(lo, o, MLCG_WAVE));
    hi = max(hi, __shfl_xor(hi, o, MLCG_WAVE));
  }
  const int w = threadIdx.x / MLCG_WAVE;
  if (mlcg_lane() == 0) {
    red[2 * w] = lo;
    red[2 * w + 1] = hi;
  }
  __syncthreads();
  lo = red[0];
  hi = red[1];
  for (int k = 1; k < (int)blockDim.x / MLCG_WAVE; ++k) {
    lo = min(lo, red[2 * k]);
    hi = max(hi, red[2 * k + 1]);
  }
  return int2{lo, hi + 1};
}

__global__ __launch_bounds__(256) void force_windows_kernel(const int2* __restrict__ rec,
                                                            const int32_t* __restrict__ bead_ptr,
                                                            int64_t n, int2* __restrict__ win) {
  __shared__ int red[8];
  const int64_t a0 = (int64_t)blockIdx.x * kRepBeads;
  const int64_t a1 = min(a0 + kRepBeads, n);
  int lo = (int)a0, hi = (int)(a1 - 1);
  for (int32_t s = bead_ptr[a0] + threadIdx.x; s < bead_ptr[a1]; s += blockDim.x) {
    const int b = rec[s].x & 0x7fffffff;
    lo = min(lo, b);
    hi = max(hi, b);
  }
  const int2 w = block_minmax(lo, hi, red);
  if (threadIdx.x == 0) win[blockIdx.x] = w;
}

__global__ __launch_bounds__(256) void energy_windows_kernel(const int64_t* __restrict__ map,
                                                             int64_t stride, int64_t M,
                                                             int2* __restrict__ win) {
  __shared__ int red[8];
  int lo = INT_MAX, hi = -1;
  for (int64_t m = (int64_t)blockIdx.x * kRepChunk + threadIdx.x;
       m < min((int64_t)(blockIdx.x + 1) * kRepChunk, M); m += blockDim.x) {
    const int bi = (int)map[m], bj = (int)map[stride + m];
    lo = min(lo, min(bi, bj));
    hi = max(hi, max(bi, bj));
  }
  const int2 w = block_minmax(lo, hi, red);
  if (threadIdx.x == 0) win[blockIdx.x] = w;
}

// Window positions into LDS (4 floats a bead); false when the window is too
// wide, and then nothing is staged.  Every thread of the workgroup calls it.
__device__ __forceinline__ bool stage_window(const float* __restrict__ pos, int2 w, float4* P) {
  const int cnt = w.y - w.x;
  if (cnt > kRepWin || cnt <= 0) return false;
  for (int k = threadIdx.x; k < cnt; k += blockDim.x) {
    const int64_t b = (int64_t)w.x + k;
    P[k] = float4{pos[3 * b], pos[3 * b + 1], pos[3 * b + 2], 0.f};
  }
  __syncthreads();
  return true;
}

__device__ __forceinline__ V3 pos_at(const float* __restrict__ pos, const float4* P, bool staged,
                                     int lo, int64_t b) {
  if (staged) {
    const float4 v = P[b - lo];
    return V3{v.x, v.y, v.z};
  }
  return ld3(pos, b);
}

// forces[a] (+)= the repulsion slot forces of bead a, each evaluated from the
// positions as prior_terms_kernel<MLCG_PRIOR_REPULSION> does (bead 0 of the
// interaction gets fi, bead 1 gets -fi) and added in prior_gather_kernel's
// lane order and butterfly.  The products of the force are rounded on their
// own (__fmul_rn), as when they were stored, before they are added.
__global__ __launch_bounds__(256) void repulsion_forces_kernel(
    const float* __restrict__ pos, const int2* __restrict__ rec, const int2* __restrict__ win,
    const int32_t* __restrict__ bead_ptr, int64_t n, int accumulate, float* __restrict__ forces) {
  __shared__ float4 P[kRepWin];
  const int2 w = win[blockIdx.x];
  const bool staged = stage_window(pos, w, P);
  const int lk = threadIdx.x % kGatherLanes;
  const int64_t a = (int64_t)blockIdx.x * kRepBeads + threadIdx.x / kGatherLanes;
  if (a >= n) return;
  float fx = 0.f, fy = 0.f, fz = 0.f;
  const V3 pa = pos_at(pos, P, staged, w.x, a);
  const int32_t s1 = bead_ptr[a + 1];
  for (int32_t s = bead_ptr[a] + lk; s < s1; s += kRepU * kGatherLanes) {
    int2 rc[kRepU];  // the records of kRepU slots requested together
#pragma unroll
    for (int u = 0; u < kRepU; ++u) rc[u] = rec[min(s + u * kGatherLanes, s1 - 1)];
#pragma unroll
    for (int u = 0; u < kRepU; ++u) {
      if (s + u * kGatherLanes >= s1) break;
      const bool second = rc[u].x < 0;  // bit 31: the bead is bead 1 of the interaction
      const V3 pb = pos_at(pos, P, staged, w.x, rc[u].x & 0x7fffffff);
      const V3 pi = second ? pb : pa, pj = second ? pa : pb;
      const V3 d = sub(pj, pi);
      const float r = sqrtf(dot(d, d));
      const float sr = __int_as_float(rc[u].y) / r;
      const float rr = sr * sr;
      const float e = rr * rr * rr;
      const float dUdr = -6.0f * e / r;
      const float c = dUdr / r;
      V3 f{__fmul_rn(c, d.x), __fmul_rn(c, d.y), __fmul_rn(c, d.z)};
      if (second) f = V3{-f.x, -f.y, -f.z};
      fx += f.x;
      fy += f.y;
      fz += f.z;
    }
  }
  // the 16 lanes of a bead are in one wave and active together
#pragma unroll
  for (int o = kGatherLanes / 2; o > 0; o >>= 1) {
    fx += __shfl_xor(fx, o, kGatherLanes);
    fy += __shfl_xor(fy, o, kGatherLanes);
    fz += __shfl_xor(fz, o, kGatherLanes);
  }
  if (lk == 0) {
    if (accumulate) {
      forces[3 * a] += fx;
      forces[3 * a + 1] += fy;
      forces[3 * a + 2] += fz;
    } else {
      forces[3 * a] = fx;
      forces[3 * a + 1] = fy;
      forces[3 * a + 2] = fz;
    }
  }
}

// Energies of the repulsion prior only (prior_terms_kernel's operations),
// kRepU interactions per thread.
__global__ __launch_bounds__(256) void repulsion_energy_kernel(
    const float* __restrict__ pos, const int64_t* __restrict__ map, int64_t stride, int64_t M,
    const float* __restrict__ params, const int2* __restrict__ win, float* __restrict__ energy) {
  __shared__ float4 P[kRepWin];
  const int2 w = win[blockIdx.x];
  int64_t bi[kRepU], bj[kRepU];
  float sg[kRepU];
#pragma unroll
  for (int u = 0; u < kRepU; ++u) {  // requested before the window is staged
    const int64_t m = min((int64_t)blockIdx.x * kRepChunk + u * 256 + threadIdx.x, M - 1);
    bi[u] = map[m];
    bj[u] = map[stride + m];
    sg[u] = params[m];
  }
  const bool staged = stage_window(pos, w, P);
#pragma unroll
  for (int u = 0; u < kRepU; ++u) {
    const int64_t m = (int64_t)blockIdx.x * kRepChunk + u * 256 + threadIdx.x;
    if (m >= M) break;
    const V3 pi = pos_at(pos, P, staged, w.x, bi[u]);
    const V3 pj = pos_at(pos, P, staged, w.x, bj[u]);
    const V3 d = sub(pj, pi);
    const float r = sqrtf(dot(d, d));
    const float sr = sg[u] / r;
    const float rr = sr * sr;
    energy[m] = rr * rr * rr;
  }
}

int order_of(int kind) {
  switch (kind) {
    case MLCG_PRIOR_BOND:
    case MLCG_PRIOR_REPULSION:
      return 2;
    case MLCG_PRIOR_ANGLE:
      return 3;
    case MLCG_PRIOR_DIHEDRAL:
      return 4;
    default:
      return 0;
  }
}

int params_of(int kind, int n_degs) {
  switch (kind) {
    case MLCG_PRIOR_BOND:
    case MLCG_PRIOR_ANGLE:
      return 3;
    case MLCG_PRIOR_REPULSION:
      return 1;
    case MLCG_PRIOR_DIHEDRAL:
      return 1 + 2 * n_degs;
    default:
      return -1;
  }
}

}  // namespace

extern "C" int mlcg_prior_order(int kind) { return order_of(kind); }

extern "C" int mlcg_prior_num_params(int kind, int n_degs) { return params_of(kind, n_degs); }

namespace {

template <typename S>
int launch_prior_terms(int kind, int n_degs, const S* pos, const int64_t* index_mapping,
                       int64_t mapping_stride, int64_t n_interactions, const S* params,
                       int n_params, S* energy, S* slot_forces, void* stream) {
  if (order_of(kind) == 0) return MLCG_ERR_UNSUPPORTED;
  MLCG_REQUIRE(n_interactions >= 0 && mapping_stride >= n_interactions);
  MLCG_REQUIRE(kind != MLCG_PRIOR_DIHEDRAL || (n_degs >= 1 && n_degs <= 64));
  MLCG_REQUIRE(n_params == params_of(kind, n_degs));
  if (n_interactions == 0) return MLCG_OK;
  MLCG_REQUIRE(pos && index_mapping && params && energy);
  const unsigned groups = mlcg_persistent_groups(mlcg_div_up(n_interactions, 256), 8);
  hipStream_t s = mlcg_stream(stream);
#define MLCG_TERMS_LAUNCH(KIND)                                                              \
  hipLaunchKernelGGL((prior_terms_kernel<KIND, S>), dim3(groups), dim3(256), 0, s, n_degs,  \
                     pos, index_mapping, mapping_stride, n_interactions, params, n_params,  \
                     energy, slot_forces)
  switch (kind) {
    case MLCG_PRIOR_BOND:
      MLCG_TERMS_LAUNCH(MLCG_PRIOR_BOND);
      break;
    case MLCG_PRIOR_ANGLE:
      MLCG_TERMS_LAUNCH(MLCG_PRIOR_ANGLE);
      break;
    case MLCG_PRIOR_DIHEDRAL:
      MLCG_TERMS_LAUNCH(MLCG_PRIOR_DIHEDRAL);
      break;
    default:
      MLCG_TERMS_LAUNCH(MLCG_PRIOR_REPULSION);
      break;
  }
#undef MLCG_TERMS_LAUNCH
  return mlcg_launch_status();
}

template <typename S>
int launch_prior_gather(const S* slot_forces, const int32_t* bead_ptr,
                        const int32_t* bead_slots, int64_t n_nodes, int accumulate, S* forces,
                        void* stream) {
  MLCG_REQUIRE(n_nodes >= 0);
  if (n_nodes == 0) return MLCG_OK;
  MLCG_REQUIRE(bead_ptr && forces);
  MLCG_REQUIRE(slot_forces || bead_slots == nullptr);
  const unsigned groups = mlcg_persistent_groups(mlcg_div_up(n_nodes * kGatherLanes, 256), 8);
  hipLaunchKernelGGL(prior_gather_kernel<S>, dim3(groups), dim3(256), 0, mlcg_stream(stream),
                     slot_forces, bead_ptr, bead_slots, n_nodes, accumulate, forces);
  return mlcg_launch_status();
}

}  // namespace

extern "C" int mlcg_prior_terms(int kind, int n_degs, const float* pos,
                                const int64_t* index_mapping, int64_t mapping_stride,
                                int64_t n_interactions, const float* params, int n_params,
                                float* energy, float* slot_forces, void* stream) {
  return launch_prior_terms(kind, n_degs, pos, index_mapping, mapping_stride, n_interactions,
                            params, n_params, energy, slot_forces, stream);
}

extern "C" int mlcg_prior_terms_f64(int kind, int n_degs, const double* pos,
                                    const int64_t* index_mapping, int64_t mapping_stride,
                                    int64_t n_interactions, const double* params, int n_params,
                                    double* energy, double* slot_forces, void* stream) {
  return launch_prior_terms(kind, n_degs, pos, index_mapping, mapping_stride, n_interactions,
                            params, n_params, energy, slot_forces, stream);
}

extern "C" int mlcg_prior_gather_forces(const float* slot_forces, const int32_t* bead_ptr,
                                        const int32_t* bead_slots, int64_t n_nodes,
                                        int accumulate, float* forces, void* stream) {
  return launch_prior_gather(slot_forces, bead_ptr, bead_slots, n_nodes, accumulate, forces,
                             stream);
}

extern "C" int mlcg_prior_gather_forces_f64(const double* slot_forces, const int32_t* bead_ptr,
                                            const int32_t* bead_slots, int64_t n_nodes,
                                            int accumulate, double* forces, void* stream) {
  return launch_prior_gather(slot_forces, bead_ptr, bead_slots, n_nodes, accumulate, forces,
                             stream);
}

namespace {
int64_t rep_force_blocks(int64_t n) { return (n + kRepBeads - 1) / kRepBeads; }
int64_t rep_energy_chunks(int64_t M) { return (M + kRepChunk - 1) / kRepChunk; }
}  // namespace

extern "C" int64_t mlcg_prior_pair_records_ints(int64_t n_nodes, int64_t n_interactions) {
  if (n_nodes < 0 || n_interactions < 0) return -1;
  return 4 * n_interactions + 2 * rep_force_blocks(n_nodes) + 2 * rep_energy_chunks(n_interactions);
}

extern "C" int mlcg_prior_pair_records(const int64_t* index_mapping, int64_t mapping_stride,
                                       int64_t n_interactions, const float* params,
                                       int n_params, const int32_t* bead_ptr,
                                       const int32_t* bead_slots, int64_t n_nodes,
                                       void* records, void* stream) {
  MLCG_REQUIRE(n_interactions >= 0 && mapping_stride >= n_interactions && n_params >= 1);
  MLCG_REQUIRE(n_nodes >= 0 && n_nodes < (int64_t(1) << 31) && n_interactions < (int64_t(1) << 30));
  if (n_nodes == 0) return MLCG_OK;
  MLCG_REQUIRE(bead_ptr && records);
  MLCG_REQUIRE(n_interactions == 0 || (index_mapping && params && bead_slots));
  hipStream_t s = mlcg_stream(stream);
  int2* rec = reinterpret_cast<int2*>(records);
  int2* fwin = rec + 2 * n_interactions;
  int2* ewin = fwin + rep_force_blocks(n_nodes);
  const int64_t n_slots = 2 * n_interactions;
  if (n_slots > 0)
    hipLaunchKernelGGL(pair_records_kernel, dim3(mlcg_persistent_groups(mlcg_div_up(n_slots, 256), 8)),
                       dim3(256), 0, s, index_mapping, mapping_stride, params, n_params,
                       bead_slots, n_slots, rec);
  hipLaunchKernelGGL(force_windows_kernel, dim3((unsigned)rep_force_blocks(n_nodes)), dim3(256),
                     0, s, rec, bead_ptr, n_nodes, fwin);
  if (n_interactions > 0)
    hipLaunchKernelGGL(energy_windows_kernel, dim3((unsigned)rep_energy_chunks(n_interactions)),
                       dim3(256), 0, s, index_mapping, mapping_stride, n_interactions, ewin);
  return mlcg_launch_status();
}

extern "C" int mlcg_prior_repulsion(const float* pos, int64_t n_nodes,
                                    const int64_t* index_mapping, int64_t mapping_stride,
                                    int64_t n_interactions, const float* params,
                                    const void* records, const int32_t* bead_ptr, float* energy,
                                    int accumulate, float* forces, void* stream) {
  MLCG_REQUIRE(n_nodes >= 0 && n_nodes < (int64_t(1) << 31));
  MLCG_REQUIRE(n_interactions >= 0 && mapping_stride >= n_interactions);
  if (n_nodes == 0) return MLCG_OK;
  MLCG_REQUIRE(pos && bead_ptr && records && forces);
  MLCG_REQUIRE(n_interactions == 0 || (index_mapping && params && energy));
  hipStream_t s = mlcg_stream(stream);
  const int2* rec = reinterpret_cast<const int2*>(records);
  const int2* fwin = rec + 2 * n_interactions;
  const int2* ewin = fwin + rep_force_blocks(n_nodes);
  if (n_interactions > 0)
    hipLaunchKernelGGL(repulsion_energy_kernel, dim3((unsigned)rep_energy_chunks(n_interactions)),
                       dim3(256), 0, s, pos, index_mapping, mapping_stride, n_interactions,
                       params, ewin, energy);
  hipLaunchKernelGGL(repulsion_forces_kernel, dim3((unsigned)rep_force_blocks(n_nodes)),
                     dim3(256), 0, s, pos, rec, fwin, bead_ptr, n_nodes, accumulate, forces);
  return mlcg_launch_status();
}
