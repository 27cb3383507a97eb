// Langevin BAOAB integrator (gfx950).
//
// Reference: LangevinSimulation.timestep (mlcg/simulation/langevin.py:100-144)
//   B  v += 0.5 dt F / m
//   A  x += v dt 0.5
//   O  v = vscale v + noisescale sqrt(1/(beta m)) xi,  xi ~ N(0, 1)
//   A  x += v dt 0.5
//   (forces at the new positions)
//   B  v += 0.5 dt F / m
// with vscale = exp(-dt gamma), noisescale = sqrt(1 - vscale^2)
// (langevin.py:75-76).  The first four sub-steps are one kernel, the last B
// another; the forces are evaluated between them.
//
// Noise: Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers:
// as easy as 1, 2, 3", SC 2011) keyed by the 64-bit seed, counter = (bead,
// step), turned into normals by the Box-Muller transform.  The step counter
// lives in device memory and the final B kernel advances it, so a captured
// graph of one step draws fresh noise on every replay.  Callers may instead
// pass explicit noise (a [N, 3] array), which the parity tests use.
#include "common.h"

namespace {

struct U4 {
  uint32_t a, b, c, d;
};

__device__ __forceinline__ U4 philox4x32_10(U4 ctr, uint32_t k0, uint32_t k1) {
  const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
  const uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)M0 * ctr.a;
    const uint64_t p1 = (uint64_t)M1 * ctr.c;
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    ctr = U4{hi1 ^ ctr.b ^ k0, lo1, hi0 ^ ctr.d ^ k1, lo0};
    k0 += W0;
    k1 += W1;
  }
  return ctr;
}

// uniform in (0, 1]
__device__ __forceinline__ float u01(uint32_t x) {
  return ((float)(x >> 8) + 1.0f) * (1.0f / 16777216.0f);
}

__device__ __forceinline__ void normals3(uint64_t seed, int64_t bead, int64_t step, float& n0,
                                         float& n1, float& n2) {
  const U4 r = philox4x32_10(U4{(uint32_t)bead, (uint32_t)((uint64_t)bead >> 32),
                                (uint32_t)step, (uint32_t)((uint64_t)step >> 32)},
                             (uint32_t)seed, (uint32_t)(seed >> 32));
  const float two_pi = 6.283185307179586f;
  const float ra = sqrtf(-2.0f * logf(u01(r.a)));
  const float rb = sqrtf(-2.0f * logf(u01(r.c)));
  float s, c;
  sincosf(two_pi * u01(r.b), &s, &c);
  n0 = ra * c;
  n1 = ra * s;
  sincosf(two_pi * u01(r.d), &s, &c);
  n2 = rb * c;
}

// T: float, or double for a simulation in double precision (the noise is the
// same float Philox/Box-Muller stream, widened).
template <typename T>
__global__ __launch_bounds__(256) void baoa_kernel(
    T* __restrict__ x, T* __restrict__ v, const T* __restrict__ F,
    const T* __restrict__ masses, const T* __restrict__ bmr, int64_t n, T half_dt,
    T vscale, T noisescale, uint64_t seed, const int64_t* __restrict__ step_dev,
    const T* __restrict__ noise) {
  const int64_t step = step_dev ? *step_dev : 0;
  for (int64_t a = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; a < n;
       a += (int64_t)gridDim.x * blockDim.x) {
    const T m = masses[a];
    const T sig = bmr[a];
    T xi[3];
    if (noise) {
      xi[0] = noise[3 * a];
      xi[1] = noise[3 * a + 1];
      xi[2] = noise[3 * a + 2];
    } else {
      float n0, n1, n2;
      normals3(seed, a, step, n0, n1, n2);
      xi[0] = n0;
      xi[1] = n1;
      xi[2] = n2;
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      T vv = v[3 * a + c] + half_dt * F[3 * a + c] / m;  // B
      T xx = x[3 * a + c] + vv * half_dt;                  // A
      vv = vv * vscale + noisescale * (sig * xi[c]);       // O
      xx = xx + vv * half_dt;                              // A
      v[3 * a + c] = vv;
      x[3 * a + c] = xx;
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void b_kernel(T* __restrict__ v, const T* __restrict__ F,
                                                const T* __restrict__ masses, int64_t n,
                                                T half_dt, int64_t* __restrict__ step_dev) {
  for (int64_t a = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; a < n;
       a += (int64_t)gridDim.x * blockDim.x) {
    const T m = masses[a];
#pragma unroll
    for (int c = 0; c < 3; ++c) v[3 * a + c] = v[3 * a + c] + half_dt * F[3 * a + c] / m;
  }
  // the counter is read only by baoa_kernel, which runs before this kernel
  // in stream order, so one lane may advance it at any point
  if (step_dev && blockIdx.x == 0 && threadIdx.x == 0) *step_dev += 1;
}

__global__ __launch_bounds__(256) void normals_kernel(uint64_t seed, int64_t step, int64_t n,
                                                      float* __restrict__ out) {
  for (int64_t a = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; a < n;
       a += (int64_t)gridDim.x * blockDim.x) {
    float n0, n1, n2;
    normals3(seed, a, step, n0, n1, n2);
    out[3 * a] = n0;
    out[3 * a + 1] = n1;
    out[3 * a + 2] = n2;
  }
}

unsigned groups_for(int64_t n) { return mlcg_persistent_groups(mlcg_div_up(n, 256), 8); }

}  // namespace

namespace {

template <typename T>
int launch_baoa(T* pos, T* vel, const T* forces, const T* masses, const T* beta_mass_ratio,
                int64_t n_nodes, double dt, double vscale, double noisescale, uint64_t seed,
                const int64_t* step_dev, const T* noise, void* stream) {
  MLCG_REQUIRE(n_nodes >= 0 && dt > 0.0);
  if (n_nodes == 0) return MLCG_OK;
  MLCG_REQUIRE(pos && vel && forces && masses && beta_mass_ratio);
  hipLaunchKernelGGL(baoa_kernel<T>, dim3(groups_for(n_nodes)), dim3(256), 0,
                     mlcg_stream(stream), pos, vel, forces, masses, beta_mass_ratio, n_nodes,
                     (T)(0.5 * dt), (T)vscale, (T)noisescale, seed, step_dev, noise);
  return mlcg_launch_status();
}

template <typename T>
int launch_b(T* vel, const T* forces, const T* masses, int64_t n_nodes, double dt,
             int64_t* step_dev, void* stream) {
  MLCG_REQUIRE(n_nodes >= 0 && dt > 0.0);
  if (n_nodes == 0 && !step_dev) return MLCG_OK;
  MLCG_REQUIRE(n_nodes == 0 || (vel && forces && masses));
  hipLaunchKernelGGL(b_kernel<T>, dim3(groups_for(n_nodes)), dim3(256), 0, mlcg_stream(stream),
                     vel, forces, masses, n_nodes, (T)(0.5 * dt), step_dev);
  return mlcg_launch_status();
}

}  // namespace

extern "C" int mlcg_langevin_baoa(float* pos, float* vel, const float* forces,
                                  const float* masses, const float* beta_mass_ratio,
                                  int64_t n_nodes, float dt, float vscale, float noisescale,
                                  uint64_t seed, const int64_t* step_dev, const float* noise,
                                  void* stream) {
  // 0.5f * dt as before: the float form keeps its single-precision constants
  MLCG_REQUIRE(n_nodes >= 0 && dt > 0.0f);
  if (n_nodes == 0) return MLCG_OK;
  MLCG_REQUIRE(pos && vel && forces && masses && beta_mass_ratio);
  hipLaunchKernelGGL(baoa_kernel<float>, dim3(groups_for(n_nodes)), dim3(256), 0,
                     mlcg_stream(stream), pos, vel, forces, masses, beta_mass_ratio, n_nodes,
                     0.5f * dt, vscale, noisescale, seed, step_dev, noise);
  return mlcg_launch_status();
}

extern "C" int mlcg_langevin_b(float* vel, const float* forces, const float* masses,
                               int64_t n_nodes, float dt, int64_t* step_dev, void* stream) {
  MLCG_REQUIRE(n_nodes >= 0 && dt > 0.0f);
  if (n_nodes == 0 && !step_dev) return MLCG_OK;
  MLCG_REQUIRE(n_nodes == 0 || (vel && forces && masses));
  hipLaunchKernelGGL(b_kernel<float>, dim3(groups_for(n_nodes)), dim3(256), 0,
                     mlcg_stream(stream), vel, forces, masses, n_nodes, 0.5f * dt, step_dev);
  return mlcg_launch_status();
}

extern "C" int mlcg_langevin_baoa_f64(double* pos, double* vel, const double* forces,
                                      const double* masses, const double* beta_mass_ratio,
                                      int64_t n_nodes, double dt, double vscale,
                                      double noisescale, uint64_t seed,
                                      const int64_t* step_dev, const double* noise,
                                      void* stream) {
  return launch_baoa(pos, vel, forces, masses, beta_mass_ratio, n_nodes, dt, vscale,
                     noisescale, seed, step_dev, noise, stream);
}

extern "C" int mlcg_langevin_b_f64(double* vel, const double* forces, const double* masses,
                                   int64_t n_nodes, double dt, int64_t* step_dev,
                                   void* stream) {
  return launch_b(vel, forces, masses, n_nodes, dt, step_dev, stream);
}

extern "C" int mlcg_philox_normals(uint64_t seed, int64_t step, int64_t n_nodes, float* out,
                                   void* stream) {
  MLCG_REQUIRE(n_nodes >= 0);
  if (n_nodes == 0) return MLCG_OK;
  MLCG_REQUIRE(out);
  hipLaunchKernelGGL(normals_kernel, dim3(groups_for(n_nodes)), dim3(256), 0,
                     mlcg_stream(stream), seed, step, n_nodes, out);
  return mlcg_launch_status();
}
