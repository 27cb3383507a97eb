// Radius graph for batches of independent frames (gfx950).
//
// Semantics follow mlcg's SchNet neighbour list (torch_cluster.radius_graph
// with flow="target_to_source", mlcg/neighbor_list/torch_impl.py:216-224) and
// the reference's own CUDA kernel (src/opt_radius/mlcg_opt_radius/radius.cu:
// strict d2 < r^2 at line 134, r^2 computed on the host at line 250, rows
// keep their lowest-index neighbours when max_num_neighbors binds, lines
// 125-141).  Output order is canonical: rows by centre i ascending, and
// within a row neighbours j ascending.
//
// Design: two passes (count, then fill at scanned offsets) give an exact,
// deterministic layout without atomics, cooperative launches or host
// synchronisation inside the library.  The count runs one or more threads per
// row over its frame; the fill one wave per row: the wave sweeps the row's frame
// 64 candidates at a time, each lane testing one candidate, a ballot gives the
// hit mask and mbcnt the rank of each hit, so every row's edges are written as
// contiguous, coalesced runs.  Both stage the positions of a workgroup's
// frames in LDS.
//
// Optional pair exclusion follows the reference kernel's CSR form
// (radius.cu:113-133, built by exclusion_pair_to_ptr in exclusion_pairs.cpp:
// 7-62): neighbour j is dropped from row i when j appears in
// xs[ptr[i] .. ptr[i+1]), a segment sorted ascending.  Excluded neighbours do
// not count towards max_num_neighbors, as in the reference.  Each lane looks
// its candidate up by binary search in the row's segment.
#include <algorithm>
#include <mutex>
#include <utility>
#include <vector>

#include "common.h"

namespace {

constexpr int kRowWaves = 4;  // waves per workgroup (256 threads)

// Positions are float32 or float64 (T); the membership test runs in T, as
// the reference's kernel runs it in its scalar type (radius.cu:243-250).
template <typename T>
struct Vec3T {
  T x, y, z;
};

template <typename T>
__device__ __forceinline__ Vec3T<T> load_pos(const T* __restrict__ pos, int64_t n) {
  Vec3T<T> v;
  v.x = pos[3 * n + 0];
  v.y = pos[3 * n + 1];
  v.z = pos[3 * n + 2];
  return v;
}

// Squared distance exactly as ((dx*dx + dy*dy) + dz*dz) with round-to-nearest
// on every operation: contraction into FMA is disabled so that membership at
// the cutoff boundary is reproducible bit for bit by a plain C restatement.
template <typename T>
__device__ __forceinline__ T sqdist_exact(Vec3T<T> a, Vec3T<T> b) {
#pragma clang fp contract(off)
  T dx = b.x - a.x;
  T dy = b.y - a.y;
  T dz = b.z - a.z;
  T s = dx * dx;
  s = s + dy * dy;
  s = s + dz * dz;
  return s;
}

// True when j occurs in the sorted segment xs[lo, hi).
__device__ __forceinline__ bool in_sorted(const int64_t* __restrict__ xs, int64_t lo,
                                          int64_t hi, int64_t j) {
  const int64_t end = hi;
  while (lo < hi) {
    const int64_t mid = lo + ((hi - lo) >> 1);
    if (xs[mid] < j)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo < end && xs[lo] == j;
}

__device__ __forceinline__ int lanes_below(uint64_t mask) {
  // number of set bits of `mask` strictly below this lane
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__global__ void frame_ptr_kernel(const int64_t* __restrict__ batch, int64_t n,
                                 int64_t n_frames, int64_t* __restrict__ ptr) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n == 0) {
    if (i <= n_frames) ptr[i] = 0;
    return;
  }
  if (i >= n) return;
  int64_t b = batch[i];
  int64_t prev = i == 0 ? -1 : batch[i - 1];
  if (b > n_frames) b = n_frames;
  for (int64_t k = prev + 1; k <= b; ++k) ptr[k] = i;
  if (i == n - 1)
    for (int64_t k = b + 1; k <= n_frames; ++k) ptr[k] = n;
}

// Fill sweep over row i: writes every kept neighbour from the lane that holds
// it (ranks by mbcnt over the hit ballot), with kPairs also the pair list and
// its edge map for the upper neighbours.  Node and edge indices are int32
// (the CSR is int32; the host entry points reject larger inputs).  Returns
// nothing; `dropped` is set when an edge or pair falls past its capacity.
template <bool kExcl, bool kStaged, bool kPairs, typename T>
__device__ __forceinline__ void fill_row(
    const T* __restrict__ pos, int base, int i, int start, int end, T r2, int loop,
    int max_nn, const int64_t* __restrict__ exs, const int64_t* __restrict__ eptr,
    int64_t* __restrict__ ei0, int64_t* __restrict__ ei1, int32_t* __restrict__ col,
    int e_base, int e_cap, int32_t* __restrict__ pi, int32_t* __restrict__ pj,
    int32_t* __restrict__ eid2pair, int p_base, int p_cap, bool& dropped) {
  const int lane = mlcg_lane();
  const Vec3T<T> a = load_pos(pos, kStaged ? i - base : i);
  int kept = 0, ukept = 0;
  int64_t x_lo = 0, x_hi = 0;
  if (kExcl) {
    x_lo = eptr[i];
    x_hi = eptr[i + 1];
  }
  for (int j0 = start; j0 < end && kept < max_nn; j0 += MLCG_WAVE) {
    const int j = j0 + lane;
    bool hit = false;
    if (j < end) {
      const T d2 = sqdist_exact(a, load_pos(pos, kStaged ? j - base : j));
      hit = (d2 < r2) && (loop || j != i);
      if (kExcl && hit) hit = !in_sorted(exs, x_lo, x_hi, (int64_t)j);
    }
    const uint64_t m = __ballot(hit);
    if (m == 0) continue;
    const int rank = lanes_below(m);
    const bool keep = hit && (kept + rank < max_nn);
    const int e = e_base + kept + rank;
    if (keep) {
      if (e < e_cap) {
        ei0[e] = i;
        ei1[e] = j;
        if (kPairs) col[e] = j;
      } else {
        dropped = true;
      }
    }
    if (kPairs) {
      const bool upper = keep && (j > i);
      const uint64_t um = __ballot(upper);
      if (upper && e < e_cap) {
        const int p = p_base + ukept + lanes_below(um);
        if (p < p_cap) {
          pi[p] = i;
          pj[p] = j;
          eid2pair[e] = p;
        } else {
          dropped = true;
        }
      }
      ukept += __popcll(um);
    }
    kept += __popcll(m);
  }
}

// Work split of the fill kernel: a workgroup of kRowWaves waves takes a block
// of kBlockRows consecutive rows, wave w the consecutive rows w R .. w R + R - 1
// (R = kRowsPerWave), so that each wave writes one contiguous run of the
// edge list and completes the cache lines its rows share.
// The nodes of the frames those rows belong to -- a contiguous node range,
// as frames are -- are staged once in LDS when they fit (kStage nodes), so
// every distance test reads LDS instead of L2 and the rows' loads are shared;
// a block whose frames are larger reads positions from global memory.
constexpr int kBlockRows = 64;
constexpr int kStage = 2048;  // nodes staged per workgroup (24 KiB of LDS)

struct BlockNodes {
  int64_t r0, r1;      // rows of the block
  int64_t c_lo, c_hi;  // nodes of its frames
  bool staged;
};

// Stages the block's nodes (every thread must call; one barrier when staged).
template <typename T>
__device__ __forceinline__ BlockNodes stage_block(const T* __restrict__ pos,
                                                  const int64_t* __restrict__ batch,
                                                  const int64_t* __restrict__ frame_ptr,
                                                  int64_t n, T* sp) {
  BlockNodes bn;
  bn.r0 = (int64_t)blockIdx.x * kBlockRows;
  bn.r1 = bn.r0 + kBlockRows < n ? bn.r0 + kBlockRows : n;
  bn.c_lo = frame_ptr[batch[bn.r0]];
  bn.c_hi = frame_ptr[batch[bn.r1 - 1] + 1];
  bn.staged = bn.c_hi >= bn.c_lo && bn.c_hi - bn.c_lo <= kStage;
  if (bn.staged) {
    const int64_t cnt = 3 * (bn.c_hi - bn.c_lo);
    for (int64_t t = threadIdx.x; t < cnt; t += blockDim.x) sp[t] = pos[3 * bn.c_lo + t];
    __syncthreads();
  }
  return bn;
}

// The per-row scalars of a wave's rows (row k of wave w: r0 + w R + k) are
// loaded once, lane k holding row k's, so that no row waits on a chain of
// dependent loads (batch -> frame_ptr -> rowptr) before its sweep; the row
// loop takes them with readlane.  Offsets are below 2^31 (int32 CSR).
constexpr int kRowsPerWave = kBlockRows / kRowWaves;
struct RowBounds {
  int start, end, e_base, p_base;
};
__device__ __forceinline__ RowBounds row_bounds(const BlockNodes& bn,
                                                const int64_t* __restrict__ batch,
                                                const int64_t* __restrict__ frame_ptr,
                                                const int32_t* __restrict__ rowptr,
                                                const int32_t* __restrict__ pairptr) {
  RowBounds rb{0, 0, 0, 0};
  const int lane = mlcg_lane();
  const int64_t i = bn.r0 + (threadIdx.x / MLCG_WAVE) * kRowsPerWave + lane;
  if (lane < kRowsPerWave && i < bn.r1) {
    const int64_t b = batch[i];
    rb.start = (int)frame_ptr[b];
    rb.end = (int)frame_ptr[b + 1];
    if (rowptr) rb.e_base = rowptr[i];
    if (pairptr) rb.p_base = pairptr[i];
  }
  return rb;
}

// Pass 1 runs `parts` threads per row (a power of two up to 64, chosen by the
// host so that the launch fills the chip): a counting sweep needs no ballots
// or ranks, and per candidate a thread spends a handful of instructions where
// a wave per row spends a few dozen on masks.  Thread p of a row visits the
// candidates start + p, start + p + parts, ...; the per-row counts are then
// summed over the row's threads (adjacent lanes) with xor shuffles.  The
// positions of the workgroup's frames are staged in LDS as in the fill pass.
// With a binding max_num_neighbors the kept neighbours are the lowest-index
// ones: kept = min(hits, max_nn) and the kept upper neighbours (j > i) are
// what remains after the lower ones and the self loop.
constexpr int kCountThreads = 256;

template <bool kExcl, typename T>
__global__ __launch_bounds__(kCountThreads) void radius_count_kernel(
    const T* __restrict__ pos, const int64_t* __restrict__ batch,
    const int64_t* __restrict__ frame_ptr, int64_t n, T r2, int loop, int64_t max_nn,
    const int64_t* __restrict__ exs, const int64_t* __restrict__ eptr, int parts,
    int32_t* __restrict__ deg, int32_t* __restrict__ udeg, int32_t* __restrict__ overflow) {
  __shared__ T sp[3 * kStage];
  const int rows_per_block = kCountThreads / parts;
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t r1 = r0 + rows_per_block < n ? r0 + rows_per_block : n;
  const int64_t c_lo = frame_ptr[batch[r0]];
  const int64_t c_hi = frame_ptr[batch[r1 - 1] + 1];
  const bool staged = c_hi >= c_lo && c_hi - c_lo <= kStage;  // uniform
  if (staged) {
    for (int64_t t = threadIdx.x; t < 3 * (c_hi - c_lo); t += blockDim.x)
      sp[t] = pos[3 * c_lo + t];
    __syncthreads();
  }
  const int64_t i = r0 + threadIdx.x / parts;
  const int part = threadIdx.x % parts;
  const bool active = i < r1;
  int lower = 0, self = 0, upper = 0;
  bool asym = false;
  if (active) {
    const int64_t b = batch[i];
    const int64_t start = frame_ptr[b], end = frame_ptr[b + 1];
    const bool local = staged && start >= c_lo && end <= c_hi;
    const Vec3T<T> a = local ? load_pos(sp, i - c_lo) : load_pos(pos, i);
    int64_t x_lo = 0, x_hi = 0;
    if (kExcl) {
      x_lo = eptr[i];
      x_hi = eptr[i + 1];
    }
    for (int64_t j = start + part; j < end; j += parts) {
      const T d2 = sqdist_exact(a, local ? load_pos(sp, j - c_lo) : load_pos(pos, j));
      bool hit = (d2 < r2) && (loop || j != i);
      if (kExcl && hit) {
        hit = !in_sorted(exs, x_lo, x_hi, j);
        if (hit && in_sorted(exs, eptr[j], eptr[j + 1], i)) asym = true;
      }
      if (hit) {
        lower += j < i;
        self += j == i;
        upper += j > i;
      }
    }
  }
  // sum over the row's `parts` adjacent lanes (every lane takes part)
  for (int o = 1; o < parts; o <<= 1) {
    lower += __shfl_xor(lower, o, MLCG_WAVE);
    self += __shfl_xor(self, o, MLCG_WAVE);
    upper += __shfl_xor(upper, o, MLCG_WAVE);
  }
  if (!active || part != 0) {
    if (kExcl && asym && overflow) atomicOr(overflow, 4);
    return;
  }
  const int64_t total = (int64_t)lower + self + upper;
  const int64_t kept = total < max_nn ? total : max_nn;
  const int64_t room = max_nn - lower - self;
  const int64_t ukept = room <= 0 ? 0 : (upper < room ? upper : room);
  deg[i] = (int32_t)kept;
  udeg[i] = (int32_t)ukept;
  if (total > max_nn && overflow) atomicOr(overflow, 1);
  if (kExcl && asym && overflow) atomicOr(overflow, 4);
}

template <bool kExcl, bool kPairs, typename T>
__global__ __launch_bounds__(kRowWaves * MLCG_WAVE) void radius_fill_kernel(
    const T* __restrict__ pos, const int64_t* __restrict__ batch,
    const int64_t* __restrict__ frame_ptr, int64_t n, T r2, int loop,
    int64_t max_nn, const int64_t* __restrict__ exs, const int64_t* __restrict__ eptr,
    const int32_t* __restrict__ rowptr, const int32_t* __restrict__ pairptr, int64_t e_cap,
    int64_t e_stride, int64_t* __restrict__ edge_index, int32_t* __restrict__ col,
    int64_t p_cap, int64_t p_stride, int32_t* __restrict__ pair_ij,
    int32_t* __restrict__ eid2pair, int32_t* __restrict__ overflow) {
  __shared__ T sp[3 * kStage];
  const BlockNodes bn = stage_block(pos, batch, frame_ptr, n, sp);
  const RowBounds rb = row_bounds(bn, batch, frame_ptr, rowptr, pairptr);
  int32_t* pi = pair_ij;
  int32_t* pj = pair_ij ? pair_ij + p_stride : nullptr;
  bool dropped = false;
  for (int k = 0; k < kRowsPerWave; ++k) {
    const int64_t i = bn.r0 + (threadIdx.x / MLCG_WAVE) * kRowsPerWave + k;
    if (i >= bn.r1) break;
    const int64_t start = __builtin_amdgcn_readlane(rb.start, k);
    const int64_t end = __builtin_amdgcn_readlane(rb.end, k);
    const int64_t e_base = __builtin_amdgcn_readlane(rb.e_base, k);
    const int64_t p_base = __builtin_amdgcn_readlane(rb.p_base, k);
    const int mnn = max_nn < (int64_t)INT32_MAX ? (int)max_nn : INT32_MAX;
    const int ecap = e_cap < (int64_t)INT32_MAX ? (int)e_cap : INT32_MAX;
    const int pcap = p_cap < (int64_t)INT32_MAX ? (int)p_cap : INT32_MAX;
    if (bn.staged && start >= bn.c_lo && end <= bn.c_hi)  // wave-uniform
      fill_row<kExcl, true, kPairs>(sp, (int)bn.c_lo, (int)i, (int)start, (int)end, r2, loop,
                                    mnn, exs, eptr, edge_index, edge_index + e_stride, col,
                                    (int)e_base, ecap, pi, pj, eid2pair, (int)p_base, pcap,
                                    dropped);
    else
      fill_row<kExcl, false, kPairs>(pos, 0, (int)i, (int)start, (int)end, r2, loop, mnn, exs,
                                     eptr, edge_index, edge_index + e_stride, col, (int)e_base,
                                     ecap, pi, pj, eid2pair, (int)p_base, pcap, dropped);
  }
  if (dropped && overflow) atomicOr(overflow, 2);
}

// eid2pair for the lower copy (j, i) of every pair (i < j): binary search of i
// in the sorted row j.
__global__ void pair_reverse_kernel(const int32_t* __restrict__ pi,
                                    const int32_t* __restrict__ pj,
                                    const int32_t* __restrict__ n_pairs_dev,
                                    int64_t max_pairs, const int32_t* __restrict__ rowptr,
                                    const int32_t* __restrict__ col,
                                    int32_t* __restrict__ eid2pair) {
  int64_t np = *n_pairs_dev;
  if (np > max_pairs) np = max_pairs;
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < np;
       p += (int64_t)gridDim.x * blockDim.x) {
    const int32_t i = pi[p];
    const int32_t j = pj[p];
    int32_t lo = rowptr[j], hi = rowptr[j + 1];
    while (lo < hi) {
      int32_t mid = (lo + hi) >> 1;
      if (col[mid] < i)
        lo = mid + 1;
      else
        hi = mid;
    }
    if (lo < rowptr[j + 1] && col[lo] == i) eid2pair[lo] = (int32_t)p;
  }
}

// ---------------------------------------------------------------------------
// Exclusive scan of two int32 vectors (tile = 1024 elements, 256 threads).
constexpr int kScanThreads = 256;
constexpr int kScanItems = 4;
constexpr int kScanTile = kScanThreads * kScanItems;

__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = mlcg_lane();
#pragma unroll
  for (int o = 1; o < MLCG_WAVE; o <<= 1) {
    int t = __shfl_up(v, o, MLCG_WAVE);
    if (lane >= o) v += t;
  }
  return v;
}

// Block-wide exclusive scan of one value per thread; returns the exclusive
// prefix and writes the block total to *total.
__device__ __forceinline__ int block_excl_scan(int v, int* smem, int* total) {
  const int lane = mlcg_lane();
  const int w = threadIdx.x / MLCG_WAVE;
  int incl = wave_incl_scan(v);
  if (lane == MLCG_WAVE - 1) smem[w] = incl;
  __syncthreads();
  int off = 0, tot = 0;
  for (int k = 0; k < kScanThreads / MLCG_WAVE; ++k) {
    if (k < w) off += smem[k];
    tot += smem[k];
  }
  __syncthreads();
  *total = tot;
  return off + incl - v;
}

__global__ __launch_bounds__(kScanThreads) void scan_tile_sums(
    const int32_t* __restrict__ a, const int32_t* __restrict__ b, int64_t n,
    int32_t* __restrict__ sa, int32_t* __restrict__ sb) {
  __shared__ int smem[2][kScanThreads / MLCG_WAVE];
  const int64_t base = (int64_t)blockIdx.x * kScanTile + threadIdx.x * kScanItems;
  int va = 0, vb = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    if (base + k < n) {
      va += a[base + k];
      vb += b[base + k];
    }
  }
  int ta, tb;
  block_excl_scan(va, smem[0], &ta);
  block_excl_scan(vb, smem[1], &tb);
  if (threadIdx.x == 0) {
    sa[blockIdx.x] = ta;
    sb[blockIdx.x] = tb;
  }
}

// Single workgroup: in-place exclusive scan of the tile sums.
__global__ __launch_bounds__(kScanThreads) void scan_tile_offsets(int32_t* __restrict__ sa,
                                                                  int32_t* __restrict__ sb,
                                                                  int64_t tiles) {
  __shared__ int smem[2][kScanThreads / MLCG_WAVE];
  int carry_a = 0, carry_b = 0;
  for (int64_t t0 = 0; t0 < tiles; t0 += kScanThreads) {
    const int64_t t = t0 + threadIdx.x;
    int va = t < tiles ? sa[t] : 0;
    int vb = t < tiles ? sb[t] : 0;
    int ta, tb;
    int ea = block_excl_scan(va, smem[0], &ta);
    int eb = block_excl_scan(vb, smem[1], &tb);
    if (t < tiles) {
      sa[t] = carry_a + ea;
      sb[t] = carry_b + eb;
    }
    carry_a += ta;
    carry_b += tb;
  }
}

__global__ __launch_bounds__(kScanThreads) void scan_tile_apply(
    const int32_t* __restrict__ a, const int32_t* __restrict__ b, int64_t n,
    const int32_t* __restrict__ sa, const int32_t* __restrict__ sb,
    int32_t* __restrict__ oa, int32_t* __restrict__ ob) {
  __shared__ int smem[2][kScanThreads / MLCG_WAVE];
  const int64_t base = (int64_t)blockIdx.x * kScanTile + threadIdx.x * kScanItems;
  int xa[kScanItems], xb[kScanItems];
  int va = 0, vb = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    xa[k] = base + k < n ? a[base + k] : 0;
    xb[k] = base + k < n ? b[base + k] : 0;
    va += xa[k];
    vb += xb[k];
  }
  int ta, tb;
  int ea = block_excl_scan(va, smem[0], &ta) + sa[blockIdx.x];
  int eb = block_excl_scan(vb, smem[1], &tb) + sb[blockIdx.x];
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    if (base + k < n) {
      oa[base + k] = ea;
      ob[base + k] = eb;
    }
    ea += xa[k];
    eb += xb[k];
  }
  if (blockIdx.x == gridDim.x - 1 && threadIdx.x == kScanThreads - 1) {
    oa[n] = ea;
    ob[n] = eb;
  }
}

// n == 0: both totals are zero (a fill kernel rather than a memset node, so
// the call stays safe inside captured graphs).
__global__ void zero_totals(int32_t* a, int32_t* b) {
  a[0] = 0;
  b[0] = 0;
}

}  // namespace

extern "C" int mlcg_frame_ptr_from_batch(const int64_t* batch, int64_t n_nodes,
                                         int64_t n_frames, int64_t* frame_ptr,
                                         void* stream) {
  MLCG_REQUIRE(frame_ptr && n_nodes >= 0 && n_frames >= 0);
  MLCG_REQUIRE(n_nodes == 0 || batch);
  int64_t work = n_nodes == 0 ? n_frames + 1 : n_nodes;
  hipLaunchKernelGGL(frame_ptr_kernel, dim3(mlcg_div_up(work, 256)), dim3(256), 0,
                     mlcg_stream(stream), batch, n_nodes, n_frames, frame_ptr);
  return mlcg_launch_status();
}

namespace {

template <typename T>
int launch_radius_count(const T* pos, const int64_t* batch, const int64_t* frame_ptr,
                        int64_t n_nodes, double r, int loop, int64_t max_num_neighbors,
                        const int64_t* exclude_pair_xs, const int64_t* ptr_exclude_pair_xs,
                        int32_t* deg, int32_t* upper_deg, int32_t* overflow, void* stream) {
  MLCG_REQUIRE(n_nodes >= 0 && n_nodes < (int64_t(1) << 31) && r >= 0.0 &&
               max_num_neighbors >= 0);
  MLCG_REQUIRE((exclude_pair_xs == nullptr) == (ptr_exclude_pair_xs == nullptr));
  if (n_nodes == 0) return MLCG_OK;
  MLCG_REQUIRE(pos && batch && frame_ptr && deg && upper_deg);
  const T r2 = (T)(r * r);  // r*r in double, then the scalar type (radius.cu:250)
  // threads per row: enough threads for about four waves per SIMD
  int parts = 1;
  while (parts < MLCG_WAVE && n_nodes * parts < (int64_t(1) << 18)) parts *= 2;
  dim3 grid(mlcg_div_up(n_nodes, kCountThreads / parts)), block(kCountThreads);
  hipStream_t s = mlcg_stream(stream);
  if (exclude_pair_xs)
    hipLaunchKernelGGL((radius_count_kernel<true, T>), grid, block, 0, s, pos, batch,
                       frame_ptr, n_nodes, r2, loop, max_num_neighbors, exclude_pair_xs,
                       ptr_exclude_pair_xs, parts, deg, upper_deg, overflow);
  else
    hipLaunchKernelGGL((radius_count_kernel<false, T>), grid, block, 0, s, pos, batch,
                       frame_ptr, n_nodes, r2, loop, max_num_neighbors, nullptr, nullptr, parts,
                       deg, upper_deg, overflow);
  return mlcg_launch_status();
}

template <typename T>
int launch_radius_fill(const T* pos, const int64_t* batch, const int64_t* frame_ptr,
                       int64_t n_nodes, double r, int loop, int64_t max_num_neighbors,
                       const int64_t* exclude_pair_xs, const int64_t* ptr_exclude_pair_xs,
                       const int32_t* rowptr, const int32_t* pairptr, int64_t edge_capacity,
                       int64_t edge_stride, int64_t* edge_index, int32_t* col,
                       int64_t pair_capacity, int64_t pair_stride, int32_t* pair_ij,
                       int32_t* eid2pair, int32_t* overflow, void* stream) {
  MLCG_REQUIRE(n_nodes >= 0 && n_nodes < (int64_t(1) << 31) && r >= 0.0 &&
               max_num_neighbors >= 0);
  MLCG_REQUIRE(edge_capacity >= 0 && edge_stride >= edge_capacity);
  MLCG_REQUIRE((exclude_pair_xs == nullptr) == (ptr_exclude_pair_xs == nullptr));
  if (n_nodes == 0 || edge_capacity == 0) return MLCG_OK;
  MLCG_REQUIRE(pos && batch && frame_ptr && rowptr && edge_index);
  MLCG_REQUIRE(!pair_ij || (pairptr && pair_stride >= pair_capacity));
  MLCG_REQUIRE(!eid2pair || pair_ij);
  const T r2 = (T)(r * r);
  dim3 grid(mlcg_div_up(n_nodes, kBlockRows)), block(kRowWaves * MLCG_WAVE);
  hipStream_t s = mlcg_stream(stream);
  // the pair structures come together (col, pair list and its edge map)
  MLCG_REQUIRE((col == nullptr && pair_ij == nullptr && eid2pair == nullptr) ||
               (col != nullptr && pair_ij != nullptr && eid2pair != nullptr));
  const bool pairs = pair_ij != nullptr;
#define MLCG_FILL_LAUNCH(EX, PR)                                                          \
  hipLaunchKernelGGL((radius_fill_kernel<EX, PR, T>), grid, block, 0, s, pos, batch,      \
                     frame_ptr, n_nodes, r2, loop, max_num_neighbors,                     \
                     EX ? exclude_pair_xs : nullptr, EX ? ptr_exclude_pair_xs : nullptr,  \
                     rowptr, pairptr, edge_capacity, edge_stride, edge_index, col,        \
                     pair_capacity, pair_stride, pair_ij, eid2pair, overflow)
  if (exclude_pair_xs && pairs) MLCG_FILL_LAUNCH(true, true);
  else if (exclude_pair_xs) MLCG_FILL_LAUNCH(true, false);
  else if (pairs) MLCG_FILL_LAUNCH(false, true);
  else MLCG_FILL_LAUNCH(false, false);
#undef MLCG_FILL_LAUNCH
  return mlcg_launch_status();
}

}  // namespace

extern "C" int mlcg_radius_count(const float* pos, const int64_t* batch,
                                 const int64_t* frame_ptr, int64_t n_nodes, double r,
                                 int loop, int64_t max_num_neighbors,
                                 const int64_t* exclude_pair_xs,
                                 const int64_t* ptr_exclude_pair_xs, int32_t* deg,
                                 int32_t* upper_deg, int32_t* overflow, void* stream) {
  return launch_radius_count(pos, batch, frame_ptr, n_nodes, r, loop, max_num_neighbors,
                             exclude_pair_xs, ptr_exclude_pair_xs, deg, upper_deg, overflow,
                             stream);
}

extern "C" int mlcg_radius_count_f64(const double* pos, const int64_t* batch,
                                     const int64_t* frame_ptr, int64_t n_nodes, double r,
                                     int loop, int64_t max_num_neighbors,
                                     const int64_t* exclude_pair_xs,
                                     const int64_t* ptr_exclude_pair_xs, int32_t* deg,
                                     int32_t* upper_deg, int32_t* overflow, void* stream) {
  return launch_radius_count(pos, batch, frame_ptr, n_nodes, r, loop, max_num_neighbors,
                             exclude_pair_xs, ptr_exclude_pair_xs, deg, upper_deg, overflow,
                             stream);
}

extern "C" int64_t mlcg_scan_workspace_ints(int64_t n) {
  return 2 * ((n + kScanTile - 1) / kScanTile + 1);
}

namespace {

// The scan proper; `workspace` holds mlcg_scan_workspace_ints(n) int32 (the
// per-tile sums, every one written before it is read: nothing needs clearing).
int launch_scan2(const int32_t* in_a, const int32_t* in_b, int64_t n, int32_t* out_a,
                 int32_t* out_b, int32_t* workspace, hipStream_t s) {
  if (n == 0) {
    hipLaunchKernelGGL(zero_totals, dim3(1), dim3(1), 0, s, out_a, out_b);
    return mlcg_launch_status();
  }
  const int64_t tiles = (n + kScanTile - 1) / kScanTile;
  int32_t* sa = workspace;
  int32_t* sb = workspace + tiles + 1;
  hipLaunchKernelGGL(scan_tile_sums, dim3((unsigned)tiles), dim3(kScanThreads), 0, s, in_a,
                     in_b, n, sa, sb);
  hipLaunchKernelGGL(scan_tile_offsets, dim3(1), dim3(kScanThreads), 0, s, sa, sb, tiles);
  hipLaunchKernelGGL(scan_tile_apply, dim3((unsigned)tiles), dim3(kScanThreads), 0, s, in_a,
                     in_b, n, sa, sb, out_a, out_b);
  return mlcg_launch_status();
}

// Workspace of mlcg_exclusive_scan2_i32_noalloc: a file-scope device array
// sized for MLCG_SCAN_NOALLOC_MAX_N elements (2 x 16,385 int32 = 128 KiB per
// device, held until the process ends).  Host code never passes `scratch`
// itself to a kernel (in host code the name is only a stand-in): its device
// address is looked up once per device with hipGetSymbolAddress and cached.
constexpr int64_t kScanNoAllocInts = 2 * ((MLCG_SCAN_NOALLOC_MAX_N + kScanTile - 1) / kScanTile + 1);
__device__ __align__(256) int32_t scratch[kScanNoAllocInts];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
int32_t* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (nullptr on failure).
int32_t* scratch_for_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr)
      return nullptr;
    g_scratch_ptr[dev] = static_cast<int32_t*>(p);
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" int mlcg_exclusive_scan2_i32(const int32_t* in_a, const int32_t* in_b, int64_t n,
                                        int32_t* out_a, int32_t* out_b, int32_t* workspace,
                                        void* stream) {
  MLCG_REQUIRE(n >= 0 && out_a && out_b && workspace);
  MLCG_REQUIRE(n == 0 || (in_a && in_b));
  return launch_scan2(in_a, in_b, n, out_a, out_b, workspace, mlcg_stream(stream));
}

extern "C" int mlcg_exclusive_scan2_i32_noalloc(const int32_t* in_a, const int32_t* in_b,
                                                int64_t n, int32_t* out_a, int32_t* out_b,
                                                void* stream) {
  MLCG_REQUIRE(n >= 0 && out_a && out_b);
  MLCG_REQUIRE(n == 0 || (in_a && in_b));
  if (n > MLCG_SCAN_NOALLOC_MAX_N) return MLCG_ERR_CAPACITY;
  int32_t* ws = scratch_for_current_device();
  if (ws == nullptr) return MLCG_ERR_LAUNCH;
  return launch_scan2(in_a, in_b, n, out_a, out_b, ws, mlcg_stream(stream));
}

extern "C" int mlcg_radius_fill(const float* pos, const int64_t* batch,
                                const int64_t* frame_ptr, int64_t n_nodes, double r,
                                int loop, int64_t max_num_neighbors,
                                const int64_t* exclude_pair_xs,
                                const int64_t* ptr_exclude_pair_xs, const int32_t* rowptr,
                                const int32_t* pairptr, int64_t edge_capacity,
                                int64_t edge_stride, int64_t* edge_index, int32_t* col,
                                int64_t pair_capacity, int64_t pair_stride,
                                int32_t* pair_ij, int32_t* eid2pair, int32_t* overflow,
                                void* stream) {
  return launch_radius_fill(pos, batch, frame_ptr, n_nodes, r, loop, max_num_neighbors,
                            exclude_pair_xs, ptr_exclude_pair_xs, rowptr, pairptr,
                            edge_capacity, edge_stride, edge_index, col, pair_capacity,
                            pair_stride, pair_ij, eid2pair, overflow, stream);
}

extern "C" int mlcg_radius_fill_f64(const double* pos, const int64_t* batch,
                                    const int64_t* frame_ptr, int64_t n_nodes, double r,
                                    int loop, int64_t max_num_neighbors,
                                    const int64_t* exclude_pair_xs,
                                    const int64_t* ptr_exclude_pair_xs,
                                    const int32_t* rowptr, int64_t edge_capacity,
                                    int64_t edge_stride, int64_t* edge_index,
                                    int32_t* overflow, void* stream) {
  return launch_radius_fill(pos, batch, frame_ptr, n_nodes, r, loop, max_num_neighbors,
                            exclude_pair_xs, ptr_exclude_pair_xs, rowptr,
                            (const int32_t*)nullptr, edge_capacity, edge_stride, edge_index,
                            (int32_t*)nullptr, 0, 0, (int32_t*)nullptr, (int32_t*)nullptr,
                            overflow, stream);
}

// Host-side conversion of an exclusion pair list to the per-row CSR the
// kernels read (exclusion_pair_to_ptr, exclusion_pairs.cpp:7-62): pairs
// (x, y) are ordered by y, then x; pair_xs lists the x of every pair in that
// order and y_ptr[n] counts the pairs with y < n.  A pair with y < 0 is an
// error once num_nodes > 0 (the reference's check at line 47); pairs with
// y >= num_nodes stay at the end of pair_xs, outside every row.
extern "C" int mlcg_exclusion_pair_to_ptr(const int64_t* exc_pair_index, int64_t num_pairs,
                                          int64_t num_nodes, int64_t* pair_xs,
                                          int64_t* y_ptr) {
  MLCG_REQUIRE(num_pairs >= 0 && num_nodes >= 0 && y_ptr);
  MLCG_REQUIRE(num_pairs == 0 || (exc_pair_index && pair_xs));
  std::vector<std::pair<int64_t, int64_t>> yx((size_t)num_pairs);
  for (int64_t k = 0; k < num_pairs; ++k)
    yx[(size_t)k] = {exc_pair_index[num_pairs + k], exc_pair_index[k]};
  std::sort(yx.begin(), yx.end());
  for (int64_t k = 0; k < num_pairs; ++k) pair_xs[k] = yx[(size_t)k].second;
  if (num_nodes > 0 && num_pairs > 0 && yx[0].first < 0) return MLCG_ERR_ARGUMENT;
  int64_t k = 0;
  y_ptr[0] = 0;
  for (int64_t node = 0; node < num_nodes; ++node) {
    while (k < num_pairs && yx[(size_t)k].first == node) ++k;
    y_ptr[node + 1] = k;
  }
  return MLCG_OK;
}

extern "C" int mlcg_pair_reverse_map(const int32_t* pair_ij, int64_t pair_stride,
                                     const int32_t* n_pairs_dev, int64_t max_pairs,
                                     const int32_t* rowptr, const int32_t* col,
                                     int32_t* eid2pair, void* stream) {
  MLCG_REQUIRE(max_pairs >= 0 && pair_stride >= max_pairs);
  if (max_pairs == 0) return MLCG_OK;
  MLCG_REQUIRE(pair_ij && n_pairs_dev && rowptr && col && eid2pair);
  unsigned groups = mlcg_persistent_groups(mlcg_div_up(max_pairs, 256), 8);
  hipLaunchKernelGGL(pair_reverse_kernel, dim3(groups), dim3(256), 0, mlcg_stream(stream),
                     pair_ij, pair_ij + pair_stride, n_pairs_dev, max_pairs, rowptr, col,
                     eid2pair);
  return mlcg_launch_status();
}
