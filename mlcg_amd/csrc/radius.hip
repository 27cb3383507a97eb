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
// Design: one row-block kernel (radius_rows_kernel) gives an exact,
// deterministic layout without atomics on the output, cooperative launches or
// host synchronisation inside the library.  A wave sweeps a row's frame 64
// candidates at a time, each lane testing one candidate; the ballot is the
// row's hit mask and mbcnt the rank of each hit, so every row's edges are
// written as contiguous runs.  Row offsets come from a block scan plus a
// decoupled look-back across blocks (the sizing pass and the one-launch
// form), or from a CSR the caller passes (the write pass).  The positions of a
// workgroup's frames are staged in LDS.  radius_count_kernel and the
// three-kernel int32 scan remain for the per-node degree entry points.
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

// Positions are float32, float64, float16 or bfloat16 (T); the membership
// test runs in T, as the reference's kernel runs it in its scalar type
// (radius.cu:243-250).
template <typename T>
struct Vec3T {
  T x, y, z;
};

// float16 / bfloat16 positions: every operation is computed in float and
// rounded to the storage type (round to nearest even), which is how the
// reference's c10::Half / c10::BFloat16 instantiation of the kernel
// evaluates `dist += (x - y) * (x - y)` and `dist < r` (each operator
// converts to float, operates and converts back).  float carries more than
// twice the significand bits of both types, so each operation equals the
// native 16-bit one (the compiler emits those); products and sums are never
// fused, as the reference rounds each of them.
template <typename S>
struct Narrow {
  S v;
  Narrow() = default;
  __host__ __device__ Narrow(float f) : v(static_cast<S>(f)) {}
  __host__ __device__ operator float() const { return static_cast<float>(v); }
};
template <typename S>
__device__ __forceinline__ Narrow<S> operator-(Narrow<S> a, Narrow<S> b) {
#pragma clang fp contract(off)
  return Narrow<S>(static_cast<float>(a) - static_cast<float>(b));
}
template <typename S>
__device__ __forceinline__ Narrow<S> operator+(Narrow<S> a, Narrow<S> b) {
#pragma clang fp contract(off)
  return Narrow<S>(static_cast<float>(a) + static_cast<float>(b));
}
template <typename S>
__device__ __forceinline__ Narrow<S> operator*(Narrow<S> a, Narrow<S> b) {
#pragma clang fp contract(off)
  return Narrow<S>(static_cast<float>(a) * static_cast<float>(b));
}
template <typename S>
__device__ __forceinline__ bool operator<(Narrow<S> a, Narrow<S> b) {
  return static_cast<float>(a) < static_cast<float>(b);
}
using H16 = Narrow<_Float16>;
using B16 = Narrow<__bf16>;
static_assert(sizeof(H16) == 2 && sizeof(B16) == 2, "16-bit position storage");

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

// Inclusive scan over the 64 lanes of a wave.
__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = mlcg_lane();
#pragma unroll
  for (int o = 1; o < MLCG_WAVE; o <<= 1) {
    int t = __shfl_up(v, o, MLCG_WAVE);
    if (lane >= o) v += t;
  }
  return v;
}

__device__ __forceinline__ int64_t wave_incl_scan64(int64_t v) {
  const int lane = mlcg_lane();
#pragma unroll
  for (int o = 1; o < MLCG_WAVE; o <<= 1) {
    int64_t t = __shfl_up(v, o, MLCG_WAVE);
    if (lane >= o) v += t;
  }
  return v;
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

constexpr int kStage = 2048;  // nodes staged per workgroup by the count kernel (24 KiB)

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

// ---------------------------------------------------------------------------
// Row-block kernel of the radius graph.  A workgroup of W waves (BlockWaves)
// takes a block of W R consecutive rows, wave w the rows w R .. w R + R - 1
// (R rows per wave, see RowsPerWave), so that each wave writes one contiguous
// run of the edge list.  The nodes of the block's frames -- a contiguous node range, as frames
// are -- are staged in LDS as 4-component records when they fit
// (StageNodes<T>); a block whose frames are larger reads positions from
// global memory.
//
// The kernel is instruction-bound, not memory-bound (a 64-wide VALU or SALU
// instruction retires at about one per cycle per CU), so the sweep is built to
// spend few instructions per 64 candidates:
// - a wave takes its rows kGroup at a time; when the kGroup rows share one
//   staged frame (the common case) every lane loads its candidate once
//   (ds_read_b128) and tests it against the kGroup centres; the compare writes
//   the row's hit mask straight into scalar registers, cut to the frame by one
//   scalar mask on the last chunk;
// - the self pair (j = i) is taken out once per row, not per candidate: the
//   count from the same distance test (d(i, i) < r^2 is what the sweep saw),
//   the mask bit when the write pass reads the row's masks;
// - the masks of a row's first kMaskWords chunks go to LDS, laid out
//   [chunk][row] so that lane 0 stores a group's kGroup masks of a chunk as
//   one 32-byte record straight from the ballots; rows with pair exclusions
//   and groups that straddle frames or are not staged take a general path
//   that tests every condition per lane, and rows longer than kMaskWords
//   chunks are tested again in the write pass.
// Rows keep their lowest-index neighbours when max_num_neighbors binds
// (radius.cu:125-141): kept = min(hits, max_nn), and the kept upper neighbours
// (j > i) are what remains after the lower ones and the self loop.
//
// Modes:
//   kModeRowptr  kept counts scanned within the block (one wave) and across
//                blocks (decoupled look-back); rowptr / pairptr written (the
//                sizing pass of the exactly-sized graph);
//   kModeFill    rowptr / pairptr given; a write pass emits every kept
//                neighbour from the lane that holds it (rank by mbcnt over the
//                row's mask; rows past 64 chunks are tested again);
//   kModeFused   both in one launch (the fixed-capacity form).
// Look-back: each block publishes its totals (edges, pairs) in a status word
// of the workspace, first as an aggregate, then as an inclusive prefix; a
// block sums the aggregates of its predecessors back to the first inclusive
// prefix, reading kLookLanes x 64 predecessors per round.  A block waits
// only for blocks of lower index, which the dispatcher started before it (it
// dispatches workgroups in index order), and every wait is bounded
// (kSpinLimit polls): a block that gives up sets overflow bit 8 and carries
// on, so the kernel always finishes and the host reports the error.
// Workspace (zero-filled by the caller before its first use, then reused):
// word 0 the launch epoch, word 1 the most blocks any launch has used, then
// two interleaved status arrays -- block b's status of a launch with epoch e
// at word 2 + 2b + (e & 1).  Every block reads the two header words first;
// each launch clears the other array's words up to the larger of the two
// block counts, and its last block advances the header after its look-back.
// When no wait timed out, every block has published by then, hence read the
// header, and the next launch's array is zero wherever it reads, with no
// clearing launch in between.  After a timeout (bit 8) a block that had not
// started yet may read the advanced header and publish into the next
// launch's array: the flag makes every caller raise, and the host discards
// the workspace when it reads bit 8 (ops.radius_flags_read).  The caller's overflow word is cleared by
// block 0 before it publishes its prefix, and every block raises its bits
// only after its own look-back has reached that prefix.
enum { kModeRowptr = 0, kModeFill = 1, kModeFused = 2 };
// Waves per workgroup: 4 in kModeFill; 8 in the look-back modes, whose
// larger blocks halve the look-back chain (512 blocks of 400 rows on 204,800
// rows) -- the chain the last blocks wait for before they write.
template <int kMode>
struct BlockWaves {
  static constexpr int value = kMode == kModeFill ? 4 : 8;
};
// Rows per wave: 8 in kModeFill, which has no look-back and gains from many
// waves hiding each other's latencies (config 3: 44 us against 48 with 16
// and 49 with 4); 8 to 64 (at most one per lane) in the
// look-back modes, where larger blocks amortise the staging, the block scan
// and the look-back, chosen per launch so that the waves spread evenly over
// the chip's SIMDs (scan_rows_per_wave).  RowsPerWave is the maximum.
template <int kMode>
struct RowsPerWave {
  static constexpr int value = kMode == kModeFill ? 8 : 64;
};
constexpr int kMinScanRows = 8;  // fewest rows per wave of the look-back modes
constexpr int kGroup = 4;                      // rows swept together
constexpr int kMaskWords = 8;                  // mask words kept per row (512 candidates)
constexpr int kLookLanes = 4;                  // statuses per lane and look-back round
constexpr int kSpinLimit = 1 << 14;
enum {
  kOvTruncated = 1,   // a row had more than max_num_neighbors neighbours
  kOvCapacity = 2,    // edges or pairs fell past their capacity
  kOvAsymmetric = 4,  // (i, j) kept while (j, i) is excluded
  kOvLookback = 8,    // a look-back wait hit its bound (never expected)
  kOvInt32 = 16       // more than 2^31 - 1 edges or pairs
};

// Staged position record (x, y, z, unused), one 16-byte (fp32) or two
// (fp64) LDS reads.
template <typename T>
struct alignas(4 * sizeof(T)) Pos4 {
  T x, y, z, w;
};
// 16 KiB of positions per workgroup (1024 fp32 or 512 fp64 nodes).
template <typename T>
struct StageNodes {
  static constexpr int value = 16384 / (4 * (int)sizeof(T));
};

template <typename T>
__device__ __forceinline__ Vec3T<T> load_pos(const Pos4<T>* __restrict__ sp, int64_t n) {
  const Pos4<T> p = sp[n];
  return Vec3T<T>{p.x, p.y, p.z};
}

// Status word: flag (bits 62-63: 0 none, 1 aggregate, 2 inclusive prefix),
// pairs (bits 31-61), edges (bits 0-30).  Totals saturate at 2^31 - 1.
constexpr uint64_t kVal31 = 0x7fffffffull;
constexpr uint64_t kFlagAgg = 1ull << 62;
constexpr uint64_t kFlagPre = 2ull << 62;
constexpr int kStatStride = 2;  // the workspace's two status arrays interleave

__device__ __forceinline__ uint64_t pack_status(uint64_t flag, uint64_t e, uint64_t p) {
  return flag | ((p < kVal31 ? p : kVal31) << 31) | (e < kVal31 ? e : kVal31);
}
__device__ __forceinline__ uint64_t ld_status(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_status(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, MLCG_WAVE);
  return v;
}

// Decoupled look-back of block t (one full wave; statuses kStatStride words
// apart from st): publishes the aggregate,
// sums the predecessors' aggregates back to the first inclusive prefix,
// publishes the inclusive prefix and returns the exclusive one.  A round reads
// kLookLanes x 64 statuses, entry o = kLookLanes l + q (lane l, slot q) being
// block k - o; it waits only while a status before the nearest inclusive
// prefix is still missing.
__device__ __forceinline__ void lookback(uint64_t* __restrict__ st, int t, uint64_t agg_e,
                                         uint64_t agg_p, uint64_t& pre_e, uint64_t& pre_p,
                                         int& ov) {
  const int lane = mlcg_lane();
  pre_e = 0;
  pre_p = 0;
  if (t > 0) {
    if (lane == 0) st_status(st + kStatStride * t, pack_status(kFlagAgg, agg_e, agg_p));
    for (int k = t - 1;; k -= kLookLanes * MLCG_WAVE) {
      uint64_t w[kLookLanes];
#pragma unroll
      for (int q = 0; q < kLookLanes; ++q) {
        const int idx = k - kLookLanes * lane - q;
        w[q] = idx >= 0 ? ld_status(st + kStatStride * idx) : kFlagPre;
      }
      int first_pre = 0, first_missing = 0;  // in entry order, 1 << 30 when absent
      for (int spins = 0;; ++spins) {
        int fp = kLookLanes, fm = kLookLanes;  // first slot of this lane
#pragma unroll
        for (int q = kLookLanes - 1; q >= 0; --q) {
          if ((w[q] >> 62) == 2) fp = q;
          if ((w[q] >> 62) == 0) fm = q;
        }
        const uint64_t pl = __ballot(fp < kLookLanes), ml = __ballot(fm < kLookLanes);
        const int lp = pl ? __builtin_ctzll(pl) : MLCG_WAVE;
        const int lm = ml ? __builtin_ctzll(ml) : MLCG_WAVE;
        first_pre = lp < MLCG_WAVE ? kLookLanes * lp + __builtin_amdgcn_readlane(fp, lp)
                                   : (1 << 30);
        first_missing = lm < MLCG_WAVE ? kLookLanes * lm + __builtin_amdgcn_readlane(fm, lm)
                                       : (1 << 30);
        if (first_missing > first_pre || (first_missing == (1 << 30))) break;
        if (spins == kSpinLimit) {  // give up: count what is missing as zero
          ov |= kOvLookback;
#pragma unroll
          for (int q = 0; q < kLookLanes; ++q)
            if ((w[q] >> 62) == 0) w[q] = kFlagPre;
          first_missing = 1 << 30;
          first_pre = lm < MLCG_WAVE ? kLookLanes * lm + __builtin_amdgcn_readlane(fm, lm) : 0;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
#pragma unroll
        for (int q = 0; q < kLookLanes; ++q) {
          const int idx = k - kLookLanes * lane - q;
          if ((w[q] >> 62) == 0) w[q] = ld_status(st + kStatStride * idx);
        }
      }
      // sum the entries up to and including the nearest inclusive prefix
      uint64_t se = 0, sp = 0;
#pragma unroll
      for (int q = 0; q < kLookLanes; ++q) {
        const bool in = kLookLanes * lane + q <= first_pre;
        se += in ? (w[q] & kVal31) : 0;
        sp += in ? ((w[q] >> 31) & kVal31) : 0;
      }
      pre_e += wave_sum_u64(se);
      pre_p += wave_sum_u64(sp);
      if (first_pre < (1 << 30)) break;
    }
  }
  // (the inclusive prefix is stored after the loads it sums have returned)
  const uint64_t inc_e = pre_e + agg_e, inc_p = pre_p + agg_p;
  if (inc_e > kVal31 || inc_p > kVal31) ov |= kOvInt32;
  if (lane == 0) st_status(st + kStatStride * t, pack_status(kFlagPre, inc_e, inc_p));
}

__device__ __forceinline__ uint64_t readlane64(uint64_t v, int k) {
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, k);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), k);
  return ((uint64_t)hi << 32) | lo;
}
// Lanes 0 .. n - 1 (n in 0 .. 64).
__device__ __forceinline__ uint64_t low_lanes(int n) {
  return n >= MLCG_WAVE ? ~0ull : (n <= 0 ? 0ull : (1ull << n) - 1);
}

// Candidate test of lane's j against row i (centre a), every condition per
// lane: inside the row's frame, within the cutoff, not the self pair unless
// loop, not excluded.
template <bool kExcl, typename PosT, typename T>
__device__ __forceinline__ bool test_candidate(const PosT* __restrict__ P, int base, Vec3T<T> a,
                                               int i, int j, int end, T r2, int loop,
                                               const int64_t* __restrict__ exs, int64_t x_lo,
                                               int64_t x_hi) {
  const bool valid = j < end;
  const T d2 = sqdist_exact(a, load_pos(P, (valid ? j : i) - base));
  bool hit = valid && (d2 < r2) && (loop || j != i);
  if (kExcl && hit) hit = !in_sorted(exs, x_lo, x_hi, (int64_t)j);
  return hit;
}

// Per-row results of the sweep of a group.
struct GroupCounts {
  uint32_t tot[kGroup];  // kept-eligible hits (self excluded unless loop)
  uint32_t low[kGroup];  // hits with j < i
  uint32_t slf[kGroup];  // the self hit (loop only)
};

// A group's masks of one chunk: the kGroup rows are consecutive in the
// [chunk][row] mask layout, so lane 0 stores them as one 32-byte record
// straight from the ballots.
typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));
static_assert(kGroup == 4, "two 16-byte stores per group");
__device__ __forceinline__ void store_group_masks(uint64_t* __restrict__ d,
                                                  const uint64_t (&m)[kGroup]) {
  if (mlcg_lane() == 0) {
    u64x2* q = reinterpret_cast<u64x2*>(d);
    q[0] = u64x2{m[0], m[1]};
    q[1] = u64x2{m[2], m[3]};
  }
}

// Fast sweep: kGroup rows ii[] of one staged frame [st, en), no exclusions.
// Lanes past the frame read the sentinel record sp[kStage] (+inf), whose
// distance never passes the test, so no lane mask is needed; each chunk's
// candidates are read from LDS one chunk ahead.  Masks of the first
// kMaskWords chunks go to smask_g (chunk c of row u at c * kRS + u) when
// kMasks, the self bit included; the caller takes the self pair out of the
// counts.  kLow accumulates the hits below the diagonal.
template <bool kMasks, bool kLow, int kStage, int kRS, typename T>
__device__ __forceinline__ void sweep_fast(const Pos4<T>* __restrict__ sp, int base,
                                           const int (&ii)[kGroup], int st, int en, int nch,
                                           T r2, uint64_t* __restrict__ smask_g,
                                           GroupCounts& gc) {
  const int lane = mlcg_lane();
  Vec3T<T> a[kGroup];
#pragma unroll
  for (int u = 0; u < kGroup; ++u) a[u] = load_pos(sp, ii[u] - base);
  const int jend = en - base;
  int idx = st - base + lane;
  Vec3T<T> p = load_pos(sp, idx < jend ? idx : kStage);
  for (int c = 0; c < nch; ++c) {
    idx += MLCG_WAVE;
    const Vec3T<T> pn = load_pos(sp, idx < jend ? idx : kStage);  // the next chunk's
    uint64_t m[kGroup];
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      m[u] = __ballot(sqdist_exact(a[u], p) < r2);
      gc.tot[u] += (uint32_t)__popcll(m[u]);
      if (kLow) gc.low[u] += (uint32_t)__popcll(m[u] & low_lanes(ii[u] - st - MLCG_WAVE * c));
    }
    if (kMasks && c < kMaskWords) store_group_masks(smask_g + c * kRS, m);
    p = pn;
  }
}

// General sweep: any kGroup rows (candidates st[u] .. en[u]), every condition
// tested per lane; counts accumulate in scalars, masks of the first
// kMaskWords chunks go to smask_g as in sweep_fast.  With kAsym a kept (i, j)
// whose (j, i) is excluded sets asym.
template <bool kExcl, bool kMasks, bool kAsym, int kRS, typename PosT, typename T>
__device__ __forceinline__ void sweep_general(
    const PosT* __restrict__ P, int base, const int (&ii)[kGroup], const int (&st)[kGroup],
    const int (&en)[kGroup], int nch, T r2, int loop, const int64_t* __restrict__ exs,
    const int64_t* __restrict__ eptr, uint64_t* __restrict__ smask_g, GroupCounts& gc,
    bool& asym) {
  const int lane = mlcg_lane();
  Vec3T<T> a[kGroup];
  int64_t x_lo[kGroup], x_hi[kGroup];
#pragma unroll
  for (int u = 0; u < kGroup; ++u) {
    a[u] = load_pos(P, ii[u] - base);
    x_lo[u] = x_hi[u] = 0;
    if (kExcl) {
      x_lo[u] = eptr[ii[u]];
      x_hi[u] = eptr[ii[u] + 1];
    }
  }
  for (int c = 0; c < nch; ++c) {
    uint64_t mm[kGroup];
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      const int jb = st[u] + MLCG_WAVE * c;
      const int j = jb + lane;
      const bool hit =
          test_candidate<kExcl>(P, base, a[u], ii[u], j, en[u], r2, loop, exs, x_lo[u], x_hi[u]);
      if (kAsym && hit && in_sorted(exs, eptr[j], eptr[j + 1], (int64_t)ii[u])) asym = true;
      const uint64_t m = __ballot(hit);
      mm[u] = m;
      gc.tot[u] += (uint32_t)__popcll(m);
      const int d = ii[u] - jb;  // lanes below d hold j < i
      gc.low[u] += (uint32_t)__popcll(m & low_lanes(d));
      if (d >= 0 && d < MLCG_WAVE) gc.slf[u] += (uint32_t)((m >> d) & 1);
    }
    if (kMasks && c < kMaskWords) store_group_masks(smask_g + c * kRS, mm);
  }
}

// Write pass of a row whose kept neighbours all fit (no truncation, inside
// the capacities): mask w holds chunk c in lane c, self bit already cleared;
// every hit lane stores at e_base + (hits before it), and with kPairs the upper
// ones (j > i) also to the pair list.  No per-lane tests beyond the mask bit.
template <bool kPairs>
__device__ __forceinline__ void emit_row_fast(uint64_t w, int nch, int st, int i,
                                              int64_t e_base, int64_t p_base,
                                              int64_t* __restrict__ ei0,
                                              int64_t* __restrict__ ei1,
                                              int32_t* __restrict__ col,
                                              int32_t* __restrict__ pi,
                                              int32_t* __restrict__ pj,
                                              int32_t* __restrict__ eid2pair) {
  const int lane = mlcg_lane();
  const int64_t vi = (int64_t)(uint32_t)i;
  // the row's scalar bases; chunk c stores at 32-bit offsets from them
  char* const b0 = (char*)(ei0 + e_base);
  char* const b1 = (char*)(ei1 + e_base);
  char* const bc = kPairs ? (char*)(col + e_base) : nullptr;
  char* const be = kPairs ? (char*)(eid2pair + e_base) : nullptr;
  char* const bpi = kPairs ? (char*)(pi + p_base) : nullptr;
  char* const bpj = kPairs ? (char*)(pj + p_base) : nullptr;
  uint32_t e = 0, p = 0;  // edges / pairs of the row written so far
  for (int c = 0; c < nch; ++c) {
    const uint64_t m = readlane64(w, c);
    const int jb = st + MLCG_WAVE * c;
    const uint64_t um = kPairs ? m & ~low_lanes(i - jb + 1) : 0ull;  // lanes with j > i
    if (__builtin_amdgcn_inverse_ballot_w64(m)) {  // exec = the lanes of m
      const uint32_t r = e + (uint32_t)lanes_below(m);
      const uint32_t j = (uint32_t)(jb + lane);
      *(int64_t*)(b0 + r * 8u) = vi;
      *(int64_t*)(b1 + r * 8u) = (int64_t)j;
      if (kPairs) {
        *(int32_t*)(bc + r * 4u) = (int32_t)j;
        // lower edges get pair 0 here and their pair from pair_reverse_kernel
        // afterwards, so every edge of the CSR holds a valid pair id even
        // when its pair fell past the pair capacity
        int32_t pid = 0;
        if (__builtin_amdgcn_inverse_ballot_w64(um)) {
          const uint32_t rp = p + (uint32_t)lanes_below(um);
          *(int32_t*)(bpi + rp * 4u) = i;
          *(int32_t*)(bpj + rp * 4u) = (int32_t)j;
          pid = (int32_t)(p_base + rp);
        }
        *(int32_t*)(be + r * 4u) = pid;
      }
    }
    e += (uint32_t)__popcll(m);
    if (kPairs) p += (uint32_t)__popcll(um);
  }
}

// Write pass of one chunk of row i with every lane tested (rows truncated by
// max_num_neighbors or running past a capacity): kept neighbours go to edges
// e_base + kept + rank, with kPairs the upper ones also to pair
// p_base + ukept + rank among upper; a lane that falls past a capacity sets
// dropped.
template <bool kPairs>
__device__ __forceinline__ void emit_chunk(uint64_t m, int jb, int i, int mnn, int64_t e_base,
                                           int& kept, int64_t p_base, int& ukept,
                                           int64_t e_cap, int64_t* __restrict__ ei0,
                                           int64_t* __restrict__ ei1, int32_t* __restrict__ col,
                                           int64_t p_cap, int32_t* __restrict__ pi,
                                           int32_t* __restrict__ pj,
                                           int32_t* __restrict__ eid2pair, bool& dropped) {
  const int lane = mlcg_lane();
  const int j = jb + lane;
  const bool hit = (m >> lane) & 1;
  const int rank = lanes_below(m);
  const bool keep = hit && (kept + rank < mnn);
  const int64_t e = e_base + kept + rank;
  if (keep) {
    if (e >= 0 && e < e_cap) {
      ei0[e] = i;
      ei1[e] = j;
      if (kPairs) {
        col[e] = j;
        eid2pair[e] = 0;  // a valid id until the edge's own pair is known
      }
    } else {
      dropped = true;
    }
  }
  if (kPairs) {
    const bool upper = keep && (j > i);
    const uint64_t kum = __ballot(upper);
    if (upper && e >= 0 && e < e_cap) {
      const int64_t p = p_base + ukept + lanes_below(kum);
      if (p >= 0 && p < p_cap) {
        pi[p] = i;
        pj[p] = j;
        eid2pair[e] = (int32_t)p;
      } else {
        dropped = true;
      }
    }
    ukept += __popcll(kum);
  }
  kept += __popcll(m);
}

template <int kMode, bool kExcl, bool kPairs, typename T>
__global__ __launch_bounds__(BlockWaves<kMode>::value * MLCG_WAVE) void radius_rows_kernel(
    const T* __restrict__ pos, const int64_t* __restrict__ batch,
    const int64_t* __restrict__ frame_ptr, int n, T r2, int loop, int mnn,
    const int64_t* __restrict__ exs, const int64_t* __restrict__ eptr,
    int32_t* __restrict__ rowptr, int32_t* __restrict__ pairptr, int64_t e_cap,
    int64_t e_stride, int64_t* __restrict__ edge_index, int32_t* __restrict__ col,
    int64_t p_cap, int64_t p_stride, int32_t* __restrict__ pair_ij,
    int32_t* __restrict__ eid2pair, uint64_t* __restrict__ ws, int32_t* __restrict__ overflow,
    int rpw) {
  constexpr bool kScan = kMode != kModeFill;
  constexpr bool kWrite = kMode != kModeRowptr;
  constexpr int kMaxRows = RowsPerWave<kMode>::value;  // rows per wave at most
  constexpr int kRBWaves = BlockWaves<kMode>::value;
  constexpr bool kMasks = kWrite || kPairs;  // kPairs needs the lower counts from the sweep
  constexpr bool kLow = kPairs;
  constexpr int kStage = StageNodes<T>::value;
  __shared__ Pos4<T> sp[kStage + 1];  // + the sentinel record
  __shared__ __attribute__((aligned(16))) uint64_t
      smask[kMasks ? kRBWaves * kMaxRows * kMaskWords : 2];
  __shared__ int64_t swt[2 * kRBWaves];  // per-wave totals (edges, pairs), then offsets
  __shared__ uint64_t spre[2];

  // Blocks take their rows in launch order: a block only waits (look-back)
  // for blocks with a lower index, which the dispatcher started before it.
  // The wave index as a scalar (the compiler cannot prove it uniform).
  const int lane = mlcg_lane();
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / MLCG_WAVE);
  const int t = blockIdx.x;
  const int rb = kRBWaves * rpw;  // rows per block
  const int nblocks = (n + rb - 1) / rb;
  const int r0 = t * rb;
  const int r1 = r0 + rb < n ? r0 + rb : n;
  // look-back modes: the workspace header, then this launch's share of the
  // clearing of the other status array (the next launch's)
  uint64_t ws_epoch = 0, ws_mark = 0;
  if (kScan) {
    ws_epoch = ld_status(ws);
    ws_mark = ld_status(ws + 1);
    const int64_t clear = (int64_t)ws_mark > nblocks ? (int64_t)ws_mark : nblocks;
    uint64_t* other = ws + 2 + (int)((ws_epoch + 1) & 1);
    for (int64_t b = (int64_t)t * blockDim.x + threadIdx.x; b < clear;
         b += (int64_t)nblocks * blockDim.x)
      st_status(other + kStatStride * b, 0);
  }
  // the block's node window (node indices are below 2^31: int32 CSR)
  const int c_lo = (int)frame_ptr[batch[r0]];
  const int c_hi = (int)frame_ptr[batch[r1 - 1] + 1];
  const bool staged = c_hi >= c_lo && c_hi - c_lo <= kStage;  // block-uniform
  if (staged) {
    const int cnt = c_hi - c_lo;
    for (int k = threadIdx.x; k < cnt; k += blockDim.x) {
      const T* q = pos + 3 * (int64_t)(c_lo + k);
      sp[k] = Pos4<T>{q[0], q[1], q[2], T(0)};
    }
    if (threadIdx.x == 0) {
      const T inf = T(__builtin_huge_valf());
      sp[kStage] = Pos4<T>{inf, inf, inf, T(0)};
    }
  }
  // lane k of wave wv holds the scalars of row rw0 + k
  const int rw0 = r0 + wv * rpw;
  const int rwe = rw0 + rpw < r1 ? rw0 + rpw : r1;  // past the wave's last row
  int rs_start = 0, rs_end = 0, rs_e = 0, rs_p = 0;
  if (rw0 + lane < rwe) {
    const int64_t b = batch[rw0 + lane];
    rs_start = (int)frame_ptr[b];
    rs_end = (int)frame_ptr[b + 1];
    if (kMode == kModeFill) {
      rs_e = rowptr[rw0 + lane];
      if (kPairs) rs_p = pairptr[rw0 + lane];
    }
  }
  if (staged) __syncthreads();
  const int base = c_lo;

  // the self pair of each row, one row per lane: the sweep's own test of j = i
  const int my_i = rw0 + lane;
  const bool my_row = my_i < rwe;
  uint64_t selfm;
  {
    bool sh = false;
    if (my_row) {
      const Vec3T<T> a = (staged && my_i >= c_lo && my_i < c_hi) ? load_pos(sp, my_i - base)
                                                                 : load_pos(pos, my_i);
      sh = sqdist_exact(a, a) < r2;
    }
    selfm = __ballot(sh);
  }

  // sweep: chunk c of row k's mask at smask_w[c * kMaxRows + k]; per-row
  // counts to lane k
  uint64_t* smask_w = smask + (kMasks ? wv * kMaxRows * kMaskWords : 0);
  int my_tot = 0, my_low = 0, my_slf = 0;
  uint64_t fastm = 0;  // rows swept by the fast path
  bool asym = false;
  for (int g = 0; rw0 + g < rwe; g += kGroup) {
    int ii[kGroup], st[kGroup], en[kGroup];
    const bool full = rw0 + g + kGroup <= rwe;
    const int st0 = __builtin_amdgcn_readlane(rs_start, g);
    const int en0 = __builtin_amdgcn_readlane(rs_end, g);
    bool fast = false;
    if (!kExcl && full) {  // rows of one frame: the first and the last share it
      const int st3 = __builtin_amdgcn_readlane(rs_start, g + kGroup - 1);
      const int en3 = __builtin_amdgcn_readlane(rs_end, g + kGroup - 1);
      fast = staged && st0 == st3 && en0 == en3 && st0 >= c_lo && en0 <= c_hi;
    }
    GroupCounts gc;
#pragma unroll
    for (int u = 0; u < kGroup; ++u) gc.tot[u] = gc.low[u] = gc.slf[u] = 0;
    uint64_t* smask_g = smask_w + g;
    if (fast) {  // wave-uniform
#pragma unroll
      for (int u = 0; u < kGroup; ++u) ii[u] = rw0 + g + u;
      sweep_fast<kMasks, kLow, kStage, kMaxRows>(sp, base, ii, st0, en0,
                                       (en0 - st0 + MLCG_WAVE - 1) / MLCG_WAVE, r2, smask_g, gc);
      fastm |= (uint64_t)((1u << kGroup) - 1) << g;
    } else {
      int nch = 0;
      bool local = staged;
#pragma unroll
      for (int u = 0; u < kGroup; ++u) {
        ii[u] = rw0 + g + u;
        st[u] = __builtin_amdgcn_readlane(rs_start, g + u);
        en[u] = __builtin_amdgcn_readlane(rs_end, g + u);
        if (ii[u] >= rwe) {  // past the wave's last row: its first row again, ignored
          ii[u] = rw0 + g;
          st[u] = st0;
          en[u] = en0;
        }
        const int ch = (en[u] - st[u] + MLCG_WAVE - 1) / MLCG_WAVE;
        nch = ch > nch ? ch : nch;
        local = local && st[u] >= c_lo && en[u] <= c_hi && ii[u] >= c_lo && ii[u] < c_hi;
      }
      if (local)
        sweep_general<kExcl, kMasks, kExcl && kScan, kMaxRows>(
            sp, base, ii, st, en, nch, r2, loop, exs, eptr, smask_g, gc, asym);
      else
        sweep_general<kExcl, kMasks, kExcl && kScan, kMaxRows>(
            pos, 0, ii, st, en, nch, r2, loop, exs, eptr, smask_g, gc, asym);
    }
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      const bool mine = lane == g + u;
      my_tot = mine ? (int)gc.tot[u] : my_tot;
      if (kLow) my_low = mine ? (int)gc.low[u] : my_low;
      my_slf = mine ? (int)gc.slf[u] : my_slf;
    }
  }

  // per-row counts, one row per lane: the fast sweep counted the self pair
  // (and kept its mask bit); take it out of the count, and out of the mask
  // unless loop, so that the write pass sees only kept candidates
  const int my_st = rs_start, my_en = rs_end;
  const int my_nch = (my_en - my_st + MLCG_WAVE - 1) / MLCG_WAVE;
  if (my_row && (((selfm & fastm) >> lane) & 1)) {
    if (loop) {
      my_slf = 1;
    } else {
      my_tot -= 1;
      if (kMasks && my_nch <= kMaskWords) {
        const int off = my_i - my_st;
        uint64_t* wd = smask_w + (off >> 6) * kMaxRows + lane;
        *wd &= ~(1ull << (off & 63));
      }
    }
  }
  const int my_kept = my_tot < mnn ? my_tot : mnn;
  const int my_up = my_tot - my_low - my_slf;
  int my_ukept = 0;
  if (kPairs) {
    const int64_t room = (int64_t)mnn - my_low - my_slf;
    my_ukept = room <= 0 ? 0 : (int)(my_up < room ? my_up : room);
  }
  const bool trunc = __ballot(my_row && my_tot > mnn) != 0;

  // offsets: the lane's row within its wave (wave scan), the wave within the
  // block, the block within the graph (look-back)
  uint64_t pre_e = 0, pre_p = 0;  // the wave's first edge / pair
  int64_t my_off_e = 0, my_off_p = 0;
  if (kScan) {
    int ov = 0;
    const int64_t ve = my_row ? my_kept : 0, vp = my_row ? my_ukept : 0;
    const int64_t ie = wave_incl_scan64(ve), ip = wave_incl_scan64(vp);
    my_off_e = ie - ve;
    my_off_p = ip - vp;
    if (lane == MLCG_WAVE - 1) {
      swt[wv] = ie;
      swt[kRBWaves + wv] = ip;
    }
    __syncthreads();
    if (wv == 0) {
      const int64_t we = lane < kRBWaves ? swt[lane] : 0;
      const int64_t wp = lane < kRBWaves ? swt[kRBWaves + lane] : 0;
      const int64_t iwe = wave_incl_scan64(we), iwp = wave_incl_scan64(wp);
      const uint64_t agg_e = readlane64((uint64_t)iwe, kRBWaves - 1);
      const uint64_t agg_p = readlane64((uint64_t)iwp, kRBWaves - 1);
      uint64_t le, lp;
      if (t == 0 && lane == 0 && overflow) {  // done before the first prefix is published
        __hip_atomic_store(overflow, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // wait for the store itself (an agent-scope release fence would also
        // write back this XCD's L2, which the status words do not need)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      lookback(ws + 2 + (int)(ws_epoch & 1), t, agg_e, agg_p, le, lp, ov);
      if (t == nblocks - 1 && lane == 0) {  // see the workspace notes above
        st_status(ws + 1, (int64_t)ws_mark > nblocks ? ws_mark : (uint64_t)nblocks);
        st_status(ws, ws_epoch + 1);
      }
      if (lane < kRBWaves) {  // every lane read its swt entry before these writes
        swt[lane] = (int64_t)le + iwe - we;
        swt[kRBWaves + lane] = (int64_t)lp + iwp - wp;
      }
      if (lane == 0) {
        spre[0] = le + agg_e;
        spre[1] = lp + agg_p;
      }
    }
    if (trunc) ov |= kOvTruncated;
    if (__ballot(asym)) ov |= kOvAsymmetric;
    __syncthreads();
    // after wave 0's look-back, hence after block 0 cleared the overflow word
    if (ov && lane == 0 && overflow) atomicOr(overflow, ov);
    pre_e = (uint64_t)swt[wv];
    pre_p = (uint64_t)swt[kRBWaves + wv];
    // the CSR, clamped to the capacities in the fused form
    const uint64_t ecl = kMode == kModeFused ? (uint64_t)e_cap : kVal31;
    const uint64_t pcl = kMode == kModeFused ? (uint64_t)p_cap : kVal31;
    if (my_row) {
      const uint64_t oe = pre_e + my_off_e, op = pre_p + my_off_p;
      rowptr[my_i] = (int32_t)(oe < ecl ? oe : ecl);
      if (kPairs) pairptr[my_i] = (int32_t)(op < pcl ? op : pcl);
    }
    if (t == nblocks - 1 && threadIdx.x == 0) {
      rowptr[n] = (int32_t)(spre[0] < ecl ? spre[0] : ecl);
      if (kPairs) pairptr[n] = (int32_t)(spre[1] < pcl ? spre[1] : pcl);
    }
  }

  if (kWrite) {
    int64_t* ei0 = edge_index;
    int64_t* ei1 = edge_index + e_stride;
    int32_t* pi = pair_ij;
    int32_t* pj = kPairs ? pair_ij + p_stride : nullptr;
    // per-row offsets, and whether the row takes the untested path (all of it
    // kept, inside the capacities, masks kept), one row per lane
    int64_t my_e = 0, my_p = 0;
    if (kMode == kModeFill) {
      my_e = rs_e;
      my_p = rs_p;
    } else {
      my_e = (int64_t)pre_e + my_off_e;
      my_p = (int64_t)pre_p + my_off_p;
    }
    const bool my_fast = my_row && my_nch <= kMaskWords && my_tot <= mnn && my_e >= 0 &&
                         my_e + my_tot <= e_cap &&
                         (!kPairs || (my_p >= 0 && my_p + my_up <= p_cap));
    const uint64_t fastw = __ballot(my_fast);
    for (int k = 0; rw0 + k < rwe; ++k) {
      const int i = rw0 + k;
      const int st = __builtin_amdgcn_readlane(my_st, k);
      const int nch = __builtin_amdgcn_readlane(my_nch, k);
      const int64_t e_base = (int64_t)readlane64((uint64_t)my_e, k);
      const int64_t p_base = kPairs ? (int64_t)readlane64((uint64_t)my_p, k) : 0;
      if ((fastw >> k) & 1) {  // wave-uniform
        const uint64_t w = lane < nch ? smask_w[lane * kMaxRows + k] : 0ull;
        emit_row_fast<kPairs>(w, nch, st, i, e_base, p_base, ei0, ei1, col, pi, pj, eid2pair);
        continue;
      }
      // truncated, past a capacity, or longer than the kept masks
      bool dropped = false;
      int kept = 0, ukept = 0;
      if (nch <= kMaskWords) {
        const uint64_t w = lane < nch ? smask_w[lane * kMaxRows + k] : 0ull;
        for (int c = 0; c < nch && kept < mnn; ++c) {
          const uint64_t m = readlane64(w, c);
          if (m)
            emit_chunk<kPairs>(m, st + MLCG_WAVE * c, i, mnn, e_base, kept, p_base, ukept,
                               e_cap, ei0, ei1, col, p_cap, pi, pj, eid2pair, dropped);
        }
      } else {  // long row: test again, chunk by chunk
        const int en = __builtin_amdgcn_readlane(my_en, k);
        const bool loc = staged && st >= c_lo && en <= c_hi && i >= c_lo && i < c_hi;
        const Vec3T<T> a = loc ? load_pos(sp, i - base) : load_pos(pos, i);
        int64_t x_lo = 0, x_hi = 0;
        if (kExcl) {
          x_lo = eptr[i];
          x_hi = eptr[i + 1];
        }
        for (int c = 0; c < nch && kept < mnn; ++c) {
          const int jb = st + MLCG_WAVE * c;
          const bool hit =
              loc ? test_candidate<kExcl>(sp, base, a, i, jb + lane, en, r2, loop, exs, x_lo,
                                          x_hi)
                  : test_candidate<kExcl>(pos, 0, a, i, jb + lane, en, r2, loop, exs, x_lo,
                                          x_hi);
          const uint64_t m = __ballot(hit);
          if (m)
            emit_chunk<kPairs>(m, jb, i, mnn, e_base, kept, p_base, ukept, e_cap, ei0, ei1, col,
                               p_cap, pi, pj, eid2pair, dropped);
        }
      }
      if (__ballot(dropped) && lane == 0 && overflow) atomicOr(overflow, (int)kOvCapacity);
    }
  }
}

// n == 0: the CSR is the single offset 0.
__global__ void radius_empty(int32_t* rowptr, int32_t* pairptr, int32_t* overflow) {
  rowptr[0] = 0;
  if (pairptr) pairptr[0] = 0;
  if (overflow) *overflow = 0;
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

// SIMDs of the current device (4 per CU), looked up once per device.
int device_simds() {
  static std::mutex mu;
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = -1;
  std::lock_guard<std::mutex> lock(mu);
  if (dev >= 0 && cached[dev] > 0) return cached[dev];
  int cus = 0;
  if (dev < 0 || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                     hipSuccess || cus <= 0)
    cus = 256;
  if (dev >= 0) cached[dev] = 4 * cus;
  return 4 * cus;
}

// Rows per wave of the look-back modes: of 8 .. 64, the count that spreads
// the waves most evenly over the SIMDs (the largest per-SIMD load of rows is
// smallest; ties go to more rows per wave).  On 256 CUs n = 204,800 takes 50
// rows (4,096 waves, four per SIMD) and n = 17,920 takes 18 (996 waves).
int scan_rows_per_wave(int64_t n) {
  const int64_t simds = device_simds();
  int best = RowsPerWave<kModeFused>::value;
  int64_t best_load = INT64_MAX;
  for (int r = RowsPerWave<kModeFused>::value; r >= kMinScanRows; --r) {
    const int64_t waves = (n + r - 1) / r;
    const int64_t load = (waves + simds - 1) / simds * r;
    if (load < best_load) {
      best_load = load;
      best = r;
    }
  }
  return best;
}

// Launches radius_rows_kernel in `mode` (argument checks of every form).  The
// pair structures (col, pair list, its edge map) come together, with pairptr;
// they are built for float32 positions only.
template <typename T>
int launch_radius_rows(int mode, const T* pos, const int64_t* batch, const int64_t* frame_ptr,
                       int64_t n_nodes, double r, int loop, int64_t max_num_neighbors,
                       const int64_t* exclude_pair_xs, const int64_t* ptr_exclude_pair_xs,
                       int32_t* rowptr, int32_t* pairptr, int64_t edge_capacity,
                       int64_t edge_stride, int64_t* edge_index, int32_t* col,
                       int64_t pair_capacity, int64_t pair_stride, int32_t* pair_ij,
                       int32_t* eid2pair, void* workspace, int32_t* overflow, void* stream) {
  MLCG_REQUIRE(n_nodes >= 0 && n_nodes < (int64_t(1) << 31) && r >= 0.0 &&
               max_num_neighbors >= 0);
  MLCG_REQUIRE((exclude_pair_xs == nullptr) == (ptr_exclude_pair_xs == nullptr));
  MLCG_REQUIRE((col == nullptr && pair_ij == nullptr && eid2pair == nullptr) ||
               (col != nullptr && pair_ij != nullptr && eid2pair != nullptr));
  const bool pairs = pair_ij != nullptr;
  MLCG_REQUIRE(!pairs || sizeof(T) == sizeof(float));
  MLCG_REQUIRE(rowptr);
  if (mode != kModeRowptr) {
    MLCG_REQUIRE(edge_capacity >= 0 && edge_capacity < (int64_t(1) << 31) &&
                 edge_stride >= edge_capacity);
    MLCG_REQUIRE(edge_capacity == 0 || edge_index);
    MLCG_REQUIRE(!pairs || (pairptr && pair_capacity >= 0 &&
                            pair_capacity < (int64_t(1) << 31) && pair_stride >= pair_capacity));
  }
  if (mode != kModeFill) MLCG_REQUIRE(workspace);
  hipStream_t s = mlcg_stream(stream);
  if (n_nodes == 0) {
    if (mode != kModeFill) hipLaunchKernelGGL(radius_empty, dim3(1), dim3(1), 0, s, rowptr,
                                              pairptr, overflow);
    return mlcg_launch_status();
  }
  if (mode == kModeFill && edge_capacity == 0) return MLCG_OK;
  MLCG_REQUIRE(pos && batch && frame_ptr);
  const T r2 = (T)(r * r);  // r*r in double, then the scalar type (radius.cu:250)
  const int mnn = max_num_neighbors < (int64_t)INT32_MAX ? (int)max_num_neighbors : INT32_MAX;
  const int n = (int)n_nodes;
  const int rpw = mode == kModeFill ? RowsPerWave<kModeFill>::value : scan_rows_per_wave(n_nodes);
  const int bw = mode == kModeFill ? BlockWaves<kModeFill>::value : BlockWaves<kModeFused>::value;
  const int64_t rb = (int64_t)bw * rpw;
  const int64_t nblocks = (n_nodes + rb - 1) / rb;
  uint64_t* ws = static_cast<uint64_t*>(workspace);
  const dim3 grid((unsigned)nblocks), block(bw * MLCG_WAVE);
  const bool ex = exclude_pair_xs != nullptr;
#define MLCG_ROWS_LAUNCH(MODE, EX, PR)                                                      \
  hipLaunchKernelGGL((radius_rows_kernel<MODE, EX, PR, T>), grid, block, 0, s, pos, batch,  \
                     frame_ptr, n, r2, loop, mnn, EX ? exclude_pair_xs : nullptr,           \
                     EX ? ptr_exclude_pair_xs : nullptr, rowptr, pairptr, edge_capacity,    \
                     edge_stride, edge_index, col, pair_capacity, pair_stride, pair_ij,     \
                     eid2pair, ws, overflow, rpw)
  if (mode == kModeRowptr) {  // pair counts with pairptr
    if (ex && pairptr) MLCG_ROWS_LAUNCH(kModeRowptr, true, true);
    else if (ex) MLCG_ROWS_LAUNCH(kModeRowptr, true, false);
    else if (pairptr) MLCG_ROWS_LAUNCH(kModeRowptr, false, true);
    else MLCG_ROWS_LAUNCH(kModeRowptr, false, false);
  } else if (mode == kModeFill) {
    if (sizeof(T) == sizeof(float) && pairs) {
      if (ex) MLCG_ROWS_LAUNCH(kModeFill, true, (sizeof(T) == sizeof(float)));
      else MLCG_ROWS_LAUNCH(kModeFill, false, (sizeof(T) == sizeof(float)));
    } else {
      if (ex) MLCG_ROWS_LAUNCH(kModeFill, true, false);
      else MLCG_ROWS_LAUNCH(kModeFill, false, false);
    }
  } else {
    if (sizeof(T) == sizeof(float) && pairs) {
      if (ex) MLCG_ROWS_LAUNCH(kModeFused, true, (sizeof(T) == sizeof(float)));
      else MLCG_ROWS_LAUNCH(kModeFused, false, (sizeof(T) == sizeof(float)));
    } else {
      if (ex) MLCG_ROWS_LAUNCH(kModeFused, true, false);
      else MLCG_ROWS_LAUNCH(kModeFused, false, false);
    }
  }
#undef MLCG_ROWS_LAUNCH
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
  return launch_radius_rows(kModeFill, pos, batch, frame_ptr, n_nodes, r, loop,
                            max_num_neighbors, exclude_pair_xs, ptr_exclude_pair_xs,
                            const_cast<int32_t*>(rowptr), const_cast<int32_t*>(pairptr),
                            edge_capacity, edge_stride, edge_index, col, pair_capacity,
                            pair_stride, pair_ij, eid2pair, nullptr, overflow, stream);
}

extern "C" int mlcg_radius_fill_f64(const double* pos, const int64_t* batch,
                                    const int64_t* frame_ptr, int64_t n_nodes, double r,
                                    int loop, int64_t max_num_neighbors,
                                    const int64_t* exclude_pair_xs,
                                    const int64_t* ptr_exclude_pair_xs,
                                    const int32_t* rowptr, int64_t edge_capacity,
                                    int64_t edge_stride, int64_t* edge_index,
                                    int32_t* overflow, void* stream) {
  return launch_radius_rows(kModeFill, pos, batch, frame_ptr, n_nodes, r, loop,
                            max_num_neighbors, exclude_pair_xs, ptr_exclude_pair_xs,
                            const_cast<int32_t*>(rowptr), (int32_t*)nullptr, edge_capacity,
                            edge_stride, edge_index, (int32_t*)nullptr, 0, 0,
                            (int32_t*)nullptr, (int32_t*)nullptr, nullptr, overflow, stream);
}

extern "C" int64_t mlcg_radius_workspace_bytes(int64_t n_nodes) {
  if (n_nodes < 0) return 0;
  const int64_t rb = (int64_t)BlockWaves<kModeFused>::value * kMinScanRows;
  return 8 * (2 + kStatStride * ((n_nodes + rb - 1) / rb));
}

extern "C" int mlcg_radius_rowptr(const float* pos, const int64_t* batch,
                                  const int64_t* frame_ptr, int64_t n_nodes, double r, int loop,
                                  int64_t max_num_neighbors, const int64_t* exclude_pair_xs,
                                  const int64_t* ptr_exclude_pair_xs, int32_t* rowptr,
                                  int32_t* pairptr, void* workspace, int32_t* overflow,
                                  void* stream) {
  return launch_radius_rows(kModeRowptr, pos, batch, frame_ptr, n_nodes, r, loop,
                            max_num_neighbors, exclude_pair_xs, ptr_exclude_pair_xs, rowptr,
                            pairptr, 0, 0, (int64_t*)nullptr, (int32_t*)nullptr, 0, 0,
                            (int32_t*)nullptr, (int32_t*)nullptr, workspace, overflow, stream);
}

extern "C" int mlcg_radius_rowptr_f64(const double* pos, const int64_t* batch,
                                      const int64_t* frame_ptr, int64_t n_nodes, double r,
                                      int loop, int64_t max_num_neighbors,
                                      const int64_t* exclude_pair_xs,
                                      const int64_t* ptr_exclude_pair_xs, int32_t* rowptr,
                                      int32_t* pairptr, void* workspace, int32_t* overflow,
                                      void* stream) {
  return launch_radius_rows(kModeRowptr, pos, batch, frame_ptr, n_nodes, r, loop,
                            max_num_neighbors, exclude_pair_xs, ptr_exclude_pair_xs, rowptr,
                            pairptr, 0, 0, (int64_t*)nullptr, (int32_t*)nullptr, 0, 0,
                            (int32_t*)nullptr, (int32_t*)nullptr, workspace, overflow, stream);
}

extern "C" int mlcg_radius_graph(const float* pos, const int64_t* batch,
                                 const int64_t* frame_ptr, int64_t n_nodes, double r, int loop,
                                 int64_t max_num_neighbors, const int64_t* exclude_pair_xs,
                                 const int64_t* ptr_exclude_pair_xs, int32_t* rowptr,
                                 int32_t* pairptr, int64_t edge_capacity, int64_t edge_stride,
                                 int64_t* edge_index, int32_t* col, int64_t pair_capacity,
                                 int64_t pair_stride, int32_t* pair_ij, int32_t* eid2pair,
                                 void* workspace, int32_t* overflow, void* stream) {
  return launch_radius_rows(kModeFused, pos, batch, frame_ptr, n_nodes, r, loop,
                            max_num_neighbors, exclude_pair_xs, ptr_exclude_pair_xs, rowptr,
                            pairptr, edge_capacity, edge_stride, edge_index, col, pair_capacity,
                            pair_stride, pair_ij, eid2pair, workspace, overflow, stream);
}

extern "C" int mlcg_radius_graph_f64(const double* pos, const int64_t* batch,
                                     const int64_t* frame_ptr, int64_t n_nodes, double r,
                                     int loop, int64_t max_num_neighbors,
                                     const int64_t* exclude_pair_xs,
                                     const int64_t* ptr_exclude_pair_xs, int32_t* rowptr,
                                     int64_t edge_capacity, int64_t edge_stride,
                                     int64_t* edge_index, void* workspace, int32_t* overflow,
                                     void* stream) {
  return launch_radius_rows(kModeFused, pos, batch, frame_ptr, n_nodes, r, loop,
                            max_num_neighbors, exclude_pair_xs, ptr_exclude_pair_xs, rowptr,
                            (int32_t*)nullptr, edge_capacity, edge_stride, edge_index,
                            (int32_t*)nullptr, 0, 0, (int32_t*)nullptr, (int32_t*)nullptr,
                            workspace, overflow, stream);
}

// float16 / bfloat16 positions (raw 16-bit storage, [N, 3]): the sizing and
// write passes of the exact edge list, as the _f64 forms (no pair map).
#define MLCG_RADIUS_NARROW(SUFFIX, TYPE)                                                     \
  extern "C" int mlcg_radius_rowptr_##SUFFIX(                                                \
      const uint16_t* pos, const int64_t* batch, const int64_t* frame_ptr, int64_t n_nodes,  \
      double r, int loop, int64_t max_num_neighbors, const int64_t* exclude_pair_xs,         \
      const int64_t* ptr_exclude_pair_xs, int32_t* rowptr, void* workspace,                  \
      int32_t* overflow, void* stream) {                                                     \
    return launch_radius_rows(kModeRowptr, reinterpret_cast<const TYPE*>(pos), batch,        \
                              frame_ptr, n_nodes, r, loop, max_num_neighbors,                \
                              exclude_pair_xs, ptr_exclude_pair_xs, rowptr, (int32_t*)nullptr, \
                              0, 0, (int64_t*)nullptr, (int32_t*)nullptr, 0, 0,              \
                              (int32_t*)nullptr, (int32_t*)nullptr, workspace, overflow,     \
                              stream);                                                       \
  }                                                                                          \
  extern "C" int mlcg_radius_fill_##SUFFIX(                                                  \
      const uint16_t* pos, const int64_t* batch, const int64_t* frame_ptr, int64_t n_nodes,  \
      double r, int loop, int64_t max_num_neighbors, const int64_t* exclude_pair_xs,         \
      const int64_t* ptr_exclude_pair_xs, const int32_t* rowptr, int64_t edge_capacity,      \
      int64_t edge_stride, int64_t* edge_index, int32_t* overflow, void* stream) {           \
    return launch_radius_rows(kModeFill, reinterpret_cast<const TYPE*>(pos), batch,          \
                              frame_ptr, n_nodes, r, loop, max_num_neighbors,                \
                              exclude_pair_xs, ptr_exclude_pair_xs,                          \
                              const_cast<int32_t*>(rowptr), (int32_t*)nullptr, edge_capacity, \
                              edge_stride, edge_index, (int32_t*)nullptr, 0, 0,              \
                              (int32_t*)nullptr, (int32_t*)nullptr, nullptr, overflow,       \
                              stream);                                                       \
  }
MLCG_RADIUS_NARROW(f16, H16)
MLCG_RADIUS_NARROW(bf16, B16)
#undef MLCG_RADIUS_NARROW

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
