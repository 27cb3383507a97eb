// Node-level linears of the interaction blocks (gfx950, MFMA).
//
// The CFConv and interaction-block linears of SchNet (conv.lin1, conv.lin2,
// lin: mlcg/nn/schnet.py:259-261,343,347) act on [N, 128] node features with
// 128 x 128 weights.  Their products and their weight gradients run here:
//
//   node_gemm     y = x W^T or x W ([N, 128]) with the elementwise work around
//                 it fused into the store: bias, residual, the activation, or
//                 the activation's first / second derivative factors of the
//                 force and force-matching sweeps.  Products on
//                 v_mfma_f32_16x16x32_f16 with split fp32 operands (three
//                 fp16 products, fp32 accumulation; split16.h).  Persistent
//                 workgroups of 4 waves keep their 32-column slice of W in
//                 registers as two fp16 planes and stream 16-row tiles of x
//                 through LDS as three planes, each row scaled by a power of
//                 two; the tile's result passes through LDS once more so that
//                 the epilogue reads and writes whole rows with float4
//                 accesses, its inputs requested before the products.
//   node_tmm      out = a1^T b1 [+ a2^T b2] ([128, 128]): the weight
//                 gradients, a reduction over N ~ 10^4-10^5 rows on
//                 v_mfma_f32_16x16x32_bf16 with each fp32 operand split
//                 exactly into three bf16 pieces (six products).  Up to 256
//                 workgroups each reduce a contiguous range of 32-row blocks
//                 (staged in LDS column-major, the row index being the MFMA
//                 reduction axis) and write their partial; a second kernel
//                 adds the partials in a fixed order -- deterministic for a
//                 given row count.
#include "common.h"
#include "split16.h"

namespace {

constexpr int kF = 128;
// ---------------------------------------------------------------------------
// node_tmm
//
// Products on v_mfma_f32_16x16x32_bf16.  Every fp32 operand x is split
// exactly into three bf16 pieces x = hi + mid + lo, each rounded to nearest
// from the remainder of the previous one (|mid| <= 2^-8 |x|, |lo| <= 2^-16
// |x|: the remainders carry at most 16 and 8 significant bits, so every
// piece is exact).  A product x y is taken as the six terms hi hi, hi mid,
// mid hi, hi lo, lo hi, mid mid; the three left out are below 2^-23 |x y|.
// bf16 x bf16 products are exact and the MFMA accumulates them in fp32.
// bf16 has fp32's exponent range, so the operands need no scaling.
constexpr int kTmmWaves = 8;
constexpr int kTmmThreads = kTmmWaves * MLCG_WAVE;
constexpr int kTmmK = 32;                   // rows per staged block (the MFMA's K)
// bf16 per staged column: an 80-byte stride puts the 16-byte reads of the 16
// lanes of a lane group (16 consecutive columns) on disjoint banks
constexpr int kTmmCol = kTmmK + 8;
constexpr int kTmmPlane = kF * kTmmCol;     // bf16 per plane
constexpr int kTmmMat = 3 * kTmmPlane;      // hi, mid, lo planes of one matrix
constexpr int kTRow = kF + 4;               // padded LDS row (node GEMM epilogue)
constexpr int kTmmMaxGroups = 256;          // one workgroup per CU
constexpr int kTmmPart = kF * kF + kF;      // partial: out [128, 128] + column sums

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Splits eight values (consecutive rows of one column) into their hi, mid
// and lo bf16 pieces, two at a time.
__device__ __forceinline__ void tmm_split8(const float (&x)[8], bf16x8& hi, bf16x8& mid,
                                           bf16x8& lo) {
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    const floatx2 v = {x[j], x[j + 1]};
    const bf16x2 h = __builtin_convertvector(v, bf16x2);
    const floatx2 r1 = v - __builtin_convertvector(h, floatx2);
    const bf16x2 m = __builtin_convertvector(r1, bf16x2);
    const bf16x2 o = __builtin_convertvector(r1 - __builtin_convertvector(m, floatx2), bf16x2);
    hi[j] = h[0];
    hi[j + 1] = h[1];
    mid[j] = m[0];
    mid[j + 1] = m[1];
    lo[j] = o[0];
    lo[j + 1] = o[1];
  }
}

// Thread i loads rows 8 g .. 8 g + 7 (g = (i / 32) % 4) of a block, columns
// 4 (i % 32) .. + 3, of matrix i / 128 (a1, b1, a2, b2); zero past r_end.
__device__ __forceinline__ void tmm_load(float4 (&v)[8], const float* __restrict__ src,
                                         int64_t r0, int64_t r_end) {
  const int g = (threadIdx.x >> 5) & 3, c = threadIdx.x & 31;
  const float* p = src + (r0 + 8 * g) * kF + 4 * c;
  if (r0 + kTmmK <= r_end) {  // a whole block (every block but a range's last)
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = *reinterpret_cast<const float4*>(p + j * kF);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      v[j] = r0 + 8 * g + j < r_end ? *reinterpret_cast<const float4*>(p + j * kF)
                                    : float4{0.f, 0.f, 0.f, 0.f};
  }
}

// Stores a loaded 8 x 4 piece as three planes, each column's eight rows as
// one 16-byte write at [column][8 g].
__device__ __forceinline__ void tmm_stage(__bf16* mat, const float4 (&v)[8]) {
  const int g = (threadIdx.x >> 5) & 3, c = threadIdx.x & 31;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = k == 0 ? v[j].x : k == 1 ? v[j].y : k == 2 ? v[j].z : v[j].w;
    bf16x8 hi, mid, lo;
    tmm_split8(x, hi, mid, lo);
    const int o = (4 * c + k) * kTmmCol + 8 * g;
    *reinterpret_cast<bf16x8*>(mat + o) = hi;
    *reinterpret_cast<bf16x8*>(mat + kTmmPlane + o) = mid;
    *reinterpret_cast<bf16x8*>(mat + 2 * kTmmPlane + o) = lo;
  }
}

// acc[rt][ct] += a^T b over one staged block for output rows 16 (4 rg + rt)
// + .. and columns 16 (2 cg + ct) + ..: lane (q, n) supplies a's column
// 16 (4 rg + rt) + n and b's column 16 (2 cg + ct) + n, rows 8q .. 8q + 7.
__device__ __forceinline__ void tmm_accumulate(const __bf16* ma, const __bf16* mb, int rg,
                                               int cg, int q, int n, floatx4 (&acc)[4][2]) {
  bf16x8 b[2][3];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int p = 0; p < 3; ++p)
      b[ct][p] = *reinterpret_cast<const bf16x8*>(mb + p * kTmmPlane +
                                                  (16 * (2 * cg + ct) + n) * kTmmCol + 8 * q);
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) {
    bf16x8 a[3];
#pragma unroll
    for (int p = 0; p < 3; ++p)
      a[p] = *reinterpret_cast<const bf16x8*>(ma + p * kTmmPlane +
                                              (16 * (4 * rg + rt) + n) * kTmmCol + 8 * q);
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      floatx4 c = acc[rt][ct];
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[2], b[ct][0], c, 0, 0, 0);  // lo hi
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[ct][2], c, 0, 0, 0);  // hi lo
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b[ct][1], c, 0, 0, 0);  // mid mid
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b[ct][0], c, 0, 0, 0);  // mid hi
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[ct][1], c, 0, 0, 0);  // hi mid
      acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[ct][0], c, 0, 0, 0);
    }
  }
}

// Workgroup g of G reduces the 32-row blocks [g B / G, (g+1) B / G) of the
// B = ceil(rows / 32) blocks: per block, each thread loads (the next block's
// loads in flight during the products) and splits one 8 x 4 piece of one
// matrix, and wave (rg, cg) = (w / 4, w % 4) accumulates output rows
// 64 rg .. + 63 and columns 32 cg .. + 31.  Writes its partial [128, 128]
// (+ the column sums of a1, added per thread in row order and over the four
// row groups in order).
__device__ __forceinline__ void tmm_body(const float* __restrict__ a1,
                                         const float* __restrict__ b1,
                                         const float* __restrict__ a2,
                                         const float* __restrict__ b2, int64_t rows,
                                         int want_colsum, float* __restrict__ o, int64_t g,
                                         int64_t G) {
  __shared__ __align__(16) __bf16 lds[4 * kTmmMat];
  __shared__ float4 csum[4][kF / 4];
  const int w = threadIdx.x / MLCG_WAVE;
  const int l = mlcg_lane();
  const int q = l >> 4, n = l & 15;
  const int rg = w >> 2, cg = w & 3;
  const bool two = a2 != nullptr;
  const int mat = threadIdx.x >> 7;  // the matrix this thread loads
  const float* src = mat == 0 ? a1 : mat == 1 ? b1 : mat == 2 ? a2 : b2;
  const bool loads = mat < 2 || two;
  const int64_t nb = (rows + kTmmK - 1) / kTmmK;
  const int64_t r_beg = kTmmK * (nb * g / G);
  const int64_t r_stop = kTmmK * (nb * (g + 1) / G);
  const int64_t r_end = r_stop < rows ? r_stop : rows;
  floatx4 acc[4][2];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) acc[rt][0] = acc[rt][1] = floatx4{0.f, 0.f, 0.f, 0.f};
  float4 cs{0.f, 0.f, 0.f, 0.f};
  float4 v[8];
  if (loads) tmm_load(v, src, r_beg, r_end);
  for (int64_t r0 = r_beg; r0 < r_end; r0 += kTmmK) {
    if (loads) {
      tmm_stage(lds + mat * kTmmMat, v);
      if (want_colsum && mat == 0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          cs.x += v[j].x;
          cs.y += v[j].y;
          cs.z += v[j].z;
          cs.w += v[j].w;
        }
      }
    }
    __syncthreads();
    if (loads && r0 + kTmmK < r_end) tmm_load(v, src, r0 + kTmmK, r_end);
    tmm_accumulate(lds, lds + kTmmMat, rg, cg, q, n, acc);
    if (two) tmm_accumulate(lds + 2 * kTmmMat, lds + 3 * kTmmMat, rg, cg, q, n, acc);
    __syncthreads();
  }
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        o[(16 * (4 * rg + rt) + 4 * q + i) * kF + 16 * (2 * cg + ct) + n] = acc[rt][ct][i];
  if (want_colsum) {
    if (mat == 0) csum[(threadIdx.x >> 5) & 3][threadIdx.x & 31] = cs;
    __syncthreads();
    if (threadIdx.x < kF / 4) {
      float4 t = csum[0][threadIdx.x];
#pragma unroll
      for (int gg = 1; gg < 4; ++gg) {
        t.x += csum[gg][threadIdx.x].x;
        t.y += csum[gg][threadIdx.x].y;
        t.z += csum[gg][threadIdx.x].z;
        t.w += csum[gg][threadIdx.x].w;
      }
      *reinterpret_cast<float4*>(o + kF * kF + 4 * threadIdx.x) = t;
    }
  }
}

__global__ __launch_bounds__(kTmmThreads) void node_tmm_kernel(
    const float* __restrict__ a1, const float* __restrict__ b1,
    const float* __restrict__ a2, const float* __restrict__ b2, int64_t rows,
    int want_colsum, float* __restrict__ partial) {
  tmm_body(a1, b1, a2, b2, rows, want_colsum, partial + (int64_t)blockIdx.x * kTmmPart,
           blockIdx.x, gridDim.x);
}

// Up to kTmmMaxProblems independent reductions over the same number of rows
// in one launch: problem blockIdx.y, its workgroup blockIdx.x of gridDim.x,
// partials at problem * gridDim.x * kTmmPart.  Each problem's result is the
// one node_tmm_kernel gives with the same group count, bit for bit.
constexpr int kTmmMaxProblems = 4;
struct TmmProblem {
  const float* a1;
  const float* b1;
  const float* a2;
  const float* b2;
  float* out;
  float* colsum;
};
struct TmmBatch {
  TmmProblem p[kTmmMaxProblems];
};

__global__ __launch_bounds__(kTmmThreads) void node_tmm_batch_kernel(TmmBatch batch,
                                                                     int64_t rows,
                                                                     float* __restrict__ partial) {
  const TmmProblem& pr = batch.p[blockIdx.y];
  tmm_body(pr.a1, pr.b1, rows == 0 ? nullptr : pr.a2, pr.b2, rows, pr.colsum != nullptr ? 1 : 0,
           partial + ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * kTmmPart, blockIdx.x,
           gridDim.x);
}

// out (+)= sum of the `slices` partials (and colsum likewise).  A block
// covers 64 outputs with 8 waves, wave g summing the partials s = g (mod 8)
// (two interleaved accumulators); the 8 wave sums are combined in a fixed
// order.
__device__ __forceinline__ void tmm_reduce_body(const float* __restrict__ partial, int slices,
                                                int accumulate, float* __restrict__ out,
                                                float* __restrict__ colsum) {
  __shared__ float part[8][64];
  const int o = threadIdx.x & 63, g = threadIdx.x >> 6;
  const int j = blockIdx.x * 64 + o;
  float a0 = 0.f, a1 = 0.f;
  int s = g;
  for (; s + 8 < slices; s += 16) {
    a0 += partial[(int64_t)s * kTmmPart + j];
    a1 += partial[(int64_t)(s + 8) * kTmmPart + j];
  }
  if (s < slices) a0 += partial[(int64_t)s * kTmmPart + j];
  part[g][o] = a0 + a1;
  __syncthreads();
  if (g == 0) {
    const float v = ((part[0][o] + part[1][o]) + (part[2][o] + part[3][o])) +
                    ((part[4][o] + part[5][o]) + (part[6][o] + part[7][o]));
    float* dst = j < kF * kF ? out + j : colsum + (j - kF * kF);
    *dst = accumulate ? *dst + v : v;
  }
}

__global__ __launch_bounds__(512) void node_tmm_reduce_kernel(const float* __restrict__ partial,
                                                              int slices, int accumulate,
                                                              float* __restrict__ out,
                                                              float* __restrict__ colsum) {
  tmm_reduce_body(partial, slices, accumulate, out, colsum);
}

// The batch form: problem blockIdx.y; blocks past the 128 x 128 outputs of a
// problem without column sums return at once.
__global__ __launch_bounds__(512) void node_tmm_reduce_batch_kernel(
    const float* __restrict__ partial, int slices, int accumulate, TmmBatch batch) {
  const TmmProblem& pr = batch.p[blockIdx.y];
  if (pr.colsum == nullptr && blockIdx.x * 64 >= kF * kF) return;
  tmm_reduce_body(partial + (int64_t)blockIdx.y * slices * kTmmPart, slices, accumulate, pr.out,
                  pr.colsum);
}

// ---------------------------------------------------------------------------
// node_gemm
// A workgroup of 4 kRT waves computes tiles of 16 kRT rows: wave w owns the
// 32 columns 32 (w % 4) .. + 31 of the rows 16 (w / 4) .. + 15 of a tile.
// One workgroup per CU; its waves share one split copy of each weight.
template <int kRT>
struct GemmShape {
  static constexpr int kThreads = 4 * kRT * MLCG_WAVE;
  static constexpr int kRows = 16 * kRT;
  static constexpr int kPlane = kRows * kF;  // halfs per plane of a staged tile
};
constexpr int kGemmXPer = 2;  // float4 per thread of a tile: 32 per row, 16 rows per 4 waves

// Activation derivatives from the pre-activation z and the value s = act(z)
// (the same expressions as the host-side act_derivs).
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

__device__ __forceinline__ float4 ld4(const float* __restrict__ p) {
  return *reinterpret_cast<const float4*>(p);
}
__device__ __forceinline__ void st4(float* __restrict__ p, float4 v) {
  *reinterpret_cast<float4*>(p) = v;
}

// Loads tile t (zero past `rows`) as kGemmXPer float4 per thread.
template <int kRT>
__device__ __forceinline__ void gemm_load_x(float4 (&v)[kGemmXPer], const float* __restrict__ x,
                                            int64_t t, int64_t rows) {
#pragma unroll
  for (int m = 0; m < kGemmXPer; ++m) {
    const int c = threadIdx.x + m * GemmShape<kRT>::kThreads;
    const int64_t r = t * GemmShape<kRT>::kRows + (c >> 5);
    v[m] = r < rows ? ld4(x + r * kF + 4 * (c & 31)) : float4{0.f, 0.f, 0.f, 0.f};
  }
}
// Split scale of the node products: x is brought into [-4, 4) per row, so
// hi S stays below 2^13; W needs |W| < 2^15.
constexpr float kNodeS = 2048.0f;

// Stages a loaded tile: per row r, sigma_r = 2^k with max_c |x[r][c]| sigma_r
// < 4; the three planes (hi, hi S, lo S) of x sigma go to LDS as [row][128]
// halfs with 16-byte chunk j of row r stored at j ^ (r & 15), and
// 1 / (S sigma_r) to rinv[r].  The 32 lanes of a wave half hold one row.
template <int kRT>
__device__ __forceinline__ void gemm_stage_x3(_Float16* xp, float* rinv,
                                              const float4 (&v)[kGemmXPer]) {
  constexpr int kXPlane = GemmShape<kRT>::kPlane;
#pragma unroll
  for (int m = 0; m < kGemmXPer; ++m) {
    const int c = threadIdx.x + m * GemmShape<kRT>::kThreads;
    const int row = c >> 5, c4 = c & 31;
    const float4 x = v[m];
    float mx = fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
    mx = pair_row_max(row16_max(mx));
    const float sg = x3_norm(mx);
    if (c4 == 0) rinv[row] = x3_norm_inv(mx) * (1.0f / kNodeS);
    const float xv[4] = {x.x, x.y, x.z, x.w};
    halfx4 ph, phs, pl;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f16split sp = split2(xv[i] * sg, kNodeS);
      ph[i] = sp.hi;
      phs[i] = (_Float16)((float)sp.hi * kNodeS);
      pl[i] = sp.lo;
    }
    const int o = row * kF + 8 * ((c4 >> 1) ^ (row & 15)) + 4 * (c4 & 1);
    *reinterpret_cast<halfx4*>(xp + o) = ph;
    *reinterpret_cast<halfx4*>(xp + kXPlane + o) = phs;
    *reinterpret_cast<halfx4*>(xp + 2 * kXPlane + o) = pl;
  }
}

// Epilogue inputs of one float4 of the product, requested ahead of it.
struct EpiIn {
  float4 res, s, z, e, f;
};

template <int MODE>
__device__ __forceinline__ void gemm_epilogue_load(EpiIn& in, int64_t r, int col,
                                                   const float* __restrict__ residual, int act,
                                                   const float* __restrict__ zin,
                                                   const float* __restrict__ sin_,
                                                   const float* __restrict__ ein,
                                                   const float* __restrict__ fin) {
  const int64_t o = r * kF + col;
  const float4 zero{0.f, 0.f, 0.f, 0.f};
  in.res = residual ? ld4(residual + o) : zero;
  if (MODE >= MLCG_NODE_DACT) {
    in.s = ld4(sin_ + o);
    in.z = act == MLCG_ACT_TANH ? in.s : ld4(zin + o);  // tanh needs s only
    if (MODE == MLCG_NODE_DACT2 && ein) {
      in.e = ld4(ein + o);
      in.f = ld4(fin + o);
    }
  }
}

// Epilogue on one float4 of the product (row r, columns col..col+3); returns
// the value a following product takes as its input (out0 for PLAIN and DACT2,
// out1 for ACT and DACT).
template <int MODE>
__device__ __forceinline__ float4 gemm_epilogue(float4 y, int64_t r, int col, const EpiIn& in,
                                              const float* __restrict__ bias, int act,
                                              bool has_ef, float* __restrict__ out0,
                                              float* __restrict__ out1) {
  const int64_t o = r * kF + col;
  if (bias) {
    const float4 b = ld4(bias + col);
    y.x += b.x; y.y += b.y; y.z += b.z; y.w += b.w;
  }
  y.x += in.res.x; y.y += in.res.y; y.z += in.res.z; y.w += in.res.w;
  if (MODE == MLCG_NODE_PLAIN) {
    st4(out0 + o, y);
    return y;
  } else if (MODE == MLCG_NODE_ACT) {
    if (out0) st4(out0 + o, y);
    const float4 a{mlcg_act_value(act, y.x), mlcg_act_value(act, y.y),
                   mlcg_act_value(act, y.z), mlcg_act_value(act, y.w)};
    st4(out1 + o, a);
    return a;
  } else {
    const float4 s = in.s, z = in.z;
    float4 d1, d2;
    act_d1d2(act, z.x, s.x, d1.x, d2.x);
    act_d1d2(act, z.y, s.y, d1.y, d2.y);
    act_d1d2(act, z.z, s.z, d1.z, d2.z);
    act_d1d2(act, z.w, s.w, d1.w, d2.w);
    if (MODE == MLCG_NODE_DACT) {
      if (out0) st4(out0 + o, y);
      const float4 v{y.x * d1.x, y.y * d1.y, y.z * d1.z, y.w * d1.w};
      if (out1) st4(out1 + o, v);  // node_gemm2 may keep v to itself
      return v;
    } else {  // MLCG_NODE_DACT2
      float4 v{y.x * d1.x, y.y * d1.y, y.z * d1.z, y.w * d1.w};
      if (has_ef) {
        const float4 e = in.e, f = in.f;
        v.x += e.x * d2.x * f.x;
        v.y += e.y * d2.y * f.y;
        v.z += e.z * d2.z * f.z;
        v.w += e.w * d2.w * f.w;
      }
      st4(out0 + o, v);
      return v;
    }
  }
}

// B = W^T (kXW = false, torch Linear) or B = W (kXW = true) as two fp16
// planes (hi, lo S), held in registers by each wave: plane[c][kb] of lane
// (q, n) in a wave of column slice cw holds B[32 kb + 8q + j][32 cw + 16 c + n],
// j = 0..7 (the B operand layout of v_mfma_f32_16x16x32_f16).  The workgroup
// splits W once into an LDS image in exactly that order -- entry
// e = ((cw 2 + c) 4 + kb) 64 + lane holds the lane's eight halfs, hi plane
// at e, lo plane at kWImg + e -- and each wave reads its 16 entries back.
constexpr int kWImg = 4 * 2 * (kF / 32) * MLCG_WAVE;  // halfx8 entries per plane
constexpr int kWImgBytes = 2 * kWImg * 16;             // 64 KiB

// The eight weights of image entry e (see above), from W as stored.
__device__ __forceinline__ void gemm_w_entry(float (&wv)[8], const float* __restrict__ W,
                                             bool xw, int e) {
  const int l = e & 63, kb = (e >> 6) & 3, c = (e >> 8) & 1, cw = e >> 9;
  const int q = l >> 4, col = 32 * cw + 16 * c + (l & 15);
  if (xw) {
#pragma unroll
    for (int j = 0; j < 8; ++j) wv[j] = W[(32 * kb + 8 * q + j) * kF + col];
  } else {  // the eight k of an entry are contiguous in row `col` of W
    const float4 v0 = *reinterpret_cast<const float4*>(W + col * kF + 32 * kb + 8 * q);
    const float4 v1 = *reinterpret_cast<const float4*>(W + col * kF + 32 * kb + 8 * q + 4);
    wv[0] = v0.x; wv[1] = v0.y; wv[2] = v0.z; wv[3] = v0.w;
    wv[4] = v1.x; wv[5] = v1.y; wv[6] = v1.z; wv[7] = v1.w;
  }
}
__device__ __forceinline__ void gemm_w_split(const float (&wv)[8], halfx8& h, halfx8& lo) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const f16split sp = split2(wv[j], kNodeS);
    h[j] = sp.hi;
    lo[j] = sp.lo;
  }
}

template <int kRT, bool kXW>
__device__ __forceinline__ void gemm_stage_w(halfx8* img, const float* __restrict__ W) {
  constexpr int kT = GemmShape<kRT>::kThreads;
  constexpr int kIt = (kWImg + kT - 1) / kT;
  constexpr int kBatch = 2;  // entries whose loads are in flight together
#pragma unroll
  for (int i0 = 0; i0 < kIt; i0 += kBatch) {
    float wv[kBatch][8];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int e = threadIdx.x + (i0 + b) * kT;
      if (i0 + b >= kIt || (kWImg % kT != 0 && e >= kWImg)) break;
      gemm_w_entry(wv[b], W, kXW, e);
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int e = threadIdx.x + (i0 + b) * kT;
      if (i0 + b >= kIt || (kWImg % kT != 0 && e >= kWImg)) break;
      halfx8 h, lo;
      gemm_w_split(wv[b], h, lo);
      img[e] = h;
      img[kWImg + e] = lo;
    }
  }
}

// The same 16 entries loaded and split by one wave directly from W (for
// node_gemm2, whose second weight leaves no registers for a staged copy).
template <bool kXW>
__device__ __forceinline__ void gemm_load_w(halfx8 (&bh)[2][kF / 32], halfx8 (&bl)[2][kF / 32],
                                            const float* __restrict__ W, int cw, int l) {
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int kb = 0; kb < kF / 32; ++kb) {
      float wv[8];
      gemm_w_entry(wv, W, kXW, ((cw * 2 + c) * (kF / 32) + kb) * MLCG_WAVE + l);
      gemm_w_split(wv, bh[c][kb], bl[c][kb]);
    }
}

__device__ __forceinline__ void gemm_read_w(halfx8 (&bh)[2][kF / 32], halfx8 (&bl)[2][kF / 32],
                                            const halfx8* img, int cw, int l) {
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int kb = 0; kb < kF / 32; ++kb) {
      const int e = ((cw * 2 + c) * (kF / 32) + kb) * MLCG_WAVE + l;
      bh[c][kb] = img[e];
      bl[c][kb] = img[kWImg + e];
    }
}

// Split images of several weights in one launch (mlcg_node_weight_images):
// job blockIdx.y, entries blockIdx.x * 256 + threadIdx.x, the same entries and
// splits gemm_stage_w makes in LDS.
constexpr int kWImgJobs = 32;
struct WImgBatch {
  const float* W[kWImgJobs];
  halfx8* img[kWImgJobs];
  int xw[kWImgJobs];
};

__global__ __launch_bounds__(256) void node_weight_image_kernel(WImgBatch b) {
  const int job = blockIdx.y;
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= kWImg) return;
  float wv[8];
  gemm_w_entry(wv, b.W[job], b.xw[job] != 0, e);
  halfx8 h, lo;
  gemm_w_split(wv, h, lo);
  b.img[job][e] = h;
  b.img[job][kWImg + e] = lo;
}

// The product of a staged tile (three planes in xs, row scales in rinv) and
// the B planes: the 32 columns 32 cw .. of the 16 rows 16 rs .. go to ys,
// with the row scales undone.
template <int kRT>
__device__ __forceinline__ void gemm_tile(const _Float16* xs, const float* rinv,
                                          const halfx8 (&bh)[2][kF / 32],
                                          const halfx8 (&bl)[2][kF / 32], float* ys, int cw,
                                          int rs, int q, int n) {
  constexpr int kP8 = GemmShape<kRT>::kPlane / 8;
  floatx4 acc[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
  const halfx8* xv = reinterpret_cast<const halfx8*>(xs);
#pragma unroll
  for (int kb = 0; kb < kF / 32; ++kb) {
    const int o = (16 * rs + n) * (kF / 8) + ((4 * kb + q) ^ n);
    const halfx8 ah = xv[o], ahs = xv[kP8 + o], al = xv[2 * kP8 + o];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahs, bh[c][kb], acc[c], 0, 0, 0);
      acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl[c][kb], acc[c], 0, 0, 0);
      acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh[c][kb], acc[c], 0, 0, 0);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 16 * rs + 4 * q + i;
    const float u = rinv[row];
#pragma unroll
    for (int c = 0; c < 2; ++c) ys[row * kTRow + 32 * cw + 16 * c + n] = acc[c][i] * u;
  }
}

// y = x B with B = W^T (kXW = false, torch Linear) or B = W (kXW = true), on
// v_mfma_f32_16x16x32_f16 with split operands: x as three planes (staged
// per tile, scaled per row), B as two planes (hi, lo S) held in registers.
// MFMA k block kb of lane group q = l/16 covers k = 32 kb + 8q .. + 7.
// LDS: the weight image first, then (over the same bytes) the tile buffers.
template <int MODE, bool kXW, int kRT>
__global__ __launch_bounds__(GemmShape<kRT>::kThreads) void node_gemm_kernel(
    const float* __restrict__ x, int64_t rows, const float* __restrict__ W,
    const float* __restrict__ bias, const float* __restrict__ residual, int act,
    const float* __restrict__ zin, const float* __restrict__ sin_,
    const float* __restrict__ ein, const float* __restrict__ fin, float* __restrict__ out0,
    float* __restrict__ out1, const halfx8* __restrict__ wimg) {
  using S = GemmShape<kRT>;
  constexpr int kXs = 2 * 3 * S::kPlane * 2, kRinv = 2 * S::kRows * 4;
  constexpr int kBytes = kXs + kRinv + S::kRows * kTRow * 4;
  static_assert(kBytes >= kWImgBytes, "the weight image overlays the tile buffers");
  __shared__ __align__(16) unsigned char smem[kBytes];
  _Float16* const xs0 = reinterpret_cast<_Float16*>(smem);
  _Float16* const xs1 = xs0 + 3 * S::kPlane;
  float* const rinv0 = reinterpret_cast<float*>(smem + kXs);
  float* const rinv1 = rinv0 + S::kRows;
  float* const ys = reinterpret_cast<float*>(smem + kXs + kRinv);
  const int w = threadIdx.x / MLCG_WAVE;
  const int l = mlcg_lane();
  const int q = l >> 4, n = l & 15;
  const int cw = w & 3, rs = w >> 2;
  const int64_t tiles = (rows + S::kRows - 1) / S::kRows;
  // the first tile's rows are requested before the weights, so that the two
  // loads' latencies overlap
  int64_t t = blockIdx.x;
  float4 pf[kGemmXPer];
  gemm_load_x<kRT>(pf, x, t, rows);
  halfx8 bh[2][kF / 32], bl[2][kF / 32];
  if (wimg != nullptr) {  // uniform: the split image made ahead (mlcg_node_weight_images)
    gemm_read_w(bh, bl, wimg, cw, l);
  } else {
    gemm_stage_w<kRT, kXW>(reinterpret_cast<halfx8*>(smem), W);
    __syncthreads();
    gemm_read_w(bh, bl, reinterpret_cast<const halfx8*>(smem), cw, l);
    __syncthreads();
  }
  gemm_stage_x3<kRT>(xs0, rinv0, pf);
  __syncthreads();
  int buf = 0;
  for (; t < tiles; t += gridDim.x) {
    const int64_t tn = t + gridDim.x;
    const bool has_next = tn < tiles;
    if (has_next) gemm_load_x<kRT>(pf, x, tn, rows);
    // this tile's epilogue inputs, requested before the products
    EpiIn ein_[kGemmXPer];
#pragma unroll
    for (int m = 0; m < kGemmXPer; ++m) {
      const int c = threadIdx.x + m * S::kThreads;
      const int64_t r = t * S::kRows + (c >> 5);
      gemm_epilogue_load<MODE>(ein_[m], r < rows ? r : 0, 4 * (c & 31), residual, act, zin,
                               sin_, ein, fin);
    }
    gemm_tile<kRT>(buf ? xs1 : xs0, buf ? rinv1 : rinv0, bh, bl, ys, cw, rs, q, n);
    if (has_next) gemm_stage_x3<kRT>(buf ? xs0 : xs1, buf ? rinv0 : rinv1, pf);
    __syncthreads();
#pragma unroll
    for (int m = 0; m < kGemmXPer; ++m) {
      const int c = threadIdx.x + m * S::kThreads;
      const int rr = c >> 5, col = 4 * (c & 31);
      const int64_t r = t * S::kRows + rr;
      if (r < rows)
        gemm_epilogue<MODE>(ld4(ys + rr * kTRow + col), r, col, ein_[m], bias, act,
                            ein != nullptr, out0, out1);
    }
    __syncthreads();
    buf ^= 1;
  }
}

// Two consecutive node linears in one pass over the rows:
//     (out0, out1) = epilogue_MODE(x B + bias [+ residual])      as node_gemm
//     out2 = v B2 [+ bias2] [+ residual2]
// where v is the first product's principal output (out1 for ACT / DACT,
// out0 for DACT2) and B, B2 are both W^T or both W (kXW).  v is stored and
// staged from registers into a second set of planes, so each tile reads x
// once and never reads v back.  The products, scalings and epilogue
// arithmetic are those of two node_gemm_kernel launches, so the results are
// the same bit for bit.  Both B operands stay in registers (about 128 VGPRs),
// each wave loading its own slices (kRT = 1: four waves, two workgroups per
// CU; an 8-wave workgroup sharing staged weights measured slower, its
// registers spilling).
template <int MODE, bool kXW, int kRT>
__global__ __launch_bounds__(GemmShape<kRT>::kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void node_gemm2_kernel(
    const float* __restrict__ x, int64_t rows, const float* __restrict__ W,
    const float* __restrict__ bias, const float* __restrict__ residual, int act,
    const float* __restrict__ zin, const float* __restrict__ sin_,
    const float* __restrict__ ein, const float* __restrict__ fin, float* __restrict__ out0,
    float* __restrict__ out1, const float* __restrict__ W2, const float* __restrict__ bias2,
    const float* __restrict__ residual2, float* __restrict__ out2,
    const halfx8* __restrict__ wimg, const halfx8* __restrict__ w2img) {
  using S = GemmShape<kRT>;
  constexpr int kXs = 3 * 3 * S::kPlane * 2, kRinv = 3 * S::kRows * 4;
  __shared__ __align__(16) unsigned char smem[kXs + kRinv + 2 * S::kRows * kTRow * 4];
  _Float16* const xs0 = reinterpret_cast<_Float16*>(smem);
  _Float16* const xs1 = xs0 + 3 * S::kPlane;
  _Float16* const vs = xs1 + 3 * S::kPlane;
  float* const rinv0 = reinterpret_cast<float*>(smem + kXs);
  float* const rinv1 = rinv0 + S::kRows;
  float* const rinv2 = rinv1 + S::kRows;
  float* const ys0 = reinterpret_cast<float*>(smem + kXs + kRinv);
  float* const ys1 = ys0 + S::kRows * kTRow;
  const int w = threadIdx.x / MLCG_WAVE;
  const int l = mlcg_lane();
  const int q = l >> 4, n = l & 15;
  const int cw = w & 3, rs = w >> 2;
  const int64_t tiles = (rows + S::kRows - 1) / S::kRows;
  int64_t t = blockIdx.x;
  float4 pf[kGemmXPer];
  gemm_load_x<kRT>(pf, x, t, rows);
  halfx8 bh[2][kF / 32], bl[2][kF / 32], ch[2][kF / 32], cl[2][kF / 32];
  if (wimg != nullptr)
    gemm_read_w(bh, bl, wimg, cw, l);
  else
    gemm_load_w<kXW>(bh, bl, W, cw, l);
  if (w2img != nullptr)
    gemm_read_w(ch, cl, w2img, cw, l);
  else
    gemm_load_w<kXW>(ch, cl, W2, cw, l);
  gemm_stage_x3<kRT>(xs0, rinv0, pf);
  __syncthreads();
  int buf = 0;
  // LDS reuse across iterations: xs[buf] and ys0 are last read before the
  // second barrier of an iteration, vs and ys1 before the third, and each
  // is next written after at least one further barrier.
  for (; t < tiles; t += gridDim.x) {
    const int64_t tn = t + gridDim.x;
    const bool has_next = tn < tiles;
    if (has_next) gemm_load_x<kRT>(pf, x, tn, rows);
    EpiIn ein_[kGemmXPer];
    float4 res2[kGemmXPer];
#pragma unroll
    for (int m = 0; m < kGemmXPer; ++m) {
      const int c = threadIdx.x + m * S::kThreads;
      const int64_t r = t * S::kRows + (c >> 5);
      const int64_t rr = r < rows ? r : 0;
      gemm_epilogue_load<MODE>(ein_[m], rr, 4 * (c & 31), residual, act, zin, sin_, ein, fin);
      res2[m] = residual2 ? ld4(residual2 + rr * kF + 4 * (c & 31)) : float4{0.f, 0.f, 0.f, 0.f};
    }
    gemm_tile<kRT>(buf ? xs1 : xs0, buf ? rinv1 : rinv0, bh, bl, ys0, cw, rs, q, n);
    if (has_next) gemm_stage_x3<kRT>(buf ? xs0 : xs1, buf ? rinv0 : rinv1, pf);
    __syncthreads();
    float4 v[kGemmXPer];
#pragma unroll
    for (int m = 0; m < kGemmXPer; ++m) {
      const int c = threadIdx.x + m * S::kThreads;
      const int rr = c >> 5, col = 4 * (c & 31);
      const int64_t r = t * S::kRows + rr;
      v[m] = float4{0.f, 0.f, 0.f, 0.f};  // rows past the end enter the product as zeros
      if (r < rows)
        v[m] = gemm_epilogue<MODE>(ld4(ys0 + rr * kTRow + col), r, col, ein_[m], bias, act,
                                   ein != nullptr, out0, out1);
    }
    gemm_stage_x3<kRT>(vs, rinv2, v);
    __syncthreads();
    gemm_tile<kRT>(vs, rinv2, ch, cl, ys1, cw, rs, q, n);
    __syncthreads();
#pragma unroll
    for (int m = 0; m < kGemmXPer; ++m) {
      const int c = threadIdx.x + m * S::kThreads;
      const int rr = c >> 5, col = 4 * (c & 31);
      const int64_t r = t * S::kRows + rr;
      if (r < rows) {
        EpiIn e2;
        e2.res = res2[m];
        gemm_epilogue<MLCG_NODE_PLAIN>(ld4(ys1 + rr * kTRow + col), r, col, e2, bias2, act,
                                       false, out2, nullptr);
      }
    }
    buf ^= 1;
  }
}

// ---------------------------------------------------------------------------
// Embedding lookup: out[i][:] = table[types[i]][:] for [T, 128] fp32 tables
// (schnet.py:132, `x = self.embedding_layer(data.atom_types)`): 32 lanes per
// row, one float4 each, grid-stride.  A type outside [0, T) writes a zero row
// and raises bit 2 of the numerics flag word (when its address is known).
__global__ __launch_bounds__(256) void embedding_gather_kernel(
    const float4* __restrict__ table, int T, const int64_t* __restrict__ types, int64_t n,
    float4* __restrict__ out, unsigned* flags) {
  const int64_t total = n * (kF / 4);
  for (int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x; k < total;
       k += (int64_t)gridDim.x * 256) {
    const int64_t r = k / (kF / 4);
    const int c = (int)(k % (kF / 4));
    const int64_t t = types[r];
    float4 v{0.f, 0.f, 0.f, 0.f};
    if (t >= 0 && t < T)
      v = table[t * (kF / 4) + c];
    else if (c == 0 && flags)
      atomicOr(flags, kFlagTypeRange);
    out[k] = v;
  }
}

// ---------------------------------------------------------------------------
// type_sum: out[t][:] = sum of the rows x[n][:] with types[n] == t, for
// t < T <= 128 -- the gradient of an embedding table.  One workgroup per
// type t walks the rows in chunks: its waves find the rows of type t
// (ballot, in ascending row order) and list them in LDS, then the rows are
// summed column by column, slot h of the eight slots per column taking the
// listed rows h, h + 8, ... in order with a compensated (Kahan) sum, and the
// slots are added in order at the end.  With many rows the chunks are shared
// among G workgroups per type (blockIdx.y = g takes the chunks g, g + G, ...),
// each writing its compensated column sums to a partial table that
// type_sum_combine_kernel adds in group order; with one chunk G = 1 and the
// workgroup writes the result itself.  No atomics: the result is the same on
// every run, and each row of x is read once in total.
constexpr int kTypeMax = 128;
constexpr int kTypeThreads = 1024;
constexpr int kTypeWaves = kTypeThreads / MLCG_WAVE;
constexpr int kTypeSteps = 24;  // 64-row steps per wave and chunk
constexpr int kTypeWaveRows = kTypeSteps * MLCG_WAVE;
constexpr int kTypeChunk = kTypeWaves * kTypeWaveRows;  // 24576 rows
constexpr int kTypeSlots = kTypeThreads / kF;           // partial sums per column
constexpr int kTypeBatch = 24;                          // row loads in flight per thread

__global__ __launch_bounds__(kTypeThreads) void type_sum_kernel(const float* __restrict__ x,
                                                                 const int64_t* __restrict__ types,
                                                                 int64_t rows, int T,
                                                                 float* __restrict__ out,
                                                                 int* __restrict__ bad,
                                                                 unsigned* __restrict__ flags,
                                                                 float* __restrict__ partial) {
  __shared__ int list[kTypeChunk];  // the chunk's matches in ascending row order
  __shared__ int cnt[kTypeWaves];
  __shared__ float red[kTypeSlots][kF], red2[kTypeSlots][kF];
  const int t = blockIdx.x;
  const int g = blockIdx.y, G = gridDim.y;
  const int w = threadIdx.x / MLCG_WAVE, l = mlcg_lane();
  const int c = threadIdx.x % kF, h = threadIdx.x / kF;
  const uint64_t below = (l == 0) ? 0ull : (~0ull >> (MLCG_WAVE - l));  // lanes < l
  float acc = 0.f, comp = 0.f;  // running sum and its lost low-order part
  for (int64_t r0 = (int64_t)g * kTypeChunk; r0 < rows; r0 += (int64_t)G * kTypeChunk) {
    const int64_t base = r0 + (int64_t)w * kTypeWaveRows;
    int64_t tt[kTypeSteps];
#pragma unroll
    for (int i = 0; i < kTypeSteps; ++i) {
      const int64_t r = base + MLCG_WAVE * i + l;
      tt[i] = r < rows ? types[r] : -1;
    }
    // count this wave's matches, then (with every wave's count known) list
    // them at the wave's offset; rows past the end have tt = -1, never t
    int n = 0;
#pragma unroll
    for (int i = 0; i < kTypeSteps; ++i) {
      // an out-of-table type is flagged (by workgroup 0: in bad, or without
      // one in bit 2 of the numerics flags) and summed nowhere
      if (t == 0 && base + MLCG_WAVE * i + l < rows && (tt[i] < 0 || tt[i] >= T)) {
        if (bad)
          bad[0] = 1;
        else
          atomicOr(flags, kFlagTypeRange);
      }
      n += __popcll(__ballot(tt[i] == t));
    }
    if (l == 0) cnt[w] = n;
    __syncthreads();
    int off = 0, total = 0;
#pragma unroll
    for (int v = 0; v < kTypeWaves; ++v) {
      const int cv = cnt[v];
      off += v < w ? cv : 0;
      total += cv;
    }
#pragma unroll
    for (int i = 0; i < kTypeSteps; ++i) {
      const bool m = tt[i] == t;
      const uint64_t bal = __ballot(m);
      if (m) list[off + __popcll(bal & below)] = (int)(base + MLCG_WAVE * i + l - r0);
      off += __popcll(bal);
    }
    __syncthreads();
    for (int m0 = h; m0 < total; m0 += kTypeSlots * kTypeBatch) {
      float xv[kTypeBatch];
#pragma unroll
      for (int u = 0; u < kTypeBatch; ++u) {
        const int m = m0 + u * kTypeSlots;
        xv[u] = m < total ? x[(r0 + list[m]) * kF + c] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < kTypeBatch; ++u)
        if (m0 + u * kTypeSlots < total) {
          const float yv = xv[u] - comp;
          const float tv = acc + yv;
          comp = (tv - acc) - yv;
          acc = tv;
        }
    }
    __syncthreads();  // list and cnt are rewritten by the next chunk
  }
  red[h][c] = acc;
  red2[h][c] = comp;
  __syncthreads();
  if (h == 0) {
    float sum = 0.f, cs = 0.f;
#pragma unroll
    for (int v = 0; v < kTypeSlots; ++v) {
      const float yv = red[v][c] - (cs + red2[v][c]);
      const float tv = sum + yv;
      cs = (tv - sum) - yv;
      sum = tv;
    }
    if (G == 1) {
      out[(int64_t)t * kF + c] = sum;
    } else {  // the group's sum and its lost low-order part
      float* pg = partial + ((int64_t)g * T + t) * 2 * kF;
      pg[c] = sum;
      pg[kF + c] = cs;
    }
  }
}

// out[t][c] = the G groups' partial sums of type t, added in group order with
// their low-order parts (compensated).
__global__ __launch_bounds__(kF) void type_sum_combine_kernel(const float* __restrict__ partial,
                                                              int G, int T,
                                                              float* __restrict__ out) {
  const int t = blockIdx.x, c = threadIdx.x;
  float sum = 0.f, cs = 0.f;
  for (int g = 0; g < G; ++g) {
    const float* pg = partial + ((int64_t)g * T + t) * 2 * kF;
    const float yv = pg[c] - (cs + pg[kF + c]);
    const float tv = sum + yv;
    cs = (tv - sum) - yv;
    sum = tv;
  }
  out[(int64_t)t * kF + c] = sum;
}

// Workgroups per type: enough to give the chip about 256 workgroups, at most
// one per chunk of rows.
int type_groups(int64_t rows, int T) {
  const int64_t chunks = rows <= 0 ? 1 : (rows + kTypeChunk - 1) / kTypeChunk;
  const int64_t want = (256 + T - 1) / T;
  const int64_t g = chunks < want ? chunks : want;
  return (int)(g < 1 ? 1 : (g > 64 ? 64 : g));
}

int tmm_groups(int64_t rows) {
  const int64_t blocks = rows == 0 ? 1 : (rows + kTmmK - 1) / kTmmK;
  return (int)(blocks < kTmmMaxGroups ? blocks : kTmmMaxGroups);
}

// Row subtiles per node_gemm workgroup: 12 waves (3 per SIMD, at most 168
// VGPRs) where the epilogue fits, else 8.
template <int MODE>
struct GemmRT {
  static constexpr int value = MODE == MLCG_NODE_DACT2 ? 2 : 3;
};
template <int kRT>
int64_t gemm_tiles(int64_t rows) {
  return (rows + GemmShape<kRT>::kRows - 1) / GemmShape<kRT>::kRows;
}

template <int MODE>
void launch_node_gemm(bool xw, hipStream_t s, const float* x, int64_t rows,
                      const float* W, const float* bias, const float* residual, int act,
                      const float* z, const float* sv, const float* e, const float* f,
                      float* out0, float* out1, const halfx8* wimg) {
  constexpr int kRT = GemmRT<MODE>::value;
  const dim3 grid(mlcg_persistent_groups(gemm_tiles<kRT>(rows), 1));
  const dim3 block(GemmShape<kRT>::kThreads);
  if (xw)
    hipLaunchKernelGGL((node_gemm_kernel<MODE, true, kRT>), grid, block, 0, s, x, rows, W, bias,
                       residual, act, z, sv, e, f, out0, out1, wimg);
  else
    hipLaunchKernelGGL((node_gemm_kernel<MODE, false, kRT>), grid, block, 0, s, x, rows, W, bias,
                       residual, act, z, sv, e, f, out0, out1, wimg);
}

template <int MODE>
void launch_node_gemm2(bool xw, hipStream_t s, const float* x, int64_t rows,
                       const float* W, const float* bias, const float* residual, int act,
                       const float* z, const float* sv, const float* e, const float* f,
                       float* out0, float* out1, const float* W2, const float* bias2,
                       const float* residual2, float* out2, const halfx8* wimg,
                       const halfx8* w2img) {
  constexpr int kRT = 1;  // both weights in registers: ~240 VGPRs, two workgroups per CU
  const dim3 grid(mlcg_persistent_groups(gemm_tiles<kRT>(rows), 2));
  const dim3 block(GemmShape<kRT>::kThreads);
  if (xw)
    hipLaunchKernelGGL((node_gemm2_kernel<MODE, true, kRT>), grid, block, 0, s, x, rows, W,
                       bias, residual, act, z, sv, e, f, out0, out1, W2, bias2, residual2, out2,
                       wimg, w2img);
  else
    hipLaunchKernelGGL((node_gemm2_kernel<MODE, false, kRT>), grid, block, 0, s, x, rows, W,
                       bias, residual, act, z, sv, e, f, out0, out1, W2, bias2, residual2, out2,
                       wimg, w2img);
}

// Argument checks shared by mlcg_node_gemm and mlcg_node_gemm2.
int check_node_gemm(const float* x, int64_t rows, const float* W, int epilogue, int act,
                    const float* z, const float* s, const float* e, const float* f,
                    const float* out0, const float* out1, bool out1_optional = false) {
  MLCG_REQUIRE(rows >= 0 && (act == MLCG_ACT_TANH || act == MLCG_ACT_SSP));
  MLCG_REQUIRE((e == nullptr) == (f == nullptr));
  MLCG_REQUIRE(epilogue >= MLCG_NODE_PLAIN && epilogue <= MLCG_NODE_DACT2);
  if (rows == 0) return MLCG_OK;
  switch (epilogue) {
    case MLCG_NODE_PLAIN: MLCG_REQUIRE(out0 != nullptr); break;
    case MLCG_NODE_ACT: MLCG_REQUIRE(out1 != nullptr); break;
    case MLCG_NODE_DACT:
      MLCG_REQUIRE((out1 || out1_optional) && s && (z || act == MLCG_ACT_TANH));
      break;
    case MLCG_NODE_DACT2: MLCG_REQUIRE(out0 && s && (z || act == MLCG_ACT_TANH)); break;
    default: break;
  }
  MLCG_REQUIRE(x && W);
  return MLCG_OK;
}

}  // namespace

extern "C" int mlcg_node_gemm(const float* x, int64_t rows, int features, const float* W,
                              int transpose_w, const float* bias, const float* residual,
                              int epilogue, int act, const float* z, const float* s,
                              const float* e, const float* f, float* out0, float* out1,
                              const void* w_image, void* stream) {
  if (features != kF) return MLCG_ERR_UNSUPPORTED;
  const int rc = check_node_gemm(x, rows, W, epilogue, act, z, s, e, f, out0, out1);
  if (rc != MLCG_OK || rows == 0) return rc;
  MLCG_REQUIRE(reinterpret_cast<uintptr_t>(w_image) % 16 == 0);
  hipStream_t st = mlcg_stream(stream);
  const bool xw = transpose_w != 0;
  const halfx8* wi = static_cast<const halfx8*>(w_image);
  switch (epilogue) {
    case MLCG_NODE_PLAIN:
      launch_node_gemm<MLCG_NODE_PLAIN>(xw, st, x, rows, W, bias, residual, act, z, s, e,
                                        f, out0, out1, wi);
      break;
    case MLCG_NODE_ACT:
      launch_node_gemm<MLCG_NODE_ACT>(xw, st, x, rows, W, bias, residual, act, z, s, e, f,
                                      out0, out1, wi);
      break;
    case MLCG_NODE_DACT:
      launch_node_gemm<MLCG_NODE_DACT>(xw, st, x, rows, W, bias, residual, act, z, s, e,
                                       f, out0, out1, wi);
      break;
    default:
      launch_node_gemm<MLCG_NODE_DACT2>(xw, st, x, rows, W, bias, residual, act, z, s, e,
                                        f, out0, out1, wi);
      break;
  }
  return mlcg_launch_status();
}

extern "C" int mlcg_node_gemm2(const float* x, int64_t rows, int features, const float* W,
                               int transpose_w, const float* bias, const float* residual,
                               int epilogue, int act, const float* z, const float* s,
                               const float* e, const float* f, float* out0, float* out1,
                               const float* W2, const float* bias2, const float* residual2,
                               float* out2, const void* w_image, const void* w2_image,
                               void* stream) {
  if (features != kF) return MLCG_ERR_UNSUPPORTED;
  MLCG_REQUIRE(epilogue != MLCG_NODE_PLAIN);
  // the DACT form's v (out1) feeds the second product from registers, so a
  // caller that needs only out2 may pass out1 = NULL
  const int rc = check_node_gemm(x, rows, W, epilogue, act, z, s, e, f, out0, out1, true);
  if (rc != MLCG_OK || rows == 0) return rc;
  MLCG_REQUIRE(W2 && out2);
  MLCG_REQUIRE(reinterpret_cast<uintptr_t>(w_image) % 16 == 0 &&
               reinterpret_cast<uintptr_t>(w2_image) % 16 == 0);
  hipStream_t st = mlcg_stream(stream);
  const bool xw = transpose_w != 0;
  const halfx8* wi = static_cast<const halfx8*>(w_image);
  const halfx8* w2i = static_cast<const halfx8*>(w2_image);
  switch (epilogue) {
    case MLCG_NODE_ACT:
      launch_node_gemm2<MLCG_NODE_ACT>(xw, st, x, rows, W, bias, residual, act, z, s, e,
                                       f, out0, out1, W2, bias2, residual2, out2, wi, w2i);
      break;
    case MLCG_NODE_DACT:
      launch_node_gemm2<MLCG_NODE_DACT>(xw, st, x, rows, W, bias, residual, act, z, s, e,
                                        f, out0, out1, W2, bias2, residual2, out2, wi, w2i);
      break;
    default:
      launch_node_gemm2<MLCG_NODE_DACT2>(xw, st, x, rows, W, bias, residual, act, z, s,
                                         e, f, out0, out1, W2, bias2, residual2, out2, wi,
                                         w2i);
      break;
  }
  return mlcg_launch_status();
}

extern "C" int64_t mlcg_node_weight_image_bytes(void) { return kWImgBytes; }

extern "C" int mlcg_node_weight_images(const float* const* weights, const int* transpose_w,
                                       int count, void* images, void* stream) {
  MLCG_REQUIRE(count >= 0 && (count == 0 || (weights && transpose_w && images)));
  if (count > kWImgJobs) return MLCG_ERR_UNSUPPORTED;
  if (count == 0) return MLCG_OK;
  MLCG_REQUIRE(reinterpret_cast<uintptr_t>(images) % 16 == 0);
  WImgBatch b{};
  for (int k = 0; k < count; ++k) {
    MLCG_REQUIRE(weights[k] != nullptr && reinterpret_cast<uintptr_t>(weights[k]) % 16 == 0);
    b.W[k] = weights[k];
    b.img[k] = reinterpret_cast<halfx8*>(static_cast<char*>(images) + (int64_t)k * kWImgBytes);
    b.xw[k] = transpose_w[k] != 0;
  }
  hipLaunchKernelGGL(node_weight_image_kernel, dim3(kWImg / 256, (unsigned)count), dim3(256), 0,
                     mlcg_stream(stream), b);
  return mlcg_launch_status();
}

extern "C" int64_t mlcg_node_tmm_workspace_floats(int64_t rows) {
  if (rows < 0) return -1;
  return (int64_t)tmm_groups(rows) * kTmmPart;
}

extern "C" int mlcg_node_tmm(const float* a1, const float* b1, const float* a2,
                             const float* b2, int64_t rows, int features, int accumulate,
                             float* out, float* colsum_a1, float* workspace,
                             int64_t workspace_floats, void* stream) {
  if (features != kF) return MLCG_ERR_UNSUPPORTED;
  MLCG_REQUIRE(rows >= 0 && out && workspace);
  MLCG_REQUIRE(rows == 0 || (a1 && b1));
  MLCG_REQUIRE((a2 == nullptr) == (b2 == nullptr));
  const int groups = tmm_groups(rows);
  MLCG_REQUIRE(workspace_floats >= (int64_t)groups * kTmmPart);
  hipStream_t s = mlcg_stream(stream);
  hipLaunchKernelGGL(node_tmm_kernel, dim3((unsigned)groups), dim3(kTmmThreads), 0, s, a1, b1,
                     rows == 0 ? nullptr : a2, b2, rows, colsum_a1 != nullptr ? 1 : 0,
                     workspace);
  const int outs = kF * kF + (colsum_a1 ? kF : 0);
  hipLaunchKernelGGL(node_tmm_reduce_kernel, dim3(outs / 64), dim3(512), 0, s, workspace, groups,
                     accumulate, out, colsum_a1);
  return mlcg_launch_status();
}

// Workgroups per problem of the batch form: together about one per CU, but
// at most 16 row blocks per workgroup while the count stays within
// kTmmMaxGroups (the fp32 accumulation error grows with the rows each
// workgroup sums; 16 blocks is what the single form reaches at ~128k rows).
int tmm_batch_groups(int64_t rows, int count) {
  const int64_t blocks = rows == 0 ? 1 : (rows + kTmmK - 1) / kTmmK;
  int64_t want = kTmmMaxGroups / (count < 1 ? 1 : count);
  const int64_t by_depth = (blocks + 15) / 16;
  if (by_depth > want) want = by_depth < kTmmMaxGroups ? by_depth : kTmmMaxGroups;
  return (int)(blocks < want ? blocks : want);
}

extern "C" int64_t mlcg_node_tmm_batch_workspace_floats(int64_t rows, int count) {
  if (rows < 0 || count < 1 || count > kTmmMaxProblems) return -1;
  return (int64_t)count * tmm_batch_groups(rows, count) * kTmmPart;
}

extern "C" int mlcg_node_tmm_batch(const void* const* problems, int count, int64_t rows,
                                   int features, int accumulate, float* workspace,
                                   int64_t workspace_floats, void* stream) {
  if (features != kF) return MLCG_ERR_UNSUPPORTED;
  MLCG_REQUIRE(problems && count >= 1 && count <= kTmmMaxProblems && rows >= 0 && workspace);
  TmmBatch batch{};
  for (int k = 0; k < count; ++k) {
    const void* const* e = problems + 6 * k;
    TmmProblem& pr = batch.p[k];
    pr.a1 = static_cast<const float*>(e[0]);
    pr.b1 = static_cast<const float*>(e[1]);
    pr.a2 = static_cast<const float*>(e[2]);
    pr.b2 = static_cast<const float*>(e[3]);
    pr.out = static_cast<float*>(const_cast<void*>(e[4]));
    pr.colsum = static_cast<float*>(const_cast<void*>(e[5]));
    MLCG_REQUIRE(pr.out && (rows == 0 || (pr.a1 && pr.b1)));
    MLCG_REQUIRE((pr.a2 == nullptr) == (pr.b2 == nullptr));
  }
  const int groups = tmm_batch_groups(rows, count);
  MLCG_REQUIRE(workspace_floats >= (int64_t)count * groups * kTmmPart);
  hipStream_t s = mlcg_stream(stream);
  hipLaunchKernelGGL(node_tmm_batch_kernel, dim3((unsigned)groups, (unsigned)count),
                     dim3(kTmmThreads), 0, s, batch, rows, workspace);
  hipLaunchKernelGGL(node_tmm_reduce_batch_kernel, dim3((kF * kF + kF) / 64, (unsigned)count),
                     dim3(512), 0, s, workspace, groups, accumulate, batch);
  return mlcg_launch_status();
}

extern "C" int mlcg_embedding_gather(const float* table, int num_types, int features,
                                     const int64_t* types, int64_t n, float* out,
                                     void* stream) {
  if (features != kF) return MLCG_ERR_UNSUPPORTED;
  MLCG_REQUIRE(n >= 0 && num_types >= 1);
  if (n == 0) return MLCG_OK;
  MLCG_REQUIRE(table && types && out);
  MLCG_REQUIRE(reinterpret_cast<uintptr_t>(table) % 16 == 0 &&
               reinterpret_cast<uintptr_t>(out) % 16 == 0);
  unsigned* const flags = mlcg_numerics_word_ptr();
  if (flags == nullptr) return MLCG_ERR_LAUNCH;  // the flag word's address is unknown
  const unsigned groups = mlcg_persistent_groups(mlcg_div_up(n * (kF / 4), 256), 16);
  hipLaunchKernelGGL(embedding_gather_kernel, dim3(groups), dim3(256), 0, mlcg_stream(stream),
                     reinterpret_cast<const float4*>(table), num_types, types, n,
                     reinterpret_cast<float4*>(out), flags);
  return mlcg_launch_status();
}

extern "C" int64_t mlcg_type_sum_workspace_floats(int64_t rows, int num_types) {
  if (rows < 0 || num_types < 1 || num_types > kTypeMax) return -1;
  const int G = type_groups(rows, num_types);
  return G == 1 ? 0 : (int64_t)2 * G * num_types * kF;  // the groups' partial sums
}

extern "C" int mlcg_type_sum(const float* x, const int64_t* types, int64_t rows, int features,
                             int num_types, float* out, int* bad, float* workspace,
                             int64_t workspace_floats, void* stream) {
  if (features != kF) return MLCG_ERR_UNSUPPORTED;
  if (num_types > kTypeMax) return MLCG_ERR_UNSUPPORTED;
  MLCG_REQUIRE(rows >= 0 && num_types >= 1 && out);
  MLCG_REQUIRE(rows == 0 || (x && types));
  const int G = type_groups(rows, num_types);
  const int64_t need = G == 1 ? 0 : (int64_t)2 * G * num_types * kF;
  MLCG_REQUIRE(workspace_floats >= need && (need == 0 || workspace));
  unsigned* const flags = bad ? nullptr : mlcg_numerics_word_ptr();
  if (bad == nullptr && flags == nullptr) return MLCG_ERR_LAUNCH;
  hipLaunchKernelGGL(type_sum_kernel, dim3((unsigned)num_types, (unsigned)G), dim3(kTypeThreads),
                     0, mlcg_stream(stream), x, types, rows, num_types, out, bad, flags,
                     workspace);
  if (G > 1)
    hipLaunchKernelGGL(type_sum_combine_kernel, dim3((unsigned)num_types), dim3(kF), 0,
                       mlcg_stream(stream), workspace, G, num_types, out);
  return mlcg_launch_status();
}
