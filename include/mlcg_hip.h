/*
 * mlcg_hip.h -- C ABI of libmlcg_hip.so, the gfx950 implementation of the
 * mlcg SchNet/CFConv hot path (radius graph, Gaussian-RBF filter network,
 * CFConv gather/scatter with its force backward and force-matching double
 * backward, bonded and repulsion priors, Langevin BAOAB).
 *
 * Conventions (shared by every entry point):
 *   - all array arguments are device pointers, row-major and contiguous;
 *   - `stream` is a hipStream_t passed as void*; work is enqueued on it and
 *     nothing synchronises with the host;
 *   - nothing allocates device memory: callers pass outputs and workspaces;
 *   - the return value is an mlcg_status; a non-zero value means nothing
 *     useful was written.  MLCG_ERR_ARGUMENT is returned before any launch.
 *   - "pair" = unordered neighbour pair {i, j} with i < j; the pair list is
 *     the upper triangle of the canonically sorted (i asc, j asc) edge list.
 *   - functions that take `n_pairs_dev` read the live pair count from device
 *     memory, so a launch sized by a capacity can be captured in a hipGraph.
 *
 * Each declaration names the reference interface it replaces
 * (paths relative to the ClementiGroup/mlcg checkout).
 */
#ifndef MLCG_HIP_H
#define MLCG_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  MLCG_OK = 0,
  MLCG_ERR_ARGUMENT = 1,
  MLCG_ERR_LAUNCH = 2,
  MLCG_ERR_CAPACITY = 3,
  MLCG_ERR_UNSUPPORTED = 4
} mlcg_status;

/* Library identification: returns a static string (build id + arch). */
const char* mlcg_version(void);

/* ---------------------------------------------------------------------- */
/* Radius graph                                                            */
/* ---------------------------------------------------------------------- */

/* frame_ptr[b] = first node of frame b, frame_ptr[n_frames] = n_nodes, from a
 * sorted `batch` vector.  Replaces the torch.bucketize call of
 * src/opt_radius/mlcg_opt_radius/radius.py:72-75. */
int mlcg_frame_ptr_from_batch(const int64_t* batch, int64_t n_nodes,
                              int64_t n_frames, int64_t* frame_ptr,
                              void* stream);

/* Pass 1 of the radius graph: per-node neighbour counts.
 * Edge (i, j) exists iff batch[i] == batch[j], (loop || i != j),
 * d2 < fl32(r*r), d2 = ((dx*dx + dy*dy) + dz*dz) in fp32 without FMA
 * contraction, dx = pos[j].x - pos[i].x, and j is not excluded from row i.
 * Exclusions (both pointers null, or both set) use the reference's CSR:
 * row i excludes exclude_pair_xs[ptr_exclude_pair_xs[i] ..
 * ptr_exclude_pair_xs[i+1]), each segment sorted ascending, ptr of length
 * n_nodes + 1 (mlcg_exclusion_pair_to_ptr builds it).  Rows keep their
 * lowest-index `max_num_neighbors` non-excluded neighbours; *overflow gets
 * bit 0 (1) if any row had more, and bit 2 (4) if a kept edge (i, j) has its
 * reverse (j, i) excluded (an asymmetric graph, which the pair-based CFConv
 * kernels cannot use).  deg[i] = kept neighbours, upper_deg[i] = kept
 * neighbours with j > i.  Replaces the counting half of radius_kernel
 * (radius.cu:88-145, exclusion test 113-133) and the
 * torch_cluster.radius_graph call of
 * src/mlcg/neighbor_list/torch_impl.py:216-224. */
int mlcg_radius_count(const float* pos, const int64_t* batch,
                      const int64_t* frame_ptr, int64_t n_nodes, double r,
                      int loop, int64_t max_num_neighbors,
                      const int64_t* exclude_pair_xs,
                      const int64_t* ptr_exclude_pair_xs, int32_t* deg,
                      int32_t* upper_deg, int32_t* overflow, void* stream);

/* mlcg_radius_count for float64 positions: the same membership test in
 * double arithmetic, d2 < r*r (r*r rounded once, in double), as the
 * reference's kernel runs it for double inputs (the AT_DISPATCH over the
 * scalar type and `scalar_t r_squared = r*r` of radius.cu:243-250). */
int mlcg_radius_count_f64(const double* pos, const int64_t* batch,
                          const int64_t* frame_ptr, int64_t n_nodes, double r,
                          int loop, int64_t max_num_neighbors,
                          const int64_t* exclude_pair_xs,
                          const int64_t* ptr_exclude_pair_xs, int32_t* deg,
                          int32_t* upper_deg, int32_t* overflow, void* stream);

/* Exclusive scan of two int32 vectors of length n into out_a/out_b (length
 * n + 1, the totals at index n).  `workspace` holds
 * mlcg_scan_workspace_ints(n) int32.  Replaces the block/grid scan of
 * radius.cu:146-181 (no cooperative launch, no host sync). */
int64_t mlcg_scan_workspace_ints(int64_t n);
int mlcg_exclusive_scan2_i32(const int32_t* in_a, const int32_t* in_b,
                             int64_t n, int32_t* out_a, int32_t* out_b,
                             int32_t* workspace, void* stream);

/* mlcg_exclusive_scan2_i32 without the workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * or MD loops, harnesses that forbid hipMalloc); it has no counterpart in the
 * reference.  Same inputs, outputs and results, bit for bit.  The per-tile
 * sums live in a file-scope device array of the library sized for at most
 * MLCG_SCAN_NOALLOC_MAX_N elements (128 KiB per device, held until the
 * process ends); a larger n returns MLCG_ERR_CAPACITY before any launch.
 * Nothing in the array needs to start at zero.  Every call on one device
 * shares that device's array: calls that overlap on one GPU (other streams,
 * other host threads) race and must be serialised by the caller.  The first
 * call on a device looks the array's address up (no allocation, no stream
 * work): make that first call outside a stream capture. */
#define MLCG_SCAN_NOALLOC_MAX_N (1LL << 24)
int mlcg_exclusive_scan2_i32_noalloc(const int32_t* in_a, const int32_t* in_b,
                                     int64_t n, int32_t* out_a, int32_t* out_b,
                                     void* stream);

/* Pass 2: writes the canonical edge list (same membership and exclusion
 * arguments as pass 1).  edge_index is [2, edge_stride]
 * int64 (row 0 = centre i, row 1 = neighbour j).  Optional (nullable)
 * outputs for the CFConv pipeline, all three or none: col[e] = j (int32),
 * pair_ij [2, pair_stride] (row 0 = i, row 1 = j, i < j) and eid2pair[e] for
 * upper edges (with pairptr).
 * Edges at index >= edge_capacity (pairs >= pair_capacity) are dropped and
 * *overflow is set to 2.  Replaces radius.cu:117-145 and compact_kernel
 * (radius.cu:60-86). */
int mlcg_radius_fill(const float* pos, const int64_t* batch,
                     const int64_t* frame_ptr, int64_t n_nodes, double r,
                     int loop, int64_t max_num_neighbors,
                     const int64_t* exclude_pair_xs,
                     const int64_t* ptr_exclude_pair_xs,
                     const int32_t* rowptr, const int32_t* pairptr,
                     int64_t edge_capacity, int64_t edge_stride,
                     int64_t* edge_index, int32_t* col,
                     int64_t pair_capacity, int64_t pair_stride,
                     int32_t* pair_ij, int32_t* eid2pair, int32_t* overflow,
                     void* stream);

/* Bytes of the workspace of mlcg_radius_rowptr / mlcg_radius_graph for up
 * to n_nodes rows: a two-word header (a call counter, the most blocks a call
 * has used) and two status words per block of at least 64 rows.  The caller
 * zero-fills it once, before its first use; every call then leaves it ready
 * for the next call (no clearing between calls), so one workspace serves a
 * sequence of calls on one stream, of any sizes up to n_nodes.  Calls that
 * may overlap (other streams) need workspaces of their own.  After a call
 * that reports overflow bit 8 the workspace must be zero-filled again. */
int64_t mlcg_radius_workspace_bytes(int64_t n_nodes);

/* Sizing pass in one launch: per-row kept counts (membership, exclusion and
 * max_num_neighbors rules of mlcg_radius_count) scanned within blocks of 32
 * to 256 rows and across blocks by a decoupled look-back,
 * written as the CSR: rowptr[n_nodes + 1] (edges) and, when non-NULL,
 * pairptr[n_nodes + 1] (upper edges j > i).  *overflow is cleared, then gets
 * bit value 1 when a row exceeded max_num_neighbors, 4 for an asymmetric
 * exclusion, 16 when the totals exceed 2^31 - 1 (offsets saturate) and 8 if a
 * look-back wait hit its bound (never expected; the output is then invalid).
 * Replaces the count, block scan and grid scan of radius_kernel
 * (radius.cu:88-181) up to the host read of the total (radius.cu:288). */
int mlcg_radius_rowptr(const float* pos, const int64_t* batch,
                       const int64_t* frame_ptr, int64_t n_nodes, double r,
                       int loop, int64_t max_num_neighbors,
                       const int64_t* exclude_pair_xs,
                       const int64_t* ptr_exclude_pair_xs, int32_t* rowptr,
                       int32_t* pairptr, void* workspace, int32_t* overflow,
                       void* stream);

/* mlcg_radius_rowptr for float64 positions (membership as in
 * mlcg_radius_count_f64, radius.cu:243-250). */
int mlcg_radius_rowptr_f64(const double* pos, const int64_t* batch,
                           const int64_t* frame_ptr, int64_t n_nodes, double r,
                           int loop, int64_t max_num_neighbors,
                           const int64_t* exclude_pair_xs,
                           const int64_t* ptr_exclude_pair_xs, int32_t* rowptr,
                           int32_t* pairptr, void* workspace, int32_t* overflow,
                           void* stream);

/* The whole radius graph in one launch, for callers that give a capacity
 * instead of reading the edge count back: the sweep,
 * the look-back of mlcg_radius_rowptr and the writes of mlcg_radius_fill,
 * with each row's distances tested once.  rowptr / pairptr come out clamped
 * to edge_capacity / pair_capacity, so every consumer stays inside the
 * buffers; rowptr[n_nodes] is the number of edges written.  *overflow is
 * cleared, then gets the bits of mlcg_radius_rowptr and 2 when edges or
 * pairs fell past their capacity.  Pair outputs as in mlcg_radius_fill
 * (pairptr required with them).  Replaces radius_kernel and compact_kernel
 * (radius.cu:60-181) with the output sized by the caller. */
int mlcg_radius_graph(const float* pos, const int64_t* batch,
                      const int64_t* frame_ptr, int64_t n_nodes, double r,
                      int loop, int64_t max_num_neighbors,
                      const int64_t* exclude_pair_xs,
                      const int64_t* ptr_exclude_pair_xs, int32_t* rowptr,
                      int32_t* pairptr, int64_t edge_capacity,
                      int64_t edge_stride, int64_t* edge_index, int32_t* col,
                      int64_t pair_capacity, int64_t pair_stride,
                      int32_t* pair_ij, int32_t* eid2pair, void* workspace,
                      int32_t* overflow, void* stream);

/* mlcg_radius_graph for float64 positions, edge list only. */
int mlcg_radius_graph_f64(const double* pos, const int64_t* batch,
                          const int64_t* frame_ptr, int64_t n_nodes, double r,
                          int loop, int64_t max_num_neighbors,
                          const int64_t* exclude_pair_xs,
                          const int64_t* ptr_exclude_pair_xs, int32_t* rowptr,
                          int64_t edge_capacity, int64_t edge_stride,
                          int64_t* edge_index, void* workspace,
                          int32_t* overflow, void* stream);

/* mlcg_radius_fill for float64 positions (membership as in
 * mlcg_radius_count_f64); writes the edge list only (the pair structures of
 * the CFConv pipeline take float32 positions).  Replaces radius.cu:117-145
 * for double inputs. */
int mlcg_radius_fill_f64(const double* pos, const int64_t* batch,
                         const int64_t* frame_ptr, int64_t n_nodes, double r,
                         int loop, int64_t max_num_neighbors,
                         const int64_t* exclude_pair_xs,
                         const int64_t* ptr_exclude_pair_xs,
                         const int32_t* rowptr, int64_t edge_capacity,
                         int64_t edge_stride, int64_t* edge_index,
                         int32_t* overflow, void* stream);

/* The sizing pass (mlcg_radius_rowptr without pairptr) and the write pass
 * (as mlcg_radius_fill_f64) for float16 / bfloat16 positions given as their
 * raw 16-bit storage [N, 3]: every operation of the membership test is
 * computed in float and rounded to the 16-bit type (round to nearest even),
 * r*r in double rounded to float then to the 16-bit type, the comparison in
 * float -- the arithmetic of the reference's Half / BFloat16 instantiations
 * (radius.cu:117-141 under the dispatch of radius.cu:243-250).  Edge list
 * only. */
int mlcg_radius_rowptr_f16(const uint16_t* pos, const int64_t* batch,
                           const int64_t* frame_ptr, int64_t n_nodes, double r, int loop,
                           int64_t max_num_neighbors, const int64_t* exclude_pair_xs,
                           const int64_t* ptr_exclude_pair_xs, int32_t* rowptr,
                           void* workspace, int32_t* overflow, void* stream);
int mlcg_radius_rowptr_bf16(const uint16_t* pos, const int64_t* batch,
                            const int64_t* frame_ptr, int64_t n_nodes, double r, int loop,
                            int64_t max_num_neighbors, const int64_t* exclude_pair_xs,
                            const int64_t* ptr_exclude_pair_xs, int32_t* rowptr,
                            void* workspace, int32_t* overflow, void* stream);
int mlcg_radius_fill_f16(const uint16_t* pos, const int64_t* batch,
                         const int64_t* frame_ptr, int64_t n_nodes, double r, int loop,
                         int64_t max_num_neighbors, const int64_t* exclude_pair_xs,
                         const int64_t* ptr_exclude_pair_xs, const int32_t* rowptr,
                         int64_t edge_capacity, int64_t edge_stride, int64_t* edge_index,
                         int32_t* overflow, void* stream);
int mlcg_radius_fill_bf16(const uint16_t* pos, const int64_t* batch,
                          const int64_t* frame_ptr, int64_t n_nodes, double r, int loop,
                          int64_t max_num_neighbors, const int64_t* exclude_pair_xs,
                          const int64_t* ptr_exclude_pair_xs, const int32_t* rowptr,
                          int64_t edge_capacity, int64_t edge_stride, int64_t* edge_index,
                          int32_t* overflow, void* stream);

/* HOST function (host pointers, no stream): the reference's
 * exclusion_pair_to_ptr (exclusion_pairs.cpp:7-62).  exc_pair_index is
 * [2, num_pairs] int64, row 0 = x (the excluded neighbour), row 1 = y (the
 * centre).  Pairs are ordered by y, then x; pair_xs[num_pairs] receives the x
 * of every pair in that order, y_ptr[num_nodes + 1] the row offsets (y_ptr[n]
 * = pairs with y < n).  Pairs with y >= num_nodes stay at the end of pair_xs,
 * outside every row; a negative y is an argument error when num_nodes > 0
 * (the reference's TORCH_CHECK at line 47). */
int mlcg_exclusion_pair_to_ptr(const int64_t* exc_pair_index,
                               int64_t num_pairs, int64_t num_nodes,
                               int64_t* pair_xs, int64_t* y_ptr);

/* Pass 3: eid2pair for lower edges (i > j), by binary search of i in row j.
 * n_pairs_dev points at the live pair count (e.g. pairptr + n_nodes). */
int mlcg_pair_reverse_map(const int32_t* pair_ij, int64_t pair_stride,
                          const int32_t* n_pairs_dev, int64_t max_pairs,
                          const int32_t* rowptr, const int32_t* col,
                          int32_t* eid2pair, void* stream);

/* ---------------------------------------------------------------------- */
/* Filter network (radial basis -> cutoff -> MLP([K, F, F]) -> x cutoff)  */
/* ---------------------------------------------------------------------- */

/* Per pair p = {i, j}: d = |pos[j] - pos[i]|, radial basis
 *   basis 0: g_k = exp(c (d - centers[k])^2) * C_rbf(d), c = widths[0]
 *            (GaussianBasis, gaussian.py:83-102: centers = offset,
 *            widths = the 0-dim coeff)
 *   basis 1: g_k = exp(-widths[k] (exp(alpha (rbf_lo - d)) - centers[k])^2)
 *            * C_rbf(d) (ExpNormalBasis, exp_normal.py:104-124: centers =
 *            means, widths = betas, alpha = 5 / (upper - lower))
 * all read on the device (no host copy of the basis parameters), then
 *   a    = W1 g + b1 ; h = act(a) ; w = W2 h                 (mlp.py:56-58)
 *   W    = w * C_conv(d)                                     (schnet.py:340-341)
 *   Wd   = dW/dd (forward-mode tangent of the same chain).
 * W1 is [F, K] (torch Linear layout), b1 [F], W2 [F, F]; F must be 128 and
 * 1 <= K <= 128.  W_out/Wd_out are [max_pairs, F]; dist_out [max_pairs] is
 * optional.  act: 0 = tanh, 1 = shifted softplus.  cut kinds: 0 = identity,
 * 1 = cosine.  `f16` selects the arithmetic:
 *   MLCG_FILTER_FP32 (0)        fp32 results; for K <= 64 the products run
 *                               on the fp16 MFMA with every operand split
 *                               into two fp16 parts (about 22 significant
 *                               bits, fp32 accumulation), wider bases on the
 *                               fp32 MFMA;
 *   MLCG_FILTER_FP16 (1)        fp16 operands, fp32 accumulation, fp16
 *                               W_out/Wd_out storage (the fp16 filter path);
 *   MLCG_FILTER_FP32_STRICT (2) fp32 results from the fp32 MFMA throughout.
 * Replaces CFConv.forward lines 340-341 plus the basis/CosineCutoff/MLP
 * (schnet.py:150,340-341). */
enum { MLCG_FILTER_FP32 = 0, MLCG_FILTER_FP16 = 1, MLCG_FILTER_FP32_STRICT = 2 };
int mlcg_filter_fwd(const float* pos, const int32_t* pair_ij,
                    int64_t pair_stride, const int32_t* n_pairs_dev,
                    int64_t max_pairs, int basis, const float* centers,
                    const float* widths, float alpha, int num_rbf, int rbf_cut_kind, float rbf_lo, float rbf_hi,
                    int conv_cut_kind, float conv_lo, float conv_hi, int act,
                    const float* W1, const float* b1, const float* W2,
                    int num_filters, int f16, void* W_out, void* Wd_out,
                    float* dist_out, void* stream);

/* Parameter gradients of the filter chain for given pair adjoints
 * Wbar = dL/dW and Wdbar = dL/dWd ([max_pairs, F] fp32, rows past the live
 * pair count ignored):
 *   dW1 [F, K] = d/dW1, db1 [F] = d/db1, dW2 [F, F] = d/dW2
 * of <Wbar, W> + <Wdbar, dW/dd>.  The per-pair reverse products and the pair
 * reductions run in one kernel (per-workgroup partial sums in `workspace`,
 * then a fixed-order reduction), so nothing per pair is written to memory.
 * `workspace` holds mlcg_filter_bwd_workspace_floats(max_pairs, num_rbf)
 * floats.  num_rbf <= 64 runs on the fp16 MFMA with split operands (about
 * 22 significant bits; activations and their derivatives must stay below
 * 2^19 in magnitude, else bit 0 of mlcg_numerics_flags is set) unless
 * fp32_strict != 0, which, like num_rbf > 64, runs every product on the fp32
 * MFMA.  Replaces the autograd double backward through mlp.py:56-58 and
 * gaussian.py:98-102 (the parameter half of the create_graph=True backward
 * of gradients.py:216-222). */
int64_t mlcg_filter_bwd_workspace_floats(int64_t max_pairs, int num_rbf);
int mlcg_filter_bwd(const float* pos, const int32_t* pair_ij,
                    int64_t pair_stride, const int32_t* n_pairs_dev,
                    int64_t max_pairs, int basis, const float* centers,
                    const float* widths, float alpha, int num_rbf,
                    int rbf_cut_kind, float rbf_lo, float rbf_hi,
                    int conv_cut_kind, float conv_lo, float conv_hi, int act,
                    const float* W1, const float* b1, const float* W2,
                    int num_filters, const float* Wbar, const float* Wdbar,
                    float* dW1, float* db1, float* dW2, float* abar_out,
                    float* adbar_out, float* workspace,
                    int64_t workspace_floats, int fp32_strict, void* stream);

/* ---------------------------------------------------------------------- */
/* CFConv gather/scatter over the receiver CSR (rowptr, col, eid2pair)      */
/* ---------------------------------------------------------------------- */

/* out[i] = sum_{e in row i, ascending j} src[col[e]] * W[eid2pair[e]].
 * F = 128.  w_f16 != 0: W is fp16.  Replaces CFConv.propagate/message
 * (schnet.py:346,368) with PyG's SumAggregation. */
int mlcg_cfconv_gather(const float* src, const void* W, int w_f16,
                       const int32_t* rowptr, const int32_t* col,
                       const int32_t* eid2pair, int64_t n_nodes,
                       int num_filters, float* out, void* stream);

/* Force backward of one CFConv: ybar[i] = sum_j gagg[j] * W_ij and, per
 * pair p = {i < j}, dbar[p] += <Wd_p, gagg[i] * y[j] + gagg[j] * y[i]>
 * (accumulate != 0) or dbar[p] = ... (accumulate == 0: dbar need not be
 * initialised; pairs past the graph's live count are left untouched).
 * ybar == NULL: dbar only (no filter row W is read; the same dbar values
 * bit for bit), for a block whose input does not depend on the positions.
 * Replaces the autograd backward of schnet.py:340-346. */
int mlcg_cfconv_gather_bwd(const float* gagg, const float* y, const void* W,
                           const void* Wd, int w_f16, const int32_t* rowptr,
                           const int32_t* col, const int32_t* eid2pair,
                           int64_t n_nodes, int num_filters, float* ybar,
                           float* dbar, int accumulate, void* stream);

/* Tangent (forward-mode) of the CFConv aggregation along a position
 * direction: out[i] = sum_j ydot[j] * W_ij + y[j] * Wd_ij * ddot_p.
 * ydot may be NULL (zero).  Part of the force-matching double backward. */
int mlcg_cfconv_gather_tangent(const float* ydot, const float* y,
                               const float* W, const float* Wd,
                               const float* ddot, const int32_t* rowptr,
                               const int32_t* col, const int32_t* eid2pair,
                               int64_t n_nodes, int num_filters, float* out,
                               void* stream);

/* Reverse over (primal, tangent) of the CFConv aggregation:
 *   ybar2[i] = sum_j gagg2[j] * W_ij + gagg1[j] * Wd_ij * ddot_p
 *   Wbar[p]  = gagg2[i] y[j] + gagg2[j] y[i] + gagg1[i] ydot[j] + gagg1[j] ydot[i]
 *   Wdbar[p] = ddot_p (gagg1[i] y[j] + gagg1[j] y[i])
 * ydot, gagg1, ddot may be NULL (zero tangent).  Wbar/Wdbar are
 * [n_pairs, F]; both may be NULL, then only ybar2 is computed (the pair
 * adjoints are then formed inside mlcg_filter_bwd_cfconv instead). */
int mlcg_cfconv_gather_rev2(const float* gagg2, const float* gagg1,
                            const float* y, const float* ydot,
                            const float* W, const float* Wd,
                            const float* ddot, const int32_t* rowptr,
                            const int32_t* col, const int32_t* eid2pair,
                            int64_t n_nodes, int num_filters, float* ybar2,
                            float* Wbar, float* Wdbar, void* stream);

/* mlcg_filter_bwd with the pair adjoints formed from node vectors of the
 * CFConv reverse instead of read from [P, F] arrays:
 *   Wbar_p  = gagg2_i y_j + gagg2_j y_i + gagg1_i ydot_j + gagg1_j ydot_i
 *   Wdbar_p = ddot_p (gagg1_i y_j + gagg1_j y_i)
 * (node arrays [N, F] fp32; gagg1, ydot, ddot may be NULL for a zero
 * tangent, ddot is [max_pairs]).  Same outputs and workspace as
 * mlcg_filter_bwd; the two [P, F] adjoint arrays are never materialised. */
int mlcg_filter_bwd_cfconv(const float* pos, const int32_t* pair_ij,
                           int64_t pair_stride, const int32_t* n_pairs_dev,
                           int64_t max_pairs, int basis, const float* centers,
                           const float* widths, float alpha, int num_rbf,
                           int rbf_cut_kind, float rbf_lo, float rbf_hi,
                           int conv_cut_kind, float conv_lo, float conv_hi,
                           int act, const float* W1, const float* b1,
                           const float* W2, int num_filters,
                           const float* gagg2, const float* y,
                           const float* gagg1, const float* ydot,
                           const float* ddot, float* dW1, float* db1,
                           float* dW2, float* abar_out, float* adbar_out,
                           float* workspace, int64_t workspace_floats,
                           int fp32_strict, void* stream);

/* Gradients of trainable basis parameters from the first-layer pair
 * adjoints abar = dL/da, adbar = dL/da' [max_pairs, F] (a = W1 g + b1,
 * a' = W1 dg/dd), which mlcg_filter_bwd / mlcg_filter_bwd_cfconv write to
 * abar_out / adbar_out when those are non-NULL.  With gbar = W1^T abar and
 * gdbar = W1^T adbar per pair:
 *   dcenters[k] (+)= sum_p gbar_pk dg_pk/dcenters[k] + gdbar_pk dg'_pk/dcenters[k]
 *   dwidths[k]  (+)= the same with d/dwidths[k]; for the Gaussian basis
 *                   (one shared coeff) sum_k dwidths[k] is d/dcoeff.
 * dist holds the pair distances (mlcg_filter_fwd's dist_out); `workspace`
 * holds mlcg_rbf_param_grad_workspace_floats(max_pairs, num_rbf) floats;
 * accumulate != 0 adds to the outputs (the blocks share one basis).
 * Replaces the autograd of GaussianBasis/ExpNormalBasis with
 * trainable=True (gaussian.py:46-52, exp_normal.py:72-78) through the
 * force-matching double backward. */
int64_t mlcg_rbf_param_grad_workspace_floats(int64_t max_pairs, int num_rbf);
int mlcg_rbf_param_grad(const float* dist, const int32_t* n_pairs_dev,
                        int64_t max_pairs, int basis, const float* centers,
                        const float* widths, float alpha, int num_rbf,
                        int rbf_cut_kind, float rbf_lo, float rbf_hi,
                        const float* W1, int num_filters, const float* abar,
                        const float* adbar, int accumulate, float* dcenters,
                        float* dwidths, float* workspace,
                        int64_t workspace_floats, void* stream);

/* ddot[p] = scale * rhat_p . (u[j] - u[i]), rhat_p = (pos[j] - pos[i]) /
 * dist[p] (scale = -1 gives the tangent along -u exactly, without negating
 * u first). */
int mlcg_pair_ddot(const float* pos, const float* dist, const int32_t* pair_ij,
                   int64_t pair_stride, const int32_t* n_pairs_dev,
                   int64_t max_pairs, const float* u, float scale, float* ddot,
                   void* stream);

/* forces[i] (+)= sum_{j in row i} dbar[p(i,j)] (pos[j] - pos[i]) / dist[p].
 * Deterministic per-node sum in ascending j.  accumulate != 0 adds to
 * forces instead of overwriting.  Replaces the autograd position gradient of
 * compute_distances (internal_coordinates.py:73-100) in GradientsOut. */
int mlcg_pair_forces(const float* pos, const float* dist, const float* dbar,
                     const int32_t* rowptr, const int32_t* col,
                     const int32_t* eid2pair, int64_t n_nodes, int accumulate,
                     float* forces, void* stream);

/* E[b] = sum_{n in frame b} values[n * stride] (ascending n).  Replaces
 * torch_geometric.utils.scatter(..., reduce="sum") of schnet.py:158. */
int mlcg_segment_sum(const float* values, int64_t stride,
                     const int64_t* frame_ptr, int64_t n_frames, float* out,
                     void* stream);

/* float64 forms for a model moved to double (the reference's simulations with
 * dtype="double", src/mlcg/simulation/base.py:162,271): per-frame sums of a
 * float64 vector (one workgroup per frame, fixed order), and the CFConv
 * gather out[i] = sum_j src[j] * W[eid2pair[e]] over the receiver CSR for
 * any feature count (each feature summed over the row in CSR order). */
int mlcg_segment_sum_f64(const double* values, const int64_t* frame_ptr, int64_t n_frames,
                         double* out, void* stream);
int mlcg_cfconv_gather_f64(const double* src, const double* W, const int32_t* rowptr,
                           const int32_t* col, const int32_t* eid2pair, int64_t n_nodes,
                           int num_filters, double* out, void* stream);

/* ---------------------------------------------------------------------- */
/* Node-level linears (F = H = 128) and their weight gradients             */
/* ---------------------------------------------------------------------- */

/* Epilogues of mlcg_node_gemm (y = x W^T, or x W when transpose_w != 0,
 * then + bias[128] and + residual[rows, 128] when those are non-NULL):
 *   PLAIN  out0 = y
 *   ACT    out0 = y (optional), out1 = act(y)
 *   DACT   out0 = y (optional), out1 = y * act'(z)
 *   DACT2  out0 = y * act'(z) + e * act''(z) * f   (e, f optional, together)
 * act'/act'' are evaluated from z and s = act(z) (tanh uses s only, and z
 * may then be NULL; shifted softplus uses z). */
typedef enum {
  MLCG_NODE_PLAIN = 0,
  MLCG_NODE_ACT = 1,
  MLCG_NODE_DACT = 2,
  MLCG_NODE_DACT2 = 3
} mlcg_node_epilogue;

/* [rows, 128] x [128, 128] product with a fused elementwise epilogue, all
 * [rows, 128] tensors row-major fp32.  Replaces the Linear calls of the
 * interaction block and CFConv (schnet.py:259-261 lin + activation,
 * 343 lin1, 347 lin2 + bias) and their transposes in the force backward and
 * the force-matching double backward, together with the activation and
 * derivative elementwise kernels around them. */
int mlcg_node_gemm(const float* x, int64_t rows, int features, const float* W,
                   int transpose_w, const float* bias, const float* residual,
                   int epilogue, int act, const float* z, const float* s,
                   const float* e, const float* f, float* out0, float* out1,
                   const void* w_image, void* stream);

/* Two consecutive linears of the interaction block in one pass over the
 * rows: mlcg_node_gemm(x, W, ..., epilogue) as above (ACT, DACT or DACT2),
 * then out2 = v W2^T (v W2 when transpose_w != 0) [+ bias2] [+ residual2],
 * v being the first call's principal output (out1 for ACT and DACT, out0 for
 * DACT2), which is still stored.  The results equal those of the two
 * separate mlcg_node_gemm calls bit for bit.  Replaces the pairs
 * schnet.py:347 lin2 -> 259-261 act + lin (+ the residual of schnet.py:153)
 * and their transposes in the backward, tangent and double backward sweeps;
 * the x -> v -> out2 chain reads x once and v never back. */
int mlcg_node_gemm2(const float* x, int64_t rows, int features, const float* W,
                    int transpose_w, const float* bias, const float* residual,
                    int epilogue, int act, const float* z, const float* s,
                    const float* e, const float* f, float* out0, float* out1,
                    const float* W2, const float* bias2, const float* residual2,
                    float* out2, const void* w_image, const void* w2_image,
                    void* stream);

/* The split operand image of a [128, 128] node weight W for mlcg_node_gemm
 * and mlcg_node_gemm2 (their w_image / w2_image arguments): the fp16 hi and
 * lo planes of W^T (transpose_w = 0) or W (transpose_w != 0) in the order
 * the kernels' MFMA fragments read them, mlcg_node_weight_image_bytes() =
 * 65,536 bytes per weight.  Without an image every launch splits W itself
 * (each workgroup, before its first row tile); with one, the launch reads the
 * image instead and its results are the same bit for bit.  An image holds W
 * as it was when the image was made: make the images again after every
 * change of the weights (the fused SchNet makes them at the start of each
 * forward, in one launch).  count <= 32 images go to images + k * 65,536
 * (16-byte aligned); the weights and flags are host arrays read during the
 * call.  No counterpart in the reference (its Linear layers keep fp32
 * weights for the library GEMM). */
int64_t mlcg_node_weight_image_bytes(void);
int mlcg_node_weight_images(const float* const* weights, const int* transpose_w,
                            int count, void* images, void* stream);

/* out [128, 128] (+)= a1^T b1 (+ a2^T b2) for [rows, 128] inputs (a2/b2 may
 * be NULL) and, when colsum_a1 is non-NULL, colsum_a1 [128] (+)= the column
 * sums of a1 (a bias gradient); deterministic split over contiguous row
 * ranges, one per workgroup; `workspace` holds
 * mlcg_node_tmm_workspace_floats(rows) floats.  accumulate != 0 adds to the
 * outputs.  Replaces the weight- and bias-gradient reductions of the same
 * linears (the autograd backward of schnet.py:259-261,343,347 through the
 * double backward). */
int64_t mlcg_node_tmm_workspace_floats(int64_t rows);
int mlcg_node_tmm(const float* a1, const float* b1, const float* a2,
                  const float* b2, int64_t rows, int features, int accumulate,
                  float* out, float* colsum_a1, float* workspace,
                  int64_t workspace_floats, void* stream);

/* `count` (1..4) independent mlcg_node_tmm reductions over the same number
 * of rows in one launch pair: problems holds 6 pointers per reduction,
 * {a1, b1, a2, b2, out, colsum_a1} (a2/b2 and colsum_a1 may be NULL), as in
 * mlcg_node_tmm.  Each reduction splits its rows over about 256 / count
 * workgroups, so each result is deterministic (run-to-run identical) though
 * not bit-equal to a single mlcg_node_tmm call.  The weight-gradient
 * reductions of one interaction block (lin, conv.lin2, conv.lin1 of
 * schnet.py:259-261,343,347 through the double backward) are one batch.
 * mlcg_node_tmm_batch_workspace_floats(rows, count) floats of workspace. */
int64_t mlcg_node_tmm_batch_workspace_floats(int64_t rows, int count);
int mlcg_node_tmm_batch(const void* const* problems, int count, int64_t rows,
                        int features, int accumulate, float* workspace,
                        int64_t workspace_floats, void* stream);

/* out [n, 128] = table[types[i]] for a [num_types, 128] fp32 table (16-byte
 * aligned): the embedding lookup of schnet.py:132
 * (`x = self.embedding_layer(data.atom_types)`, torch.nn.Embedding).  A type
 * outside [0, num_types) gives a zero row and sets bit 2 of
 * mlcg_numerics_flags (torch raises a device-side assertion there). */
int mlcg_embedding_gather(const float* table, int num_types, int features,
                          const int64_t* types, int64_t n, float* out,
                          void* stream);

/* out [num_types, 128] = for each type t the sum of the rows of x [rows, 128]
 * whose types[row] == t: the gradient of the bead-type embedding table
 * (schnet.py:132, `x = self.embedding_layer(data.atom_types)`, whose
 * autograd backward scatters the adjoint of x into the table).  Workgroups
 * per type list their rows in ascending order and sum them in a fixed order
 * (with many rows, G groups of row chunks per type whose partial sums are
 * added in group order), so the result is run-to-run identical.
 * num_types <= 128 (MLCG_ERR_UNSUPPORTED beyond); a type outside
 * [0, num_types) is skipped and sets *bad = 1 (bad is not cleared here),
 * or, with bad == NULL, bit 2 of the numerics flags (mlcg_numerics_flags).
 * mlcg_type_sum_workspace_floats gives the workspace the call needs: 0 up to
 * 24,576 rows or when one group per type fills the chip (workspace may then
 * be NULL), else 2 G num_types 128 floats. */
int64_t mlcg_type_sum_workspace_floats(int64_t rows, int num_types);
int mlcg_type_sum(const float* x, const int64_t* types, int64_t rows, int features,
                  int num_types, float* out, int* bad, float* workspace,
                  int64_t workspace_floats, void* stream);

/* ---------------------------------------------------------------------- */
/* Output network MLP([128, HH, 1]) with its reverse and tangent sweeps    */
/* ---------------------------------------------------------------------- */

/* Per node n (x [rows, 128], W0 [HH, 128], b0 [HH] or NULL, w1 [HH] = the
 * final Linear's weight row, b1 [1] or NULL, HH in {32, 64, 128}):
 *   oz = x W0^T + b0 ; os = act(oz) ; o = os . w1 + b1
 * writes o [rows] (nullable), oz/os [rows, HH] (nullable, saved for the
 * sweeps below) and, when reverse != 0, the adjoint entering the interaction
 * blocks for the objective sum_n seed_n o_n (seed NULL = all ones):
 *   xbar = ((seed w1) * act'(oz)) W0   [rows, 128].
 * Replaces the output_network MLP of schnet.py:156,462-467 (mlp.py:56-58)
 * and the first step of its autograd backward (gradients.py:216-222). */
int mlcg_out_forward(const float* x, int64_t rows, int in_features, int hidden,
                     const float* W0, const float* b0, const float* w1,
                     const float* b1, int act, int reverse, const float* seed,
                     float* o, float* oz, float* os, float* xbar, void* stream);

/* Second-order sweep of the same network for sum_n tw_n odot_n + pw_n o_n
 * (tw, pw nullable), with odot the tangent of o along xdot (xdot NULL = no
 * tangent):
 *   ozdot = xdot W0^T ; hdot = act'(oz) ozdot ; odot = hdot . w1
 *   zbar2 = pw w1 act'(oz) + tw w1 act''(oz) ozdot ; xbar2 = zbar2 W0
 *   gW0 = sum_n (tw w1 act'(oz))^T xdot + zbar2^T x ; gb0 = sum_n zbar2
 *   gW1 = sum_n tw hdot + pw os ; gb1 = sum_n pw.
 * oz may be NULL for tanh.  Outputs odot [rows] (nullable), xbar2 [rows, 128],
 * gW0 [HH, 128], gb0 [HH] (nullable), gW1 [HH], gb1 [1] (nullable).
 * `workspace` holds mlcg_out_rev2_workspace_floats(rows, HH) floats; the
 * reductions are in a fixed order.  Replaces the output-network part of the
 * force-matching double backward (losses.py:167-181 through
 * gradients.py:216-222 with create_graph=True, pl/model.py:113-131). */
int64_t mlcg_out_rev2_workspace_floats(int64_t rows, int hidden);
int mlcg_out_rev2(const float* x, const float* xdot, int64_t rows,
                  int in_features, int hidden, const float* W0, const float* w1,
                  const float* oz, const float* os, int act, const float* tw,
                  const float* pw, float* odot, float* xbar2, float* gW0,
                  float* gb0, float* gW1, float* gb1, float* workspace,
                  int64_t workspace_floats, void* stream);

/* ---------------------------------------------------------------------- */
/* Priors: harmonic bonds and angles, Fourier dihedrals, repulsion          */
/* ---------------------------------------------------------------------- */

typedef enum {
  MLCG_PRIOR_BOND = 0,      /* order 2, params [x0, k, V0]                  */
  MLCG_PRIOR_ANGLE = 1,     /* order 3, params [x0, k, V0] on cos(theta)    */
  MLCG_PRIOR_DIHEDRAL = 2,  /* order 4, params [v0, k1_1..k1_n, k2_1..k2_n] */
  MLCG_PRIOR_REPULSION = 3  /* order 2, params [sigma]                      */
} mlcg_prior_kind;

/* Interaction order and number of per-interaction parameters of a kind
 * (n_degs is the Fourier order of MLCG_PRIOR_DIHEDRAL, ignored otherwise);
 * 0 / -1 for an unknown kind. */
int mlcg_prior_order(int kind);
int mlcg_prior_num_params(int kind, int n_degs);

/* Per interaction m (index_mapping [order, mapping_stride] int64, bead
 * index_mapping[s][m] in slot s; params [M, n_params] float32):
 *   energy[m]            the interaction energy,
 *   slot_forces[m, s, :] the force -dU_m/dpos on the bead of slot s
 *                        (slot_forces may be NULL: energies only).
 * Replaces the forward of HarmonicBonds / HarmonicAngles
 * (src/mlcg/nn/prior/harmonic.py:90-120,199-298), Dihedral / FourierSeries
 * (src/mlcg/nn/prior/fourier_series.py:120-198,446-483) and Repulsion
 * (src/mlcg/nn/prior/repulsion.py:111-140) together with the autograd
 * position gradient GradientsOut takes of them (src/mlcg/nn/gradients.py:
 * 208-226); the static pre-gathered parameter layout is the one of
 * src/mlcg/simulation/specialize_prior.py:49-72,175-206. */
int mlcg_prior_terms(int kind, int n_degs, const float* pos,
                     const int64_t* index_mapping, int64_t mapping_stride,
                     int64_t n_interactions, const float* params, int n_params,
                     float* energy, float* slot_forces, void* stream);

/* forces[a] (+)= sum of slot_forces over the slots of bead a: CSR bead_ptr
 * [N + 1] int32 over bead_slots (flat slot ids m * order + s, ascending within
 * a bead).  accumulate != 0 adds to forces.  Deterministic, atomic-free
 * replacement of the per-prior autograd scatter into pos.grad. */
int mlcg_prior_gather_forces(const float* slot_forces, const int32_t* bead_ptr,
                             const int32_t* bead_slots, int64_t n_nodes,
                             int accumulate, float* forces, void* stream);

/* mlcg_prior_terms / mlcg_prior_gather_forces for a model moved to double
 * (positions, parameters, energies and forces float64; every kind evaluated
 * in double). */
int mlcg_prior_terms_f64(int kind, int n_degs, const double* pos,
                         const int64_t* index_mapping, int64_t mapping_stride,
                         int64_t n_interactions, const double* params, int n_params,
                         double* energy, double* slot_forces, void* stream);
int mlcg_prior_gather_forces_f64(const double* slot_forces, const int32_t* bead_ptr,
                                 const int32_t* bead_slots, int64_t n_nodes, int accumulate,
                                 double* forces, void* stream);

/* The repulsion prior (MLCG_PRIOR_REPULSION) in one call, without slot force
 * arrays: energy[m] of every interaction (as mlcg_prior_terms) and forces[a]
 * set or added (accumulate != 0) per bead straight from the positions.
 * mlcg_prior_pair_records fills `records` (mlcg_prior_pair_records_ints int32
 * values; once per topology and parameter table): for each position s of
 * bead_slots the record {partner bead | k << 31, params[m][0]} of slot 2m + k,
 * followed by the bead windows the kernels stage in LDS (the range of beads
 * that each block of 16 beads and each chunk of 1024 interactions touches).
 * mlcg_prior_repulsion reads them over the same CSR bead_ptr.  Energies and
 * forces are bit-identical to mlcg_prior_terms(MLCG_PRIOR_REPULSION) followed
 * by mlcg_prior_gather_forces.  Replaces Repulsion.forward
 * (src/mlcg/nn/prior/repulsion.py:111-140) with the autograd position
 * gradient of src/mlcg/nn/gradients.py:208-226. */
int64_t mlcg_prior_pair_records_ints(int64_t n_nodes, int64_t n_interactions);
int mlcg_prior_pair_records(const int64_t* index_mapping, int64_t mapping_stride,
                            int64_t n_interactions, const float* params, int n_params,
                            const int32_t* bead_ptr, const int32_t* bead_slots,
                            int64_t n_nodes, void* records, void* stream);
int mlcg_prior_repulsion(const float* pos, int64_t n_nodes, const int64_t* index_mapping,
                         int64_t mapping_stride, int64_t n_interactions, const float* params,
                         const void* records, const int32_t* bead_ptr, float* energy,
                         int accumulate, float* forces, void* stream);

/* ---------------------------------------------------------------------- */
/* Langevin BAOAB                                                          */
/* ---------------------------------------------------------------------- */

/* B, A, O, A sub-steps of LangevinSimulation.timestep
 * (src/mlcg/simulation/langevin.py:100-137) for [N, 3] float32 pos / vel
 * and the forces at the current positions; beta_mass_ratio [N] =
 * sqrt(1 / (beta m)) (langevin.py:176-180).  Noise is `noise` [N, 3] when
 * non-NULL, else Philox4x32-10 normals keyed by `seed` at counter (bead,
 * *step_dev) (step 0 when step_dev is NULL). */
int mlcg_langevin_baoa(float* pos, float* vel, const float* forces,
                       const float* masses, const float* beta_mass_ratio,
                       int64_t n_nodes, float dt, float vscale, float noisescale,
                       uint64_t seed, const int64_t* step_dev, const float* noise,
                       void* stream);

/* Final B sub-step (langevin.py:141) with the forces at the new positions;
 * advances *step_dev by one when step_dev is non-NULL. */
int mlcg_langevin_b(float* vel, const float* forces, const float* masses,
                    int64_t n_nodes, float dt, int64_t* step_dev, void* stream);

/* mlcg_langevin_baoa / mlcg_langevin_b for a simulation in double precision
 * (LangevinSimulation with dtype="double", src/mlcg/simulation/base.py:162):
 * every array float64; the noise is the same float Philox4x32-10 /
 * Box-Muller stream, widened (explicit noise is float64). */
int mlcg_langevin_baoa_f64(double* pos, double* vel, const double* forces,
                           const double* masses, const double* beta_mass_ratio,
                           int64_t n_nodes, double dt, double vscale, double noisescale,
                           uint64_t seed, const int64_t* step_dev, const double* noise,
                           void* stream);
int mlcg_langevin_b_f64(double* vel, const double* forces, const double* masses,
                        int64_t n_nodes, double dt, int64_t* step_dev, void* stream);

/* The normals mlcg_langevin_baoa draws at `step`: out [N, 3].  Replaces the
 * torch.randn draw of langevin.py:129-134 (used by the statistics tests). */
int mlcg_philox_normals(uint64_t seed, int64_t step, int64_t n_nodes, float* out,
                        void* stream);

/* ---------------------------------------------------------------------- */
/* Elementary functions (accuracy checks)                                  */
/* ---------------------------------------------------------------------- */

/* y[i] = f(x[i]) for the library's own fp32 elementary functions, the ones
 * the filter, node and output kernels evaluate inline: tanh (the reference's
 * default activation, schnet.py:419), the sigmoid and softplus of the
 * shifted-softplus activation, and sin(pi u) / cos(pi u) of the cosine
 * cutoff (cutoff.py:145-153).  Exposed so that their accuracy can be
 * measured against fp64; no reference interface is replaced. */
enum { MLCG_MATH_TANH = 0, MLCG_MATH_SIGMOID = 1, MLCG_MATH_SOFTPLUS = 2,
       MLCG_MATH_SINPI = 3, MLCG_MATH_COSPI = 4 };
int mlcg_math_eval(int fn, const float* x, int64_t n, float* y, void* stream);

/* Numerics flags of the split-product (fp16 MFMA) kernels: writes the
 * device's flag word to out[0] and, with clear != 0, clears it (both on the
 * stream, no host synchronisation; capturable).  Bit 0: a filter backward
 * (mlcg_filter_bwd, mlcg_filter_bwd_cfconv) met an activation value or
 * derivative of magnitude 2^19 or more (or a non-finite one), past the range
 * of its split operands, so its weight gradients may be non-finite.  Bit 1:
 * a split filter kernel (forward or backward) met a weight of magnitude 65504
 * (the fp16 maximum) or more, past what its fp16 weight planes hold.  The split filter forward
 * needs no flag for large activations: tiles whose activations pass its 2^15
 * bound are recomputed with an exact power-of-two scale.  No counterpart in the reference (its fp32
 * products have no such bound); callers that must not return non-finite
 * gradients silently read it after a training step. */
int mlcg_numerics_flags(int* out, int clear, void* stream);

/* ---------------------------------------------------------------------- */
/* HBM ceiling probes                                                      */
/* ---------------------------------------------------------------------- */

/* Streaming read of n floats (n % 4 == 0, src 16-byte aligned) by `groups`
 * 256-thread workgroups in a grid-stride loop with `unroll` (1, 4, 8, 16)
 * 16-byte loads in flight per thread; partial[g] = sum of what workgroup g
 * read.  No counterpart in the reference: it measures the HBM read ceiling
 * that the memory-bound kernels above are compared with. */
int mlcg_stream_read(const float* src, int64_t n, int groups, int unroll,
                     float* partial, void* stream);

/* Streaming copy dst[i] = src[i] of n floats, the same launch shapes as
 * mlcg_stream_read.  No counterpart in the reference: the read + write
 * ceiling. */
int mlcg_stream_copy(const float* src, float* dst, int64_t n, int groups,
                     int unroll, void* stream);

/* MFMA-loop probe: `groups` workgroups of 4 waves, each wave issuing `iters`
 * iterations of 8 independent MFMAs of one shape on register operands;
 * out[groups * 256] receives one float per thread (the accumulators' sum).
 * kind: 0 v_mfma_f32_16x16x32_f16, 1 v_mfma_f32_16x16x16_f16,
 * 2 v_mfma_f32_16x16x4_f32, 3 v_mfma_f32_16x16x32_bf16,
 * 4 v_mfma_f32_32x32x16_f16.  No counterpart in the reference: the sustained
 * matrix-core rate the MFMA-bound kernels are compared with. */
int mlcg_mfma_loop(int kind, int64_t iters, int groups, float* out, void* stream);

/* FLOP of one wave iteration of mlcg_mfma_loop for `kind` (-1 if unknown). */
int64_t mlcg_mfma_loop_flops_per_wave_iter(int kind);

/* The force-matching loss (ForceMSE with reduction "mean",
 * mlcg/nn/losses.py:130-181 -> torch.nn.functional.mse_loss):
 * *loss = sum_k (x[k] - y[k])^2 / n over n >= 1 fp32 elements, summed per
 * 64 Ki-element chunk and then over the chunks in a fixed order; `workspace`
 * holds mlcg_mse_workspace_floats(n) floats (0 up to 65,536 elements: may be
 * NULL).  mlcg_mse_mean_backward: grad_x[k] = (2/n) (x[k] - y[k]) g with g =
 * *grad_loss (a device scalar), evaluated as torch's mse_loss backward does,
 * so bit-identical to it. */
int64_t mlcg_mse_workspace_floats(int64_t n);
int mlcg_mse_mean(const float* x, const float* y, int64_t n, float* loss,
                  float* workspace, int64_t workspace_floats, void* stream);
int mlcg_mse_mean_backward(const float* x, const float* y, const float* grad_loss,
                           int64_t n, float* grad_x, void* stream);

/* out[k] = ((0 + a_0[k]) + a_1[k]) + ... for count <= 8 fp32 arrays of n
 * elements (MLCG_ERR_UNSUPPORTED beyond): SumOut's running sum of its
 * models' energies or forces (mlcg/nn/gradients.py SumOut.forward) in one
 * launch, bit-identical to the sequence of adds it replaces.  The array of
 * pointers is host memory, read during the call; out may alias none of the
 * inputs. */
int mlcg_sum_arrays(const float* const* arrays, int count, int64_t n, float* out,
                    void* stream);

/* Device-to-device copies dsts[k][0 .. bytes[k]) = srcs[k][...] for
 * k < count <= 8 (MLCG_ERR_UNSUPPORTED beyond) in one launch; every pointer
 * 16-byte aligned, the ranges must not overlap.  The pointer and size arrays
 * are host memory, read before the call returns.  No counterpart in the
 * reference (its batches arrive through the data loader): it loads a new
 * batch into the inputs of a training step recorded as a HIP graph. */
int mlcg_copy_batch(const void* const* srcs, void* const* dsts,
                    const int64_t* bytes, int count, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MLCG_HIP_H */
