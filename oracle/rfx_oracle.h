/*
 * rfx_oracle.h -- CPU restatement of RFX-Fuse's Breiman-Cutler proximity path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP product
 * path: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it.  The product library never links or calls it.
 *
 * Every function cites the reference file:line it restates.  Layout
 * conventions (shared with the HIP path):
 *   leaf[t*N + i]   int32 terminal-leaf label of sample i in tree t
 *                   (tree-major, as leaf_assignments_ in
 *                   include/rf_random_forest.hpp:496-501); a label outside
 *                   [0, nleaf) means "no valid terminal node" and the sample
 *                   takes no part in tree t (src/rf_proximity.cpp:126-135,184-186).
 *   oob[t*N + i]    uint8, 1 when sample i is out-of-bag in tree t (nin == 0,
 *                   src/rf_bootstrap.cpp:67-82).
 *   packed upper triangle, row-wise with the diagonal:
 *                   idx(i,j) = i*N - i*(i+1)/2 + j  for i <= j
 *                   (cuda/rf_proximity_upper_triangle.cu:34-39, 64-bit here).
 *
 * Output formats of the triangle (enum values of RFXP_FMT_* in
 * include/rfx_prox.h):
 *   0 F32   (float)P                              4 B/entry
 *   1 F16   IEEE half, RN-even, of (float)P         2 B/entry
 *   2 I8    reference fp32_to_int8((float)P, scale, zp)
 *                                  (include/rf_quantization_kernels.hpp:24-29)
 *   3 NF4   reference fp32_to_nf4((float)P), 2 entries per byte, entry e in
 *           byte e/2 at bit (e%2)*4 (cuda/rf_proximity_upper_triangle.cu:486-519)
 *   4 U8    trunc(clamp((float)P/scale + zp, 0, 255))
 *   5 U16   raw co-occurrence count U (no normalisation)
 */
#ifndef RFX_ORACLE_H
#define RFX_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- reference-shaped restatements (column-major N x N double) ---------- */

/* src/rf_proximity.cpp:99-231 (dense branch): one tree, accumulates
 * prox[n + kk*N] += w for OOB n and in-bag kk in the same terminal node. */
void orc_cpu_proximity(const int32_t* nodestatus, const int32_t* nodextr, const int32_t* nin,
                       int32_t nsample, int32_t nnode, int use_casewise, double* prox);

/* src/rf_finishprox.cpp:12-74 */
void orc_finishprox(int32_t nsample, const int32_t* nout, const double* prox, double* proxsym);

/* src/rf_proximity.cpp:238-397; nin/nodextr tree-major [t*nsample + i]. */
void orc_rfgap(int32_t ntree, int32_t nsample, const int32_t* nin_flat,
               const int32_t* nodextr_flat, double* prox);

/* src/rf_proximity.cpp:110-135: node index -> terminal ordinal, -1 if the
 * node is not terminal or out of range. */
void orc_terminal_leaf(const int32_t* nodestatus, int32_t nnode, const int32_t* nodextr,
                       int32_t nsample, int32_t* leaf_out);

/* ---- normalisation and quantizers ---------------------------------------- */

/* src/rf_finishprox.cpp:33-73 for one off-diagonal pair with count U. */
double orc_p(uint32_t U, int32_t n_i, int32_t n_j);
uint16_t orc_f32_to_f16(float f);
int8_t orc_q_i8(float v, float scale, float zp);   /* rf_quantization_kernels.hpp:24-29 */
uint8_t orc_q_nf4(float v);                        /* rf_quantization_kernels.hpp:37-50 */
uint8_t orc_q_u8(float v, float scale, float zp);
/* reference host min/max rule (cuda/rf_quantization_kernels.cu:107-119) */
void orc_u8_scale_from_minmax(float vmin, float vmax, float* scale, float* zp);

/* ---- packed upper triangle ---------------------------------------------- */

/* Sum over trees of oob bits. */
void orc_nout(const uint8_t* oob, int64_t N, int32_t T, int32_t* nout);

/* Reference-shaped count: per tree bucket the samples by leaf, then for every
 * OOB n and in-bag kk of the bucket add 1 at (min(n,kk), max(n,kk))
 * (src/rf_proximity.cpp:110-230 folded as cuda/rf_proximity_upper_triangle.cu:229-237).
 * U has N(N+1)/2 entries, zeroed here. */
void orc_upper_counts_scatter(const int32_t* leaf, const uint8_t* oob, int64_t N, int32_t T,
                              int32_t nleaf, uint16_t* U);

/* Row-oriented restatement of the same count for rows [r0, r1): for row i
 * and tree t, the members j > i of i's bucket whose OOB bit differs from
 * i's.  Writes the rows' packed entries (diagonal included) starting at
 * idx(r0, r0), in format fmt (see above).  nout may be NULL (computed).
 * threads <= 0 uses the OpenMP default.  Returns 0 on success. */
int orc_upper_rows(const int32_t* leaf, const uint8_t* oob, int64_t N, int32_t T, int32_t nleaf,
                   const int32_t* nout, int fmt, float scale, float zp, int64_t r0, int64_t r1,
                   void* out, int threads);

/* The "both OOB" proximity (R randomForest's oob.prox, named by the
 * benchmark's first configuration), which the reference does not
 * implement: for i != j
 *   num_ij = #{t : oob_i(t), oob_j(t), leaf_i(t) == leaf_j(t), label valid}
 *   den_ij = #{t : oob_i(t), oob_j(t)}
 *   P_ij   = den_ij > 0 ? (float)num_ij / (float)den_ij : 0,   P_ii = 1.
 * Rows [r0, r1) of the packed triangle in fmt 0 (F32, P) or 5 (U16, num;
 * 0 on the diagonal).  A brute force over pairs and trees. */
int orc_both_oob_rows(const int32_t* leaf, const uint8_t* oob, int64_t N, int32_t T, int32_t nleaf, int fmt,
                      int64_t r0, int64_t r1, void* out, int threads);

/* The same, split so the per-tree buckets are built once and rows are
 * produced in several calls (the CPU baseline times them separately).
 * leaf/oob must outlive the index. */
typedef struct orc_index orc_index;
orc_index* orc_index_build(const int32_t* leaf, const uint8_t* oob, int64_t N, int32_t T,
                           int32_t nleaf, const int32_t* nout, int threads);
int orc_index_rows(const orc_index* x, int fmt, float scale, float zp, int64_t r0, int64_t r1,
                   void* out, int threads);
void orc_index_free(orc_index* x);

/* Convert a full packed count triangle to format fmt. */
void orc_upper_from_counts(const uint16_t* U, const int32_t* nout, int64_t N, int fmt, float scale,
                           float zp, void* out);

/* ---- top-K --------------------------------------------------------------- */

/* All-trees semantics (python/randomforest_py.cpp:2496-2568, :624-672):
 * count(q,j) = #{t : qleaf[q*T+t] == ref_leaf[t*N+j], label in [0, nleaf)};
 * the K best j by (count desc, j asc), zero counts included; exclude[q] >= 0
 * removes that j.  exclude may be NULL.  idx_out/cnt_out are Q x K.  The
 * reference compares its int16 labels as they are and never produces one
 * outside [0, nleaf); here, as in the library, such a label matches nothing. */
void orc_topk_all(const int32_t* ref_leaf, int64_t N, int32_t T, int32_t nleaf, const int32_t* qleaf, int64_t Q,
                  int32_t K, const int32_t* exclude, int32_t* idx_out, uint16_t* cnt_out, int threads);

/* OOB-query semantics (src/rf_random_forest.cpp:4677-4782): trees where q is
 * OOB, j != q when exclude_self, counts > 0 only, ordered (count desc, j asc);
 * a query label outside [0, nleaf) matches nothing (its tree still counts in
 * |OOB(q)|).  Returns the number of results (<= K). */
int32_t orc_topk_oob(const int32_t* leaf, const uint8_t* oob, int64_t N, int32_t T, int32_t nleaf, int64_t q,
                     int32_t K, int exclude_self, int32_t* idx_out, uint16_t* cnt_out,
                     float* score_out);

/* ---- per-tree triangles (cuda/rf_proximity_upper_triangle.cu) ------------ */

/* One tree's packed upper triangle over the first np samples (np = n_real
 * when 0 < n_real < N, else N), zeroed first, as the reference's per-tree
 * kernels update it (sample by sample, read-modify-write per pair):
 *   fmt 1 (F16, :149-285): OOB n, in-bag kk of n's terminal node (nodes with
 *         nodesize > 0 or not casewise), entry = half(half_to_float(entry) + w),
 *         w = casewise ? (float)nin[kk]/(float)nodesize : 1;
 *   fmt 3 (NF4, :368-519): the same pairs, nibble = fp32_to_nf4(
 *         nf4_to_fp32(nibble) + w), entry e in byte e/2 at bit (e%2)*4;
 *   fmt 2 (I8, :288-365): every sample n with a terminal node (no OOB test)
 *         and in-bag kk, nodesize > 0, entry += fp32_to_int8(
 *         (float)nin[kk]/(float)nodesize, scale, zp) modulo 256. */
void orc_tree_upper(int fmt, const int32_t* nodestatus, const int32_t* nodextr, const int32_t* nin, int32_t nsample,
                    int32_t nnode, int casewise, int32_t n_real, float scale, float zp, void* out);

/* One tree's RF-GAP FP16 triangle (:1621-1660): OOB i < np with nodextr
 * >= 0, mult = sum of nin over in-bag samples of that node, in-bag j of the
 * node with i <= j < np: entry = half(half_to_float(entry) + nin[j] * (1/mult)). */
void orc_rfgap_tree_upper(const int32_t* nin, const int32_t* nodextr, int32_t nsample, int32_t n_real,
                          uint16_t* out);

/* ---- low rank ------------------------------------------------------------ */

/* Y = P V with P = A A^T / T, A the one-hot leaf matrix (all trees):
 * Y[i] = (1/T) sum_t W_t[leaf_i(t)], W_t[l] = sum_{j: leaf_j(t)=l} V[j].
 * V and Y are N x r row-major double; labels outside [0,nleaf) take no part.
 * threads <= 0: all OpenMP threads; results do not depend on the count. */
void orc_lowrank_pv(const int32_t* leaf, int64_t N, int32_t T, int32_t nleaf, const double* V,
                    int32_t r, double* Y, int threads);

/* ---- quantization dispatcher (cuda/rf_quantization_kernels.cu:195-406) --- */

/* One launch of QuantizationDispatcher::launch_proximity_kernel at `level`
 * (0 FP32 -> double, 1 FP16 -> uint16 half bits, 2 INT8 -> int8 with the
 * dispatcher's scale 1/127 and zero point 0, 3 NF4 -> one byte per entry)
 * into the caller-zeroed column-major N x N `out`: for every sample n with a
 * terminal ordinal k = nodexb[n] >= 0 and every in-bag member kk >= n of
 * node k (CSR ndbegin / npcase as src/rf_proximity.cpp:110-171 builds it),
 * entry n + kk*N takes the weight nin[kk] / nodesize in that level's type. */
void orc_dispatch_prox(int level, const int32_t* nodexb, const int32_t* nin, int32_t nsample,
                       const int32_t* ndbegin, const int32_t* npcase, void* out);

/* ---- pair proximity and outlier scores ------------------------------------ */

/* src/rf_random_forest.cpp:4605-4642: #{t : oob_i(t), leaf_i(t) == leaf_j(t)
 * valid} / |OOB(i)| as a float division; 0 for bad indices or no OOB tree. */
float orc_pair_proximity(const int32_t* leaf, const uint8_t* oob, int64_t N, int32_t T, int32_t nleaf, int64_t i,
                         int64_t j);

/* src/rf_random_forest.cpp:4100-4193 (full / anchor modes): for query q
 * (qleaf[q*T + t], sample-major) against the references (ref_leaf[t*N + j]),
 * c_j = #{t : labels equal and valid}; s = sum over j != exclude[q], c_j > 0,
 * ascending j, in double, of the float (c_j / (float)T)^2; raw_q = (float)s
 * > 1e-10 ? numerator / (float)s : isolated.  exclude may be NULL. */
void orc_outlier_raw(const int32_t* ref_leaf, int64_t N, int32_t T, int32_t nleaf, const int32_t* qleaf, int64_t Q,
                     const int32_t* exclude, float numerator, float isolated, float* raw_out, int threads);

/* src/rf_random_forest.cpp:4196-4273: per class (ascending) or overall,
 * median = sorted[size/2], MAD = sorted |raw - median|[size/2] (1 below
 * 1e-10), score = (raw - median) / MAD.  classes may be NULL. */
void orc_outlier_normalize(const float* raw, int64_t N, const int32_t* classes, float* scores);

/* ---- leaf assignments on a forest ------------------------------------------ */

/* Per tree t (arrays of RandomForest, include/rf_random_forest.hpp: nodestatus
 * / bestvar / xbestsplit [t*maxnode + k], treemap [t*maxnode*2 + 2k (+1)],
 * catgoleft [t*maxnode*maxcat + k*maxcat + c], cat [mdim] or NULL = all
 * numeric) and sample n (X[n*mdim + v]), the node leaf_out[t*N + n]:
 *   mode 0: predict_leaf_assignments' walk (src/rf_random_forest.cpp:4800-4845);
 *   mode 1: training assignment (:1581-1609): OOB samples (nin[t*N+n] == 0)
 *           by cpu_testreebag's walk (src/rf_testreebag.cpp:43-119), in-bag
 *           samples by find_terminal_node (src/rf_random_forest.cpp:3724-3774).
 * A child index outside [0, maxnode) ends a walk (predict: at the parent;
 * find_terminal_node: node 0; testreebag: at the parent); testreebag with a
 * split variable outside [0, mdim) stops at that node; a category code at
 * or above maxcat counts as invalid (cat <= maxcat in a well-formed forest). */
void orc_forest_leaves(int mode, const int32_t* nodestatus, const int32_t* bestvar, const float* xbestsplit,
                       const int32_t* treemap, const int32_t* catgoleft, const int32_t* cat, int32_t T, int32_t maxnode,
                       int32_t maxcat, int32_t mdim, const float* X, int64_t N, const int32_t* nin, int32_t* leaf_out);

#ifdef __cplusplus
}
#endif
#endif
