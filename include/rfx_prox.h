/*
 * rfx_prox.h -- C ABI of the MI355X (gfx950) proximity library librfxprox.so.
 *
 * Plain pointers and sizes only: no C++ or torch types cross this boundary,
 * and no exception escapes it.  Every function returns RFXP_OK or an error
 * code; the message of the last error on a context is read with
 * rfxp_last_error().  Device pointers are HIP device allocations on the
 * context's device unless a function says "host".
 *
 * The reference's C++ entry points for this path (include/rf_proximity.hpp,
 * rf_finishprox.hpp, rf_proximity_upper_triangle.hpp,
 * rf_quantization_kernels.hpp, rf_proximity_lowrank.hpp,
 * rf_lowrank_helpers.hpp) are re-implemented on top of this ABI with their
 * original signatures in the same library; each function below names the
 * reference interface it serves.
 *
 * Layout conventions
 *   leaf (i, t)   int32 leaf[i*stride_i + t*stride_t]; the reference keeps
 *                 tree-major [t*N + i] (include/rf_random_forest.hpp:496-501,
 *                 stride_i = 1, stride_t = N) and sample-major [i*T + t] for
 *                 new queries (src/rf_random_forest.cpp:4789-4852,
 *                 stride_i = T, stride_t = 1).  Labels outside [0, nleaf)
 *                 mean "no valid terminal node" (src/rf_proximity.cpp:126-135).
 *   oob (i, t)    bit (i & 31) of oob_words[t*oob_ld + (i >> 5)]: 1 when
 *                 sample i is out-of-bag in tree t (nin == 0,
 *                 src/rf_bootstrap.cpp:67-82).
 *   triangle      row-wise packed upper triangle with the diagonal,
 *                 idx(i,j) = i*N - i*(i+1)/2 + j for i <= j, 64-bit
 *                 (cuda/rf_proximity_upper_triangle.cu:34-39).
 */
#ifndef RFX_PROX_H
#define RFX_PROX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define RFXP_OK 0
#define RFXP_ERR_INVALID 1     /* bad argument, size or pointer */
#define RFXP_ERR_HIP 2         /* a HIP runtime call failed */
#define RFXP_ERR_NOMEM 3       /* device allocation failed */
#define RFXP_ERR_STATE 4       /* call out of order (e.g. no forest set) */
#define RFXP_ERR_UNSUPPORTED 5 /* size or mode outside what the kernels handle */

/* Triangle output formats.  The numbering extends the reference's
 * QuantizationLevel (FP32=0, FP16=1, INT8=2, NF4=3;
 * include/rf_quantization_kernels.hpp:13-18). */
#define RFXP_FMT_F32 0 /* (float)P                                        */
#define RFXP_FMT_F16 1 /* IEEE half of (float)P, RN-even                  */
#define RFXP_FMT_I8 2  /* fp32_to_int8((float)P, scale, zp)               */
#define RFXP_FMT_NF4 3 /* fp32_to_nf4((float)P), 2 entries per byte,
                          entry e in byte e/2 at bit (e%2)*4              */
#define RFXP_FMT_U8 4  /* trunc(clamp((float)P / scale + zp, 0, 255))     */
#define RFXP_FMT_U16 5 /* raw co-occurrence count U                       */

typedef struct rfxp_ctx rfxp_ctx;

/* ---- context --------------------------------------------------------- */

/* Creates a context on HIP device `device` with its own stream.
 * Replaces the reference's implicit device-0/stream-0 state
 * (cuda/rf_growtree.cu:5209, cuda/rf_config_cuda.cu:37). */
int rfxp_ctx_create(int device, rfxp_ctx** out);
int rfxp_ctx_destroy(rfxp_ctx* ctx);
/* Work is queued on `hip_stream` (a hipStream_t) from now on; NULL is the
 * null (legacy default) stream.  A new context uses a non-blocking stream of
 * its own, which rfxp_ctx_own_stream returns.  Streams must be of default
 * priority. */
int rfxp_ctx_set_stream(rfxp_ctx* ctx, void* hip_stream);
void* rfxp_ctx_stream(rfxp_ctx* ctx);
void* rfxp_ctx_own_stream(rfxp_ctx* ctx);
int rfxp_sync(rfxp_ctx* ctx);
/* Copies the last error message (NUL-terminated, truncated to n); ctx may
 * be NULL for errors of rfxp_ctx_create.  Returns the last status code. */
int rfxp_last_error(rfxp_ctx* ctx, char* buf, size_t n);
/* Per-kernel timing with HIP events on the context stream (off by
 * default).  rfxp_kernel_time returns the summed milliseconds and launch
 * count of kernel `name` since the last reset. */
int rfxp_set_timing(rfxp_ctx* ctx, int on);
int rfxp_kernel_time(rfxp_ctx* ctx, const char* name, double* ms, int64_t* launches);
int rfxp_reset_timing(rfxp_ctx* ctx);

/* ---- forest leaves (input of the batched paths) ------------------------ */

/* Loads the N x T leaf matrix and OOB bitmask (device pointers, read during
 * this call only) and builds the device-resident bucket index used by the
 * triangle: per tree, samples grouped by (leaf, OOB bit).  nout (device
 * int32[N]) may be NULL, in which case nout_i = number of trees where i is
 * OOB (src/rf_bootstrap.cpp:67-70).  Serves the per-tree accumulation done
 * through rf::cpu_proximity (include/rf_proximity.hpp:10-14) and
 * rf::cuda::gpu_proximity_upper_triangle* (include/rf_proximity_upper_triangle.hpp:42-156)
 * as one batched call over all trees. */
int rfxp_set_forest(rfxp_ctx* ctx, const int32_t* leaf, int64_t stride_i, int64_t stride_t,
                    const uint32_t* oob_words, int64_t oob_ld, int64_t N, int32_t T,
                    int32_t nleaf, const int32_t* nout);

/* Computes rows [row_begin, row_end) of the packed upper triangle over all
 * trees of the current forest and writes them, in format fmt, to the device
 * buffer `out`, whose first entry is idx(row_begin, row_begin).  For NF4,
 * `out` points at the byte holding that entry; nibbles of boundary bytes
 * that belong to entries outside the range are left untouched.
 * The entries are, for i < j (src/rf_proximity.cpp:179-230 with
 * src/rf_finishprox.cpp:12-74):
 *   U_ij = #{t : leaf_i(t) == leaf_j(t) valid, oob_i(t) != oob_j(t)}
 *   P_ij = 0.5 * ((U/2)*r_i + (U/2)*r_j),  r = nout > 0 ? 1/nout : 1
 * and P_ii = 1 (U_ii = 0).  scale/zp are the affine parameters of I8 and U8
 * (finite, scale != 0).  Replaces the N x N double accumulation of
 * rf::cpu_proximity + rf::cpu_finishprox for the large-N case. */
int rfxp_upper(rfxp_ctx* ctx, int fmt, float scale, float zp, int64_t row_begin, int64_t row_end,
               void* out);

/* Size in bytes of the output of rfxp_upper for rows [row_begin, row_end). */
int64_t rfxp_upper_nbytes(int fmt, int64_t N, int64_t row_begin, int64_t row_end);

/* Number of row segments rfxp_upper recounted with 16-bit counters since
 * rfxp_set_forest (their 8-bit counters wrapped; T > 255 only).  Host
 * int64; synchronises the context stream. */
int rfxp_upper_recounts(rfxp_ctx* ctx, int64_t* count);

/* The per-sample nout actually used (device int32[N] copy into `nout`). */
int rfxp_get_nout(rfxp_ctx* ctx, int32_t* nout);

/* Minimum and maximum of the fp32 entries (float)P of rows
 * [row_begin, row_end) of the triangle (diagonal 1 included), as rfxp_upper
 * with RFXP_FMT_F32 writes them, into the host array minmax[2].  This is the
 * data the reference's quantizer rule reads: compute_minmax_kernel and
 * reduce_minmax_final_kernel over static_cast<float> of the proximity values
 * (cuda/rf_quantization_kernels.cu:24-86); rfxp_quant_scale then gives the
 * scale and zero point of compute_scale_from_minmax_kernel (:88-101), for
 * the I8 / U8 formats of rfxp_upper.  The rows are evaluated in bands of at
 * most 2^26 entries into a context workspace (256 MB), never all at once.
 * Needs row_begin < row_end; synchronises the context stream. */
int rfxp_upper_minmax(rfxp_ctx* ctx, int64_t row_begin, int64_t row_end, float* minmax);

/* The reference's affine quantizer parameters from a min and max
 * (cuda/rf_quantization_kernels.cu:88-101, float arithmetic):
 * scale = (max - min) / 255, 1/127 when that is below 1e-10; zp = -min/scale.
 * Host only. */
void rfxp_quant_scale(float min_val, float max_val, float* scale, float* zero_point);

/* Work decomposition of rfxp_upper, host-only (no device needed): row i of
 * the band [row_begin, row_end) is cut into segments of S columns starting
 * at i, i + S, ...; one workgroup slot per segment, rows taken in groups of
 * 8 so that all segments of a row run on one XCD, plus idle slots where a
 * group's rows have fewer segments than its first.  Returns the number of
 * slots (-1 for bad arguments) and, when 0 <= e < that number, the row and
 * first column of the segment of slot e (-1, -1 for an idle slot).
 * rfxp_upper_launches is the number of kernel launches n slots take (at
 * most 2^22 - 8 workgroups of 1024 threads each).  Lets callers size row
 * bands for several devices; no reference counterpart. */
int64_t rfxp_upper_work_item(int64_t N, int32_t S, int64_t row_begin, int64_t row_end, int64_t e,
                             int64_t* row, int64_t* col);
int64_t rfxp_upper_launches(int64_t n_items);

/* How rfxp_set_forest packs a forest of N samples, T trees and nleaf leaves
 * per tree on a device whose workgroups may use max_lds bytes of LDS
 * (163840 on gfx950), host-only.  Large forests with B = 2 * nleaf <= 8192
 * buckets per tree, N >= 32768 and N >= 16 * B have the samples of each
 * tree cut into 8 parts, and each part's members go to their buckets
 * directly (PARTS_DIRECT: parts too large for the staging below) or after a
 * counting sort by bucket in LDS (SORTED2, SORTED4: 2- or 4-byte staging
 * entries, whichever keeps more workgroups per CU).  Other forests take the
 * whole-tree path, with the bucket histogram in one LDS array or in LDS
 * ranges.  Returns one of these codes, -1 for bad arguments.  Lets callers
 * and tests see which kernels a forest takes; no reference counterpart. */
#define RFXP_PACK_PARTS_DIRECT 0
#define RFXP_PACK_PARTS_SORTED2 1
#define RFXP_PACK_PARTS_SORTED4 2
#define RFXP_PACK_TREE_LDS 3
#define RFXP_PACK_TREE_RANGES 4
int rfxp_pack_plan(int64_t N, int32_t T, int32_t nleaf, int32_t max_lds);

/* The "both OOB" proximity (R randomForest's oob.prox), which the reference
 * does not implement -- its rule is OOB x in-bag normalised by nout
 * (src/rf_proximity.cpp:179-230, src/rf_finishprox.cpp:47-73) -- and which
 * the mid-size benchmark configuration's description names.  For i != j
 *   num_ij = #{t : i and j both OOB in t, leaf_i(t) == leaf_j(t), label valid}
 *   den_ij = #{t : i and j both OOB in t}
 *   P_ij   = den_ij > 0 ? (float)num_ij / (float)den_ij : 0,   P_ii = 1,
 * rows [row_begin, row_end) of the packed triangle into `out` (device) as
 * RFXP_FMT_F32 (P) or RFXP_FMT_U16 (num, 0 on the diagonal).  Leaf matrix
 * and OOB words (device) in rfxp_set_forest's layout; no forest index is
 * used.  Work O(N^2 T / 2): a dense tiled kernel, for the sizes a dense
 * N x N result is asked for. */
int rfxp_both_oob(rfxp_ctx* ctx, const int32_t* leaf, int64_t stride_i, int64_t stride_t,
                  const uint32_t* oob_words, int64_t oob_ld, int64_t N, int32_t T, int32_t nleaf, int fmt,
                  int64_t row_begin, int64_t row_end, void* out);
/* ---- allocation-free one-shot triangle ------------------------------------ */

/* Maximum device workspace of rfxp_upper_noalloc, per GPU (64 MiB). */
#define RFXP_UPPER_NOALLOC_MAX_BYTES (64LL << 20)

/* rfxp_set_forest + rfxp_upper (same arguments, same output) in one call
 * that allocates no device memory: the forest index goes to a static
 * workspace of RFXP_UPPER_NOALLOC_MAX_BYTES per GPU, which each GPU the
 * library runs on holds until the process ends.  No counterpart in the
 * reference: it is for callers that cannot allocate (stream capture, tight
 * loops over many small forests, harnesses that forbid hipMalloc).  Forests
 * whose index exceeds the workspace (rfxp_upper_noalloc_workspace) are
 * rejected with RFXP_ERR_UNSUPPORTED.  All calls on one GPU share its
 * workspace: calls that overlap on one GPU race, so callers serialise them
 * (one stream, one host thread at a time).  The context's forest of
 * rfxp_set_forest is left as it was. */
int rfxp_upper_noalloc(rfxp_ctx* ctx, const int32_t* leaf, int64_t stride_i, int64_t stride_t,
                       const uint32_t* oob_words, int64_t oob_ld, int64_t N, int32_t T, int32_t nleaf,
                       const int32_t* nout, int fmt, float scale, float zp, int64_t row_begin, int64_t row_end,
                       void* out);
/* Workspace bytes rfxp_upper_noalloc needs for a forest (host only; -1 for
 * bad arguments); nout_given: a caller nout is passed. */
int64_t rfxp_upper_noalloc_workspace(int64_t N, int32_t T, int32_t nleaf, int nout_given);

/* ---- leaf assignments (producer of the forest input) ---------------------- */

#define RFXP_LEAVES_PREDICT 0 /* predict_leaf_assignments (src/rf_random_forest.cpp:4789-4852) */
#define RFXP_LEAVES_TRAIN 1   /* training assignment (src/rf_random_forest.cpp:1581-1609) */

/* Walks every sample through every tree (device arrays in RandomForest's
 * layout, include/rf_random_forest.hpp: nodestatus / bestvar / xbestsplit
 * [t*maxnode + k], treemap [t*maxnode*2 + 2k (+1)], catgoleft
 * [t*maxnode*maxcat + k*maxcat + c], cat [mdim] or NULL for all-numeric
 * features; X [n*mdim + v] float) and writes the node reached to
 * leaf_out[t*N + n] (int32, tree-major: rfxp_set_forest's stride_i = 1,
 * stride_t = N).
 *   RFXP_LEAVES_PREDICT: predict_leaf_assignments' walk (cat == 1 numeric,
 *     categories (int)(x + 0.5), a bad split variable or category leaves
 *     the walk where it is, at most maxnode steps);
 *   RFXP_LEAVES_TRAIN: with nin [t*N + n] (bootstrap counts), OOB samples
 *     (nin == 0) by cpu_testreebag's walk (src/rf_testreebag.cpp:13-122:
 *     split nodes only, cat <= 2 numeric, categories (int)x, invalid codes
 *     right, the node if terminal or status 2 else 0) and in-bag samples
 *     by find_terminal_node (src/rf_random_forest.cpp:3724-3774: node 0 on
 *     a bad split variable or category); oob_words (optional, T x oob_ld
 *     words) gets the OOB bits in rfxp_set_forest's layout.
 * A child index outside [0, maxnode) ends a walk (predict and testreebag
 * at the parent, find_terminal_node at 0); a category code at or above
 * maxcat is invalid.  The reference keeps the node as int16; here it is
 * int32.  terminal_only != 0 writes -1 where the node reached is not
 * terminal (nodestatus != -1): those samples take no part in the proximity
 * (src/rf_proximity.cpp:126-135), so the output feeds rfxp_set_forest with
 * nleaf = maxnode directly. */
int rfxp_forest_leaves(rfxp_ctx* ctx, int mode, const int32_t* nodestatus, const int32_t* bestvar,
                       const float* xbestsplit, const int32_t* treemap, const int32_t* catgoleft, const int32_t* cat,
                       int32_t T, int32_t maxnode, int32_t maxcat, int32_t mdim, const float* X, int64_t N,
                       const int32_t* nin, int terminal_only, int32_t* leaf_out, uint32_t* oob_words,
                       int64_t oob_ld);

/* ---- top-K similarity retrieval ----------------------------------------- */

/* Indexes a reference set (N samples x T trees of leaf labels, same layout
 * rules as rfxp_set_forest, no OOB bits) for rfxp_topk.  Replaces the
 * per-tree inverted index of RandomForest::get_top_k_similar
 * (src/rf_random_forest.cpp:4644-4675) and the dense scan of
 * predict_top_k_similar (python/randomforest_py.cpp:2534-2545).  T <= 65534. */
int rfxp_set_reference(rfxp_ctx* ctx, const int32_t* leaf, int64_t stride_i, int64_t stride_t, int64_t N,
                       int32_t T, int32_t nleaf);

/* For each of Q queries (leaf labels q_leaf[q*q_stride_i + t*q_stride_t],
 * device), the K (<= 64) reference indices with the largest
 *   count(q, j) = #{t in trees(q) : leaf_q(t) == leaf_j(t), label valid}
 * ordered by (count desc, index asc), into idx_out[q*K + k] (int32) and
 * cnt_out[q*K + k] (uint16), device.
 *   trees(q) = all trees when q_oob_words is NULL (new queries,
 *              python/randomforest_py.cpp:2496-2568); otherwise the trees
 *              whose bit (q & 31) of q_oob_words[t*q_oob_ld + q/32] is set
 *              (OOB queries, src/rf_random_forest.cpp:4677-4782).
 *   exclude_base >= 0: query q never returns reference exclude_base + q
 *              (a training sample querying itself); < 0: nothing excluded.
 *   positive_only: only counts > 0 are returned (OOB-query semantics);
 *              otherwise zero counts fill the list in index order.
 * Slots without a result get index -1 and count 0. */
int rfxp_topk(rfxp_ctx* ctx, const int32_t* q_leaf, int64_t q_stride_i, int64_t q_stride_t, int64_t Q,
              const uint32_t* q_oob_words, int64_t q_oob_ld, int64_t exclude_base, int32_t K,
              int positive_only, int32_t* idx_out, uint16_t* cnt_out);

/* Float scores of rfxp_topk results (Q x K, device): for OOB queries
 * (q_oob_words as given to rfxp_topk) (float)count * (1.0f / |OOB(q)|),
 * the score of RandomForest::get_top_k_similar
 * (src/rf_random_forest.cpp:4744, 4775-4778); for new queries
 * (q_oob_words NULL) (float)count / (float)T, the similarity of
 * predict_top_k_similar (python/randomforest_py.cpp:2538-2550).  Slots
 * without a result (idx < 0) get 0. */
int rfxp_topk_scores(rfxp_ctx* ctx, const uint32_t* q_oob_words, int64_t q_oob_ld, int64_t Q, int32_t T,
                     int32_t K, const int32_t* idx, const uint16_t* cnt, float* score_out);

/* RandomForest::compute_proximity_from_leaves (src/rf_random_forest.cpp:4605-4642)
 * for npairs pairs (pair_i[p], pair_j[p]) (device int64): the float quotient
 *   #{t : i OOB in t, leaf_i(t) == leaf_j(t) valid} / |OOB(i)|
 * into out[p] (device float); 0 when an index is out of range or i is never
 * OOB.  Leaf matrix and OOB bits as for rfxp_set_forest. */
int rfxp_pair_proximity(rfxp_ctx* ctx, const int32_t* leaf, int64_t stride_i, int64_t stride_t,
                        const uint32_t* oob_words, int64_t oob_ld, int64_t N, int32_t T, int32_t nleaf,
                        const int64_t* pair_i, const int64_t* pair_j, int64_t npairs, float* out);

/* ---- outlier scores ----------------------------------------------------- */

/* Raw outlier measure of RandomForest::compute_outlier_scores
 * (src/rf_random_forest.cpp:4100-4193) for Q queries against the current
 * reference set (rfxp_set_reference), all trees:
 *   s_q = sum over references j != excluded of (c_qj / T)^2,
 *   c_qj = #{t : leaf_q(t) == leaf_j(t) valid},
 *   raw_q = s_q > 1e-10 ? numerator / s_q : isolated     (device float[Q]).
 * (c/T) is a float division and its square a float product, as in the
 * reference; the sum runs in double and is rounded to float (the
 * reference's float sum runs in hash-map order).  Full mode: the reference
 * set is the training forest, queries = its samples, exclude_base = 0,
 * numerator = N - 1, isolated = N * 1e10.  Anchor ("greedy") mode: the
 * reference set is the anchors' leaf rows, exclude_idx[q] = the anchor
 * position of sample q or -1 (device int32[Q]; NULL uses exclude_base as in
 * rfxp_topk), numerator = number of anchors, isolated = anchors * 1e10. */
int rfxp_outlier_raw(rfxp_ctx* ctx, const int32_t* q_leaf, int64_t q_stride_i, int64_t q_stride_t, int64_t Q,
                     int64_t exclude_base, const int32_t* exclude_idx, float numerator, float isolated,
                     float* raw_out);

/* Host only (no device): the robust normalisation of the raw scores
 * (src/rf_random_forest.cpp:4196-4273).  classes (host int32[N]) or NULL;
 * per class in ascending class order (one group when NULL): median = the
 * sorted group's element size/2, MAD = the sorted |raw - median|'s element
 * size/2 (1 when below 1e-10), scores[n] = (raw[n] - median) / MAD.
 * medians / mads (host float, one per group) may be NULL. */
int rfxp_outlier_normalize(const float* raw, int64_t N, const int32_t* classes, float* scores, float* medians,
                           float* mads);

/* ---- low-rank form of the all-trees proximity ---------------------------- */

/* Y = P V with P = A A^T / T, A the N x (T*nleaf) one-hot leaf matrix of the
 * reference set (rfxp_set_reference; P_ij = fraction of trees in which i and
 * j share a leaf, P_ii = 1 for valid labels):
 *   Y_i = (1/T) sum_t W_t[leaf_i(t)],  W_t[l] = sum_{j: leaf_j(t) = l} V_j.
 * V, Y: device, N x r row-major fp32, 1 <= r <= 64, not aliased.  Reads the
 * leaf matrix given to rfxp_set_reference, which must still be valid.
 * The SpMM contract of the reference's LowRankProximityMatrix
 * (include/rf_proximity_lowrank.hpp:27-433), without forming P. */
int rfxp_lowrank_pv(rfxp_ctx* ctx, const float* V, int32_t r, float* Y);

/* Subspace iteration for a rank-r factor of P (1 <= r <= 32):
 *   Q_0 = orth(V0), Q_k = orth(P Q_{k-1}) for k = 1..iters, B = Q^T P Q,
 * orth = QR with a positive diagonal of R (CholeskyQR2), so P ~ Q B Q^T.
 * V0, Q: device N x r fp32 (distinct); B: host r x r double, row-major.
 * Synchronises the context stream. */
int rfxp_lowrank_subspace(rfxp_ctx* ctx, const float* V0, int32_t r, int32_t iters, float* Q, double* B);

/* ---- accumulated symmetric proximity and its factor ----------------------
 * The engine of the reference's LowRankProximityMatrix class
 * (include/rf_proximity_lowrank.hpp:27-433, rf_lowrank_helpers.hpp:13-34),
 * which is built on these calls in the same library.  The context holds one
 * accumulator: M = sum of the symmetric contributions added since
 * rfxp_symacc_reset, kept in device memory as a list of the contributions'
 * nonzero entries while that list and its symmetric CSR (28 bytes an entry)
 * take less than the packed upper triangle of M in doubles, and as that
 * triangle from then on.  Its memory is so at most 8 N(N+1)/2 + 24 (N+1)
 * bytes plus one staging buffer for host inputs (at most 256 MiB, or one row
 * and a byte), and up to 1.43 times the triangle while an add switches
 * forms; the number of contributions does not enter. */

/* Empties the accumulator and sets its order N (1 <= N < 2^31 - 1);
 * releases what a previous accumulation held beyond this N's list limit. */
int rfxp_symacc_reset(rfxp_ctx* ctx, int64_t N);
/* Number of stored entries (i <= j) so far: the listed nonzeros, or
 * N(N+1)/2 once the accumulator holds the dense triangle; -1 for a NULL
 * context. */
int64_t rfxp_symacc_nnz(rfxp_ctx* ctx);
/* Bytes of device memory the accumulator holds now (list, CSR, triangle,
 * staging; not the factor's work blocks); -1 for a NULL context.  No
 * counterpart in the reference: it makes the memory bound above checkable. */
int64_t rfxp_symacc_device_bytes(rfxp_ctx* ctx);
/* Adds the symmetric matrix whose packed upper triangle (N(N+1)/2 entries,
 * host or device) is `tri`, read as the reference's low-rank path reads
 * per-tree triangles (cuda/rf_proximity_lowrank.cu:687-789):
 *   RFXP_FMT_F16  IEEE half entries;
 *   RFXP_FMT_F32  float entries;
 *   RFXP_FMT_I8   half((q - zp) * scale) (int8_to_fp32, then FP16);
 *   RFXP_FMT_NF4  half(nf4_to_fp32(nibble)), entry e in byte e/2 at bit (e%2)*4. */
int rfxp_symacc_add_upper(rfxp_ctx* ctx, int fmt, const void* tri, float scale, float zp);
/* Adds the symmetric matrix with upper triangle half((float)full[i*N + j])
 * for i <= j from a dense N x N double (host or device), as
 * add_tree_contribution_incremental reads it (:654-685). */
int rfxp_symacc_add_dense(rfxp_ctx* ctx, const double* full);
/* Y = M X for X, Y device N x b row-major doubles (b >= 1). */
int rfxp_symacc_apply(rfxp_ctx* ctx, const double* X, int32_t b, double* Y);
/* Rank-r factor of M: block subspace iteration (block b = 2r + 16, capped
 * at N, room for the negative eigenvalues of an indefinite M among the
 * largest magnitudes; random normal start from `seed`; `iters` products,
 * each followed by CholeskyQR2 or, for a singular Gram matrix, SVQB), then
 * Rayleigh-Ritz: A[:, c] = Q u_c sqrt(lambda_c) for the r largest Ritz
 * values (descending), a zero column where lambda_c <= 0, so that A A^T is
 * the rank-r positive part of M.  A: device N x r column-major double
 * (the layout of LowRankProximityMatrix::get_factors); evals: host r
 * doubles (the Ritz values) or NULL.  1 <= r <= min(N, 4096). */
int rfxp_symacc_factor(rfxp_ctx* ctx, int32_t rank, int32_t iters, uint64_t seed, double* A, double* evals);

/* P = A B^T (A, B device N x rank column-major) into the device column-major
 * N x N `out`, as reconstruct_full_matrix forms it
 * (cuda/rf_proximity_lowrank.cu:1274-1376): P_ii = 1; with oob_counts (host
 * int32[N], RF-GAP) and w_i = 1/s_i where s_i > 0 (else 1): P_ii = w_i and,
 * for i != j, 0.5 * (P_ij w_lo + P_ij w_hi), lo = min(i,j), hi = max(i,j). */
int rfxp_factor_reconstruct(rfxp_ctx* ctx, const double* A, const double* B, int64_t N, int32_t rank,
                            const int32_t* oob_counts, double* out);
/* Classical MDS from a factor (compute_mds_from_factors, :1902-2498), never
 * forming an N x N matrix: P = A A^T (RF-GAP counts: 0.5 (W P + P W),
 * W = diag(w) as above), m = max_i P_ii (1 when below 1e-10),
 * D = 1 - P/m, C = -1/2 J (D o D) J, J the centring matrix.  The k largest
 * eigenpairs of C by block subspace iteration with Rayleigh-Ritz (block
 * k + 4, at most `iters` products, stopping when the Ritz values settle to
 * 1e-12 relative); coords (host, N x k row-major) = v_c sqrt(|lambda_c|) in
 * descending eigenvalue order; evals (host k) or NULL. */
int rfxp_factor_mds(rfxp_ctx* ctx, const double* A, int64_t N, int32_t rank, int32_t k, const int32_t* oob_counts,
                    int32_t iters, double* coords, double* evals);
/* Factor storage of the reference's quantize_factors / dequantize_factors
 * (:242-400, :1379-1718): F32 and F16 as IEEE halves, I8 as
 * fp32_to_int8((float)a, scale, zp) with (scale, zp) in device memory
 * (scale_zp[0], scale_zp[1]), NF4 two per byte (element e in byte e/2, bits
 * (e%2)*4).  Bytes of `count` quantized elements, or -1. */
int64_t rfxp_factor_quantized_bytes(int level, int64_t count);
int rfxp_factor_quantize(rfxp_ctx* ctx, int level, const double* A, int64_t count, const float* scale_zp, void* q);
int rfxp_factor_dequantize(rfxp_ctx* ctx, int level, const void* q, int64_t count, const float* scale_zp, double* A);

/* Host only: eigenvalues (descending) and, when v is not NULL, eigenvectors
 * (columns of the row-major n x n v) of the symmetric row-major n x n `a`
 * by cyclic Jacobi rotations; the b x b eigensolver of the calls above. */
int rfxp_host_symeig(int32_t n, const double* a, double* w, double* v);

/* Y = P V for the OOB-normalised proximity of the current forest
 * (rfxp_set_forest): P = 1/4 (D^-1 U + U D^-1) + I, U the OOB co-occurrence
 * counts of rfxp_upper (U_ii = 0), D^-1 = diag(nout > 0 ? 1/nout : 1) --
 * the matrix of rf::cpu_finishprox (src/rf_finishprox.cpp:12-74) -- as
 * bucket SpMMs (U = B A^T + A B^T - 2 B B^T, A the one-hot leaf matrix, B
 * its OOB entries), never forming P.  V, Y: device N x r row-major fp32,
 * 1 <= r <= 32, not aliased; sums in double.  Reads the leaf matrix and OOB
 * words given to rfxp_set_forest, which must still be valid. */
int rfxp_lowrank_oob_pv(rfxp_ctx* ctx, const float* V, int32_t r, float* Y);

/* ---- per-tree and dense small-N operations -------------------------------
 * A tree is (nodestatus[nnode], nodextr[N], nin[N]): sample n lies in node
 * nodextr[n], which takes part when nodestatus of it is -1 (terminal);
 * nin[n] is its bootstrap multiplicity, 0 when out-of-bag.  These arrays
 * may be host or device pointers. */

/* The OOB x in-bag pairs of one tree as (n + kk*N, w), the terms that
 * rf::cpu_proximity adds into its column-major N x N matrix
 * (src/rf_proximity.cpp:99-231, dense branch): OOB n, in-bag kk of n's
 * terminal node, w = casewise ? nin[kk]/nodesize : 1, nodes with nodesize
 * = 0 skipped when casewise.  *idx_host / *w_host point into host memory
 * owned by the context, valid until its next call. */
int rfxp_tree_pairs(rfxp_ctx* ctx, const int32_t* nodestatus, const int32_t* nodextr, const int32_t* nin,
                    int32_t N, int32_t nnode, int casewise, int64_t** idx_host, double** w_host, int64_t* npairs);

/* prox[idx] += w over the pairs of rfxp_tree_pairs: one call of
 * rf::cpu_proximity / rf::gpu_proximity (include/rf_proximity.hpp:10-21) on
 * the caller's host matrix prox (N x N, column-major). */
int rfxp_tree_accumulate(rfxp_ctx* ctx, const int32_t* nodestatus, const int32_t* nodextr, const int32_t* nin,
                         int32_t N, int32_t nnode, int casewise, double* prox);

/* One tree's packed upper triangle over the first np samples (np = n_real
 * when 0 < n_real < N, else N), zeroed first, host or device output, in the
 * per-tree formats of cuda/rf_proximity_upper_triangle.cu:
 *   RFXP_FMT_F16: OOB n x in-bag kk, entry = half(w), w as above in float
 *                 (gpu_proximity_upper_triangle_fp16, :149-285);
 *   RFXP_FMT_NF4: the same pairs, entry = fp32_to_nf4(w) (:368-519);
 *   RFXP_FMT_I8:  every sample n with a terminal node x in-bag kk,
 *                 entry += fp32_to_int8(nin[kk]/nodesize, scale, zp)
 *                 modulo 256 (:288-365).
 * A device output is written in place when 4-byte aligned with a byte size
 * divisible by 4, else through a staging buffer; exactly the triangle's
 * bytes are written either way. */
int rfxp_tree_upper(rfxp_ctx* ctx, int fmt, const int32_t* nodestatus, const int32_t* nodextr, const int32_t* nin,
                    int32_t N, int32_t nnode, int casewise, int32_t n_real, float scale, float zp, void* out);

/* One tree's RF-GAP contributions as an FP16 packed upper triangle over the
 * first np samples (cuda/rf_proximity_upper_triangle.cu:1621-1660): OOB i,
 * in-bag j >= i of the same node (raw nodextr values, >= 0), entry =
 * half(c_j / sum c over the node's in-bag samples). */
int rfxp_rfgap_tree_upper(rfxp_ctx* ctx, const int32_t* nin, const int32_t* nodextr, int32_t N, int32_t n_real,
                          uint16_t* out);

/* rf::cpu_finishprox (src/rf_finishprox.cpp:12-74) on dense N x N
 * column-major matrices (host or device): proxsym_ii = 1, and for i != j
 * the reference's symmetrise / nout-normalise / symmetrise in the same IEEE
 * double operations. */
int rfxp_finishprox(rfxp_ctx* ctx, int32_t N, const int32_t* nout, const double* prox, double* proxsym);

/* rf::cpu_proximity_rfgap (src/rf_proximity.cpp:238-397): RF-GAP proximity
 * of T trees given tree-major nin / nodextr [t*N + i], into the dense N x N
 * column-major prox (host or device), symmetrised; each entry summed over
 * trees in ascending order as the reference does. */
int rfxp_rfgap(rfxp_ctx* ctx, int32_t T, int32_t N, const int32_t* nin_flat, const int32_t* nodextr_flat,
               double* prox);

#ifdef __cplusplus
}
#endif
#endif
