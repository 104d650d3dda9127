// Device-resident forest index shared by the proximity kernels.
//
// Built once per forest by rfxp_set_forest (rfxp_pack.hip) from the N x T
// leaf matrix and OOB bitmask, then read by the triangle, top-K and
// low-rank kernels.  Layout in HBM:
//   mem  [T][ms]  uint32  sample ids + 1 grouped, per tree, by bucket
//                         b = 2*leaf + oob (buckets hold the samples of one
//                         leaf with one OOB bit); the +1 keeps 0 free as "no
//                         member" for masked loads.  The tree stride ms is N
//                         on the whole-tree packing path, where buckets lie
//                         back to back.  The per-part path places them in
//                         the line-fit layout (fit_start below): a bucket of
//                         at most 32 members never straddles a 128-byte line
//                         and a larger one ends on a line, so ms exceeds N by
//                         the padding bound fit_stride
//   off  [T][2L+1] int32  per-tree bucket starts in mem[t] (off[2L]: the
//                         length used)
//   bend [T][2L]  int32   bucket ends (per-part path; on the whole-tree path
//                         a bucket ends where the next begins, off[b+1])
//   roff [N][ldr] uint32  for sample i and tree t, the byte offset in mem
//                         (4*(t*ms + start)) of the run of i: the bucket of
//                         i's leaf with the other OOB bit holds exactly the
//                         samples that pair with i in tree t
//                         (src/rf_proximity.cpp:179-230).  On the per-part
//                         packing path members are placed part by part
//                         (contiguous sample ranges, ascending), so the run
//                         starts where the members from i's own part begin:
//                         every member j > i is in the run, and of the
//                         members j < i only those of i's part.  On the
//                         whole-tree path the run is the whole bucket
//   rlen [N][ldr] uint16  the run's length in bytes, 4*min(len, REC_LONG);
//                         4*REC_LONG means "REC_LONG or more members: the run
//                         ends where its bucket ends", found in lng below; 0
//                         when i has no valid leaf in t.  In bytes so that
//                         it serves directly as the range of a buffer load.
//                         Rows are ldr = T rounded up to 16 long (padding
//                         trees have empty records), and both arrays have
//                         REC_PAD entries of slack (whole-group record loads)
//   lng  [T][lmax] uint2  per tree, the start and end byte offsets in mem of
//                         the buckets of REC_LONG or more members (lngn[t]
//                         of them, lmax = N / REC_LONG + 1)
//   nout [N] int32, rinv [N] double (nout > 0 ? 1/nout : 1), and the min and
//   max of rinv as IEEE bits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rfxp_internal.hpp"

namespace rfxp {

constexpr uint32_t MEM_ID = 0x7fffffffu;  // the id bits of a mem entry
constexpr uint32_t REC_LONG = 16383u;  // 4*REC_LONG fits the uint16 length
constexpr int64_t MAX_FOREST_N = 0x7ffffffe;
constexpr int REC_PAD = 64;
constexpr int MEM_PAD = 64;                   // readable slack after mem

// Line-fit placement of a tree's buckets (per-part packing path).  A run is
// a suffix of a bucket (from the first member of some part on) and costs one
// 128-byte line of mem per line it touches.  Buckets placed back to back
// straddle line boundaries at random: at N = 100,000 with 2,048 leaves a run
// of ~12 ids touches 1.37 lines on average.  Here buckets are placed in
// groups of FIT_GROUP, each group starting on a line.  Inside a group a
// bucket of at most LINE_IDS members that does not fit in the rest of the
// current line starts on the next one, and a larger bucket is placed so that
// it ends on a line boundary (then every suffix of at most LINE_IDS ids lies
// in its last line).  The same shape then needs 1.03 lines per run.  Each
// non-empty bucket and each group wastes fewer than LINE_IDS ids.
constexpr uint32_t LINE_IDS = 32;  // 128 bytes of 4-byte ids
constexpr int FIT_GROUP = 16;

// Start of a bucket of s members placed at or after pos (ids from a
// line-aligned group start).
__host__ __device__ inline uint32_t fit_start(uint32_t pos, uint32_t s) {
    if (s == 0) return pos;
    const uint32_t r = (0u - pos) & (LINE_IDS - 1u);  // ids left in the current line
    if (s <= LINE_IDS) return s > r ? pos + r : pos;
    return pos + ((0u - (pos + s)) & (LINE_IDS - 1u));
}

// Upper bound of a tree's mem length in the line-fit layout (a multiple of
// LINE_IDS): N members, fewer than LINE_IDS ids of padding per non-empty
// bucket and per group.
__host__ __device__ inline int64_t fit_stride(int64_t N, int32_t nb) {
    const int64_t ng = (nb + FIT_GROUP - 1) / FIT_GROUP;
    const int64_t nonempty = N < nb ? N : nb;
    return (N + (int64_t)(LINE_IDS - 1) * (nonempty + ng) + LINE_IDS - 1) / LINE_IDS * LINE_IDS;
}

struct LeafView {
    const int32_t* leaf;
    int64_t si, st;
    const uint32_t* oob;
    int64_t old;
    int64_t N;
    int32_t T;
    int32_t L;
    // 0: forest buckets b = 2*leaf + oob.  > 0: reference-set buckets
    // b = leaf*nseg + (i >> seg_shift) (top-K: one bucket per leaf and
    // column segment, OOB bits unused).
    int32_t nseg;
    int32_t seg_shift;
};

// Bucket id of sample i in tree t, in two steps, so that a kernel can issue
// the loads of many samples before it uses any of them (a branch on a loaded
// label between the two loads would make every sample wait for its own
// label).  key_load reads the label and, in forest mode, the OOB word of
// sample i (a valid index: the caller clamps it); key_bucket turns them into
// the bucket id (forest: 2 * leaf + OOB bit; reference set: leaf * nseg +
// segment), -1 for an invalid label.
struct KeyLoad {
    int32_t l;
    uint32_t w;
};

__device__ __forceinline__ KeyLoad key_load(const LeafView& v, int64_t i, int32_t t) {
    KeyLoad k;
    k.l = v.leaf[i * v.si + (int64_t)t * v.st];
    k.w = v.nseg > 0 ? 0u : v.oob[(int64_t)t * v.old + (i >> 5)];
    return k;
}

__device__ __forceinline__ int32_t key_bucket(const LeafView& v, KeyLoad k, int64_t i) {
    const uint32_t l = (uint32_t)k.l;
    const uint32_t b = v.nseg > 0 ? l * (uint32_t)v.nseg + (uint32_t)(i >> v.seg_shift)
                                  : 2u * l + ((k.w >> (i & 31)) & 1u);
    return (k.l >= 0 && k.l < v.L) ? (int32_t)b : -1;
}

// Buckets per tree of a view (even: packing windows split at even buckets).
__host__ __device__ inline int32_t view_buckets(const LeafView& v) {
    if (v.nseg == 0) return 2 * v.L;
    const int64_t nb = (int64_t)v.L * v.nseg;
    return (int32_t)((nb + 1) / 2 * 2);
}

// Every buffer of a forest index, as pointers into device memory (the
// context's own buffers, or a static workspace).  Forest mode (v.nseg == 0)
// builds buckets, records, the long-bucket table and nout / rinv / rrange;
// reference mode (top-K, low rank) builds the buckets only.
enum ForestBuf {
    FB_OFF, FB_BEND, FB_MEM, FB_ROFF, FB_RLEN, FB_ROFFT, FB_RLENT, FB_SCRATCH, FB_SCRATCH2, FB_KEY16, FB_NOUT, FB_RINV,
    FB_RRANGE, FB_LNG, FB_LNGN, FB_FLAGS, FB_COUNT
};

// Element counts of each buffer (n[FB_*], 0 when unused) for a view.
struct ForestSizes {
    size_t n[FB_COUNT] = {};
    int64_t ldr = 0;
    int32_t lmax = 0;
    int64_t ms = 0;          // mem stride per tree (ids)
    bool fit = false;        // line-fit bucket layout (per-part path, while T * ms + MEM_PAD < 2^30)
    bool part_path = false;  // per-part packing (forest mode, 2L <= 8192)
    bool seg_path = false;   // per-segment packing (reference mode, L <= 16384)
    bool lds_path = false;   // whole-tree histogram in LDS
    bool tree_rec = false;   // whole-tree records through k_tree_records + k_rec_transpose
};
ForestSizes forest_sizes(const LeafView& v, bool count_nout, int max_lds);
size_t forest_elem_bytes(int k);

// The context's own buffers for sizes z (grown as needed), with off / mem
// the given ones (forest or reference set).
int ctx_forest_bufs(rfxp_ctx* ctx, const ForestSizes& z, DevBuf<int32_t>& off, DevBuf<uint32_t>& mem,
                    ForestBufs& fb);

// Builds the index into fb on ctx->stream (rfxp_pack.hip).  nout_in
// (device int32[N]) or NULL: counted from the OOB bits.
int pack_forest(rfxp_ctx* ctx, const LeafView& v, const int32_t* nout_in, const ForestBufs& fb);

// Argument checks of rfxp_upper-like calls (status, message on ctx), and
// rows [r0, r1) of the triangle of index fb into out on ctx->stream
// (rfxp_triangle.hip).
int upper_check_args(rfxp_ctx* ctx, const char* who, int64_t N, int fmt, float scale, float zp, int64_t r0,
                     int64_t r1, const void* out);
int upper_launch(rfxp_ctx* ctx, const ForestBufs& fb, int64_t N, int32_t T, int fmt, float scale, float zp,
                 int64_t r0, int64_t r1, void* out);

// p[0..n) = val on ctx->stream (a fill kernel, capturable).
void fill_u32(rfxp_ctx* ctx, uint32_t* p, int64_t n, uint32_t val);

}  // namespace rfxp
