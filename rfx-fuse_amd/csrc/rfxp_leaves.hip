// Leaf assignments of samples on a forest, on the device: the producer of
// the leaf matrix and OOB bits that rfxp_set_forest and rfxp_set_reference
// index.  The reference walks trees on the host:
//   * predict_leaf_assignments (src/rf_random_forest.cpp:4789-4852) for new
//     samples;
//   * while training (:1581-1609), OOB samples take the node cpu_testreebag
//     reached (src/rf_testreebag.cpp:13-122) and in-bag samples
//     find_terminal_node's (src/rf_random_forest.cpp:3724-3774).
// The three walks differ in their rules for categorical splits and bad
// inputs; each is restated exactly here.  One thread per (sample, tree):
// the tree's node arrays are small and stay in the caches, the output
// row of a tree is written coalesced, and the OOB bits of 64 samples come
// from one ballot.
#include <algorithm>

#include "rfx_prox.h"
#include "rfxp_internal.hpp"

namespace rfxp {

struct LeafForest {
    const int32_t *ns, *bv, *tm, *cg, *cat;
    const float* sp;
    int32_t T, maxnode, maxcat, mdim;
    const float* X;
    int64_t N;
    const int32_t* nin;  // [T][N], training mode
    int32_t* leaf;       // [T][N]
    uint32_t* oob;       // [T][oob_ld] or NULL
    int64_t oob_ld;
    int mode;
    int terminal_only;   // non-terminal nodes reached -> -1
};

struct TreeView {
    const int32_t *ns, *bv, *tm, *cg, *cat;
    const float* sp;
    int32_t maxnode, maxcat, mdim;
};

__device__ __forceinline__ bool node_ok(const TreeView& t, int32_t k) { return k >= 0 && k < t.maxnode; }

// (int)(f + 0.5) with the sum in double; outside int32: -1 (invalid)
__device__ __forceinline__ int32_t round_cat(float f) {
    const double d = (double)f + 0.5;
    if (!(d > -2147483649.0 && d < 2147483648.0)) return -1;
    return (int32_t)d;
}
__device__ __forceinline__ int32_t trunc_cat(float f) {
    if (!(f > -2147483649.0f && f < 2147483648.0f)) return -1;
    return (int32_t)f;
}

// predict_leaf_assignments (src/rf_random_forest.cpp:4800-4845): up to
// maxnode steps; a bad split variable or category leaves the node as is.
__device__ int32_t walk_predict(const TreeView& t, const float* x) {
    int32_t cur = 0;
    for (int32_t k = 0; k < t.maxnode; ++k) {
        if (t.ns[cur] == -1) break;
        const int32_t v = t.bv[cur];
        int32_t nxt = cur;
        if (v >= 0 && v < t.mdim) {
            const float f = x[v];
            const int32_t c = t.cat ? t.cat[v] : 1;
            if (c == 1) {
                nxt = f <= t.sp[cur] ? t.tm[2 * cur] : t.tm[2 * cur + 1];
            } else {
                const int32_t j = round_cat(f);
                if (j >= 0 && j < c && j < t.maxcat)
                    nxt = t.cg[(int64_t)cur * t.maxcat + j] == 1 ? t.tm[2 * cur] : t.tm[2 * cur + 1];
            }
        }
        if (!node_ok(t, nxt)) break;
        cur = nxt;
    }
    return cur;
}

// find_terminal_node (src/rf_random_forest.cpp:3724-3774): node 0 for a bad
// split variable or category, or when no terminal node is reached.
__device__ int32_t walk_inbag(const TreeView& t, const float* x) {
    int32_t cur = 0;
    for (int32_t k = 0; k < t.maxnode; ++k) {
        if (t.ns[cur] == -1) return cur;
        const int32_t v = t.bv[cur];
        if (!(v >= 0 && v < t.mdim)) return 0;
        const float f = x[v];
        const int32_t c = t.cat ? t.cat[v] : 1;
        int32_t nxt;
        if (c == 1) {
            nxt = f <= t.sp[cur] ? t.tm[2 * cur] : t.tm[2 * cur + 1];
        } else {
            const int32_t j = round_cat(f);
            if (!(j >= 0 && j < c && j < t.maxcat)) return 0;
            nxt = t.cg[(int64_t)cur * t.maxcat + j] == 1 ? t.tm[2 * cur] : t.tm[2 * cur + 1];
        }
        if (!node_ok(t, nxt)) return 0;
        cur = nxt;
    }
    return 0;
}

// cpu_testreebag's walk (src/rf_testreebag.cpp:43-119): split nodes only,
// at most 1000 steps, cat <= 2 (or no cat table) numeric, (int)x codes,
// invalid codes to the right; the node reached if terminal or status 2,
// else 0.
__device__ int32_t walk_oob(const TreeView& t, const float* x) {
    int32_t kt = 0, count = 0;
    while (t.ns[kt] == 1 && count < 1000) {
        ++count;
        const int32_t mvar = t.bv[kt];
        if (!(mvar >= 0 && mvar < t.mdim)) break;
        int32_t nxt;
        if (!t.cat || t.cat[mvar] <= 2) {
            nxt = x[mvar] <= t.sp[kt] ? t.tm[2 * kt] : t.tm[2 * kt + 1];
        } else {
            const int32_t cv = trunc_cat(x[mvar]);
            if (cv >= 0 && cv < t.cat[mvar] && cv < t.maxcat)
                nxt = t.cg[cv + (int64_t)kt * t.maxcat] == 1 ? t.tm[2 * kt] : t.tm[2 * kt + 1];
            else
                nxt = t.tm[2 * kt + 1];
        }
        if (!node_ok(t, nxt)) break;
        kt = nxt;
        if (t.ns[kt] != 1) break;
    }
    return (t.ns[kt] == -1 || t.ns[kt] == 2) ? kt : 0;
}

__global__ __launch_bounds__(256) void k_forest_leaves(LeafForest f) {
    const int32_t tr = blockIdx.y;
    const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
    TreeView t;
    t.ns = f.ns + (int64_t)tr * f.maxnode;
    t.bv = f.bv + (int64_t)tr * f.maxnode;
    t.sp = f.sp + (int64_t)tr * f.maxnode;
    t.tm = f.tm + (int64_t)tr * f.maxnode * 2;
    t.cg = f.cg ? f.cg + (int64_t)tr * f.maxnode * f.maxcat : nullptr;
    t.cat = f.cat;
    t.maxnode = f.maxnode;
    t.maxcat = f.maxcat;
    t.mdim = f.mdim;
    bool is_oob = false;
    if (n < f.N) {
        const float* x = f.X + n * f.mdim;
        int32_t leaf;
        if (f.mode == RFXP_LEAVES_PREDICT) {
            leaf = walk_predict(t, x);
        } else {
            is_oob = f.nin[(int64_t)tr * f.N + n] == 0;
            leaf = is_oob ? walk_oob(t, x) : walk_inbag(t, x);
        }
        if (f.terminal_only && t.ns[leaf] != -1) leaf = -1;
        f.leaf[(int64_t)tr * f.N + n] = leaf;
    }
    if (f.oob) {
        const uint64_t m = __ballot(is_oob);
        const uint32_t lane = threadIdx.x & 63u;
        const int64_t n0 = n - lane;  // first sample of this wave (a multiple of 64)
        if (lane == 0 && n0 < f.N) f.oob[(int64_t)tr * f.oob_ld + (n0 >> 5)] = (uint32_t)m;
        if (lane == 32 && n0 + 32 < f.N) f.oob[(int64_t)tr * f.oob_ld + (n0 >> 5) + 1] = (uint32_t)(m >> 32);
    }
}

}  // namespace rfxp

using namespace rfxp;

extern "C" int rfxp_forest_leaves(rfxp_ctx* ctx, int mode, const int32_t* nodestatus, const int32_t* bestvar,
                                  const float* xbestsplit, const int32_t* treemap, const int32_t* catgoleft,
                                  const int32_t* cat, int32_t T, int32_t maxnode, int32_t maxcat, int32_t mdim,
                                  const float* X, int64_t N, const int32_t* nin, int terminal_only,
                                  int32_t* leaf_out, uint32_t* oob_words, int64_t oob_ld) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (mode != RFXP_LEAVES_PREDICT && mode != RFXP_LEAVES_TRAIN)
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_forest_leaves: mode must be RFXP_LEAVES_PREDICT or _TRAIN");
    if (T < 1 || T > 65535 || maxnode < 1 || mdim < 1 || N < 0 || (cat && maxcat < 1))
        return set_error(ctx, RFXP_ERR_INVALID,
                         "rfxp_forest_leaves: need 1 <= T <= 65535, maxnode >= 1, mdim >= 1, N >= 0, maxcat >= 1 with cat");
    if (N == 0) return RFXP_OK;
    if (!nodestatus || !bestvar || !xbestsplit || !treemap || !X || !leaf_out || (cat && !catgoleft) ||
        (mode == RFXP_LEAVES_TRAIN && !nin))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_forest_leaves: a required array is NULL");
    for (const void* p : {(const void*)nodestatus, (const void*)bestvar, (const void*)xbestsplit, (const void*)treemap,
                          (const void*)X, (const void*)leaf_out})
        if (!is_device_pointer(p)) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_forest_leaves: arrays must be device pointers");
    if ((cat && (!is_device_pointer(cat) || !is_device_pointer(catgoleft))) || (nin && !is_device_pointer(nin)) ||
        (oob_words && !is_device_pointer(oob_words)))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_forest_leaves: arrays must be device pointers");
    if (oob_words && (mode != RFXP_LEAVES_TRAIN || oob_ld < (N + 31) / 32))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_forest_leaves: OOB words need the training mode and oob_ld >= ceil(N/32)");
    if ((N + 255) / 256 > 0x7fffffffLL) return set_error(ctx, RFXP_ERR_UNSUPPORTED, "rfxp_forest_leaves: N too large");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    LeafForest f{nodestatus, bestvar, treemap, cat ? catgoleft : nullptr, cat, xbestsplit, T, maxnode, cat ? maxcat : 1,
                 mdim, X, N, nin, leaf_out, oob_words, oob_ld, mode, terminal_only ? 1 : 0};
    {
        LaunchTimer tm(ctx, "leaves");
        hipLaunchKernelGGL(k_forest_leaves, dim3((unsigned)((N + 255) / 256), (unsigned)T), dim3(256), 0, ctx->stream, f);
    }
    return check_launch(ctx, "k_forest_leaves launch");
}
