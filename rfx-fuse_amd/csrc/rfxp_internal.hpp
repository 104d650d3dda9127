// Host-side internals of librfxprox: the context object behind the C ABI,
// device buffers, error plumbing and launch timing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <map>
#include <string>
#include <vector>

#include "rfx_prox.h"

template <class T>
struct DevBuf {
    T* p = nullptr;
    size_t n = 0;
    // Grows (never shrinks) to hold `count` elements; contents are not kept.
    hipError_t ensure(size_t count) {
        if (count == 0) count = 1;
        if (count <= n) return hipSuccess;
        release();
        hipError_t e = hipMalloc((void**)&p, count * sizeof(T));
        if (e != hipSuccess) {
            p = nullptr;
            n = 0;
            (void)hipGetLastError();
            return e;
        }
        n = count;
        return hipSuccess;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
    }
};

// Every buffer of a forest index (rfxp_forest.hpp, ForestBuf), as pointers
// into device memory: the context's own buffers, or a static workspace.
struct ForestBufs {
    int32_t* off = nullptr;        // [T][nb+1] bucket starts (off[nb]: the tree's used length)
    int32_t* bend = nullptr;       // [T][nb] bucket ends (line-fit layout), or NULL: end = off[b+1]
    uint32_t* mem = nullptr;       // [T][ms] + MEM_PAD members
    uint32_t* roff = nullptr;      // [N][ldr] + REC_PAD records (forest mode)
    uint16_t* rlen = nullptr;
    uint32_t* roffT = nullptr;     // [T][N] tree-major records (whole-tree packing, before k_rec_transpose)
    uint16_t* rlenT = nullptr;
    uint32_t* scratch = nullptr;   // part histograms, or whole-tree counters / cursors
    uint32_t* scratch2 = nullptr;  // [N] OOB counts (nout not given)
    uint16_t* key16 = nullptr;     // [T][ceil8(N)] bucket ids
    int32_t* nout = nullptr;       // [N]
    double* rinv = nullptr;        // [N]
    unsigned long long* rrange = nullptr;  // [2]
    uint2* lng = nullptr;          // [T][lmax] long buckets
    int32_t* lngn = nullptr;       // [T]
    int32_t* flags = nullptr;      // [16] device status words
    int64_t ldr = 0;
    int32_t lmax = 0;
    int64_t ms = 0;                // mem stride per tree (ids): N, or more for the line-fit layout
};

struct KernelTiming {
    double ms = 0.0;
    int64_t launches = 0;
};

struct rfxp_ctx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    int last_status = RFXP_OK;
    std::string last_error;
    int max_lds = 65536;  // dynamic LDS bytes a workgroup may use
    int n_cu = 0;

    // forest state (rfxp_set_forest)
    bool forest_ready = false;
    int64_t N = 0;
    int32_t T = 0;
    int32_t L = 0;
    DevBuf<int32_t> bkt_off;   // T x (2L+1): bucket b = 2*leaf + oob
    DevBuf<int32_t> bkt_end;   // T x 2L: bucket ends of the line-fit layout
    DevBuf<uint32_t> bkt_mem;  // T x ms (+ padding): sample ids grouped by bucket
    int64_t ldr = 0;           // record row stride: T rounded up to 16
    DevBuf<uint32_t> roff;     // N x ldr (+pad): offset of the opposite-OOB bucket of (i, t)
    DevBuf<uint16_t> rlen;     // N x ldr (+pad): its length in bytes (see rfxp_forest.hpp)
    DevBuf<uint2> lng;         // T x lmax: start, end byte offsets of buckets of REC_LONG+ members
    DevBuf<int32_t> lngn;      // T: entries of lng per tree
    int32_t lmax = 0;
    DevBuf<uint32_t> roffT;    // T x N: records, tree-major (whole-tree packing)
    DevBuf<uint16_t> rlenT;
    DevBuf<uint32_t> scratch;  // packing scratch (part histograms, large leaf counts)
    DevBuf<uint32_t> scratch2; // per-sample OOB counts
    DevBuf<uint16_t> key16;    // T x ceil8(N) bucket ids (packing pass B)
    DevBuf<int32_t> nout;      // N
    DevBuf<double> rinv;       // N: nout > 0 ? 1/nout : 1
    DevBuf<unsigned long long> rrange;  // [min, max] of rinv as IEEE bits
    DevBuf<int32_t> flags;     // device status words
    DevBuf<float> mm_ws;       // rfxp_upper_minmax: one band of fp32 entries
    DevBuf<float> mm_part;     // rfxp_upper_minmax: block minima / maxima, then the running pair
    ForestBufs fb;             // the forest index of rfxp_set_forest (pointers into the buffers above)
    const int32_t* fo_leaf = nullptr;   // the caller's leaf matrix and OOB words given to rfxp_set_forest
    int64_t fo_si = 0, fo_st = 0;       // (rfxp_lowrank_oob_pv reads them)
    const uint32_t* fo_oob = nullptr;
    int64_t fo_old = 0;

    // reference set for top-K (rfxp_set_reference)
    bool ref_ready = false;
    int64_t ref_N = 0;
    int32_t ref_T = 0, ref_L = 0, ref_nseg = 0, ref_shift = 0, ref_nb = 0;
    DevBuf<int32_t> ref_off;   // T x (nb+1): bucket b = leaf*nseg + segment
    DevBuf<uint32_t> ref_mem;  // T x N (+ padding)
    const int32_t* ref_leaf = nullptr;  // the caller's leaf matrix (low-rank reads it)
    int64_t ref_si = 0, ref_st = 0;

    // low-rank (rfxp_lowrank_*)
    bool lr_index_ready = false;
    DevBuf<int32_t> lr_start, lr_tot, lr_pmap;  // piece index of the reference set
    DevBuf<float> lr_w, lr_z, lr_tmp;           // W = A^T V, iteration block, scratch
    DevBuf<double> lr_part, lr_rinv;            // Gram partials, R^-1

    // per-tree and dense small-N operations (rfxp_tree.hip)
    DevBuf<int32_t> tr_status, tr_nodextr, tr_nin, tr_term, tr_members, tr_node, tr_pofs;
    DevBuf<int64_t> tr_idx;
    DevBuf<double> tr_w;
    DevBuf<uint32_t> tr_out;
    std::vector<int64_t> tr_idx_host;
    std::vector<double> tr_w_host;
    DevBuf<double> dn_prox, dn_out;
    DevBuf<int32_t> dn_nout;

    // symmetric accumulator of the low-rank class (rfxp_symacc_*)
    int64_t sa_N = 0, sa_nnz = 0;
    bool sa_csr_ok = false;
    bool sa_dense = false;                       // entries in sa_tri instead of the COO list
    DevBuf<int32_t> sa_i, sa_j, sa_col, sa_sv;  // COO rows / cols, CSR columns, RF-GAP counts
    DevBuf<float> sa_v, sa_val;                  // COO / CSR values
    DevBuf<int64_t> sa_cnt, sa_rowptr;
    DevBuf<unsigned long long> sa_deg;
    DevBuf<double> sa_tri;                       // packed upper triangle (dense form)
    DevBuf<double> sa_stage, sa_x, sa_y, sa_z, sa_part, sa_g, sa_w, sa_wv;

    // timing
    bool timing = false;
    std::vector<std::pair<std::string, std::pair<hipEvent_t, hipEvent_t>>> pending;
    std::vector<hipEvent_t> event_pool;
    std::map<std::string, KernelTiming> times;
};

namespace rfxp {

int set_error(rfxp_ctx* ctx, int status, const std::string& msg);
int hip_error(rfxp_ctx* ctx, hipError_t e, const char* what);
// Brackets one launch with events when timing is on.
struct LaunchTimer {
    rfxp_ctx* ctx;
    const char* name;
    hipEvent_t a = nullptr, b = nullptr;
    LaunchTimer(rfxp_ctx* c, const char* n);
    ~LaunchTimer();
};
int check_launch(rfxp_ctx* ctx, const char* what);

// Workgroups of a grid-stride launch over n units, per units per workgroup:
// enough to fill the device, and at most RFXP_GS_MAX_BLOCKS, so that the
// launch's work-items per dimension stay within the dispatch packet's 32
// bits whatever n is.  (The CPU emulation's build lowers the bound, so that
// its tests run every such kernel through several strides.)
#ifndef RFXP_GS_MAX_BLOCKS
#define RFXP_GS_MAX_BLOCKS (1 << 20)
#endif
inline unsigned grid_stride_blocks(int64_t n, int64_t per_block) {
    const int64_t b = (n + per_block - 1) / per_block;
    return (unsigned)(b < (int64_t)(RFXP_GS_MAX_BLOCKS) ? b : (int64_t)(RFXP_GS_MAX_BLOCKS));
}
// Device address of rfxp_upper_noalloc's static workspace on `device`
// (current), taken once per device (rfxp_noalloc.hip).
void noalloc_setup(int device);
bool is_device_pointer(const void* p);
// Failure reporting of the reference-signature layer (rfxp_compat.hip): one
// stderr line, readable through rfx_compat_last_error().
void compat_report(const char* fn, rfxp_ctx* ctx, int rc);
void compat_report_msg(const char* fn, const char* msg);

}  // namespace rfxp

#define RFXP_HIP(ctx, call)                                            \
    do {                                                               \
        hipError_t _e = (call);                                        \
        if (_e != hipSuccess) return rfxp::hip_error((ctx), _e, #call); \
    } while (0)
