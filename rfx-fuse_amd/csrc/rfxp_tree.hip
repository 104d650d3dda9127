// Per-tree and dense (small-N) proximity operations behind the
// reference's per-tree entry points, plus RF-GAP and the dense finishprox.
//
//   rfxp_tree_pairs      one tree (nodestatus, nodextr, nin): the OOB x
//                        in-bag pairs of each terminal node and their
//                        weights, as (n + kk*N, w) -- what rf::cpu_proximity
//                        adds into its column-major N x N matrix
//                        (src/rf_proximity.cpp:99-231, dense branch)
//   rfxp_tree_upper      one tree's packed upper triangle in the formats
//                        of gpu_proximity_upper_triangle_{fp16,int8,nf4}
//                        (cuda/rf_proximity_upper_triangle.cu:149-519)
//   rfxp_rfgap_tree_upper  one tree's RF-GAP fp16 triangle
//                        (cuda/rf_proximity_upper_triangle.cu:1621-1660)
//   rfxp_finishprox      rf::cpu_finishprox on a dense N x N matrix
//                        (src/rf_finishprox.cpp:12-74)
//   rfxp_rfgap           rf::cpu_proximity_rfgap (src/rf_proximity.cpp:238-397)
//
// A tree is staged on the device and grouped by terminal node: node of
// sample n is nodextr[n] when it indexes a terminal node (nodestatus ==
// -1), else none; per node, the in-bag member list (CSR, counting sort) and
// nodesize = sum of nin over in-bag members.  Pair enumeration and the
// per-format triangle writes are per-sample kernels over those lists.
#include <string.h>

#include <algorithm>
#include <vector>

#include "rfxp_device.hpp"
#include "rfxp_internal.hpp"

namespace rfxp {

constexpr int32_t NODE_TERMINAL = -1;  // nodestatus value of a terminal node
// Dense N x N outputs: one thread per entry in a 1-D grid, whose work-item
// count must stay below 2^32.
constexpr int64_t DENSE_MAX_ENTRIES = (int64_t)1 << 31;

struct TreeDev {
    const int32_t* status;  // [nnode]
    const int32_t* nodextr; // [N]
    const int32_t* nin;     // [N]
    int32_t N, nnode;
    int32_t* term;          // [N]: node of n or -1
    int32_t* inb_cnt;       // [nnode + 1] in-bag members per node -> CSR offsets
    int32_t* nodesize;      // [nnode] sum of nin over in-bag members
    int32_t* cursor;        // [nnode]
    int32_t* members;       // [N] in-bag members grouped by node
};

__global__ void k_tree_fill(int32_t* p, int64_t n, int32_t v) {
    for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < n; k += (int64_t)gridDim.x * blockDim.x)
        p[k] = v;
}

__global__ void k_tree_term(TreeDev d) {
    const int32_t n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= d.N) return;
    const int32_t node = d.nodextr[n];
    const bool ok = node >= 0 && node < d.nnode && d.status[node] == NODE_TERMINAL;
    d.term[n] = ok ? node : -1;
    if (ok && d.nin[n] > 0) {
        atomicAdd(&d.inb_cnt[node], 1);
        atomicAdd(&d.nodesize[node], d.nin[n]);
    }
}

// Exclusive scan of n int32 values in place (one 1024-thread workgroup),
// total into *tot.
__global__ __launch_bounds__(1024) void k_tree_scan(int32_t* p, int32_t n, int32_t* tot) {
    __shared__ int32_t part[1024];
    const int32_t chunk = (n + 1023) / 1024;
    const int32_t a = threadIdx.x * chunk, b = min(n, a + chunk);
    int32_t s = 0;
    for (int32_t k = a; k < b; ++k) s += p[k];
    part[threadIdx.x] = s;
    __syncthreads();
    for (int d = 1; d < 1024; d <<= 1) {
        const int32_t v = threadIdx.x >= (unsigned)d ? part[threadIdx.x - d] : 0;
        __syncthreads();
        part[threadIdx.x] += v;
        __syncthreads();
    }
    int32_t run = part[threadIdx.x] - s;
    for (int32_t k = a; k < b; ++k) {
        const int32_t c = p[k];
        p[k] = run;
        run += c;
    }
    if (threadIdx.x == 1023 && tot) *tot = part[1023];
}

__global__ void k_tree_place(TreeDev d) {
    const int32_t n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= d.N) return;
    const int32_t node = d.term[n];
    if (node < 0 || d.nin[n] <= 0) return;
    const int32_t pos = d.inb_cnt[node] + atomicAdd(&d.cursor[node], 1);
    d.members[pos] = n;
}

// Pairs per OOB sample n (its node's in-bag members when the node takes
// part), for the pair offsets.
__global__ void k_tree_npairs(TreeDev d, int32_t casewise, int32_t* np) {
    const int32_t n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= d.N) return;
    int32_t c = 0;
    const int32_t node = d.term[n];
    if (d.nin[n] == 0 && node >= 0 && (d.nodesize[node] > 0 || !casewise))
        c = d.inb_cnt[node + 1] - d.inb_cnt[node];
    np[n] = c;
}

// (n + kk*N, w): w = nin[kk]/nodesize (double division) when casewise with
// nodesize > 0, else 1 (src/rf_proximity.cpp:196-223).
__global__ void k_tree_pairs(TreeDev d, int32_t casewise, const int32_t* pofs, int64_t* idx, double* w) {
    const int32_t n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= d.N) return;
    const int32_t node = d.term[n];
    if (d.nin[n] != 0 || node < 0) return;
    const int32_t nsz = d.nodesize[node];
    if (!(nsz > 0 || !casewise)) return;
    int32_t o = pofs[n];
    for (int32_t p = d.inb_cnt[node]; p < d.inb_cnt[node + 1]; ++p) {
        const int32_t kk = d.members[p];
        idx[o] = (int64_t)n + (int64_t)kk * d.N;
        w[o] = (casewise && nsz > 0) ? (double)d.nin[kk] / (double)nsz : 1.0;
        ++o;
    }
}

__device__ __forceinline__ int64_t tri_ix(int64_t n, int64_t i, int64_t j) { return i * n - i * (i + 1) / 2 + j; }

// Per-tree FP16 / NF4 triangle (cuda/rf_proximity_upper_triangle.cu:149-285,
// :368-519): OOB n < np, in-bag kk < np of its terminal node, entry
// (min, max) += w with w = casewise ? (float)nin[kk]/(float)nodesize : 1.
// Within one tree an entry receives at most one pair (one side OOB, the
// other in-bag), so the accumulation is a store of the converted weight.
template <int F>
__global__ void k_tree_tri(TreeDev d, int32_t casewise, int32_t np, void* out) {
    const int32_t n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= np || d.nin[n] != 0) return;
    const int32_t node = d.term[n];
    if (node < 0) return;
    const int32_t nsz = d.nodesize[node];
    if (!(nsz > 0 || !casewise)) return;
    for (int32_t p = d.inb_cnt[node]; p < d.inb_cnt[node + 1]; ++p) {
        const int32_t kk = d.members[p];
        if (kk >= np) continue;
        const float w = casewise ? (float)d.nin[kk] / (float)nsz : 1.0f;
        const int64_t e = tri_ix(np, min(n, kk), max(n, kk));
        if constexpr (F == F16) {
            ((uint16_t*)out)[e] = f32_to_f16_bits(0.0f + w);
        } else {  // NF4: nibble e%2 of byte e/2, into a zeroed buffer
            const uint32_t code = q_nf4(0.0f + w);
            const uint64_t byte = (uint64_t)e >> 1;
            uint32_t* word = (uint32_t*)((char*)out + (byte & ~(uint64_t)3));
            atomicOr(word, code << ((uint32_t)(byte & 3u) * 8u + (uint32_t)(e & 1) * 4u));
        }
    }
}

// Per-tree INT8 triangle (cuda/rf_proximity_upper_triangle.cu:288-365): as
// that kernel, every sample n < np with a terminal node (OOB or not) and
// every in-bag kk < np of the node add fp32_to_int8(nin[kk]/nodesize) to
// entry (min(n,kk), max(n,kk)), wrapping modulo 256; only nodes with
// nodesize > 0.
__global__ void k_tree_tri_i8(TreeDev d, int32_t np, float scale, float zp, int8_t* out) {
    const int32_t n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= np) return;
    const int32_t node = d.term[n];
    if (node < 0) return;
    const int32_t nsz = d.nodesize[node];
    if (nsz <= 0) return;
    for (int32_t p = d.inb_cnt[node]; p < d.inb_cnt[node + 1]; ++p) {
        const int32_t kk = d.members[p];
        if (kk >= np) continue;
        const float w = (float)d.nin[kk] / (float)nsz;
        const uint32_t q = (uint32_t)(uint8_t)(int8_t)q_i8(w, scale, zp);
        const int64_t e = tri_ix(np, min(n, kk), max(n, kk));
        uint32_t* word = (uint32_t*)((char*)out + (e & ~(int64_t)3));
        const uint32_t sh = (uint32_t)(e & 3) * 8u;
        uint32_t old = *word, assumed;
        do {
            assumed = old;
            const uint32_t b = ((assumed >> sh) + q) & 0xffu;
            old = atomicCAS(word, assumed, (assumed & ~(0xffu << sh)) | (b << sh));
        } while (old != assumed);
    }
}

// Per-tree RF-GAP FP16 triangle (cuda/rf_proximity_upper_triangle.cu:1621-1660):
// OOB i < np with a node >= 0; mult = sum of c_j over in-bag j of that node
// (all samples); for in-bag j of the node with i <= j < np, entry (i, j)
// gets (float)c_j * (1/(float)mult).  Nodes are raw nodextr values here.
__global__ void k_rfgap_tree_tri(const int32_t* nin, const int32_t* ndx, int32_t N, int32_t np, uint16_t* out) {
    const int32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= np || nin[i] != 0) return;
    const int32_t node = ndx[i];
    if (node < 0) return;
    int32_t mult = 0;
    for (int32_t j = 0; j < N; ++j)
        if (nin[j] > 0 && ndx[j] == node) mult += nin[j];
    if (mult == 0) return;
    const float inv = 1.0f / (float)mult;
    for (int32_t j = i; j < np; ++j)
        if (nin[j] > 0 && ndx[j] == node) out[tri_ix(np, i, j)] = f32_to_f16_bits(0.0f + (float)nin[j] * inv);
}

// Dense finishprox: proxsym = P with, for i != j,
//   avg = (prox_ij + prox_ji) / 2.0; a = nout_i > 0 ? avg * (1.0/nout_i) : avg;
//   b = nout_j > 0 ? avg * (1.0/nout_j) : avg; P_ij = 0.5 * (a + b)
// and P_ii = 1 -- the reference's four passes entry by entry, same IEEE
// operations.  Column-major, one thread per entry.
__global__ void k_finishprox(int64_t N, const int32_t* nout, const double* prox, double* proxsym) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= N * N) return;
    const int64_t i = e % N, j = e / N;
    if (i == j) {
        proxsym[e] = 1.0;
        return;
    }
    const double avg = (prox[i + j * N] + prox[j + i * N]) / 2.0;
    const double a = nout[i] > 0 ? avg * (1.0 / (double)nout[i]) : avg;
    const double b = nout[j] > 0 ? avg * (1.0 / (double)nout[j]) : avg;
    proxsym[e] = 0.5 * (a + b);
}

// RF-GAP rows (src/rf_proximity.cpp:238-375): one workgroup per sample i,
// trees in ascending order; row i of the (not yet symmetrised) matrix goes
// to R[i*N + j] (row-major scratch).  Each thread owns columns j = tid mod
// 256, so every entry is summed in tree order.
__global__ __launch_bounds__(256) void k_rfgap_rows(int32_t T, int32_t N, const int32_t* nin_f, const int32_t* ndx_f,
                                                   double* R) {
    __shared__ int32_t red[4];
    const int32_t i = blockIdx.x;
    double* row = R + (int64_t)i * N;
    for (int32_t j = threadIdx.x; j < N; j += 256) row[j] = 0.0;
    int32_t n_oob = 0;
    for (int32_t t = 0; t < T; ++t) {
        const int32_t* nin = nin_f + (int64_t)t * N;
        const int32_t* ndx = ndx_f + (int64_t)t * N;
        if (nin[i] != 0) continue;
        ++n_oob;
        const int32_t node = ndx[i];
        if (node < 0) continue;
        int32_t m = 0;
        for (int32_t j = threadIdx.x; j < N; j += 256)
            if (nin[j] > 0 && ndx[j] == node) m += nin[j];
#pragma unroll
        for (int d = 32; d > 0; d >>= 1) m += __shfl_xor(m, d, 64);
        __syncthreads();
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
        __syncthreads();
        const int32_t mult = red[0] + red[1] + red[2] + red[3];
        if (mult == 0) continue;
        const double inv = 1.0 / (double)mult;
        for (int32_t j = threadIdx.x; j < N; j += 256)
            if (nin[j] > 0 && ndx[j] == node) row[j] += (double)nin[j] * inv;
    }
    if (n_oob == 0) {
        // the thread that zeroed row[i] sets it (no barrier was passed)
        if (threadIdx.x == (uint32_t)(i & 255)) row[i] = 1.0;
        return;
    }
    const double norm = 1.0 / (double)n_oob;
    for (int32_t j = threadIdx.x; j < N; j += 256) row[j] *= norm;
}

// Symmetrise (src/rf_proximity.cpp:383-396) into the column-major output.
__global__ void k_rfgap_sym(int64_t N, const double* R, double* prox) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= N * N) return;
    const int64_t i = e % N, j = e / N;  // output (i, j) at i + j*N
    if (i == j) {
        prox[e] = R[i * N + i];
        return;
    }
    const int64_t a = min(i, j), b = max(i, j);
    // p(a, b) = R[a][b] before symmetrisation; avg = (p(a,b) + p(b,a)) / 2.0
    prox[e] = (R[a * N + b] + R[b * N + a]) / 2.0;
}

static int64_t cdiv64(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Stages a tree (host or device arrays) and builds its node lists.
static int stage_tree(rfxp_ctx* ctx, const int32_t* nodestatus, const int32_t* nodextr, const int32_t* nin,
                      int32_t N, int32_t nnode, TreeDev& d) {
    hipStream_t s = ctx->stream;
    const size_t n1 = (size_t)std::max(N, 1), m1 = (size_t)std::max(nnode, 1) + 1;
    RFXP_HIP(ctx, ctx->tr_status.ensure(m1));
    RFXP_HIP(ctx, ctx->tr_nodextr.ensure(n1));
    RFXP_HIP(ctx, ctx->tr_nin.ensure(n1));
    RFXP_HIP(ctx, ctx->tr_term.ensure(n1));
    RFXP_HIP(ctx, ctx->tr_members.ensure(n1));
    RFXP_HIP(ctx, ctx->tr_node.ensure(3 * m1));
    RFXP_HIP(ctx, hipMemcpyAsync(ctx->tr_status.p, nodestatus, sizeof(int32_t) * nnode, hipMemcpyDefault, s));
    RFXP_HIP(ctx, hipMemcpyAsync(ctx->tr_nodextr.p, nodextr, sizeof(int32_t) * N, hipMemcpyDefault, s));
    RFXP_HIP(ctx, hipMemcpyAsync(ctx->tr_nin.p, nin, sizeof(int32_t) * N, hipMemcpyDefault, s));
    d.status = ctx->tr_status.p;
    d.nodextr = ctx->tr_nodextr.p;
    d.nin = ctx->tr_nin.p;
    d.N = N;
    d.nnode = nnode;
    d.term = ctx->tr_term.p;
    d.inb_cnt = ctx->tr_node.p;
    d.nodesize = ctx->tr_node.p + m1;
    d.cursor = ctx->tr_node.p + 2 * m1;
    d.members = ctx->tr_members.p;
    hipLaunchKernelGGL(k_tree_fill, dim3((unsigned)std::min<int64_t>(cdiv64(3 * m1, 256), 4096)), dim3(256), 0, s,
                       ctx->tr_node.p, (int64_t)(3 * m1), 0);
    if (N > 0) {
        hipLaunchKernelGGL(k_tree_term, dim3((unsigned)cdiv64(N, 256)), dim3(256), 0, s, d);
        hipLaunchKernelGGL(k_tree_scan, dim3(1), dim3(1024), 0, s, d.inb_cnt, nnode + 1, (int32_t*)nullptr);
        hipLaunchKernelGGL(k_tree_place, dim3((unsigned)cdiv64(N, 256)), dim3(256), 0, s, d);
    }
    return check_launch(ctx, "tree staging");
}

}  // namespace rfxp

using namespace rfxp;

extern "C" int rfxp_tree_pairs(rfxp_ctx* ctx, const int32_t* nodestatus, const int32_t* nodextr, const int32_t* nin,
                               int32_t N, int32_t nnode, int casewise, int64_t** idx_host, double** w_host,
                               int64_t* npairs) {
    if (!ctx || !npairs || !idx_host || !w_host) return RFXP_ERR_INVALID;
    *npairs = 0;
    *idx_host = nullptr;
    *w_host = nullptr;
    if (N < 0 || nnode < 0 || (N > 0 && (!nodextr || !nin)) || (nnode > 0 && !nodestatus))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_tree_pairs: bad arguments");
    if (N == 0) return RFXP_OK;
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    TreeDev d;
    if (int rc = stage_tree(ctx, nodestatus, nodextr, nin, N, nnode, d)) return rc;
    hipStream_t s = ctx->stream;
    RFXP_HIP(ctx, ctx->tr_pofs.ensure((size_t)N + 1));
    hipLaunchKernelGGL(k_tree_npairs, dim3((unsigned)cdiv64(N, 256)), dim3(256), 0, s, d, casewise, ctx->tr_pofs.p);
    hipLaunchKernelGGL(k_tree_scan, dim3(1), dim3(1024), 0, s, ctx->tr_pofs.p, N, ctx->tr_pofs.p + N);
    if (int rc = check_launch(ctx, "k_tree_npairs")) return rc;
    int32_t total = 0;
    RFXP_HIP(ctx, hipMemcpyAsync(&total, ctx->tr_pofs.p + N, sizeof(int32_t), hipMemcpyDeviceToHost, s));
    RFXP_HIP(ctx, hipStreamSynchronize(s));
    if (total > 0) {
        RFXP_HIP(ctx, ctx->tr_idx.ensure((size_t)total));
        RFXP_HIP(ctx, ctx->tr_w.ensure((size_t)total));
        hipLaunchKernelGGL(k_tree_pairs, dim3((unsigned)cdiv64(N, 256)), dim3(256), 0, s, d, casewise,
                           ctx->tr_pofs.p, ctx->tr_idx.p, ctx->tr_w.p);
        if (int rc = check_launch(ctx, "k_tree_pairs")) return rc;
        ctx->tr_idx_host.resize((size_t)total);
        ctx->tr_w_host.resize((size_t)total);
        RFXP_HIP(ctx, hipMemcpyAsync(ctx->tr_idx_host.data(), ctx->tr_idx.p, sizeof(int64_t) * total,
                                     hipMemcpyDeviceToHost, s));
        RFXP_HIP(ctx, hipMemcpyAsync(ctx->tr_w_host.data(), ctx->tr_w.p, sizeof(double) * total,
                                     hipMemcpyDeviceToHost, s));
        RFXP_HIP(ctx, hipStreamSynchronize(s));
        *idx_host = ctx->tr_idx_host.data();
        *w_host = ctx->tr_w_host.data();
    }
    *npairs = total;
    return RFXP_OK;
}

extern "C" int rfxp_tree_accumulate(rfxp_ctx* ctx, const int32_t* nodestatus, const int32_t* nodextr,
                                    const int32_t* nin, int32_t N, int32_t nnode, int casewise, double* prox) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (N > 0 && !prox) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_tree_accumulate: prox is NULL");
    if (N > 0 && is_device_pointer(prox))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_tree_accumulate: prox is the caller's host matrix");
    int64_t* idx = nullptr;
    double* w = nullptr;
    int64_t np = 0;
    if (int rc = rfxp_tree_pairs(ctx, nodestatus, nodextr, nin, N, nnode, casewise, &idx, &w, &np)) return rc;
    for (int64_t k = 0; k < np; ++k) prox[idx[k]] += w[k];
    return RFXP_OK;
}

extern "C" int rfxp_tree_upper(rfxp_ctx* ctx, int fmt, const int32_t* nodestatus, const int32_t* nodextr,
                               const int32_t* nin, int32_t N, int32_t nnode, int casewise, int32_t n_real,
                               float scale, float zp, void* out) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (fmt != F16 && fmt != I8 && fmt != NF4)
        return set_error(ctx, RFXP_ERR_UNSUPPORTED, "rfxp_tree_upper: formats F16, I8, NF4");
    if (N < 0 || nnode < 0 || !out) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_tree_upper: bad arguments");
    const int32_t np = (n_real > 0 && n_real < N) ? n_real : N;
    const int64_t ne = (int64_t)np * (np + 1) / 2;
    const int64_t nbytes = fmt == F16 ? 2 * ne : fmt == I8 ? ne : (ne + 1) / 2;
    if (N == 0 || ne == 0) return RFXP_OK;
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    TreeDev d;
    if (int rc = stage_tree(ctx, nodestatus, nodextr, nin, N, nnode, d)) return rc;
    hipStream_t s = ctx->stream;
    // The kernels update whole 32-bit words, so they write the caller's
    // device buffer directly only when it is word-aligned and word-sized;
    // otherwise (and for host outputs) they write a staging buffer whose
    // first nbytes are then copied out.
    const bool dev_out = is_device_pointer(out);
    const bool direct = dev_out && !((uintptr_t)out & 3u) && !(nbytes & 3);
    char* o = (char*)out;
    const int64_t nw = cdiv64(nbytes, 4);
    if (!direct) {
        RFXP_HIP(ctx, ctx->tr_out.ensure((size_t)nw));
        o = (char*)ctx->tr_out.p;
    }
    hipLaunchKernelGGL(k_tree_fill, dim3((unsigned)std::min<int64_t>(cdiv64(nw, 256), 65536)), dim3(256), 0, s,
                       (int32_t*)o, nw, 0);
    const dim3 g((unsigned)cdiv64(np, 256));
    if (fmt == F16) hipLaunchKernelGGL(k_tree_tri<F16>, g, dim3(256), 0, s, d, casewise, np, (void*)o);
    else if (fmt == NF4) hipLaunchKernelGGL(k_tree_tri<NF4>, g, dim3(256), 0, s, d, casewise, np, (void*)o);
    else hipLaunchKernelGGL(k_tree_tri_i8, g, dim3(256), 0, s, d, np, scale, zp, (int8_t*)o);
    if (int rc = check_launch(ctx, "k_tree_tri")) return rc;
    if (!direct) {
        RFXP_HIP(ctx, hipMemcpyAsync(out, o, (size_t)nbytes, dev_out ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost,
                                     s));
        if (!dev_out) RFXP_HIP(ctx, hipStreamSynchronize(s));
    }
    return RFXP_OK;
}

extern "C" int rfxp_rfgap_tree_upper(rfxp_ctx* ctx, const int32_t* nin, const int32_t* nodextr, int32_t N,
                                     int32_t n_real, uint16_t* out) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (N < 0 || (N > 0 && (!nin || !nodextr || !out)))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_rfgap_tree_upper: bad arguments");
    const int32_t np = (n_real > 0 && n_real < N) ? n_real : N;
    const int64_t ne = (int64_t)np * (np + 1) / 2;
    if (ne == 0) return RFXP_OK;
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    hipStream_t s = ctx->stream;
    RFXP_HIP(ctx, ctx->tr_nin.ensure((size_t)N));
    RFXP_HIP(ctx, ctx->tr_nodextr.ensure((size_t)N));
    RFXP_HIP(ctx, hipMemcpyAsync(ctx->tr_nin.p, nin, sizeof(int32_t) * N, hipMemcpyDefault, s));
    RFXP_HIP(ctx, hipMemcpyAsync(ctx->tr_nodextr.p, nodextr, sizeof(int32_t) * N, hipMemcpyDefault, s));
    const bool dev_out = is_device_pointer(out);
    const bool direct = dev_out && !((uintptr_t)out & 3u) && !((2 * ne) & 3);
    uint16_t* o = out;
    const int64_t nw = cdiv64(2 * ne, 4);
    if (!direct) {
        RFXP_HIP(ctx, ctx->tr_out.ensure((size_t)nw));
        o = (uint16_t*)ctx->tr_out.p;
    }
    hipLaunchKernelGGL(k_tree_fill, dim3((unsigned)std::min<int64_t>(cdiv64(nw, 256), 65536)), dim3(256), 0, s,
                       (int32_t*)o, nw, 0);
    hipLaunchKernelGGL(k_rfgap_tree_tri, dim3((unsigned)cdiv64(np, 256)), dim3(256), 0, s, ctx->tr_nin.p,
                       ctx->tr_nodextr.p, N, np, o);
    if (int rc = check_launch(ctx, "k_rfgap_tree_tri")) return rc;
    if (!direct) {
        RFXP_HIP(ctx, hipMemcpyAsync(out, o, (size_t)(2 * ne), dev_out ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost,
                                     s));
        if (!dev_out) RFXP_HIP(ctx, hipStreamSynchronize(s));
    }
    return RFXP_OK;
}

// Copies n elements of type Tp to a device buffer unless already on device.
template <class Tp>
static int to_device(rfxp_ctx* ctx, const Tp* src, int64_t n, DevBuf<Tp>& buf, const Tp** dst) {
    if (is_device_pointer(src)) {
        *dst = src;
        return RFXP_OK;
    }
    RFXP_HIP(ctx, buf.ensure((size_t)n));
    RFXP_HIP(ctx, hipMemcpyAsync(buf.p, src, sizeof(Tp) * (size_t)n, hipMemcpyHostToDevice, ctx->stream));
    *dst = buf.p;
    return RFXP_OK;
}

extern "C" int rfxp_finishprox(rfxp_ctx* ctx, int32_t N, const int32_t* nout, const double* prox, double* proxsym) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (N < 0 || (N > 0 && (!nout || !prox || !proxsym)))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_finishprox: bad arguments");
    if (N == 0) return RFXP_OK;
    if ((int64_t)N * N > DENSE_MAX_ENTRIES)
        return set_error(ctx, RFXP_ERR_UNSUPPORTED, "rfxp_finishprox: dense N x N above 2^31 entries (N > 46340)");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    const int64_t nn = (int64_t)N * N;
    const double* pd;
    const int32_t* nd;
    if (int rc = to_device(ctx, prox, nn, ctx->dn_prox, &pd)) return rc;
    if (int rc = to_device(ctx, nout, (int64_t)N, ctx->dn_nout, &nd)) return rc;
    const bool dev_out = is_device_pointer(proxsym);
    double* od = proxsym;
    if (!dev_out) {
        RFXP_HIP(ctx, ctx->dn_out.ensure((size_t)nn));
        od = ctx->dn_out.p;
    }
    hipLaunchKernelGGL(k_finishprox, dim3((unsigned)cdiv64(nn, 256)), dim3(256), 0, ctx->stream, (int64_t)N, nd, pd, od);
    if (int rc = check_launch(ctx, "k_finishprox")) return rc;
    if (!dev_out) {
        RFXP_HIP(ctx, hipMemcpyAsync(proxsym, od, sizeof(double) * (size_t)nn, hipMemcpyDeviceToHost, ctx->stream));
        RFXP_HIP(ctx, hipStreamSynchronize(ctx->stream));
    }
    return RFXP_OK;
}

extern "C" int rfxp_rfgap(rfxp_ctx* ctx, int32_t T, int32_t N, const int32_t* nin_flat, const int32_t* nodextr_flat,
                          double* prox) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (T < 0 || N < 0 || (N > 0 && T > 0 && (!nin_flat || !nodextr_flat)) || (N > 0 && !prox))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_rfgap: bad arguments");
    if (N == 0) return RFXP_OK;
    if ((int64_t)N * N > DENSE_MAX_ENTRIES)
        return set_error(ctx, RFXP_ERR_UNSUPPORTED, "rfxp_rfgap: dense N x N above 2^31 entries (N > 46340)");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    const int64_t nn = (int64_t)N * N, tn = (int64_t)T * N;
    const int32_t *nind = nullptr, *ndxd = nullptr;
    if (T > 0) {
        if (int rc = to_device(ctx, nin_flat, tn, ctx->tr_nin, &nind)) return rc;
        if (int rc = to_device(ctx, nodextr_flat, tn, ctx->tr_nodextr, &ndxd)) return rc;
    }
    RFXP_HIP(ctx, ctx->dn_prox.ensure((size_t)nn));
    double* R = ctx->dn_prox.p;
    const bool dev_out = is_device_pointer(prox);
    double* od = prox;
    if (!dev_out) {
        RFXP_HIP(ctx, ctx->dn_out.ensure((size_t)nn));
        od = ctx->dn_out.p;
    }
    hipLaunchKernelGGL(k_rfgap_rows, dim3((unsigned)N), dim3(256), 0, ctx->stream, T, N, nind, ndxd, R);
    hipLaunchKernelGGL(k_rfgap_sym, dim3((unsigned)cdiv64(nn, 256)), dim3(256), 0, ctx->stream, (int64_t)N, R, od);
    if (int rc = check_launch(ctx, "k_rfgap")) return rc;
    if (!dev_out) {
        RFXP_HIP(ctx, hipMemcpyAsync(prox, od, sizeof(double) * (size_t)nn, hipMemcpyDeviceToHost, ctx->stream));
        RFXP_HIP(ctx, hipStreamSynchronize(ctx->stream));
    }
    return RFXP_OK;
}
