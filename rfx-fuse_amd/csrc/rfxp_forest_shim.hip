// rfx::ForestProximity (include/rfx_forest.hpp): RandomForest's proximity
// queries over its leaf_assignments_ / oob_trees_ state, on the C ABI.
//
// Device state, built once from the host arrays: the leaf matrix as int32
// (tree-major), the OOB words of every sample, nout = |oob_trees[i]|; the
// reference-set index (rfxp_set_reference) and the forest index
// (rfxp_set_forest) on first use.  Each query is a few kernel launches on
// the object's context; results come back to the host as the methods
// return them.
#include <hip/hip_runtime.h>
#include <stdio.h>

#include <algorithm>
#include <string>
#include <vector>

#include "rfx_forest.hpp"
#include "rfx_prox.h"
#include "rfxp_device.hpp"
#include "rfxp_internal.hpp"

namespace rfxp {

// N x N from the packed F32 triangle: out[i*N + j] = tri[idx(min, max)],
// one 64 x 64 tile per workgroup (rows 64 blockIdx.y, columns 64
// blockIdx.x).  A tile on or above the diagonal reads along the triangle's
// rows; a tile below it (every j < i) reads rows j of the triangle into LDS
// and writes them transposed, so that reads and writes stay coalesced.
constexpr int EX_T = 64;
__global__ __launch_bounds__(256) void k_expand_sym(const float* tri, int64_t N, float* out) {
    __shared__ float tile[EX_T][EX_T + 1];
    const int64_t i0 = (int64_t)blockIdx.y * EX_T, j0 = (int64_t)blockIdx.x * EX_T;
    const int tx = threadIdx.x & (EX_T - 1), ty = threadIdx.x / EX_T;
    if (j0 >= i0) {  // the diagonal tile mixes both sides: per entry
        for (int r = ty; r < EX_T; r += 256 / EX_T) {
            const int64_t i = i0 + r, j = j0 + tx;
            if (i >= N || j >= N) continue;
            const int64_t a = i < j ? i : j, b = i < j ? j : i;
            out[i * N + j] = tri[tri_idx(N, a, b)];
        }
        return;
    }
    for (int r = ty; r < EX_T; r += 256 / EX_T) {
        const int64_t j = j0 + r, i = i0 + tx;
        if (i < N) tile[r][tx] = tri[tri_idx(N, j, i)];  // j < i0 <= N
    }
    __syncthreads();
    for (int r = ty; r < EX_T; r += 256 / EX_T) {
        const int64_t i = i0 + r, j = j0 + tx;
        if (i < N) out[i * N + j] = tile[tx][r];
    }
}

__global__ void k_i16_to_i32(const int16_t* in, int64_t n, int32_t* out) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e < n) out[e] = in[e];
}

}  // namespace rfxp

namespace rfx {

using rfxp::compat_report;
using rfxp::compat_report_msg;

struct ForestProximity::Impl {
    rfxp_ctx* ctx = nullptr;
    int32_t N = 0, T = 0, L = 1;
    bool good = false;
    int32_t* leaf = nullptr;   // device [T][N]
    uint32_t* oob = nullptr;   // device [T][ld]
    int64_t ld = 0;
    int32_t* nout = nullptr;   // device [N]
    std::vector<std::vector<int32_t>> oob_trees;
    bool ref_ready = false, forest_ready = false;

    ~Impl() {
        if (ctx) (void)hipSetDevice(ctx->device);
        for (void* p : {(void*)leaf, (void*)oob, (void*)nout})
            if (p) (void)hipFree(p);
        if (ctx) rfxp_ctx_destroy(ctx);
        (void)hipGetLastError();
    }
    bool check(const char* fn, int rc) const {
        if (rc == RFXP_OK) return true;
        compat_report(fn, ctx, rc);
        return false;
    }
    bool reference(const char* fn) {
        if (ref_ready) return true;
        ref_ready = check(fn, rfxp_set_reference(ctx, leaf, 1, N, N, T, L));
        return ref_ready;
    }
    bool forest(const char* fn) {
        if (forest_ready) return true;
        forest_ready = check(fn, rfxp_set_forest(ctx, leaf, 1, N, oob, ld, N, T, L, nout));
        return forest_ready;
    }
};

// Device scratch freed on scope exit.
template <class T>
struct Scratch {
    T* p = nullptr;
    bool alloc(size_t n) {
        if (hipMalloc((void**)&p, sizeof(T) * std::max<size_t>(n, 1)) != hipSuccess) {
            (void)hipGetLastError();
            p = nullptr;
            return false;
        }
        return true;
    }
    ~Scratch() {
        if (p) (void)hipFree(p);
    }
};

ForestProximity::ForestProximity(const int16_t* leaf_assignments, int32_t nsample, int32_t ntree,
                                 const std::vector<std::vector<int32_t>>& oob_trees, int device)
    : p_(new Impl()) {
    const char* fn = "rfx::ForestProximity";
    Impl& s = *p_;
    if (!leaf_assignments || nsample < 1 || ntree < 1 || (int64_t)oob_trees.size() != nsample) {
        compat_report_msg(fn, "need leaf assignments, nsample >= 1, ntree >= 1 and one OOB tree list per sample");
        return;
    }
    if (!s.check(fn, rfxp_ctx_create(device, &s.ctx))) return;
    s.N = nsample;
    s.T = ntree;
    s.oob_trees = oob_trees;
    const int64_t nt = (int64_t)nsample * ntree;
    int32_t lmax = -1;
    for (int64_t e = 0; e < nt; ++e) lmax = std::max<int32_t>(lmax, leaf_assignments[e]);
    s.L = std::max(1, lmax + 1);
    s.ld = (nsample + 31) / 32;
    std::vector<uint32_t> words((size_t)(ntree * s.ld), 0u);
    std::vector<int32_t> nout(nsample, 0);
    for (int32_t i = 0; i < nsample; ++i)
        for (int32_t t : oob_trees[i])
            if (t >= 0 && t < ntree) {
                uint32_t& w = words[(size_t)t * s.ld + (i >> 5)];
                if (!((w >> (i & 31)) & 1u)) ++nout[i];
                w |= 1u << (i & 31);
            }
    Scratch<int16_t> l16;
    if (hipMalloc((void**)&s.leaf, sizeof(int32_t) * nt) != hipSuccess ||
        hipMalloc((void**)&s.oob, sizeof(uint32_t) * words.size()) != hipSuccess ||
        hipMalloc((void**)&s.nout, sizeof(int32_t) * nsample) != hipSuccess || !l16.alloc((size_t)nt)) {
        (void)hipGetLastError();
        compat_report_msg(fn, "out of device memory");
        return;
    }
    hipStream_t st = (hipStream_t)rfxp_ctx_stream(s.ctx);
    if (hipMemcpyAsync(l16.p, leaf_assignments, sizeof(int16_t) * nt, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipMemcpyAsync(s.oob, words.data(), sizeof(uint32_t) * words.size(), hipMemcpyHostToDevice, st) != hipSuccess ||
        hipMemcpyAsync(s.nout, nout.data(), sizeof(int32_t) * nsample, hipMemcpyHostToDevice, st) != hipSuccess) {
        compat_report_msg(fn, "copy to the device failed");
        return;
    }
    hipLaunchKernelGGL(rfxp::k_i16_to_i32, dim3((unsigned)((nt + 255) / 256)), dim3(256), 0, st, l16.p, nt, s.leaf);
    s.good = hipGetLastError() == hipSuccess && hipStreamSynchronize(st) == hipSuccess;
    if (!s.good) compat_report_msg(fn, "leaf conversion failed");
}

ForestProximity::~ForestProximity() { delete p_; }

bool ForestProximity::ok() const { return p_->good; }

float ForestProximity::compute_proximity_from_leaves(int32_t sample_i, int32_t sample_j) const {
    const char* fn = "rfx::ForestProximity::compute_proximity_from_leaves";
    Impl& s = *p_;
    if (!s.good) return 0.0f;
    Scratch<int64_t> pr;
    Scratch<float> out;
    if (!pr.alloc(2) || !out.alloc(1)) return 0.0f;
    const int64_t h[2] = {sample_i, sample_j};
    hipStream_t st = (hipStream_t)rfxp_ctx_stream(s.ctx);
    if (hipMemcpyAsync(pr.p, h, sizeof(h), hipMemcpyHostToDevice, st) != hipSuccess) return 0.0f;
    if (!s.check(fn, rfxp_pair_proximity(s.ctx, s.leaf, 1, s.N, s.oob, s.ld, s.N, s.T, s.L, pr.p, pr.p + 1, 1, out.p)))
        return 0.0f;
    float v = 0.0f;
    if (hipMemcpyAsync(&v, out.p, sizeof(float), hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return 0.0f;
    return v;
}

std::vector<std::pair<int32_t, float>> ForestProximity::get_top_k_similar(int32_t query_idx, int32_t k,
                                                                          bool exclude_self) const {
    const char* fn = "rfx::ForestProximity::get_top_k_similar";
    Impl& s = *p_;
    std::vector<std::pair<int32_t, float>> res;
    if (!s.good || query_idx < 0 || query_idx >= s.N || s.oob_trees[query_idx].empty() || k < 1) return res;
    if (k > 64) {
        compat_report_msg(fn, "k above 64 is not supported");
        return res;
    }
    if (!s.reference(fn)) return res;
    // the query's OOB trees as one word per tree (bit 0)
    std::vector<uint32_t> qw((size_t)s.T, 0u);
    for (int32_t t : s.oob_trees[query_idx])
        if (t >= 0 && t < s.T) qw[t] = 1u;
    Scratch<uint32_t> dq;
    Scratch<int32_t> idx;
    Scratch<uint16_t> cnt;
    Scratch<float> sc;
    if (!dq.alloc(qw.size()) || !idx.alloc(k) || !cnt.alloc(k) || !sc.alloc(k)) return res;
    hipStream_t st = (hipStream_t)rfxp_ctx_stream(s.ctx);
    if (hipMemcpyAsync(dq.p, qw.data(), sizeof(uint32_t) * qw.size(), hipMemcpyHostToDevice, st) != hipSuccess)
        return res;
    if (!s.check(fn, rfxp_topk(s.ctx, s.leaf + query_idx, 1, s.N, 1, dq.p, 1, exclude_self ? query_idx : -1, k, 1,
                               idx.p, cnt.p)) ||
        !s.check(fn, rfxp_topk_scores(s.ctx, dq.p, 1, 1, s.T, k, idx.p, cnt.p, sc.p)))
        return res;
    std::vector<int32_t> hi(k);
    std::vector<float> hs(k);
    if (hipMemcpyAsync(hi.data(), idx.p, sizeof(int32_t) * k, hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipMemcpyAsync(hs.data(), sc.p, sizeof(float) * k, hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return res;
    for (int32_t c = 0; c < k && hi[c] >= 0; ++c) res.emplace_back(hi[c], hs[c]);
    return res;
}

bool ForestProximity::predict_top_k_similar(const int16_t* new_leaves, int32_t nq, int32_t k, int32_t* idx_out,
                                            float* score_out) const {
    const char* fn = "rfx::ForestProximity::predict_top_k_similar";
    Impl& s = *p_;
    if (!s.good || !new_leaves || nq < 0 || k < 1 || !idx_out || !score_out) return false;
    if (k > 64) {
        compat_report_msg(fn, "k above 64 is not supported");
        return false;
    }
    if (nq == 0) return true;
    if (!s.reference(fn)) return false;
    const int64_t nl = (int64_t)nq * s.T, no = (int64_t)nq * k;
    Scratch<int16_t> q16;
    Scratch<int32_t> q32, idx;
    Scratch<uint16_t> cnt;
    Scratch<float> sc;
    if (!q16.alloc((size_t)nl) || !q32.alloc((size_t)nl) || !idx.alloc((size_t)no) || !cnt.alloc((size_t)no) ||
        !sc.alloc((size_t)no))
        return false;
    hipStream_t st = (hipStream_t)rfxp_ctx_stream(s.ctx);
    if (hipMemcpyAsync(q16.p, new_leaves, sizeof(int16_t) * nl, hipMemcpyHostToDevice, st) != hipSuccess) return false;
    hipLaunchKernelGGL(rfxp::k_i16_to_i32, dim3((unsigned)((nl + 255) / 256)), dim3(256), 0, st, q16.p, nl, q32.p);
    if (!s.check(fn, rfxp_topk(s.ctx, q32.p, s.T, 1, nq, nullptr, 0, -1, k, 0, idx.p, cnt.p)) ||
        !s.check(fn, rfxp_topk_scores(s.ctx, nullptr, 0, nq, s.T, k, idx.p, cnt.p, sc.p)))
        return false;
    return hipMemcpyAsync(idx_out, idx.p, sizeof(int32_t) * no, hipMemcpyDeviceToHost, st) == hipSuccess &&
           hipMemcpyAsync(score_out, sc.p, sizeof(float) * no, hipMemcpyDeviceToHost, st) == hipSuccess &&
           hipStreamSynchronize(st) == hipSuccess;
}

bool ForestProximity::get_proximity_matrix(float* out) const {
    const char* fn = "rfx::ForestProximity::get_proximity_matrix";
    Impl& s = *p_;
    if (!s.good || !out) return false;
    if (!s.forest(fn)) return false;
    const int64_t N = s.N, nn = N * N;
    Scratch<float> tri, full;
    if (!tri.alloc((size_t)(rfxp_upper_nbytes(RFXP_FMT_F32, N, 0, N) / 4)) || !full.alloc((size_t)nn)) {
        compat_report_msg(fn, "out of device memory");
        return false;
    }
    if (!s.check(fn, rfxp_upper(s.ctx, RFXP_FMT_F32, 1.0f, 0.0f, 0, N, tri.p))) return false;
    hipStream_t st = (hipStream_t)rfxp_ctx_stream(s.ctx);
    const unsigned nt = (unsigned)((N + rfxp::EX_T - 1) / rfxp::EX_T);
    hipLaunchKernelGGL(rfxp::k_expand_sym, dim3(nt, nt), dim3(256), 0, st, tri.p, N, full.p);
    return hipGetLastError() == hipSuccess &&
           hipMemcpyAsync(out, full.p, sizeof(float) * nn, hipMemcpyDeviceToHost, st) == hipSuccess &&
           hipStreamSynchronize(st) == hipSuccess;
}

std::vector<float> ForestProximity::compute_outlier_scores(const int32_t* classes) const {
    const char* fn = "rfx::ForestProximity::compute_outlier_scores";
    Impl& s = *p_;
    std::vector<float> scores;
    if (!s.good || !s.reference(fn)) return scores;
    Scratch<float> raw;
    if (!raw.alloc((size_t)s.N)) return scores;
    if (!s.check(fn, rfxp_outlier_raw(s.ctx, s.leaf, 1, s.N, s.N, 0, nullptr, (float)(s.N - 1), (float)s.N * 1e10f,
                                      raw.p)))
        return scores;
    std::vector<float> h((size_t)s.N);
    hipStream_t st = (hipStream_t)rfxp_ctx_stream(s.ctx);
    if (hipMemcpyAsync(h.data(), raw.p, sizeof(float) * s.N, hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return scores;
    scores.resize((size_t)s.N);
    if (rfxp_outlier_normalize(h.data(), s.N, classes, scores.data(), nullptr, nullptr) != RFXP_OK) scores.clear();
    return scores;
}

}  // namespace rfx
