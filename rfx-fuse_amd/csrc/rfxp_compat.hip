// The reference's C++ entry points (include/rfx_compat.hpp) over the C ABI.
//
// Each thread that calls them gets its own rfxp context on device 0 with
// the null stream (the reference's device-0 / stream-0 state,
// cuda/rf_growtree.cu:5209).  Per-tree calls stage the tree on the device
// (rfxp_tree.hip); the dense N x N matrices stay the caller's host arrays.
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <string>
#include <vector>

#include "rfx_compat.hpp"
#include "rfx_prox.h"
#include "rfxp_device.hpp"
#include "rfxp_internal.hpp"

namespace {

struct CompatConfig {
    int use_casewise = 0;
    int32_t n_real = 0;
};
CompatConfig g_compat;
thread_local std::string t_last_error;

struct CompatCtx {
    rfxp_ctx* ctx = nullptr;
    ~CompatCtx() {
        if (ctx) rfxp_ctx_destroy(ctx);
    }
};
thread_local CompatCtx t_ctx;

void report(const char* fn, rfxp_ctx* ctx, int rc) {
    char buf[512] = {0};
    rfxp_last_error(ctx, buf, sizeof(buf));
    t_last_error = std::string(fn) + ": " + (buf[0] ? buf : "error " + std::to_string(rc));
    fprintf(stderr, "[rfxprox] %s\n", t_last_error.c_str());
}

// The thread's context (device 0, null stream), or nullptr after reporting.
rfxp_ctx* compat_ctx(const char* fn) {
    if (!t_ctx.ctx) {
        rfxp_ctx* c = nullptr;
        const int rc = rfxp_ctx_create(0, &c);
        if (rc != RFXP_OK) {
            report(fn, nullptr, rc);
            return nullptr;
        }
        rfxp_ctx_set_stream(c, nullptr);
        t_ctx.ctx = c;
    }
    return t_ctx.ctx;
}

bool ok(const char* fn, rfxp_ctx* ctx, int rc) {
    if (rc == RFXP_OK) return true;
    report(fn, ctx, rc);
    return false;
}

}  // namespace

namespace rfxp {
// Failure reporting of the reference-signature layer, for the other
// translation units that implement part of it (rfxp_lrclass.hip).
void compat_report(const char* fn, rfxp_ctx* ctx, int rc) { report(fn, ctx, rc); }
void compat_report_msg(const char* fn, const char* msg) {
    t_last_error = std::string(fn) + ": " + msg;
    fprintf(stderr, "[rfxprox] %s\n", t_last_error.c_str());
}
}  // namespace rfxp

extern "C" void rfx_compat_configure(int use_casewise, int32_t n_real_samples) {
    g_compat.use_casewise = use_casewise ? 1 : 0;
    g_compat.n_real = n_real_samples > 0 ? n_real_samples : 0;
}

extern "C" const char* rfx_compat_last_error(void) { return t_last_error.c_str(); }

namespace rf {

static void tree_accumulate(const char* fn, const integer_t* nodestatus, const integer_t* nodextr,
                            const integer_t* nin, integer_t nsample, integer_t nnode, dp_t* prox) {
    rfxp_ctx* ctx = compat_ctx(fn);
    if (!ctx) return;
    ok(fn, ctx, rfxp_tree_accumulate(ctx, nodestatus, nodextr, nin, nsample, nnode, g_compat.use_casewise, prox));
}

void cpu_proximity(const integer_t* nodestatus, const integer_t* nodextr, const integer_t* nin, integer_t nsample,
                   integer_t nnode, dp_t* prox, integer_t*, integer_t*, integer_t*, integer_t*, integer_t*,
                   integer_t*) {
    tree_accumulate("rf::cpu_proximity", nodestatus, nodextr, nin, nsample, nnode, prox);
}

void gpu_proximity(const integer_t* nodestatus, const integer_t* nodextr, const integer_t* nin, integer_t nsample,
                   integer_t nnode, dp_t* prox, integer_t*, integer_t*, integer_t*, integer_t*, integer_t*,
                   integer_t*) {
    tree_accumulate("rf::gpu_proximity", nodestatus, nodextr, nin, nsample, nnode, prox);
}

void cpu_finishprox(integer_t nsample, const integer_t* nout, dp_t* prox, dp_t* proxsym) {
    rfxp_ctx* ctx = compat_ctx("rf::cpu_finishprox");
    if (!ctx) return;
    ok("rf::cpu_finishprox", ctx, rfxp_finishprox(ctx, nsample, nout, prox, proxsym));
}

void gpu_finishprox(integer_t nsample, const integer_t* nout, dp_t* prox, dp_t* proxsym) {
    rfxp_ctx* ctx = compat_ctx("rf::gpu_finishprox");
    if (!ctx) return;
    ok("rf::gpu_finishprox", ctx, rfxp_finishprox(ctx, nsample, nout, prox, proxsym));
}

void cpu_proximity_rfgap(integer_t ntree, integer_t nsample, const std::vector<std::vector<integer_t>>& tree_nin,
                         const std::vector<std::vector<integer_t>>& tree_nodextr, dp_t* prox) {
    const char* fn = "rf::cpu_proximity_rfgap";
    if (ntree < 0 || nsample < 0) {
        t_last_error = std::string(fn) + ": negative ntree or nsample";
        fprintf(stderr, "[rfxprox] %s\n", t_last_error.c_str());
        return;
    }
    if ((integer_t)tree_nin.size() < ntree || (integer_t)tree_nodextr.size() < ntree) {
        t_last_error = std::string(fn) + ": fewer tree arrays than ntree";
        fprintf(stderr, "[rfxprox] %s\n", t_last_error.c_str());
        return;
    }
    std::vector<integer_t> nin_f((size_t)ntree * nsample), ndx_f((size_t)ntree * nsample);
    for (integer_t t = 0; t < ntree; ++t) {
        if ((integer_t)tree_nin[t].size() < nsample || (integer_t)tree_nodextr[t].size() < nsample) {
            t_last_error = std::string(fn) + ": a tree array is shorter than nsample";
            fprintf(stderr, "[rfxprox] %s\n", t_last_error.c_str());
            return;
        }
        std::copy(tree_nin[t].begin(), tree_nin[t].begin() + nsample, nin_f.begin() + (size_t)t * nsample);
        std::copy(tree_nodextr[t].begin(), tree_nodextr[t].begin() + nsample, ndx_f.begin() + (size_t)t * nsample);
    }
    rfxp_ctx* ctx = compat_ctx(fn);
    if (!ctx) return;
    ok(fn, ctx, rfxp_rfgap(ctx, ntree, nsample, nin_f.data(), ndx_f.data(), prox));
}

void gpu_proximity_rfgap(integer_t ntree, integer_t nsample, const integer_t* tree_nin_flat,
                         const integer_t* tree_nodextr_flat, dp_t* prox) {
    rfxp_ctx* ctx = compat_ctx("rf::gpu_proximity_rfgap");
    if (!ctx) return;
    ok("rf::gpu_proximity_rfgap", ctx, rfxp_rfgap(ctx, ntree, nsample, tree_nin_flat, tree_nodextr_flat, prox));
}

namespace cuda {

static void tree_upper(const char* fn, int fmt, const integer_t* nodestatus, const integer_t* nodextr,
                       const integer_t* nin, integer_t nsample, integer_t nnode, float scale, float zp, void* out) {
    rfxp_ctx* ctx = compat_ctx(fn);
    if (!ctx) return;
    // complete on return, as the reference's device synchronisation makes
    // it (cuda/rf_proximity_upper_triangle.cu uses cudaDeviceSynchronize)
    if (ok(fn, ctx, rfxp_tree_upper(ctx, fmt, nodestatus, nodextr, nin, nsample, nnode, g_compat.use_casewise,
                                    g_compat.n_real, scale, zp, out)))
        ok(fn, ctx, rfxp_sync(ctx));
}

void gpu_proximity_upper_triangle_fp16(const integer_t* nodestatus, const integer_t* nodextr, const integer_t* nin,
                                       integer_t nsample, integer_t nnode, __half* prox_upper_fp16, integer_t*,
                                       integer_t*, integer_t*, integer_t*, integer_t*, integer_t*) {
    const char* fn = "rf::cuda::gpu_proximity_upper_triangle_fp16";
    if (!rfxp::is_device_pointer(prox_upper_fp16)) {  // as cuda/rf_proximity_upper_triangle.cu:853-858
        t_last_error = std::string(fn) + ": output must be device memory";
        fprintf(stderr, "[rfxprox] %s\n", t_last_error.c_str());
        return;
    }
    tree_upper(fn, RFXP_FMT_F16, nodestatus, nodextr, nin, nsample, nnode, 1.f, 0.f, prox_upper_fp16);
}

void gpu_proximity_upper_triangle_int8(const integer_t* nodestatus, const integer_t* nodextr, const integer_t* nin,
                                       integer_t nsample, integer_t nnode, int8_t* prox_upper_int8, float scale,
                                       float zero_point, integer_t*, integer_t*, integer_t*, integer_t*, integer_t*,
                                       integer_t*) {
    tree_upper("rf::cuda::gpu_proximity_upper_triangle_int8", RFXP_FMT_I8, nodestatus, nodextr, nin, nsample, nnode,
               scale, zero_point, prox_upper_int8);
}

void gpu_proximity_upper_triangle_nf4(const integer_t* nodestatus, const integer_t* nodextr, const integer_t* nin,
                                      integer_t nsample, integer_t nnode, uint8_t* prox_upper_nf4, integer_t*,
                                      integer_t*, integer_t*, integer_t*, integer_t*, integer_t*) {
    tree_upper("rf::cuda::gpu_proximity_upper_triangle_nf4", RFXP_FMT_NF4, nodestatus, nodextr, nin, nsample, nnode,
               1.f, 0.f, prox_upper_nf4);
}

// cuda/rf_proximity_upper_triangle.cu:1559-1611: FP32 and FP16 go to the
// FP16 triangle, INT8 uses scale 1/127 and zero point 0.
void gpu_proximity_upper_triangle(const integer_t* nodestatus, const integer_t* nodextr, const integer_t* nin,
                                  integer_t nsample, integer_t nnode, QuantizationLevel quant_level,
                                  void* prox_upper_output, integer_t* nod, integer_t* ncount, integer_t* ncn,
                                  integer_t* nodexb, integer_t* ndbegin, integer_t* npcase) {
    switch (quant_level) {
        case QuantizationLevel::FP32:
        case QuantizationLevel::FP16:
            gpu_proximity_upper_triangle_fp16(nodestatus, nodextr, nin, nsample, nnode, (__half*)prox_upper_output,
                                              nod, ncount, ncn, nodexb, ndbegin, npcase);
            break;
        case QuantizationLevel::INT8:
            gpu_proximity_upper_triangle_int8(nodestatus, nodextr, nin, nsample, nnode, (int8_t*)prox_upper_output,
                                              1.0f / 127.0f, 0.0f, nod, ncount, ncn, nodexb, ndbegin, npcase);
            break;
        case QuantizationLevel::NF4:
            gpu_proximity_upper_triangle_nf4(nodestatus, nodextr, nin, nsample, nnode, (uint8_t*)prox_upper_output,
                                             nod, ncount, ncn, nodexb, ndbegin, npcase);
            break;
    }
}

void gpu_proximity_rfgap_upper_triangle_fp16(const integer_t* nin_tree, const integer_t* nodextr_tree,
                                             integer_t nsample, __half* prox_upper_fp16) {
    const char* fn = "rf::cuda::gpu_proximity_rfgap_upper_triangle_fp16";
    rfxp_ctx* ctx = compat_ctx(fn);
    if (!ctx) return;
    if (ok(fn, ctx, rfxp_rfgap_tree_upper(ctx, nin_tree, nodextr_tree, nsample, g_compat.n_real,
                                          (uint16_t*)prox_upper_fp16)))
        ok(fn, ctx, rfxp_sync(ctx));
}

// ---- quantization utilities (cuda/rf_quantization_kernels.cu:24-406) ------

void QuantizationUtils::compute_int8_scaling(const float* data, size_t count, float& scale, float& zero_point) {
    // host data, as cuda/rf_quantization_kernels.cu:107-119, which reads
    // data[0] unconditionally: an empty input is reported instead
    if (count == 0 || !data) {
        t_last_error = "rf::cuda::QuantizationUtils::compute_int8_scaling: no data";
        fprintf(stderr, "[rfxprox] %s\n", t_last_error.c_str());
        return;
    }
    float mn = data[0], mx = data[0];
    for (size_t i = 1; i < count; ++i) {
        mn = std::min(mn, data[i]);
        mx = std::max(mx, data[i]);
    }
    scale = (mx - mn) / 255.0f;
    zero_point = -mn / scale;
}

// Block min / max of (float)data, one pair per block; then one block folds
// all block results (every block, in index order).  Internal linkage: these
// helpers are not part of the exported rf::cuda interface.
namespace {
__global__ __launch_bounds__(256) void k_q_minmax(const dp_t* data, size_t count, float* mins, float* maxs) {
    __shared__ float smn[256], smx[256];
    float mn = 1e30f, mx = -1e30f;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (size_t)gridDim.x * 256) {
        const float v = (float)data[i];
        mn = fminf(mn, v);
        mx = fmaxf(mx, v);
    }
    smn[threadIdx.x] = mn;
    smx[threadIdx.x] = mx;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (threadIdx.x < (unsigned)s) {
            smn[threadIdx.x] = fminf(smn[threadIdx.x], smn[threadIdx.x + s]);
            smx[threadIdx.x] = fmaxf(smx[threadIdx.x], smx[threadIdx.x + s]);
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        mins[blockIdx.x] = smn[0];
        maxs[blockIdx.x] = smx[0];
    }
}

__global__ void k_q_scale(const float* mins, const float* maxs, int nblk, size_t count, float* d_scale,
                          float* d_zp) {
    if (threadIdx.x != 0) return;
    if (count == 0) {
        *d_scale = 1.0f / 127.0f;
        *d_zp = 127.0f;
        return;
    }
    float mn = mins[0], mx = maxs[0];
    for (int b = 1; b < nblk; ++b) {
        mn = fminf(mn, mins[b]);
        mx = fmaxf(mx, maxs[b]);
    }
    float scale = (mx - mn) / 255.0f;
    if (scale < 1e-10f) scale = 1.0f / 127.0f;
    *d_scale = scale;
    *d_zp = -mn / scale;
}
}  // namespace

void QuantizationUtils::compute_int8_scaling_gpu(const dp_t* data_gpu, size_t count, float* d_scale,
                                                 float* d_zero_point) {
    const char* fn = "rf::cuda::QuantizationUtils::compute_int8_scaling_gpu";
    rfxp_ctx* ctx = compat_ctx(fn);
    if (!ctx) return;
    const int nblk = (int)std::max<size_t>(1, std::min<size_t>(1024, (count + 255) / 256));
    float* tmp = nullptr;
    if (hipMalloc((void**)&tmp, sizeof(float) * 2 * nblk) != hipSuccess) {
        (void)hipGetLastError();
        t_last_error = std::string(fn) + ": device allocation failed";
        fprintf(stderr, "[rfxprox] %s\n", t_last_error.c_str());
        return;
    }
    if (count > 0) hipLaunchKernelGGL(k_q_minmax, dim3(nblk), dim3(256), 0, 0, data_gpu, count, tmp, tmp + nblk);
    hipLaunchKernelGGL(k_q_scale, dim3(1), dim3(64), 0, 0, tmp, tmp + nblk, nblk, count, d_scale, d_zero_point);
    (void)hipStreamSynchronize(0);
    (void)hipFree(tmp);
}

// Per-tree dense kernels (cuda/rf_quantization_kernels.cu:195-355): for
// every sample n with terminal ordinal k = nodexb[n] and every in-bag kk of
// node k with n <= kk, entry n + kk*nsample accumulates the weight
// nin[kk]/nodesize (nodesize = sum of nin over the node's in-bag members,
// > 0).  The accumulations are typed atomics of the entry's own width.
static __device__ __forceinline__ int32_t node_size(const integer_t* nin, const integer_t* ndbegin,
                                                    const integer_t* npcase, int32_t k) {
    int32_t s = 0;
    for (int32_t j = ndbegin[k]; j < ndbegin[k + 1]; ++j)
        if (nin[npcase[j]] > 0) s += nin[npcase[j]];
    return s;
}

static __device__ __forceinline__ void add_byte(uint8_t* p, uint32_t v) {
    uint32_t* word = (uint32_t*)((uintptr_t)p & ~(uintptr_t)3);
    const uint32_t sh = (uint32_t)((uintptr_t)p & 3) * 8u;
    uint32_t old = *word, assumed;
    do {
        assumed = old;
        const uint32_t b = ((assumed >> sh) + v) & 0xffu;
        old = atomicCAS(word, assumed, (assumed & ~(0xffu << sh)) | (b << sh));
    } while (old != assumed);
}

static __device__ __forceinline__ void add_half(__half* p, float v) {
    uint32_t* word = (uint32_t*)((uintptr_t)p & ~(uintptr_t)3);
    const uint32_t sh = (uint32_t)((uintptr_t)p & 2) * 8u;
    uint32_t old = *word, assumed;
    do {
        assumed = old;
        const uint16_t cur = (uint16_t)(assumed >> sh);
        const float nv = __half2float(__ushort_as_half(cur)) + v;
        const uint32_t h = (uint32_t)__half_as_ushort(__float2half(nv));
        old = atomicCAS(word, assumed, (assumed & ~(0xffffu << sh)) | (h << sh));
    } while (old != assumed);
}

// The 32-bit word CAS of add_byte / add_half reads and writes back the whole
// word that holds an entry.  When the N*N entries do not fill a whole number
// of words, the last word runs past the buffer's end; the entries in it (at
// most 3, all in column N-1) are left out of the CAS path and updated by the
// thread of sample N-1 alone, with loads and stores of the entry's own width,
// so no access leaves the buffer.  partial_word_start gives the first of
// them (N*N when there are none).
static __device__ __forceinline__ int64_t partial_word_start(integer_t nsample, int bytes) {
    const int64_t ne = (int64_t)nsample * nsample, total = ne * bytes;
    return (total & 3) ? (total & ~(int64_t)3) / bytes : ne;
}

// For each entry e >= e0: what the thread of its row r would add, as
// add(e, nin[kk], nodesize), once per listing of kk among node k's members.
template <class Add>
static __device__ void partial_word_entries(const integer_t* nodexb, const integer_t* nin, integer_t nsample,
                                            const integer_t* ndbegin, const integer_t* npcase, int64_t e0, Add add) {
    const int64_t ne = (int64_t)nsample * nsample;
    for (int64_t e = e0; e < ne; ++e) {
        const int32_t r = (int32_t)(e % nsample), kk = (int32_t)(e / nsample);
        const int32_t k = nodexb[r];
        if (r > kk || k < 0 || nin[kk] <= 0) continue;
        const int32_t nsz = node_size(nin, ndbegin, npcase, k);
        if (nsz <= 0) continue;
        for (int32_t j = ndbegin[k]; j < ndbegin[k + 1]; ++j)
            if (npcase[j] == kk) add(e, nin[kk], nsz);
    }
}

__global__ void cuda_proximity_fp16_kernel(const integer_t* nodexb, const integer_t* nin, integer_t nsample,
                                           const integer_t* ndbegin, const integer_t* npcase, __half* prox_fp16) {
    const int64_t e_tail = partial_word_start(nsample, 2);
    for (int32_t n = blockIdx.x * blockDim.x + threadIdx.x; n < nsample; n += blockDim.x * gridDim.x) {
        if (n == nsample - 1)
            partial_word_entries(nodexb, nin, nsample, ndbegin, npcase, e_tail, [&](int64_t e, int32_t w, int32_t nsz) {
                const float v = __half2float(__float2half((float)w / (float)nsz));
                prox_fp16[e] = __float2half(__half2float(prox_fp16[e]) + v);
            });
        const int32_t k = nodexb[n];
        if (k < 0) continue;
        const int32_t nsz = node_size(nin, ndbegin, npcase, k);
        if (nsz <= 0) continue;
        for (int32_t j = ndbegin[k]; j < ndbegin[k + 1]; ++j) {
            const int32_t kk = npcase[j];
            const int64_t e = (int64_t)n + (int64_t)kk * nsample;
            if (nin[kk] > 0 && n <= kk && e < e_tail)
                add_half(&prox_fp16[e], __half2float(__float2half((float)nin[kk] / (float)nsz)));
        }
    }
}

__global__ void cuda_proximity_kernel(const integer_t* nodexb, const integer_t* nin, integer_t nsample,
                                      const integer_t* ndbegin, const integer_t* npcase, dp_t* prox) {
    for (int32_t n = blockIdx.x * blockDim.x + threadIdx.x; n < nsample; n += blockDim.x * gridDim.x) {
        const int32_t k = nodexb[n];
        if (k < 0) continue;
        const int32_t nsz = node_size(nin, ndbegin, npcase, k);
        if (nsz <= 0) continue;
        for (int32_t j = ndbegin[k]; j < ndbegin[k + 1]; ++j) {
            const int32_t kk = npcase[j];
            if (nin[kk] > 0 && n <= kk)
                atomicAdd(&prox[(int64_t)n + (int64_t)kk * nsample], (double)nin[kk] / (double)nsz);
        }
    }
}

__global__ void cuda_proximity_int8_kernel(const integer_t* nodexb, const integer_t* nin, integer_t nsample,
                                           const integer_t* ndbegin, const integer_t* npcase, int8_t* prox_int8,
                                           float scale, float zero_point) {
    const int64_t e_tail = partial_word_start(nsample, 1);
    uint8_t* const p = (uint8_t*)prox_int8;
    for (int32_t n = blockIdx.x * blockDim.x + threadIdx.x; n < nsample; n += blockDim.x * gridDim.x) {
        if (n == nsample - 1)
            partial_word_entries(nodexb, nin, nsample, ndbegin, npcase, e_tail, [&](int64_t e, int32_t w, int32_t nsz) {
                const int8_t q = QuantizationUtils::fp32_to_int8((float)w / (float)nsz, scale, zero_point);
                p[e] = (uint8_t)(p[e] + (uint8_t)q);
            });
        const int32_t k = nodexb[n];
        if (k < 0) continue;
        const int32_t nsz = node_size(nin, ndbegin, npcase, k);
        if (nsz <= 0) continue;
        for (int32_t j = ndbegin[k]; j < ndbegin[k + 1]; ++j) {
            const int32_t kk = npcase[j];
            const int64_t e = (int64_t)n + (int64_t)kk * nsample;
            if (nin[kk] > 0 && n <= kk && e < e_tail) {
                const int8_t q = QuantizationUtils::fp32_to_int8((float)nin[kk] / (float)nsz, scale, zero_point);
                add_byte(&p[e], (uint32_t)(uint8_t)q);
            }
        }
    }
}

__global__ void cuda_proximity_nf4_kernel(const integer_t* nodexb, const integer_t* nin, integer_t nsample,
                                          const integer_t* ndbegin, const integer_t* npcase, uint8_t* prox_nf4) {
    const int64_t e_tail = partial_word_start(nsample, 1);
    for (int32_t n = blockIdx.x * blockDim.x + threadIdx.x; n < nsample; n += blockDim.x * gridDim.x) {
        if (n == nsample - 1)
            partial_word_entries(nodexb, nin, nsample, ndbegin, npcase, e_tail, [&](int64_t e, int32_t w, int32_t nsz) {
                prox_nf4[e] = (uint8_t)(prox_nf4[e] + QuantizationUtils::fp32_to_nf4((float)w / (float)nsz));
            });
        const int32_t k = nodexb[n];
        if (k < 0) continue;
        const int32_t nsz = node_size(nin, ndbegin, npcase, k);
        if (nsz <= 0) continue;
        for (int32_t j = ndbegin[k]; j < ndbegin[k + 1]; ++j) {
            const int32_t kk = npcase[j];
            const int64_t e = (int64_t)n + (int64_t)kk * nsample;
            if (nin[kk] > 0 && n <= kk && e < e_tail)
                add_byte(&prox_nf4[e], QuantizationUtils::fp32_to_nf4((float)nin[kk] / (float)nsz));
        }
    }
}

void QuantizationDispatcher::launch_proximity_kernel(QuantizationLevel level, const integer_t* nodexb,
                                                     const integer_t* nin, integer_t nsample,
                                                     const integer_t* ndbegin, const integer_t* npcase,
                                                     void* prox_data, int blocks, int threads) {
    // the kernels' atomics act on whole aligned words (8 bytes for FP32's
    // doubles, 4 for the narrower levels), so the output starts on one, as
    // a device allocation does
    if ((uintptr_t)prox_data & (level == QuantizationLevel::FP32 ? 7u : 3u)) {
        ::rfxp::compat_report_msg("launch_proximity_kernel", "the output is not aligned to its word size");
        return;
    }
    switch (level) {
        case QuantizationLevel::FP32:
            hipLaunchKernelGGL(cuda_proximity_kernel, dim3(blocks), dim3(threads), 0, 0, nodexb, nin, nsample, ndbegin,
                               npcase, (dp_t*)prox_data);
            break;
        case QuantizationLevel::FP16:
            hipLaunchKernelGGL(cuda_proximity_fp16_kernel, dim3(blocks), dim3(threads), 0, 0, nodexb, nin, nsample,
                               ndbegin, npcase, (__half*)prox_data);
            break;
        case QuantizationLevel::INT8:  // :372-378
            hipLaunchKernelGGL(cuda_proximity_int8_kernel, dim3(blocks), dim3(threads), 0, 0, nodexb, nin, nsample,
                               ndbegin, npcase, (int8_t*)prox_data, 1.0f / 127.0f, 0.0f);
            break;
        case QuantizationLevel::NF4:
            hipLaunchKernelGGL(cuda_proximity_nf4_kernel, dim3(blocks), dim3(threads), 0, 0, nodexb, nin, nsample,
                               ndbegin, npcase, (uint8_t*)prox_data);
            break;
    }
}

// cuda/rf_quantization_kernels.cu:393-406: bytes of base_size entries (NF4
// counted as one byte per entry, FP32 as a double, as the reference does).
size_t QuantizationDispatcher::get_quantized_size(QuantizationLevel level, size_t base_size) {
    switch (level) {
        case QuantizationLevel::FP32: return base_size * sizeof(dp_t);
        case QuantizationLevel::FP16: return base_size * 2;
        case QuantizationLevel::INT8: return base_size;
        case QuantizationLevel::NF4: return base_size;
    }
    return base_size * sizeof(dp_t);
}

}  // namespace cuda
}  // namespace rf
