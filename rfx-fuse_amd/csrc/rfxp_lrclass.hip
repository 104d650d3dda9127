// rf::cuda::LowRankProximityMatrix and the rf_lowrank_helpers.hpp functions
// (include/rf_proximity_lowrank.hpp:27-433, include/rf_lowrank_helpers.hpp:13-34)
// over the accumulator / factor calls of the C ABI (rfxp_symacc_*,
// rfxp_factor_*).
//
// What is kept from the reference (cuda/rf_proximity_lowrank.cu):
//   * the call sequence of its users: construct, initialize, add per-tree
//     triangles, finalize_accumulation(n, final_call = true), get_factors /
//     reconstruct / MDS (cuda/rf_growtree.cu:5219-5410,
//     src/rf_random_forest.cpp:2567-2597, 4588);
//   * the rank rule (initial_rank, or estimate_optimal_rank when <= 0,
//     :432-434), factors as device column-major N x rank doubles with B = A
//     (:1720-1747), quantisation of the factors at the object's level on the
//     final finalize call and dequantisation on access (:1250-1267,
//     :1379-1718), with the INT8 scale computed once from A by
//     compute_int8_scaling_gpu and shared by B;
//   * reconstruct_full_matrix's diagonal and RF-GAP conventions (:1274-1376),
//     get_memory_usage's byte counts (:2508-2534, NF4 counting 0 bytes per
//     element as its integer division does), should_use_incremental and
//     estimate_optimal_rank (:2536-2541, :2626-2640);
//   * compute_distances_from_factors writes the reconstruction (:1749-1751).
// What differs: the factor is the positive part of the exact accumulated
// matrix (rfxp_symacc_factor) instead of one power-iteration vector per
// tree, and MDS is classical MDS through the factor (rfxp_factor_mds).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>

#include <algorithm>
#include <vector>

#include "rfx_compat.hpp"
#include "rfx_prox.h"
#include "rfxp_forest.hpp"
#include "rfxp_internal.hpp"

namespace rf {
namespace cuda {

namespace {

int level_fmt(QuantizationLevel q) {
    switch (q) {
        case QuantizationLevel::FP32: return RFXP_FMT_F32;
        case QuantizationLevel::FP16: return RFXP_FMT_F16;
        case QuantizationLevel::INT8: return RFXP_FMT_I8;
        default: return RFXP_FMT_NF4;
    }
}

constexpr uint64_t FACTOR_SEED = 20261201ull;

}  // namespace

struct LowRankProximityMatrix::State {
    rfxp_ctx* ctx = nullptr;
    bool acc_ready = false;  // rfxp_symacc_reset done
    int64_t contributions = 0;
    bool dirty = false;      // contributions since the last factorisation
    int32_t rank = 0;        // columns of the factors (0: none)
    double* A = nullptr;     // device N x rank, column-major
    double* B = nullptr;
    void* qA = nullptr;      // quantised storage
    void* qB = nullptr;
    int qlevel = -1;         // level of qA / qB
    float* sz = nullptr;     // device: A scale, A zero point, B scale, B zero point
    bool sz_set = false;
    std::vector<integer_t> oob_counts;
    int32_t trees_processed = 0;

    ~State() {
        if (ctx) (void)hipSetDevice(ctx->device);
        for (void* p : {(void*)A, (void*)B, qA, qB, (void*)sz})
            if (p) (void)hipFree(p);
        if (ctx) rfxp_ctx_destroy(ctx);
        (void)hipGetLastError();
    }
};

static bool ensure_ctx(LowRankProximityMatrix::State* st, const char* fn) {
    if (st->ctx) return true;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        dev = 0;
    }
    rfxp_ctx* c = nullptr;
    const int rc = rfxp_ctx_create(dev, &c);
    if (rc != RFXP_OK) {
        rfxp::compat_report(fn, nullptr, rc);
        return false;
    }
    // the null stream, as the reference's object uses: its work is ordered
    // with the caller's (e.g. the per-tree triangle it is handed)
    rfxp_ctx_set_stream(c, nullptr);
    st->ctx = c;
    return true;
}

LowRankProximityMatrix::LowRankProximityMatrix(integer_t nsample, integer_t initial_rank, QuantizationLevel quant_level,
                                               integer_t max_rank, integer_t power_iterations)
    : st_(new State()),
      nsample_(nsample),
      rank_(initial_rank),
      max_rank_(max_rank),
      power_iterations_(power_iterations),
      current_quant_level_(quant_level) {
    if (initial_rank <= 0) rank_ = estimate_optimal_rank(nsample, max_rank_);
}

LowRankProximityMatrix::~LowRankProximityMatrix() { delete st_; }

bool LowRankProximityMatrix::initialize() {
    if (nsample_ < 1) {
        rfxp::compat_report_msg("LowRankProximityMatrix::initialize", "nsample must be positive");
        return false;
    }
    return ensure_ctx(st_, "LowRankProximityMatrix::initialize");
}

// The accumulator on first use.
static bool ensure_acc(LowRankProximityMatrix::State* st, integer_t nsample, const char* fn) {
    if (!ensure_ctx(st, fn)) return false;
    if (st->acc_ready) return true;
    const int rc = rfxp_symacc_reset(st->ctx, nsample);
    if (rc != RFXP_OK) {
        rfxp::compat_report(fn, st->ctx, rc);
        return false;
    }
    st->acc_ready = true;
    return true;
}

void LowRankProximityMatrix::add_tree_contribution(const dp_t* tree_proximity, integer_t nsample, bool) {
    add_tree_contribution_incremental(tree_proximity, nsample);
}

void LowRankProximityMatrix::add_tree_contribution_incremental(const dp_t* tree_proximity, integer_t nsample) {
    const char* fn = "LowRankProximityMatrix::add_tree_contribution_incremental";
    if (nsample != nsample_ || !tree_proximity) {
        rfxp::compat_report_msg(fn, "nsample differs from the object's, or the matrix is NULL");
        return;
    }
    if (!ensure_acc(st_, nsample_, fn)) return;
    const int rc = rfxp_symacc_add_dense(st_->ctx, tree_proximity);
    if (rc != RFXP_OK) {
        rfxp::compat_report(fn, st_->ctx, rc);
        return;
    }
    st_->contributions++;
    st_->dirty = true;
}

void LowRankProximityMatrix::add_tree_contribution_incremental_upper_triangle(const void* tree_proximity_upper,
                                                                             integer_t nsample,
                                                                             QuantizationLevel quant_level,
                                                                             float int8_scale, float int8_zero_point) {
    const char* fn = "LowRankProximityMatrix::add_tree_contribution_incremental_upper_triangle";
    if (nsample != nsample_ || !tree_proximity_upper) {
        rfxp::compat_report_msg(fn, "nsample differs from the object's, or the triangle is NULL");
        return;
    }
    if (!ensure_acc(st_, nsample_, fn)) return;
    // FP32 triangles are read as FP16 data (cuda/rf_proximity_lowrank.cu:770-778)
    const int fmt = quant_level == QuantizationLevel::INT8  ? RFXP_FMT_I8
                    : quant_level == QuantizationLevel::NF4 ? RFXP_FMT_NF4
                                                            : RFXP_FMT_F16;
    const int rc = rfxp_symacc_add_upper(st_->ctx, fmt, tree_proximity_upper, int8_scale, int8_zero_point);
    if (rc != RFXP_OK) {
        rfxp::compat_report(fn, st_->ctx, rc);
        return;
    }
    st_->contributions++;
    st_->dirty = true;
}

void LowRankProximityMatrix::add_tree_contribution_incremental_upper_triangle_fp16(
    const __half* tree_proximity_upper_fp16, integer_t nsample) {
    add_tree_contribution_incremental_upper_triangle(tree_proximity_upper_fp16, nsample, QuantizationLevel::FP16);
}

// Factors of the current accumulation (FP64 A and B) when contributions
// arrived since the last factorisation.
static bool refactor(LowRankProximityMatrix::State* st, integer_t N, integer_t rank, integer_t iters, const char* fn) {
    if (!st->dirty) return true;
    if (!ensure_acc(st, N, fn)) return false;
    const int32_t r = std::max(1, std::min<int32_t>(std::min<int32_t>(rank, N), 4096));
    if (st->rank != r || !st->A) {
        if (st->A) (void)hipFree(st->A);
        if (st->B) (void)hipFree(st->B);
        st->A = st->B = nullptr;
        if (hipMalloc((void**)&st->A, sizeof(double) * (size_t)N * r) != hipSuccess ||
            hipMalloc((void**)&st->B, sizeof(double) * (size_t)N * r) != hipSuccess) {
            (void)hipGetLastError();
            if (st->A) (void)hipFree(st->A);
            st->A = nullptr;
            st->rank = 0;
            rfxp::compat_report_msg(fn, "out of device memory for the factors");
            return false;
        }
        st->rank = r;
    }
    int rc = rfxp_symacc_factor(st->ctx, r, std::max(0, (int32_t)iters), FACTOR_SEED, st->A, nullptr);
    if (rc == RFXP_OK) {
        hipStream_t s = (hipStream_t)rfxp_ctx_stream(st->ctx);
        if (hipMemcpyAsync(st->B, st->A, sizeof(double) * (size_t)N * r, hipMemcpyDeviceToDevice, s) != hipSuccess ||
            hipStreamSynchronize(s) != hipSuccess)
            rc = RFXP_ERR_HIP;
    }
    if (rc != RFXP_OK) {
        rfxp::compat_report(fn, st->ctx, rc);
        return false;
    }
    // the quantised copies describe an older factor now
    if (st->qA) (void)hipFree(st->qA);
    if (st->qB) (void)hipFree(st->qB);
    st->qA = st->qB = nullptr;
    st->qlevel = -1;
    st->dirty = false;
    return true;
}

// FP64 factors from the quantised storage when only that is held.
static bool restore_fp64(LowRankProximityMatrix::State* st, integer_t N, const char* fn) {
    if (st->A || !st->qA || st->rank == 0) return true;
    const size_t n = (size_t)N * st->rank;
    if (hipMalloc((void**)&st->A, sizeof(double) * n) != hipSuccess ||
        hipMalloc((void**)&st->B, sizeof(double) * n) != hipSuccess) {
        (void)hipGetLastError();
        if (st->A) (void)hipFree(st->A);
        st->A = nullptr;
        rfxp::compat_report_msg(fn, "out of device memory for the factors");
        return false;
    }
    int rc = rfxp_factor_dequantize(st->ctx, st->qlevel, st->qA, (int64_t)n, st->sz, st->A);
    if (rc == RFXP_OK) rc = rfxp_factor_dequantize(st->ctx, st->qlevel, st->qB, (int64_t)n, st->sz ? st->sz + 2 : nullptr,
                                                   st->B);
    if (rc == RFXP_OK) rc = rfxp_sync(st->ctx);
    if (rc != RFXP_OK) {
        rfxp::compat_report(fn, st->ctx, rc);
        return false;
    }
    return true;
}

// Quantises the FP64 factors at `level` into qA / qB.
static bool store_quantized(LowRankProximityMatrix::State* st, integer_t N, int level, const char* fn) {
    const size_t n = (size_t)N * st->rank;
    if (st->qA) (void)hipFree(st->qA);
    if (st->qB) (void)hipFree(st->qB);
    st->qA = st->qB = nullptr;
    const int64_t nb = rfxp_factor_quantized_bytes(level, (int64_t)n);
    if (hipMalloc(&st->qA, (size_t)std::max<int64_t>(nb, 1)) != hipSuccess ||
        hipMalloc(&st->qB, (size_t)std::max<int64_t>(nb, 1)) != hipSuccess) {
        (void)hipGetLastError();
        rfxp::compat_report_msg(fn, "out of device memory for the quantised factors");
        return false;
    }
    if (level == RFXP_FMT_I8 && !st->sz_set) {
        // the scale of A, computed on the first INT8 quantisation and given
        // to B as well (cuda/rf_proximity_lowrank.cu:1414-1438)
        if (!st->sz && hipMalloc((void**)&st->sz, 4 * sizeof(float)) != hipSuccess) {
            (void)hipGetLastError();
            rfxp::compat_report_msg(fn, "out of device memory");
            return false;
        }
        QuantizationUtils::compute_int8_scaling_gpu(st->A, n, st->sz, st->sz + 1);
        if (hipMemcpy(st->sz + 2, st->sz, 2 * sizeof(float), hipMemcpyDeviceToDevice) != hipSuccess) {
            rfxp::compat_report_msg(fn, "copy of the INT8 scale failed");
            return false;
        }
        st->sz_set = true;
    }
    int rc = rfxp_factor_quantize(st->ctx, level, st->A, (int64_t)n, st->sz, st->qA);
    if (rc == RFXP_OK) rc = rfxp_factor_quantize(st->ctx, level, st->B, (int64_t)n, st->sz ? st->sz + 2 : nullptr, st->qB);
    if (rc == RFXP_OK) rc = rfxp_sync(st->ctx);
    if (rc != RFXP_OK) {
        rfxp::compat_report(fn, st->ctx, rc);
        return false;
    }
    st->qlevel = level;
    return true;
}

void LowRankProximityMatrix::finalize_accumulation(integer_t n_trees_processed, bool final_call) {
    const char* fn = "LowRankProximityMatrix::finalize_accumulation";
    st_->trees_processed = n_trees_processed;
    if (st_->contributions == 0) return;
    if (!refactor(st_, nsample_, rank_, power_iterations_, fn)) return;
    if (final_call && current_quant_level_ != QuantizationLevel::FP32 && st_->A) {
        if (!store_quantized(st_, nsample_, level_fmt(current_quant_level_), fn)) return;
        // the FP64 factors are dropped; get_factors dequantises (:1258-1265)
        (void)hipFree(st_->A);
        (void)hipFree(st_->B);
        st_->A = st_->B = nullptr;
    }
}

void LowRankProximityMatrix::quantize_factors(QuantizationLevel quant_level) {
    const char* fn = "LowRankProximityMatrix::quantize_factors";
    if (quant_level == QuantizationLevel::FP32 || !st_->A) {
        current_quant_level_ = quant_level;
        return;
    }
    if (!store_quantized(st_, nsample_, level_fmt(quant_level), fn)) return;
    current_quant_level_ = quant_level;
}

void LowRankProximityMatrix::dequantize_factors() {
    const char* fn = "LowRankProximityMatrix::dequantize_factors";
    if (st_->dirty && !refactor(st_, nsample_, rank_, power_iterations_, fn)) return;
    restore_fp64(st_, nsample_, fn);
}

void LowRankProximityMatrix::get_factors(dp_t** A_gpu, dp_t** B_gpu, integer_t* rank) {
    dequantize_factors();
    if (st_->A && st_->B && st_->rank > 0) {
        // B = A (:1730-1740)
        hipStream_t s = (hipStream_t)rfxp_ctx_stream(st_->ctx);
        if (hipMemcpyAsync(st_->B, st_->A, sizeof(double) * (size_t)nsample_ * st_->rank, hipMemcpyDeviceToDevice, s) !=
                hipSuccess ||
            hipStreamSynchronize(s) != hipSuccess)
            rfxp::compat_report_msg("LowRankProximityMatrix::get_factors", "copy of A into B failed");
    }
    if (A_gpu) *A_gpu = st_->A;
    if (B_gpu) *B_gpu = st_->B;
    if (rank) *rank = st_->rank > 0 ? st_->rank : rank_;
}

void LowRankProximityMatrix::reconstruct_full_matrix(dp_t* output_prox, integer_t nsample, QuantizationLevel) {
    const char* fn = "LowRankProximityMatrix::reconstruct_full_matrix";
    if (!output_prox || nsample != nsample_) {
        rfxp::compat_report_msg(fn, "output is NULL or nsample differs from the object's");
        return;
    }
    if (!ensure_ctx(st_, fn)) return;
    dequantize_factors();
    const int64_t N = nsample_;
    const size_t bytes = sizeof(double) * (size_t)N * N;
    const bool host_out = !rfxp::is_device_pointer(output_prox);
    double* out = output_prox;
    if (host_out && hipMalloc((void**)&out, bytes) != hipSuccess) {
        (void)hipGetLastError();
        rfxp::compat_report_msg(fn, "out of device memory for the N x N matrix");
        return;
    }
    int rc = RFXP_OK;
    hipStream_t s = (hipStream_t)rfxp_ctx_stream(st_->ctx);
    if (!st_->A || !st_->B || st_->rank == 0) {
        rfxp::fill_u32(st_->ctx, (uint32_t*)out, 2 * N * N, 0u);  // no factors: zeros (:1318-1322)
        rc = rfxp::check_launch(st_->ctx, "fill");
    } else {
        rc = rfxp_factor_reconstruct(st_->ctx, st_->A, st_->B, N, st_->rank,
                                     st_->oob_counts.empty() ? nullptr : st_->oob_counts.data(), out);
    }
    if (rc == RFXP_OK && host_out && hipMemcpyAsync(output_prox, out, bytes, hipMemcpyDeviceToHost, s) != hipSuccess)
        rc = RFXP_ERR_HIP;
    if (rc == RFXP_OK && hipStreamSynchronize(s) != hipSuccess) rc = RFXP_ERR_HIP;
    if (host_out) (void)hipFree(out);
    if (rc != RFXP_OK) rfxp::compat_report(fn, st_->ctx, rc);
}

void LowRankProximityMatrix::get_accumulated_proximity(dp_t* output_prox, integer_t nsample) {
    reconstruct_full_matrix(output_prox, nsample, QuantizationLevel::FP32);
}

void LowRankProximityMatrix::compute_distances_from_factors(dp_t* output_distances, integer_t nsample) {
    reconstruct_full_matrix(output_distances, nsample);
}

void LowRankProximityMatrix::set_oob_counts_for_rfgap(const integer_t* oob_counts) {
    if (!oob_counts) return;
    st_->oob_counts.assign(oob_counts, oob_counts + nsample_);
}

std::vector<double> LowRankProximityMatrix::compute_mds_from_factors(integer_t k) {
    const char* fn = "LowRankProximityMatrix::compute_mds_from_factors";
    if (k < 1 || k > nsample_ || nsample_ < 2) return std::vector<double>();
    if (!ensure_ctx(st_, fn)) return std::vector<double>();
    dequantize_factors();
    if (!st_->A || st_->rank == 0) return std::vector<double>();
    std::vector<double> coords((size_t)nsample_ * k);
    const int rc = rfxp_factor_mds(st_->ctx, st_->A, nsample_, st_->rank, k,
                                   st_->oob_counts.empty() ? nullptr : st_->oob_counts.data(), 100, coords.data(),
                                   nullptr);
    if (rc != RFXP_OK) {
        rfxp::compat_report(fn, st_->ctx, rc);
        return std::vector<double>();
    }
    return coords;
}

integer_t LowRankProximityMatrix::auto_adjust_rank(double) { return rank_; }

size_t LowRankProximityMatrix::get_memory_usage() const { return get_memory_usage(current_quant_level_); }

size_t LowRankProximityMatrix::get_memory_usage(QuantizationLevel quant_level) const {
    const size_t n = (size_t)nsample_ * (size_t)(st_->rank > 0 ? st_->rank : rank_);
    size_t bpe = 0;
    switch (quant_level) {
        case QuantizationLevel::FP32:
        case QuantizationLevel::FP16: bpe = 2; break;
        case QuantizationLevel::INT8: bpe = 1; break;
        case QuantizationLevel::NF4: bpe = 1 / 2; break;  // 0, as the reference's sizeof(uint8_t) / 2
    }
    return 2 * n * bpe;
}

bool LowRankProximityMatrix::should_use_incremental(integer_t nsample, size_t available_memory) {
    const size_t full = (size_t)nsample * (size_t)nsample * sizeof(dp_t);
    return available_memory == 0 || (double)full > (double)available_memory * 0.5;
}

integer_t estimate_optimal_rank(integer_t nsample, integer_t max_rank) {
    if (max_rank <= 0) max_rank = 100;
    if (nsample <= 0) return max_rank;
    integer_t rank = (integer_t)sqrt((double)nsample);
    rank = std::min(rank, max_rank);
    return std::max(1, rank);
}

bool get_lowrank_factors_host(void* lowrank_proximity_ptr, dp_t** A_host, dp_t** B_host, integer_t* rank,
                              integer_t nsamples) {
    if (!lowrank_proximity_ptr || !A_host || !B_host || !rank) return false;
    auto* lr = static_cast<LowRankProximityMatrix*>(lowrank_proximity_ptr);
    dp_t *A = nullptr, *B = nullptr;
    integer_t r = 0;
    lr->get_factors(&A, &B, &r);
    if (!A || !B || r == 0) return false;
    const size_t n = (size_t)nsamples * r;
    *rank = r;
    *A_host = new dp_t[n];
    *B_host = new dp_t[n];
    if (hipMemcpy(*A_host, A, sizeof(dp_t) * n, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(*B_host, B, sizeof(dp_t) * n, hipMemcpyDeviceToHost) != hipSuccess) {
        (void)hipGetLastError();
        delete[] * A_host;
        delete[] * B_host;
        *A_host = *B_host = nullptr;
        rfxp::compat_report_msg("get_lowrank_factors_host", "copy of the factors failed");
        return false;
    }
    return true;
}

std::vector<double> compute_mds_from_factors_host(void* lowrank_proximity_ptr, integer_t k) {
    if (!lowrank_proximity_ptr) return std::vector<double>();
    return static_cast<LowRankProximityMatrix*>(lowrank_proximity_ptr)->compute_mds_from_factors(k);
}

bool reconstruct_proximity_matrix_host(void* lowrank_proximity_ptr, dp_t** output_prox, integer_t nsamples) {
    if (!lowrank_proximity_ptr || !output_prox || nsamples < 1) return false;
    if (nsamples > 50000) {  // rf_lowrank_helpers.cu:87-92
        rfxp::compat_report_msg("reconstruct_proximity_matrix_host", "more than 50000 samples: refused");
        return false;
    }
    const size_t nn = (size_t)nsamples * nsamples;
    double* dev = nullptr;
    if (hipMalloc((void**)&dev, sizeof(double) * nn) != hipSuccess) {
        (void)hipGetLastError();
        rfxp::compat_report_msg("reconstruct_proximity_matrix_host", "out of device memory");
        return false;
    }
    auto* lr = static_cast<LowRankProximityMatrix*>(lowrank_proximity_ptr);
    lr->reconstruct_full_matrix(dev, nsamples, QuantizationLevel::FP32);
    *output_prox = new dp_t[nn];
    const bool ok = hipMemcpy(*output_prox, dev, sizeof(double) * nn, hipMemcpyDeviceToHost) == hipSuccess;
    (void)hipFree(dev);
    if (!ok) {
        (void)hipGetLastError();
        delete[] * output_prox;
        *output_prox = nullptr;
        return false;
    }
    return true;
}

}  // namespace cuda
}  // namespace rf
