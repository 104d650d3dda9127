// Test driver of rf::cuda::LowRankProximityMatrix and the rf_lowrank_helpers
// functions of librfxprox (include/rfx_compat.hpp), called the way RFX-Fuse
// calls them:
//   growtree  cuda/rf_growtree.cu:5219-5410 -- new LowRankProximityMatrix(N,
//             0, level, 1000, 30), initialize, per tree
//             gpu_proximity_upper_triangle_fp16 into a device triangle and
//             add_tree_contribution_incremental_upper_triangle_fp16, then
//             finalize_accumulation(T, true); then
//             get_lowrank_factors_host (src/rf_random_forest.cpp:4588),
//             compute_mds_from_factors_host, reconstruct_proximity_matrix_host;
//   rfgap     src/rf_random_forest.cpp:2567-2597 -- the dense RF-GAP matrix
//             (cpu_proximity_rfgap) through add_tree_contribution into
//             new LowRankProximityMatrix(N, 8, level, 16, 30), then
//             set_oob_counts_for_rfgap(nout), no finalize call.
//   measure   the growtree sequence, timed: per tree the wall time of the
//             caller's steps (device synchronised after each), the device
//             memory in use after the add (hipMemGetInfo, the tree's FP16
//             triangle still allocated), then finalize, the factor copy and
//             MDS; no reconstruction (N x N doubles).
// Input: the forest dump of tests/test_gpu_compat.py.  Output (binary):
// int32 rank, is_quantized, level; A, B (N*rank f64 each, column-major);
// int64 n_coords, coords (f64, N x 3 row-major); int32 reconstructed
// (1/0), P (N*N f64 column-major); get_memory_usage at the four levels
// (4 x u64); should_use_incremental(N, 0) and (N, 2^40) (2 x i32);
// estimate_optimal_rank at (N,1000), (N,5), (0,7), (-3,0) (4 x i32);
// get_factors' rank and pointer state before any contribution (2 x i32).
// measure appends: int32 T; per tree f64 triangle_ms, add_ms, step_ms
// (allocation, clearing, triangle, add and free); per tree u64 device
// bytes in use after the add; u64 bytes in use before the object existed;
// f64 finalize_ms, factors_ms, mds_ms.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <chrono>
#include <vector>

#include "rfx_compat.hpp"

using rf::cuda::LowRankProximityMatrix;
using rf::cuda::QuantizationLevel;

static double now_ms() {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

static uint64_t device_used() {
    size_t fr = 0, tot = 0;
    if (hipMemGetInfo(&fr, &tot) != hipSuccess) return 0;
    return (uint64_t)(tot - fr);
}

static void rd(FILE* f, void* p, size_t n) {
    if (fread(p, 1, n, f) != n) {
        fprintf(stderr, "short read\n");
        exit(2);
    }
}

int main(int argc, char** argv) {
    if (argc != 5) {
        fprintf(stderr, "usage: lowrank_driver in.bin out.bin growtree|rfgap|measure level\n");
        return 2;
    }
    const bool rfgap = strcmp(argv[3], "rfgap") == 0;
    const bool measure = strcmp(argv[3], "measure") == 0;
    const int level = atoi(argv[4]);
    FILE* f = fopen(argv[1], "rb");
    if (!f) return 2;
    int32_t hdr[3];
    rd(f, hdr, sizeof(hdr));
    const int32_t N = hdr[0], T = hdr[1];
    std::vector<std::vector<int32_t>> status(T), nodextr(T, std::vector<int32_t>(N)), nin(T, std::vector<int32_t>(N));
    std::vector<int32_t> nnode(T);
    for (int32_t t = 0; t < T; ++t) {
        rd(f, &nnode[t], 4);
        status[t].resize(nnode[t]);
        rd(f, status[t].data(), 4 * (size_t)nnode[t]);
        rd(f, nodextr[t].data(), 4 * (size_t)N);
        rd(f, nin[t].data(), 4 * (size_t)N);
    }
    std::vector<int32_t> nout(N);
    rd(f, nout.data(), 4 * (size_t)N);
    fclose(f);
    rfx_compat_configure(0, 0);

    // an object with no contribution: no factors yet
    int32_t empty_state[2];
    {
        LowRankProximityMatrix e(N, 0, QuantizationLevel::FP16, 1000, 30);
        double *a = nullptr, *b = nullptr;
        rf::integer_t r = -1;
        e.get_factors(&a, &b, &r);
        empty_state[0] = r;
        empty_state[1] = (a == nullptr && b == nullptr) ? 1 : 0;
    }

    LowRankProximityMatrix* lr = nullptr;
    const QuantizationLevel q = (QuantizationLevel)level;
    std::vector<double> tri_ms(T), add_ms(T), step_ms(T);
    std::vector<uint64_t> used(T);
    double fin_ms = 0.0, fac_ms = 0.0, mds_ms = 0.0;
    (void)hipDeviceSynchronize();
    const uint64_t used0 = device_used();
    if (!rfgap) {
        lr = new LowRankProximityMatrix(N, 0, q, 1000, 30);
        if (!lr->initialize()) return 3;
        const size_t ne = (size_t)N * (N + 1) / 2;
        for (int32_t t = 0; t < T; ++t) {
            const double t0 = now_ms();
            __half* d16 = nullptr;
            if (hipMalloc((void**)&d16, ne * sizeof(__half)) != hipSuccess) return 3;
            (void)hipMemset(d16, 0, ne * sizeof(__half));
            if (measure) (void)hipDeviceSynchronize();
            const double t1 = now_ms();
            rf::cuda::gpu_proximity_upper_triangle_fp16(status[t].data(), nodextr[t].data(), nin[t].data(), N,
                                                        nnode[t], d16, nullptr, nullptr, nullptr, nullptr, nullptr,
                                                        nullptr);
            if (measure) (void)hipDeviceSynchronize();
            const double t2 = now_ms();
            lr->add_tree_contribution_incremental_upper_triangle_fp16(d16, N);
            if (measure) {
                (void)hipDeviceSynchronize();
                used[t] = device_used();
            }
            const double t3 = now_ms();
            (void)hipFree(d16);
            if (measure) (void)hipDeviceSynchronize();
            tri_ms[t] = t2 - t1;
            add_ms[t] = t3 - t2;
            step_ms[t] = now_ms() - t0;
        }
        (void)hipDeviceSynchronize();
        const double t0 = now_ms();
        lr->finalize_accumulation(T, /*final_call=*/true);
        (void)hipDeviceSynchronize();
        fin_ms = now_ms() - t0;
    } else {
        std::vector<double> rg((size_t)N * N, 0.0);
        rf::cpu_proximity_rfgap(T, N, nin, nodextr, rg.data());
        lr = new LowRankProximityMatrix(N, 8, q, 16, 30);
        if (!lr->initialize()) return 3;
        lr->add_tree_contribution(rg.data(), N, false);
        lr->set_oob_counts_for_rfgap(nout.data());
    }

    double *A = nullptr, *B = nullptr;
    rf::integer_t r = 0;
    double tm = now_ms();
    if (!rf::cuda::get_lowrank_factors_host(lr, &A, &B, &r, N)) {
        fprintf(stderr, "no factors: %s\n", rfx_compat_last_error());
        return 4;
    }
    fac_ms = now_ms() - tm;
    tm = now_ms();
    std::vector<double> coords = rf::cuda::compute_mds_from_factors_host(lr, 3);
    mds_ms = now_ms() - tm;
    double* P = nullptr;
    const int32_t rec = !measure && rf::cuda::reconstruct_proximity_matrix_host(lr, &P, N) ? 1 : 0;
    uint64_t mem[4];
    for (int l = 0; l < 4; ++l) mem[l] = lr->get_memory_usage((QuantizationLevel)l);
    int32_t inc[2] = {LowRankProximityMatrix::should_use_incremental(N, 0) ? 1 : 0,
                      LowRankProximityMatrix::should_use_incremental(N, (size_t)1 << 40) ? 1 : 0};
    int32_t est[4] = {rf::cuda::estimate_optimal_rank(N, 1000), rf::cuda::estimate_optimal_rank(N, 5),
                      rf::cuda::estimate_optimal_rank(0, 7), rf::cuda::estimate_optimal_rank(-3, 0)};
    int32_t st[3] = {r, lr->is_quantized() ? 1 : 0, (int32_t)lr->get_quantization_level()};
    if (rfx_compat_last_error()[0]) {
        fprintf(stderr, "compat error: %s\n", rfx_compat_last_error());
        return 4;
    }

    FILE* o = fopen(argv[2], "wb");
    if (!o) return 2;
    fwrite(st, 4, 3, o);
    fwrite(A, 8, (size_t)N * r, o);
    fwrite(B, 8, (size_t)N * r, o);
    const int64_t nc = (int64_t)coords.size();
    fwrite(&nc, 8, 1, o);
    fwrite(coords.data(), 8, coords.size(), o);
    fwrite(&rec, 4, 1, o);
    if (rec) fwrite(P, 8, (size_t)N * N, o);
    fwrite(mem, 8, 4, o);
    fwrite(inc, 4, 2, o);
    fwrite(est, 4, 4, o);
    fwrite(empty_state, 4, 2, o);
    if (measure) {
        fwrite(&T, 4, 1, o);
        for (int32_t t = 0; t < T; ++t) {
            const double x[3] = {tri_ms[t], add_ms[t], step_ms[t]};
            fwrite(x, 8, 3, o);
        }
        fwrite(used.data(), 8, (size_t)T, o);
        fwrite(&used0, 8, 1, o);
        const double y[3] = {fin_ms, fac_ms, mds_ms};
        fwrite(y, 8, 3, o);
    }
    fclose(o);
    delete[] A;
    delete[] B;
    delete[] P;
    delete lr;
    printf("lowrank_driver ok N=%d T=%d mode=%s level=%d rank=%d\n", N, T, argv[3], level, r);
    return 0;
}
