// Test driver for the reference-signature entry points of librfxprox
// (include/rfx_compat.hpp): reads a forest dump written by
// tests/test_gpu_compat.py, calls the rf:: functions the way RFX-Fuse's
// callers do (src/rf_random_forest.cpp:1953-1991 and :2659-2662 per tree and
// once; cuda/rf_growtree.cu:5294 per-tree FP16 triangle), and writes every
// output to a binary file.
//
// Input (little-endian int32 unless noted):
//   N, T, casewise, then per tree: nnode, nodestatus[nnode], nodextr[N], nin[N];
//   then nout[N].
// Output: prox (N*N f64), proxsym (N*N f64), prox via gpu_proximity (N*N
// f64), RF-GAP via cpu_ and gpu_proximity_rfgap (2 x N*N f64), tree 0's
// triangles: fp16 (ne u16), int8 (ne i8), nf4 ((ne+1)/2 u8), unified INT8
// (ne i8), RF-GAP fp16 (ne u16); get_quantized_size for 4 levels x 1000
// (4 x u64); compute_int8_scaling of proxsym's first column (2 f32) and
// compute_int8_scaling_gpu of proxsym (2 f32); proxsym via gpu_finishprox
// (N*N f64); tree 0's terminal CSR: nterm (i32), nodexb[N], ndbegin[nterm+1],
// npcase[N]; launch_proximity_kernel at FP32, FP16, INT8, NF4 for tree 0
// (N*N f64, u16, i8, u8).
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>

#include <vector>

#include "rfx_compat.hpp"

static void rd(FILE* f, void* p, size_t n) {
    if (fread(p, 1, n, f) != n) {
        fprintf(stderr, "short read\n");
        exit(2);
    }
}

int main(int argc, char** argv) {
    if (argc != 3) {
        fprintf(stderr, "usage: compat_driver in.bin out.bin\n");
        return 2;
    }
    FILE* f = fopen(argv[1], "rb");
    if (!f) return 2;
    int32_t hdr[3];
    rd(f, hdr, sizeof(hdr));
    const int32_t N = hdr[0], T = hdr[1], casewise = hdr[2];
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
    rfx_compat_configure(casewise, 0);

    const size_t nn = (size_t)N * N;
    std::vector<double> prox(nn, 0.0), prox2(nn, 0.0), sym(nn, 0.0), rg(nn, 0.0), rg2(nn, 0.0);
    for (int32_t t = 0; t < T; ++t) {
        rf::cpu_proximity(status[t].data(), nodextr[t].data(), nin[t].data(), N, nnode[t], prox.data(), nullptr,
                          nullptr, nullptr, nullptr, nullptr, nullptr);
        rf::gpu_proximity(status[t].data(), nodextr[t].data(), nin[t].data(), N, nnode[t], prox2.data(), nullptr,
                          nullptr, nullptr, nullptr, nullptr, nullptr);
    }
    rf::cpu_finishprox(N, nout.data(), prox.data(), sym.data());
    rf::cpu_proximity_rfgap(T, N, nin, nodextr, rg.data());
    std::vector<int32_t> nin_f((size_t)T * N), ndx_f((size_t)T * N);
    for (int32_t t = 0; t < T; ++t)
        for (int32_t i = 0; i < N; ++i) {
            nin_f[(size_t)t * N + i] = nin[t][i];
            ndx_f[(size_t)t * N + i] = nodextr[t][i];
        }
    rf::gpu_proximity_rfgap(T, N, nin_f.data(), ndx_f.data(), rg2.data());

    const size_t ne = (size_t)N * (N + 1) / 2;
    std::vector<uint16_t> f16(ne), gap16(ne);
    std::vector<int8_t> i8(ne), i8u(ne);
    std::vector<uint8_t> nf4((ne + 1) / 2);
    __half* d16 = nullptr;
    const size_t b16 = (2 * ne + 3) / 4 * 4;
    if (hipMalloc((void**)&d16, b16) != hipSuccess) return 3;
    rf::cuda::gpu_proximity_upper_triangle_fp16(status[0].data(), nodextr[0].data(), nin[0].data(), N, nnode[0], d16,
                                                nullptr, nullptr, nullptr, nullptr, nullptr, nullptr);
    if (hipMemcpy(f16.data(), d16, 2 * ne, hipMemcpyDeviceToHost) != hipSuccess) return 3;
    (void)hipFree(d16);
    rf::cuda::gpu_proximity_upper_triangle_int8(status[0].data(), nodextr[0].data(), nin[0].data(), N, nnode[0],
                                                i8.data(), 1.0f / 60.0f, 0.5f, nullptr, nullptr, nullptr, nullptr,
                                                nullptr, nullptr);
    rf::cuda::gpu_proximity_upper_triangle_nf4(status[0].data(), nodextr[0].data(), nin[0].data(), N, nnode[0],
                                               nf4.data(), nullptr, nullptr, nullptr, nullptr, nullptr, nullptr);
    rf::cuda::gpu_proximity_upper_triangle(status[0].data(), nodextr[0].data(), nin[0].data(), N, nnode[0],
                                           rf::cuda::QuantizationLevel::INT8, i8u.data(), nullptr, nullptr, nullptr,
                                           nullptr, nullptr, nullptr);
    rf::cuda::gpu_proximity_rfgap_upper_triangle_fp16(nin[0].data(), nodextr[0].data(), N, (__half*)gap16.data());

    uint64_t qs[4];
    for (int l = 0; l < 4; ++l)
        qs[l] = rf::cuda::QuantizationDispatcher::get_quantized_size((rf::cuda::QuantizationLevel)l, 1000);
    std::vector<float> col(N);
    for (int32_t i = 0; i < N; ++i) col[i] = (float)sym[i];
    float sc[4] = {0, 0, 0, 0};
    rf::cuda::QuantizationUtils::compute_int8_scaling(col.data(), N, sc[0], sc[1]);
    double* dsym = nullptr;
    float* dsz = nullptr;
    if (hipMalloc((void**)&dsym, sizeof(double) * nn) != hipSuccess || hipMalloc((void**)&dsz, 8) != hipSuccess)
        return 3;
    if (hipMemcpy(dsym, sym.data(), sizeof(double) * nn, hipMemcpyHostToDevice) != hipSuccess) return 3;
    rf::cuda::QuantizationUtils::compute_int8_scaling_gpu(dsym, nn, dsz, dsz + 1);
    if (hipMemcpy(sc + 2, dsz, 8, hipMemcpyDeviceToHost) != hipSuccess) return 3;
    (void)hipFree(dsym);
    (void)hipFree(dsz);

    // rf::gpu_finishprox on the accumulated prox (its only form is the
    // reference's; no caller in the reference, include/rf_finishprox.hpp:12)
    std::vector<double> sym2(nn, 0.0);
    rf::gpu_finishprox(N, nout.data(), prox.data(), sym2.data());

    // QuantizationDispatcher::launch_proximity_kernel for tree 0 at all four
    // levels, the way cuda/rf_proximity.cu:440-485 calls it: terminal CSR of
    // the tree built on the host (src/rf_proximity.cpp:110-171), device
    // inputs, a zeroed get_quantized_size(level, N*N) output, 256-thread
    // blocks over the samples.
    const std::vector<int32_t>& st0 = status[0];
    // ncount is indexed by terminal ordinal, and a tree can hold more
    // terminal nodes than samples, so it is sized by the node count
    std::vector<int32_t> nod(nnode[0] > 0 ? nnode[0] : 1, -1), ncount(nnode[0] > 0 ? nnode[0] : 1, 0), ncn(N, 0),
        nodexb(N, -1);
    int32_t nterm = 0;
    for (int32_t k = 0; k < nnode[0]; ++k)
        if (st0[k] == -1) nod[k] = nterm++;
    for (int32_t n = 0; n < N; ++n) {
        const int32_t nd = nodextr[0][n];
        if (nd >= 0 && nd < nnode[0] && nod[nd] >= 0) {
            const int32_t k = nod[nd];
            ncn[n] = ++ncount[k];
            nodexb[n] = k;
        }
    }
    std::vector<int32_t> ndbegin(nterm + 1, 0), npcase(N, -1);
    for (int32_t k = 1; k <= nterm; ++k) ndbegin[k] = ndbegin[k - 1] + ncount[k - 1];
    for (int32_t n = 0; n < N; ++n)
        if (nodexb[n] >= 0) npcase[ndbegin[nodexb[n]] + ncn[n] - 1] = n;
    int32_t *d_xb = nullptr, *d_nin = nullptr, *d_beg = nullptr, *d_pc = nullptr;
    if (hipMalloc((void**)&d_xb, 4 * (size_t)N) != hipSuccess || hipMalloc((void**)&d_nin, 4 * (size_t)N) != hipSuccess ||
        hipMalloc((void**)&d_beg, 4 * (size_t)(nterm + 1)) != hipSuccess ||
        hipMalloc((void**)&d_pc, 4 * (size_t)N) != hipSuccess)
        return 3;
    if (hipMemcpy(d_xb, nodexb.data(), 4 * (size_t)N, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(d_nin, nin[0].data(), 4 * (size_t)N, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(d_beg, ndbegin.data(), 4 * (size_t)(nterm + 1), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(d_pc, npcase.data(), 4 * (size_t)N, hipMemcpyHostToDevice) != hipSuccess)
        return 3;
    std::vector<std::vector<uint8_t>> lev(4);
    for (int l = 0; l < 4; ++l) {
        const auto q = (rf::cuda::QuantizationLevel)l;
        const size_t nb = rf::cuda::QuantizationDispatcher::get_quantized_size(q, nn);
        void* d = nullptr;
        if (hipMalloc(&d, nb) != hipSuccess || hipMemset(d, 0, nb) != hipSuccess) return 3;
        rf::cuda::QuantizationDispatcher::launch_proximity_kernel(q, d_xb, d_nin, N, d_beg, d_pc, d, (N + 255) / 256,
                                                                  256);
        if (hipDeviceSynchronize() != hipSuccess) return 3;
        lev[l].resize(nb);
        if (hipMemcpy(lev[l].data(), d, nb, hipMemcpyDeviceToHost) != hipSuccess) return 3;
        (void)hipFree(d);
    }
    (void)hipFree(d_xb);
    (void)hipFree(d_nin);
    (void)hipFree(d_beg);
    (void)hipFree(d_pc);

    if (rfx_compat_last_error()[0]) {
        fprintf(stderr, "compat error: %s\n", rfx_compat_last_error());
        return 4;
    }

    FILE* o = fopen(argv[2], "wb");
    if (!o) return 2;
    fwrite(prox.data(), 8, nn, o);
    fwrite(sym.data(), 8, nn, o);
    fwrite(prox2.data(), 8, nn, o);
    fwrite(rg.data(), 8, nn, o);
    fwrite(rg2.data(), 8, nn, o);
    fwrite(f16.data(), 2, ne, o);
    fwrite(i8.data(), 1, ne, o);
    fwrite(nf4.data(), 1, nf4.size(), o);
    fwrite(i8u.data(), 1, ne, o);
    fwrite(gap16.data(), 2, ne, o);
    fwrite(qs, 8, 4, o);
    fwrite(sc, 4, 4, o);
    fwrite(sym2.data(), 8, nn, o);
    fwrite(&nterm, 4, 1, o);
    fwrite(nodexb.data(), 4, N, o);
    fwrite(ndbegin.data(), 4, nterm + 1, o);
    fwrite(npcase.data(), 4, N, o);
    for (int l = 0; l < 4; ++l) fwrite(lev[l].data(), 1, lev[l].size(), o);
    fclose(o);
    printf("compat_driver ok N=%d T=%d\n", N, T);
    return 0;
}
