// Driver of the CPU emulation build (tests/emu): runs the library's C ABI
// (include/rfx_prox.h) with its kernels executed by the emulator, on inputs
// from a file, and writes the results for tests/test_emu_cpu.py to compare
// with the oracle.
//
// usage: emu_driver in.bin out.bin
// in:  int32 mode (1 rfxp_upper, 2 rfxp_upper_minmax, 3 rfxp_upper_noalloc,
//      4 rfxp_lowrank_oob_pv: fmt is r, and N x r float32 V follows),
//      int64 N, int32 T, int32 nleaf, int32 fmt, float scale, float zp,
//      int64 r0, int64 r1, int32 has_nout, int32 layout (0 tree-major, 1
//      sample-major), then the int32 leaf matrix, the T x ceil(N/32) OOB
//      words and, with has_nout, N int32 nout
// out: int32 status, then for modes 1 and 3: int64 nbytes, the bytes, int32
//      1 when the 64 guard bytes after the output are untouched, int64 the
//      recount counter (mode 1); for mode 2: float min, float max; for mode
//      4: N x r float32 Y
//
// mode 5 (the symmetric accumulator, rfxp_symacc_*) reads instead: int64 N,
//      int32 contributions, int32 b, int32 rank, int32 iters, then per
//      contribution int32 fmt (-1: dense N x N double), int32 on_device (0:
//      passed as host memory), float scale, float zp, int64 nbytes, the
//      bytes; then N x b double X.  It writes int32 status, then per
//      contribution int64 nnz, int64 device bytes and the N x b double
//      Y = M X after that add; then, with rank > 0, the N x rank
//      column-major factor A and rank Ritz values.
//
// mode 6 (a script of C ABI calls, for any function of include/rfx_prox.h)
//      reads instead: int32 buffers, then per buffer int32 host (1: plain
//      host memory, else hipMalloc), int32 want (written back), int64
//      nbytes, int32 has_data, the bytes when has_data (else zero-filled);
//      then int32 calls, per call int32 name length, the name, int32 args,
//      per argument int32 tag (0 integer, 1 real, 2 buffer pointer, 3 NULL,
//      4 the context), int64 value (the integer, the real's bits, or the
//      buffer index), int64 byte offset into the buffer.  It writes int32 0,
//      int32 calls, int64 each call's result (-999999 for an unknown name
//      or a wrong argument count, and the script stops there), then the
//      bytes of every buffer with want set.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include <hip/hip_runtime.h>

#include "rfx_prox.h"

template <class T>
static void rd(FILE* f, T* p, size_t n) {
    if (n && fread(p, sizeof(T), n, f) != n) {
        fprintf(stderr, "short read\n");
        exit(2);
    }
}

extern "C" void emu_track_host_memory(int on);

static int run_symacc(FILE* f, FILE* o) {
    int64_t N;
    int32_t nc, b, rank, iters;
    rd(f, &N, 1);
    rd(f, &nc, 1);
    rd(f, &b, 1);
    rd(f, &rank, 1);
    rd(f, &iters, 1);
    struct Contrib {
        int32_t fmt, on_device;
        float scale, zp;
        std::vector<unsigned char> bytes;
    };
    std::vector<Contrib> cs((size_t)nc);
    for (auto& c : cs) {
        int64_t nb;
        rd(f, &c.fmt, 1);
        rd(f, &c.on_device, 1);
        rd(f, &c.scale, 1);
        rd(f, &c.zp, 1);
        rd(f, &nb, 1);
        c.bytes.resize((size_t)nb);
        rd(f, c.bytes.data(), c.bytes.size());
    }
    std::vector<double> X((size_t)N * b);
    rd(f, X.data(), X.size());
    fclose(f);
    emu_track_host_memory(1);
    rfxp_ctx* ctx = nullptr;
    auto fail = [&](int code) {
        char msg[512] = {0};
        if (ctx) rfxp_last_error(ctx, msg, sizeof msg);
        fprintf(stderr, "status %d: %s\n", code, msg);
        fwrite(&code, 4, 1, o);
        fclose(o);
        return 0;
    };
    int rc = rfxp_ctx_create(0, &ctx);
    if (rc) return fail(rc);
    if ((rc = rfxp_symacc_reset(ctx, N))) return fail(rc);
    double *Xd = nullptr, *Yd = nullptr;
    hipMalloc((void**)&Xd, 8 * X.size());
    hipMalloc((void**)&Yd, 8 * X.size());
    hipMemcpy(Xd, X.data(), 8 * X.size(), hipMemcpyHostToDevice);
    std::vector<unsigned char> out;
    auto put = [&](const void* p, size_t n) {
        out.insert(out.end(), (const unsigned char*)p, (const unsigned char*)p + n);
    };
    std::vector<double> Y(X.size());
    for (auto& c : cs) {
        void* src = c.bytes.data();
        void* dsrc = nullptr;
        if (c.on_device) {
            hipMalloc(&dsrc, c.bytes.size());
            hipMemcpy(dsrc, c.bytes.data(), c.bytes.size(), hipMemcpyHostToDevice);
            src = dsrc;
        }
        rc = c.fmt < 0 ? rfxp_symacc_add_dense(ctx, (const double*)src)
                       : rfxp_symacc_add_upper(ctx, c.fmt, src, c.scale, c.zp);
        if (dsrc) hipFree(dsrc);
        if (rc) return fail(rc);
        const int64_t nnz = rfxp_symacc_nnz(ctx), bytes = rfxp_symacc_device_bytes(ctx);
        if ((rc = rfxp_symacc_apply(ctx, Xd, b, Yd))) return fail(rc);
        hipMemcpy(Y.data(), Yd, 8 * Y.size(), hipMemcpyDeviceToHost);
        put(&nnz, 8);
        put(&bytes, 8);
        put(Y.data(), 8 * Y.size());
    }
    if (rank > 0) {
        double* Ad = nullptr;
        hipMalloc((void**)&Ad, 8 * (size_t)N * rank);
        std::vector<double> A((size_t)N * rank), ev((size_t)rank);
        if ((rc = rfxp_symacc_factor(ctx, rank, iters, 7, Ad, ev.data()))) return fail(rc);
        hipMemcpy(A.data(), Ad, 8 * A.size(), hipMemcpyDeviceToHost);
        hipFree(Ad);
        put(A.data(), 8 * A.size());
        put(ev.data(), 8 * ev.size());
    }
    hipFree(Xd);
    hipFree(Yd);
    fwrite(&rc, 4, 1, o);
    fwrite(out.data(), 1, out.size(), o);
    fclose(o);
    rfxp_ctx_destroy(ctx);
    return 0;
}

struct Arg {
    int64_t i;
    double f;
    void* p;
};
struct CallEntry {
    const char* name;
    int nargs;
    int64_t (*fn)(const Arg*);
};
static const CallEntry CALLS[] = {
#include "emu_calls.inc"
};

static int run_script(FILE* f, FILE* o) {
    int32_t nb;
    rd(f, &nb, 1);
    std::vector<void*> bufs((size_t)nb, nullptr);
    std::vector<int64_t> sizes((size_t)nb);
    std::vector<int32_t> want((size_t)nb), host((size_t)nb);
    emu_track_host_memory(1);
    for (int32_t k = 0; k < nb; ++k) {
        int32_t has;
        rd(f, &host[k], 1);
        rd(f, &want[k], 1);
        rd(f, &sizes[k], 1);
        rd(f, &has, 1);
        const size_t n = (size_t)sizes[k];
        if (host[k]) bufs[k] = malloc(n ? n : 1);
        else hipMalloc(&bufs[k], n);
        if (has) rd(f, (unsigned char*)bufs[k], n);
        else memset(bufs[k], 0, n);
    }
    rfxp_ctx* ctx = nullptr;
    int rc = rfxp_ctx_create(0, &ctx);
    int32_t nc;
    rd(f, &nc, 1);
    std::vector<int64_t> results;
    for (int32_t c = 0; c < nc && rc == 0; ++c) {
        int32_t len, na;
        rd(f, &len, 1);
        std::string name((size_t)len, ' ');
        rd(f, &name[0], (size_t)len);
        rd(f, &na, 1);
        std::vector<Arg> args((size_t)na);
        for (auto& a : args) {
            int32_t tag;
            int64_t v, off;
            rd(f, &tag, 1);
            rd(f, &v, 1);
            rd(f, &off, 1);
            a = Arg{0, 0.0, nullptr};
            if (tag == 0) {
                a.i = v;
                a.f = (double)v;
            } else if (tag == 1) {
                memcpy(&a.f, &v, 8);
                a.i = (int64_t)a.f;
            } else if (tag == 2) {
                a.p = (unsigned char*)bufs.at((size_t)v) + off;
            } else if (tag == 4) {
                a.p = ctx;
            }
        }
        const CallEntry* e = nullptr;
        for (const auto& x : CALLS)
            if (name == x.name) e = &x;
        if (!e || e->nargs != na) {
            fprintf(stderr, "script: unknown call or argument count: %s/%d\n", name.c_str(), na);
            results.push_back(-999999);
            break;
        }
        results.push_back(e->fn(args.data()));
        rfxp_sync(ctx);
    }
    fclose(f);
    if (rc) {
        fwrite(&rc, 4, 1, o);
        fclose(o);
        return 0;
    }
    const int32_t zero = 0, nres = (int32_t)results.size();
    fwrite(&zero, 4, 1, o);
    fwrite(&nres, 4, 1, o);
    fwrite(results.data(), 8, results.size(), o);
    for (int32_t k = 0; k < nb; ++k)
        if (want[k]) fwrite(bufs[k], 1, (size_t)sizes[k], o);
    fclose(o);
    rfxp_ctx_destroy(ctx);
    for (int32_t k = 0; k < nb; ++k) {
        if (host[k]) free(bufs[k]);
        else hipFree(bufs[k]);
    }
    return 0;
}

int main(int argc, char** argv) {
    if (argc != 3) return 2;
    FILE* f = fopen(argv[1], "rb");
    if (!f) return 2;
    int32_t mode, T, nleaf, fmt, has_nout, layout;
    int64_t N, r0, r1;
    float scale, zp;
    rd(f, &mode, 1);
    if (mode == 5 || mode == 6) {
        FILE* o = fopen(argv[2], "wb");
        if (!o) return 2;
        return mode == 5 ? run_symacc(f, o) : run_script(f, o);
    }
    rd(f, &N, 1);
    rd(f, &T, 1);
    rd(f, &nleaf, 1);
    rd(f, &fmt, 1);
    rd(f, &scale, 1);
    rd(f, &zp, 1);
    rd(f, &r0, 1);
    rd(f, &r1, 1);
    rd(f, &has_nout, 1);
    rd(f, &layout, 1);
    const int64_t ld = (N + 31) / 32;
    std::vector<int32_t> leaf((size_t)N * T);
    std::vector<uint32_t> oob((size_t)T * ld);
    std::vector<int32_t> nout(has_nout ? (size_t)N : 0);
    rd(f, leaf.data(), leaf.size());
    rd(f, oob.data(), oob.size());
    rd(f, nout.data(), nout.size());
    std::vector<float> V(mode == 4 ? (size_t)N * fmt : 0);
    rd(f, V.data(), V.size());
    fclose(f);
    const int64_t si = layout ? T : 1, st = layout ? 1 : N;
    FILE* o = fopen(argv[2], "wb");
    rfxp_ctx* ctx = nullptr;
    int rc = rfxp_ctx_create(0, &ctx);
    auto fail = [&](int code) {
        char msg[512] = {0};
        if (ctx) rfxp_last_error(ctx, msg, sizeof msg);
        fprintf(stderr, "status %d: %s\n", code, msg);
        fwrite(&code, 4, 1, o);
        fclose(o);
        return 0;
    };
    if (rc) return fail(rc);
    // the inputs and outputs in device memory, as the C ABI requires of them
    auto to_dev = [](const void* h, size_t n) {
        void* d = nullptr;
        hipMalloc(&d, n ? n : 1);
        if (n) hipMemcpy(d, h, n, hipMemcpyHostToDevice);
        return d;
    };
    const int32_t* leaf_d = (const int32_t*)to_dev(leaf.data(), 4 * leaf.size());
    const uint32_t* oob_d = (const uint32_t*)to_dev(oob.data(), 4 * oob.size());
    const int32_t* np = has_nout ? (const int32_t*)to_dev(nout.data(), 4 * nout.size()) : nullptr;
    if (mode == 1 || mode == 3) {
        const int64_t nb = rfxp_upper_nbytes(fmt, N, r0, r1);
        std::vector<unsigned char> out((size_t)nb + 64, 0xA5);
        unsigned char* out_d = (unsigned char*)to_dev(out.data(), out.size());
        if (mode == 1) {
            if ((rc = rfxp_set_forest(ctx, leaf_d, si, st, oob_d, ld, N, T, nleaf, np))) return fail(rc);
            if ((rc = rfxp_upper(ctx, fmt, scale, zp, r0, r1, out_d))) return fail(rc);
        } else {
            if ((rc = rfxp_upper_noalloc(ctx, leaf_d, si, st, oob_d, ld, N, T, nleaf, np, fmt, scale, zp, r0, r1,
                                         out_d)))
                return fail(rc);
        }
        rfxp_sync(ctx);
        hipMemcpy(out.data(), out_d, out.size(), hipMemcpyDeviceToHost);
        int32_t ok = 1;
        for (int k = 0; k < 64; ++k) ok &= out[(size_t)nb + k] == 0xA5;
        int64_t rec = -1;
        if (mode == 1) rfxp_upper_recounts(ctx, &rec);
        fwrite(&rc, 4, 1, o);
        fwrite(&nb, 8, 1, o);
        fwrite(out.data(), 1, (size_t)nb, o);
        fwrite(&ok, 4, 1, o);
        fwrite(&rec, 8, 1, o);
    } else if (mode == 2) {
        if ((rc = rfxp_set_forest(ctx, leaf_d, si, st, oob_d, ld, N, T, nleaf, np))) return fail(rc);
        float mm[2] = {0, 0};
        if ((rc = rfxp_upper_minmax(ctx, r0, r1, mm))) return fail(rc);
        fwrite(&rc, 4, 1, o);
        fwrite(mm, 4, 2, o);
    } else if (mode == 4) {
        if ((rc = rfxp_set_forest(ctx, leaf_d, si, st, oob_d, ld, N, T, nleaf, np))) return fail(rc);
        std::vector<float> Y(V.size(), -7.0f);
        const float* V_d = (const float*)to_dev(V.data(), 4 * V.size());
        float* Y_d = (float*)to_dev(Y.data(), 4 * Y.size());
        if ((rc = rfxp_lowrank_oob_pv(ctx, V_d, fmt, Y_d))) return fail(rc);
        rfxp_sync(ctx);
        hipMemcpy(Y.data(), Y_d, 4 * Y.size(), hipMemcpyDeviceToHost);
        fwrite(&rc, 4, 1, o);
        fwrite(Y.data(), 4, Y.size(), o);
    } else {
        return fail(-1);
    }
    fclose(o);
    rfxp_ctx_destroy(ctx);
    return 0;
}
