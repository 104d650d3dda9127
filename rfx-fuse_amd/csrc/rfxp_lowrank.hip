// Low-rank form of the all-trees proximity P = A A^T / T, where A is the
// N x (T*L) one-hot leaf matrix (A[i, (t, l)] = [leaf_i(t) == l]), applied
// without forming P:
//     W_t[l] = sum_{j : leaf_j(t) = l} V_j            (A^T V)
//     Y_i    = (1/T) sum_t W_t[leaf_i(t)]             (A W / T)
// This is the SpMM contract of the reference's low-rank path
// (include/rf_proximity_lowrank.hpp:27-433; cuda/rf_proximity_lowrank.cu
// builds it per tree by power iteration on dense triangles instead).  On top
// of it, subspace iteration: Q_0 = orth(V), Q_k = orth(P Q_{k-1}), and the
// Ritz matrix B = Q^T P Q, so that P ~ Q B Q^T.  orth is CholeskyQR2 (Gram
// matrix in double, Cholesky of an r x r matrix on the host, triangular
// solve), which gives the QR factor with a positive diagonal.
//
// The forest index is the reference set of rfxp_set_reference: in tree t,
// the references of leaf l are the contiguous sub-buckets
// [off[t][l*nseg], off[t][(l+1)*nseg]) of mem[t].
//
// Kernels:
//   k_lr_pieces, k_lr_scan, k_lr_pmap  (once per reference set) split every
//                leaf into pieces of at most LR_PIECE members: per-tree
//                piece offsets and a piece -> leaf map;
//   k_lr_w       one wave per piece: sums its members' rows of V; a leaf
//                with one piece stores its W row, a leaf split into several
//                adds with atomics into the zeroed W (the order of those
//                additions is not fixed: results of such leaves can differ
//                in the last bits between runs);
//   k_lr_y       lane = (sample, 8 columns), four trees per step: a label
//                load and a W row slice per tree.
#include <math.h>

#include <algorithm>
#include <vector>

#include "rfxp_device.hpp"
#include "rfxp_forest.hpp"
#include "rfxp_internal.hpp"

namespace rfxp {

constexpr int LR_PIECE = 1024;  // members per k_lr_w wave
constexpr int LR_MAX_R = 64;

struct LrIndex {
    const uint32_t* mem;
    const int32_t* off;
    int32_t nb, nseg, L, T;
    int64_t N;
};

__global__ __launch_bounds__(256) void k_lr_pieces(LrIndex x, int32_t* npieces) {
    const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;  // t * L + l
    if (k >= (int64_t)x.T * x.L) return;
    const int32_t t = (int32_t)(k / x.L), l = (int32_t)(k % x.L);
    const int32_t* ot = x.off + (int64_t)t * (x.nb + 1);
    const int32_t len = ot[(int64_t)(l + 1) * x.nseg] - ot[(int64_t)l * x.nseg];
    npieces[k] = (len + LR_PIECE - 1) / LR_PIECE;
}

// Per tree, in place: exclusive scan of npieces over the L leaves, and the
// tree's total into tot[t].  One 1024-thread workgroup per tree.
__global__ __launch_bounds__(1024) void k_lr_scan(int32_t* npieces, int32_t L, int32_t* tot) {
    __shared__ int32_t part[1024];
    int32_t* p = npieces + (int64_t)blockIdx.x * L;
    const int32_t chunk = (L + 1023) / 1024;
    const int32_t a = threadIdx.x * chunk, b = min(L, a + chunk);
    int32_t s = 0;
    for (int32_t l = a; l < b; ++l) s += p[l];
    part[threadIdx.x] = s;
    __syncthreads();
    for (int d = 1; d < 1024; d <<= 1) {
        const int32_t v = threadIdx.x >= (unsigned)d ? part[threadIdx.x - d] : 0;
        __syncthreads();
        part[threadIdx.x] += v;
        __syncthreads();
    }
    int32_t run = part[threadIdx.x] - s;
    for (int32_t l = a; l < b; ++l) {
        const int32_t c = p[l];
        p[l] = run;
        run += c;
    }
    if (threadIdx.x == 1023) tot[blockIdx.x] = part[1023];
}

// Piece map: pmap[t*maxp + p] = leaf of piece p of tree t (one thread per
// (tree, leaf)).
__global__ __launch_bounds__(256) void k_lr_pmap(LrIndex x, const int32_t* start, int64_t maxp, int32_t* pmap) {
    const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;  // t * L + l
    if (k >= (int64_t)x.T * x.L) return;
    const int32_t t = (int32_t)(k / x.L), l = (int32_t)(k % x.L);
    const int32_t* ot = x.off + (int64_t)t * (x.nb + 1);
    const int32_t len = ot[(int64_t)(l + 1) * x.nseg] - ot[(int64_t)l * x.nseg];
    const int32_t n = (len + LR_PIECE - 1) / LR_PIECE;
    for (int32_t q = 0; q < n; ++q) pmap[t * maxp + start[k] + q] = l;
}

// One wave per piece; grid (ceil(max pieces per tree / 4), T), 4 waves per
// block.  r columns per row, RP = r rounded up to a power of two (8..64),
// 64 / RP rows per step.  Member ids come in 64 at a time (one coalesced
// load) and are broadcast to the row slots, so that RP row loads per lane
// are in flight together.
template <int RP>
__global__ __launch_bounds__(256) void k_lr_w(LrIndex x, const int32_t* start, const int32_t* tot,
                                             const int32_t* pmap, int64_t maxp, const float* V, int32_t r, float* W) {
    constexpr int SLOTS = 64 / RP;
    const int32_t t = blockIdx.y;
    const int32_t pc = (int32_t)__builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    if (pc >= tot[t]) return;
    const int32_t l = pmap[t * maxp + pc];
    const int32_t* ot = x.off + (int64_t)t * (x.nb + 1);
    const int32_t m0 = ot[(int64_t)l * x.nseg], m1 = ot[(int64_t)(l + 1) * x.nseg];
    const int32_t k = pc - start[(int64_t)t * x.L + l];
    const int32_t p0 = m0 + k * LR_PIECE, p1 = min(m1, p0 + LR_PIECE);
    const bool split = (m1 - m0) > LR_PIECE;
    const int32_t lane = threadIdx.x & 63;
    const int32_t slot = lane / RP, col = lane % RP;
    const uint32_t* mt = x.mem + (int64_t)t * x.N;
    float acc = 0.f;
    for (int32_t p = p0; p < p1; p += 64) {
        const uint32_t mid = p + lane < p1 ? (mt[p + lane] & MEM_ID) : 0u;  // j + 1, 0: none
        float v[RP];
#pragma unroll
        for (int q = 0; q < RP; ++q) {
            const uint32_t jj = (uint32_t)__shfl((int)mid, q * SLOTS + slot, 64);
            v[q] = (jj != 0u && col < r) ? V[(int64_t)(jj - 1u) * r + col] : 0.f;
        }
#pragma unroll
        for (int q = 0; q < RP; ++q) acc += v[q];
    }
#pragma unroll
    for (int d = RP; d < 64; d <<= 1) acc += __shfl_xor(acc, d, 64);
    if (slot == 0 && col < r) {
        float* w = W + ((int64_t)t * x.L + l) * r + col;
        if (split) atomicAdd(w, acc);
        else *w = acc;
    }
}

// Y_i = (1/T) sum_t W_t[leaf_i(t)].  Lane = (sample, group of 8 columns):
// RP/8 lanes per sample, 64*8/RP samples per wave; four trees per step.
template <int RP>
__global__ __launch_bounds__(256) void k_lr_y(const int32_t* leaf, int64_t si, int64_t st, int64_t N, int32_t T,
                                             int32_t L, const float* W, int32_t r, float* Y) {
    constexpr int CG = RP / 8;
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t i = g / CG;
    const int32_t c0 = (int32_t)(g % CG) * 8;
    if (i >= N) return;
    float acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = 0.f;
    const bool r8 = (r & 7) == 0;  // uniform
    int32_t t = 0;
    for (; t + 4 <= T; t += 4) {
        int32_t lv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) lv[u] = leaf[i * si + (int64_t)(t + u) * st];
        float w[4][8];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const bool ok = lv[u] >= 0 && lv[u] < L;
            const float* wr = W + ((int64_t)(t + u) * L + (ok ? lv[u] : 0)) * r;
            if (r8) {
                // whole 8-float slices, 16-byte aligned rows: two 16-byte loads
                float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
                if (ok && c0 < r) {
                    a = *(const float4*)(wr + c0);
                    b = *(const float4*)(wr + c0 + 4);
                }
                w[u][0] = a.x; w[u][1] = a.y; w[u][2] = a.z; w[u][3] = a.w;
                w[u][4] = b.x; w[u][5] = b.y; w[u][6] = b.z; w[u][7] = b.w;
            } else {
#pragma unroll
                for (int c = 0; c < 8; ++c) w[u][c] = (ok && c0 + c < r) ? wr[c0 + c] : 0.f;
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[c] += w[u][c];
    }
    for (; t < T; ++t) {
        const int32_t l = leaf[i * si + (int64_t)t * st];
        if (l < 0 || l >= L) continue;
        const float* wr = W + ((int64_t)t * L + l) * r;
#pragma unroll
        for (int c = 0; c < 8; ++c)
            if (c0 + c < r) acc[c] += wr[c0 + c];
    }
    const float inv_t = 1.0f / (float)T;
#pragma unroll
    for (int c = 0; c < 8; ++c)
        if (c0 + c < r) Y[i * r + c0 + c] = acc[c] * inv_t;
}

__global__ void k_lr_fill0(float* p, int64_t n) {
    for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < n; k += (int64_t)gridDim.x * blockDim.x)
        p[k] = 0.f;
}

// Gram partials G_b = X_b^T Y_b over row blocks of 2048 rows, in double:
// thread (a, c) of an r x r grid (r <= 32: 1024 threads) accumulates one
// entry.  Rows are staged in LDS.
constexpr int LR_GRAM_ROWS = 2048;
constexpr int LR_GRAM_STAGE = 64;
__global__ __launch_bounds__(1024) void k_lr_gram(const float* X, const float* Y, int64_t N, int32_t r,
                                                  double* part) {
    __shared__ float xs[LR_GRAM_STAGE][LR_MAX_R];
    __shared__ float ys[LR_GRAM_STAGE][LR_MAX_R];
    const int32_t a = threadIdx.x / 32, c = threadIdx.x % 32;  // r <= 32 on this path
    const int64_t i0 = (int64_t)blockIdx.x * LR_GRAM_ROWS;
    const int64_t i1 = min(N, i0 + LR_GRAM_ROWS);
    double acc = 0.0;
    for (int64_t b = i0; b < i1; b += LR_GRAM_STAGE) {
        const int32_t nrow = (int32_t)min((int64_t)LR_GRAM_STAGE, i1 - b);
        __syncthreads();
        for (int32_t e = threadIdx.x; e < nrow * r; e += 1024) {
            xs[e / r][e % r] = X[(b + e / r) * r + e % r];
            ys[e / r][e % r] = Y[(b + e / r) * r + e % r];
        }
        __syncthreads();
        if (a < r && c < r)
            for (int32_t k = 0; k < nrow; ++k) acc += (double)xs[k][a] * (double)ys[k][c];
    }
    if (a < r && c < r) part[(int64_t)blockIdx.x * r * r + a * r + c] = acc;
}

// Sums the Gram partials of nb blocks (one thread per entry, fixed order).
__global__ void k_lr_gram_sum(const double* part, int64_t nblk, int32_t rr, double* G) {
    const int32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= rr) return;
    double s = 0.0;
    for (int64_t b = 0; b < nblk; ++b) s += part[b * rr + e];
    G[e] = s;
}

// Q = X Rinv (Rinv upper triangular r x r, double), one thread per entry.
__global__ __launch_bounds__(256) void k_lr_trmm(const float* X, const double* Rinv, int64_t N, int32_t r, float* Q) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= N * r) return;
    const int64_t i = e / r;
    const int32_t c = (int32_t)(e % r);
    double s = 0.0;
    for (int32_t a = 0; a <= c; ++a) s += (double)X[i * r + a] * Rinv[a * r + c];
    Q[e] = (float)s;
}

static int64_t cdivl(int64_t a, int64_t b) { return (a + b - 1) / b; }

static int rp_of(int32_t r) {
    int rp = 1;
    while (rp < r) rp <<= 1;
    return rp;
}

}  // namespace rfxp

using namespace rfxp;

// W = A^T V and Y = A W / T on the context stream; V, Y device, N x r
// row-major fp32.
template <int RP>
static void launch_lr(rfxp_ctx* ctx, const LrIndex& x, dim3 gw, int64_t maxp, const float* V, int32_t r, float* Y) {
    hipStream_t s = ctx->stream;
    {
        LaunchTimer tm(ctx, "lr_w");
        hipLaunchKernelGGL(k_lr_w<RP>, gw, dim3(256), 0, s, x, ctx->lr_start.p, ctx->lr_tot.p, ctx->lr_pmap.p, maxp, V,
                           r, ctx->lr_w.p);
    }
    {
        LaunchTimer tm(ctx, "lr_y");
        const int64_t nthreads = x.N * (RP / 8);
        hipLaunchKernelGGL(k_lr_y<RP>, dim3((unsigned)cdivl(nthreads, 256)), dim3(256), 0, s, ctx->ref_leaf,
                           ctx->ref_si, ctx->ref_st, x.N, x.T, x.L, ctx->lr_w.p, r, Y);
    }
}

static int lowrank_apply(rfxp_ctx* ctx, const float* V, int32_t r, float* Y) {
    const int64_t N = ctx->ref_N;
    const int32_t T = ctx->ref_T, L = ctx->ref_L;
    hipStream_t s = ctx->stream;
    LrIndex x{ctx->ref_mem.p, ctx->ref_off.p, ctx->ref_nb, ctx->ref_nseg, L, T, N};
    // pieces per tree <= L + N / LR_PIECE
    const int64_t maxp = L + N / LR_PIECE + 1;
    RFXP_HIP(ctx, ctx->lr_w.ensure((size_t)T * L * r));
    if (!ctx->lr_index_ready) {
        // piece index of the reference set (rebuilt by rfxp_set_reference)
        RFXP_HIP(ctx, ctx->lr_start.ensure((size_t)T * L));
        RFXP_HIP(ctx, ctx->lr_tot.ensure((size_t)T));
        RFXP_HIP(ctx, ctx->lr_pmap.ensure((size_t)T * maxp));
        LaunchTimer tm(ctx, "lr_pieces");
        const unsigned gl = (unsigned)cdivl((int64_t)T * L, 256);
        hipLaunchKernelGGL(k_lr_pieces, dim3(gl), dim3(256), 0, s, x, ctx->lr_start.p);
        hipLaunchKernelGGL(k_lr_scan, dim3((unsigned)T), dim3(1024), 0, s, ctx->lr_start.p, L, ctx->lr_tot.p);
        hipLaunchKernelGGL(k_lr_pmap, dim3(gl), dim3(256), 0, s, x, ctx->lr_start.p, maxp, ctx->lr_pmap.p);
        if (int rc = check_launch(ctx, "k_lr_pieces")) return rc;
        ctx->lr_index_ready = true;
    }
    const int64_t nw = (int64_t)T * L * r;
    hipLaunchKernelGGL(k_lr_fill0, dim3((unsigned)std::min<int64_t>(cdivl(nw, 256), 65536)), dim3(256), 0, s,
                       ctx->lr_w.p, nw);
    const dim3 gw((unsigned)cdivl(maxp, 4), (unsigned)T);
    switch (rp_of(r)) {
        case 1: case 2: case 4: case 8: launch_lr<8>(ctx, x, gw, maxp, V, r, Y); break;
        case 16: launch_lr<16>(ctx, x, gw, maxp, V, r, Y); break;
        case 32: launch_lr<32>(ctx, x, gw, maxp, V, r, Y); break;
        default: launch_lr<64>(ctx, x, gw, maxp, V, r, Y); break;
    }
    return check_launch(ctx, "k_lr_w/k_lr_y");
}

// G = X^T Y (r x r, double, host) for N x r fp32 device matrices (r <= 32).
static int lowrank_gram(rfxp_ctx* ctx, const float* X, const float* Y, int32_t r, std::vector<double>& G) {
    const int64_t N = ctx->ref_N;
    const int64_t nblk = cdivl(N, LR_GRAM_ROWS);
    RFXP_HIP(ctx, ctx->lr_part.ensure((size_t)nblk * r * r + (size_t)r * r));
    double* Gd = ctx->lr_part.p + nblk * r * r;
    hipLaunchKernelGGL(k_lr_gram, dim3((unsigned)nblk), dim3(1024), 0, ctx->stream, X, Y, N, r, ctx->lr_part.p);
    hipLaunchKernelGGL(k_lr_gram_sum, dim3((unsigned)cdivl(r * r, 256)), dim3(256), 0, ctx->stream, ctx->lr_part.p,
                       nblk, r * r, Gd);
    if (int rc = check_launch(ctx, "k_lr_gram")) return rc;
    G.resize((size_t)r * r);
    RFXP_HIP(ctx, hipMemcpyAsync(G.data(), Gd, sizeof(double) * r * r, hipMemcpyDeviceToHost, ctx->stream));
    RFXP_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return RFXP_OK;
}

// One CholeskyQR step: X = Q R with R upper triangular, positive diagonal;
// Q written to `Q` (may alias X).
static int lowrank_cholqr(rfxp_ctx* ctx, const float* X, int32_t r, float* Q) {
    std::vector<double> G;
    if (int rc = lowrank_gram(ctx, X, X, r, G)) return rc;
    // G = R^T R (Cholesky, upper R)
    std::vector<double> R((size_t)r * r, 0.0), Ri((size_t)r * r, 0.0);
    for (int32_t j = 0; j < r; ++j) {
        double d = G[(size_t)j * r + j];
        for (int32_t k = 0; k < j; ++k) d -= R[(size_t)k * r + j] * R[(size_t)k * r + j];
        if (!(d > 0.0)) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_lowrank_subspace: block is rank deficient");
        const double rjj = std::sqrt(d);
        R[(size_t)j * r + j] = rjj;
        for (int32_t c = j + 1; c < r; ++c) {
            double v = G[(size_t)j * r + c];
            for (int32_t k = 0; k < j; ++k) v -= R[(size_t)k * r + j] * R[(size_t)k * r + c];
            R[(size_t)j * r + c] = v / rjj;
        }
    }
    // Ri = R^-1 (upper triangular), column by column
    for (int32_t c = 0; c < r; ++c) {
        for (int32_t a = c; a >= 0; --a) {
            double v = (a == c) ? 1.0 : 0.0;
            for (int32_t k = a + 1; k <= c; ++k) v -= R[(size_t)a * r + k] * Ri[(size_t)k * r + c];
            Ri[(size_t)a * r + c] = v / R[(size_t)a * r + a];
        }
    }
    RFXP_HIP(ctx, ctx->lr_rinv.ensure((size_t)r * r));
    RFXP_HIP(ctx, hipMemcpyAsync(ctx->lr_rinv.p, Ri.data(), sizeof(double) * r * r, hipMemcpyHostToDevice,
                                 ctx->stream));
    const int64_t N = ctx->ref_N;
    if (X == Q) {
        RFXP_HIP(ctx, ctx->lr_tmp.ensure((size_t)N * r));
        RFXP_HIP(ctx, hipMemcpyAsync(ctx->lr_tmp.p, X, sizeof(float) * N * r, hipMemcpyDeviceToDevice, ctx->stream));
        X = ctx->lr_tmp.p;
    }
    hipLaunchKernelGGL(k_lr_trmm, dim3((unsigned)cdivl(N * r, 256)), dim3(256), 0, ctx->stream, X, ctx->lr_rinv.p, N,
                       r, Q);
    if (int rc = check_launch(ctx, "k_lr_trmm")) return rc;
    RFXP_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return RFXP_OK;
}

extern "C" int rfxp_lowrank_pv(rfxp_ctx* ctx, const float* V, int32_t r, float* Y) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (!ctx->ref_ready) return set_error(ctx, RFXP_ERR_STATE, "rfxp_lowrank_pv: no reference set");
    if (r < 1 || r > LR_MAX_R) return set_error(ctx, RFXP_ERR_UNSUPPORTED, "rfxp_lowrank_pv: need 1 <= r <= 64");
    if (!V || !Y || !is_device_pointer(V) || !is_device_pointer(Y))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_lowrank_pv: V and Y must be device pointers");
    if (V == Y) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_lowrank_pv: V and Y must not alias");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    return lowrank_apply(ctx, V, r, Y);
}

extern "C" int rfxp_lowrank_subspace(rfxp_ctx* ctx, const float* V0, int32_t r, int32_t iters, float* Q, double* B) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (!ctx->ref_ready) return set_error(ctx, RFXP_ERR_STATE, "rfxp_lowrank_subspace: no reference set");
    if (r < 1 || r > 32) return set_error(ctx, RFXP_ERR_UNSUPPORTED, "rfxp_lowrank_subspace: need 1 <= r <= 32");
    if (iters < 0) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_lowrank_subspace: iters < 0");
    if (!V0 || !Q || !B || !is_device_pointer(V0) || !is_device_pointer(Q) || V0 == Q)
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_lowrank_subspace: V0, Q device, distinct; B host");
    if (ctx->ref_N < r) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_lowrank_subspace: N < r");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    const int64_t N = ctx->ref_N;
    RFXP_HIP(ctx, ctx->lr_z.ensure((size_t)N * r));
    float* Z = ctx->lr_z.p;
    // Q0 = orth(V0), CholeskyQR2
    if (int rc = lowrank_cholqr(ctx, V0, r, Q)) return rc;
    if (int rc = lowrank_cholqr(ctx, Q, r, Q)) return rc;
    for (int32_t k = 0; k < iters; ++k) {
        if (int rc = lowrank_apply(ctx, Q, r, Z)) return rc;
        if (int rc = lowrank_cholqr(ctx, Z, r, Q)) return rc;
        if (int rc = lowrank_cholqr(ctx, Q, r, Q)) return rc;
    }
    // Ritz matrix B = Q^T P Q
    if (int rc = lowrank_apply(ctx, Q, r, Z)) return rc;
    std::vector<double> G;
    if (int rc = lowrank_gram(ctx, Q, Z, r, G)) return rc;
    std::copy(G.begin(), G.end(), B);
    return RFXP_OK;
}

// ---------------------------------------------------------------------------
// OOB-normalised proximity applied through the forest's buckets
// ---------------------------------------------------------------------------
// P = 1/4 (D^-1 U + U D^-1) + I with U_ij = #{t : same leaf, oob_i != oob_j}
// and D^-1 = diag(r), r = nout > 0 ? 1/nout : 1: the matrix
// cpu_finishprox produces from the OOB co-occurrence counts
// (src/rf_finishprox.cpp:12-74; 1/4 (r_i + r_j) U_ij is its
// 0.5 (U/2 r_i + U/2 r_j), and the diagonal is 1).  U X is a bucket SpMM on
// the forest index of rfxp_set_forest (bucket b = 2 leaf + oob):
//     W_t[b] = sum over the members j of bucket b of X_j,
//     (U X)_i = sum_t W_t[b(i, t) xor 1]   (the bucket of the other OOB bit),
// which is B A^T + A B^T - 2 B B^T applied to X, A the one-hot leaf matrix
// and B its OOB entries.  X = [V, r o V] gives both products in one pass.

namespace rfxp {

// W[(t*nb + b)*c2 + c] = sum over bucket b of tree t of X[j*c2 + c].  The
// bucket's members are mem[t][off[b] .. end), end = bend[b] (line-fit
// layout, tree stride ms) or off[b + 1].
__global__ __launch_bounds__(256) void k_oob_w(const int32_t* off, const int32_t* bend, const uint32_t* mem,
                                               int64_t ms, int32_t T, int32_t nb, const float* X, int32_t c2,
                                               float* W) {
    const int64_t wb = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wb >= (int64_t)T * nb) return;
    const int32_t t = (int32_t)(wb / nb), b = (int32_t)(wb % nb);
    const int32_t c = threadIdx.x & 63;
    const int32_t* ot = off + (int64_t)t * (nb + 1);
    const uint32_t* m = mem + (int64_t)t * ms;
    const int32_t s = ot[b], e = bend ? bend[(int64_t)t * nb + b] : ot[b + 1];
    double acc = 0.0;
    if (c < c2)
        for (int32_t k = s; k < e; ++k) acc += (double)X[(int64_t)((m[k] & MEM_ID) - 1u) * c2 + c];
    if (c < c2) W[wb * c2 + c] = (float)acc;
}

// Y[i*r + c] = 1/4 (r_i Z_i,c + Z_i,r+c) + V_i,c with Z = U [V, r o V]
// formed per sample from the other bucket's W row in every tree.
__global__ __launch_bounds__(256) void k_oob_y(const int32_t* leaf, int64_t si, int64_t st, const uint32_t* oob,
                                               int64_t old, int64_t N, int32_t T, int32_t L, int32_t nb,
                                               const float* W, const float* V, const double* rinv, int32_t r,
                                               float* Y) {
    const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= N) return;
    const int32_t c = threadIdx.x & 63;
    const int32_t c2 = 2 * r;
    double acc = 0.0;
    for (int32_t t = 0; t < T; ++t) {
        const int32_t l = leaf[i * si + (int64_t)t * st];
        if (l < 0 || l >= L) continue;
        const uint32_t o = (oob[(int64_t)t * old + (i >> 5)] >> (i & 31)) & 1u;
        const int32_t ob = 2 * l + (int32_t)(o ^ 1u);
        if (c < c2) acc += (double)W[((int64_t)t * nb + ob) * c2 + c];
    }
    // lanes r..2r-1 hold U (r o V); lane c < r combines with lane c + r
    const double other = __shfl_down(acc, r, 64);
    if (c < r) Y[i * r + c] = (float)(0.25 * (rinv[i] * acc + other) + (double)V[i * r + c]);
}

__global__ void k_oob_x2(const float* V, const double* rinv, int64_t N, int32_t r, float* X2) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= N * r) return;
    const int64_t i = e / r;
    const int32_t c = (int32_t)(e % r);
    const float v = V[e];
    X2[i * 2 * r + c] = v;
    X2[i * 2 * r + r + c] = (float)(rinv[i] * (double)v);
}

}  // namespace rfxp

extern "C" int rfxp_lowrank_oob_pv(rfxp_ctx* ctx, const float* V, int32_t r, float* Y) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (!ctx->forest_ready) return set_error(ctx, RFXP_ERR_STATE, "rfxp_lowrank_oob_pv: no forest set");
    if (r < 1 || r > 32) return set_error(ctx, RFXP_ERR_UNSUPPORTED, "rfxp_lowrank_oob_pv: need 1 <= r <= 32");
    if (!V || !Y || !is_device_pointer(V) || !is_device_pointer(Y) || V == Y)
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_lowrank_oob_pv: V and Y distinct device pointers");
    const int64_t N = ctx->N;
    const int32_t T = ctx->T, L = ctx->L, nb = 2 * L;
    if (N == 0) return RFXP_OK;
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    RFXP_HIP(ctx, ctx->lr_tmp.ensure((size_t)N * 2 * r));
    RFXP_HIP(ctx, ctx->lr_w.ensure((size_t)T * nb * 2 * r));
    const unsigned nx = (unsigned)((N * r + 255) / 256);
    hipLaunchKernelGGL(k_oob_x2, dim3(nx), dim3(256), 0, ctx->stream, V, ctx->fb.rinv, N, r, ctx->lr_tmp.p);
    const int64_t nw = (int64_t)T * nb;
    {
        LaunchTimer tm(ctx, "lr_oob_w");
        hipLaunchKernelGGL(k_oob_w, dim3((unsigned)((nw + 3) / 4)), dim3(256), 0, ctx->stream, ctx->fb.off, ctx->fb.bend,
                           ctx->fb.mem, ctx->fb.ms, T, nb, ctx->lr_tmp.p, 2 * r, ctx->lr_w.p);
    }
    {
        LaunchTimer tm(ctx, "lr_oob_y");
        hipLaunchKernelGGL(k_oob_y, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, ctx->stream, ctx->fo_leaf, ctx->fo_si,
                           ctx->fo_st, ctx->fo_oob, ctx->fo_old, N, T, L, nb, ctx->lr_w.p, V, ctx->fb.rinv, r, Y);
    }
    return check_launch(ctx, "k_oob launch");
}
