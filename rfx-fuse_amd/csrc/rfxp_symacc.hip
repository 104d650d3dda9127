// Engine of the LowRankProximityMatrix surface (include/rf_proximity_lowrank.hpp:27-433):
// a sparse accumulator of symmetric contributions and what is computed from
// it, all in double on the device.
//
// The reference keeps, per added tree, a rank-1 power-iteration factor of
// that tree's FP16 triangle (cuda/rf_proximity_lowrank.cu:865-1038).  Here
// the contributions themselves are kept, exactly, as a sparse matrix
//     M = sum over contributions C of C   (C symmetric, given as its packed
//                                         upper triangle or as a dense matrix)
// and the factor is computed from M when it is asked for:
//   * accumulation, sparse form: per contribution, a row-count pass, a
//     device prefix scan of the counts (the host reads back only their
//     total, to size the list) and an ordered emit pass append the nonzero
//     entries (i <= j, value) to a device COO list; values are read the way
//     the reference's low-rank path reads them (FP16 as is, INT8 and NF4
//     dequantised and rounded to FP16, cuda/rf_proximity_lowrank.cu:199-240,
//     744-789; a dense matrix's upper triangle rounded to FP16, :654-685);
//   * accumulation, dense form: once the list and its CSR (12 + 16 bytes an
//     entry) would take more than the packed upper triangle of M in doubles
//     (8 bytes an entry of N(N+1)/2), the list is summed into that triangle
//     and every later contribution is added to it in place, one pass over
//     the input.  The accumulator's memory is so bounded by the triangle,
//     whatever the number of contributions.  Sums of FP16-valued entries
//     (every format but F32) are exact in double up to 8192 contributions
//     (multiples of 2^-24 below 2^16), so they do not depend on the order of
//     the additions;
//   * inputs in host memory are staged through the device in bands of rows
//     of at most SA_STAGE_BYTES;
//   * factor: the COO list becomes a symmetric CSR (both halves), then block
//     subspace iteration with Rayleigh-Ritz: X_0 random normal, Q_k =
//     orth(M Q_{k-1}), H = Q^T M Q = U diag(lambda) U^T, and
//     A[:, c] = Q U[:, c] sqrt(lambda_c) for the r largest lambda_c > 0 (0
//     for the others), so that A A^T is the rank-r positive part of M.  orth
//     is CholeskyQR2, or, when the Gram matrix is numerically singular, the
//     eigenvalue-based SVQB that drops null directions;
//   * reconstruction and MDS from a factor (B = A): P = A A^T with the
//     reference's diagonal and RF-GAP conventions, and classical MDS of
//     D = 1 - P/max diag P applied through the factor (no N x N matrix).
//
// Dense blocks are N x b row-major doubles.  The host does the b x b linear
// algebra (Cholesky, Jacobi eigenvalues).  The CSR is built with atomics,
// so the order of the terms within a row -- and the last bits of the
// double sums -- may change from run to run; in the dense form the
// products M X are summed in a fixed order.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <numeric>
#include <string>
#include <vector>

#include "rfxp_device.hpp"
#include "rfxp_forest.hpp"
#include "rfxp_internal.hpp"

namespace rfxp {

// ---------------------------------------------------------------------------
// host linear algebra (b x b, row-major)
// ---------------------------------------------------------------------------

// Cyclic Jacobi eigenvalue iteration of the symmetric n x n matrix a
// (destroyed).  w gets the eigenvalues in descending order, v (n x n,
// row-major) the matching eigenvectors as columns.
void host_symeig(int n, std::vector<double>& a, std::vector<double>& w, std::vector<double>& v) {
    v.assign((size_t)n * n, 0.0);
    for (int i = 0; i < n; ++i) v[(size_t)i * n + i] = 1.0;
    auto A = [&](int r, int c) -> double& { return a[(size_t)r * n + c]; };
    auto V = [&](int r, int c) -> double& { return v[(size_t)r * n + c]; };
    double fro = 0.0;
    for (size_t k = 0; k < (size_t)n * n; ++k) fro += a[k] * a[k];
    fro = sqrt(fro);
    for (int sweep = 0; sweep < 100 && fro > 0.0; ++sweep) {
        double off = 0.0;
        for (int p = 0; p < n; ++p)
            for (int q = p + 1; q < n; ++q) off += A(p, q) * A(p, q);
        if (sqrt(2.0 * off) <= 1e-15 * fro) break;
        for (int p = 0; p < n; ++p) {
            for (int q = p + 1; q < n; ++q) {
                const double apq = A(p, q);
                if (fabs(apq) <= 1e-300) continue;
                // rotation angle that zeroes a_pq
                const double theta = (A(q, q) - A(p, p)) / (2.0 * apq);
                const double t = (theta >= 0.0 ? 1.0 : -1.0) / (fabs(theta) + sqrt(theta * theta + 1.0));
                const double c = 1.0 / sqrt(t * t + 1.0), s = t * c;
                for (int k = 0; k < n; ++k) {  // columns p, q
                    const double akp = A(k, p), akq = A(k, q);
                    A(k, p) = c * akp - s * akq;
                    A(k, q) = s * akp + c * akq;
                }
                for (int k = 0; k < n; ++k) {  // rows p, q
                    const double apk = A(p, k), aqk = A(q, k);
                    A(p, k) = c * apk - s * aqk;
                    A(q, k) = s * apk + c * aqk;
                }
                for (int k = 0; k < n; ++k) {
                    const double vkp = V(k, p), vkq = V(k, q);
                    V(k, p) = c * vkp - s * vkq;
                    V(k, q) = s * vkp + c * vkq;
                }
            }
        }
    }
    std::vector<int> ord(n);
    std::iota(ord.begin(), ord.end(), 0);
    std::vector<double> d(n);
    for (int i = 0; i < n; ++i) d[i] = A(i, i);
    std::stable_sort(ord.begin(), ord.end(), [&](int x, int y) { return d[x] > d[y]; });
    std::vector<double> vs((size_t)n * n);
    w.resize(n);
    for (int c = 0; c < n; ++c) {
        w[c] = d[ord[c]];
        for (int r = 0; r < n; ++r) vs[(size_t)r * n + c] = V(r, ord[c]);
    }
    v.swap(vs);
}

// Upper-triangular R with G = R^T R (row-major); false when a pivot is not
// clearly positive (relative to the largest diagonal entry).
static bool host_cholesky(int n, const std::vector<double>& g, std::vector<double>& R) {
    R.assign((size_t)n * n, 0.0);
    double dmax = 0.0;
    for (int i = 0; i < n; ++i) dmax = std::max(dmax, g[(size_t)i * n + i]);
    if (!(dmax > 0.0)) return false;
    for (int i = 0; i < n; ++i) {
        double s = g[(size_t)i * n + i];
        for (int k = 0; k < i; ++k) s -= R[(size_t)k * n + i] * R[(size_t)k * n + i];
        if (!(s > 1e-13 * dmax)) return false;
        const double rii = sqrt(s);
        R[(size_t)i * n + i] = rii;
        for (int j = i + 1; j < n; ++j) {
            double t = g[(size_t)i * n + j];
            for (int k = 0; k < i; ++k) t -= R[(size_t)k * n + i] * R[(size_t)k * n + j];
            R[(size_t)i * n + j] = t / rii;
        }
    }
    return true;
}

// Inverse of an upper-triangular matrix (row-major).
static void host_triu_inv(int n, const std::vector<double>& R, std::vector<double>& Ri) {
    Ri.assign((size_t)n * n, 0.0);
    for (int j = 0; j < n; ++j) {
        Ri[(size_t)j * n + j] = 1.0 / R[(size_t)j * n + j];
        for (int i = j - 1; i >= 0; --i) {
            double s = 0.0;
            for (int k = i + 1; k <= j; ++k) s += R[(size_t)i * n + k] * Ri[(size_t)k * n + j];
            Ri[(size_t)i * n + j] = -s / R[(size_t)i * n + i];
        }
    }
}

// ---------------------------------------------------------------------------
// device kernels
// ---------------------------------------------------------------------------

// Source of a contribution: a packed upper triangle in one of the formats,
// or a dense N x N matrix read row-major (element (i, j) at p[i*N + j]).
// p may hold only a band of it: then p points at packed entry `base` (even
// for NF4) or at row `base` of the dense matrix.
enum SrcKind { SRC_F16 = 0, SRC_F32 = 1, SRC_I8 = 2, SRC_NF4 = 3, SRC_DENSE = 4 };
struct SymSrc {
    const void* p;
    int kind;
    float scale, zp;  // INT8 dequantisation
    int64_t N;
    int64_t base;
};

__device__ __forceinline__ float half_bits_to_float(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ float round_half(float v) { return (float)(_Float16)v; }

// Value of entry (i, j), i <= j, with packed index e.
__device__ __forceinline__ float src_value(const SymSrc& s, int64_t i, int64_t j, int64_t e) {
    const int64_t k = e - s.base;
    switch (s.kind) {
        case SRC_F16: return half_bits_to_float(((const uint16_t*)s.p)[k]);
        case SRC_F32: return ((const float*)s.p)[k];
        case SRC_I8: {
            // int8_to_fp32 (include/rf_quantization_kernels.hpp:32-34), then FP16
            const float v = ((float)((const int8_t*)s.p)[k] - s.zp) * s.scale;
            return round_half(v);
        }
        case SRC_NF4: {
            const uint32_t q = (((const uint8_t*)s.p)[k >> 1] >> ((k & 1) * 4)) & 0xfu;
            const float v = q <= 7u ? (float)q / 7.0f : -((float)(q - 8u)) / 7.0f;  // nf4_to_fp32
            return round_half(v);
        }
        default: return round_half((float)((const double*)s.p)[(i - s.base) * s.N + j]);
    }
}

constexpr int SA_THREADS = 256;

// Nonzero entries of rows row0 + blockIdx.x into cnt[row].
__global__ __launch_bounds__(SA_THREADS) void k_sa_rowcount(SymSrc s, int64_t row0, int64_t* cnt) {
    __shared__ int64_t part[SA_THREADS / 64];
    const int64_t i = row0 + blockIdx.x;
    const int64_t e0 = tri_idx(s.N, i, i);
    int64_t c = 0;
    for (int64_t j = i + threadIdx.x; j < s.N; j += SA_THREADS) c += src_value(s, i, j, e0 + (j - i)) != 0.0f;
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) c += __shfl_xor(c, d, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = c;
    __syncthreads();
    if (threadIdx.x == 0) cnt[i] = part[0] + part[1] + part[2] + part[3];
}

// The nonzero entries of the rows, in column order, at off[row].
__global__ __launch_bounds__(SA_THREADS) void k_sa_rowemit(SymSrc s, int64_t row0, const int64_t* off, int32_t* ci,
                                                           int32_t* cj, float* cv) {
    __shared__ uint32_t wsum[SA_THREADS / 64];
    const int64_t i = row0 + blockIdx.x;
    const int64_t e0 = tri_idx(s.N, i, i);
    int64_t pos = off[i];
    const uint32_t wave = threadIdx.x >> 6;
    for (int64_t jb = i; jb < s.N; jb += SA_THREADS) {
        const int64_t j = jb + threadIdx.x;
        const float v = j < s.N ? src_value(s, i, j, e0 + (j - i)) : 0.0f;
        const bool nz = v != 0.0f;
        const uint64_t m = __ballot(nz);
        const uint32_t before = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
        if ((threadIdx.x & 63) == 0) wsum[wave] = (uint32_t)__popcll(m);
        __syncthreads();
        uint32_t wbase = 0, tot = 0;
#pragma unroll
        for (uint32_t w = 0; w < SA_THREADS / 64; ++w) {
            wbase += w < wave ? wsum[w] : 0u;
            tot += wsum[w];
        }
        if (nz) {
            const int64_t p = pos + wbase + before;
            ci[p] = (int32_t)i;
            cj[p] = (int32_t)j;
            cv[p] = v;
        }
        pos += tot;
        __syncthreads();
    }
}

// cnt[r0 .. r0 + nr) replaced by its exclusive prefix sums plus base, the
// total into *tot: one workgroup, each thread over a contiguous chunk, the
// chunk sums scanned in LDS.
constexpr int SCAN_T = 1024;
__global__ __launch_bounds__(SCAN_T) void k_sa_scan(int64_t* cnt, int64_t r0, int64_t nr, int64_t base,
                                                    int64_t* tot) {
    __shared__ int64_t part[SCAN_T];
    const int64_t per = (nr + SCAN_T - 1) / SCAN_T;
    const int64_t b = r0 + min(nr, per * threadIdx.x), e = r0 + min(nr, per * (threadIdx.x + 1));
    int64_t sum = 0;
    for (int64_t i = b; i < e; ++i) sum += cnt[i];
    part[threadIdx.x] = sum;
    __syncthreads();
    for (int d = 1; d < SCAN_T; d <<= 1) {  // inclusive scan of the chunk sums
        const int64_t v = threadIdx.x >= (unsigned)d ? part[threadIdx.x - d] : 0;
        __syncthreads();
        part[threadIdx.x] += v;
        __syncthreads();
    }
    int64_t run = base + (threadIdx.x ? part[threadIdx.x - 1] : 0);
    for (int64_t i = b; i < e; ++i) {
        const int64_t c = cnt[i];
        cnt[i] = run;
        run += c;
    }
    if (threadIdx.x == SCAN_T - 1) *tot = part[SCAN_T - 1];
}

// Symmetric CSR from the COO list: degrees, then placement at cursors.
__global__ void k_sa_degree(const int32_t* ci, const int32_t* cj, int64_t nnz, unsigned long long* deg) {
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < nnz; e += (int64_t)gridDim.x * blockDim.x) {
        const int32_t i = ci[e], j = cj[e];
        atomicAdd(&deg[i], 1ull);
        if (j != i) atomicAdd(&deg[j], 1ull);
    }
}

__global__ void k_sa_place(const int32_t* ci, const int32_t* cj, const float* cv, int64_t nnz,
                           unsigned long long* cur, int32_t* col, float* val) {
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < nnz; e += (int64_t)gridDim.x * blockDim.x) {
        const int32_t i = ci[e], j = cj[e];
        const float v = cv[e];
        const unsigned long long p = atomicAdd(&cur[i], 1ull);
        col[p] = j;
        val[p] = v;
        if (j != i) {
            const unsigned long long q = atomicAdd(&cur[j], 1ull);
            col[q] = i;
            val[q] = v;
        }
    }
}

// Y = M X, X and Y N x b row-major: one wave per row, lanes over columns.
__global__ __launch_bounds__(256) void k_sa_spmm(const int64_t* rowptr, const int32_t* col, const float* val,
                                                 const double* X, int64_t N, int32_t b, double* Y) {
    const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= N) return;
    const int32_t lane = threadIdx.x & 63;
    const int64_t k0 = rowptr[i], k1 = rowptr[i + 1];
    for (int32_t cb = 0; cb < b; cb += 64) {
        const int32_t c = cb + lane;
        double acc = 0.0;
        if (c < b)
            for (int64_t k = k0; k < k1; ++k) acc += (double)val[k] * X[(int64_t)col[k] * b + c];
        if (c < b) Y[i * b + c] = acc;
    }
}

// Dense form: the entries of rows row0 + blockIdx.x added to the packed
// triangle tri, in place (each entry is written by one thread).
__global__ __launch_bounds__(SA_THREADS) void k_sa_tri_add(SymSrc s, int64_t row0, double* tri) {
    const int64_t i = row0 + blockIdx.x;
    const int64_t e0 = tri_idx(s.N, i, i);
    for (int64_t j = i + threadIdx.x; j < s.N; j += SA_THREADS) {
        const int64_t e = e0 + (j - i);
        tri[e] += (double)src_value(s, i, j, e);
    }
}

// The COO list summed into the zeroed packed triangle (entries repeat
// across contributions: atomic adds).
__global__ void k_sa_list_to_tri(const int32_t* ci, const int32_t* cj, const float* cv, int64_t nnz, int64_t N,
                                 double* tri) {
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < nnz; e += (int64_t)gridDim.x * blockDim.x)
        atomicAdd(&tri[tri_idx(N, ci[e], cj[e])], (double)cv[e]);
}

// Dense form of Y = M X: M symmetric from its packed upper triangle, X and Y
// N x b row-major.  A workgroup computes the 64 x 64 tile of Y at rows
// 64 blockIdx.x, columns 64 blockIdx.y, over slabs of 16 of the inner index
// j with both operands in LDS, 4 x 4 outputs per thread.  A slab of M is
// read along row i where it lies on or above the diagonal (j >= i) and
// along row j, transposed, where it lies wholly below it, so that
// neighbouring threads read neighbouring entries.
constexpr int TS_T = 64, TS_K = 16;
__global__ __launch_bounds__(256) void k_sa_tri_spmm(const double* tri, const double* X, int64_t N, int32_t b,
                                                     double* Y) {
    __shared__ double ms[TS_K][TS_T + 1];
    __shared__ double xs[TS_K][TS_T];
    const int64_t i0 = (int64_t)blockIdx.x * TS_T;
    const int32_t c0 = blockIdx.y * TS_T;
    const int32_t tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    double acc[4][4] = {};
    for (int64_t j0 = 0; j0 < N; j0 += TS_K) {
        const bool below = i0 >= j0 + TS_K;  // every i of the tile > every j of the slab
        for (int32_t t = threadIdx.x; t < TS_K * TS_T; t += 256) {
            const int32_t ii = below ? t % TS_T : t / TS_K, kk = below ? t / TS_T : t % TS_K;
            const int64_t i = i0 + ii, j = j0 + kk;
            double v = 0.0;
            if (i < N && j < N) v = i <= j ? tri[tri_idx(N, i, j)] : tri[tri_idx(N, j, i)];
            ms[kk][ii] = v;
        }
        for (int32_t t = threadIdx.x; t < TS_K * TS_T; t += 256) {
            const int32_t kk = t / TS_T, cc = t % TS_T;
            const int64_t j = j0 + kk;
            xs[kk][cc] = j < N && c0 + cc < b ? X[j * b + c0 + cc] : 0.0;
        }
        __syncthreads();
#pragma unroll 4
        for (int32_t kk = 0; kk < TS_K; ++kk) {
            double ma[4], xc[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                ma[u] = ms[kk][ty * 4 + u];
                xc[u] = xs[kk][tx * 4 + u];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[u][v] += ma[u] * xc[v];
        }
        __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int64_t i = i0 + ty * 4 + u;
            const int32_t c = c0 + tx * 4 + v;
            if (i < N && c < b) Y[i * b + c] = acc[u][v];
        }
}

// Partial sums of G = X^T diag(w) Y over chunks of GR rows: X is N x bx,
// Y is N x by (row-major), w optional; one 64 x 64 tile of G per
// workgroup and chunk, 4 x 4 outputs per thread.
constexpr int GT = 64, GR = 2048, GS = 16;
__global__ __launch_bounds__(256) void k_gram_part(const double* X, int32_t bx, const double* Y, int32_t by,
                                                   const double* w, int64_t N, double* part) {
    __shared__ double xs[GS][GT];
    __shared__ double ys[GS][GT];
    const int32_t a0 = blockIdx.x * GT, c0 = blockIdx.y * GT;
    const int64_t r0 = (int64_t)blockIdx.z * GR, r1 = min(N, r0 + GR);
    const int32_t tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    double acc[4][4] = {};
    for (int64_t rb = r0; rb < r1; rb += GS) {
        for (int32_t k = threadIdx.x; k < GS * GT; k += 256) {
            const int32_t rr = k / GT, cc = k % GT;
            const int64_t row = rb + rr;
            double xv = 0.0, yv = 0.0;
            if (row < r1) {
                if (a0 + cc < bx) xv = X[row * bx + a0 + cc];
                if (c0 + cc < by) yv = Y[row * by + c0 + cc];
                if (w) xv *= w[row];
            }
            xs[rr][cc] = xv;
            ys[rr][cc] = yv;
        }
        __syncthreads();
#pragma unroll 4
        for (int32_t rr = 0; rr < GS; ++rr) {
            double xa[4], yc[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                xa[u] = xs[rr][ty * 4 + u];
                yc[u] = ys[rr][tx * 4 + u];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[u][v] += xa[u] * yc[v];
        }
        __syncthreads();
    }
    double* out = part + (int64_t)blockIdx.z * bx * by;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int32_t a = a0 + ty * 4 + u, c = c0 + tx * 4 + v;
            if (a < bx && c < by) out[(int64_t)a * by + c] = acc[u][v];
        }
}

__global__ void k_gram_sum(const double* part, int64_t nchunk, int64_t n, double* G) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n) return;
    double s = 0.0;
    for (int64_t c = 0; c < nchunk; ++c) s += part[c * n + e];
    G[e] = s;
}

// Z = X W: X N x b (row-major, leading dimension b), W b x c row-major on the
// device; Z row-major N x c, or column-major (Z[i + k*N]) when colmajor.
// A workgroup stages R rows of X in LDS.
__global__ __launch_bounds__(256) void k_gemm_nn(const double* X, int32_t b, const double* W, int32_t c, int64_t N,
                                                 int32_t R, double* Z, int colmajor) {
    extern __shared__ double xs[];
    const int64_t r0 = (int64_t)blockIdx.x * R;
    const int32_t nr = (int32_t)min((int64_t)R, N - r0);
    for (int32_t k = threadIdx.x; k < nr * b; k += 256) xs[k] = X[r0 * b + k];
    __syncthreads();
    for (int32_t o = threadIdx.x; o < nr * c; o += 256) {
        const int32_t rr = o / c, cc = o % c;
        const double* xr = xs + (int64_t)rr * b;
        double acc = 0.0;
        for (int32_t k = 0; k < b; ++k) acc += xr[k] * W[(int64_t)k * c + cc];
        if (colmajor) Z[r0 + rr + (int64_t)cc * N] = acc;
        else Z[(r0 + rr) * c + cc] = acc;
    }
}

// Standard normal entries from a counter-based hash (splitmix64) and the
// Box-Muller transform: entry e depends only on (seed, e).
__device__ __forceinline__ uint64_t splitmix(uint64_t x) {
    x += 0x9e3779b97f4a7c15ull;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
    return x ^ (x >> 31);
}
__global__ void k_randn(double* X, int64_t n, uint64_t seed) {
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
        const uint64_t h1 = splitmix(seed ^ splitmix((uint64_t)e * 2u));
        const uint64_t h2 = splitmix(seed ^ splitmix((uint64_t)e * 2u + 1u));
        const double u1 = ((double)(h1 >> 11) + 1.0) * (1.0 / 9007199254740993.0);  // (0, 1]
        const double u2 = (double)(h2 >> 11) * (1.0 / 9007199254740992.0);         // [0, 1)
        X[e] = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
    }
}

// Column-major N x r -> row-major N x r.
__global__ void k_to_rowmajor(const double* A, int64_t N, int32_t r, double* Ar) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= N * r) return;
    const int64_t i = e / r;
    const int32_t c = (int32_t)(e % r);
    Ar[e] = A[i + (int64_t)c * N];
}

// Reconstruction P = A B^T into the column-major N x N `out`
// (cuda/rf_proximity_lowrank.cu:1274-1376): the dot products in column
// order, the diagonal set to 1, and, with RF-GAP counts s (w = 1/s where
// s > 0), each row scaled by its w and every off-diagonal pair averaged,
// 0.5 * (P*w_lo + P*w_hi), lo = min(i, j), hi = max(i, j), with w_i on the
// diagonal.  The reference's symmetrisation launch (:1356-1372) covers only
// about N of the N^2 linear indices (row 0's pairs), leaving the rest with
// one-sided scales; this kernel symmetrises every pair instead, as that
// step intends.
__global__ void k_reconstruct(const double* A, const double* B, int64_t N, int32_t r, const double* winv,
                              const int32_t* s, double* out) {
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < N * N;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = e % N, cl = e / N;
        double p = 0.0;
        if (row == cl) {
            p = 1.0;
            if (s && s[row] > 0) p *= winv[row];
        } else {
            for (int32_t c = 0; c < r; ++c) p += A[row + (int64_t)c * N] * B[cl + (int64_t)c * N];
            if (s) {
                const int64_t lo = min(row, cl), hi = max(row, cl);
                const double x = s[lo] > 0 ? p * winv[lo] : p;
                const double y = s[hi] > 0 ? p * winv[hi] : p;
                p = 0.5 * (x + y);
            }
        }
        out[e] = p;
    }
}

// Per-row elementwise helpers of the MDS operator (row-major blocks).
// V <- V - column means (mean[c] precomputed), in place.
__global__ void k_center_cols(double* V, int64_t N, int32_t c, const double* mean) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= N * c) return;
    V[e] -= mean[e % c];
}
// out[i, k] = sum_c Z[i, c] * A[i, c]  (row quadratic forms; Z, A N x r)
__global__ void k_rowdot(const double* Z, const double* A, int64_t N, int32_t r, double* out, int32_t ldo, int32_t k) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    double s = 0.0;
    for (int32_t c = 0; c < r; ++c) s += Z[i * r + c] * A[i * r + c];
    out[i * ldo + k] = s;
}
// Y[i, c] = alpha * T1[i, c] + beta * T2[i, c] (T2 may alias nothing)
__global__ void k_axpby(const double* T1, const double* T2, double alpha, double beta, int64_t n, double* Y) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n) return;
    Y[e] = alpha * T1[e] + beta * T2[e];
}
// Y[i, c] *= w[i]
__global__ void k_scale_rows(double* Y, const double* w, int64_t N, int32_t c) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= N * c) return;
    Y[e] *= w[e / c];
}
// column k of T2 (N x c) = 1/4 (w^2 h0 + 2 w h1 + h2), h = H3 (N x 3)
__global__ void k_rfgap_combine(const double* H3, const double* w, const double* w2, int64_t N, double* T2, int32_t c,
                                int32_t k) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    T2[i * c + k] = 0.25 * (w2[i] * H3[i * 3] + 2.0 * w[i] * H3[i * 3 + 1] + H3[i * 3 + 2]);
}
// column c of X (N x b row-major) into v (N)
__global__ void k_get_col(const double* X, int64_t N, int32_t b, int32_t c, double* v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    v[i] = X[i * b + c];
}
// squared row norms of A (N x r row-major)
__global__ void k_rownorm2(const double* A, int64_t N, int32_t r, double* d) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    double s = 0.0;
    for (int32_t c = 0; c < r; ++c) s += A[i * r + c] * A[i * r + c];
    d[i] = s;
}

static unsigned nblk(int64_t n, int t = 256) { return (unsigned)((n + t - 1) / t); }

// Grid of a grid-stride kernel over n elements, 256 threads a workgroup.
static unsigned gsblk(int64_t n) { return grid_stride_blocks(n, 256); }

// ---------------------------------------------------------------------------
// dense block operations (host drivers)
// ---------------------------------------------------------------------------

struct Blocks {
    rfxp_ctx* ctx;
    DevBuf<double> part, gdev, wdev;
};

// G (host, bx x by row-major) = X^T diag(w) Y.
static int gram(rfxp_ctx* ctx, DevBuf<double>& part, DevBuf<double>& gdev, const double* X, int32_t bx, const double* Y,
                int32_t by, const double* w, int64_t N, std::vector<double>& G) {
    const int64_t nchunk = (N + GR - 1) / GR;
    const int64_t n = (int64_t)bx * by;
    RFXP_HIP(ctx, part.ensure((size_t)(nchunk * n)));
    RFXP_HIP(ctx, gdev.ensure((size_t)n));
    dim3 grid((unsigned)((bx + GT - 1) / GT), (unsigned)((by + GT - 1) / GT), (unsigned)nchunk);
    hipLaunchKernelGGL(k_gram_part, grid, dim3(256), 0, ctx->stream, X, bx, Y, by, w, N, part.p);
    hipLaunchKernelGGL(k_gram_sum, dim3(nblk(n)), dim3(256), 0, ctx->stream, part.p, nchunk, n, gdev.p);
    if (int rc = check_launch(ctx, "k_gram")) return rc;
    G.resize((size_t)n);
    RFXP_HIP(ctx, hipMemcpyAsync(G.data(), gdev.p, sizeof(double) * n, hipMemcpyDeviceToHost, ctx->stream));
    RFXP_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return RFXP_OK;
}

// Z = X W with W (b x c) from the host.
static int gemm_nn(rfxp_ctx* ctx, DevBuf<double>& wdev, const double* X, int32_t b, const std::vector<double>& W,
                   int32_t c, int64_t N, double* Z, bool colmajor) {
    RFXP_HIP(ctx, wdev.ensure((size_t)b * c));
    RFXP_HIP(ctx, hipMemcpyAsync(wdev.p, W.data(), sizeof(double) * b * c, hipMemcpyHostToDevice, ctx->stream));
    const int32_t R = std::max(1, std::min(64, 8192 / std::max(1, b)));
    const size_t lds = sizeof(double) * (size_t)R * b;
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute((const void*)k_gemm_nn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return hip_error(ctx, e, "k_gemm_nn attribute");
    }
    hipLaunchKernelGGL(k_gemm_nn, dim3((unsigned)((N + R - 1) / R)), dim3(256), lds, ctx->stream, X, b, wdev.p, c, N, R, Z,
                       colmajor ? 1 : 0);
    if (int rc = check_launch(ctx, "k_gemm_nn")) return rc;
    // wdev is reused by the next call: keep this one ordered before it
    RFXP_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return RFXP_OK;
}

// Q = orth(Y) (N x b, Q may alias nothing of Y): CholeskyQR2, or SVQB when
// the Gram matrix is numerically singular (null directions become zero
// columns).  tmp: an N x b scratch block.
static int orth(rfxp_ctx* ctx, DevBuf<double>& part, DevBuf<double>& gdev, DevBuf<double>& wdev, const double* Y,
                double* Q, double* tmp, int32_t b, int64_t N) {
    const double* src = Y;
    for (int pass = 0; pass < 2; ++pass) {
        std::vector<double> G, R, W;
        if (int rc = gram(ctx, part, gdev, src, b, src, b, nullptr, N, G)) return rc;
        if (host_cholesky(b, G, R)) {
            host_triu_inv(b, R, W);
        } else {
            std::vector<double> w, V;
            host_symeig(b, G, w, V);
            W.assign((size_t)b * b, 0.0);
            const double wmax = w.empty() ? 0.0 : w[0];
            for (int c = 0; c < b; ++c) {
                if (!(w[c] > 1e-13 * wmax)) continue;
                const double f = 1.0 / sqrt(w[c]);
                for (int k = 0; k < b; ++k) W[(size_t)k * b + c] = V[(size_t)k * b + c] * f;
            }
        }
        double* dst = pass == 0 ? tmp : Q;
        if (int rc = gemm_nn(ctx, wdev, src, b, W, b, N, dst, false)) return rc;
        src = dst;
    }
    return RFXP_OK;
}

}  // namespace rfxp

using namespace rfxp;

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------

extern "C" int rfxp_host_symeig(int32_t n, const double* a, double* w, double* v) {
    if (n < 1 || !a || !w) return RFXP_ERR_INVALID;
    std::vector<double> A(a, a + (size_t)n * n), W, V;
    host_symeig(n, A, W, V);
    std::copy(W.begin(), W.end(), w);
    if (v) std::copy(V.begin(), V.end(), v);
    return RFXP_OK;
}

namespace rfxp {

#ifndef RFXP_SA_STAGE_BYTES
#define RFXP_SA_STAGE_BYTES (256LL << 20)
#endif
// Largest band of a host input staged on the device at once.
constexpr int64_t SA_STAGE_BYTES = RFXP_SA_STAGE_BYTES;

static int64_t sa_entries(int64_t N) { return N * (N + 1) / 2; }

// Largest COO list of the sparse form: beyond it, the list (12 bytes an
// entry) and its symmetric CSR (up to 16 bytes an entry) would take more
// than the triangle of doubles (8 bytes an entry).
static int64_t sa_list_limit(int64_t N) { return sa_entries(N) / 7 * 2; }

// Bytes of the source holding packed entries [e0, e1) (e0 even for NF4), or
// dense rows [e0, e1).
static int64_t src_bytes(int kind, int64_t N, int64_t e0, int64_t e1) {
    switch (kind) {
        case SRC_F16: return 2 * (e1 - e0);
        case SRC_F32: return 4 * (e1 - e0);
        case SRC_I8: return e1 - e0;
        case SRC_NF4: return (e1 - e0 + 1) / 2;
        default: return 8 * N * (e1 - e0);
    }
}

// Switches the accumulator to the dense form: the CSR is dropped, the list
// summed into a zeroed triangle and released.
static int symacc_to_dense(rfxp_ctx* ctx) {
    const int64_t N = ctx->sa_N, ne = sa_entries(N);
    ctx->sa_col.release();
    ctx->sa_val.release();
    ctx->sa_csr_ok = false;
    if (ctx->sa_tri.ensure((size_t)ne) != hipSuccess)
        return set_error(ctx, RFXP_ERR_NOMEM,
                         "rfxp_symacc: cannot allocate the dense triangle (" + std::to_string(8 * ne) + " bytes)");
    fill_u32(ctx, (uint32_t*)ctx->sa_tri.p, 2 * ne, 0u);
    if (ctx->sa_nnz > 0)
        hipLaunchKernelGGL(k_sa_list_to_tri, dim3(gsblk(ctx->sa_nnz)), dim3(256), 0, ctx->stream, ctx->sa_i.p,
                           ctx->sa_j.p, ctx->sa_v.p, ctx->sa_nnz, N, ctx->sa_tri.p);
    if (int rc = check_launch(ctx, "k_sa_list_to_tri")) return rc;
    RFXP_HIP(ctx, hipStreamSynchronize(ctx->stream));
    ctx->sa_i.release();
    ctx->sa_j.release();
    ctx->sa_v.release();
    ctx->sa_dense = true;
    ctx->sa_nnz = ne;
    return RFXP_OK;
}

// Appends the nonzero entries of rows [r0, r1) (source s, staged) to the
// list, or, when the list would pass its limit, switches to the dense form
// and adds them there.  Row counts and their prefix sums stay on the device
// (sa_cnt[0 .. N)); only the total (sa_cnt[N]) is read back.
static int symacc_add_rows_sparse(rfxp_ctx* ctx, const SymSrc& s, int64_t r0, int64_t r1) {
    const int64_t nr = r1 - r0, N = ctx->sa_N;
    hipLaunchKernelGGL(k_sa_rowcount, dim3((unsigned)nr), dim3(SA_THREADS), 0, ctx->stream, s, r0, ctx->sa_cnt.p);
    hipLaunchKernelGGL(k_sa_scan, dim3(1), dim3(SCAN_T), 0, ctx->stream, ctx->sa_cnt.p, r0, nr, ctx->sa_nnz,
                       ctx->sa_cnt.p + N);
    if (int rc = check_launch(ctx, "k_sa_rowcount / k_sa_scan")) return rc;
    int64_t tot = 0;
    RFXP_HIP(ctx, hipMemcpyAsync(&tot, ctx->sa_cnt.p + N, sizeof(int64_t), hipMemcpyDeviceToHost, ctx->stream));
    RFXP_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (tot == 0) return RFXP_OK;
    const int64_t need = ctx->sa_nnz + tot, limit = sa_list_limit(ctx->sa_N);
    if (need > limit) {
        if (int rc = symacc_to_dense(ctx)) return rc;
        hipLaunchKernelGGL(k_sa_tri_add, dim3((unsigned)nr), dim3(SA_THREADS), 0, ctx->stream, s, r0, ctx->sa_tri.p);
        return check_launch(ctx, "k_sa_tri_add");
    }
    if ((size_t)need > ctx->sa_i.n) {  // grow by half again (up to the limit), keeping the entries
        ctx->sa_col.release();          // the CSR is rebuilt after an add anyway
        ctx->sa_val.release();
        const size_t cap =
            std::min<size_t>((size_t)limit, std::max<size_t>((size_t)need, ctx->sa_i.n + ctx->sa_i.n / 2));
        DevBuf<int32_t> ni, nj;
        DevBuf<float> nv;
        if (ni.ensure(cap) != hipSuccess || nj.ensure(cap) != hipSuccess || nv.ensure(cap) != hipSuccess) {
            ni.release();
            nj.release();
            nv.release();
            return set_error(ctx, RFXP_ERR_NOMEM, "rfxp_symacc: cannot grow the entry list");
        }
        if (ctx->sa_nnz > 0) {
            RFXP_HIP(ctx, hipMemcpyAsync(ni.p, ctx->sa_i.p, 4 * ctx->sa_nnz, hipMemcpyDeviceToDevice, ctx->stream));
            RFXP_HIP(ctx, hipMemcpyAsync(nj.p, ctx->sa_j.p, 4 * ctx->sa_nnz, hipMemcpyDeviceToDevice, ctx->stream));
            RFXP_HIP(ctx, hipMemcpyAsync(nv.p, ctx->sa_v.p, 4 * ctx->sa_nnz, hipMemcpyDeviceToDevice, ctx->stream));
            RFXP_HIP(ctx, hipStreamSynchronize(ctx->stream));
        }
        std::swap(ctx->sa_i, ni);
        std::swap(ctx->sa_j, nj);
        std::swap(ctx->sa_v, nv);
        ni.release();
        nj.release();
        nv.release();
    }
    hipLaunchKernelGGL(k_sa_rowemit, dim3((unsigned)nr), dim3(SA_THREADS), 0, ctx->stream, s, r0, ctx->sa_cnt.p,
                       ctx->sa_i.p, ctx->sa_j.p, ctx->sa_v.p);
    if (int rc = check_launch(ctx, "k_sa_rowemit")) return rc;
    ctx->sa_nnz = need;
    return RFXP_OK;
}

static int symacc_add(rfxp_ctx* ctx, SymSrc s) {
    const int64_t N = ctx->sa_N;
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    const bool host = !is_device_pointer(s.p);
    const bool packed = s.kind != SRC_DENSE;
    if (!ctx->sa_dense) RFXP_HIP(ctx, ctx->sa_cnt.ensure((size_t)N + 1));
    ctx->sa_csr_ok = false;
    if (host) {
        // one staging buffer for every band, sized before the first, so that
        // an add never frees and reallocates it (hipFree synchronises the
        // whole device) between bands.  A band is at most SA_STAGE_BYTES or
        // one row (the first row is the longest; NF4 adds a byte for a band
        // that starts at an odd entry).
        const int64_t total = src_bytes(s.kind, N, 0, packed ? sa_entries(N) : N);
        const int64_t row0 = src_bytes(s.kind, N, 0, packed ? N : 1) + 1;
        const int64_t cap = std::min(total, std::max(SA_STAGE_BYTES, row0));
        RFXP_HIP(ctx, ctx->sa_stage.ensure((size_t)(cap + 7) / 8));
    }
    int64_t r0 = 0;
    while (r0 < N) {
        // band of rows [r0, r1): everything for a device input, else at most
        // SA_STAGE_BYTES of the source (at least one row)
        int64_t r1 = N;
        SymSrc band = s;
        if (host) {
            const int64_t e0 = packed ? tri_idx(N, r0, r0) : r0;
            const int64_t b0 = packed && s.kind == SRC_NF4 ? e0 & ~1LL : e0;
            auto bytes_to = [&](int64_t r) { return src_bytes(s.kind, N, b0, packed ? tri_idx(N, r, r) : r); };
            if (bytes_to(N) > SA_STAGE_BYTES) {  // the largest r1 whose band fits, at least r0 + 1
                r1 = r0 + 1;
                for (int64_t step = int64_t(1) << 40; step > 0; step >>= 1)
                    if (r1 + step <= N && bytes_to(r1 + step) <= SA_STAGE_BYTES) r1 += step;
            }
            const int64_t nbytes = bytes_to(r1);
            const int64_t off = src_bytes(s.kind, N, 0, b0);
            if ((size_t)nbytes > 8 * ctx->sa_stage.n)
                return set_error(ctx, RFXP_ERR_INVALID, "rfxp_symacc: staging band larger than its buffer");
            RFXP_HIP(ctx, hipMemcpyAsync(ctx->sa_stage.p, (const unsigned char*)s.p + off, (size_t)nbytes,
                                         hipMemcpyHostToDevice, ctx->stream));
            band.p = ctx->sa_stage.p;
            band.base = b0;
        }
        if (ctx->sa_dense) {
            hipLaunchKernelGGL(k_sa_tri_add, dim3((unsigned)(r1 - r0)), dim3(SA_THREADS), 0, ctx->stream, band, r0,
                               ctx->sa_tri.p);
            if (int rc = check_launch(ctx, "k_sa_tri_add")) return rc;
        } else if (int rc = symacc_add_rows_sparse(ctx, band, r0, r1)) {
            return rc;
        }
        r0 = r1;
    }
    // the input (and the staging band) may be reused once this returns
    RFXP_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return RFXP_OK;
}

}  // namespace rfxp

extern "C" int rfxp_symacc_reset(rfxp_ctx* ctx, int64_t N) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (N < 1 || N > 0x7ffffffeLL) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_symacc_reset: need 1 <= N < 2^31 - 1");
    ctx->sa_N = N;
    ctx->sa_nnz = 0;
    ctx->sa_csr_ok = false;
    ctx->sa_dense = false;
    // nothing of a previous accumulation is kept beyond what this N allows
    ctx->sa_tri.release();
    ctx->sa_stage.release();
    if (ctx->sa_i.n > (size_t)sa_list_limit(N)) {
        ctx->sa_i.release();
        ctx->sa_j.release();
        ctx->sa_v.release();
        ctx->sa_col.release();
        ctx->sa_val.release();
    }
    if (ctx->sa_cnt.n > (size_t)N + 1) ctx->sa_cnt.release();
    if (ctx->sa_rowptr.n > (size_t)N + 1) ctx->sa_rowptr.release();
    if (ctx->sa_deg.n > (size_t)N + 1) ctx->sa_deg.release();
    return RFXP_OK;
}

extern "C" int64_t rfxp_symacc_nnz(rfxp_ctx* ctx) { return ctx ? ctx->sa_nnz : -1; }

extern "C" int64_t rfxp_symacc_device_bytes(rfxp_ctx* ctx) {
    if (!ctx) return -1;
    return (int64_t)(4 * (ctx->sa_i.n + ctx->sa_j.n + ctx->sa_col.n) + 4 * (ctx->sa_v.n + ctx->sa_val.n) +
                     8 * (ctx->sa_cnt.n + ctx->sa_rowptr.n + ctx->sa_deg.n + ctx->sa_tri.n + ctx->sa_stage.n));
}

extern "C" int rfxp_symacc_add_upper(rfxp_ctx* ctx, int fmt, const void* tri, float scale, float zp) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (ctx->sa_N < 1) return set_error(ctx, RFXP_ERR_STATE, "rfxp_symacc_add_upper: no accumulator (rfxp_symacc_reset)");
    if (!tri) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_symacc_add_upper: tri is NULL");
    SymSrc s{tri, 0, scale, zp, ctx->sa_N, 0};
    switch (fmt) {
        case RFXP_FMT_F16: s.kind = SRC_F16; break;
        case RFXP_FMT_F32: s.kind = SRC_F32; break;
        case RFXP_FMT_I8:
            if (!std::isfinite(scale) || !std::isfinite(zp))
                return set_error(ctx, RFXP_ERR_INVALID, "rfxp_symacc_add_upper: scale / zp must be finite");
            s.kind = SRC_I8;
            break;
        case RFXP_FMT_NF4: s.kind = SRC_NF4; break;
        default: return set_error(ctx, RFXP_ERR_INVALID, "rfxp_symacc_add_upper: format must be F16, F32, I8 or NF4");
    }
    return symacc_add(ctx, s);
}

extern "C" int rfxp_symacc_add_dense(rfxp_ctx* ctx, const double* full) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (ctx->sa_N < 1) return set_error(ctx, RFXP_ERR_STATE, "rfxp_symacc_add_dense: no accumulator (rfxp_symacc_reset)");
    if (!full) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_symacc_add_dense: full is NULL");
    SymSrc s{full, SRC_DENSE, 1.0f, 0.0f, ctx->sa_N, 0};
    return symacc_add(ctx, s);
}

namespace rfxp {

static int symacc_csr(rfxp_ctx* ctx) {
    if (ctx->sa_csr_ok || ctx->sa_dense) return RFXP_OK;
    const int64_t N = ctx->sa_N, nnz = ctx->sa_nnz;
    RFXP_HIP(ctx, ctx->sa_deg.ensure((size_t)N + 1));
    RFXP_HIP(ctx, ctx->sa_rowptr.ensure((size_t)N + 1));
    fill_u32(ctx, (uint32_t*)ctx->sa_deg.p, 2 * (N + 1), 0u);
    if (nnz > 0) {
        hipLaunchKernelGGL(k_sa_degree, dim3(gsblk(nnz)), dim3(256), 0, ctx->stream, ctx->sa_i.p, ctx->sa_j.p, nnz,
                           ctx->sa_deg.p);
        if (int rc = check_launch(ctx, "k_sa_degree")) return rc;
    }
    std::vector<unsigned long long> deg((size_t)N);
    RFXP_HIP(ctx, hipMemcpyAsync(deg.data(), ctx->sa_deg.p, 8 * N, hipMemcpyDeviceToHost, ctx->stream));
    RFXP_HIP(ctx, hipStreamSynchronize(ctx->stream));
    std::vector<int64_t> rp((size_t)N + 1);
    rp[0] = 0;
    for (int64_t i = 0; i < N; ++i) rp[i + 1] = rp[i] + (int64_t)deg[i];
    const int64_t tot = rp[N];
    RFXP_HIP(ctx, ctx->sa_col.ensure((size_t)tot));
    RFXP_HIP(ctx, ctx->sa_val.ensure((size_t)tot));
    RFXP_HIP(ctx, hipMemcpyAsync(ctx->sa_rowptr.p, rp.data(), 8 * (N + 1), hipMemcpyHostToDevice, ctx->stream));
    RFXP_HIP(ctx, hipMemcpyAsync(ctx->sa_deg.p, rp.data(), 8 * N, hipMemcpyHostToDevice, ctx->stream));  // cursors
    if (nnz > 0) {
        hipLaunchKernelGGL(k_sa_place, dim3(gsblk(nnz)), dim3(256), 0, ctx->stream, ctx->sa_i.p, ctx->sa_j.p, ctx->sa_v.p,
                           nnz, ctx->sa_deg.p, ctx->sa_col.p, ctx->sa_val.p);
        if (int rc = check_launch(ctx, "k_sa_place")) return rc;
    }
    RFXP_HIP(ctx, hipStreamSynchronize(ctx->stream));
    ctx->sa_csr_ok = true;
    return RFXP_OK;
}

static int symacc_spmm(rfxp_ctx* ctx, const double* X, int32_t b, double* Y) {
    const int64_t N = ctx->sa_N;
    if (ctx->sa_dense) {
        const dim3 grid((unsigned)((N + TS_T - 1) / TS_T), (unsigned)((b + TS_T - 1) / TS_T));
        hipLaunchKernelGGL(k_sa_tri_spmm, grid, dim3(256), 0, ctx->stream, ctx->sa_tri.p, X, N, b, Y);
        return check_launch(ctx, "k_sa_tri_spmm");
    }
    hipLaunchKernelGGL(k_sa_spmm, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, ctx->stream, ctx->sa_rowptr.p,
                       ctx->sa_col.p, ctx->sa_val.p, X, N, b, Y);
    return check_launch(ctx, "k_sa_spmm");
}

}  // namespace rfxp

extern "C" int rfxp_symacc_apply(rfxp_ctx* ctx, const double* X, int32_t b, double* Y) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (ctx->sa_N < 1) return set_error(ctx, RFXP_ERR_STATE, "rfxp_symacc_apply: no accumulator");
    if (b < 1 || !X || !Y || !is_device_pointer(X) || !is_device_pointer(Y))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_symacc_apply: need b >= 1 and device X, Y");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    if (int rc = symacc_csr(ctx)) return rc;
    return symacc_spmm(ctx, X, b, Y);
}

extern "C" int rfxp_symacc_factor(rfxp_ctx* ctx, int32_t rank, int32_t iters, uint64_t seed, double* A, double* evals) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (ctx->sa_N < 1) return set_error(ctx, RFXP_ERR_STATE, "rfxp_symacc_factor: no accumulator");
    const int64_t N = ctx->sa_N;
    if (rank < 1 || rank > 4096 || rank > N || iters < 0 || !A || !is_device_pointer(A))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_symacc_factor: need 1 <= rank <= min(N, 4096), iters >= 0, device A");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    if (int rc = symacc_csr(ctx)) return rc;
    const int32_t b = (int32_t)std::min<int64_t>(N, 2 * (int64_t)rank + 16);
    RFXP_HIP(ctx, ctx->sa_x.ensure((size_t)(N * b)));
    RFXP_HIP(ctx, ctx->sa_y.ensure((size_t)(N * b)));
    RFXP_HIP(ctx, ctx->sa_z.ensure((size_t)(N * b)));
    double *X = ctx->sa_x.p, *Y = ctx->sa_y.p, *Z = ctx->sa_z.p;
    hipLaunchKernelGGL(k_randn, dim3(gsblk(N * b)), dim3(256), 0, ctx->stream, X, N * b, seed);
    if (int rc = check_launch(ctx, "k_randn")) return rc;
    if (int rc = orth(ctx, ctx->sa_part, ctx->sa_g, ctx->sa_w, X, Y, Z, b, N)) return rc;  // Q in Y
    // Ritz values and vectors of M on the current basis Q (in Y); X = M Q
    std::vector<double> H, w, U;
    auto ritz = [&]() -> int {
        if (int rc = symacc_spmm(ctx, Y, b, X)) return rc;
        if (int rc = gram(ctx, ctx->sa_part, ctx->sa_g, Y, b, X, b, nullptr, N, H)) return rc;
        for (int i = 0; i < b; ++i)
            for (int j = i + 1; j < b; ++j) {
                const double m = 0.5 * (H[(size_t)i * b + j] + H[(size_t)j * b + i]);
                H[(size_t)i * b + j] = H[(size_t)j * b + i] = m;
            }
        host_symeig(b, H, w, U);
        return RFXP_OK;
    };
    // The block converges to the eigenvalues of largest magnitude, which for
    // an indefinite M include negative ones; a block of about twice the rank
    // leaves room for them next to the r largest positive ones.
    for (int32_t it = 0; it < iters; ++it) {
        if (int rc = symacc_spmm(ctx, Y, b, X)) return rc;                                   // X = M Q
        if (int rc = orth(ctx, ctx->sa_part, ctx->sa_g, ctx->sa_w, X, Y, Z, b, N)) return rc;  // Q = orth(X)
    }
    if (int rc = ritz()) return rc;
    std::vector<double> W((size_t)b * rank, 0.0);
    for (int32_t c = 0; c < rank; ++c) {
        const double lam = c < b ? w[c] : 0.0;
        if (evals) evals[c] = lam;
        if (!(lam > 0.0)) continue;
        const double f = sqrt(lam);
        for (int32_t k = 0; k < b; ++k) W[(size_t)k * rank + c] = U[(size_t)k * b + c] * f;
    }
    return gemm_nn(ctx, ctx->sa_w, Y, b, W, rank, N, A, true);
}

extern "C" int rfxp_factor_reconstruct(rfxp_ctx* ctx, const double* A, const double* B, int64_t N, int32_t rank,
                                       const int32_t* oob_counts, double* out) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (N < 1 || rank < 0 || (rank > 0 && (!A || !B)) || !out)
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_factor_reconstruct: bad arguments");
    if (N > 3037000499LL) return set_error(ctx, RFXP_ERR_UNSUPPORTED, "rfxp_factor_reconstruct: N x N too large");
    if ((rank > 0 && (!is_device_pointer(A) || !is_device_pointer(B))) || !is_device_pointer(out))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_factor_reconstruct: A, B and out must be device pointers");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    const int32_t* sdev = nullptr;
    const double* wdev = nullptr;
    if (oob_counts) {  // host counts: 1/s on the device
        std::vector<double> winv((size_t)N);
        for (int64_t i = 0; i < N; ++i) winv[i] = oob_counts[i] > 0 ? 1.0 / (double)oob_counts[i] : 1.0;
        RFXP_HIP(ctx, ctx->sa_wv.ensure((size_t)N));
        RFXP_HIP(ctx, ctx->sa_sv.ensure((size_t)N));
        RFXP_HIP(ctx, hipMemcpyAsync(ctx->sa_wv.p, winv.data(), 8 * N, hipMemcpyHostToDevice, ctx->stream));
        RFXP_HIP(ctx, hipMemcpyAsync(ctx->sa_sv.p, oob_counts, 4 * N, hipMemcpyHostToDevice, ctx->stream));
        RFXP_HIP(ctx, hipStreamSynchronize(ctx->stream));
        sdev = ctx->sa_sv.p;
        wdev = ctx->sa_wv.p;
    }
    const int64_t nn = N * N;
    hipLaunchKernelGGL(k_reconstruct, dim3(gsblk(nn)), dim3(256), 0, ctx->stream, A, B, N, rank, wdev, sdev, out);
    return check_launch(ctx, "k_reconstruct");
}

namespace rfxp {

// y = C v for the MDS operator C = -1/2 J (D o D) J, D = 1 - Pt/m, through
// the factor (row-major Ar, N x r):
//   C = J (Pt/m - (Pt o Pt)/(2 m^2)) J,
//   Pt = P (no counts) or 1/2 (diag(w) P + P diag(w)) (RF-GAP counts),
//   (P o P) u = rowdot(Ar G_u, Ar),  G_u = Ar^T diag(u) Ar,
//   (Pt o Pt) u = 1/4 (w^2 o (P o P) u + 2 w o (P o P)(w o u) + (P o P)(w^2 o u)).
struct MdsOp {
    rfxp_ctx* ctx;
    const double* Ar;
    int64_t N;
    int32_t r;
    const double* w;   // device, or NULL
    const double* w2;  // device w^2, or NULL
    double m;
    DevBuf<double> part, gdev, wdev, t1, t2, u, v, z, q, h3, col;  // col: the column of 1/N
};

// V <- J V (column means removed), the means from a Gram with the 1/N column.
static int mds_center(MdsOp& op, double* V, int32_t c) {
    const int64_t N = op.N;
    std::vector<double> mean;
    if (int rc = gram(op.ctx, op.part, op.gdev, op.col.p, 1, V, c, nullptr, N, mean)) return rc;
    RFXP_HIP(op.ctx, op.wdev.ensure((size_t)c));
    RFXP_HIP(op.ctx, hipMemcpyAsync(op.wdev.p, mean.data(), 8 * c, hipMemcpyHostToDevice, op.ctx->stream));
    hipLaunchKernelGGL(k_center_cols, dim3(nblk(N * c)), dim3(256), 0, op.ctx->stream, V, N, c, op.wdev.p);
    if (int rc = check_launch(op.ctx, "k_center_cols")) return rc;
    RFXP_HIP(op.ctx, hipStreamSynchronize(op.ctx->stream));
    return RFXP_OK;
}

// out[:, k] = (P o P) u for the column vector u (device, N), scaled rows by sw (or NULL)
static int mds_hadamard(MdsOp& op, const double* u, double* out, int32_t ldo, int32_t k) {
    std::vector<double> G;
    if (int rc = gram(op.ctx, op.part, op.gdev, op.Ar, op.r, op.Ar, op.r, u, op.N, G)) return rc;
    if (int rc = gemm_nn(op.ctx, op.wdev, op.Ar, op.r, G, op.r, op.N, op.z.p, false)) return rc;
    hipLaunchKernelGGL(k_rowdot, dim3(nblk(op.N)), dim3(256), 0, op.ctx->stream, op.z.p, op.Ar, op.N, op.r, out, ldo, k);
    return check_launch(op.ctx, "k_rowdot");
}

static int mds_apply(MdsOp& op, const double* Vin, int32_t c, double* Y) {
    const int64_t N = op.N;
    rfxp_ctx* ctx = op.ctx;
    RFXP_HIP(ctx, op.u.ensure((size_t)(N * c)));
    RFXP_HIP(ctx, op.t1.ensure((size_t)(N * c)));
    RFXP_HIP(ctx, op.t2.ensure((size_t)(N * c)));
    RFXP_HIP(ctx, op.z.ensure((size_t)(N * op.r)));
    RFXP_HIP(ctx, op.v.ensure((size_t)N));
    RFXP_HIP(ctx, op.q.ensure((size_t)N));
    RFXP_HIP(ctx, op.h3.ensure((size_t)(3 * N)));
    RFXP_HIP(ctx, hipMemcpyAsync(op.u.p, Vin, 8 * N * c, hipMemcpyDeviceToDevice, ctx->stream));
    if (int rc = mds_center(op, op.u.p, c)) return rc;  // U = J V
    // T1 = Pt U
    std::vector<double> S;
    if (int rc = gram(ctx, op.part, op.gdev, op.Ar, op.r, op.u.p, c, nullptr, N, S)) return rc;  // Ar^T U
    if (int rc = gemm_nn(ctx, op.wdev, op.Ar, op.r, S, c, N, op.t1.p, false)) return rc;     // P U
    if (op.w) {
        // 1/2 (w o P U + P (w o U))
        RFXP_HIP(ctx, hipMemcpyAsync(op.t2.p, op.u.p, 8 * N * c, hipMemcpyDeviceToDevice, ctx->stream));
        hipLaunchKernelGGL(k_scale_rows, dim3(nblk(N * c)), dim3(256), 0, ctx->stream, op.t2.p, op.w, N, c);
        std::vector<double> S2;
        if (int rc = gram(ctx, op.part, op.gdev, op.Ar, op.r, op.t2.p, c, nullptr, N, S2)) return rc;
        hipLaunchKernelGGL(k_scale_rows, dim3(nblk(N * c)), dim3(256), 0, ctx->stream, op.t1.p, op.w, N, c);
        if (int rc = gemm_nn(ctx, op.wdev, op.Ar, op.r, S2, c, N, op.t2.p, false)) return rc;
        hipLaunchKernelGGL(k_axpby, dim3(nblk(N * c)), dim3(256), 0, ctx->stream, op.t1.p, op.t2.p, 0.5, 0.5, N * c,
                           op.t1.p);
        if (int rc = check_launch(ctx, "mds rf-gap terms")) return rc;
    }
    // T2 = (Pt o Pt) U, column by column
    for (int32_t k = 0; k < c; ++k) {
        hipLaunchKernelGGL(k_get_col, dim3(nblk(N)), dim3(256), 0, ctx->stream, op.u.p, N, c, k, op.v.p);
        if (!op.w) {
            if (int rc = mds_hadamard(op, op.v.p, op.t2.p, c, k)) return rc;
            continue;
        }
        // three Hadamard products h0 = (P o P) u, h1 = (P o P)(w o u),
        // h2 = (P o P)(w^2 o u), combined as 1/4 (w^2 h0 + 2 w h1 + h2)
        for (int vnt = 0; vnt < 3; ++vnt) {
            RFXP_HIP(ctx, hipMemcpyAsync(op.q.p, op.v.p, 8 * N, hipMemcpyDeviceToDevice, ctx->stream));
            if (vnt == 1) hipLaunchKernelGGL(k_scale_rows, dim3(nblk(N)), dim3(256), 0, ctx->stream, op.q.p, op.w, N, 1);
            if (vnt == 2) hipLaunchKernelGGL(k_scale_rows, dim3(nblk(N)), dim3(256), 0, ctx->stream, op.q.p, op.w2, N, 1);
            if (int rc = mds_hadamard(op, op.q.p, op.h3.p, 3, vnt)) return rc;
        }
        hipLaunchKernelGGL(k_rfgap_combine, dim3(nblk(N)), dim3(256), 0, ctx->stream, op.h3.p, op.w, op.w2, N, op.t2.p, c,
                           k);
        if (int rc = check_launch(ctx, "k_rfgap_combine")) return rc;
    }
    // Y = J (T1/m - T2/(2 m^2))
    hipLaunchKernelGGL(k_axpby, dim3(nblk(N * c)), dim3(256), 0, ctx->stream, op.t1.p, op.t2.p, 1.0 / op.m,
                       -1.0 / (2.0 * op.m * op.m), N * c, Y);
    if (int rc = check_launch(ctx, "k_axpby")) return rc;
    return mds_center(op, Y, c);
}

}  // namespace rfxp

extern "C" int rfxp_factor_mds(rfxp_ctx* ctx, const double* A, int64_t N, int32_t rank, int32_t k,
                               const int32_t* oob_counts, int32_t iters, double* coords, double* evals) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (N < 2 || rank < 1 || k < 1 || k > N || iters < 1 || !A || !coords || !is_device_pointer(A))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_factor_mds: need N >= 2, rank >= 1, 1 <= k <= N, iters >= 1, device A");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    MdsOp op{};
    op.ctx = ctx;
    op.N = N;
    op.r = rank;
    DevBuf<double> ar, wd, w2d, X, Y, Z, diag;
    auto cleanup = [&]() {
        for (auto* d : {&ar, &wd, &w2d, &X, &Y, &Z, &diag, &op.part, &op.gdev, &op.wdev, &op.t1, &op.t2, &op.u, &op.v,
                        &op.z, &op.q, &op.h3, &op.col})
            d->release();
    };
    int rc = RFXP_OK;
    do {
        if (ar.ensure((size_t)(N * rank)) != hipSuccess || diag.ensure((size_t)N) != hipSuccess ||
            op.col.ensure((size_t)N) != hipSuccess) {
            rc = set_error(ctx, RFXP_ERR_NOMEM, "rfxp_factor_mds: out of device memory");
            break;
        }
        {
            const std::vector<double> ones((size_t)N, 1.0 / (double)N);
            if (hipMemcpyAsync(op.col.p, ones.data(), 8 * N, hipMemcpyHostToDevice, ctx->stream) != hipSuccess ||
                hipStreamSynchronize(ctx->stream) != hipSuccess) {
                rc = set_error(ctx, RFXP_ERR_HIP, "rfxp_factor_mds: copy failed");
                break;
            }
        }
        hipLaunchKernelGGL(k_to_rowmajor, dim3(nblk(N * rank)), dim3(256), 0, ctx->stream, A, N, rank, ar.p);
        hipLaunchKernelGGL(k_rownorm2, dim3(nblk(N)), dim3(256), 0, ctx->stream, ar.p, N, rank, diag.p);
        if ((rc = check_launch(ctx, "mds setup"))) break;
        op.Ar = ar.p;
        std::vector<double> d((size_t)N), winv;
        if (hipMemcpyAsync(d.data(), diag.p, 8 * N, hipMemcpyDeviceToHost, ctx->stream) != hipSuccess ||
            hipStreamSynchronize(ctx->stream) != hipSuccess) {
            rc = set_error(ctx, RFXP_ERR_HIP, "rfxp_factor_mds: copy failed");
            break;
        }
        if (oob_counts) {
            winv.resize((size_t)N);
            std::vector<double> w2((size_t)N);
            for (int64_t i = 0; i < N; ++i) {
                winv[i] = oob_counts[i] > 0 ? 1.0 / (double)oob_counts[i] : 1.0;
                w2[i] = winv[i] * winv[i];
                d[i] *= winv[i];  // Pt_ii = w_i P_ii
            }
            if (wd.ensure((size_t)N) != hipSuccess || w2d.ensure((size_t)N) != hipSuccess) {
                rc = set_error(ctx, RFXP_ERR_NOMEM, "rfxp_factor_mds: out of device memory");
                break;
            }
            (void)hipMemcpyAsync(wd.p, winv.data(), 8 * N, hipMemcpyHostToDevice, ctx->stream);
            (void)hipMemcpyAsync(w2d.p, w2.data(), 8 * N, hipMemcpyHostToDevice, ctx->stream);
            (void)hipStreamSynchronize(ctx->stream);
            op.w = wd.p;
            op.w2 = w2d.p;
        }
        double m = 0.0;
        for (int64_t i = 0; i < N; ++i) m = std::max(m, d[i]);
        op.m = m < 1e-10 ? 1.0 : m;
        // subspace iteration on C with Rayleigh-Ritz, block k + p
        const int32_t c = (int32_t)std::min<int64_t>(N, (int64_t)k + 4);
        if (X.ensure((size_t)(N * c)) != hipSuccess || Y.ensure((size_t)(N * c)) != hipSuccess ||
            Z.ensure((size_t)(N * c)) != hipSuccess) {
            rc = set_error(ctx, RFXP_ERR_NOMEM, "rfxp_factor_mds: out of device memory");
            break;
        }
        hipLaunchKernelGGL(k_randn, dim3(nblk(N * c)), dim3(256), 0, ctx->stream, X.p, N * c, 12345ull);
        if ((rc = orth(ctx, op.part, op.gdev, op.wdev, X.p, Y.p, Z.p, c, N))) break;  // Q in Y
        std::vector<double> prev, H, w, U;
        for (int32_t it = 0; it < iters; ++it) {
            if ((rc = mds_apply(op, Y.p, c, X.p))) break;                     // X = C Q
            if ((rc = gram(ctx, op.part, op.gdev, Y.p, c, X.p, c, nullptr, N, H))) break;  // Q^T C Q
            for (int i = 0; i < c; ++i)
                for (int j = i + 1; j < c; ++j) {
                    const double mm = 0.5 * (H[(size_t)i * c + j] + H[(size_t)j * c + i]);
                    H[(size_t)i * c + j] = H[(size_t)j * c + i] = mm;
                }
            std::vector<double> Hc = H;
            host_symeig(c, Hc, w, U);
            bool done = !prev.empty();
            for (int32_t q = 0; q < k && done; ++q)
                done = fabs(w[q] - prev[q]) <= 1e-12 * std::max(fabs(w[0]), 1e-300);
            prev = w;
            if (done || it + 1 == iters) {
                // Ritz vectors of the current basis: coords = (Q U)[:, q] sqrt|lambda_q|
                std::vector<double> W((size_t)c * k, 0.0);
                for (int32_t q = 0; q < k; ++q) {
                    const double f = sqrt(fabs(w[q]));
                    for (int32_t j = 0; j < c; ++j) W[(size_t)j * k + q] = U[(size_t)j * c + q] * f;
                    if (evals) evals[q] = w[q];
                }
                if ((rc = gemm_nn(ctx, op.wdev, Y.p, c, W, k, N, Z.p, false))) break;
                if (hipMemcpyAsync(coords, Z.p, 8 * N * k, hipMemcpyDeviceToHost, ctx->stream) != hipSuccess ||
                    hipStreamSynchronize(ctx->stream) != hipSuccess)
                    rc = set_error(ctx, RFXP_ERR_HIP, "rfxp_factor_mds: copy failed");
                break;
            }
            if ((rc = orth(ctx, op.part, op.gdev, op.wdev, X.p, Y.p, Z.p, c, N))) break;
        }
    } while (false);
    cleanup();
    return rc;
}

// ---------------------------------------------------------------------------
// factor storage formats (cuda/rf_proximity_lowrank.cu:242-400)
// ---------------------------------------------------------------------------

namespace rfxp {

__global__ void k_fq_f16(const double* A, int64_t n, uint16_t* q) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e < n) q[e] = f32_to_f16_bits((float)A[e]);
}
__global__ void k_fq_i8(const double* A, int64_t n, const float* sz, int8_t* q) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e < n) q[e] = q_i8((float)A[e], sz[0], sz[1]);
}
__global__ void k_fq_nf4(const double* A, int64_t n, uint8_t* q) {
    const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t e = 2 * p;
    if (e >= n) return;
    const uint32_t a = q_nf4((float)A[e]) & 0xfu;
    const uint32_t b = e + 1 < n ? (q_nf4((float)A[e + 1]) & 0xfu) : 0u;
    q[p] = (uint8_t)(a | (b << 4));
}
__global__ void k_fd_f16(const uint16_t* q, int64_t n, double* A) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e < n) A[e] = (double)half_bits_to_float(q[e]);
}
__global__ void k_fd_i8(const int8_t* q, int64_t n, const float* sz, double* A) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e < n) A[e] = (double)(((float)q[e] - sz[1]) * sz[0]);
}
__global__ void k_fd_nf4(const uint8_t* q, int64_t n, double* A) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n) return;
    const uint32_t v = (q[e >> 1] >> ((e & 1) * 4)) & 0xfu;
    A[e] = (double)(v <= 7u ? (float)v / 7.0f : -((float)(v - 8u)) / 7.0f);
}

}  // namespace rfxp

extern "C" int64_t rfxp_factor_quantized_bytes(int level, int64_t count) {
    if (count < 0) return -1;
    switch (level) {
        case RFXP_FMT_F32:
        case RFXP_FMT_F16: return 2 * count;
        case RFXP_FMT_I8: return count;
        case RFXP_FMT_NF4: return (count + 1) / 2;
        default: return -1;
    }
}

extern "C" int rfxp_factor_quantize(rfxp_ctx* ctx, int level, const double* A, int64_t count, const float* scale_zp,
                                    void* q) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (count < 0 || !A || !q || !is_device_pointer(A) || !is_device_pointer(q) ||
        (level == RFXP_FMT_I8 && (!scale_zp || !is_device_pointer(scale_zp))))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_factor_quantize: bad arguments");
    if (count == 0) return RFXP_OK;
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    switch (level) {
        case RFXP_FMT_F32:
        case RFXP_FMT_F16:
            hipLaunchKernelGGL(k_fq_f16, dim3(nblk(count)), dim3(256), 0, ctx->stream, A, count, (uint16_t*)q);
            break;
        case RFXP_FMT_I8:
            hipLaunchKernelGGL(k_fq_i8, dim3(nblk(count)), dim3(256), 0, ctx->stream, A, count, scale_zp, (int8_t*)q);
            break;
        case RFXP_FMT_NF4:
            hipLaunchKernelGGL(k_fq_nf4, dim3(nblk((count + 1) / 2)), dim3(256), 0, ctx->stream, A, count, (uint8_t*)q);
            break;
        default: return set_error(ctx, RFXP_ERR_INVALID, "rfxp_factor_quantize: level must be F32, F16, I8 or NF4");
    }
    return check_launch(ctx, "factor quantize");
}

extern "C" int rfxp_factor_dequantize(rfxp_ctx* ctx, int level, const void* q, int64_t count, const float* scale_zp,
                                      double* A) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (count < 0 || !A || !q || !is_device_pointer(A) || !is_device_pointer(q) ||
        (level == RFXP_FMT_I8 && (!scale_zp || !is_device_pointer(scale_zp))))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_factor_dequantize: bad arguments");
    if (count == 0) return RFXP_OK;
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    switch (level) {
        case RFXP_FMT_F32:
        case RFXP_FMT_F16:
            hipLaunchKernelGGL(k_fd_f16, dim3(nblk(count)), dim3(256), 0, ctx->stream, (const uint16_t*)q, count, A);
            break;
        case RFXP_FMT_I8:
            hipLaunchKernelGGL(k_fd_i8, dim3(nblk(count)), dim3(256), 0, ctx->stream, (const int8_t*)q, count, scale_zp, A);
            break;
        case RFXP_FMT_NF4:
            hipLaunchKernelGGL(k_fd_nf4, dim3(nblk(count)), dim3(256), 0, ctx->stream, (const uint8_t*)q, count, A);
            break;
        default: return set_error(ctx, RFXP_ERR_INVALID, "rfxp_factor_dequantize: level must be F32, F16, I8 or NF4");
    }
    return check_launch(ctx, "factor dequantize");
}
