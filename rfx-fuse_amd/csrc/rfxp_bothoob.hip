// The "both OOB" proximity: co-occurrence over the trees in which both
// samples are out-of-bag, normalised by the number of such trees (R
// randomForest's oob.prox).  The reference does not implement it (its rule is
// OOB x in-bag normalised by nout, src/rf_proximity.cpp:179-230 and
// src/rf_finishprox.cpp:47-73); it is the normalisation that the mid-size
// benchmark configuration's description names.  For i != j
//     num_ij = #{t : oob_i(t), oob_j(t), leaf_i(t) == leaf_j(t), label valid}
//     den_ij = #{t : oob_i(t), oob_j(t)}
//     P_ij   = den_ij > 0 ? (float)num_ij / (float)den_ij : 0,   P_ii = 1.
//
// den is a dense N x N x T binary contraction, so this is a tiled kernel
// rather than the bucketed triangle: one workgroup per 64 x 64 tile of the
// upper triangle, 256 threads with 4 x 4 pairs each.  Per chunk of 32 trees
// the tile's 64 row and 64 column samples are staged in LDS as
//     key = (oob && label valid) ? label : -1 - sample
// (so equal keys mean "both OOB, same valid leaf", and two distinct samples
// that are not both OOB never match), plus one 32-tree OOB word per sample;
// num takes one compare per pair and tree, den one AND + popcount per pair
// and chunk.  Cost O(N^2 T / 2): meant for the sizes the both-OOB matrix is
// asked for (a dense N x N result).
#include "rfxp_device.hpp"
#include "rfxp_internal.hpp"

namespace rfxp {

constexpr int BO_TILE = 64;
constexpr int BO_THREADS = 256;
constexpr int BO_CHUNK = 32;  // trees per staging round (one OOB word)

struct BothOobArgs {
    const int32_t* leaf;
    int64_t si, st;
    const uint32_t* oob;  // bit (i & 31) of oob[t*old + (i >> 5)]
    int64_t old;
    int64_t N;
    int32_t T, L;
    int64_t r0, r1;       // row band
    int64_t tile_r0;      // first tile row of the band (r0 / 64)
    int64_t e_base;       // idx(r0, r0)
    int fmt;              // F32 or U16
    void* out;
};

__global__ __launch_bounds__(BO_THREADS) void k_both_oob(BothOobArgs a) {
    __shared__ int32_t kr[BO_CHUNK][BO_TILE];  // row keys [tree][sample]
    __shared__ int32_t kc[BO_CHUNK][BO_TILE];  // column keys
    __shared__ uint32_t wr[BO_TILE], wc[BO_TILE];  // 32-tree OOB words
    const int64_t I = a.tile_r0 + blockIdx.y, J = blockIdx.x;
    if (J < I) return;  // lower-triangle tiles: nothing to do (uniform)
    const int64_t i0 = I * BO_TILE, j0 = J * BO_TILE;
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    uint32_t num[4][4], den[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int v = 0; v < 4; ++v) num[u][v] = den[u][v] = 0u;

    for (int32_t t0 = 0; t0 < a.T; t0 += BO_CHUNK) {
        if (threadIdx.x < BO_TILE) {
            wr[threadIdx.x] = 0u;
            wc[threadIdx.x] = 0u;
        }
        __syncthreads();
        // stage keys and OOB words: element e = (tree tt, sample s) of each side
        for (int e = threadIdx.x; e < 2 * BO_CHUNK * BO_TILE; e += BO_THREADS) {
            const int side = e / (BO_CHUNK * BO_TILE);
            const int r = e % (BO_CHUNK * BO_TILE);
            const int tt = r / BO_TILE, s = r % BO_TILE;
            const int64_t i = (side ? j0 : i0) + s;
            const int32_t t = t0 + tt;
            int32_t key = -1 - (int32_t)s - (side ? 2 * BO_TILE : 0);  // never equal across samples or sides
            bool o = false;
            if (i < a.N && t < a.T) {
                o = ((a.oob[(int64_t)t * a.old + (i >> 5)] >> (i & 31)) & 1u) != 0u;
                const int32_t l = a.leaf[i * a.si + (int64_t)t * a.st];
                if (o && l >= 0 && l < a.L) key = l;
            }
            if (side) kc[tt][s] = key;
            else kr[tt][s] = key;
            if (o) atomicOr(side ? &wc[s] : &wr[s], 1u << tt);
        }
        __syncthreads();
#pragma unroll 4
        for (int tt = 0; tt < BO_CHUNK; ++tt) {
            const int4 x = *(const int4*)&kr[tt][ty * 4];
            const int4 y = *(const int4*)&kc[tt][tx * 4];
            const int32_t xr[4] = {x.x, x.y, x.z, x.w}, yc[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int v = 0; v < 4; ++v) num[u][v] += xr[u] == yc[v] ? 1u : 0u;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int v = 0; v < 4; ++v) den[u][v] += (uint32_t)__popc(wr[ty * 4 + u] & wc[tx * 4 + v]);
        __syncthreads();
    }
    // store the tile's entries of the band's rows, j >= i
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int64_t i = i0 + ty * 4 + u;
        if (i < a.r0 || i >= a.r1) continue;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int64_t j = j0 + tx * 4 + v;
            if (j < i || j >= a.N) continue;
            const int64_t e = tri_idx(a.N, i, j) - a.e_base;
            if (a.fmt == U16) {
                ((uint16_t*)a.out)[e] = j == i ? (uint16_t)0 : (uint16_t)num[u][v];
            } else {
                const float p = j == i ? 1.0f : (den[u][v] ? (float)num[u][v] / (float)den[u][v] : 0.0f);
                ((float*)a.out)[e] = p;
            }
        }
    }
}

}  // namespace rfxp

using namespace rfxp;

extern "C" int rfxp_both_oob(rfxp_ctx* ctx, const int32_t* leaf, int64_t stride_i, int64_t stride_t,
                             const uint32_t* oob_words, int64_t oob_ld, int64_t N, int32_t T, int32_t nleaf,
                             int fmt, int64_t row_begin, int64_t row_end, void* out) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (N < 0 || T < 1 || T > 65535 || nleaf < 1)
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_both_oob: need N >= 0, 1 <= T <= 65535, nleaf >= 1");
    if (fmt != F32 && fmt != U16) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_both_oob: fmt must be F32 or U16");
    if (row_begin < 0 || row_end > N || row_begin > row_end)
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_both_oob: bad row range");
    if (row_begin == row_end) return RFXP_OK;
    if (oob_ld < (N + 31) / 32) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_both_oob: oob_ld < ceil(N/32)");
    if (!leaf || !oob_words || !out || !is_device_pointer(leaf) || !is_device_pointer(oob_words) ||
        !is_device_pointer(out))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_both_oob: pointers must be device pointers");
    const int64_t nJ = (N + BO_TILE - 1) / BO_TILE;
    const int64_t t_r0 = row_begin / BO_TILE, t_r1 = (row_end + BO_TILE - 1) / BO_TILE;
    // work-items per dimension within 32 bits, y within 65,535 workgroups
    if (nJ * BO_THREADS > 0xffffffffLL || t_r1 - t_r0 > 65535)
        return set_error(ctx, RFXP_ERR_UNSUPPORTED, "rfxp_both_oob: row band too large for one launch");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    BothOobArgs a{leaf, stride_i, stride_t, oob_words, oob_ld, N, T, nleaf, row_begin, row_end, t_r0,
                  tri_idx(N, row_begin, row_begin), fmt, out};
    {
        LaunchTimer tm(ctx, "both_oob");
        hipLaunchKernelGGL(k_both_oob, dim3((unsigned)nJ, (unsigned)(t_r1 - t_r0)), dim3(BO_THREADS), 0, ctx->stream,
                           a);
    }
    return check_launch(ctx, "k_both_oob launch");
}
