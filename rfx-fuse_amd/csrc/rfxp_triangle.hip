// Batched OOB co-occurrence proximity into the packed upper triangle.
//
// Reference path restated here (one batched pass instead of T per-tree
// calls):  src/rf_proximity.cpp:179-230 accumulates, per tree, +1 at
// (OOB n, in-bag kk) of the same terminal node; src/rf_finishprox.cpp:12-74
// symmetrises and normalises by nout.  Folding (n,kk) to (min,max) as
// cuda/rf_proximity_upper_triangle.cu:229-237 does gives, for i < j,
//     U_ij = #{t : leaf_i(t) == leaf_j(t) valid, oob_i(t) != oob_j(t)}.
//
// Data layout in HBM (built by rfxp_set_forest):
//   bkt_off [T][2L+1]  int32  per-tree offsets of bucket b = 2*leaf + oob
//   bkt_mem [T][N]     int32  sample ids grouped by bucket
//   rec     [N][T]     uint2  for sample i and tree t: (offset, length) of
//                             the bucket holding i's leaf with the other
//                             OOB bit -- exactly the j that pair with i
//   nout [N] int32, rinv [N] double (1/nout or 1)
//
// Triangle kernel: one workgroup per (row i, column segment [lo, hi)) item.
// It zeroes a byte counter per column in LDS, walks row i's T records,
// gathers the member ids of each opposite bucket (one wave-wide coalesced
// load per bucket, eight buckets in flight per wave) and bumps the LDS
// counter of every member j in the segment with j > i.  The epilogue turns
// the counters into the output format and streams the row segment to HBM
// with aligned 16-byte non-temporal stores.  Integer formats are
// table-driven: per row, codes for U < uc (those that do not depend on the
// column) sit in an 8-entry table applied four bytes at a time with
// v_perm_b32; other counts take the exact IEEE path.
#include <string.h>

#include <algorithm>
#include <cmath>
#include <string>
#include <vector>

#include "rfxp_device.hpp"
#include "rfxp_internal.hpp"

namespace rfxp {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int PACK_THREADS = 1024;
constexpr int TRI_THREADS = 512;
constexpr int TRI_WAVES = TRI_THREADS / 64;

struct LeafView {
    const int32_t* leaf;
    int64_t si, st;
    const uint32_t* oob;
    int64_t old;
    int64_t N;
    int32_t T;
    int32_t L;
};

// Bucket id of sample i in tree t, -1 when its label is not a valid leaf.
__device__ __forceinline__ int32_t bucket_of(const LeafView& v, int64_t i, int32_t t) {
    int32_t l = v.leaf[i * v.si + (int64_t)t * v.st];
    if (l < 0 || l >= v.L) return -1;
    uint32_t w = v.oob[(int64_t)t * v.old + (i >> 5)];
    return 2 * l + (int32_t)((w >> (i & 31)) & 1u);
}

// Exclusive scan of cnt[0..nb) in place (one workgroup), also written to
// off[0..nb] with off[nb] = total.  `part` is PACK_THREADS words of scratch.
template <class CntPtr>
__device__ void block_exclusive_scan(CntPtr cnt, int32_t nb, uint32_t* part, int32_t* off) {
    const int tid = threadIdx.x;
    const int32_t chunk = (nb + PACK_THREADS - 1) / PACK_THREADS;
    const int32_t b0 = tid * chunk;
    const int32_t b1 = min(nb, b0 + chunk);
    uint32_t s = 0;
    for (int32_t b = b0; b < b1; ++b) s += cnt[b];
    part[tid] = s;
    __syncthreads();
    for (int d = 1; d < PACK_THREADS; d <<= 1) {
        uint32_t v = tid >= d ? part[tid - d] : 0u;
        __syncthreads();
        part[tid] += v;
        __syncthreads();
    }
    uint32_t run = part[tid] - s;  // exclusive prefix of this thread's chunk
    for (int32_t b = b0; b < b1; ++b) {
        uint32_t c = cnt[b];
        cnt[b] = run;
        off[b] = (int32_t)run;
        run += c;
    }
    if (tid == PACK_THREADS - 1) off[nb] = (int32_t)part[tid];
    __syncthreads();
}

// One workgroup per tree: histogram of buckets in LDS, scan, then scatter of
// the sample ids through LDS cursors.  Used when 2L counters fit in LDS.
__global__ __launch_bounds__(PACK_THREADS) void k_bucket_lds(LeafView v, int32_t* bkt_off,
                                                            int32_t* bkt_mem) {
    extern __shared__ uint32_t sh[];
    const int32_t t = blockIdx.x;
    const int32_t nb = 2 * v.L;
    uint32_t* cnt = sh;
    uint32_t* part = sh + nb;
    for (int32_t b = threadIdx.x; b < nb; b += PACK_THREADS) cnt[b] = 0;
    __syncthreads();
    for (int64_t i = threadIdx.x; i < v.N; i += PACK_THREADS) {
        int32_t b = bucket_of(v, i, t);
        if (b >= 0) atomicAdd(&cnt[b], 1u);
    }
    __syncthreads();
    int32_t* off = bkt_off + (int64_t)t * (nb + 1);
    block_exclusive_scan(cnt, nb, part, off);
    int32_t* mem = bkt_mem + (int64_t)t * v.N;
    for (int64_t i = threadIdx.x; i < v.N; i += PACK_THREADS) {
        int32_t b = bucket_of(v, i, t);
        if (b >= 0) {
            uint32_t pos = atomicAdd(&cnt[b], 1u);
            mem[pos] = (int32_t)i;
        }
    }
}

// Same with the counters in global memory (large leaf counts).  cnt is a
// zeroed T x 2L scratch.
__global__ __launch_bounds__(PACK_THREADS) void k_bucket_global(LeafView v, uint32_t* cnt_all,
                                                               int32_t* bkt_off, int32_t* bkt_mem) {
    __shared__ uint32_t part[PACK_THREADS];
    const int32_t t = blockIdx.x;
    const int32_t nb = 2 * v.L;
    uint32_t* cnt = cnt_all + (int64_t)t * nb;
    for (int64_t i = threadIdx.x; i < v.N; i += PACK_THREADS) {
        int32_t b = bucket_of(v, i, t);
        if (b >= 0) atomicAdd(&cnt[b], 1u);
    }
    __syncthreads();
    __threadfence_block();
    int32_t* off = bkt_off + (int64_t)t * (nb + 1);
    block_exclusive_scan((volatile uint32_t*)cnt, nb, part, off);
    __threadfence_block();
    int32_t* mem = bkt_mem + (int64_t)t * v.N;
    for (int64_t i = threadIdx.x; i < v.N; i += PACK_THREADS) {
        int32_t b = bucket_of(v, i, t);
        if (b >= 0) {
            uint32_t pos = atomicAdd(&cnt[b], 1u);
            mem[pos] = (int32_t)i;
        }
    }
}

__global__ void k_fill_u32(uint32_t* p, int64_t n, uint32_t v) {
    int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; k < n; k += stride) p[k] = v;
}

// rec[i][t] = (offset, length) of the opposite-OOB bucket of i's leaf, via a
// 64 x 64 LDS tile so both the leaf reads and the rec writes are coalesced.
__global__ __launch_bounds__(256) void k_records(LeafView v, const int32_t* bkt_off, uint2* rec) {
    __shared__ uint2 tile[64][65];
    const int64_t i0 = (int64_t)blockIdx.x * 64;
    const int32_t t0 = blockIdx.y * 64;
    const int32_t nb1 = 2 * v.L + 1;
    for (int k = threadIdx.x; k < 64 * 64; k += 256) {
        int tl = k >> 6, il = k & 63;
        int64_t i = i0 + il;
        int32_t t = t0 + tl;
        uint2 r = make_uint2(0u, 0u);
        if (i < v.N && t < v.T) {
            int32_t b = bucket_of(v, i, t);
            if (b >= 0) {
                const int32_t* off = bkt_off + (int64_t)t * nb1;
                int32_t ob = b ^ 1;
                int32_t s = off[ob];
                r = make_uint2((uint32_t)s, (uint32_t)(off[ob + 1] - s));
            }
        }
        tile[tl][il] = r;
    }
    __syncthreads();
    for (int k = threadIdx.x; k < 64 * 64; k += 256) {
        int il = k >> 6, tl = k & 63;
        int64_t i = i0 + il;
        int32_t t = t0 + tl;
        if (i < v.N && t < v.T) rec[i * v.T + t] = tile[tl][il];
    }
}

// nout_i (counted from the OOB bits unless given), its reciprocal, and the
// min/max reciprocal over all samples (as IEEE bits; positive doubles order
// like their bit patterns).
__global__ void k_nout(LeafView v, const int32_t* nout_in, int32_t* nout, double* rinv,
                       unsigned long long* rr) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= v.N) return;
    int32_t n = 0;
    if (nout_in) {
        n = nout_in[i];
    } else {
        for (int32_t t = 0; t < v.T; ++t) n += (int32_t)((v.oob[(int64_t)t * v.old + (i >> 5)] >> (i & 31)) & 1u);
    }
    nout[i] = n;
    double r = nout_recip(n);
    rinv[i] = r;
    unsigned long long bits = (unsigned long long)__double_as_longlong(r);
    atomicMin(&rr[0], bits);
    atomicMax(&rr[1], bits);
}

__global__ void k_rr_init(unsigned long long* rr) {
    rr[0] = 0x7ff0000000000000ull;
    rr[1] = 0ull;
}

// ---------------------------------------------------------------------------
// triangle
// ---------------------------------------------------------------------------

struct TriArgs {
    const uint2* rec;
    const int32_t* mem;
    const double* rinv;
    const unsigned long long* rr;
    const int2* items;
    int64_t N;
    int32_t T;
    int32_t S;          // columns per item
    int64_t e_base;     // idx(row_begin, row_begin)
    char* out;          // byte address of entry e_base (NF4: of its byte)
    float scale, zp;
    int32_t* flags;     // [0]: items redone with 16-bit counters
};

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int b) { return (w >> (8 * b)) & 0xffu; }

// Replaces byte b (runtime index) of the 4-word little-endian array w with
// the low byte of v, without dynamic register indexing.
template <int NW>
__device__ __forceinline__ void set_byte(uint32_t (&w)[NW], int b, uint32_t v) {
    const uint32_t sh = 8u * (uint32_t)(b & 3);
#pragma unroll
    for (int q = 0; q < NW; ++q)
        w[q] = (q == (b >> 2)) ? ((w[q] & ~(0xffu << sh)) | ((v & 0xffu) << sh)) : w[q];
}

// Same for 32-bit entries.
template <int NW>
__device__ __forceinline__ void set_word(uint32_t (&w)[NW], int k, uint32_t v) {
#pragma unroll
    for (int q = 0; q < NW; ++q) w[q] = (q == k) ? v : w[q];
}

// Bytes per output entry; NF4 is handled in nibbles.
template <int F>
struct FmtInfo;
template <> struct FmtInfo<F32> { static constexpr int esz = 4; };
template <> struct FmtInfo<F16> { static constexpr int esz = 2; };
template <> struct FmtInfo<U16> { static constexpr int esz = 2; };
template <> struct FmtInfo<I8> { static constexpr int esz = 1; };
template <> struct FmtInfo<U8> { static constexpr int esz = 1; };

// Entry of an off-diagonal count U for column j, float formats.
template <int F>
__device__ __forceinline__ uint32_t float_entry(uint32_t U, double ri, const double* rinv, int64_t j) {
    if (U == 0) return 0u;
    float pf = (float)pair_p(U, ri, rinv[j]);
    if constexpr (F == F32) return __float_as_uint(pf);
    else return (uint32_t)f32_to_f16_bits(pf);
}

// Table-driven byte codes for I8 / U8 / NF4: lut_lo/lut_hi hold the codes
// of U = 0..7, valid for U < uc.
template <int F>
__device__ __forceinline__ uint32_t code_word(uint32_t w, uint32_t lut_lo, uint32_t lut_hi, uint32_t uc,
                                              double ri, const double* rinv, int64_t j0, float scale,
                                              float zp) {
    // all four counts < uc  <=>  no byte has its top bit set after adding 0x80 - uc
    const uint32_t k = (0x80u - uc) * 0x01010101u;
    if ((((w + k) | w) & 0x80808080u) == 0u) return __builtin_amdgcn_perm(lut_hi, lut_lo, w);
    uint32_t o = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        uint32_t U = byte_of(w, b);
        uint32_t c;
        if (U < uc) c = (U < 4 ? lut_lo >> (8 * U) : lut_hi >> (8 * (U - 4))) & 0xffu;
        else c = code_of<F>(pair_p(U, ri, rinv[j0 + b]), scale, zp);
        o |= c << (8 * b);
    }
    return o;
}

// Hit phase: every member j of row i's opposite buckets with lo <= j < hi
// bumps its counter.  Counter c of column j sits at unit (j - lo + shift)
// of the LDS array; BITS is 8 or 16.  Returns true when an 8-bit counter
// wrapped (only checked when T can exceed 255).
template <int BITS, bool CHECK>
__device__ __forceinline__ bool hit_phase(const TriArgs& a, uint32_t* cnt, int64_t i, int64_t lo,
                                          int32_t width, int32_t shift) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const uint2* recrow = a.rec + i * a.T;
    bool wrapped = false;
    auto hit = [&](int32_t j) {
        uint32_t d = (uint32_t)(j - (int32_t)lo);
        if (d < (uint32_t)width) {
            uint32_t c = d + (uint32_t)shift;
            if constexpr (BITS == 8) {
                uint32_t sh = (c & 3u) * 8u;
                if constexpr (CHECK) {
                    uint32_t old = atomicAdd(&cnt[c >> 2], 1u << sh);
                    wrapped |= ((old >> sh) & 0xffu) == 0xffu;
                } else {
                    atomicAdd(&cnt[c >> 2], 1u << sh);
                }
            } else {
                atomicAdd(&cnt[c >> 1], 1u << ((c & 1u) * 16u));
            }
        }
    };
    // Trees go to waves in groups of 8 (group g = trees 8g..8g+7, wave
    // g % 8); one record load fetches a wave's next 8 groups.  Records of
    // trees >= T read as (0, 0), so their buckets are empty.
    const int32_t ngroup = (a.T + 7) / 8;
    for (int32_t gb = wave; gb < ngroup; gb += 8 * TRI_WAVES) {
        const int32_t t = 8 * (gb + TRI_WAVES * (lane >> 3)) + (lane & 7);
        const uint2 r = t < a.T ? recrow[t] : make_uint2(0u, 0u);
        for (int32_t q = 0; q < 8; ++q) {
            const int32_t g = gb + TRI_WAVES * q;
            if (g >= ngroup) break;
            int32_t jv[8];
            uint32_t len[8];
            const int32_t* base[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int kk = 8 * q + u;
                const uint32_t st = (uint32_t)__builtin_amdgcn_readlane((int)r.x, kk);
                len[u] = (uint32_t)__builtin_amdgcn_readlane((int)r.y, kk);
                base[u] = a.mem + (int64_t)(8 * g + u) * a.N + st;
                jv[u] = (uint32_t)lane < len[u] ? base[u][lane] : -1;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) hit(jv[u]);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (len[u] > 64u) {
                    for (uint32_t p = 64u + lane; p < len[u]; p += 64u) hit(base[u][p]);
                }
            }
        }
    }
    return wrapped;
}

// Exact per-entry epilogue with 16-bit counters (segments whose 8-bit
// counters wrapped).  Writes entries [lo, lo+width) of row i.
template <int F>
__device__ void store_exact16(const TriArgs& a, const uint32_t* cnt, int64_t i, int64_t lo, int32_t width,
                              double ri) {
    const int64_t e0 = tri_idx(a.N, i, lo) - a.e_base;
    for (int32_t d = threadIdx.x; d < width; d += TRI_THREADS) {
        const int64_t j = lo + d;
        const uint32_t U = (cnt[d >> 1] >> ((d & 1) * 16)) & 0xffffu;
        const bool diag = (j == i);
        const int64_t e = e0 + d;
        if constexpr (F == U16) {
            ((uint16_t*)a.out)[e] = diag ? 0 : (uint16_t)U;
        } else {
            double P = diag ? 1.0 : (U == 0 ? 0.0 : pair_p(U, ri, a.rinv[j]));
            if constexpr (F == F32) ((float*)a.out)[e] = (float)P;
            else if constexpr (F == F16) ((uint16_t*)a.out)[e] = f32_to_f16_bits((float)P);
            else ((uint8_t*)a.out)[e] = (uint8_t)code_of<F>(P, a.scale, a.zp);
        }
    }
}

template <int F>
__global__ __launch_bounds__(TRI_THREADS) void k_tri(TriArgs a) {
    extern __shared__ uint32_t cnt[];
    __shared__ uint32_t s_lut[2];
    __shared__ uint32_t s_uc;
    __shared__ int s_wrapped;
    constexpr int esz = FmtInfo<F>::esz;
    constexpr int epc = 16 / esz;  // entries per 16-byte chunk

    const int2 it = a.items[blockIdx.x];
    const int64_t i = it.x;
    const int64_t lo = it.y;
    const int32_t width = (int32_t)min((int64_t)a.S, a.N - lo);
    const double ri = a.rinv[i];

    // Align counters to the output: chunk c of the LDS array maps to the
    // 16-byte aligned output chunk c.
    char* const dst0 = a.out + (tri_idx(a.N, i, lo) - a.e_base) * esz;
    const int32_t shift = (int32_t)(((uintptr_t)dst0 & 15u) / esz);
    char* const dst_al = dst0 - shift * esz;
    const int32_t nchunk = (shift + width + epc - 1) / epc;
    const int32_t nwords = nchunk * epc / 4;  // 8-bit counters

    for (int32_t w = threadIdx.x; w < nwords; w += TRI_THREADS) cnt[w] = 0u;
    if (threadIdx.x == 0) s_wrapped = 0;
    if constexpr (F == I8 || F == U8) {
        // Per-row code table: U < uc give the same code for every column
        // (the code is monotone in r_j, so equal codes at min and max r_j
        // mean equal codes everywhere).
        if (threadIdx.x < 64) {
            const int u = threadIdx.x & 7;
            const double rmin = __longlong_as_double((long long)a.rr[0]);
            const double rmax = __longlong_as_double((long long)a.rr[1]);
            const uint32_t c0 = code_of<F>(pair_p(u, ri, rmin), a.scale, a.zp);
            const uint32_t c1 = code_of<F>(pair_p(u, ri, rmax), a.scale, a.zp);
            const unsigned long long eq = __ballot(c0 == c1 && threadIdx.x < 8);
            if (threadIdx.x == 0) {
                uint32_t uc = 0;
                while (uc < 8 && ((eq >> uc) & 1ull)) ++uc;
                s_uc = uc;
            }
            uint32_t lo4 = 0, hi4 = 0;
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                uint32_t cb = (uint32_t)__shfl((int)c0, b, 64);
                if (b < 4) lo4 |= cb << (8 * b);
                else hi4 |= cb << (8 * (b - 4));
            }
            if (threadIdx.x == 0) {
                s_lut[0] = lo4;
                s_lut[1] = hi4;
            }
        }
    }
    __syncthreads();

    bool wrapped;
    if (a.T > 255) wrapped = hit_phase<8, true>(a, cnt, i, lo, width, shift);
    else wrapped = hit_phase<8, false>(a, cnt, i, lo, width, shift);
    if (wrapped) s_wrapped = 1;
    __syncthreads();

    if (s_wrapped) {
        // Some count reached 256: redo the segment with 16-bit counters in
        // two halves of the same LDS space.
        if (threadIdx.x == 0) atomicAdd(&a.flags[0], 1);
        const int32_t half_cap = nwords * 2;  // 16-bit counters that fit
        for (int32_t d0 = 0; d0 < width; d0 += half_cap) {
            const int32_t w2 = min(half_cap, width - d0);
            __syncthreads();
            for (int32_t w = threadIdx.x; w < (w2 + 1) / 2; w += TRI_THREADS) cnt[w] = 0u;
            __syncthreads();
            hit_phase<16, false>(a, cnt, i, lo + d0, w2, 0);
            __syncthreads();
            store_exact16<F>(a, cnt, i, lo + d0, w2, ri);
        }
        return;
    }

    const bool has_diag = (lo == i);
    const uint4* c4 = (const uint4*)cnt;
    if constexpr (F == I8 || F == U8) {
        const uint32_t lut_lo = s_lut[0], lut_hi = s_lut[1], uc = s_uc;
        const uint32_t dcode = code_of<F>(1.0, a.scale, a.zp);
        for (int32_t ck = threadIdx.x; ck < nchunk; ck += TRI_THREADS) {
            const uint4 w = c4[ck];
            const int64_t jb = lo + (int64_t)ck * 16 - shift;  // column of byte 0
            uint32_t o[4];
            o[0] = code_word<F>(w.x, lut_lo, lut_hi, uc, ri, a.rinv, jb + 0, a.scale, a.zp);
            o[1] = code_word<F>(w.y, lut_lo, lut_hi, uc, ri, a.rinv, jb + 4, a.scale, a.zp);
            o[2] = code_word<F>(w.z, lut_lo, lut_hi, uc, ri, a.rinv, jb + 8, a.scale, a.zp);
            o[3] = code_word<F>(w.w, lut_lo, lut_hi, uc, ri, a.rinv, jb + 12, a.scale, a.zp);
            // the diagonal is column lo, byte `shift` of chunk 0
            if (has_diag && ck == 0) set_byte(o, shift, dcode);
            char* d = dst_al + (int64_t)ck * 16;
            const int32_t first = ck * 16, last = first + 16;
            if (first >= shift && last <= shift + width) {
                u32x4 v4 = {o[0], o[1], o[2], o[3]};
                __builtin_nontemporal_store(v4, (u32x4*)d);
            } else {
#pragma unroll
                for (int b = 0; b < 16; ++b) {
                    const int32_t e = first + b;
                    if (e >= shift && e < shift + width) d[b] = (char)byte_of(o[b >> 2], b & 3);
                }
            }
        }
    } else {
        // F32 / F16 / U16: epc entries per chunk = epc counters (bytes)
        for (int32_t ck = threadIdx.x; ck < nchunk; ck += TRI_THREADS) {
            uint32_t cw[2];
            if constexpr (epc == 4) {
                cw[0] = cnt[ck];
                cw[1] = 0;
            } else {
                cw[0] = cnt[2 * ck];
                cw[1] = cnt[2 * ck + 1];
            }
            const int64_t jb = lo + (int64_t)ck * epc - shift;
            uint32_t o[4];
            if constexpr (F == F32) {
#pragma unroll
                for (int b = 0; b < 4; ++b) o[b] = float_entry<F32>(byte_of(cw[0], b), ri, a.rinv, jb + b);
                if (has_diag && ck == 0) set_word(o, shift, __float_as_uint(1.0f));
            } else {
                uint32_t h[8];
#pragma unroll
                for (int b = 0; b < 8; ++b) {
                    const uint32_t U = byte_of(cw[b >> 2], b & 3);
                    if constexpr (F == F16) h[b] = float_entry<F16>(U, ri, a.rinv, jb + b);
                    else h[b] = U;
                }
                if (has_diag && ck == 0) set_word(h, shift, (F == F16) ? 0x3c00u : 0u);
#pragma unroll
                for (int b = 0; b < 4; ++b) o[b] = h[2 * b] | (h[2 * b + 1] << 16);
            }
            char* d = dst_al + (int64_t)ck * 16;
            const int32_t first = ck * epc, last = first + epc;
            if (first >= shift && last <= shift + width) {
                u32x4 v4 = {o[0], o[1], o[2], o[3]};
                __builtin_nontemporal_store(v4, (u32x4*)d);
            } else {
#pragma unroll
                for (int b = 0; b < epc; ++b) {
                    const int32_t e = first + b;
                    if (e < shift || e >= shift + width) continue;
                    if constexpr (esz == 4) ((uint32_t*)d)[b] = o[b];
                    else ((uint16_t*)d)[b] = (uint16_t)(o[b >> 1] >> (16 * (b & 1)));
                }
            }
        }
    }
}

// NF4: two entries per byte.  Nibble position g(e) = e - e_base + (e_base & 1)
// relative to the byte `out`.  Bytes with both nibbles inside the item are
// stored whole; a byte shared with a neighbouring item (row boundaries) is
// merged with 32-bit atomics on its own nibble only.
__global__ __launch_bounds__(TRI_THREADS) void k_tri_nf4(TriArgs a) {
    extern __shared__ uint32_t cnt[];
    __shared__ uint32_t s_lut[2];
    __shared__ uint32_t s_uc;
    __shared__ int s_wrapped;

    const int2 it = a.items[blockIdx.x];
    const int64_t i = it.x;
    const int64_t lo = it.y;
    const int32_t width = (int32_t)min((int64_t)a.S, a.N - lo);
    const double ri = a.rinv[i];

    const int64_t g0 = tri_idx(a.N, i, lo) - a.e_base + (a.e_base & 1);  // nibble index
    char* const byte0 = a.out + (g0 >> 1);
    const int32_t shift = (int32_t)(((uintptr_t)byte0 & 15u) * 2 + (g0 & 1));  // nibbles
    char* const dst_al = byte0 - ((uintptr_t)byte0 & 15u);
    const int32_t nchunk = (shift + width + 31) / 32;  // 32 nibbles per 16 bytes
    const int32_t nwords = nchunk * 8;

    for (int32_t w = threadIdx.x; w < nwords; w += TRI_THREADS) cnt[w] = 0u;
    if (threadIdx.x == 0) s_wrapped = 0;
    if (threadIdx.x < 64) {
        const int u = threadIdx.x & 7;
        const double rmin = __longlong_as_double((long long)a.rr[0]);
        const double rmax = __longlong_as_double((long long)a.rr[1]);
        const uint32_t c0 = code_of<NF4>(pair_p(u, ri, rmin), 0.f, 0.f);
        const uint32_t c1 = code_of<NF4>(pair_p(u, ri, rmax), 0.f, 0.f);
        const unsigned long long eq = __ballot(c0 == c1 && threadIdx.x < 8);
        uint32_t lo4 = 0, hi4 = 0;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            uint32_t cb = (uint32_t)__shfl((int)c0, b, 64);
            if (b < 4) lo4 |= cb << (8 * b);
            else hi4 |= cb << (8 * (b - 4));
        }
        if (threadIdx.x == 0) {
            uint32_t uc = 0;
            while (uc < 8 && ((eq >> uc) & 1ull)) ++uc;
            s_uc = uc;
            s_lut[0] = lo4;
            s_lut[1] = hi4;
        }
    }
    __syncthreads();
    bool wrapped;
    if (a.T > 255) wrapped = hit_phase<8, true>(a, cnt, i, lo, width, shift);
    else wrapped = hit_phase<8, false>(a, cnt, i, lo, width, shift);
    if (wrapped) s_wrapped = 1;
    __syncthreads();

    const uint32_t dcode = code_of<NF4>(1.0, 0.f, 0.f);
    if (s_wrapped) {
        if (threadIdx.x == 0) atomicAdd(&a.flags[0], 1);
        const int32_t half_cap = nwords * 2;
        for (int32_t d0 = 0; d0 < width; d0 += half_cap) {
            const int32_t w2 = min(half_cap, width - d0);
            __syncthreads();
            for (int32_t w = threadIdx.x; w < (w2 + 1) / 2; w += TRI_THREADS) cnt[w] = 0u;
            __syncthreads();
            hit_phase<16, false>(a, cnt, i, lo + d0, w2, 0);
            __syncthreads();
            for (int32_t d = threadIdx.x; d < w2; d += TRI_THREADS) {
                const int64_t j = lo + d0 + d;
                const uint32_t U = (cnt[d >> 1] >> ((d & 1) * 16)) & 0xffffu;
                const uint32_t c = (j == i) ? dcode : (U == 0 ? code_of<NF4>(0.0, 0.f, 0.f)
                                                              : code_of<NF4>(pair_p(U, ri, a.rinv[j]), 0.f, 0.f));
                const int64_t g = g0 + d0 + d;
                const uintptr_t ba = (uintptr_t)a.out + (uintptr_t)(g >> 1);
                uint32_t* word = (uint32_t*)(ba & ~(uintptr_t)3);
                const uint32_t sh = (uint32_t)((ba & 3u) * 8u + (uint32_t)(g & 1) * 4u);
                atomicAnd(word, ~(0xfu << sh));
                atomicOr(word, c << sh);
            }
        }
        return;
    }

    const uint32_t lut_lo = s_lut[0], lut_hi = s_lut[1], uc = s_uc;
    const bool has_diag = (lo == i);
    const uint4* c4 = (const uint4*)cnt;
    for (int32_t ck = threadIdx.x; ck < nchunk; ck += TRI_THREADS) {
        // 32 counters -> 32 nibble codes -> 16 bytes
        uint32_t cw[8];
        const uint4 wa = c4[2 * ck], wb = c4[2 * ck + 1];
        cw[0] = wa.x; cw[1] = wa.y; cw[2] = wa.z; cw[3] = wa.w;
        cw[4] = wb.x; cw[5] = wb.y; cw[6] = wb.z; cw[7] = wb.w;
        const int64_t jb = lo + (int64_t)ck * 32 - shift;
        uint32_t codes[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
            codes[q] = code_word<NF4>(cw[q], lut_lo, lut_hi, uc, ri, a.rinv, jb + 4 * q, 0.f, 0.f);
        if (has_diag && ck == 0) set_byte(codes, shift, dcode);
        // pack byte codes c0..c3 of each word into two nibble-bytes
        uint32_t ob[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t x = codes[2 * q], y = codes[2 * q + 1];
            const uint32_t px = (x & 0x000f000fu) | ((x & 0x0f000f00u) >> 4);  // bytes 0,2
            const uint32_t py = (y & 0x000f000fu) | ((y & 0x0f000f00u) >> 4);
            ob[q] = (px & 0xffu) | (((px >> 16) & 0xffu) << 8) | ((py & 0xffu) << 16) | (((py >> 16) & 0xffu) << 24);
        }
        char* d = dst_al + (int64_t)ck * 16;
        const int32_t first = ck * 32, last = first + 32;
        if (first >= shift && last <= shift + width) {
            u32x4 v4 = {ob[0], ob[1], ob[2], ob[3]};
            __builtin_nontemporal_store(v4, (u32x4*)d);
        } else {
#pragma unroll
            for (int b = 0; b < 16; ++b) {
                const int32_t e0 = first + 2 * b, e1 = e0 + 1;
                const bool in0 = e0 >= shift && e0 < shift + width;
                const bool in1 = e1 >= shift && e1 < shift + width;
                const uint32_t v = byte_of(ob[b >> 2], b & 3);
                if (in0 && in1) {
                    d[b] = (char)v;
                } else if (in0 || in1) {
                    uint32_t* word = (uint32_t*)(d + (b & ~3));
                    const uint32_t sh = (uint32_t)((b & 3) * 8 + (in1 ? 4 : 0));
                    const uint32_t nib = in1 ? (v >> 4) : (v & 0xfu);
                    atomicAnd(word, ~(0xfu << sh));
                    atomicOr(word, nib << sh);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

static int tri_segment_cols(rfxp_ctx* ctx, int fmt) {
    // Counter bytes per workgroup; leave room for the static LDS words and
    // for the 16-byte alignment shift.  Two workgroups per CU on gfx950.
    int budget = std::min(ctx->max_lds, 160 * 1024) / 2 - 1024;
    budget = std::max(budget, 4096);
    budget &= ~63;
    if (fmt == NF4) return budget;  // one counter byte per nibble entry
    return budget;
}

static int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace rfxp

using namespace rfxp;

extern "C" int64_t rfxp_upper_nbytes(int fmt, int64_t N, int64_t r0, int64_t r1) {
    if (N < 0 || r0 < 0 || r1 > N || r0 > r1) return -1;
    const int64_t e0 = tri_idx(N, r0, r0), e1 = tri_idx(N, r1, r1);
    switch (fmt) {
        case F32: return (e1 - e0) * 4;
        case F16:
        case U16: return (e1 - e0) * 2;
        case I8:
        case U8: return e1 - e0;
        case NF4: return e1 > e0 ? ((e1 - 1) >> 1) - (e0 >> 1) + 1 : 0;
        default: return -1;
    }
}

extern "C" int rfxp_set_forest(rfxp_ctx* ctx, const int32_t* leaf, int64_t stride_i, int64_t stride_t,
                               const uint32_t* oob_words, int64_t oob_ld, int64_t N, int32_t T, int32_t nleaf,
                               const int32_t* nout) {
    if (!ctx) return RFXP_ERR_INVALID;
    ctx->forest_ready = false;
    if (N < 0 || N > 0x7fffffffLL || T < 1 || T > 65535 || nleaf < 1 || nleaf > (1 << 29))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_set_forest: need 0 <= N < 2^31, 1 <= T <= 65535, 1 <= nleaf <= 2^29");
    if (N > 0 && (!leaf || !oob_words))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_set_forest: leaf / oob_words are NULL");
    if (oob_ld < (N + 31) / 32)
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_set_forest: oob_ld < ceil(N/32)");
    if (N > 0 && (!is_device_pointer(leaf) || !is_device_pointer(oob_words) || (nout && !is_device_pointer(nout))))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_set_forest: inputs must be device pointers");
    if ((int64_t)N * T > 0xffffffffLL)
        return set_error(ctx, RFXP_ERR_UNSUPPORTED, "rfxp_set_forest: N*T must stay below 2^32");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    ctx->N = N;
    ctx->T = T;
    ctx->L = nleaf;
    const int32_t nb = 2 * nleaf;
    RFXP_HIP(ctx, ctx->bkt_off.ensure((size_t)T * (nb + 1)));
    RFXP_HIP(ctx, ctx->bkt_mem.ensure((size_t)T * (size_t)std::max<int64_t>(N, 1)));
    RFXP_HIP(ctx, ctx->rec.ensure((size_t)std::max<int64_t>(N, 1) * T));
    RFXP_HIP(ctx, ctx->nout.ensure((size_t)std::max<int64_t>(N, 1)));
    RFXP_HIP(ctx, ctx->rinv.ensure((size_t)std::max<int64_t>(N, 1)));
    RFXP_HIP(ctx, ctx->rrange.ensure(2));
    RFXP_HIP(ctx, ctx->flags.ensure(16));
    LeafView v{leaf, stride_i, stride_t, oob_words, oob_ld, N, T, nleaf};
    hipStream_t s = ctx->stream;
    {
        LaunchTimer tm(ctx, "rr_init");
        hipLaunchKernelGGL(k_rr_init, dim3(1), dim3(1), 0, s, ctx->rrange.p);
    }
    if (int rc = check_launch(ctx, "k_rr_init")) return rc;
    if (N == 0) {
        ctx->forest_ready = true;
        return RFXP_OK;
    }
    const size_t lds_bytes = (size_t)(nb + PACK_THREADS) * 4;
    if ((int64_t)lds_bytes <= ctx->max_lds) {
        if (lds_bytes > 65536)
            RFXP_HIP(ctx, hipFuncSetAttribute((const void*)k_bucket_lds, hipFuncAttributeMaxDynamicSharedMemorySize,
                                              (int)lds_bytes));
        LaunchTimer tm(ctx, "bucket");
        hipLaunchKernelGGL(k_bucket_lds, dim3(T), dim3(PACK_THREADS), lds_bytes, s, v, ctx->bkt_off.p, ctx->bkt_mem.p);
    } else {
        RFXP_HIP(ctx, ctx->bkt_cnt.ensure((size_t)T * nb));
        const int64_t n = (int64_t)T * nb;
        hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)std::min<int64_t>(ceil_div(n, 256), 65536)), dim3(256), 0, s,
                           ctx->bkt_cnt.p, n, 0u);
        LaunchTimer tm(ctx, "bucket");
        hipLaunchKernelGGL(k_bucket_global, dim3(T), dim3(PACK_THREADS), 0, s, v, ctx->bkt_cnt.p, ctx->bkt_off.p,
                           ctx->bkt_mem.p);
    }
    if (int rc = check_launch(ctx, "k_bucket")) return rc;
    {
        LaunchTimer tm(ctx, "records");
        hipLaunchKernelGGL(k_records, dim3((unsigned)ceil_div(N, 64), (unsigned)ceil_div(T, 64)), dim3(256), 0, s, v,
                           ctx->bkt_off.p, ctx->rec.p);
    }
    if (int rc = check_launch(ctx, "k_records")) return rc;
    {
        LaunchTimer tm(ctx, "nout");
        hipLaunchKernelGGL(k_nout, dim3((unsigned)ceil_div(N, 256)), dim3(256), 0, s, v, nout, ctx->nout.p,
                           ctx->rinv.p, ctx->rrange.p);
    }
    if (int rc = check_launch(ctx, "k_nout")) return rc;
    ctx->forest_ready = true;
    return RFXP_OK;
}

template <int F>
static hipError_t launch_tri(rfxp_ctx* ctx, const TriArgs& a, int64_t n_items, size_t lds) {
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute((const void*)k_tri<F>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k_tri<F>, dim3((unsigned)n_items), dim3(TRI_THREADS), lds, ctx->stream, a);
    return hipGetLastError();
}

static hipError_t launch_tri_nf4(rfxp_ctx* ctx, const TriArgs& a, int64_t n_items, size_t lds) {
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute((const void*)k_tri_nf4, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k_tri_nf4, dim3((unsigned)n_items), dim3(TRI_THREADS), lds, ctx->stream, a);
    return hipGetLastError();
}

extern "C" int rfxp_upper(rfxp_ctx* ctx, int fmt, float scale, float zp, int64_t r0, int64_t r1, void* out) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (!ctx->forest_ready) return set_error(ctx, RFXP_ERR_STATE, "rfxp_upper: no forest set");
    const int64_t N = ctx->N;
    if (fmt < F32 || fmt > U16) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_upper: unknown format");
    if (r0 < 0 || r1 > N || r0 > r1) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_upper: bad row range");
    if ((fmt == I8 || fmt == U8) && (!std::isfinite(scale) || scale == 0.0f || !std::isfinite(zp)))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_upper: scale must be finite and non-zero, zp finite");
    if (r0 == r1) return RFXP_OK;
    if (!out || !is_device_pointer(out)) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_upper: out must be a device pointer");
    const int esz = (fmt == F32) ? 4 : (fmt == F16 || fmt == U16) ? 2 : 1;
    if (((uintptr_t)out) % esz != 0) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_upper: out is not aligned to its entry size");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));

    const int32_t S = tri_segment_cols(ctx, fmt);
    // work list: rows in increasing order, each split into S-column segments
    if (ctx->items_key[0] != N || ctx->items_key[1] != r0 || ctx->items_key[2] != r1 || ctx->items_key[3] != S) {
        std::vector<int2> items;
        for (int64_t i = r0; i < r1; ++i)
            for (int64_t lo = i; lo < N; lo += S) items.push_back(make_int2((int)i, (int)lo));
        if ((int64_t)items.size() > 0x7fffffffLL) return set_error(ctx, RFXP_ERR_UNSUPPORTED, "rfxp_upper: too many work items");
        RFXP_HIP(ctx, ctx->items.ensure(items.size()));
        RFXP_HIP(ctx, hipMemcpy(ctx->items.p, items.data(), items.size() * sizeof(int2), hipMemcpyHostToDevice));
        ctx->n_items = (int64_t)items.size();
        ctx->items_key[0] = N;
        ctx->items_key[1] = r0;
        ctx->items_key[2] = r1;
        ctx->items_key[3] = S;
    }
    TriArgs a;
    a.rec = ctx->rec.p;
    a.mem = ctx->bkt_mem.p;
    a.rinv = ctx->rinv.p;
    a.rr = ctx->rrange.p;
    a.items = ctx->items.p;
    a.N = N;
    a.T = ctx->T;
    a.S = S;
    a.e_base = tri_idx(N, r0, r0);
    a.out = (char*)out;
    a.scale = scale;
    a.zp = zp;
    a.flags = ctx->flags.p;
    // counters: S units + up to one 16-byte chunk of alignment shift,
    // rounded to whole chunks (NF4: 32 nibbles per chunk)
    const size_t lds = (size_t)S + 64;
    hipError_t e;
    {
        LaunchTimer tm(ctx, "tri");
        switch (fmt) {
            case F32: e = launch_tri<F32>(ctx, a, ctx->n_items, lds); break;
            case F16: e = launch_tri<F16>(ctx, a, ctx->n_items, lds); break;
            case I8: e = launch_tri<I8>(ctx, a, ctx->n_items, lds); break;
            case U8: e = launch_tri<U8>(ctx, a, ctx->n_items, lds); break;
            case U16: e = launch_tri<U16>(ctx, a, ctx->n_items, lds); break;
            default: e = launch_tri_nf4(ctx, a, ctx->n_items, lds); break;
        }
    }
    if (e != hipSuccess) return hip_error(ctx, e, "k_tri launch");
    return RFXP_OK;
}

extern "C" int rfxp_get_nout(rfxp_ctx* ctx, int32_t* nout) {
    if (!ctx || !nout) return RFXP_ERR_INVALID;
    if (!ctx->forest_ready) return set_error(ctx, RFXP_ERR_STATE, "rfxp_get_nout: no forest set");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    if (ctx->N == 0) return RFXP_OK;
    RFXP_HIP(ctx, hipMemcpyAsync(nout, ctx->nout.p, sizeof(int32_t) * ctx->N, hipMemcpyDeviceToDevice, ctx->stream));
    return RFXP_OK;
}
