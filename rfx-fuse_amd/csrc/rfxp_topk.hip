// Per-query top-K of the most proximate reference samples, without the
// query x reference proximity matrix.
//
// Reference semantics restated:
//   * new queries, all trees (python/randomforest_py.cpp:2496-2568, and
//     LoadedModel::get_top_k_similar :624-672): count(q, j) = #{t : leaf_q(t)
//     == leaf_j(t)}; the top K over all N references, zero counts included;
//   * OOB queries (src/rf_random_forest.cpp:4677-4782): only the trees where
//     the query sample is out-of-bag, the query itself excluded, counts > 0
//     only (the caller scales by 1/|OOB(q)|).
// Ties are broken by the lower reference index (the reference leaves them to
// std::partial_sort, whose order is unspecified).
//
// Layout: the reference set is packed like a forest, but bucket
// b = leaf*nseg + (j >> seg_shift) holds the references of one leaf and one
// column segment of S = 2^seg_shift references (rfxp_set_reference).  A
// query's bucket in tree t and segment s is then one contiguous run, found
// from its leaf label with two offset loads.
//
// Kernel k_topk: one workgroup per query walks the segments in order.  Per
// segment, 16-bit LDS counters (one per reference of the segment) take the
// query's T buckets exactly as the triangle's hit phase does; then the
// counters become keys (count + 1, 0 for references that may not be chosen)
// and only keys above the running K-th best key are looked at: entries of a
// later segment lose every tie against the running list, which holds lower
// indices.  Selection is exact: a binary search over key levels for the
// threshold, ordered compaction of the winners, and a rank merge with the
// running list by one wave.
#include <algorithm>
#include <string>

#include "rfxp_device.hpp"
#include "rfxp_forest.hpp"
#include "rfxp_internal.hpp"

namespace rfxp {

constexpr int TOPK_THREADS = 1024;
constexpr int TOPK_WAVES = TOPK_THREADS / 64;
constexpr int TOPK_MAX_K = 64;
constexpr int TOPK_MAX_SHIFT = 15;  // 32768 16-bit counters: 64 KB, two workgroups per CU
constexpr int TOPK_MIN_SHIFT = 11;  // at least 2 counters per thread

struct TopkArgs {
    const uint32_t* mem;  // reference members (j + 1), [T][N]
    uint32_t mem_bytes;
    const int32_t* off;   // [T][nb + 1]
    int32_t nb;
    int64_t N;
    int32_t T, L, nseg, shift;
    const int32_t* qleaf;
    int64_t qsi, qst;
    const uint32_t* qoob;  // NULL: all trees
    int64_t qold;
    int64_t exclude_base;  // query q excludes reference exclude_base + q; < 0: none
    int64_t q0;            // query of workgroup 0 of this launch
    int32_t K;
    int32_t floor_key;     // smallest selectable key: 1 (zeros allowed) or 2 (counts > 0)
    int32_t* idx_out;
    uint16_t* cnt_out;
};

// LDS layout: counters (S/2 words) | dummy words (1024) | per-segment
// bucket records of up to 1024 trees (offset, length) | reduction scratch |
// candidate and running lists.
__host__ __device__ constexpr uint32_t topk_dummy_off(int32_t shift) { return (1u << shift) * 2u; }
constexpr uint32_t TOPK_REC_WORDS = 2 * TOPK_THREADS;
constexpr uint32_t TOPK_RED_WORDS = 64;                     // wave partials
constexpr uint32_t TOPK_LIST_WORDS = 4 * TOPK_MAX_K + 8;    // candidate / running lists
__host__ __device__ constexpr uint32_t topk_lds_bytes(int32_t shift) {
    return topk_dummy_off(shift) + (TOPK_THREADS + TOPK_REC_WORDS + TOPK_RED_WORDS + TOPK_LIST_WORDS) * 4;
}

typedef __attribute__((address_space(3))) uint32_t lds_w;
__device__ __forceinline__ void lds_add16(uint32_t addr, uint32_t val) {
    __hip_atomic_fetch_add((lds_w*)(uintptr_t)addr, val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t ref_rsrc(const uint32_t* mem, uint32_t nbytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)mem, (short)0, (int)nbytes, 0x00020000);
}

// Bucket (byte offset, byte length) of query q in tree t, segment s.
__device__ __forceinline__ void query_bucket(const TopkArgs& a, int64_t q, int32_t t, int32_t s, uint32_t& soff,
                                             uint32_t& len4) {
    soff = 0u;
    len4 = 0u;
    if (t >= a.T) return;
    const int32_t l = a.qleaf[q * a.qsi + (int64_t)t * a.qst];
    if (l < 0 || l >= a.L) return;
    if (a.qoob) {
        const uint32_t w = a.qoob[(int64_t)t * a.qold + (q >> 5)];
        if (((w >> (q & 31)) & 1u) == 0u) return;
    }
    const int32_t* ot = a.off + (int64_t)t * (a.nb + 1) + (int64_t)l * a.nseg + s;
    const uint32_t o0 = (uint32_t)ot[0], o1 = (uint32_t)ot[1];
    soff = 4u * ((uint32_t)t * (uint32_t)a.N + o0);
    len4 = 4u * (o1 - o0);
}

__device__ __forceinline__ void count16(uint32_t m, uint32_t base1, uint32_t width, uint32_t dummy) {
    // m = j + 1 (0: no member); 16-bit counter unit c = j - lo
    const uint32_t c = m - base1;
    const bool h = c < width;
    lds_add16(h ? ((c << 1) & ~3u) : dummy, 1u << ((c << 4) & 16u));
}

// 16 bucket loads of record group g (records rec_off/rec_len in LDS); a
// group outside [.., g1) loads nothing.  Returns whether a bucket of the
// group has more than 64 members.
__device__ __forceinline__ bool load16(const TopkArgs& a, const uint32_t* rec_off, const uint32_t* rec_len, int32_t g,
                                       bool ok, uint32_t lane4, uint32_t (&m)[16]) {
    bool lng = false;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const uint32_t soff = ok ? __builtin_amdgcn_readfirstlane(rec_off[16 * g + u]) : 0u;
        const uint32_t len4 = ok ? __builtin_amdgcn_readfirstlane(rec_len[16 * g + u]) : 0u;
        lng |= len4 > 256u;
        m[u] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(ref_rsrc(a.mem, soff + len4), lane4, soff, 0);
    }
    return lng;
}

__device__ __forceinline__ void tails16(const TopkArgs& a, const uint32_t* rec_off, const uint32_t* rec_len, int32_t g,
                                        uint32_t lane4, uint32_t base1, uint32_t width, uint32_t dummy) {
    for (int u = 0; u < 16; ++u) {
        const uint32_t len4 = __builtin_amdgcn_readfirstlane(rec_len[16 * g + u]);
        if (len4 <= 256u) continue;
        const uint32_t soff = __builtin_amdgcn_readfirstlane(rec_off[16 * g + u]);
        const __amdgpu_buffer_rsrc_t rs = ref_rsrc(a.mem, soff + len4);
        for (uint32_t p4 = 256u; p4 < len4; p4 += 256u)
            count16((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs, p4 + lane4, soff, 0), base1, width, dummy);
    }
}

// Per-thread level counts of keys >= c0 + d for d = 0..3, two 16-bit fields
// per word (a thread holds at most 32 keys, a workgroup at most 32768, so
// the fields of a block sum do not carry into each other).
template <int NW>
__device__ __forceinline__ void level_counts(const uint32_t (&key)[NW], uint32_t c0, uint32_t& w01, uint32_t& w23) {
    uint32_t n0 = 0, n1 = 0, n2 = 0, n3 = 0;
#pragma unroll
    for (int k = 0; k < NW; ++k) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t v = (key[k] >> (16 * h)) & 0xffffu;
            n0 += v >= c0;
            n1 += v >= c0 + 1u;
            n2 += v >= c0 + 2u;
            n3 += v >= c0 + 3u;
        }
    }
    w01 = n0 | (n1 << 16);
    w23 = n2 | (n3 << 16);
}

// Wave-wide sum / maximum through DPP lane moves (no lane-index registers):
// quad swaps, then half-row and row mirrors leave every lane with its
// 16-lane row total; the four row totals are read as scalars.  The whole
// wave must be active.
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v, int ctrl) {
    switch (ctrl) {
        case 0: return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);   // quad_perm 1,0,3,2
        case 1: return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);   // quad_perm 2,3,0,1
        case 2: return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, false);  // row_half_mirror
        default: return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, false); // row_mirror
    }
}
__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
#pragma unroll
    for (int c = 0; c < 4; ++c) v += dpp_mov(v, c);
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 0) + (uint32_t)__builtin_amdgcn_readlane((int)v, 16) +
           (uint32_t)__builtin_amdgcn_readlane((int)v, 32) + (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
}
__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
#pragma unroll
    for (int c = 0; c < 4; ++c) v = max(v, dpp_mov(v, c));
    return max(max((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 16)),
               max((uint32_t)__builtin_amdgcn_readlane((int)v, 32), (uint32_t)__builtin_amdgcn_readlane((int)v, 48)));
}

// Block sums of w01 and w23 and block maximum of m through `red` (48
// words); every thread gets the results.  Two barriers.
__device__ __forceinline__ void block_levels(uint32_t& w01, uint32_t& w23, uint32_t& m, uint32_t* red) {
    const uint32_t s01 = wave_sum(w01), s23 = wave_sum(w23), mx = wave_max(m);
    if ((threadIdx.x & 63) == 0) {
        red[3 * (threadIdx.x >> 6)] = s01;
        red[3 * (threadIdx.x >> 6) + 1] = s23;
        red[3 * (threadIdx.x >> 6) + 2] = mx;
    }
    __syncthreads();
    // lane w < 16 of every wave picks up wave w's partials
    const uint32_t l = threadIdx.x & 63u;
    const bool have = l < (uint32_t)TOPK_WAVES;
    const uint32_t a = have ? red[3 * l] : 0u, b = have ? red[3 * l + 1] : 0u, c = have ? red[3 * l + 2] : 0u;
    w01 = wave_sum(a);
    w23 = wave_sum(b);
    m = wave_max(c);
    __syncthreads();
}

// Exclusive prefix sum over threads in thread order of v = a | (b << 16)
// with a, b <= 63; *total gets the sum.  Within a wave the prefix is built
// bit by bit from ballots (mbcnt counts the set lanes below this one).
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* red, uint32_t* total) {
    uint32_t pre = 0, wt = 0;
#pragma unroll
    for (int b = 0; b < 22; ++b) {
        if (b >= 6 && b < 16) continue;
        const uint64_t m = __ballot((v >> b) & 1u);
        pre += __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u)) << b;
        wt += (uint32_t)__popcll(m) << b;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = wt;
    __syncthreads();
    const uint32_t l = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t x = l < (uint32_t)TOPK_WAVES ? red[l] : 0u;
    const uint32_t before = wave_sum(l < wave ? x : 0u);
    *total = wave_sum(x);
    __syncthreads();
    return before + pre;
}

// Number of this thread's keys (16-bit halves of its NW key words) >= c.
template <int NW>
__device__ __forceinline__ uint32_t count_ge(const uint32_t (&key)[NW], uint32_t c) {
    uint32_t n = 0;
#pragma unroll
    for (int k = 0; k < NW; ++k) n += ((key[k] & 0xffffu) >= c) + ((key[k] >> 16) >= c);
    return n;
}

// (key desc, index asc): does (ka, ia) come before (kb, ib)?
__device__ __forceinline__ bool better(uint32_t ka, uint32_t ia, uint32_t kb, uint32_t ib) {
    return ka > kb || (ka == kb && ia < ib);
}

template <int NW>  // 16-bit words per thread: S = 2 * NW * TOPK_THREADS
__global__ __launch_bounds__(TOPK_THREADS) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_topk(TopkArgs a) {
    extern __shared__ uint32_t sm[];
    const int32_t shift = a.shift;
    const uint32_t S = 1u << shift;
    uint32_t* const rec_off = sm + (topk_dummy_off(shift) + TOPK_THREADS * 4) / 4;
    uint32_t* const rec_len = rec_off + TOPK_THREADS;
    uint32_t* const red = rec_len + TOPK_THREADS;
    uint32_t* const cand_k = red + TOPK_RED_WORDS;  // candidates of a segment
    uint32_t* const cand_i = cand_k + TOPK_MAX_K;
    uint32_t* const run_k = cand_i + TOPK_MAX_K;    // running top-K (sorted)
    uint32_t* const run_i = run_k + TOPK_MAX_K;
    uint32_t* const nrun_p = run_i + TOPK_MAX_K;
    uint32_t* const kw = sm + threadIdx.x * NW;     // this thread's counter / key words
    const uint32_t dummy = topk_dummy_off(shift) + threadIdx.x * 4u;
    const uint32_t lane4 = (threadIdx.x & 63u) * 4u;
    const int32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t q = a.q0 + blockIdx.x;
    const uint32_t K = (uint32_t)a.K;
    const int64_t ex = a.exclude_base >= 0 ? a.exclude_base + q : -1;

    uint32_t nrun = 0;  // entries in the running list (uniform)
    uint32_t kmin = 0;  // key of the running K-th entry once the list is full
    for (int32_t s = 0; s < a.nseg; ++s) {
        const uint32_t lo = (uint32_t)s << shift;
        const uint32_t width = (uint32_t)min((int64_t)S, a.N - (int64_t)lo);
        const uint32_t base1 = lo + 1u;
        uint4* c4 = (uint4*)sm;
        for (uint32_t w = threadIdx.x; w < S / 8u; w += TOPK_THREADS) c4[w] = make_uint4(0u, 0u, 0u, 0u);
        sm[dummy >> 2] = 0u;
        for (int32_t tc = 0; tc < a.T; tc += TOPK_THREADS) {
            // the query's bucket records of trees tc .. tc+1023, one per thread
            uint32_t soff, len4;
            query_bucket(a, q, tc + (int32_t)threadIdx.x, s, soff, len4);
            rec_off[threadIdx.x] = soff;
            rec_len[threadIdx.x] = len4;
            __syncthreads();
            const int32_t nt = min(a.T - tc, TOPK_THREADS);
            const int32_t ng = (nt + 15) >> 4;
            const int32_t g0 = (ng * wave) / TOPK_WAVES, g1 = (ng * (wave + 1)) / TOPK_WAVES;
            // two groups in ping-pong: one is counted while the other loads
            uint32_t A[16], B[16];
            bool la = load16(a, rec_off, rec_len, g0, g0 < g1, lane4, A);
            for (int32_t g = g0; g < g1; g += 2) {
                const bool lb = load16(a, rec_off, rec_len, g + 1, g + 1 < g1, lane4, B);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int u = 0; u < 16; ++u) count16(A[u], base1, width, dummy);
                if (la) tails16(a, rec_off, rec_len, g, lane4, base1, width, dummy);
                la = load16(a, rec_off, rec_len, g + 2, g + 2 < g1, lane4, A);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int u = 0; u < 16; ++u) count16(B[u], base1, width, dummy);
                if (lb) tails16(a, rec_off, rec_len, g + 1, lane4, base1, width, dummy);
            }
            __syncthreads();
        }
        // counters -> keys, held in registers from here on: count + 1, or
        // 0 where the reference may not be chosen (past the end, or excluded)
        const uint32_t u0 = threadIdx.x * 2u * NW;
        uint32_t key[NW];
        if constexpr (NW >= 4) {
#pragma unroll
            for (int k = 0; k < NW; k += 4) {
                const uint4 x = *(const uint4*)(kw + k);
                key[k] = x.x;
                key[k + 1] = x.y;
                key[k + 2] = x.z;
                key[k + 3] = x.w;
            }
        } else {
#pragma unroll
            for (int k = 0; k < NW; ++k) key[k] = kw[k];
        }
        // this thread's units u0 + h (h < 2 NW): valid below `rem`, and not the
        // excluded unit `exu` (offsets against constants keep no per-unit
        // index live across the segment loop)
        const int32_t rem = (int32_t)width - (int32_t)u0;
        const int64_t exd = ex - (int64_t)lo - (int64_t)u0;
        const int32_t exu = exd >= 0 && exd < 2 * NW ? (int32_t)exd : -1;
        uint32_t mloc = 0;
#pragma unroll
        for (int k = 0; k < NW; ++k) {
            const uint32_t w = key[k];
            const bool va = 2 * k < rem && 2 * k != exu;
            const bool vb = 2 * k + 1 < rem && 2 * k + 1 != exu;
            const uint32_t ka = va ? (w & 0xffffu) + 1u : 0u;
            const uint32_t kb = vb ? (w >> 16) + 1u : 0u;
            key[k] = ka | (kb << 16);
            mloc = max(mloc, max(ka, kb));
        }
        // only keys above the running threshold can enter the list.  cstar:
        // keys > cstar all enter, keys == cstar in index order up to K; it is
        // the largest c with #(keys >= c) >= K, or `lowest` when fewer than K
        // keys reach `lowest`.  Each round counts four levels at once.
        const uint32_t lowest = max((uint32_t)a.floor_key, nrun == K ? kmin + 1u : 0u);
        uint32_t c0 = lowest, w01, w23, M = mloc;
        level_counts<NW>(key, c0, w01, w23);
        block_levels(w01, w23, M, red);  // also orders the key reads before the next segment's clear
        if (M < lowest) continue;
        uint32_t cstar = lowest;
        if ((w01 & 0xffffu) > K) {
            for (;;) {
                const uint32_t f1 = w01 >> 16, f2 = w23 & 0xffffu, f3 = w23 >> 16;
                const uint32_t d = f3 >= K ? 3u : f2 >= K ? 2u : f1 >= K ? 1u : 0u;
                if (d < 3u || c0 + 3u >= M) {
                    cstar = c0 + d;
                    break;
                }
                c0 += 3u;
                uint32_t m2 = 0;
                level_counts<NW>(key, c0, w01, w23);
                block_levels(w01, w23, m2, red);
            }
        }
        const uint32_t ngt = count_ge<NW>(key, cstar + 1u);
        const uint32_t neq = count_ge<NW>(key, cstar) - ngt;
        uint32_t tot;
        const uint32_t pre = block_excl_scan(ngt | (neq << 16), red, &tot);
        const uint32_t G = tot & 0xffffu, E = tot >> 16;
        const uint32_t take = min(E, K - G);
        uint32_t rg = pre & 0xffffu, re = pre >> 16;
        if (ngt + neq) {
            const uint32_t j0 = lo + u0;
#pragma unroll
            for (int k = 0; k < 2 * NW; ++k) {
                const uint32_t kk = (key[k >> 1] >> (16 * (k & 1))) & 0xffffu;
                const uint32_t j = j0 + (uint32_t)k;
                if (kk > cstar) {
                    cand_k[rg] = kk;
                    cand_i[rg] = j;
                    ++rg;
                } else if (kk == cstar) {
                    if (re < take) {
                        cand_k[G + re] = kk;
                        cand_i[G + re] = j;
                    }
                    ++re;
                }
            }
        }
        __syncthreads();
        // merge by rank (first wave): running entries precede candidates of
        // equal key, since they have lower indices
        const uint32_t nc = G + take;
        if (threadIdx.x < 64) {
            const uint32_t ntot = nrun + nc;
            uint32_t mk[4], mi[4], rk[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t e = threadIdx.x + 64u * r;
                mk[r] = 0u;
                mi[r] = 0xffffffffu;
                if (e < nrun) {
                    mk[r] = run_k[e];
                    mi[r] = run_i[e];
                } else if (e < ntot) {
                    mk[r] = cand_k[e - nrun];
                    mi[r] = cand_i[e - nrun];
                }
                uint32_t rank = 0;
                for (uint32_t f = 0; f < ntot; ++f) {
                    const uint32_t fk = f < nrun ? run_k[f] : cand_k[f - nrun];
                    const uint32_t fi = f < nrun ? run_i[f] : cand_i[f - nrun];
                    rank += better(fk, fi, mk[r], mi[r]) ? 1u : 0u;
                }
                rk[r] = e < ntot ? rank : 0xffffffffu;
            }
            // one wave: its reads of the old list precede these writes
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (rk[r] < K) {
                    run_k[rk[r]] = mk[r];
                    run_i[rk[r]] = mi[r];
                }
            }
            if (threadIdx.x == 0) *nrun_p = min(ntot, K);
        }
        __syncthreads();
        nrun = *nrun_p;
        kmin = nrun ? run_k[nrun - 1] : 0u;
        __syncthreads();
    }
    if (threadIdx.x < K) {
        const bool have = threadIdx.x < nrun;
        a.idx_out[q * K + threadIdx.x] = have ? (int32_t)run_i[threadIdx.x] : -1;
        a.cnt_out[q * K + threadIdx.x] = have ? (uint16_t)(run_k[threadIdx.x] - 1u) : (uint16_t)0;
    }
}

// Queries per launch: gridDim.x * blockDim.x must stay below 2^32.
constexpr int64_t TOPK_MAX_GRID = 1LL << 21;

template <int NW>
static hipError_t launch_topk(rfxp_ctx* ctx, TopkArgs a, int64_t Q) {
    const size_t lds = topk_lds_bytes(a.shift);
    hipError_t e = hipFuncSetAttribute((const void*)k_topk<NW>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    for (int64_t q0 = 0; q0 < Q; q0 += TOPK_MAX_GRID) {
        a.q0 = q0;
        const unsigned nq = (unsigned)std::min(TOPK_MAX_GRID, Q - q0);
        hipLaunchKernelGGL(k_topk<NW>, dim3(nq), dim3(TOPK_THREADS), lds, ctx->stream, a);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace rfxp

using namespace rfxp;

extern "C" int rfxp_set_reference(rfxp_ctx* ctx, const int32_t* leaf, int64_t stride_i, int64_t stride_t, int64_t N,
                                  int32_t T, int32_t nleaf) {
    if (!ctx) return RFXP_ERR_INVALID;
    ctx->ref_ready = false;
    if (N < 1 || T < 1 || T > 65534 || nleaf < 1)
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_set_reference: need N >= 1, 1 <= T <= 65534, nleaf >= 1");
    if (!leaf || !is_device_pointer(leaf))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_set_reference: leaf must be a device pointer");
    if (N * (int64_t)T + MEM_PAD > (1LL << 30) - 1)
        return set_error(ctx, RFXP_ERR_UNSUPPORTED, "rfxp_set_reference: N*T must stay below 2^30");
    int32_t shift = TOPK_MIN_SHIFT;
    while (shift < TOPK_MAX_SHIFT && (1LL << shift) < N) ++shift;
    const int64_t nseg = (N + (1LL << shift) - 1) >> shift;
    if ((int64_t)nleaf * nseg > (1LL << 29))
        return set_error(ctx, RFXP_ERR_UNSUPPORTED, "rfxp_set_reference: nleaf * segments too large");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    LeafView v{leaf, stride_i, stride_t, nullptr, 0, N, T, nleaf, (int32_t)nseg, shift};
    const int32_t nb = view_buckets(v);
    const ForestSizes z = forest_sizes(v, false, ctx->max_lds);
    ForestBufs fb;
    if (int rc = ctx_forest_bufs(ctx, z, ctx->ref_off, ctx->ref_mem, fb)) return rc;
    if (int rc = pack_forest(ctx, v, nullptr, fb)) return rc;
    ctx->ref_N = N;
    ctx->ref_T = T;
    ctx->ref_L = nleaf;
    ctx->ref_nseg = (int32_t)nseg;
    ctx->ref_shift = shift;
    ctx->ref_nb = nb;
    ctx->ref_leaf = leaf;
    ctx->ref_si = stride_i;
    ctx->ref_st = stride_t;
    ctx->lr_index_ready = false;
    ctx->ref_ready = true;
    return RFXP_OK;
}

extern "C" int rfxp_topk(rfxp_ctx* ctx, const int32_t* q_leaf, int64_t q_stride_i, int64_t q_stride_t, int64_t Q,
                         const uint32_t* q_oob_words, int64_t q_oob_ld, int64_t exclude_base, int32_t K,
                         int positive_only, int32_t* idx_out, uint16_t* cnt_out) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (!ctx->ref_ready) return set_error(ctx, RFXP_ERR_STATE, "rfxp_topk: no reference set");
    if (Q < 0 || K < 1) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_topk: need Q >= 0, K >= 1");
    if (K > TOPK_MAX_K) return set_error(ctx, RFXP_ERR_UNSUPPORTED, "rfxp_topk: K above 64 is not supported");
    if (Q == 0) return RFXP_OK;
    if (Q > 0x7fffffffLL) return set_error(ctx, RFXP_ERR_UNSUPPORTED, "rfxp_topk: too many queries");
    if (!q_leaf || !idx_out || !cnt_out || !is_device_pointer(q_leaf) || !is_device_pointer(idx_out) ||
        !is_device_pointer(cnt_out) || (q_oob_words && !is_device_pointer(q_oob_words)))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_topk: pointers must be device pointers");
    if (q_oob_words && q_oob_ld < (Q + 31) / 32)
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_topk: q_oob_ld < ceil(Q/32)");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    TopkArgs a;
    a.mem = ctx->ref_mem.p;
    a.mem_bytes = (uint32_t)(((uint64_t)ctx->ref_T * (uint64_t)ctx->ref_N + MEM_PAD) * 4u);
    a.off = ctx->ref_off.p;
    a.nb = ctx->ref_nb;
    a.N = ctx->ref_N;
    a.T = ctx->ref_T;
    a.L = ctx->ref_L;
    a.nseg = ctx->ref_nseg;
    a.shift = ctx->ref_shift;
    a.qleaf = q_leaf;
    a.qsi = q_stride_i;
    a.qst = q_stride_t;
    a.qoob = q_oob_words;
    a.qold = q_oob_ld;
    a.exclude_base = exclude_base;
    a.K = K;
    a.floor_key = positive_only ? 2 : 1;
    a.idx_out = idx_out;
    a.cnt_out = cnt_out;
    hipError_t e;
    {
        LaunchTimer tm(ctx, "topk");
        switch (a.shift) {
            case 11: e = launch_topk<1>(ctx, a, Q); break;
            case 12: e = launch_topk<2>(ctx, a, Q); break;
            case 13: e = launch_topk<4>(ctx, a, Q); break;
            case 14: e = launch_topk<8>(ctx, a, Q); break;
            default: e = launch_topk<16>(ctx, a, Q); break;
        }
    }
    if (e != hipSuccess) return hip_error(ctx, e, "k_topk launch");
    return RFXP_OK;
}
