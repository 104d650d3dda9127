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
// Kernels k_topk (16-bit counters) and k_topk8 (8-bit counters): a
// workgroup takes one query at a time (about one workgroup per resident
// slot, looping over the queries) and walks its segments in order.  Per
// segment, LDS counters (one per reference of the segment) take the query's
// T buckets exactly as the triangle's hit phase does; then the counts become
// keys (count + 1, 0 for references that may not be chosen) and only keys
// above the running K-th best key are looked at: entries of a later segment
// lose every tie against the running list, which holds lower indices.
// Selection is exact: the keys at or above the threshold when at most K
// reach it, else a search over key levels for the K-th key, ordered
// compaction of the winners, and a rank merge with the running list by one
// wave.
#include <algorithm>
#include <cmath>
#include <string>
#include <vector>

#include "rfxp_device.hpp"
#include "rfxp_forest.hpp"
#include "rfxp_internal.hpp"

namespace rfxp {

constexpr int TOPK_THREADS = 1024;
constexpr int TOPK_WAVES = TOPK_THREADS / 64;
constexpr int TOPK_MAX_K = 64;
constexpr int TOPK_MAX_SHIFT16 = 15;  // 32768 16-bit counters: 64 KB, two workgroups per CU
constexpr int TOPK_SHIFT8 = 16;       // 65536 8-bit counters: 64 KB (top-K with T <= TOPK_MAX_T8)
constexpr int TOPK_MAX_SHIFT8 = 17;   // 131072 8-bit counters: 128 KB, one workgroup per CU
constexpr uint32_t TOPK_BLOCK = 32768;  // references selected at once (32 units per thread)
constexpr int TOPK_MAX_T8 = 2048;     // at most 128 trees, 128 counting steps, per wave and segment
constexpr int TOPK_MIN_SHIFT = 11;  // at least 2 counters per thread

struct TopkArgs {
    const uint32_t* mem;  // reference members (j + 1), [T][N]
    const int32_t* off;   // [T][nb + 1]
    int32_t nb;
    int64_t N;
    int32_t T, L, nseg, shift;
    const int32_t* qleaf;
    int64_t qsi, qst;
    const uint32_t* qoob;  // NULL: all trees
    int64_t qold;
    int64_t exclude_base;  // query q excludes reference exclude_base + q; < 0: none
    const int32_t* exclude_idx;  // or, when not NULL, reference exclude_idx[q] (< 0: none)
    int64_t q0;            // query of workgroup 0 of this launch
    int64_t q1;            // end of this launch's queries (top-K kernels loop over them)
    int32_t K;
    int32_t floor_key;     // smallest selectable key: 1 (zeros allowed) or 2 (counts > 0)
    int32_t* idx_out;
    uint16_t* cnt_out;
};

// LDS layout: counters (2^shift 16-bit counters, shift <= 15, or 2^shift
// 8-bit ones, shift 16 or 17) | dummy words (1024) | reduction scratch |
// candidate and running lists.
__host__ __device__ constexpr uint32_t topk_dummy_off(int32_t shift) {
    return shift >= TOPK_SHIFT8 ? (1u << shift) : (1u << shift) * 2u;
}
// wave partials (48), two segment slots (2 x 80: five words per wave), a
// selection slot (16)
constexpr uint32_t TOPK_RED_WORDS = 224;
constexpr uint32_t TOPK_LIST_WORDS = 4 * TOPK_MAX_K + 8;    // candidate / running lists
__host__ __device__ constexpr uint32_t topk_lds_bytes(int32_t shift) {
    return topk_dummy_off(shift) + (TOPK_THREADS + TOPK_RED_WORDS + TOPK_LIST_WORDS) * 4;
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

// Counting step of a query run with BITS-bit counters (8 or 16): m = j + 1
// of a member (0: an empty lane), counter unit c = j - lo.  Units at or past
// xlim -- empty lanes, and members outside the units being counted -- are
// clamped to xlim, the unit of byte 0 of this thread's dummy word, which
// sits after the counters with the other threads' dummy words; units between
// the counters and xlim fall on those.  (A run holds only members of its
// segment, lo <= j < lo + 2^shift, so a member never lands on a counter
// past the segment's references.)
template <int BITS>
__device__ __forceinline__ void count_bits(uint32_t m, uint32_t base1, uint32_t xlim) {
    const uint32_t c = min(m - base1, xlim);
    if constexpr (BITS == 8) lds_add16(c & ~3u, 1u << ((c << 3) & 31u));
    else lds_add16((c << 1) & ~3u, 1u << ((c << 4) & 31u));
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

// The reference query q may not return (< 0: none).
__device__ __forceinline__ int64_t query_exclusion(const TopkArgs& a, int64_t q) {
    if (a.exclude_idx) return a.exclude_idx[q];
    return a.exclude_base >= 0 ? a.exclude_base + q : -1;
}

// (key desc, index asc): does (ka, ia) come before (kb, ib)?
__device__ __forceinline__ bool better(uint32_t ka, uint32_t ia, uint32_t kb, uint32_t ib) {
    return ka > kb || (ka == kb && ia < ib);
}

// A wave's bucket runs of one segment, counted into the LDS counters
// (BITS 8 or 16).  Lane l holds the run (byte offset soff, byte length len4
// <= 256: at most 64 ids, count_runs_chunked cuts longer runs) of the wave's
// l-th tree or chunk; n_trees (<= 64, uniform) lanes hold one.  The runs are
// loaded sixteen at a time, two groups in flight.  Returns the wave's 64-lane
// counting steps (uniform): every lane of a step adds 1 to one counter or
// dummy byte.
template <int BITS>
__device__ __forceinline__ uint32_t count_lane_runs(const TopkArgs& a, uint32_t soff, uint32_t len4,
                                                    int32_t n_trees, uint32_t lane4, uint32_t base1, uint32_t dummy) {
    const uint32_t xlim = BITS == 8 ? dummy : dummy >> 1;
    const int32_t ng = (n_trees + 15) >> 4;
    if (ng == 0) return 0u;
    uint32_t A[16], B[16];
    auto load = [&](int32_t g, uint32_t (&m)[16]) {
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const uint32_t so = (uint32_t)__builtin_amdgcn_readlane((int)soff, 16 * g + u);
            const uint32_t ln = (uint32_t)__builtin_amdgcn_readlane((int)len4, 16 * g + u);
            // non-temporal (cache policy nt): a run is read once per query;
            // streaming the runs keeps the offset rows, reread every segment,
            // in L2
            m[u] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(ref_rsrc(a.mem, so + ln), lane4, so, 2);
        }
    };
    load(0, A);
    if (ng > 1) load(1, B);
    for (int32_t g = 0;; g += 2) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 16; ++u) count_bits<BITS>(A[u], base1, xlim);
        if (g + 2 < ng) load(g + 2, A);
        if (g + 1 >= ng) break;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 16; ++u) count_bits<BITS>(B[u], base1, xlim);
        if (g + 3 < ng) load(g + 3, B);
        if (g + 2 >= ng) break;
    }
    return 16u * (uint32_t)ng;
}

// Packed maximum of the two 16-bit halves of a and b.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t max_u16x2(uint32_t a, uint32_t b) {
    const u16x2 m = __builtin_elementwise_max(__builtin_bit_cast(u16x2, a), __builtin_bit_cast(u16x2, b));
    return __builtin_bit_cast(uint32_t, m);
}

// LDS pointers of a top-K workgroup.
struct TopkLds {
    uint32_t* red;     // reduction scratch (TOPK_RED_WORDS)
    uint32_t* cand_k;  // candidates of a segment
    uint32_t* cand_i;
    uint32_t* run_k;   // running top-K (sorted)
    uint32_t* run_i;
};

__device__ __forceinline__ TopkLds topk_lds(uint32_t* sm, int32_t shift) {
    TopkLds L;
    L.red = sm + (topk_dummy_off(shift) + TOPK_THREADS * 4) / 4;
    L.cand_k = L.red + TOPK_RED_WORDS;
    L.cand_i = L.cand_k + TOPK_MAX_K;
    L.run_k = L.cand_i + TOPK_MAX_K;
    L.run_i = L.run_k + TOPK_MAX_K;
    return L;
}

// Keys of a thread's 2 NW units u0 .. u0 + 2 NW - 1 (relative to the
// segment start) from their 16-bit counts, two per word: count + 1, or 0
// where the reference may not be chosen (at or past `rem`, or the excluded
// unit `exu`).  Returns the thread's largest key.
template <int NW>
__device__ __forceinline__ uint32_t keys_of_counts(uint32_t (&key)[NW], int32_t rem, int32_t exu) {
    uint32_t mloc = 0;
    if (rem >= 2 * NW && exu < 0) {
        // every unit valid: key = count + 1 in both halves (counts stay
        // below 65535, so no half carries into the other)
        uint32_t m2 = 0u;
#pragma unroll
        for (int k = 0; k < NW; ++k) {
            key[k] += 0x00010001u;
            m2 = max_u16x2(m2, key[k]);
        }
        mloc = max(m2 & 0xffffu, m2 >> 16);
    } else {
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
    }
    return mloc;
}

// Block maximum of v through 16 words of `slot`; one barrier.  A slot may be
// reused only after a later barrier.
__device__ __forceinline__ uint32_t block_max(uint32_t v, uint32_t* slot) {
    const uint32_t wm = wave_max(v);
    if ((threadIdx.x & 63) == 0) slot[threadIdx.x >> 6] = wm;
    __syncthreads();
    return wave_max((threadIdx.x & 63u) < (uint32_t)TOPK_WAVES ? slot[threadIdx.x & 63u] : 0u);
}

// Exclusive prefix over the lanes of a wave of n < 64, bit by bit from
// ballots (mbcnt counts the set lanes below this one).
__device__ __forceinline__ uint32_t wave_excl_prefix6(uint32_t n) {
    uint32_t pre = 0;
#pragma unroll
    for (int b = 0; b < 6; ++b) {
        const uint64_t m = __ballot((n >> b) & 1u);
        pre += __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u)) << b;
    }
    return pre;
}

// Block total of n (< 2^16 per thread) and the total of the waves before
// this one, through 16 words of the selection slot; one barrier.
__device__ __forceinline__ void block_count(uint32_t n, const TopkLds& L, uint32_t& tot, uint32_t& wpre) {
    uint32_t* const slot = L.red + TOPK_RED_WORDS - 16;
    const uint32_t ws = wave_sum(n);
    if ((threadIdx.x & 63) == 0) slot[threadIdx.x >> 6] = ws;
    __syncthreads();
    const uint32_t l = threadIdx.x & 63u;
    const uint32_t x = l < (uint32_t)TOPK_WAVES ? slot[l] : 0u;
    tot = wave_sum(x);
    wpre = wave_sum(l < (threadIdx.x >> 6) ? x : 0u);
}

// More than K keys reach `lowest`: cstar is the largest c with
// #(keys >= c) >= K, found by a search over key levels from the top (four
// per round, M bounding the largest key, so that keys above the first
// round's levels number fewer than K); keys > cstar become candidates, and
// keys == cstar in index order up to K.  Returns the candidate count; ends with a
// barrier.  Keys are read only in waves with wlive set.
template <int NW>
__device__ __forceinline__ uint32_t select_search(const TopkArgs& a, const uint32_t (&key)[NW], bool wlive,
                                                  uint32_t M, uint32_t lowest, uint32_t j0, const TopkLds& L) {
    const uint32_t K = (uint32_t)a.K;
    uint32_t* const red = L.red;
    // levels c0 .. c0 + 3 per round, from the top (c0 = M - 3) down by four
    // while fewer than K keys reach c0; at c0 == lowest at least K do
    uint32_t c0 = M >= lowest + 3u ? M - 3u : lowest;
    uint32_t cstar;
    for (;;) {
        uint32_t w01 = 0u, w23 = 0u, m1 = 0u;
        if (wlive) level_counts<NW>(key, c0, w01, w23);
        block_levels(w01, w23, m1, red);
        const uint32_t f0 = w01 & 0xffffu, f1 = w01 >> 16, f2 = w23 & 0xffffu, f3 = w23 >> 16;
        if (f0 >= K || c0 == lowest) {
            cstar = c0 + (f3 >= K ? 3u : f2 >= K ? 2u : f1 >= K ? 1u : 0u);
            break;
        }
        c0 = c0 >= lowest + 4u ? c0 - 4u : lowest;
    }
    uint32_t ngt = 0u, neq = 0u;
    if (wlive) {
        ngt = count_ge<NW>(key, cstar + 1u);
        neq = count_ge<NW>(key, cstar) - ngt;
    }
    uint32_t tot;
    const uint32_t pre = block_excl_scan(ngt | (neq << 16), red, &tot);
    const uint32_t G = tot & 0xffffu, E = tot >> 16;
    const uint32_t take = min(E, K - G);
    uint32_t rg = pre & 0xffffu, re = pre >> 16;
    if (ngt + neq) {
#pragma unroll
        for (int k = 0; k < 2 * NW; ++k) {
            const uint32_t kk = (key[k >> 1] >> (16 * (k & 1))) & 0xffffu;
            const uint32_t j = j0 + (uint32_t)k;
            if (kk > cstar) {
                L.cand_k[rg] = kk;
                L.cand_i[rg] = j;
                ++rg;
            } else if (kk == cstar) {
                if (re < take) {
                    L.cand_k[G + re] = kk;
                    L.cand_i[G + re] = j;
                }
                ++re;
            }
        }
    }
    __syncthreads();
    return G + take;
}

// Merges the nc candidates (in LDS, any order) into the running list by
// rank (first wave; nrun, nc <= K <= 64, lane e holds running entry e and
// candidate e, and reads the others' with readlane).  The running list is
// sorted; candidates have higher indices than every running entry, so a
// running entry keeps its place among running entries and precedes
// candidates of equal key.  Ends with nrun / kmin updated.  The LDS a
// selection writes (reduction slots, candidate and running lists) is next
// written after the first barrier of the next selection, which every thread
// reaches only after its reads here, so no closing barrier is needed.
__device__ __forceinline__ void merge_candidates(const TopkArgs& a, uint32_t nc, const TopkLds& L, uint32_t& nrun,
                                                 uint32_t& kmin) {
    const uint32_t K = (uint32_t)a.K;
    if (threadIdx.x < 64) {
        const uint32_t e = threadIdx.x;
        const bool has_r = e < nrun, has_c = e < nc;
        const uint32_t rk = has_r ? L.run_k[e] : 0u, ri = has_r ? L.run_i[e] : 0u;
        const uint32_t ck = has_c ? L.cand_k[e] : 0u, ci = has_c ? L.cand_i[e] : 0xffffffffu;
        uint32_t rank_r = e, rank_c = 0u;
        for (uint32_t c = 0; c < nc; ++c) {
            const uint32_t fk = (uint32_t)__builtin_amdgcn_readlane((int)ck, (int)c);
            const uint32_t fi = (uint32_t)__builtin_amdgcn_readlane((int)ci, (int)c);
            rank_r += fk > rk ? 1u : 0u;
            rank_c += better(fk, fi, ck, ci) ? 1u : 0u;
        }
        for (uint32_t f = 0; f < nrun; ++f)
            rank_c += (uint32_t)__builtin_amdgcn_readlane((int)rk, (int)f) >= ck ? 1u : 0u;
        // one wave: its reads of the old list precede these writes
        if (has_r && rank_r < K) {
            L.run_k[rank_r] = rk;
            L.run_i[rank_r] = ri;
        }
        if (has_c && rank_c < K) {
            L.run_k[rank_c] = ck;
            L.run_i[rank_c] = ci;
        }
    }
    __syncthreads();
    nrun = min(nrun + nc, K);
    kmin = nrun ? L.run_k[nrun - 1] : 0u;
}

// Merges the keys of one segment (thread x: units lo + u0 .. of key[NW],
// u0 = 2 NW x) into the running list; M is the block's largest key (or an
// upper bound of it), at least `lowest` (the smallest key that can still
// enter); tmax is this thread's largest key.  Keys are read only in waves
// where some tmax reaches `lowest`: a wave without such a key skips every
// pass over them.  Usually (always once the list is full) at most K keys
// reach `lowest` and they all enter, in slots of thread order; otherwise
// select_search picks them.  Every thread calls it; it ends with nrun / kmin
// updated.
template <int NW>
__device__ __forceinline__ void select_into(const TopkArgs& a, const uint32_t (&key)[NW], uint32_t tmax, uint32_t M,
                                            uint32_t lowest, uint32_t lo, uint32_t u0, const TopkLds& L,
                                            uint32_t& nrun, uint32_t& kmin) {
    const uint32_t K = (uint32_t)a.K;
    const bool wlive = __ballot(tmax >= lowest) != 0ull;  // uniform
    const uint32_t j0 = lo + u0;
    uint32_t n = 0;  // this thread's keys >= lowest
    if (wlive) n = count_ge<NW>(key, lowest);
    uint32_t tot, wpre;
    block_count(n, L, tot, wpre);
    uint32_t nc = tot;
    if (tot <= K) {
        if (wlive) {
            uint32_t r = wpre + wave_excl_prefix6(n);
            if (n) {
#pragma unroll
                for (int k = 0; k < 2 * NW; ++k) {
                    const uint32_t kk = (key[k >> 1] >> (16 * (k & 1))) & 0xffffu;
                    if (kk >= lowest) {
                        L.cand_k[r] = kk;
                        L.cand_i[r] = j0 + (uint32_t)k;
                        ++r;
                    }
                }
            }
        }
        __syncthreads();
    } else {
        nc = select_search<NW>(a, key, wlive, M, lowest, j0, L);
    }
    merge_candidates(a, nc, L, nrun, kmin);
}

// Byte flags (bit 7 of each byte) of the bytes of w that are >= t (t <= 255).
__device__ __forceinline__ uint32_t bytes_ge(uint32_t w, uint32_t t) {
    const uint32_t hi = w & 0x80808080u, lo7 = w & 0x7f7f7f7fu;
    return t <= 128u ? hi | ((lo7 + (128u - t) * 0x01010101u) & 0x80808080u)
                     : hi & (lo7 + (256u - t) * 0x01010101u);
}

// select_into for the 8-bit counters of one block: thread x's 32 counts,
// units lo + u0 + 4k + b in byte b of w8[k] (read only in waves with wlive
// set), key = count + 1; units at or past rem, and unit exu, may not be
// chosen.  The counts are tested against the threshold four at a time, and
// only the flagged bytes are visited; when more than K keys reach `lowest`,
// 16-bit keys are formed for select_search.
__device__ __forceinline__ void select_bytes(const TopkArgs& a, const uint32_t (&w8)[8], bool wlive, int32_t rem,
                                             int32_t exu, uint32_t M, uint32_t lowest, uint32_t lo, uint32_t u0,
                                             const TopkLds& L, uint32_t& nrun, uint32_t& kmin) {
    const uint32_t K = (uint32_t)a.K;
    const uint32_t j0 = lo + u0;
    uint32_t f8[8];
    uint32_t n = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) f8[k] = 0u;
    if (wlive) {
        // lowest <= M <= 256 here, so the count threshold is at most 255
        const uint32_t t = lowest - 1u;
#pragma unroll
        for (int k = 0; k < 8; ++k) f8[k] = bytes_ge(w8[k], t);
        if (rem < 32 || exu >= 0) {
#pragma unroll
            for (int k = 0; k < 8; ++k)
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    if (4 * k + b >= rem || 4 * k + b == exu) f8[k] &= ~(0x80u << (8 * b));
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) n += (uint32_t)__popc(f8[k]);
    }
    uint32_t tot, wpre;
    block_count(n, L, tot, wpre);
    uint32_t nc = tot;
    if (tot <= K) {
        if (n) {
            // lanes with n = 0 are inactive here and add no ballot bits
            uint32_t r = wpre + wave_excl_prefix6(n);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                uint32_t f = f8[k];
                while (f) {
                    const uint32_t sh = (uint32_t)__builtin_ctz(f) - 7u;  // 8 * byte index
                    L.cand_k[r] = ((w8[k] >> sh) & 0xffu) + 1u;
                    L.cand_i[r] = j0 + 4u * (uint32_t)k + (sh >> 3);
                    ++r;
                    f &= f - 1u;
                }
            }
        }
        __syncthreads();
    } else {
        uint32_t key[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) key[k] = 0u;
        if (wlive) {
#pragma unroll
            for (int k = 0; k < 16; ++k)
                key[k] = __builtin_amdgcn_perm(0u, w8[k >> 1], (k & 1) ? 0x0c030c02u : 0x0c010c00u);
            keys_of_counts<16>(key, rem, exu);
        }
        nc = select_search<16>(a, key, wlive, M, lowest, j0, L);
    }
    merge_candidates(a, nc, L, nrun, kmin);
}

// Per-lane bucket runs of a query.  The wave's trees are [tw0, tw1); lane l
// holds tree tw0 + l.  The lane's offset-row entries of segments s, s + 1,
// s + 2 are kept in o0, o1, o2, the last one loaded a segment ahead, so a
// segment's runs need no dependent load.  Trees past the first 64 of a
// wave (T > 1024) are looked up per segment.
struct LaneRuns {
    int64_t ob;   // offset-row index of the lane tree's bucket in segment 0 (-1: none)
    uint32_t tb;  // byte offset of the lane tree's members in mem
    uint32_t o0, o1, o2;
};

__device__ __forceinline__ LaneRuns lane_runs_init(const TopkArgs& a, int64_t q, int32_t tw0, int32_t tw1,
                                                   int32_t lane) {
    LaneRuns r{-1, 0u, 0u, 0u, 0u};
    if (lane < tw1 - tw0) {
        const int32_t t = tw0 + lane;
        const int32_t l = a.qleaf[q * a.qsi + (int64_t)t * a.qst];
        bool ok = l >= 0 && l < a.L;
        if (ok && a.qoob) ok = ((a.qoob[(int64_t)t * a.qold + (q >> 5)] >> (q & 31)) & 1u) != 0u;
        if (ok) {
            r.ob = (int64_t)t * (a.nb + 1) + (int64_t)l * a.nseg;
            r.tb = 4u * (uint32_t)t * (uint32_t)a.N;
            r.o0 = (uint32_t)a.off[r.ob];
            r.o1 = (uint32_t)a.off[r.ob + 1];
            r.o2 = a.nseg >= 2 ? (uint32_t)a.off[r.ob + 2] : r.o1;
        }
    }
    return r;
}

// A wave's runs (lanes < nt, as in count_lane_runs; lanes >= nt hold empty
// runs) cut into chunks of at most 64 ids, all of them counted through the
// load pipeline of count_lane_runs, 64 chunks per call: a run of thousands
// of ids (a popular leaf) costs its chunks' loads, overlapped like any other
// run's, rather than a chain of dependent loads.  Chunk g of the wave belongs
// to the first lane whose inclusive chunk prefix exceeds g.
template <int BITS>
__device__ __forceinline__ uint32_t count_runs_chunked(const TopkArgs& a, uint32_t soff, uint32_t len4, int32_t nt,
                                                       int32_t lane, uint32_t lane4, uint32_t base1, uint32_t dummy) {
    if (__ballot(len4 > 256u) == 0ull) return count_lane_runs<BITS>(a, soff, len4, nt, lane4, base1, dummy);
    const uint32_t c = (len4 + 255u) >> 8;  // chunks of this lane's run
    uint32_t incl = c;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t o = (uint32_t)__shfl_up((int)incl, d, 64);
        if (lane >= d) incl += o;
    }
    const uint32_t total = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
    uint32_t steps = 0;
    for (uint32_t g0 = 0; g0 < total; g0 += 64u) {
        const uint32_t g = g0 + (uint32_t)lane;
        int32_t lo = 0, hi = 63;
#pragma unroll
        for (int it = 0; it < 6; ++it) {
            const int32_t mid = (lo + hi) >> 1;
            if ((uint32_t)__shfl((int)incl, mid, 64) > g) hi = mid;
            else lo = mid + 1;
        }
        lo = min(lo, 63);
        const uint32_t m = g - ((uint32_t)__shfl((int)incl, lo, 64) - (uint32_t)__shfl((int)c, lo, 64));
        const uint32_t so_r = (uint32_t)__shfl((int)soff, lo, 64), ln_r = (uint32_t)__shfl((int)len4, lo, 64);
        const bool ok = g < total;
        const uint32_t so = ok ? so_r + 256u * m : 0u;
        const uint32_t ln = ok ? min(ln_r - 256u * m, 256u) : 0u;
        steps += count_lane_runs<BITS>(a, so, ln, (int32_t)min(total - g0, 64u), lane4, base1, dummy);
    }
    return steps;
}

// Counts the query's runs of segment s into the BITS-bit counters (member j
// at unit j + 1 - base1; the counters end where the dummy words begin);
// returns the wave's counting steps.
template <int BITS>
__device__ __forceinline__ uint32_t count_query_segment(const TopkArgs& a, int64_t q, int32_t s, uint32_t soff,
                                                        uint32_t len4, int32_t tw0, int32_t tw1, int32_t lane,
                                                        uint32_t lane4, uint32_t base1, uint32_t dummy) {
    uint32_t steps = count_runs_chunked<BITS>(a, soff, len4, min(tw1 - tw0, 64), lane, lane4, base1, dummy);
    for (int32_t r0 = tw0 + 64; r0 < tw1; r0 += 64) {
        uint32_t so2, ln2;
        query_bucket(a, q, r0 + lane < tw1 ? r0 + lane : a.T, s, so2, ln2);
        steps += count_runs_chunked<BITS>(a, so2, ln2, min(tw1 - r0, 64), lane, lane4, base1, dummy);
    }
    return steps;
}

__device__ __forceinline__ void topk_write(const TopkArgs& a, int64_t q, const TopkLds& L, uint32_t nrun) {
    if (threadIdx.x < (uint32_t)a.K) {
        const bool have = threadIdx.x < nrun;
        a.idx_out[q * a.K + threadIdx.x] = have ? (int32_t)L.run_i[threadIdx.x] : -1;
        a.cnt_out[q * a.K + threadIdx.x] = have ? (uint16_t)(L.run_k[threadIdx.x] - 1u) : (uint16_t)0;
    }
}

// 16-bit counters, S = 2^shift = 2 NW * TOPK_THREADS references per segment
// (reference sets of up to 32768 samples, or more than TOPK_MAX_T8 trees).
template <int NW>
__global__ __launch_bounds__(TOPK_THREADS) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_topk(TopkArgs a) {
    extern __shared__ uint32_t sm[];
    const int32_t shift = a.shift;
    const uint32_t S = 1u << shift;
    const TopkLds L = topk_lds(sm, shift);
    uint32_t* const kw = sm + threadIdx.x * NW;  // this thread's counter / key words
    const uint32_t dummy = topk_dummy_off(shift) + threadIdx.x * 4u;
    const uint32_t lane4 = (threadIdx.x & 63u) * 4u;
    const int32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int32_t lane = (int32_t)(threadIdx.x & 63u);
    const uint32_t K = (uint32_t)a.K;
    const int32_t tw0 = (int32_t)(((int64_t)a.T * wave) / TOPK_WAVES);
    const int32_t tw1 = (int32_t)(((int64_t)a.T * (wave + 1)) / TOPK_WAVES);
    // counters start at zero; afterwards each thread zeroes its own words as
    // it reads them
    {
        uint4* c4 = (uint4*)sm;
        for (uint32_t w = threadIdx.x; w < S / 8u; w += TOPK_THREADS) c4[w] = make_uint4(0u, 0u, 0u, 0u);
    }
    __syncthreads();

    // queries q0 + blockIdx.x, + gridDim.x, ... below q1: about one workgroup
    // per resident slot, so no workgroup starts or clears its counters per
    // query (they are zero again after every segment)
    for (int64_t q = a.q0 + blockIdx.x; q < a.q1; q += gridDim.x) {
        const int64_t ex = query_exclusion(a, q);
        LaneRuns lr = lane_runs_init(a, q, tw0, tw1, lane);
        uint32_t nrun = 0;  // entries in the running list (uniform)
        uint32_t kmin = 0;  // key of the running K-th entry once the list is full
        for (int32_t s = 0; s < a.nseg; ++s) {
            const uint32_t lo = (uint32_t)s << shift;
            const uint32_t width = (uint32_t)min((int64_t)S, a.N - (int64_t)lo);
            const uint32_t soff = lr.tb + 4u * lr.o0;
            const uint32_t len4 = 4u * (lr.o1 - lr.o0);
            const uint32_t o3 = (lr.ob >= 0 && s + 3 <= a.nseg) ? (uint32_t)a.off[lr.ob + s + 3] : lr.o2;
            count_query_segment<16>(a, q, s, soff, len4, tw0, tw1, lane, lane4, lo + 1u, dummy);
            lr.o0 = lr.o1;
            lr.o1 = lr.o2;
            lr.o2 = o3;
            __syncthreads();  // every count is in LDS
            // counters -> keys, held in registers from here on; the counter
            // words are zeroed for the next segment
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
                    *(uint4*)(kw + k) = make_uint4(0u, 0u, 0u, 0u);
                }
            } else {
#pragma unroll
                for (int k = 0; k < NW; ++k) {
                    key[k] = kw[k];
                    kw[k] = 0u;
                }
            }
            // this thread's units u0 + h (h < 2 NW): valid below `rem`, and not the
            // excluded unit `exu`
            const int32_t rem = (int32_t)width - (int32_t)u0;
            const int64_t exd = ex - (int64_t)lo - (int64_t)u0;
            const int32_t exu = exd >= 0 && exd < 2 * NW ? (int32_t)exd : -1;
            const uint32_t mloc = keys_of_counts<NW>(key, rem, exu);
            // the segment's largest key; the barrier also orders every zeroing
            // before the next segment's counts (two alternating slots)
            const uint32_t M = block_max(mloc, L.red + 48 + 16 * (s & 1));
            const uint32_t lowest = max((uint32_t)a.floor_key, nrun == K ? kmin + 1u : 0u);
            if (M < lowest) continue;
            select_into<NW>(a, key, mloc, M, lowest, lo, u0, L, nrun, kmin);
        }
        topk_write(a, q, L, nrun);
    }
}

// 8-bit counters, NB blocks of TOPK_BLOCK = 32768 references per segment
// (S = 65536 for reference sets of up to 65536 samples, two workgroups per
// CU; S = 131072 above, one workgroup per CU), T <= TOPK_MAX_T8: a quarter
// of the bucket runs per query that 16-bit counters allow in 64 KB of LDS,
// and runs long enough to fill most of a 64-lane load.  Thread x reads the
// counter bytes of units 32x .. 32x + 31 of each block h (units
// h * 32768 + ...), so each block is selected exactly like a 16-bit segment
// of 32768 references, in index order.  CHECK (T > 255): a count of 256 or
// more wraps its byte; every lane of every counting step adds 1 to one
// counter byte or to byte 0 of its thread's dummy word (empty lanes), so the
// counts are exact iff the counter bytes plus the dummy words (plain counts,
// read as integers so that many empty steps cannot look like a wrap) sum to
// 64 x the counting steps.  A segment that fails the check is recounted with
// 16-bit counters, block by block.
template <bool CHECK, int NB>
__global__ __launch_bounds__(TOPK_THREADS) __attribute__((amdgpu_waves_per_eu(16 / NB, 16 / NB))) void k_topk8(
    TopkArgs a) {
    static_assert(NB == 2 || NB == 4, "two or four blocks per segment");
    extern __shared__ uint32_t sm[];
    constexpr int32_t SHIFT = NB == 2 ? TOPK_SHIFT8 : TOPK_SHIFT8 + 1;
    constexpr uint32_t S = 1u << SHIFT;
    constexpr uint32_t B = TOPK_BLOCK;
    static_assert(S == NB * B, "segment = NB blocks");
    const TopkLds L = topk_lds(sm, SHIFT);
    uint32_t* const dw = sm + (topk_dummy_off(SHIFT) >> 2) + threadIdx.x;  // this thread's dummy word
    const uint32_t dummy = topk_dummy_off(SHIFT) + threadIdx.x * 4u;
    // the 16-bit recount of a block counts into bytes 0 .. 2B - 1; its
    // out-of-block members go to the words 2B/4 + x (x < 1024) right after
    const uint32_t dummy16 = 2u * B + threadIdx.x * 4u;
    const uint32_t lane4 = (threadIdx.x & 63u) * 4u;
    const int32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int32_t lane = (int32_t)(threadIdx.x & 63u);
    const uint32_t K = (uint32_t)a.K;
    const int32_t tw0 = (int32_t)(((int64_t)a.T * wave) / TOPK_WAVES);
    const int32_t tw1 = (int32_t)(((int64_t)a.T * (wave + 1)) / TOPK_WAVES);
    {
        uint4* c4 = (uint4*)sm;
        for (uint32_t w = threadIdx.x; w < S / 16u; w += TOPK_THREADS) c4[w] = make_uint4(0u, 0u, 0u, 0u);
        *dw = 0u;
    }
    __syncthreads();

    // queries q0 + blockIdx.x, + gridDim.x, ... below q1: about one workgroup
    // per resident slot, so no workgroup starts or clears its counters per
    // query (they are zero again after every segment)
    for (int64_t q = a.q0 + blockIdx.x; q < a.q1; q += gridDim.x) {
        const int64_t ex = query_exclusion(a, q);
        LaneRuns lr = lane_runs_init(a, q, tw0, tw1, lane);
        const uint32_t u0 = threadIdx.x * 32u;  // first unit of this thread in each block
        uint32_t nrun = 0;
        uint32_t kmin = 0;
        for (int32_t s = 0; s < a.nseg; ++s) {
            const uint32_t lo = (uint32_t)s << SHIFT;
            const uint32_t width = (uint32_t)min((int64_t)S, a.N - (int64_t)lo);
            const uint32_t soff = lr.tb + 4u * lr.o0;
            const uint32_t len4 = 4u * (lr.o1 - lr.o0);
            const uint32_t o3 = (lr.ob >= 0 && s + 3 <= a.nseg) ? (uint32_t)a.off[lr.ob + s + 3] : lr.o2;
            const uint32_t steps =
                count_query_segment<8>(a, q, s, soff, len4, tw0, tw1, lane, lane4, lo + 1u, dummy);
            lr.o0 = lr.o1;
            lr.o1 = lr.o2;
            lr.o2 = o3;
            __syncthreads();  // every count is in LDS
            // the thread's counter bytes of every block (units 32x .. 32x + 31 of
            // each, 8 words): per-block largest count (every unit, valid or not:
            // an upper bound) and, for the check, the byte sum with the dummy word
            uint4* pw[NB];
            uint32_t mh[NB];
            int32_t bal = 0;
#pragma unroll
            for (int h = 0; h < NB; ++h) {
                pw[h] = (uint4*)(sm + (uint32_t)h * (B / 4u) + 8u * threadIdx.x);
                const uint4 x = pw[h][0], y = pw[h][1];
                const uint32_t w8[8] = {x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
                uint32_t m2 = 0u;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    m2 = max_u16x2(m2, w8[k] & 0x00ff00ffu);
                    m2 = max_u16x2(m2, (w8[k] >> 8) & 0x00ff00ffu);
                    if constexpr (CHECK) bal = (int32_t)__builtin_amdgcn_sad_u8(w8[k], 0u, (uint32_t)bal);
                }
                mh[h] = max(m2 & 0xffffu, m2 >> 16);
            }
            if constexpr (CHECK) {
                bal += (int32_t)*dw;  // empty lanes only, all in byte 0: a plain count
                if (lane == 0) bal -= 64 * (int32_t)steps;
            }
            // block reduction of (max of each block, byte balance): NB + 1 words
            // per wave in one of two alternating slots
            uint32_t M[NB];
            bool exact = true;
            {
                constexpr uint32_t SW = NB + 1;
                uint32_t* const slot = L.red + 48 + SW * TOPK_WAVES * (uint32_t)(s & 1);
                uint32_t wm[NB];
#pragma unroll
                for (int h = 0; h < NB; ++h) wm[h] = wave_max(mh[h]);
                const uint32_t wb = CHECK ? wave_sum((uint32_t)bal) : 0u;
                if (lane == 0) {
#pragma unroll
                    for (int h = 0; h < NB; ++h) slot[SW * (threadIdx.x >> 6) + h] = wm[h];
                    slot[SW * (threadIdx.x >> 6) + NB] = wb;
                }
                __syncthreads();
                const bool have = (uint32_t)lane < (uint32_t)TOPK_WAVES;
#pragma unroll
                for (int h = 0; h < NB; ++h) M[h] = wave_max(have ? slot[SW * lane + h] : 0u) + 1u;
                if constexpr (CHECK) exact = wave_sum(have ? slot[SW * lane + NB] : 0u) == 0u;
            }
            if (exact) {
                // keys of each block from its counter bytes; a block past the
                // references, or whose largest key cannot enter the list, is
                // skipped
    #pragma unroll 1
                for (int h = 0; h < NB; ++h) {
                    if ((uint32_t)h * B >= width) break;
                    const uint32_t lowest = max((uint32_t)a.floor_key, nrun == K ? kmin + 1u : 0u);
                    uint32_t Mh = M[0];
#pragma unroll
                    for (int g = 1; g < NB; ++g) Mh = h == g ? M[g] : Mh;
                    if (Mh < lowest) continue;
                    const uint32_t loh = lo + (uint32_t)h * B;
                    // counts are read only in waves where some thread's largest
                    // count can enter
                    uint32_t mt = mh[0];
#pragma unroll
                    for (int g = 1; g < NB; ++g) mt = h == g ? mh[g] : mt;
                    const bool wl = __ballot(mt + 1u >= lowest) != 0ull;
                    uint32_t w8[8];
                    if (wl) {
                        const uint4* const ph = (const uint4*)(sm + (uint32_t)h * (B / 4u) + 8u * threadIdx.x);
                        const uint4 x = ph[0], y = ph[1];
                        w8[0] = x.x, w8[1] = x.y, w8[2] = x.z, w8[3] = x.w;
                        w8[4] = y.x, w8[5] = y.y, w8[6] = y.z, w8[7] = y.w;
                    } else {
#pragma unroll
                        for (int k = 0; k < 8; ++k) w8[k] = 0u;
                    }
                    const int32_t rem = (int32_t)width - (int32_t)(h * B) - (int32_t)u0;
                    const int64_t exd = ex - (int64_t)loh - (int64_t)u0;
                    const int32_t exu = exd >= 0 && exd < 32 ? (int32_t)exd : -1;
                    select_bytes(a, w8, wl, rem, exu, Mh, lowest, loh, u0, L, nrun, kmin);
                }
#pragma unroll
                for (int h = 0; h < NB; ++h) {
                    pw[h][0] = make_uint4(0u, 0u, 0u, 0u);
                    pw[h][1] = make_uint4(0u, 0u, 0u, 0u);
                }
                if constexpr (CHECK) *dw = 0u;
            } else {
                // some count wrapped: recount the segment with 16-bit counters,
                // block by block, zeroing each block's words as they are read
#pragma unroll
                for (int h = 0; h < NB; ++h) {
                    pw[h][0] = make_uint4(0u, 0u, 0u, 0u);
                    pw[h][1] = make_uint4(0u, 0u, 0u, 0u);
                }
                *dw = 0u;
                __syncthreads();
                uint32_t* const kw = sm + 16u * threadIdx.x;
                for (int h = 0; h < NB; ++h) {
                    if ((uint32_t)h * B >= width) break;
                    const uint32_t loh = lo + (uint32_t)h * B;
                    const uint32_t wh = min(width - (uint32_t)h * B, B);
                    count_query_segment<16>(a, q, s, soff, len4, tw0, tw1, lane, lane4, loh + 1u, dummy16);
                    __syncthreads();
                    uint32_t key[16];
#pragma unroll
                    for (int k = 0; k < 16; k += 4) {
                        const uint4 x = *(const uint4*)(kw + k);
                        key[k] = x.x;
                        key[k + 1] = x.y;
                        key[k + 2] = x.z;
                        key[k + 3] = x.w;
                        *(uint4*)(kw + k) = make_uint4(0u, 0u, 0u, 0u);
                    }
                    const int32_t rem = (int32_t)wh - (int32_t)u0;
                    const int64_t exd = ex - (int64_t)loh - (int64_t)u0;
                    const int32_t exu = exd >= 0 && exd < 32 ? (int32_t)exd : -1;
                    const uint32_t mloc = keys_of_counts<16>(key, rem, exu);
                    const uint32_t Mh = block_max(mloc, L.red + 48 + 16 * h);
                    const uint32_t lowest = max((uint32_t)a.floor_key, nrun == K ? kmin + 1u : 0u);
                    if (Mh >= lowest) select_into<16>(a, key, mloc, Mh, lowest, loh, u0, L, nrun, kmin);
                    __syncthreads();  // the block_max slot is read before its next use
                }
                // the recount's out-of-block members: words 2B/4 .. 2B/4 + 1023
                sm[(2u * B) / 4u + threadIdx.x] = 0u;
            }
            __syncthreads();  // every counter word is zero again before the next segment's counts
        }
        topk_write(a, q, L, nrun);
    }
}

// Outlier scores, full and anchor modes of RandomForest::compute_outlier_scores
// (src/rf_random_forest.cpp:4100-4193): for query q, with c_j the all-trees
// co-occurrence count of q and reference j (every j except the excluded
// one),
//     s_q = sum_j (c_j / T)^2,   raw_q = s_q > 1e-10 ? numerator / s_q : isolated
// with c_j / T a float division and its square a float product, as the
// reference computes them; the terms are summed in double (the reference
// sums floats in hash-map order, which no order reproduces), then rounded
// to float.  The counts come from the top-K counting, segment by segment.
struct OutlierArgs {
    float numerator, isolated;
    float* raw_out;
};

// One term (c / T)^2, rounded as the reference rounds it.
__device__ __forceinline__ double outlier_term(uint32_t c, float fT) {
    const float p = (float)c / fT;
    return (double)(p * p);
}

// Block sum of the threads' acc and the raw score of query q (thread 0);
// red: TOPK_WAVES doubles.
__device__ __forceinline__ void outlier_finish(double acc, double* red, const OutlierArgs& o, int64_t q) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) acc += __shfl_xor(acc, d, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int w = 0; w < TOPK_WAVES; ++w) t += red[w];
        const float sq = (float)t;
        o.raw_out[q] = sq > 1e-10f ? o.numerator / sq : o.isolated;
    }
}

// 16-bit counters, segments of S = 2^shift <= 32768 references (reference
// sets of up to 32768 samples, or more than TOPK_MAX_T8 trees), counted as
// k_topk counts them.
template <int NW>
__global__ __launch_bounds__(TOPK_THREADS) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_outlier(TopkArgs a,
                                                                                                    OutlierArgs o) {
    extern __shared__ uint32_t sm[];
    const int32_t shift = a.shift;
    const uint32_t S = 1u << shift;
    const TopkLds L = topk_lds(sm, shift);
    uint32_t* const kw = sm + threadIdx.x * NW;  // this thread's counter words
    const uint32_t dummy = topk_dummy_off(shift) + threadIdx.x * 4u;
    const uint32_t lane4 = (threadIdx.x & 63u) * 4u;
    const int32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int32_t lane = (int32_t)(threadIdx.x & 63u);
    const int64_t q = a.q0 + blockIdx.x;
    const int64_t ex = query_exclusion(a, q);
    const float fT = (float)a.T;
    const int32_t tw0 = (int32_t)(((int64_t)a.T * wave) / TOPK_WAVES);
    const int32_t tw1 = (int32_t)(((int64_t)a.T * (wave + 1)) / TOPK_WAVES);
    LaneRuns lr = lane_runs_init(a, q, tw0, tw1, lane);
    {
        uint4* c4 = (uint4*)sm;
        for (uint32_t w = threadIdx.x; w < S / 8u; w += TOPK_THREADS) c4[w] = make_uint4(0u, 0u, 0u, 0u);
    }
    __syncthreads();

    double acc = 0.0;
    for (int32_t s = 0; s < a.nseg; ++s) {
        const uint32_t lo = (uint32_t)s << shift;
        const uint32_t width = (uint32_t)min((int64_t)S, a.N - (int64_t)lo);
        const uint32_t soff = lr.tb + 4u * lr.o0;
        const uint32_t len4 = 4u * (lr.o1 - lr.o0);
        const uint32_t o3 = (lr.ob >= 0 && s + 3 <= a.nseg) ? (uint32_t)a.off[lr.ob + s + 3] : lr.o2;
        count_query_segment<16>(a, q, s, soff, len4, tw0, tw1, lane, lane4, lo + 1u, dummy);
        lr.o0 = lr.o1;
        lr.o1 = lr.o2;
        lr.o2 = o3;
        __syncthreads();  // every count is in LDS
        const uint32_t u0 = threadIdx.x * 2u * NW;
        const int32_t rem = (int32_t)width - (int32_t)u0;
        const int64_t exd = ex - (int64_t)lo - (int64_t)u0;
        const int32_t exu = exd >= 0 && exd < 2 * NW ? (int32_t)exd : -1;
#pragma unroll
        for (int k = 0; k < NW; ++k) {
            const uint32_t w = kw[k];
            kw[k] = 0u;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t c = (w >> (16 * h)) & 0xffffu;
                if (c != 0u && 2 * k + h < rem && 2 * k + h != exu) acc += outlier_term(c, fT);
            }
        }
        __syncthreads();  // every counter word is zero again before the next segment's counts
    }
    outlier_finish(acc, (double*)L.red, o, q);
}

// 8-bit counters in the segments of k_topk8 (NB blocks of TOPK_BLOCK
// references; reference sets above 32768 samples, T <= TOPK_MAX_T8): one
// pass over the query's runs per segment.  Every thread then adds the terms
// of its counter bytes from a table of the 256 possible ones (tab[c] =
// (c / T)^2, tab[0] = 0, so units without members -- those past the
// references included -- add nothing) and takes the excluded reference's
// term back out.  A segment whose byte sum fails the check (T > 255) is
// recounted with 16-bit counters, block by block, as in k_topk8.
constexpr uint32_t OUTLIER_TAB_BYTES = 256 * 8;

template <bool CHECK, int NB>
__global__ __launch_bounds__(TOPK_THREADS) __attribute__((amdgpu_waves_per_eu(16 / NB, 16 / NB))) void k_outlier8(
    TopkArgs a, OutlierArgs o) {
    static_assert(NB == 2 || NB == 4, "two or four blocks per segment");
    extern __shared__ uint32_t sm[];
    constexpr int32_t SHIFT = NB == 2 ? TOPK_SHIFT8 : TOPK_SHIFT8 + 1;
    constexpr uint32_t S = 1u << SHIFT;
    constexpr uint32_t B = TOPK_BLOCK;
    const TopkLds L = topk_lds(sm, SHIFT);
    double* const tab = (double*)(sm + topk_lds_bytes(SHIFT) / 4u);
    double* const red = (double*)L.red;  // TOPK_WAVES doubles at the end
    uint32_t* const dw = sm + (topk_dummy_off(SHIFT) >> 2) + threadIdx.x;
    const uint32_t dummy = topk_dummy_off(SHIFT) + threadIdx.x * 4u;
    const uint32_t dummy16 = 2u * B + threadIdx.x * 4u;  // as in k_topk8
    const uint32_t lane4 = (threadIdx.x & 63u) * 4u;
    const int32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int32_t lane = (int32_t)(threadIdx.x & 63u);
    const int64_t q = a.q0 + blockIdx.x;
    const int64_t ex = query_exclusion(a, q);
    const float fT = (float)a.T;
    const int32_t tw0 = (int32_t)(((int64_t)a.T * wave) / TOPK_WAVES);
    const int32_t tw1 = (int32_t)(((int64_t)a.T * (wave + 1)) / TOPK_WAVES);
    LaneRuns lr = lane_runs_init(a, q, tw0, tw1, lane);
    if (threadIdx.x < 256) tab[threadIdx.x] = threadIdx.x ? outlier_term(threadIdx.x, fT) : 0.0;
    {
        uint4* c4 = (uint4*)sm;
        for (uint32_t w = threadIdx.x; w < S / 16u; w += TOPK_THREADS) c4[w] = make_uint4(0u, 0u, 0u, 0u);
        *dw = 0u;
    }
    __syncthreads();

    const uint32_t u0 = threadIdx.x * 32u;  // first unit of this thread in each block
    double acc = 0.0;
    for (int32_t s = 0; s < a.nseg; ++s) {
        const uint32_t lo = (uint32_t)s << SHIFT;
        const uint32_t width = (uint32_t)min((int64_t)S, a.N - (int64_t)lo);
        const uint32_t soff = lr.tb + 4u * lr.o0;
        const uint32_t len4 = 4u * (lr.o1 - lr.o0);
        const uint32_t o3 = (lr.ob >= 0 && s + 3 <= a.nseg) ? (uint32_t)a.off[lr.ob + s + 3] : lr.o2;
        const uint32_t steps =
            count_query_segment<8>(a, q, s, soff, len4, tw0, tw1, lane, lane4, lo + 1u, dummy);
        lr.o0 = lr.o1;
        lr.o1 = lr.o2;
        lr.o2 = o3;
        __syncthreads();  // every count is in LDS
        uint4* pw[NB];
#pragma unroll
        for (int h = 0; h < NB; ++h) pw[h] = (uint4*)(sm + (uint32_t)h * (B / 4u) + 8u * threadIdx.x);
        bool exact = true;
        if constexpr (CHECK) {
            int32_t bal = 0;
#pragma unroll
            for (int h = 0; h < NB; ++h) {
                const uint4 x = pw[h][0], y = pw[h][1];
                bal = (int32_t)__builtin_amdgcn_sad_u8(x.x, 0u, (uint32_t)bal);
                bal = (int32_t)__builtin_amdgcn_sad_u8(x.y, 0u, (uint32_t)bal);
                bal = (int32_t)__builtin_amdgcn_sad_u8(x.z, 0u, (uint32_t)bal);
                bal = (int32_t)__builtin_amdgcn_sad_u8(x.w, 0u, (uint32_t)bal);
                bal = (int32_t)__builtin_amdgcn_sad_u8(y.x, 0u, (uint32_t)bal);
                bal = (int32_t)__builtin_amdgcn_sad_u8(y.y, 0u, (uint32_t)bal);
                bal = (int32_t)__builtin_amdgcn_sad_u8(y.z, 0u, (uint32_t)bal);
                bal = (int32_t)__builtin_amdgcn_sad_u8(y.w, 0u, (uint32_t)bal);
            }
            bal += (int32_t)*dw;  // empty lanes only, all in byte 0: a plain count
            if (lane == 0) bal -= 64 * (int32_t)steps;
            uint32_t* const slot = L.red + 48 + 16 * (uint32_t)(s & 1);
            const uint32_t wb = wave_sum((uint32_t)bal);
            if (lane == 0) slot[threadIdx.x >> 6] = wb;
            __syncthreads();
            exact = wave_sum((uint32_t)lane < (uint32_t)TOPK_WAVES ? slot[lane] : 0u) == 0u;
        }
        if (exact) {
#pragma unroll
            for (int h = 0; h < NB; ++h) {
#pragma unroll
                for (int v = 0; v < 2; ++v) {
                    const uint4 x = pw[h][v];
                    const uint32_t w4[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
                    for (int k = 0; k < 4; ++k)
#pragma unroll
                        for (int b = 0; b < 4; ++b) acc += tab[(w4[k] >> (8 * b)) & 0xffu];
                }
            }
            // the excluded reference, if in this segment: unit h * B + 32 x + r
            const int64_t exd = ex - (int64_t)lo;
            if (exd >= 0 && exd < (int64_t)width) {
                const uint32_t eu = (uint32_t)exd;
                if ((eu % B) / 32u == threadIdx.x) {
                    const uint32_t r = eu % 32u;
                    const uint32_t w = sm[(eu / B) * (B / 4u) + 8u * threadIdx.x + r / 4u];
                    acc -= tab[(w >> (8u * (r % 4u))) & 0xffu];
                }
            }
#pragma unroll
            for (int h = 0; h < NB; ++h) {
                pw[h][0] = make_uint4(0u, 0u, 0u, 0u);
                pw[h][1] = make_uint4(0u, 0u, 0u, 0u);
            }
            if constexpr (CHECK) *dw = 0u;
        } else {
            // some count wrapped: recount the segment with 16-bit counters,
            // block by block, zeroing each block's words as they are read
#pragma unroll
            for (int h = 0; h < NB; ++h) {
                pw[h][0] = make_uint4(0u, 0u, 0u, 0u);
                pw[h][1] = make_uint4(0u, 0u, 0u, 0u);
            }
            *dw = 0u;
            __syncthreads();
            uint32_t* const kw = sm + 16u * threadIdx.x;
            for (int h = 0; h < NB; ++h) {
                if ((uint32_t)h * B >= width) break;
                const uint32_t loh = lo + (uint32_t)h * B;
                count_query_segment<16>(a, q, s, soff, len4, tw0, tw1, lane, lane4, loh + 1u, dummy16);
                __syncthreads();
                const int32_t rem = (int32_t)min(width - (uint32_t)h * B, B) - (int32_t)u0;
                const int64_t exd = ex - (int64_t)loh - (int64_t)u0;
                const int32_t exu = exd >= 0 && exd < 32 ? (int32_t)exd : -1;
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    const uint32_t w = kw[k];
                    kw[k] = 0u;
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        const uint32_t c = (w >> (16 * hh)) & 0xffffu;
                        if (c != 0u && 2 * k + hh < rem && 2 * k + hh != exu) acc += outlier_term(c, fT);
                    }
                }
                __syncthreads();  // every counter word is zero before the next block's counts
            }
            // the recount's out-of-block members: words 2B/4 .. 2B/4 + 1023
            sm[(2u * B) / 4u + threadIdx.x] = 0u;
        }
        __syncthreads();  // every counter word is zero again before the next segment's counts
    }
    outlier_finish(acc, red, o, q);
}

// compute_proximity_from_leaves (src/rf_random_forest.cpp:4605-4642) for a
// batch of pairs: #{t : i OOB in t, leaf_i(t) == leaf_j(t)} / |OOB(i)| as a
// float division; 0 for indices out of range or |OOB(i)| = 0.  One wave per
// pair, lanes over trees.
struct PairArgs {
    const int32_t* leaf;
    int64_t si, st;
    const uint32_t* oob;
    int64_t old;
    int64_t N;
    int32_t T, L;
    const int64_t* pi;
    const int64_t* pj;
    int64_t npairs;
    float* out;
};

__global__ __launch_bounds__(256) void k_pair_prox(PairArgs a) {
    // one wave per pair, grid-stride over the pairs (p is uniform in a wave)
    for (int64_t p = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); p < a.npairs; p += (int64_t)gridDim.x * 4) {
        const int64_t i = a.pi[p], j = a.pj[p];
        const bool ok = i >= 0 && i < a.N && j >= 0 && j < a.N;
        uint32_t match = 0, noob = 0;
        if (ok) {
            for (int32_t t = threadIdx.x & 63; t < a.T; t += 64) {
                const uint32_t w = a.oob[(int64_t)t * a.old + (i >> 5)];
                if (!((w >> (i & 31)) & 1u)) continue;
                ++noob;
                const int32_t li = a.leaf[i * a.si + (int64_t)t * a.st];
                const int32_t lj = a.leaf[j * a.si + (int64_t)t * a.st];
                match += (li == lj && li >= 0 && li < a.L) ? 1u : 0u;
            }
        }
#pragma unroll
        for (int d = 32; d > 0; d >>= 1) {
            match += (uint32_t)__shfl_xor((int)match, d, 64);
            noob += (uint32_t)__shfl_xor((int)noob, d, 64);
        }
        if ((threadIdx.x & 63) == 0) a.out[p] = (ok && noob) ? (float)match / (float)noob : 0.0f;
    }
}

// Float scores of top-K results (src/rf_random_forest.cpp:4744, 4775-4778
// for OOB queries: (float)count * (1.0f / |OOB(q)|);
// python/randomforest_py.cpp:2538-2550 for new queries: the count summed
// as floats, divided by (float)T); 0 where a slot holds no result.
struct ScoreArgs {
    const uint32_t* qoob;
    int64_t qold;
    int64_t Q;
    int32_t T, K;
    const int32_t* idx;
    const uint16_t* cnt;
    float* score;
};

__global__ __launch_bounds__(256) void k_topk_scores(ScoreArgs a) {
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < a.Q * a.K; e += (int64_t)gridDim.x * 256) {
        const int64_t q = e / a.K;
        float sc = 0.0f;
        if (a.idx[e] >= 0) {
            const float c = (float)a.cnt[e];
            if (a.qoob) {
                uint32_t n = 0;
                for (int32_t t = 0; t < a.T; ++t) n += (a.qoob[(int64_t)t * a.qold + (q >> 5)] >> (q & 31)) & 1u;
                sc = n ? c * (1.0f / (float)n) : 0.0f;
            } else {
                sc = c / (float)a.T;
            }
        }
        a.score[e] = sc;
    }
}

// Queries per launch: gridDim.x * blockDim.x must stay below 2^32.
constexpr int64_t TOPK_MAX_GRID = 1LL << 21;

// One launch over all Q queries with at most per_cu workgroups per CU (what
// the kernel's LDS and waves let one CU hold): each workgroup loops over
// queries blockIdx.x, + gridDim.x, ...
template <typename Kern>
static hipError_t launch_topk_kernel(rfxp_ctx* ctx, Kern kern, TopkArgs a, int64_t Q, int per_cu) {
    const size_t lds = topk_lds_bytes(a.shift);
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    const int64_t slots = (int64_t)std::max(ctx->n_cu, 1) * per_cu;
    a.q0 = 0;
    a.q1 = Q;
    hipLaunchKernelGGL(kern, dim3((unsigned)std::min(slots, Q)), dim3(TOPK_THREADS), lds, ctx->stream, a);
    return hipGetLastError();
}

template <int NW>
static hipError_t launch_topk(rfxp_ctx* ctx, TopkArgs a, int64_t Q) {
    return launch_topk_kernel(ctx, k_topk<NW>, a, Q, 2);
}

template <typename Kern>
static hipError_t launch_outlier_kernel(rfxp_ctx* ctx, Kern kern, TopkArgs a, const OutlierArgs& o, int64_t Q,
                                        size_t lds) {
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    for (int64_t q0 = 0; q0 < Q; q0 += TOPK_MAX_GRID) {
        a.q0 = q0;
        const unsigned nq = (unsigned)std::min(TOPK_MAX_GRID, Q - q0);
        hipLaunchKernelGGL(kern, dim3(nq), dim3(TOPK_THREADS), lds, ctx->stream, a, o);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    return hipSuccess;
}

template <int NW>
static hipError_t launch_outlier(rfxp_ctx* ctx, TopkArgs a, const OutlierArgs& o, int64_t Q) {
    return launch_outlier_kernel(ctx, k_outlier<NW>, a, o, Q, topk_lds_bytes(a.shift));
}

template <int NB>
static hipError_t launch_outlier8(rfxp_ctx* ctx, TopkArgs a, const OutlierArgs& o, int64_t Q) {
    const size_t lds = topk_lds_bytes(a.shift) + OUTLIER_TAB_BYTES;
    return a.T <= 255 ? launch_outlier_kernel(ctx, k_outlier8<false, NB>, a, o, Q, lds)
                      : launch_outlier_kernel(ctx, k_outlier8<true, NB>, a, o, Q, lds);
}

// Arguments of a query launch over the context's reference set.
static TopkArgs ref_args(rfxp_ctx* ctx, const int32_t* q_leaf, int64_t q_stride_i, int64_t q_stride_t,
                         const uint32_t* q_oob_words, int64_t q_oob_ld, int64_t exclude_base,
                         const int32_t* exclude_idx) {
    TopkArgs a;
    a.mem = ctx->ref_mem.p;
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
    a.exclude_idx = exclude_idx;
    a.q0 = 0;
    a.q1 = 0;
    a.K = 1;
    a.floor_key = 1;
    a.idx_out = nullptr;
    a.cnt_out = nullptr;
    return a;
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
    // segments of 2^shift references: 8-bit counters (65536 or 131072 per
    // segment) when the counts of a wave's trees fit their check, else
    // 16-bit ones (at most 32768)
    const int32_t max_shift = T <= TOPK_MAX_T8 ? TOPK_MAX_SHIFT8 : TOPK_MAX_SHIFT16;
    int32_t shift = TOPK_MIN_SHIFT;
    while (shift < max_shift && (1LL << shift) < N) ++shift;
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
    TopkArgs a = ref_args(ctx, q_leaf, q_stride_i, q_stride_t, q_oob_words, q_oob_ld, exclude_base, nullptr);
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
            case 15: e = launch_topk<16>(ctx, a, Q); break;
            case TOPK_SHIFT8:
                e = a.T <= 255 ? launch_topk_kernel(ctx, k_topk8<false, 2>, a, Q, 2)
                               : launch_topk_kernel(ctx, k_topk8<true, 2>, a, Q, 2);
                break;
            default:
                e = a.T <= 255 ? launch_topk_kernel(ctx, k_topk8<false, 4>, a, Q, 1)
                               : launch_topk_kernel(ctx, k_topk8<true, 4>, a, Q, 1);
                break;
        }
    }
    if (e != hipSuccess) return hip_error(ctx, e, "k_topk launch");
    return RFXP_OK;
}

extern "C" int rfxp_topk_scores(rfxp_ctx* ctx, const uint32_t* q_oob_words, int64_t q_oob_ld, int64_t Q, int32_t T,
                                int32_t K, const int32_t* idx, const uint16_t* cnt, float* score_out) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (Q < 0 || K < 1 || T < 1) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_topk_scores: need Q >= 0, K >= 1, T >= 1");
    if (Q == 0) return RFXP_OK;
    if (Q > (1LL << 40) / K) return set_error(ctx, RFXP_ERR_UNSUPPORTED, "rfxp_topk_scores: Q * K too large");
    if (!idx || !cnt || !score_out || !is_device_pointer(idx) || !is_device_pointer(cnt) ||
        !is_device_pointer(score_out) || (q_oob_words && !is_device_pointer(q_oob_words)))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_topk_scores: pointers must be device pointers");
    if (q_oob_words && q_oob_ld < (Q + 31) / 32)
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_topk_scores: q_oob_ld < ceil(Q/32)");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    ScoreArgs a{q_oob_words, q_oob_ld, Q, T, K, idx, cnt, score_out};
    hipLaunchKernelGGL(k_topk_scores, dim3(grid_stride_blocks(Q * K, 256)), dim3(256), 0, ctx->stream, a);
    return check_launch(ctx, "k_topk_scores launch");
}

extern "C" int rfxp_pair_proximity(rfxp_ctx* ctx, const int32_t* leaf, int64_t stride_i, int64_t stride_t,
                                   const uint32_t* oob_words, int64_t oob_ld, int64_t N, int32_t T, int32_t nleaf,
                                   const int64_t* pair_i, const int64_t* pair_j, int64_t npairs, float* out) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (N < 0 || T < 1 || nleaf < 1 || npairs < 0)
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_pair_proximity: need N >= 0, T >= 1, nleaf >= 1, npairs >= 0");
    if (npairs == 0) return RFXP_OK;
    if (oob_ld < (N + 31) / 32) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_pair_proximity: oob_ld < ceil(N/32)");
    if (!leaf || !oob_words || !pair_i || !pair_j || !out || !is_device_pointer(leaf) ||
        !is_device_pointer(oob_words) || !is_device_pointer(pair_i) || !is_device_pointer(pair_j) ||
        !is_device_pointer(out))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_pair_proximity: pointers must be device pointers");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    PairArgs a{leaf, stride_i, stride_t, oob_words, oob_ld, N, T, nleaf, pair_i, pair_j, npairs, out};
    // four pairs per workgroup and stride
    hipLaunchKernelGGL(k_pair_prox, dim3(grid_stride_blocks(npairs, 4)), dim3(256), 0, ctx->stream, a);
    return check_launch(ctx, "k_pair_prox launch");
}

extern "C" int rfxp_outlier_raw(rfxp_ctx* ctx, const int32_t* q_leaf, int64_t q_stride_i, int64_t q_stride_t,
                                int64_t Q, int64_t exclude_base, const int32_t* exclude_idx, float numerator,
                                float isolated, float* raw_out) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (!ctx->ref_ready) return set_error(ctx, RFXP_ERR_STATE, "rfxp_outlier_raw: no reference set");
    if (Q < 0) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_outlier_raw: need Q >= 0");
    if (Q == 0) return RFXP_OK;
    if (Q > 0x7fffffffLL) return set_error(ctx, RFXP_ERR_UNSUPPORTED, "rfxp_outlier_raw: too many queries");
    if (!q_leaf || !raw_out || !is_device_pointer(q_leaf) || !is_device_pointer(raw_out) ||
        (exclude_idx && !is_device_pointer(exclude_idx)))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_outlier_raw: pointers must be device pointers");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    const TopkArgs a = ref_args(ctx, q_leaf, q_stride_i, q_stride_t, nullptr, 0, exclude_base, exclude_idx);
    const OutlierArgs o{numerator, isolated, raw_out};
    hipError_t e;
    {
        LaunchTimer tm(ctx, "outlier");
        switch (a.shift) {
            case 11: e = launch_outlier<1>(ctx, a, o, Q); break;
            case 12: e = launch_outlier<2>(ctx, a, o, Q); break;
            case 13: e = launch_outlier<4>(ctx, a, o, Q); break;
            case 14: e = launch_outlier<8>(ctx, a, o, Q); break;
            case 15: e = launch_outlier<16>(ctx, a, o, Q); break;
            case TOPK_SHIFT8: e = launch_outlier8<2>(ctx, a, o, Q); break;
            default: e = launch_outlier8<4>(ctx, a, o, Q); break;
        }
    }
    if (e != hipSuccess) return hip_error(ctx, e, "k_outlier launch");
    return RFXP_OK;
}

// src/rf_random_forest.cpp:4196-4273: robust normalisation of the raw
// scores, per class in ascending class order when classes are given (else
// over all samples): median = the sorted values' element size/2, MAD = the
// sorted absolute deviations' element size/2 (1 when below 1e-10),
// score = (raw - median) / MAD.  Host memory, no device needed.
extern "C" int rfxp_outlier_normalize(const float* raw, int64_t N, const int32_t* classes, float* scores,
                                      float* medians, float* mads) {
    if (N < 1 || !raw || !scores) return RFXP_ERR_INVALID;
    std::vector<int32_t> cls;
    if (classes) {
        cls.assign(classes, classes + N);
        std::sort(cls.begin(), cls.end());
        cls.erase(std::unique(cls.begin(), cls.end()), cls.end());
    } else {
        cls.push_back(-1);
    }
    std::vector<int64_t> members;
    std::vector<float> v, dev;
    for (size_t c = 0; c < cls.size(); ++c) {
        members.clear();
        for (int64_t n = 0; n < N; ++n)
            if (!classes || classes[n] == cls[c]) members.push_back(n);
        v.resize(members.size());
        for (size_t k = 0; k < members.size(); ++k) v[k] = raw[members[k]];
        std::vector<float> sorted = v;
        std::sort(sorted.begin(), sorted.end());
        const float median = sorted[sorted.size() / 2];
        dev.resize(v.size());
        for (size_t k = 0; k < v.size(); ++k) dev[k] = std::fabs(v[k] - median);
        std::sort(dev.begin(), dev.end());
        float mad = dev[dev.size() / 2];
        if (mad < 1e-10f) mad = 1.0f;
        if (medians) medians[c] = median;
        if (mads) mads[c] = mad;
        for (size_t k = 0; k < members.size(); ++k) scores[members[k]] = (raw[members[k]] - median) / mad;
    }
    return RFXP_OK;
}
