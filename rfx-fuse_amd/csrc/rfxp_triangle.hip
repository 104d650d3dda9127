// Batched OOB co-occurrence proximity into the packed upper triangle.
//
// Reference path restated here (one batched pass instead of T per-tree
// calls):  src/rf_proximity.cpp:179-230 accumulates, per tree, +1 at
// (OOB n, in-bag kk) of the same terminal node; src/rf_finishprox.cpp:12-74
// symmetrises and normalises by nout.  Folding (n,kk) to (min,max) as
// cuda/rf_proximity_upper_triangle.cu:229-237 does gives, for i < j,
//     U_ij = #{t : leaf_i(t) == leaf_j(t) valid, oob_i(t) != oob_j(t)}.
//
// The forest index it reads (mem, rec, nout, rinv) is described in
// rfxp_forest.hpp.
//
// Triangle kernel: one workgroup per (row i, column segment [lo, hi)) item.
// It zeroes a byte counter per column in LDS, walks row i's T records,
// gathers the member ids of each opposite bucket (one wave-wide coalesced
// load per bucket, sixteen buckets in flight per wave) and bumps the LDS
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
#include "rfxp_forest.hpp"
#include "rfxp_internal.hpp"

namespace rfxp {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int TRI_THREADS = 1024;
constexpr int TRI_WAVES = TRI_THREADS / 64;

// ---------------------------------------------------------------------------
// triangle
// ---------------------------------------------------------------------------


// Work items of a row band [r0, r1): row i is cut into segments of S
// columns starting at i, i + S, ...; segment k of row i starts at i + k*S
// and exists while N - i > k*S.  Rows are taken in groups of 8 (group g:
// rows r0 + 8g .. r0 + 8g + 7); a group occupies 8 * n_g consecutive
// workgroup slots, level-major (slot 8k + r: segment k of row r of the
// group), n_g = the number of segments of its first row.  Workgroups are
// dealt to the 8 XCDs round-robin by index, so every segment of a row runs
// on the same XCD, one slot after the other, and the later segments find
// the row's records and bucket runs -- which they read in full, as the
// first segment does -- in that XCD's L2.  Slots of rows past the band or
// of segments a row does not have are idle.
//
// G_k = number of groups with a segment k = min(G, ceil((N - r0 - k*S)/8)),
// slots before group g = 8 * sum_k min(g, G_k); tri_slot() inverts that by
// binary search over g.  The divisions (G, nlev) are done on the host.
struct TriLevels {
    int64_t N, S, r0, r1, G, nlev;
};

__host__ __device__ inline TriLevels tri_levels_of(int64_t N, int64_t S, int64_t r0, int64_t r1) {
    TriLevels L;
    L.N = N;
    L.S = S;
    L.r0 = r0;
    L.r1 = r1;
    L.G = (r1 - r0 + 7) / 8;
    L.nlev = (N - r0 + S - 1) / S;
    return L;
}

__host__ __device__ inline int64_t tri_groups_with_level(const TriLevels& L, int64_t k) {
    const int64_t rem = L.N - L.r0 - k * L.S;
    if (rem <= 0) return 0;
    const int64_t g = (rem + 7) >> 3;
    return g < L.G ? g : L.G;
}

__host__ __device__ inline int64_t tri_slots_before(const TriLevels& L, int64_t g) {
    int64_t s = 0;
    for (int64_t k = 0; k < L.nlev; ++k) {
        const int64_t gk = tri_groups_with_level(L, k);
        s += g < gk ? g : gk;
    }
    return 8 * s;
}

// Row i and segment k of slot b; false for an idle slot.  Groups
// [G_m, G_{m-1}) have exactly m segments (G_nlev = 0), so the slots are
// walked segment count by segment count, most segments (first groups)
// first.
__host__ __device__ inline bool tri_slot(const TriLevels& L, int64_t b, int64_t& i, int64_t& k) {
    int64_t start = 0, g0 = 0;
    for (int64_t m = L.nlev; m >= 1; --m) {
        const int64_t g1 = tri_groups_with_level(L, m - 1);
        const int64_t per = 8 * m;
        const int64_t cnt = (g1 - g0) * per;
        if (b < start + cnt) {
            const int64_t off = b - start;
            const int64_t gq = (int64_t)((uint64_t)off / (uint64_t)per);
            const int64_t loc = off - gq * per;
            k = loc >> 3;
            i = L.r0 + 8 * (g0 + gq) + (loc & 7);
            return i < L.r1 && L.N - i > k * L.S;
        }
        start += cnt;
        g0 = g1;
    }
    return false;
}

struct TriArgs {
    const uint32_t* roff;  // [N][ldr] run byte offsets in mem (+ REC_PAD)
    const uint16_t* rlen;  // [N][ldr] run lengths in bytes (+ REC_PAD)
    const uint32_t* mem;
    uint32_t mem_bytes;  // readable bytes of mem (buffer-load range)
    int64_t ldr;         // record row stride (T rounded up to 16)
    const uint2* lng;    // [T][lmax] long buckets: start, end byte offsets in mem
    const int32_t* lngn; // [T] entries of lng per tree
    int32_t lmax;
    const double* rinv;
    const unsigned long long* rr;
    int64_t N;
    int32_t T;
    int32_t S;          // columns per item
    TriLevels lev;      // work decomposition of the row band
    int64_t item_base;  // item index of blockIdx.x == 0 (launches in chunks)
    int64_t e_base;     // idx(row_begin, row_begin)
    char* out;          // byte address of entry e_base (NF4: of its byte)
    float scale, zp;
    int32_t* flags;     // [0]: items redone with 16-bit counters
    int32_t mode;       // TRI_MODE_*
    uint32_t dbytes;    // dummy area bytes (TRI_DUMMY_BYTES or TRI_DUMMY_SHARED_BYTES)
};

// Counter width / exactness check per launch:
//   EXACT8  T <= 255: 8-bit counters cannot wrap;
//   CHECK8  8-bit counters, a byte-sum check after the hit phase, items
//           whose counters wrapped are redone with 16-bit counters;
//   WIDE16  every item counted with 16-bit counters (very many trees per
//           wave, where the check's own dummy bytes could wrap).
enum { TRI_MODE_EXACT8 = 0, TRI_MODE_CHECK8 = 1, TRI_MODE_WIDE16 = 2 };

// LDS layout of one workgroup (dynamic shared memory, at address 0):
//   [0, cap)                 the item's counters, cap = 16 * chunks <= S + 32
//                            (8-bit, or 16-bit when redoing)
//   [cap, cap + dbytes)      dummy words (see count_hits): one per thread
//                            (dbytes 4096), or one per lane shared by the
//                            waves (dbytes 256, 3,840 more columns), see
//                            tri_dummy_bytes
//   [misc_off, +64)          item scalars (geometry, row table, sums),
//                            misc_off = round16(S + 64) + dbytes
constexpr uint32_t TRI_DUMMY_BYTES = TRI_THREADS * 4;
constexpr uint32_t TRI_DUMMY_SHARED_BYTES = 64 * 4;
constexpr int TRI_MISC_WORDS = 16;
enum {
    MISC_LUT_LO = 0, MISC_LUT_HI = 1, MISC_UC = 2, MISC_SUM = 3, MISC_SLOTS = 4,  // cleared per item
    MISC_ROW = 5, MISC_LO = 6, MISC_WIDTH = 7, MISC_SHIFT = 8, MISC_NCHUNK = 9, MISC_DST_LO = 10, MISC_DST_HI = 11
};
constexpr int TRI_MISC_ZEROED = 5;  // words cleared per item (the row table and the sums)

__host__ __device__ constexpr uint32_t tri_misc_off(int32_t S, uint32_t dbytes) {
    return (((uint32_t)S + 64u + 15u) & ~15u) + dbytes;
}
__host__ __device__ constexpr uint32_t tri_lds_bytes(int32_t S, uint32_t dbytes) {
    return tri_misc_off(S, dbytes) + TRI_MISC_WORDS * 4;
}

// This thread's dummy unit past the counters: 8-bit units (bytes), or 16-bit
// ones.  With one dummy word per thread, byte 0 (half 0) of its own word;
// with shared words, byte (wave & 3) (half (wave & 1)) of its lane's word,
// so that four (eight) waves share a unit.
__device__ __forceinline__ uint32_t dummy_unit8(uint32_t dbytes) {
    return dbytes == TRI_DUMMY_BYTES ? 4u * threadIdx.x : 4u * (threadIdx.x & 63u) + ((threadIdx.x >> 6) & 3u);
}
__device__ __forceinline__ uint32_t dummy_unit16(uint32_t dbytes) {
    return dbytes == TRI_DUMMY_BYTES ? 2u * threadIdx.x : 2u * (threadIdx.x & 63u) + ((threadIdx.x >> 6) & 1u);
}

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

// Nonzero when some byte of w is >= uc (or >= 0x80): kuc = (0x80 - uc) * 0x01010101.
__device__ __forceinline__ uint32_t over_uc(uint32_t w, uint32_t kuc) { return ((w + kuc) | w) & 0x80808080u; }

// Exact codes (I8 / U8 / NF4) for the counts >= uc of a chunk of NW words
// of byte counters w, whose table codes are already in o: only those bytes
// are recomputed from the closed form, each with its column's r_j (byte b
// of the chunk is column j0 + b).  Only the bytes of the item's own columns
// count, bytes [b0, b1) of the chunk: a byte before or after them holds no
// column (in a checked launch, the carry of a wrapped last column lands in
// the byte after it, before the item is recounted), so its r_j would be
// read outside rinv, and its code is never stored.  Inlined: the chunks
// that need it are rare, and a call would make the kernel save registers
// around it.
template <int F, int NW>
__device__ __forceinline__ void fix_codes(uint32_t (&o)[NW], const uint32_t (&w)[NW], uint32_t uc, double ri,
                                          const double* rinv, int64_t j0, int32_t b0, int32_t b1, float scale,
                                          float zp) {
    uint32_t m = 0;  // bit b: byte b holds a count >= uc and a column of the item
#pragma unroll
    for (int b = 0; b < 4 * NW; ++b)
        m |= (byte_of(w[b >> 2], b & 3) >= uc && b >= b0 && b < b1 ? 1u : 0u) << b;
    while (m) {
        const int b = __builtin_ctz(m);
        m &= m - 1u;
        uint32_t U = 0;
#pragma unroll
        for (int q = 0; q < NW; ++q) U = (q == (b >> 2)) ? byte_of(w[q], b & 3) : U;
        set_byte(o, b, code_of<F>(pair_p(U, ri, rinv[j0 + b]), scale, zp));
    }
}

// Hit phase: every member j of row i's opposite buckets with lo <= j < hi
// bumps its counter.  Counter c of column j sits at unit (j - lo + shift)
// of the LDS array (cap units); BITS is 8 or 16.  Returns the number of
// 64-lane counting steps this wave made (wave-uniform).
//
// Each wave owns a contiguous range of trees and walks it in groups of 16.
// A group's records come in through scalar loads (16 offsets, 16 lengths);
// each bucket load is a buffer load with the bucket offset as its scalar
// offset and a range (checked on scalar + lane offset) ending at the bucket
// end, so lanes past the end read 0 (no stored id is 0) with no per-lane
// masking.  The loads of group q + 1 are issued before group q is counted.
// Counting is branch-free: a lane without a hit adds into its own dummy
// word, so every lane of every step lands somewhere countable.
struct Group {
    uint32_t m[16];
    bool has_long;  // some run of the group may have more than 63 members
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t mem_rsrc(const uint32_t* mem, uint32_t nbytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)mem, (short)0, (int)nbytes, 0x00020000);
}

// The 16 bucket loads of one record group (ro, rl point at its records).
// Each load's range ends at its run's end, and never past mem_bytes, the
// readable bytes of mem.
__device__ __forceinline__ void load_group(const uint32_t* mem, uint32_t mem_bytes, const uint32_t* __restrict__ ro,
                                           const uint16_t* __restrict__ rl, uint32_t lane4, Group& G) {
    uint32_t off[16];
    uint32_t lw[8];
#pragma unroll
    for (int u = 0; u < 16; ++u) off[u] = __builtin_amdgcn_readfirstlane(ro[u]);
#pragma unroll
    for (int k = 0; k < 8; ++k) lw[k] = __builtin_amdgcn_readfirstlane(((const uint32_t*)rl)[k]);
    // a length of 256 bytes or more (64+ members) may need the tail loop
    uint32_t lng = 0u;
#pragma unroll
    for (int k = 0; k < 8; ++k) lng |= lw[k];
    G.has_long = (lng & 0xff00ff00u) != 0u;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const uint32_t len4 = (lw[u >> 1] >> (16 * (u & 1))) & 0xffffu;
        G.m[u] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(mem_rsrc(mem, min(off[u] + len4, mem_bytes)), lane4,
                                                                off[u], 0);
    }
}

// LDS atomic add at a byte address of the workgroup's LDS.  The counters are
// the dynamic LDS array and the kernels declare no static LDS, so the array
// starts at LDS address 0 and counter byte offsets are LDS addresses.
typedef __attribute__((address_space(3))) uint32_t lds_u32;
__device__ __forceinline__ void lds_add(uint32_t addr, uint32_t val) {
    __hip_atomic_fetch_add((lds_u32*)(uintptr_t)addr, val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// One counting step: m = j + 1 of a member (0: no member); counter unit
// c = j - lo + shift.  Units c >= xlim -- members outside the item, empty
// lanes -- are clamped to xlim, the unit of this thread's dummy word, which
// sits with the other dummy words right after the item's counters; units
// between the counters and xlim fall on other threads' dummy words.  Every
// lane of every step thus adds 1 to some byte (16-bit unit) of the
// counter-and-dummy area, without a compare or select.  base1 = lo + 1 -
// shift; when it is not positive (an item that starts within the first
// output chunk of the triangle, lo < shift) an empty lane's m - base1 is a
// small padding unit, so those items (EMPTY_FIX) send m = 0 to xlim
// explicitly.
template <int BITS, bool EMPTY_FIX = false>
__device__ __forceinline__ void count_hits(uint32_t m, uint32_t base1, uint32_t xlim) {
    uint32_t c = min(m - base1, xlim);
    if constexpr (EMPTY_FIX) c = m ? c : xlim;
    if constexpr (BITS == 8) lds_add(c & ~3u, 1u << ((c << 3) & 31u));
    else lds_add((c << 1) & ~3u, 1u << ((c << 4) & 31u));
}

// Runs of REC_LONG or more members: their end, from the per-tree table of
// long buckets (start and end byte offsets in mem) that contains `off`.
__device__ __forceinline__ uint32_t long_run_end(const TriArgs& a, int32_t t, uint32_t off, uint32_t fallback) {
    const uint2* L = a.lng + (int64_t)t * a.lmax;
    const int32_t n = min(a.lngn[t], a.lmax);
    for (int32_t e = 0; e < n; ++e) {
        const uint2 r = L[e];
        if (r.x <= off && off < r.y) return r.y;
    }
    return fallback;
}

// Hit phase of one item: every member j of row i's runs bumps counter unit
// j - lo + shift (see count_hits).  Each wave owns a contiguous range of
// record groups (16 trees each) and keeps two groups' loads in flight; no
// load is issued past its range.  Returns the wave's 64-lane counting steps
// (uniform).
template <int BITS, bool EMPTY_FIX = false>
__device__ __forceinline__ uint32_t hit_phase(const TriArgs& a, int64_t i, int64_t lo, int32_t shift, uint32_t xlim) {
    const uint32_t lane4 = (threadIdx.x & 63) * 4u;
    const int32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // whole groups of 16 trees per wave, so record rows stay 16-aligned
    const int32_t ng = (a.T + 15) >> 4;
    const int32_t g0 = (ng * wave) / TRI_WAVES;
    const int32_t g1 = (ng * (wave + 1)) / TRI_WAVES;
    if (g0 >= g1) return 0u;
    const uint32_t* ro = a.roff + i * a.ldr;
    const uint16_t* rl = a.rlen + i * a.ldr;
    const uint32_t base1 = (uint32_t)lo + 1u - (uint32_t)shift;
    uint32_t steps = 0;
    // members past the first 64 of a run (rare for per-leaf buckets), eight
    // 64-member loads in flight at a time: loads past the run's end read 0
    // (the buffer range ends there) and count into the dummy word, so every
    // lane of each of the eight steps still adds 1 somewhere
    auto long_tail = [&](int32_t t0) {
        for (int u = 0; u < 16; ++u) {
            const uint32_t len4 = __builtin_amdgcn_readfirstlane((uint32_t)rl[t0 + u]);
            if (len4 <= 256u) continue;
            const uint32_t off = __builtin_amdgcn_readfirstlane(ro[t0 + u]);
            const uint32_t end = min(len4 == 4u * REC_LONG ? long_run_end(a, t0 + u, off, off + len4) : off + len4,
                                     a.mem_bytes);
            const __amdgpu_buffer_rsrc_t rs = mem_rsrc(a.mem, end);
            for (uint32_t p4 = 256u; off + p4 < end; p4 += 8u * 256u) {
                uint32_t m[8];
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    m[k] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs, p4 + 256u * k + lane4, off, 0);
#pragma unroll
                for (int k = 0; k < 8; ++k) count_hits<BITS, EMPTY_FIX>(m[k], base1, xlim);
                steps += 8;
            }
        }
    };
    // A and B in ping-pong: one group is counted while the other's loads
    // are in flight (no register copies between them)
    Group A, B;
    load_group(a.mem, a.mem_bytes, ro + 16 * g0, rl + 16 * g0, lane4, A);
    if (g0 + 1 < g1) load_group(a.mem, a.mem_bytes, ro + 16 * (g0 + 1), rl + 16 * (g0 + 1), lane4, B);
    for (int32_t g = g0;; g += 2) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 16; ++u) count_hits<BITS, EMPTY_FIX>(A.m[u], base1, xlim);
        steps += 16;
        if (A.has_long) long_tail(16 * g);
        if (g + 2 < g1) load_group(a.mem, a.mem_bytes, ro + 16 * (g + 2), rl + 16 * (g + 2), lane4, A);
        if (g + 1 >= g1) break;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 16; ++u) count_hits<BITS, EMPTY_FIX>(B.m[u], base1, xlim);
        steps += 16;
        if (B.has_long) long_tail(16 * (g + 1));
        if (g + 3 < g1) load_group(a.mem, a.mem_bytes, ro + 16 * (g + 3), rl + 16 * (g + 3), lane4, B);
        if (g + 2 >= g1) break;
    }
    return steps;
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
        } else if constexpr (F == NF4) {
            const uint32_t c = code_of<NF4>(diag ? 1.0 : (U == 0 ? 0.0 : pair_p(U, ri, a.rinv[j])), 0.f, 0.f);
            const int64_t g = e + (a.e_base & 1);
            const uintptr_t ba = (uintptr_t)a.out + (uintptr_t)(g >> 1);
            uint32_t* word = (uint32_t*)(ba & ~(uintptr_t)3);
            const uint32_t sh = (uint32_t)((ba & 3u) * 8u + (uint32_t)(g & 1) * 4u);
            atomicAnd(word, ~(0xfu << sh));
            atomicOr(word, c << sh);
        } else {
            double P = diag ? 1.0 : (U == 0 ? 0.0 : pair_p(U, ri, a.rinv[j]));
            if constexpr (F == F32) ((float*)a.out)[e] = (float)P;
            else if constexpr (F == F16) ((uint16_t*)a.out)[e] = f32_to_f16_bits((float)P);
            else ((uint8_t*)a.out)[e] = (uint8_t)code_of<F>(P, a.scale, a.zp);
        }
    }
}

// Per-row table of the integer codes of U = 0..7 (I8, U8, NF4): uc is the
// number of leading counts whose code does not depend on the column (the
// code is monotone in r_j, so equal codes at the smallest and largest r_j
// mean equal codes for every column).  Run by the first wave.
template <int F>
__device__ __forceinline__ void row_table(const TriArgs& a, double ri, uint32_t* misc) {
    if (threadIdx.x >= 64) return;
    const int u = threadIdx.x & 7;
    const double rmin = __longlong_as_double((long long)a.rr[0]);
    const double rmax = __longlong_as_double((long long)a.rr[1]);
    const uint32_t c0 = code_of<F>(pair_p(u, ri, rmin), a.scale, a.zp);
    const uint32_t c1 = code_of<F>(pair_p(u, ri, rmax), a.scale, a.zp);
    const unsigned long long eq = __ballot(c0 == c1 && threadIdx.x < 8);
    uint32_t lo4 = 0, hi4 = 0;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const uint32_t cb = (uint32_t)__shfl((int)c0, b, 64);
        if (b < 4) lo4 |= cb << (8 * b);
        else hi4 |= cb << (8 * (b - 4));
    }
    if (threadIdx.x == 0) {
        uint32_t uc = 0;
        while (uc < 8 && ((eq >> uc) & 1ull)) ++uc;
        misc[MISC_UC] = uc;
        misc[MISC_LUT_LO] = lo4;
        misc[MISC_LUT_HI] = hi4;
    }
}

// Item geometry, worked out by thread 0 (tri_slot, the 64-bit entry index
// and the output alignment) and read by every wave from LDS.
struct ItemGeom {
    int64_t i, lo;
    int32_t width, shift, nchunk, nwords;
    int64_t dst;  // byte offset of the item's first 16-byte output chunk from a.out
};

// Thread 0: the item of this workgroup into misc (MISC_ROW = ~0 when idle).
// Byte formats: entries of esz bytes, a counter byte per entry, epc entries
// per 16-byte chunk.  NF4 (esz = 0): a counter byte per nibble entry, 32
// entries per 16-byte chunk.
template <int esz>
__device__ __forceinline__ void item_to_lds(const TriArgs& a, uint32_t* misc) {
    int64_t i, k;
    if (!tri_slot(a.lev, a.item_base + blockIdx.x, i, k)) {
        misc[MISC_ROW] = 0xffffffffu;
        return;
    }
    const int64_t lo = i + k * a.S;
    const int32_t width = (int32_t)min((int64_t)a.S, a.N - lo);
    int64_t dst;
    int32_t shift, nchunk;
    if constexpr (esz == 0) {
        const int64_t g0 = tri_idx(a.N, i, lo) - a.e_base + (a.e_base & 1);  // nibble index
        const int64_t b0 = (g0 >> 1) + (int64_t)((uintptr_t)a.out & 15u);
        shift = (int32_t)((b0 & 15) * 2 + (g0 & 1));
        dst = (b0 & ~(int64_t)15) - (int64_t)((uintptr_t)a.out & 15u);
        nchunk = (shift + width + 31) / 32;
    } else {
        constexpr int epc = 16 / esz;
        const int64_t b0 = (tri_idx(a.N, i, lo) - a.e_base) * esz + (int64_t)((uintptr_t)a.out & 15u);
        shift = (int32_t)((b0 & 15) / esz);
        dst = (b0 & ~(int64_t)15) - (int64_t)((uintptr_t)a.out & 15u);
        nchunk = (shift + width + epc - 1) / epc;
    }
    misc[MISC_ROW] = (uint32_t)i;
    misc[MISC_LO] = (uint32_t)lo;
    misc[MISC_WIDTH] = (uint32_t)width;
    misc[MISC_SHIFT] = (uint32_t)shift;
    misc[MISC_NCHUNK] = (uint32_t)nchunk;
    misc[MISC_DST_LO] = (uint32_t)(uint64_t)dst;
    misc[MISC_DST_HI] = (uint32_t)((uint64_t)dst >> 32);
}

template <int esz>
__device__ __forceinline__ bool item_from_lds(const uint32_t* misc, ItemGeom& gm) {
    const uint32_t row = misc[MISC_ROW];
    if (row == 0xffffffffu) return false;
    gm.i = row;
    gm.lo = misc[MISC_LO];
    gm.width = (int32_t)misc[MISC_WIDTH];
    gm.shift = (int32_t)misc[MISC_SHIFT];
    gm.nchunk = (int32_t)misc[MISC_NCHUNK];
    gm.dst = (int64_t)(((uint64_t)misc[MISC_DST_HI] << 32) | misc[MISC_DST_LO]);
    gm.nwords = esz == 0 ? gm.nchunk * 8 : gm.nchunk * (16 / esz) / 4;
    return true;
}

// 16-bit recount of an item (its 8-bit counters wrapped, or the launch is
// WIDE16): passes of half the counter capacity, exact stores.  The dummy
// words follow the pass's counters, 16-byte aligned, inside the item's
// counter-and-dummy area.
template <int F>
__device__ void redo_wide(const TriArgs& a, uint32_t* cnt, const ItemGeom& gm, double ri) {
    if (threadIdx.x == 0) atomicAdd(&a.flags[0], 1);
    const int32_t half_cap = gm.nwords * 2;  // 16-bit counters that fit
    for (int32_t d0 = 0; d0 < gm.width; d0 += half_cap) {
        const int32_t w2 = min(half_cap, gm.width - d0);
        const uint32_t cap16 = ((uint32_t)w2 + 7u) & ~7u;
        __syncthreads();
        for (int32_t w = threadIdx.x; w < (int32_t)cap16 / 2; w += TRI_THREADS) cnt[w] = 0u;
        __syncthreads();
        hit_phase<16>(a, gm.i, gm.lo + d0, 0, cap16 + dummy_unit16(a.dbytes));
        __syncthreads();
        store_exact16<F>(a, cnt, gm.i, gm.lo + d0, w2, ri);
    }
}

// Zeroes the item's counter words [0, nwords) and the dwords dummy words
// after them (rounded up to whole 16-byte stores: at most 3 words past the
// last dummy word, inside the 64-byte gap before the item scalars).
__device__ __forceinline__ void zero_counters(uint32_t* cnt, int32_t nwords, int32_t dwords) {
    uint4* c4 = (uint4*)cnt;
    const int32_t n4 = (nwords + dwords + 3) >> 2;
    for (int32_t w = threadIdx.x; w < n4; w += TRI_THREADS) c4[w] = make_uint4(0u, 0u, 0u, 0u);
}

// After the hit phase of a CHECK8 item: every lane of every counting step
// added 1 to exactly one byte of the counter-and-dummy area, and a byte that
// reached 256 wrapped (carrying into its neighbour), which lowers the byte
// sum.  So the counters are exact iff
//   sum of counter bytes + sum of dummy bytes == 64 * counting steps.
// (A dummy byte that wraps only costs a recount.)
__device__ __forceinline__ bool counts_exact(uint32_t* misc, uint32_t bsum, const uint32_t* cnt, uint32_t nwords,
                                             uint32_t dwords) {
    if (threadIdx.x < dwords) bsum = __builtin_amdgcn_sad_u8(cnt[nwords + threadIdx.x], 0u, bsum);
    // wave reduction, then one atomic per wave
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) bsum += (uint32_t)__shfl_xor((int)bsum, d, 64);
    if ((threadIdx.x & 63) == 0 && bsum) atomicAdd(&misc[MISC_SUM], bsum);
    __syncthreads();
    return misc[MISC_SUM] == 64u * misc[MISC_SLOTS];
}

template <int F>
__global__ __launch_bounds__(TRI_THREADS) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_tri(TriArgs a) {
    extern __shared__ uint32_t cnt[];
    constexpr int esz = FmtInfo<F>::esz;
    constexpr int epc = 16 / esz;  // entries per 16-byte chunk
    uint32_t* const misc = cnt + tri_misc_off(a.S, a.dbytes) / 4;

    if (threadIdx.x == 0) item_to_lds<esz>(a, misc);
    __syncthreads();
    ItemGeom gm;
    if (!item_from_lds<esz>(misc, gm)) return;
    const int64_t i = gm.i, lo = gm.lo;
    const int32_t width = gm.width, shift = gm.shift, nchunk = gm.nchunk;
    char* const dst_al = a.out + gm.dst;
    const double ri = a.rinv[i];

    if (a.mode == TRI_MODE_WIDE16) {
        redo_wide<F>(a, cnt, gm, ri);
        return;
    }
    zero_counters(cnt, gm.nwords, (int32_t)(a.dbytes / 4u));
    if (threadIdx.x < TRI_MISC_ZEROED) misc[threadIdx.x] = 0u;
    if constexpr (F == I8 || F == U8) row_table<F>(a, ri, misc);
    __syncthreads();
    // counters cover units [0, nchunk * units-per-chunk): hits outside the
    // item's columns but inside that range land in the unstored padding
    const bool check = a.mode == TRI_MODE_CHECK8;
    const uint32_t cap = (uint32_t)gm.nwords * 4u;
    const uint32_t steps = lo >= shift ? hit_phase<8>(a, i, lo, shift, cap + dummy_unit8(a.dbytes))
                                       : hit_phase<8, true>(a, i, lo, shift, cap + dummy_unit8(a.dbytes));
    if (check && (threadIdx.x & 63) == 0) atomicAdd(&misc[MISC_SLOTS], steps);
    __syncthreads();

    uint32_t bsum = 0;  // sum of the counter bytes this thread read
    const bool has_diag = (lo == i);
    const uint4* c4 = (const uint4*)cnt;
    if constexpr (F == I8 || F == U8) {
        const uint32_t lut_lo = misc[MISC_LUT_LO], lut_hi = misc[MISC_LUT_HI], uc = misc[MISC_UC];
        const uint32_t kuc = (0x80u - uc) * 0x01010101u;
        const uint32_t dcode = code_of<F>(1.0, a.scale, a.zp);
        // Stores chunk ck's codes o: whole chunks with one 16-byte
        // non-temporal store, the first and last chunk of the item byte by
        // byte (only the item's own entries).
        auto store_chunk = [&](int32_t ck, uint32_t (&o)[4]) {
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
        };
        // Chunks whose 16 counts are all below uc are coded by the row table,
        // four bytes at a time.  A chunk with a count >= uc needs its
        // columns' r_j; it is only marked here (bit k of `defer`: chunk
        // threadIdx.x + k * TRI_THREADS; nchunk <= S/16 + 2, so k < 32) and coded
        // after the loop, so the loop stays free of calls and loads.
        uint32_t defer = 0;
        int32_t k = 0;
        for (int32_t ck = threadIdx.x; ck < nchunk; ck += TRI_THREADS, ++k) {
            const uint4 w = c4[ck];
            if (check) {
                bsum = __builtin_amdgcn_sad_u8(w.x, 0u, bsum);
                bsum = __builtin_amdgcn_sad_u8(w.y, 0u, bsum);
                bsum = __builtin_amdgcn_sad_u8(w.z, 0u, bsum);
                bsum = __builtin_amdgcn_sad_u8(w.w, 0u, bsum);
            }
            if ((over_uc(w.x, kuc) | over_uc(w.y, kuc) | over_uc(w.z, kuc) | over_uc(w.w, kuc)) != 0u) {
                defer |= 1u << k;
                continue;
            }
            uint32_t o[4];
            o[0] = __builtin_amdgcn_perm(lut_hi, lut_lo, w.x);
            o[1] = __builtin_amdgcn_perm(lut_hi, lut_lo, w.y);
            o[2] = __builtin_amdgcn_perm(lut_hi, lut_lo, w.z);
            o[3] = __builtin_amdgcn_perm(lut_hi, lut_lo, w.w);
            store_chunk(ck, o);
        }
        // the marked chunks: exact codes for the counts >= uc
        while (defer) {
            const int32_t ck = threadIdx.x + __builtin_ctz(defer) * TRI_THREADS;
            defer &= defer - 1u;
            const uint4 w = c4[ck];
            const int64_t jb = lo + (int64_t)ck * 16 - shift;  // column of byte 0
            const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
            uint32_t o[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) o[q] = __builtin_amdgcn_perm(lut_hi, lut_lo, wv[q]);
            fix_codes<F>(o, wv, uc, ri, a.rinv, jb, shift - ck * 16, shift + width - ck * 16, a.scale, a.zp);
            store_chunk(ck, o);
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
            if (check) {
                bsum = __builtin_amdgcn_sad_u8(cw[0], 0u, bsum);
                bsum = __builtin_amdgcn_sad_u8(cw[1], 0u, bsum);
            }
            const int32_t first = ck * epc, last = first + epc;
            const bool whole = first >= shift && last <= shift + width;
            if (!whole) {
                // the item's first or last chunk: counters outside the item
                // hold no column (a wrapped last column's carry can land in
                // the byte after it); as zeros they read no r_j
#pragma unroll
                for (int b = 0; b < epc; ++b)
                    if (first + b < shift || first + b >= shift + width) cw[b >> 2] &= ~(0xffu << (8 * (b & 3)));
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
            if (whole) {
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
    if (check && !counts_exact(misc, bsum, cnt, (uint32_t)gm.nwords, a.dbytes / 4u)) redo_wide<F>(a, cnt, gm, ri);
}

// NF4: two entries per byte.  Nibble position g(e) = e - e_base + (e_base & 1)
// relative to the byte `out`.  Bytes with both nibbles inside the item are
// stored whole; a byte shared with a neighbouring item (row boundaries) is
// merged with 32-bit atomics on its own nibble only.
__global__ __launch_bounds__(TRI_THREADS) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_tri_nf4(TriArgs a) {
    extern __shared__ uint32_t cnt[];
    uint32_t* const misc = cnt + tri_misc_off(a.S, a.dbytes) / 4;

    if (threadIdx.x == 0) item_to_lds<0>(a, misc);
    __syncthreads();
    ItemGeom gm;
    if (!item_from_lds<0>(misc, gm)) return;
    const int64_t i = gm.i, lo = gm.lo;
    const int32_t width = gm.width, shift = gm.shift, nchunk = gm.nchunk;
    char* const dst_al = a.out + gm.dst;
    const double ri = a.rinv[i];

    if (a.mode == TRI_MODE_WIDE16) {
        redo_wide<NF4>(a, cnt, gm, ri);
        return;
    }
    zero_counters(cnt, gm.nwords, (int32_t)(a.dbytes / 4u));
    if (threadIdx.x < TRI_MISC_ZEROED) misc[threadIdx.x] = 0u;
    row_table<NF4>(a, ri, misc);
    __syncthreads();
    const bool check = a.mode == TRI_MODE_CHECK8;
    const uint32_t cap = (uint32_t)gm.nwords * 4u;
    const uint32_t steps = lo >= shift ? hit_phase<8>(a, i, lo, shift, cap + dummy_unit8(a.dbytes))
                                       : hit_phase<8, true>(a, i, lo, shift, cap + dummy_unit8(a.dbytes));
    if (check && (threadIdx.x & 63) == 0) atomicAdd(&misc[MISC_SLOTS], steps);
    __syncthreads();

    uint32_t bsum = 0;
    const uint32_t dcode = code_of<NF4>(1.0, 0.f, 0.f);
    const uint32_t lut_lo = misc[MISC_LUT_LO], lut_hi = misc[MISC_LUT_HI], uc = misc[MISC_UC];
    const uint32_t kuc = (0x80u - uc) * 0x01010101u;
    const bool has_diag = (lo == i);
    const uint4* c4 = (const uint4*)cnt;
    // Packs the byte codes of chunk ck (32 entries) into 16 nibble bytes and
    // stores them: whole chunks with one non-temporal store, boundary bytes
    // shared with a neighbouring item merged on their own nibble.
    auto store_chunk = [&](int32_t ck, uint32_t (&codes)[8]) {
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
    };
    // as in k_tri: chunks with a count >= uc are marked (bit k of defer)
    // and coded exactly after the table-driven loop
    uint32_t defer = 0;
    int32_t k = 0;
    for (int32_t ck = threadIdx.x; ck < nchunk; ck += TRI_THREADS, ++k) {
        // 32 counters -> 32 nibble codes -> 16 bytes
        uint32_t cw[8];
        const uint4 wa = c4[2 * ck], wb = c4[2 * ck + 1];
        cw[0] = wa.x; cw[1] = wa.y; cw[2] = wa.z; cw[3] = wa.w;
        cw[4] = wb.x; cw[5] = wb.y; cw[6] = wb.z; cw[7] = wb.w;
        uint32_t over = 0u;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            if (check) bsum = __builtin_amdgcn_sad_u8(cw[q], 0u, bsum);
            over |= over_uc(cw[q], kuc);
        }
        if (over != 0u) {
            defer |= 1u << k;
            continue;
        }
        uint32_t codes[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) codes[q] = __builtin_amdgcn_perm(lut_hi, lut_lo, cw[q]);
        store_chunk(ck, codes);
    }
    while (defer) {
        const int32_t ck = threadIdx.x + __builtin_ctz(defer) * TRI_THREADS;
        defer &= defer - 1u;
        const uint4 wa = c4[2 * ck], wb = c4[2 * ck + 1];
        const uint32_t cw[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
        const int64_t jb = lo + (int64_t)ck * 32 - shift;
        uint32_t codes[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) codes[q] = __builtin_amdgcn_perm(lut_hi, lut_lo, cw[q]);
        fix_codes<NF4>(codes, cw, uc, ri, a.rinv, jb, shift - ck * 32, shift + width - ck * 32, 0.f, 0.f);
        store_chunk(ck, codes);
    }
    if (check && !counts_exact(misc, bsum, cnt, (uint32_t)gm.nwords, a.dbytes / 4u)) redo_wide<NF4>(a, cnt, gm, ri);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

static int64_t ceil_div_i(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Dummy area of a launch of T trees: one word per lane shared by the waves
// when no dummy byte can reach 256 in a checked launch (T <= 255, which is
// not checked, or four waves' counting steps within the CHECK8 limit of
// 192), else one word per thread.
static uint32_t tri_dummy_bytes(int32_t T) {
    if (T <= 255) return TRI_DUMMY_SHARED_BYTES;
    const int64_t groups = ceil_div_i((T + 15) / 16, TRI_WAVES);
    return 4 * 16 * groups <= 192 ? TRI_DUMMY_SHARED_BYTES : TRI_DUMMY_BYTES;
}

static int tri_segment_cols(rfxp_ctx* ctx, uint32_t dbytes) {
    // Columns per item: one counter byte each (NF4: one per nibble entry),
    // plus the alignment slack, the dummy words and the item scalars
    // (tri_lds_bytes), two workgroups per CU (160 KB of LDS on gfx950).
    const int half = std::min(ctx->max_lds, 160 * 1024) / 2;
    int S = half - (int)dbytes - TRI_MISC_WORDS * 4 - 64 - 16;
    S = std::max(S, 4096) & ~63;
    return S;
}

// Counter mode of a launch (TRI_MODE_*).
static int tri_mode(int32_t T) {
    if (T <= 255) return TRI_MODE_EXACT8;
    // counting steps of the busiest wave: one per group of 16 trees and
    // record (runs past 64 members add steps, which at worst cost a recount)
    const int64_t groups = ceil_div_i((T + 15) / 16, TRI_WAVES);
    const int64_t steps = 16 * groups;
    return steps <= 192 ? TRI_MODE_CHECK8 : TRI_MODE_WIDE16;
}

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
    if (N < 0 || T < 1 || T > 65535 || nleaf < 1 || nleaf > (1 << 29))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_set_forest: need N >= 0, 1 <= T <= 65535, 1 <= nleaf <= 2^29");
    if (N > MAX_FOREST_N)
        return set_error(ctx, RFXP_ERR_UNSUPPORTED, "rfxp_set_forest: N above 2^31 - 2 is not supported");
    if (N > 0 && (!leaf || !oob_words))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_set_forest: leaf / oob_words are NULL");
    if (oob_ld < (N + 31) / 32)
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_set_forest: oob_ld < ceil(N/32)");
    if (N > 0 && (!is_device_pointer(leaf) || !is_device_pointer(oob_words) || (nout && !is_device_pointer(nout))))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_set_forest: inputs must be device pointers");
    if ((int64_t)N * T + MEM_PAD > (1LL << 30) - 1)
        return set_error(ctx, RFXP_ERR_UNSUPPORTED, "rfxp_set_forest: N*T must stay below 2^30");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    ctx->N = N;
    ctx->T = T;
    ctx->L = nleaf;
    LeafView v{leaf, stride_i, stride_t, oob_words, oob_ld, N, T, nleaf, 0, 0};
    const ForestSizes z = forest_sizes(v, nout == nullptr, ctx->max_lds);
    if (int rc = ctx_forest_bufs(ctx, z, ctx->bkt_off, ctx->bkt_mem, ctx->fb)) return rc;
    ctx->ldr = z.ldr;
    ctx->lmax = z.lmax;
    if (int rc = pack_forest(ctx, v, nout, ctx->fb)) return rc;
    ctx->fo_leaf = leaf;
    ctx->fo_si = stride_i;
    ctx->fo_st = stride_t;
    ctx->fo_oob = oob_words;
    ctx->fo_old = oob_ld;
    ctx->forest_ready = true;
    return RFXP_OK;
}

// Workgroups per launch: gridDim.x * blockDim.x must stay below 2^32, and a
// multiple of 8 keeps the slot -> XCD mapping of every chunk aligned.
constexpr int64_t TRI_MAX_GRID = (int64_t)((1ull << 32) / TRI_THREADS) - 8;

// Number of workgroup slots of a row band (idle slots included).
static int64_t tri_slot_count(int64_t N, int32_t S, int64_t r0, int64_t r1) {
    if (r0 >= r1) return 0;
    const TriLevels L = tri_levels_of(N, S, r0, r1);
    return tri_slots_before(L, L.G);
}

extern "C" int64_t rfxp_upper_work_item(int64_t N, int32_t S, int64_t r0, int64_t r1, int64_t e, int64_t* row,
                                        int64_t* col) {
    if (N < 1 || S < 1 || r0 < 0 || r1 > N || r0 >= r1) return -1;
    const int64_t n = tri_slot_count(N, S, r0, r1);
    if (e >= 0 && e < n && row && col) {
        int64_t i, k;
        const bool ok = tri_slot(tri_levels_of(N, S, r0, r1), e, i, k);
        *row = ok ? i : -1;
        *col = ok ? i + k * S : -1;
    }
    return n;
}

extern "C" int64_t rfxp_upper_launches(int64_t n_items) {
    return n_items <= 0 ? 0 : (n_items + TRI_MAX_GRID - 1) / TRI_MAX_GRID;
}

template <class K>
static hipError_t launch_items(rfxp_ctx* ctx, K kernel, TriArgs a, int64_t n_items, size_t lds) {
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    // items in chunks of at most TRI_MAX_GRID workgroups, in stream order
    for (int64_t b = 0; b < n_items; b += TRI_MAX_GRID) {
        a.item_base = b;
        const int64_t n = std::min<int64_t>(TRI_MAX_GRID, n_items - b);
        hipLaunchKernelGGL(kernel, dim3((unsigned)n), dim3(TRI_THREADS), lds, ctx->stream, a);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

namespace rfxp {

int upper_check_args(rfxp_ctx* ctx, const char* who, int64_t N, int fmt, float scale, float zp, int64_t r0,
                     int64_t r1, const void* out) {
    if (fmt < F32 || fmt > U16) return set_error(ctx, RFXP_ERR_INVALID, std::string(who) + ": unknown format");
    if (r0 < 0 || r1 > N || r0 > r1) return set_error(ctx, RFXP_ERR_INVALID, std::string(who) + ": bad row range");
    if ((fmt == I8 || fmt == U8) && (!std::isfinite(scale) || scale == 0.0f || !std::isfinite(zp)))
        return set_error(ctx, RFXP_ERR_INVALID, std::string(who) + ": scale must be finite and non-zero, zp finite");
    if (r0 == r1) return RFXP_OK;
    if (!out || !is_device_pointer(out))
        return set_error(ctx, RFXP_ERR_INVALID, std::string(who) + ": out must be a device pointer");
    const int esz = (fmt == F32) ? 4 : (fmt == F16 || fmt == U16) ? 2 : 1;
    if (((uintptr_t)out) % esz != 0)
        return set_error(ctx, RFXP_ERR_INVALID, std::string(who) + ": out is not aligned to its entry size");
    return RFXP_OK;
}

// Rows [r0, r1) of the triangle of the forest index fb (N samples, T trees)
// on ctx->stream.  The kernels derive each item's (row, segment) from its
// index, so consecutive calls on one stream share no host-written state.
int upper_launch(rfxp_ctx* ctx, const ForestBufs& fb, int64_t N, int32_t T, int fmt, float scale, float zp,
                 int64_t r0, int64_t r1, void* out) {
    if (r0 == r1) return RFXP_OK;
    const uint32_t dbytes = tri_dummy_bytes(T);
    const int32_t S = tri_segment_cols(ctx, dbytes);
    TriArgs a;
    a.roff = fb.roff;
    a.rlen = fb.rlen;
    a.ldr = fb.ldr;
    a.lng = fb.lng;
    a.lngn = fb.lngn;
    a.lmax = fb.lmax;
    a.mem = fb.mem;
    a.mem_bytes = (uint32_t)(((uint64_t)T * (uint64_t)fb.ms + MEM_PAD) * 4u);
    a.rinv = fb.rinv;
    a.rr = fb.rrange;
    a.N = N;
    a.T = T;
    a.S = S;
    a.lev = tri_levels_of(N, S, r0, r1);
    a.item_base = 0;
    a.e_base = tri_idx(N, r0, r0);
    a.out = (char*)out;
    a.scale = scale;
    a.zp = zp;
    a.flags = fb.flags;
    a.mode = tri_mode(T);
    a.dbytes = dbytes;
    const int64_t n_items = tri_slot_count(N, S, r0, r1);
    const size_t lds = tri_lds_bytes(S, dbytes);
    hipError_t e;
    {
        LaunchTimer tm(ctx, "tri");
        switch (fmt) {
            case F32: e = launch_items(ctx, k_tri<F32>, a, n_items, lds); break;
            case F16: e = launch_items(ctx, k_tri<F16>, a, n_items, lds); break;
            case I8: e = launch_items(ctx, k_tri<I8>, a, n_items, lds); break;
            case U8: e = launch_items(ctx, k_tri<U8>, a, n_items, lds); break;
            case U16: e = launch_items(ctx, k_tri<U16>, a, n_items, lds); break;
            default: e = launch_items(ctx, k_tri_nf4, a, n_items, lds); break;
        }
    }
    if (e != hipSuccess) return hip_error(ctx, e, "k_tri launch");
    return RFXP_OK;
}

}  // namespace rfxp

extern "C" int rfxp_upper(rfxp_ctx* ctx, int fmt, float scale, float zp, int64_t r0, int64_t r1, void* out) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (!ctx->forest_ready) return set_error(ctx, RFXP_ERR_STATE, "rfxp_upper: no forest set");
    if (int rc = upper_check_args(ctx, "rfxp_upper", ctx->N, fmt, scale, zp, r0, r1, out)) return rc;
    if (r0 == r1) return RFXP_OK;
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    return upper_launch(ctx, ctx->fb, ctx->N, ctx->T, fmt, scale, zp, r0, r1, out);
}

extern "C" int rfxp_upper_recounts(rfxp_ctx* ctx, int64_t* count) {
    if (!ctx || !count) return RFXP_ERR_INVALID;
    if (!ctx->forest_ready) return set_error(ctx, RFXP_ERR_STATE, "rfxp_upper_recounts: no forest set");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    int32_t v = 0;
    RFXP_HIP(ctx, hipMemcpyAsync(&v, ctx->fb.flags, sizeof(v), hipMemcpyDeviceToHost, ctx->stream));
    RFXP_HIP(ctx, hipStreamSynchronize(ctx->stream));
    *count = v;
    return RFXP_OK;
}

namespace rfxp {

// Min and max of x[0, n): one (min, max) pair per block from a grid-stride
// loop, into part[2 * blockIdx.x], part[2 * blockIdx.x + 1].
__global__ __launch_bounds__(256) void k_minmax_f32(const float* x, int64_t n, float* part) {
    __shared__ float smn[256], smx[256];
    float mn = 3.0e38f, mx = -3.0e38f;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const float v = x[i];
        mn = fminf(mn, v);
        mx = fmaxf(mx, v);
    }
    smn[threadIdx.x] = mn;
    smx[threadIdx.x] = mx;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (threadIdx.x < (unsigned)s) {
            smn[threadIdx.x] = fminf(smn[threadIdx.x], smn[threadIdx.x + s]);
            smx[threadIdx.x] = fmaxf(smx[threadIdx.x], smx[threadIdx.x + s]);
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        part[2 * blockIdx.x] = smn[0];
        part[2 * blockIdx.x + 1] = smx[0];
    }
}

// Folds the nblk block pairs into run[0..1], starting from run's previous
// contents unless first.
__global__ void k_minmax_fold(const float* part, int32_t nblk, float* run, int32_t first) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    float mn = first ? 3.0e38f : run[0], mx = first ? -3.0e38f : run[1];
    for (int32_t b = 0; b < nblk; ++b) {
        mn = fminf(mn, part[2 * b]);
        mx = fmaxf(mx, part[2 * b + 1]);
    }
    run[0] = mn;
    run[1] = mx;
}

// Entries per band of rfxp_upper_minmax.
constexpr int64_t MINMAX_BAND = (int64_t)1 << 26;
constexpr int32_t MINMAX_BLOCKS = 1024;

}  // namespace rfxp

extern "C" int rfxp_upper_minmax(rfxp_ctx* ctx, int64_t r0, int64_t r1, float* minmax) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (!ctx->forest_ready) return set_error(ctx, RFXP_ERR_STATE, "rfxp_upper_minmax: no forest set");
    const int64_t N = ctx->N;
    if (!minmax || r0 < 0 || r1 > N || r0 >= r1)
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_upper_minmax: need 0 <= row_begin < row_end <= N, minmax");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    // a band holds whole rows: at least one row (N - r0 <= N entries)
    const int64_t band = std::max<int64_t>(MINMAX_BAND, N);
    RFXP_HIP(ctx, ctx->mm_ws.ensure((size_t)band));
    RFXP_HIP(ctx, ctx->mm_part.ensure((size_t)2 * MINMAX_BLOCKS + 2));
    float* run = ctx->mm_part.p + 2 * MINMAX_BLOCKS;
    bool first = true;
    for (int64_t a = r0; a < r1;) {
        // rows [a, b): as many whole rows as the band holds (at least one)
        int64_t b = a + 1;
        while (b < r1 && tri_idx(N, b + 1, b + 1) - tri_idx(N, a, a) <= band) ++b;
        const int64_t count = tri_idx(N, b, b) - tri_idx(N, a, a);
        if (int rc = upper_launch(ctx, ctx->fb, N, ctx->T, F32, 1.0f, 0.0f, a, b, ctx->mm_ws.p)) return rc;
        const int32_t nblk = (int32_t)std::min<int64_t>(MINMAX_BLOCKS, (count + 255) / 256);
        hipLaunchKernelGGL(k_minmax_f32, dim3((unsigned)nblk), dim3(256), 0, ctx->stream, ctx->mm_ws.p, count,
                           ctx->mm_part.p);
        hipLaunchKernelGGL(k_minmax_fold, dim3(1), dim3(64), 0, ctx->stream, ctx->mm_part.p, nblk, run,
                           (int32_t)first);
        if (int rc = check_launch(ctx, "k_minmax launch")) return rc;
        first = false;
        a = b;
    }
    float host[2];
    RFXP_HIP(ctx, hipMemcpyAsync(host, run, sizeof(host), hipMemcpyDeviceToHost, ctx->stream));
    RFXP_HIP(ctx, hipStreamSynchronize(ctx->stream));
    minmax[0] = host[0];
    minmax[1] = host[1];
    return RFXP_OK;
}

extern "C" void rfxp_quant_scale(float min_val, float max_val, float* scale, float* zero_point) {
    float s = (max_val - min_val) / 255.0f;
    if (s < 1e-10f) s = 1.0f / 127.0f;
    if (scale) *scale = s;
    if (zero_point) *zero_point = -min_val / s;
}

extern "C" int rfxp_get_nout(rfxp_ctx* ctx, int32_t* nout) {
    if (!ctx || !nout) return RFXP_ERR_INVALID;
    if (!ctx->forest_ready) return set_error(ctx, RFXP_ERR_STATE, "rfxp_get_nout: no forest set");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    if (ctx->N == 0) return RFXP_OK;
    RFXP_HIP(ctx, hipMemcpyAsync(nout, ctx->nout.p, sizeof(int32_t) * ctx->N, hipMemcpyDeviceToDevice, ctx->stream));
    return RFXP_OK;
}
