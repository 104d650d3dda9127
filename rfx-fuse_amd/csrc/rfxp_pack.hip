// Forest index construction (see rfxp_forest.hpp for the layout).
//
// Forests with 2L <= 8192 buckets per tree take the per-part path (see
// k_part_hist below); larger ones the whole-tree path: k_pack_hist (one
// workgroup per tree) or k_tree_hist + k_seg_scan (bucket histogram and
// offsets, and the tree's 16-bit bucket keys), k_tree_records +
// k_rec_transpose (the sample-major records), k_pack_scatter (one workgroup
// per tree and window of members: member lists built in LDS and written out
// coalesced -- scattering 4-byte ids straight to HBM costs a partial-line
// write each).  Trees are mapped to workgroups so that related work lands on
// one XCD, where the later workgroups of a tree read its data from L2.
//
// nout_i = sum over trees of the OOB bits (src/rf_bootstrap.cpp:67-70) is
// summed by the kernel that writes the sample-major records (k_part_records
// on the per-part path, k_rec_transpose on the whole-tree path) into a zeroed
// array; k_nout_final takes its reciprocal and the reciprocal's range.
// Reference sets (top-K, low rank) take the per-segment path (k_seg_*).
#include <algorithm>

#include "rfxp_device.hpp"
#include "rfxp_forest.hpp"

namespace rfxp {

constexpr int PACK_THREADS = 1024;
constexpr int PACK_KR = 8;  // keys per thread per round

// Exclusive scan of cnt[0..nb) (one workgroup) into off0[0..nb] and the
// global offsets table; cnt becomes the running cursor.
__device__ void scan_offsets(uint32_t* cnt, uint32_t* off0, int32_t nb, uint32_t* part, int32_t* goff) {
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
    uint32_t run = part[tid] - s;
    for (int32_t b = b0; b < b1; ++b) {
        uint32_t c = cnt[b];
        cnt[b] = run;
        off0[b] = run;
        goff[b] = (int32_t)run;
        run += c;
    }
    if (tid == PACK_THREADS - 1) {
        off0[nb] = part[tid];
        goff[nb] = (int32_t)part[tid];
    }
    __syncthreads();
}

// Pass A, one 1024-thread workgroup per tree when its 2L + 1 counters fit
// in LDS: bucket histogram, exclusive scan into the global offsets, and the
// tree's bucket ids as uint16 (`key16`, rows of ldk entries, pads 0xffff;
// written only when 2L < 0xffff, else NULL).  Keys are held in registers,
// PACK_KR per thread per round, all loads of a round issued before the first
// atomic.
__global__ __launch_bounds__(PACK_THREADS) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_pack_hist(
    LeafView v, int32_t* goff_all, uint16_t* key16, int64_t ldk) {
    extern __shared__ uint32_t sh[];
    __shared__ uint32_t part[PACK_THREADS];
    const uint32_t bid = blockIdx.x;
    const int32_t t = (int32_t)((((bid >> 3) >> 4) << 3) + (bid & 7)) * 16 + (int32_t)((bid >> 3) & 15);
    if (t >= v.T) return;
    const int32_t nb = view_buckets(v);
    uint32_t* cnt = sh;
    uint32_t* off0 = cnt + (nb + 1);
    for (int32_t b = threadIdx.x; b <= nb; b += PACK_THREADS) cnt[b] = 0u;
    __syncthreads();
    const int64_t N = v.N;
    const int64_t round = (int64_t)PACK_THREADS * PACK_KR;
    uint16_t* kt = key16 ? key16 + (int64_t)t * ldk : nullptr;
    for (int64_t base = 0; base < N; base += round) {
        KeyLoad ld[PACK_KR];
#pragma unroll
        for (int k = 0; k < PACK_KR; ++k) {
            const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
            ld[k] = key_load(v, i < N ? i : 0, t);
        }
        int32_t key[PACK_KR];
#pragma unroll
        for (int k = 0; k < PACK_KR; ++k) {
            const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
            key[k] = i < N ? key_bucket(v, ld[k], i) : -1;
        }
#pragma unroll
        for (int k = 0; k < PACK_KR; ++k) {
            if (key[k] >= 0) atomicAdd(&cnt[key[k]], 1u);
            const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
            if (kt && i < ldk) kt[i] = key[k] >= 0 ? (uint16_t)key[k] : (uint16_t)0xffffu;
        }
    }
    __syncthreads();
    scan_offsets(cnt, off0, nb, part, goff_all + (int64_t)t * (nb + 1));
}

// Pass A for trees whose 2L + 1 counters do not fit in LDS: workgroup
// (tree t, range r) counts the buckets [r * TREE_HR, (r + 1) * TREE_HR) of
// tree t in LDS, reading all of the tree's labels (the ranges of a tree run
// one after another on one XCD, so the later ones read them from L2), and
// writes its range of cnt[t]; range 0 also writes the tree's 16-bit keys
// (when key16 is not NULL).  k_seg_scan then turns the counts into offsets.
constexpr int TREE_HR = 16384;  // buckets per range (64 KB of LDS)

__global__ __launch_bounds__(PACK_THREADS) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_tree_hist(
    LeafView v, int32_t nrange, uint32_t* cnt_all, uint16_t* key16, int64_t ldk) {
    extern __shared__ uint32_t sh[];
    const uint32_t bid = blockIdx.x;
    const uint32_t xcd = bid & 7, slot = bid >> 3;
    const int64_t lin = (int64_t)xcd * (gridDim.x >> 3) + slot;
    const int32_t t = (int32_t)(lin / nrange), r = (int32_t)(lin % nrange);
    if (t >= v.T) return;
    const int32_t nb = view_buckets(v);
    const int32_t b0 = r * TREE_HR, nr = min(nb - b0, TREE_HR);
    for (int32_t b = threadIdx.x; b < nr; b += PACK_THREADS) sh[b] = 0u;
    __syncthreads();
    const int64_t N = v.N;
    const int64_t round = (int64_t)PACK_THREADS * PACK_KR;
    uint16_t* kt = (key16 && r == 0) ? key16 + (int64_t)t * ldk : nullptr;
    for (int64_t base = 0; base < N; base += round) {
        KeyLoad ld[PACK_KR];
#pragma unroll
        for (int k = 0; k < PACK_KR; ++k) {
            const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
            ld[k] = key_load(v, i < N ? i : 0, t);
        }
#pragma unroll
        for (int k = 0; k < PACK_KR; ++k) {
            const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
            const int32_t b = i < N ? key_bucket(v, ld[k], i) : -1;
            const uint32_t rb = (uint32_t)(b - b0);
            if (b >= 0 && rb < (uint32_t)nr) atomicAdd(&sh[rb], 1u);
            if (kt && i < ldk) kt[i] = b >= 0 ? (uint16_t)b : (uint16_t)0xffffu;
        }
    }
    __syncthreads();
    uint32_t* cnt = cnt_all + (int64_t)t * (nb + 1) + b0;
    for (int32_t b = threadIdx.x; b < nr; b += PACK_THREADS) cnt[b] = sh[b];
}

// Tree-major records for the whole-tree path: workgroup (tree t, chunk c of
// TREE_REC_CHUNK samples) writes the records of its samples in sample order
// (the run of (i, t) is the whole bucket with the other OOB bit), so every
// store is coalesced; k_rec_transpose then makes them sample-major.  The
// tree's bucket offsets (2L + 1 words) are looked up in LDS when they fit
// (IN_LDS), else in global memory, where they stay in L2: the chunks of a
// tree run one after another on one XCD.
constexpr int TREE_REC_CHUNK = 32768;

template <bool IN_LDS>
__global__ __launch_bounds__(PACK_THREADS) void k_tree_records(LeafView v, const uint16_t* key16, int64_t ldk,
                                                             const int32_t* goff_all, int32_t nchunk, uint32_t* roffT,
                                                             uint16_t* rlenT) {
    extern __shared__ uint32_t off_lds[];
    const uint32_t bid = blockIdx.x;
    const uint32_t xcd = bid & 7, slot = bid >> 3;
    const int64_t lin = (int64_t)xcd * (gridDim.x >> 3) + slot;
    const int32_t t = (int32_t)(lin / nchunk), c = (int32_t)(lin % nchunk);
    if (t >= v.T) return;
    const int32_t nb = view_buckets(v);
    const int32_t* goff = goff_all + (int64_t)t * (nb + 1);
    const uint32_t* off = IN_LDS ? off_lds : (const uint32_t*)goff;
    if constexpr (IN_LDS) {
        for (int32_t b = threadIdx.x; b <= nb; b += PACK_THREADS) off_lds[b] = (uint32_t)goff[b];
        __syncthreads();
    }
    const int64_t N = v.N;
    const int64_t i0 = (int64_t)c * TREE_REC_CHUNK, i1 = min(N, i0 + TREE_REC_CHUNK);
    uint32_t* ro = roffT + (int64_t)t * N;
    uint16_t* rl = rlenT + (int64_t)t * N;
    const uint32_t tbase = (uint32_t)t * (uint32_t)N;
    const int64_t round = (int64_t)PACK_THREADS * PACK_KR;
    for (int64_t base = i0; base < i1; base += round) {
        int32_t key[PACK_KR];
        if (key16) {
            const uint16_t* kt = key16 + (int64_t)t * ldk;
            uint32_t kk[PACK_KR];
#pragma unroll
            for (int k = 0; k < PACK_KR; ++k) {
                const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
                kk[k] = kt[i < i1 ? i : i0];
            }
#pragma unroll
            for (int k = 0; k < PACK_KR; ++k) key[k] = kk[k] == 0xffffu ? -1 : (int32_t)kk[k];
        } else {
            KeyLoad ld[PACK_KR];
#pragma unroll
            for (int k = 0; k < PACK_KR; ++k) {
                const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
                ld[k] = key_load(v, i < i1 ? i : i0, t);
            }
#pragma unroll
            for (int k = 0; k < PACK_KR; ++k) {
                const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
                key[k] = key_bucket(v, ld[k], i);
            }
        }
        // every lookup of the round first (bucket 0's for empty records)
        uint32_t st[PACK_KR], en[PACK_KR];
#pragma unroll
        for (int k = 0; k < PACK_KR; ++k) {
            const uint32_t ob = key[k] >= 0 ? (uint32_t)(key[k] ^ 1) : 0u;
            st[k] = off[ob];
            en[k] = off[ob + 1];
        }
#pragma unroll
        for (int k = 0; k < PACK_KR; ++k) {
            const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
            if (i >= i1) continue;
            const bool ok = key[k] >= 0;
            ro[i] = ok ? (tbase + st[k]) * 4u : 0u;
            rl[i] = ok ? (uint16_t)(min(en[k] - st[k], REC_LONG) * 4u) : (uint16_t)0;
        }
    }
}

// Pass B: workgroup (tree t, window w) owns the buckets whose offsets start
// in [w*win, (w+1)*win) (bucket pairs kept together).  It reads
// the tree's bucket ids again -- from key16, eight per 16-byte load, when
// pass A wrote it, else from the leaves -- places its members in an LDS
// copy of its slice of mem[t] through LDS cursors, and writes the slice
// with coalesced stores.  Members beyond the LDS slice (a window grown by
// one very large bucket) are written directly.
// The LDS holds win staged members and ncur cursors, win + ncur =
// PACK_STAGE_WORDS (plus 8 bytes of statics: two workgroups per CU).  The
// host splits it by the forest's members per bucket: a window of win members
// spans about win * 2L / N buckets, and ncur leaves room for half as many
// again (windows whose buckets do not fit use global cursors).
constexpr int PACK_STAGE_WORDS = 20464;
constexpr int SCAT_LOADS = 4;    // 16-byte key loads in flight per thread

__device__ __forceinline__ int32_t first_bucket_at(const int32_t* off, int32_t nb, int64_t pos) {
    // smallest even b in [0, nb] with off[b] >= pos (nb when none)
    int32_t lo = 0, hi = nb / 2;  // search over pair index
    while (lo < hi) {
        const int32_t mid = (lo + hi) >> 1;
        if ((int64_t)off[2 * mid] >= pos) hi = mid;
        else lo = mid + 1;
    }
    return 2 * lo;
}

__global__ __launch_bounds__(PACK_THREADS) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_pack_scatter(LeafView v, const int32_t* goff_all, uint32_t* mem,
                                                              uint32_t* gcur_all, int32_t nwin, int32_t win,
                                                              const uint16_t* key16, int64_t ldk) {
    extern __shared__ uint32_t sh[];
    __shared__ int32_t s_b0, s_b1;
    // (tree, window) -> workgroup: the windows of a tree are consecutive
    // in dispatch order on one XCD
    const uint32_t bid = blockIdx.x;
    const uint32_t xcd = bid & 7, slot = bid >> 3;
    const int64_t lin = (int64_t)xcd * (gridDim.x >> 3) + slot;
    const int32_t t = (int32_t)(lin / nwin);
    const int32_t w = (int32_t)(lin % nwin);
    if (t >= v.T) return;
    const int32_t nb = view_buckets(v);
    const int32_t* off = goff_all + (int64_t)t * (nb + 1);
    if (threadIdx.x == 0) {
        s_b0 = first_bucket_at(off, nb, (int64_t)w * win);
        s_b1 = first_bucket_at(off, nb, (int64_t)(w + 1) * win);
    }
    __syncthreads();
    const int32_t b0 = s_b0, b1 = s_b1;
    if (b0 >= b1) return;
    const uint32_t base_pos = (uint32_t)off[b0];
    const uint32_t end_pos = (uint32_t)off[b1];
    if (end_pos == base_pos) return;
    const int32_t nbk = b1 - b0;
    const bool lds_cur = nbk <= PACK_STAGE_WORDS - win;
    uint32_t* stage = sh;                 // win words
    uint32_t* cur = sh + win;             // the rest: relative cursors
    uint32_t* gcur = gcur_all + (int64_t)t * (nb + 1);
    if (lds_cur) {
        for (int32_t k = threadIdx.x; k < nbk; k += PACK_THREADS) cur[k] = (uint32_t)off[b0 + k] - base_pos;
    } else {
        for (int32_t k = threadIdx.x; k < nbk; k += PACK_THREADS) gcur[b0 + k] = (uint32_t)off[b0 + k] - base_pos;
        __threadfence();
    }
    __syncthreads();
    const int64_t N = v.N;
    uint32_t* memt = mem + (int64_t)t * N;
    auto place = [&](int64_t i, int32_t b) {
        if (b < b0 || b >= b1) return;
        const uint32_t rel = lds_cur ? atomicAdd(&cur[b - b0], 1u) : atomicAdd(&gcur[b], 1u);
        const uint32_t m = (uint32_t)(i + 1);
        if (rel < (uint32_t)win) stage[rel] = m;
        else memt[base_pos + rel] = m;
    };
    if (key16) {
        // eight ids per thread per 16-byte load, SCAT_LOADS loads in flight
        const uint4* k4 = (const uint4*)(key16 + (int64_t)t * ldk);
        const int64_t n8 = ldk / 8;
        for (int64_t q0 = threadIdx.x; q0 < n8; q0 += SCAT_LOADS * PACK_THREADS) {
            uint4 x[SCAT_LOADS];
#pragma unroll
            for (int u = 0; u < SCAT_LOADS; ++u) {
                const int64_t q = q0 + (int64_t)u * PACK_THREADS;
                x[u] = q < n8 ? k4[q] : make_uint4(0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu);
            }
#pragma unroll
            for (int u = 0; u < SCAT_LOADS; ++u) {
                const int64_t i8 = 8 * (q0 + (int64_t)u * PACK_THREADS);
                const uint32_t wv[4] = {x[u].x, x[u].y, x[u].z, x[u].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t lo16 = wv[k] & 0xffffu, hi16 = wv[k] >> 16;
                    if (lo16 != 0xffffu) place(i8 + 2 * k, (int32_t)lo16);
                    if (hi16 != 0xffffu) place(i8 + 2 * k + 1, (int32_t)hi16);
                }
            }
        }
    } else {
        const int64_t round = (int64_t)PACK_THREADS * PACK_KR;
        for (int64_t base = 0; base < N; base += round) {
            KeyLoad ld[PACK_KR];
#pragma unroll
            for (int k = 0; k < PACK_KR; ++k) {
                const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
                ld[k] = key_load(v, i < N ? i : 0, t);
            }
            int32_t key[PACK_KR];
#pragma unroll
            for (int k = 0; k < PACK_KR; ++k) {
                const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
                key[k] = i < N ? key_bucket(v, ld[k], i) : -1;
            }
#pragma unroll
            for (int k = 0; k < PACK_KR; ++k) place(base + (int64_t)k * PACK_THREADS + threadIdx.x, key[k]);
        }
    }
    __syncthreads();
    const uint32_t nst = min(end_pos - base_pos, (uint32_t)win);
    for (uint32_t k = threadIdx.x; k < nst; k += PACK_THREADS) memt[base_pos + k] = stage[k];
}

// ---------------------------------------------------------------------------
// Reference-set path (buckets b = leaf * nseg + segment, L <= SEG_MAX_L): the
// samples of bucket (l, s) all lie in segment s, so one workgroup per
// (tree, segment) sees every member of its L buckets.
//   k_seg_hist    (tree, segment): LDS histogram over the leaves -> the
//                 bucket counts cnt[t][l * nseg + s];
//   k_seg_scan    (tree): exclusive scan of the counts into the offsets;
//   k_seg_scatter (tree, segment): LDS cursors from the offsets; each
//                 member goes straight to its slot in mem[t].
// Every leaf label is read twice in all (once per pass), instead of once per
// member window of the whole-tree path.  The segments of a tree run
// together on one XCD: the buckets (l, s) and (l, s + 1) are neighbours in
// mem[t], so the scattered member writes of a tree merge in that XCD's L2.
// ---------------------------------------------------------------------------
constexpr int SEG_MAX_L = 16384;  // LDS counters per workgroup (64 KB)

// (tree, segment) of a k_seg_* workgroup: consecutive dispatch slots of one
// XCD walk the segments of a tree, trees x, x + 8, x + 16, ... on XCD x.
__device__ __forceinline__ void seg_of_block(uint32_t bid, int32_t nseg, int32_t& t, int32_t& sg) {
    const uint32_t xcd = bid & 7, slot = bid >> 3;
    t = (int32_t)(xcd + 8 * (slot / (uint32_t)nseg));
    sg = (int32_t)(slot % (uint32_t)nseg);
}

__global__ __launch_bounds__(PACK_THREADS) void k_seg_hist(LeafView v, uint32_t* cnt_all) {
    extern __shared__ uint32_t sh[];
    int32_t t, sg;
    seg_of_block(blockIdx.x, v.nseg, t, sg);
    if (t >= v.T) return;
    for (int32_t l = threadIdx.x; l < v.L; l += PACK_THREADS) sh[l] = 0u;
    __syncthreads();
    const int64_t i0 = (int64_t)sg << v.seg_shift, i1 = min(v.N, i0 + ((int64_t)1 << v.seg_shift));
    const int64_t round = (int64_t)PACK_THREADS * PACK_KR;
    for (int64_t base = i0; base < i1; base += round) {
        int32_t lv[PACK_KR];
#pragma unroll
        for (int k = 0; k < PACK_KR; ++k) {
            const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
            lv[k] = i < i1 ? v.leaf[i * v.si + (int64_t)t * v.st] : -1;
        }
#pragma unroll
        for (int k = 0; k < PACK_KR; ++k)
            if (lv[k] >= 0 && lv[k] < v.L) atomicAdd(&sh[lv[k]], 1u);
    }
    __syncthreads();
    const int32_t nb = view_buckets(v);
    uint32_t* cnt = cnt_all + (int64_t)t * (nb + 1);
    for (int32_t l = threadIdx.x; l < v.L; l += PACK_THREADS) cnt[(int64_t)l * v.nseg + sg] = sh[l];
    // the padding bucket of an odd L * nseg is empty
    if (sg == 0 && threadIdx.x == 0 && nb > v.L * v.nseg) cnt[nb - 1] = 0u;
}

// Exclusive scan of a tree's bucket counts in global memory, in place, into
// cnt[0..nb] and goff[0..nb] (one workgroup per tree).  The counts are taken
// SCAN_BATCH chunks of 1024 at a time, one per thread, so every load is
// coalesced and a batch's loads are in flight together; each chunk is scanned
// within its waves, the wave totals go through LDS, and a running carry
// joins the chunks.
constexpr int SCAN_BATCH = 8;

__global__ __launch_bounds__(PACK_THREADS) void k_seg_scan(int32_t nb, int32_t T, uint32_t* cnt_all,
                                                           int32_t* goff_all) {
    __shared__ uint32_t wsum[SCAN_BATCH][PACK_THREADS / 64];
    const int32_t t = blockIdx.x;
    if (t >= T) return;
    uint32_t* cnt = cnt_all + (int64_t)t * (nb + 1);
    int32_t* goff = goff_all + (int64_t)t * (nb + 1);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t carry = 0;
    for (int32_t c0 = 0; c0 < nb; c0 += SCAN_BATCH * PACK_THREADS) {
        uint32_t x[SCAN_BATCH], incl[SCAN_BATCH];
#pragma unroll
        for (int q = 0; q < SCAN_BATCH; ++q) {
            const int32_t b = c0 + q * PACK_THREADS + tid;
            x[q] = b < nb ? cnt[b] : 0u;
        }
#pragma unroll
        for (int q = 0; q < SCAN_BATCH; ++q) {
            uint32_t v = x[q];
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const uint32_t o = (uint32_t)__shfl_up((int)v, d, 64);
                if (lane >= d) v += o;
            }
            incl[q] = v;
            if (lane == 63) wsum[q][wave] = v;
        }
        __syncthreads();
        uint32_t run = carry;
#pragma unroll
        for (int q = 0; q < SCAN_BATCH; ++q) {
            uint32_t before = 0, total = 0;
#pragma unroll
            for (int w = 0; w < PACK_THREADS / 64; ++w) {
                const uint32_t y = wsum[q][w];
                before += w < wave ? y : 0u;
                total += y;
            }
            const int32_t b = c0 + q * PACK_THREADS + tid;
            const uint32_t e = run + before + incl[q] - x[q];
            if (b < nb) {
                cnt[b] = e;
                goff[b] = (int32_t)e;
            }
            run += total;
        }
        carry = run;
        __syncthreads();
    }
    if (tid == 0) {
        cnt[nb] = carry;
        goff[nb] = (int32_t)carry;
    }
}

__global__ __launch_bounds__(PACK_THREADS) void k_seg_scatter(LeafView v, const int32_t* goff_all, uint32_t* mem) {
    extern __shared__ uint32_t cur[];
    int32_t t, sg;
    seg_of_block(blockIdx.x, v.nseg, t, sg);
    if (t >= v.T) return;
    const int32_t nb = view_buckets(v);
    const int32_t* goff = goff_all + (int64_t)t * (nb + 1);
    for (int32_t l = threadIdx.x; l < v.L; l += PACK_THREADS) cur[l] = (uint32_t)goff[(int64_t)l * v.nseg + sg];
    __syncthreads();
    uint32_t* memt = mem + (int64_t)t * v.N;
    const int64_t i0 = (int64_t)sg << v.seg_shift, i1 = min(v.N, i0 + ((int64_t)1 << v.seg_shift));
    const int64_t round = (int64_t)PACK_THREADS * PACK_KR;
    for (int64_t base = i0; base < i1; base += round) {
        int32_t lv[PACK_KR];
#pragma unroll
        for (int k = 0; k < PACK_KR; ++k) {
            const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
            lv[k] = i < i1 ? v.leaf[i * v.si + (int64_t)t * v.st] : -1;
        }
#pragma unroll
        for (int k = 0; k < PACK_KR; ++k) {
            if (lv[k] < 0 || lv[k] >= v.L) continue;
            const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
            memt[atomicAdd(&cur[lv[k]], 1u)] = (uint32_t)(i + 1);
        }
    }
}

// k_seg_scatter with the member writes in leaf order.  A segment's buckets
// (l, s) are spread over the whole of mem[t] (buckets of one segment are
// nseg apart), so the direct 4-byte writes of the trees in flight cover far
// more than the L2 and reach HBM as partial lines.  Here the segment is
// swept in sub-chunks of sc samples: an LDS histogram gives each sample its
// rank in its leaf, a scan gives each leaf's staged run, the members are
// staged as (leaf << 16 | offset in the sub-chunk) and thread k writes
// staged member k to gcur[leaf] + (k - start of the leaf's run).  The
// segments of a tree, on one XCD, sweep the leaves in the same order, so
// the lines they share are written close together in time.
// LDS: cnt[L + 1] (counts, then staged-run starts), gcur[L] (next slot of
// each bucket (l, s) in mem[t]), wsum[16], stg[sc].
constexpr int SEG_SORT_KR = 8;  // samples per thread and sub-chunk, at most

static size_t seg_sorted_lds(int32_t L, int32_t sc) { return (size_t)(2 * L + 1 + 16 + sc) * 4; }

__global__ __launch_bounds__(PACK_THREADS) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_seg_scatter_sorted(
    LeafView v, const int32_t* goff_all, uint32_t* mem, int32_t sc) {
    extern __shared__ uint32_t sh[];
    int32_t t, sg;
    seg_of_block(blockIdx.x, v.nseg, t, sg);
    if (t >= v.T) return;
    const int32_t L = v.L;
    const int32_t nb = view_buckets(v);
    uint32_t* cnt = sh;
    uint32_t* gcur = cnt + L + 1;
    uint32_t* wsum = gcur + L;
    uint32_t* stg = wsum + 16;
    const int32_t* goff = goff_all + (int64_t)t * (nb + 1);
    for (int32_t l = threadIdx.x; l <= L; l += PACK_THREADS) {
        cnt[l] = 0u;
        if (l < L) gcur[l] = (uint32_t)goff[(int64_t)l * v.nseg + sg];
    }
    __syncthreads();
    uint32_t* memt = mem + (int64_t)t * v.N;
    const int64_t i0 = (int64_t)sg << v.seg_shift, i1 = min(v.N, i0 + ((int64_t)1 << v.seg_shift));
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int32_t E = (L + PACK_THREADS - 1) / PACK_THREADS;
    const int32_t l0 = min(L, tid * E), l1 = min(L, l0 + E);
    for (int64_t base = i0; base < i1; base += sc) {
        const int64_t end = min(i1, base + sc);
        // leaves of the sub-chunk (samples base + k * 1024 + tid), and each
        // sample's rank among the sub-chunk's members of its leaf
        uint32_t lr[SEG_SORT_KR];  // leaf << 16 | rank, or ~0u
        int32_t lv[SEG_SORT_KR];
#pragma unroll
        for (int k = 0; k < SEG_SORT_KR; ++k) {
            const int64_t i = base + (int64_t)k * PACK_THREADS + tid;
            lv[k] = v.leaf[(i < end ? i : i0) * v.si + (int64_t)t * v.st];
        }
#pragma unroll
        for (int k = 0; k < SEG_SORT_KR; ++k) {
            const int64_t i = base + (int64_t)k * PACK_THREADS + tid;
            const bool ok = i < end && lv[k] >= 0 && lv[k] < L;
            lr[k] = ok ? ((uint32_t)lv[k] << 16) | atomicAdd(&cnt[lv[k]], 1u) : ~0u;
        }
        __syncthreads();
        // exclusive scan of the counts into staged-run starts; cnt[L] = total
        {
            uint32_t sum = 0;
            for (int32_t l = l0; l < l1; ++l) sum += cnt[l];
            uint32_t incl = sum;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const uint32_t o = (uint32_t)__shfl_up((int)incl, d, 64);
                if (lane >= d) incl += o;
            }
            if (lane == 63) wsum[wave] = incl;
            __syncthreads();
            uint32_t run = incl - sum;
            for (int w = 0; w < wave; ++w) run += wsum[w];
            for (int32_t l = l0; l < l1; ++l) {
                const uint32_t c = cnt[l];
                cnt[l] = run;
                run += c;
            }
            if (tid == PACK_THREADS - 1) cnt[L] = run;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < SEG_SORT_KR; ++k) {
            if (lr[k] == ~0u) continue;
            const uint32_t l = lr[k] >> 16;
            const uint32_t off = (uint32_t)(k * PACK_THREADS + tid);
            stg[cnt[l] + (lr[k] & 0xffffu)] = (l << 16) | off;
        }
        __syncthreads();
        const uint32_t total = cnt[L];
        const uint32_t id0 = (uint32_t)base + 1u;
        for (uint32_t k = tid; k < total; k += PACK_THREADS) {
            const uint32_t e = stg[k];
            const uint32_t l = e >> 16;
            memt[gcur[l] + (k - cnt[l])] = id0 + (e & 0xffffu);
        }
        __syncthreads();
        // advance the buckets' next slots; clear the counts
        for (int32_t l = tid; l < L; l += PACK_THREADS) gcur[l] += cnt[l + 1] - cnt[l];
        __syncthreads();
        for (int32_t l = tid; l <= L; l += PACK_THREADS) cnt[l] = 0u;
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Forest path with per-part cursors (2L <= PART_MAX_NB, N >= PART_MIN_N and
// N >= 16 * 2L, see forest_sizes): each tree's samples are cut into
// PACK_PARTS contiguous parts.
//   k_part_hist    (tree, part): LDS histogram of the part's buckets -> ph,
//                  and the part's 16-bit keys;
//   k_part_scan    (tree): bucket starts (off) and ends (bend) in the
//                  line-fit layout and, per part, the start of its members in
//                  each bucket (ph, in place);
//   k_part_scatter (tree, part): LDS cursors from ph; each member goes
//                  straight to its slot in mem[t].  The parts of a tree run
//                  at once on one XCD, eight trees per XCD: the 4-byte member
//                  writes of those trees (8 x 4N bytes) merge in that XCD's
//                  L2 before they reach HBM while that region fits the L2;
//   k_part_scatter_sorted / _sorted4: the same, with the part's members
//                  sorted by bucket in LDS first and written in bucket order
//                  (larger forests, where the direct writes no longer merge);
//   k_part_records (sample block, tree block): the sample-major run records
//                  from the keys and the part table.
// ---------------------------------------------------------------------------
constexpr int PACK_PARTS = 8;
constexpr int PART_MAX_NB = 8192;
constexpr int64_t PART_MIN_N = 32768;

__device__ __forceinline__ int64_t part_begin(int64_t N, int p) {
    const int64_t chunk = (N + PACK_PARTS - 1) / PACK_PARTS;
    return min(N, (int64_t)p * chunk);
}

// (tree, part) of a k_part_* workgroup: consecutive dispatch slots of one
// XCD walk the parts of a tree, trees x, x + 8, x + 16, ... on XCD x.
__device__ __forceinline__ void part_of_block(uint32_t bid, int32_t& t, int& p) {
    const uint32_t xcd = bid & 7, slot = bid >> 3;
    t = (int32_t)(xcd + 8 * (slot / PACK_PARTS));
    p = (int)(slot % PACK_PARTS);
}

__global__ __launch_bounds__(PACK_THREADS) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_part_hist(
    LeafView v, uint32_t* ph, uint16_t* key16, int64_t ldk) {
    extern __shared__ uint32_t sh[];
    int32_t t;
    int p;
    part_of_block(blockIdx.x, t, p);
    if (t >= v.T) return;
    const int32_t nb = view_buckets(v);
    for (int32_t b = threadIdx.x; b < nb; b += PACK_THREADS) sh[b] = 0u;
    __syncthreads();
    const int64_t i0 = part_begin(v.N, p), i1 = part_begin(v.N, p + 1);
    const int64_t round = (int64_t)PACK_THREADS * PACK_KR;
    uint16_t* kt = key16 + (int64_t)t * ldk;
    for (int64_t base = i0; base < i1; base += round) {
        // every load of the round first (indices past the part read sample i0)
        KeyLoad ld[PACK_KR];
#pragma unroll
        for (int k = 0; k < PACK_KR; ++k) {
            const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
            ld[k] = key_load(v, i < i1 ? i : i0, t);
        }
        int32_t key[PACK_KR];
#pragma unroll
        for (int k = 0; k < PACK_KR; ++k) {
            const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
            key[k] = i < i1 ? key_bucket(v, ld[k], i) : -2;
        }
#pragma unroll
        for (int k = 0; k < PACK_KR; ++k) {
            const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
            if (key[k] >= 0) atomicAdd(&sh[key[k]], 1u);
            if (key[k] != -2) kt[i] = key[k] >= 0 ? (uint16_t)key[k] : (uint16_t)0xffffu;
        }
    }
    // the row's padding keys (ldk > N) are written by the last part
    if (p == PACK_PARTS - 1)
        for (int64_t i = v.N + threadIdx.x; i < ldk; i += PACK_THREADS) kt[i] = (uint16_t)0xffffu;
    __syncthreads();
    uint32_t* out = ph + ((int64_t)t * PACK_PARTS + p) * nb;
    for (int32_t b = threadIdx.x; b < nb; b += PACK_THREADS) out[b] = sh[b];
}

// One workgroup per tree.  Thread tid places the FIT_GROUP consecutive
// buckets of group tid from a line-aligned group start (fit_start, the
// line-fit layout), or back to back when fit is 0; a workgroup-wide
// exclusive scan of the group lengths gives each group's start, so every
// bucket gets its start (off) and end (bend) in mem[t], and each part's start
// in each bucket replaces its count in the part table.  off[nb] is the
// tree's used length (at most ms).  The kernel also lists the tree's buckets
// of REC_LONG or more members (start and end byte offsets in mem, in
// lng[t][0 .. lngn[t]), lngn zeroed before).
__global__ __launch_bounds__(PACK_THREADS) void k_part_scan(int32_t nb, int32_t T, int64_t ms, int32_t fit,
                                                            uint32_t* ph, int32_t* goff_all, int32_t* gend_all,
                                                            uint2* lng, int32_t* lngn, int32_t lmax) {
    __shared__ uint32_t wsum[PACK_THREADS / 64];
    const int32_t t = blockIdx.x;
    if (t >= T) return;
    uint32_t* pt = ph + (int64_t)t * PACK_PARTS * nb;
    int32_t* goff = goff_all + (int64_t)t * (nb + 1);
    int32_t* gend = gend_all + (int64_t)t * nb;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t tbase = (uint32_t)((int64_t)t * ms);  // T * ms < 2^30 (forest_sizes)
    uint32_t carry = 0;
    for (int32_t c0 = 0; c0 < nb; c0 += PACK_THREADS * FIT_GROUP) {
        const int32_t b0 = c0 + tid * FIT_GROUP;
        // the group's bucket sizes (parts outer, so that the loads of one
        // part's 16 counts are in flight together)
        uint32_t sz[FIT_GROUP];
#pragma unroll
        for (int k = 0; k < FIT_GROUP; ++k) sz[k] = 0u;
        for (int q = 0; q < PACK_PARTS; ++q) {
            const uint32_t* row = pt + (int64_t)q * nb;
#pragma unroll
            for (int k = 0; k < FIT_GROUP; ++k) sz[k] += b0 + k < nb ? row[b0 + k] : 0u;
        }
        uint32_t st[FIT_GROUP];
        uint32_t pos = 0;
#pragma unroll
        for (int k = 0; k < FIT_GROUP; ++k) {
            st[k] = fit ? fit_start(pos, sz[k]) : pos;
            pos = st[k] + sz[k];
        }
        const uint32_t len = fit ? (pos + LINE_IDS - 1u) & ~(LINE_IDS - 1u) : pos;
        // exclusive scan of the group lengths: within the wave, then across
        uint32_t incl = len;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t o = (uint32_t)__shfl_up((int)incl, d, 64);
            if (lane >= d) incl += o;
        }
        if (lane == 63) wsum[wave] = incl;
        __syncthreads();
        uint32_t before = 0, total = 0;
#pragma unroll
        for (int w = 0; w < PACK_THREADS / 64; ++w) {
            const uint32_t x = wsum[w];
            before += w < wave ? x : 0u;
            total += x;
        }
        __syncthreads();
        const uint32_t gbase = carry + before + incl - len;
#pragma unroll
        for (int k = 0; k < FIT_GROUP; ++k) {
            const int32_t b = b0 + k;
            if (b < nb) {
                const uint32_t start = gbase + st[k], n = sz[k];
                goff[b] = (int32_t)start;
                gend[b] = (int32_t)(start + n);
                if (n >= REC_LONG) {
                    const int32_t slot = atomicAdd(&lngn[t], 1);
                    if (slot < lmax)
                        lng[(int64_t)t * lmax + slot] = make_uint2(4u * (tbase + start), 4u * (tbase + start + n));
                }
                uint32_t run = start;
                for (int q = 0; q < PACK_PARTS; ++q) {
                    uint32_t* e = pt + (int64_t)q * nb + b;
                    const uint32_t c = *e;
                    *e = run;
                    run += c;
                }
            }
        }
        carry += total;
    }
    if (tid == 0) goff[nb] = (int32_t)carry;
}

__global__ __launch_bounds__(PACK_THREADS) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_part_scatter(
    LeafView v, const uint32_t* ph, const int32_t* gend_all, int64_t ms, const uint16_t* key16, int64_t ldk,
    uint32_t* mem) {
    extern __shared__ uint32_t sh[];
    int32_t t;
    int p;
    part_of_block(blockIdx.x, t, p);
    if (t >= v.T) return;
    const int32_t nb = view_buckets(v);
    uint32_t* cur = sh;       // nb cursors
    uint32_t* end = sh + nb;  // nb bucket ends
    const uint32_t* pp = ph + ((int64_t)t * PACK_PARTS + p) * nb;
    const int32_t* gend = gend_all + (int64_t)t * nb;
    for (int32_t b = threadIdx.x; b < nb; b += PACK_THREADS) {
        cur[b] = pp[b];
        end[b] = (uint32_t)gend[b];
    }
    __syncthreads();
    const int64_t N = v.N;
    const int64_t i0 = part_begin(N, p), i1 = part_begin(N, p + 1);
    uint32_t* memt = mem + (int64_t)t * ms;
    const uint16_t* kt = key16 + (int64_t)t * ldk;
    const int64_t round = (int64_t)PACK_THREADS * PACK_KR;
    for (int64_t base = i0; base < i1; base += round) {
        uint32_t key[PACK_KR];
#pragma unroll
        for (int k = 0; k < PACK_KR; ++k) {
            const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
            key[k] = i < i1 ? (uint32_t)kt[i] : 0xffffu;
        }
#pragma unroll
        for (int k = 0; k < PACK_KR; ++k) {
            const uint32_t b = key[k];
            if (b == 0xffffu) continue;
            const uint32_t pos = atomicAdd(&cur[b], 1u);
            if (pos < end[b]) memt[pos] = (uint32_t)(base + (int64_t)k * PACK_THREADS + threadIdx.x + 1);
        }
    }
}

// k_part_scatter with the member writes in bucket order.  The part's members
// are first counting-sorted by bucket in LDS, as 16-bit offsets from the
// part's first sample; then thread k writes staged member k to its slot.
// Consecutive lanes thus write consecutive slots of a bucket's part range,
// and the parts of a tree, which run at once on one XCD, sweep mem[t] in the
// same bucket order, so the lines they share fill up in L2 before they are
// written back (random 4-byte stores leave most lines partial).  Parts of at
// most PART_SORT_MAX samples.
//
// LDS: lcur[nb] (the exclusive prefix of the part's bucket counts, used as
// cursors, which leaves each bucket's inclusive end), end[nb + 1], ps0[nb],
// wsum[16], stg[part size] (uint16).
constexpr int64_t PART_SORT_MAX = 65536;
constexpr int64_t PART_SORT_MIN_N = 32768;
constexpr int32_t PART_SORT_MAX_NB = 4096;

static size_t part_sorted_lds(int32_t nb, int64_t part) {
    return (size_t)(3 * nb + 1 + 16) * 4 + (size_t)((part + 1) / 2) * 4;
}

__global__ __launch_bounds__(PACK_THREADS) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_part_scatter_sorted(
    LeafView v, const uint32_t* ph, const int32_t* gend_all, int64_t ms, const uint16_t* key16, int64_t ldk,
    uint32_t* mem) {
    extern __shared__ uint32_t sh[];
    int32_t t;
    int p;
    part_of_block(blockIdx.x, t, p);
    if (t >= v.T) return;
    const int32_t nb = view_buckets(v);
    uint32_t* lcur = sh;
    uint32_t* end = sh + nb;
    uint32_t* ps0 = end + nb + 1;
    uint32_t* wsum = ps0 + nb;
    uint16_t* stg = (uint16_t*)(wsum + 16);
    const uint32_t* pp = ph + ((int64_t)t * PACK_PARTS + p) * nb;
    const int32_t* gend = gend_all + (int64_t)t * nb;
    // the part's count in bucket b runs up to the next part's start there
    // (the bucket's end for the last part)
    const uint32_t* pn = p + 1 == PACK_PARTS ? (const uint32_t*)gend : pp + nb;
    for (int32_t b = threadIdx.x; b < nb; b += PACK_THREADS) {
        end[b] = (uint32_t)gend[b];
        const uint32_t s = pp[b];
        ps0[b] = s;
        lcur[b] = pn[b] - s;
    }
    __syncthreads();
    // exclusive scan of the counts: thread tid takes buckets [tid*E, tid*E + E)
    {
        const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
        const int32_t E = (nb + PACK_THREADS - 1) / PACK_THREADS;
        const int32_t b0 = min(nb, tid * E), b1 = min(nb, b0 + E);
        uint32_t s = 0;
        for (int32_t b = b0; b < b1; ++b) s += lcur[b];
        uint32_t incl = s;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t o = (uint32_t)__shfl_up((int)incl, d, 64);
            if (lane >= d) incl += o;
        }
        if (lane == 63) wsum[wave] = incl;
        __syncthreads();
        uint32_t run = incl - s;
        for (int w = 0; w < wave; ++w) run += wsum[w];
        for (int32_t b = b0; b < b1; ++b) {
            const uint32_t c = lcur[b];
            lcur[b] = run;
            run += c;
        }
    }
    __syncthreads();
    const int64_t N = v.N;
    const int64_t i0 = part_begin(N, p), i1 = part_begin(N, p + 1);
    const uint16_t* kt = key16 + (int64_t)t * ldk;
    const int64_t round = (int64_t)PACK_THREADS * PACK_KR;
    for (int64_t base = i0; base < i1; base += round) {
        uint32_t key[PACK_KR];
#pragma unroll
        for (int k = 0; k < PACK_KR; ++k) {
            const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
            key[k] = i < i1 ? (uint32_t)kt[i] : 0xffffu;
        }
#pragma unroll
        for (int k = 0; k < PACK_KR; ++k) {
            const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
            const uint32_t b = key[k];
            if (b != 0xffffu) stg[atomicAdd(&lcur[b], 1u)] = (uint16_t)(i - i0);
        }
    }
    __syncthreads();
    // staged member k belongs to the first bucket b with lcur[b] > k
    const uint32_t total = nb > 0 ? lcur[nb - 1] : 0u;
    uint32_t* memt = mem + (int64_t)t * ms;
    const uint32_t id0 = (uint32_t)i0 + 1u;
    for (uint32_t k = threadIdx.x; k < total; k += PACK_THREADS) {
        int32_t lo = 0, hi = nb - 1;
        while (lo < hi) {
            const int32_t mid = (lo + hi) >> 1;
            if (lcur[mid] > k) hi = mid;
            else lo = mid + 1;
        }
        const uint32_t first = lo > 0 ? lcur[lo - 1] : 0u;
        const uint32_t pos = ps0[lo] + (k - first);
        if (pos < end[lo]) memt[pos] = id0 + (uint32_t)stg[k];
    }
}

// k_part_scatter_sorted with 4-byte staging entries (bucket << 16 | offset
// in the part), so that staged member k finds its slot without a search:
// slot = ps0[b] + (k - start of b's staged run).  To keep the LDS at two
// workgroups per CU at part sizes like 12,500 with 4,096 buckets, the local
// cursors are 16-bit halves of 32-bit words counting down from each bucket's
// end, so that they end at its start (counts stay below 2^16: parts of at
// most PART_SORT4_MAX samples).
// LDS: ps0[nb], wsum[16], lc[nb] (uint16, padded to a word), stg[part].
constexpr int64_t PART_SORT4_MAX = 65535;

static size_t part_sorted4_lds(int32_t nb, int64_t part) {
    const int64_t un = std::max<int64_t>(nb + 1, part);
    return (size_t)(nb + 16 + (nb + 1) / 2 + un) * 4;
}

__global__ __launch_bounds__(PACK_THREADS) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_part_scatter_sorted4(
    LeafView v, const uint32_t* ph, const int32_t* gend_all, int64_t ms, const uint16_t* key16, int64_t ldk,
    uint32_t* mem) {
    extern __shared__ uint32_t sh[];
    int32_t t;
    int p;
    part_of_block(blockIdx.x, t, p);
    if (t >= v.T) return;
    const int32_t nb = view_buckets(v);
    uint32_t* ps0 = sh;
    uint32_t* wsum = ps0 + nb;
    uint16_t* lc = (uint16_t*)(wsum + 16);
    uint32_t* lc32 = wsum + 16;
    uint32_t* stg = wsum + 16 + (nb + 1) / 2;
    const uint32_t* pp = ph + ((int64_t)t * PACK_PARTS + p) * nb;
    const int32_t* gend = gend_all + (int64_t)t * nb;
    // the part's count in bucket b runs up to the next part's start there
    // (the bucket's end for the last part)
    const uint32_t* pn = p + 1 == PACK_PARTS ? (const uint32_t*)gend : pp + nb;
    for (int32_t b = threadIdx.x; b < nb; b += PACK_THREADS) {
        const uint32_t s = pp[b];
        ps0[b] = s;
        lc[b] = (uint16_t)(pn[b] - s);
    }
    __syncthreads();
    // inclusive scan of the counts: thread tid takes buckets [tid*E, tid*E + E)
    {
        const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
        const int32_t E = (nb + PACK_THREADS - 1) / PACK_THREADS;
        const int32_t b0 = min(nb, tid * E), b1 = min(nb, b0 + E);
        uint32_t s = 0;
        for (int32_t b = b0; b < b1; ++b) s += lc[b];
        uint32_t incl = s;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t o = (uint32_t)__shfl_up((int)incl, d, 64);
            if (lane >= d) incl += o;
        }
        if (lane == 63) wsum[wave] = incl;
        __syncthreads();
        uint32_t run = incl - s;
        for (int w = 0; w < wave; ++w) run += wsum[w];
        for (int32_t b = b0; b < b1; ++b) {
            run += lc[b];
            lc[b] = (uint16_t)run;
        }
    }
    __syncthreads();  // every bucket's count-down cursor is in place
    const int64_t N = v.N;
    const int64_t i0 = part_begin(N, p), i1 = part_begin(N, p + 1);
    const uint16_t* kt = key16 + (int64_t)t * ldk;
    const int64_t round = (int64_t)PACK_THREADS * PACK_KR;
    for (int64_t base = i0; base < i1; base += round) {
        uint32_t key[PACK_KR];
#pragma unroll
        for (int k = 0; k < PACK_KR; ++k) {
            const int64_t i = base + (int64_t)k * PACK_THREADS + threadIdx.x;
            key[k] = i < i1 ? (uint32_t)kt[i] : 0xffffu;
        }
#pragma unroll
        for (int k = 0; k < PACK_KR; ++k) {
            const uint32_t b = key[k];
            if (b == 0xffffu) continue;
            const uint32_t sh16 = (b & 1u) * 16u;
            const uint32_t old = atomicSub(&lc32[b >> 1], 1u << sh16);
            stg[((old >> sh16) & 0xffffu) - 1u] = (b << 16) | (uint32_t)(base + (int64_t)k * PACK_THREADS + threadIdx.x - i0);
        }
    }
    __syncthreads();
    // lc[b] is now the start of bucket b's staged run
    uint32_t nval = 0;
    for (int w = 0; w < PACK_THREADS / 64; ++w) nval += wsum[w];
    uint32_t* memt = mem + (int64_t)t * ms;
    const uint32_t id0 = (uint32_t)i0 + 1u;
    // a member's slot lies below its bucket's end, which is at most ms
    const uint32_t lim = (uint32_t)ms;
    for (uint32_t k = threadIdx.x; k < nval; k += PACK_THREADS) {
        const uint32_t e = stg[k];
        const uint32_t b = e >> 16;
        const uint32_t pos = ps0[b] + (k - (uint32_t)lc[b]);
        if (pos < lim) memt[pos] = id0 + (e & 0xffffu);
    }
}

// Sample-major run records of the per-part path, from the keys: workgroup
// (block x of PREC_S samples, block y of PREC_T trees) looks up, for every
// (sample i, tree t) of its tile, the start of i's own part in i's opposite
// bucket (the part table after k_part_scan) and that bucket's end, and
// writes the tile's rows of roff / rlen through LDS (one 128-byte row piece
// per sample).  Consecutive workgroups take consecutive sample blocks of one
// tree block, so the table slices they read (PREC_T trees of one part) stay
// in L2.  Padding trees T..ldr-1 get empty records.  With acc (nout counted
// here), each tile adds its trees' OOB bits of its samples to acc[i], one
// atomic per sample and tile: nout_i = sum over trees of the OOB bits
// (src/rf_bootstrap.cpp:67-70).
constexpr int PREC_S = 128, PREC_T = 32;

__global__ __launch_bounds__(256) void k_part_records(const uint16_t* key16, int64_t ldk, const uint32_t* ph,
                                                     const int32_t* gend_all, int32_t nb, int64_t N, int32_t T,
                                                     int64_t ms, int64_t ldr, uint32_t* roff, uint16_t* rlen,
                                                     const uint32_t* oob, int64_t old, uint32_t* acc) {
    __shared__ uint32_t so[PREC_S][PREC_T + 1];
    __shared__ uint16_t sl[PREC_S][PREC_T + 2];
    __shared__ uint32_t part[2][PREC_S];
    const int64_t i0 = (int64_t)blockIdx.x * PREC_S;
    const int32_t t0 = (int32_t)blockIdx.y * PREC_T;
    const int64_t chunk = (N + PACK_PARTS - 1) / PACK_PARTS;
    const int c = threadIdx.x & 63;
    // keys of sample pair (i0 + 2c, i0 + 2c + 1) in trees t0 + r, r = w + 4q
    // (w = threadIdx.x >> 6): all loads first
    uint32_t kw[PREC_T / 4];
#pragma unroll
    for (int q = 0; q < PREC_T / 4; ++q) {
        const int32_t t = t0 + (int32_t)(threadIdx.x >> 6) + 4 * q;
        const int64_t i = i0 + 2 * c;
        kw[q] = (t < T && i < N) ? *(const uint32_t*)(key16 + (int64_t)t * ldk + i) : 0xffffffffu;
    }
#pragma unroll
    for (int q = 0; q < PREC_T / 4; ++q) {
        const int r = (int)(threadIdx.x >> 6) + 4 * q;
        const int32_t t = t0 + r;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t i = i0 + 2 * c + h;
            const uint32_t b = (kw[q] >> (16 * h)) & 0xffffu;
            uint32_t o = 0u, len = 0u;
            if (b != 0xffffu && i < N) {
                // the run of (i, t): members of the opposite bucket placed by
                // i's part and the later ones, i.e. every member j from the
                // part's first sample on
                const uint32_t ob = b ^ 1u;
                const int64_t p = i / chunk;
                const uint32_t rs = ph[((int64_t)t * PACK_PARTS + p) * nb + ob];
                const uint32_t e = (uint32_t)gend_all[(int64_t)t * nb + ob];
                o = (uint32_t)((int64_t)t * ms + rs) * 4u;
                len = min(e - rs, REC_LONG) * 4u;
            }
            so[2 * c + h][r] = o;
            sl[2 * c + h][r] = (uint16_t)len;
        }
    }
    if (acc) {
        // thread (sample s, half g of the tile's trees): its OOB bits
        const int s = threadIdx.x & (PREC_S - 1), g = threadIdx.x >> 7;
        const int64_t i = i0 + s;
        const int64_t ic = i < N ? i : 0;
        uint32_t n = 0;
#pragma unroll
        for (int k = 0; k < PREC_T / 2; ++k) {
            const int32_t t = t0 + g * (PREC_T / 2) + k;
            const uint32_t w = t < T ? oob[(int64_t)t * old + (ic >> 5)] : 0u;
            n += (w >> (ic & 31)) & 1u;
        }
        part[g][s] = n;
    }
    __syncthreads();
    for (int k = threadIdx.x; k < PREC_S * PREC_T; k += 256) {
        const int s = k / PREC_T, r = k % PREC_T;
        const int64_t i = i0 + s;
        const int64_t t = t0 + r;
        if (i < N && t < ldr) {
            roff[i * ldr + t] = so[s][r];
            rlen[i * ldr + t] = sl[s][r];
        }
    }
    if (acc && threadIdx.x < PREC_S && i0 + threadIdx.x < N)
        atomicAdd(&acc[i0 + threadIdx.x], part[0][threadIdx.x] + part[1][threadIdx.x]);
}

// [T][N] -> [N][ldr] for both record arrays, 64 x 64 tiles through LDS.
// With acc (forest mode, nout counted here), each tile also adds its trees'
// OOB bits of its 64 samples to acc[i] (one atomic per sample and tile):
// nout_i = sum over trees of the OOB bits (src/rf_bootstrap.cpp:67-70).
__global__ __launch_bounds__(256) void k_rec_transpose(const uint32_t* roffT, const uint16_t* rlenT, int64_t N,
                                                      int32_t T, int64_t ldr, uint32_t* roff, uint16_t* rlen,
                                                      const uint32_t* oob, int64_t old, uint32_t* acc) {
    __shared__ uint32_t to[64][65];
    __shared__ uint16_t tl[64][66];
    const int64_t i0 = (int64_t)blockIdx.x * 64;
    const int32_t t0 = blockIdx.y * 64;
    // all 16 loads of a thread first, at clamped indices
    uint32_t o[16];
    uint16_t l[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const int k = threadIdx.x + 256 * q;
        const int r = k >> 6, c = k & 63;  // r: tree, c: sample
        const int64_t i = i0 + c;
        const int32_t t = t0 + r;
        const int64_t e = (i < N && t < T) ? (int64_t)t * N + i : 0;
        o[q] = roffT[e];
        l[q] = rlenT[e];
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const int k = threadIdx.x + 256 * q;
        const int r = k >> 6, c = k & 63;
        const bool ok = i0 + c < N && t0 + r < T;
        to[r][c] = ok ? o[q] : 0u;
        tl[r][c] = ok ? l[q] : (uint16_t)0;
    }
    __syncthreads();
    for (int k = threadIdx.x; k < 64 * 64; k += 256) {
        const int r = k >> 6, c = k & 63;  // r: sample, c: tree
        const int64_t i = i0 + r;
        const int32_t t = t0 + c;
        // padding trees T..ldr-1 get empty records
        if (i < N && t < ldr) {
            roff[i * ldr + t] = t < T ? to[c][r] : 0u;
            rlen[i * ldr + t] = t < T ? tl[c][r] : (uint16_t)0;
        }
    }
    if (acc) {
        // thread (sample c, tree group g of 16): its OOB bits, then the four
        // groups' sums through LDS
        __shared__ uint32_t part[4][64];
        const int c = threadIdx.x & 63, g = threadIdx.x >> 6;
        const int64_t i = i0 + c;
        const int64_t ic = i < N ? i : 0;
        uint32_t w[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int32_t t = t0 + 16 * g + k;
            w[k] = t < T ? oob[(int64_t)t * old + (ic >> 5)] : 0u;
        }
        uint32_t n = 0;
#pragma unroll
        for (int k = 0; k < 16; ++k) n += (w[k] >> (ic & 31)) & 1u;
        part[g][c] = n;
        __syncthreads();
        if (g == 0 && i < N) atomicAdd(&acc[i], part[0][c] + part[1][c] + part[2][c] + part[3][c]);
    }
}

__global__ void k_fill_u32(uint32_t* p, int64_t n, uint32_t val) {
    int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; k < n; k += stride) p[k] = val;
}

__global__ __launch_bounds__(256) void k_nout_final(int64_t N, const int32_t* nout_in, const uint32_t* acc,
                                                   int32_t* nout, double* rinv, unsigned long long* rr) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    double r = 1.0;
    bool ok = i < N;
    if (ok) {
        const int32_t n = nout_in ? nout_in[i] : (int32_t)acc[i];
        nout[i] = n;
        r = nout_recip(n);
        rinv[i] = r;
    }
    // block-level min/max, then one atomic pair per block
    __shared__ unsigned long long smin[256], smax[256];
    const unsigned long long bits = (unsigned long long)__double_as_longlong(r);
    smin[threadIdx.x] = ok ? bits : 0x7ff0000000000000ull;
    smax[threadIdx.x] = ok ? bits : 0ull;
    __syncthreads();
    for (int d = 128; d > 0; d >>= 1) {
        if (threadIdx.x < d) {
            smin[threadIdx.x] = min(smin[threadIdx.x], smin[threadIdx.x + d]);
            smax[threadIdx.x] = max(smax[threadIdx.x], smax[threadIdx.x + d]);
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        atomicMin(&rr[0], smin[0]);
        atomicMax(&rr[1], smax[0]);
    }
}

// Everything the forest kernels accumulate into, or read as slack, cleared
// in one launch: the record slack after the last row (empty records), the
// status words, the per-tree long-bucket counts, the OOB-count accumulator
// (acc, N words, or NULL) and the 1/nout range (min = +inf, max = 0, as
// IEEE bits).
struct ForestInit {
    uint32_t* roff_slack;
    uint32_t* rlen_slack;
    uint32_t* flags;
    uint32_t* lngn;
    int32_t T;
    uint32_t* acc;
    int64_t N;
    unsigned long long* rr;
};

__global__ __launch_bounds__(256) void k_forest_init(ForestInit a) {
    const int64_t k0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * 256;
    if (a.acc)
        for (int64_t k = k0; k < a.N; k += stride) a.acc[k] = 0u;
    for (int64_t k = k0; k < a.T; k += stride) a.lngn[k] = 0u;
    if (k0 < REC_PAD) a.roff_slack[k0] = 0u;
    if (k0 < REC_PAD / 2) a.rlen_slack[k0] = 0u;
    if (k0 < 16) a.flags[k0] = 0u;
    if (k0 == 0) {
        a.rr[0] = 0x7ff0000000000000ull;
        a.rr[1] = 0ull;
    }
}

// Buckets of REC_LONG or more members (forest mode): their start and end
// byte offsets in mem, per tree, in lng[t][0 .. lngn[t]) (lngn zeroed
// first).  One thread per (tree, bucket).
__global__ __launch_bounds__(256) void k_long_runs(const int32_t* goff_all, int32_t nb, int32_t T, int64_t N,
                                                   uint2* lng, int32_t* lngn, int32_t lmax) {
    const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (k >= (int64_t)T * nb) return;
    const int32_t t = (int32_t)(k / nb), b = (int32_t)(k % nb);
    const int32_t* off = goff_all + (int64_t)t * (nb + 1);
    const uint32_t s = (uint32_t)off[b], e = (uint32_t)off[b + 1];
    if (e - s < REC_LONG) return;
    const int32_t slot = atomicAdd(&lngn[t], 1);
    const uint32_t base = (uint32_t)t * (uint32_t)N;
    if (slot < lmax) lng[(int64_t)t * lmax + slot] = make_uint2(4u * (base + s), 4u * (base + e));
}

static int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

void fill_u32(rfxp_ctx* ctx, uint32_t* p, int64_t n, uint32_t val) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)std::min<int64_t>(cdiv(n, 256), 65536)), dim3(256), 0, ctx->stream,
                       p, n, val);
}

// Bound of T * ms + MEM_PAD (ids) for the line-fit layout: byte offsets of
// mem below 2^32.  A build may lower it (the CPU emulation's tests do, to
// run the per-part path's back-to-back placement on small forests).
#ifndef RFXP_FIT_LIMIT
#define RFXP_FIT_LIMIT (1LL << 30)
#endif

ForestSizes forest_sizes(const LeafView& v, bool count_nout, int max_lds) {
    ForestSizes z;
    const int64_t N = v.N, n1 = std::max<int64_t>(N, 1);
    const int32_t T = v.T;
    const int32_t nb = view_buckets(v);
    const bool forest = v.nseg == 0;
    const int64_t ldk = cdiv(N, 8) * 8;
    z.ldr = ((int64_t)T + 15) / 16 * 16;
    z.lmax = (int32_t)(N / REC_LONG + 1);
    // Per-part packing pays off for large forests with many members per
    // bucket and part: below N = 32,768 or 16 members per bucket (parts of
    // fewer than 2 members per bucket) its per-part tables cost more than
    // the whole-tree path's repeated key reads, and the runs it shortens
    // fit a line either way.  Step (packing + triangle, T = 500) measured
    // both ways: N = 20,000 with 1,000-4,096 leaves 0.68 -> 0.55 ms whole
    // tree; N = 100,000 / 2,048 leaves 3.18 (per part) against 3.31 ms;
    // N = 200,000 / 2,048 leaves 12.5 against 17.1 ms.
    z.part_path = forest && nb <= PART_MAX_NB && N >= PART_MIN_N && N >= 16 * (int64_t)nb;
    z.seg_path = !forest && v.L <= SEG_MAX_L;
    const size_t lds_bytes = (size_t)2 * (nb + 1) * 4;
    z.lds_path = (int64_t)lds_bytes + PACK_THREADS * 4 + 1024 <= max_lds;
    // the line-fit layout keeps every byte offset of mem within 32 bits
    // (mem_bytes of the triangle's buffer loads); past that the per-part
    // path places its buckets back to back
    z.fit = z.part_path && (int64_t)T * fit_stride(N, nb) + MEM_PAD < (int64_t)(RFXP_FIT_LIMIT);
    z.ms = z.fit ? fit_stride(N, nb) : n1;
    z.n[FB_OFF] = (size_t)T * (nb + 1);
    z.n[FB_MEM] = (size_t)T * z.ms + MEM_PAD;
    if (z.part_path) {
        z.n[FB_BEND] = (size_t)T * nb;
        z.n[FB_KEY16] = (size_t)T * ldk;
        z.n[FB_SCRATCH] = (size_t)T * PACK_PARTS * nb;
    } else if (z.seg_path) {
        z.n[FB_SCRATCH] = (size_t)T * (nb + 1);
    } else {
        z.n[FB_KEY16] = nb < 0xffff ? (size_t)T * ldk : 0;
        z.n[FB_SCRATCH] = (size_t)T * (nb + 1);  // counts, then the global cursors
        // tree-major records (k_tree_records) in forest mode
        z.tree_rec = forest;
        if (z.tree_rec) {
            z.n[FB_ROFFT] = (size_t)T * N;
            z.n[FB_RLENT] = (size_t)T * N;
        }
    }
    if (forest) {
        z.n[FB_ROFF] = (size_t)n1 * z.ldr + REC_PAD;
        z.n[FB_RLEN] = (size_t)n1 * z.ldr + REC_PAD;
        z.n[FB_SCRATCH2] = count_nout ? (size_t)n1 : 0;
        z.n[FB_NOUT] = (size_t)n1;
        z.n[FB_RINV] = (size_t)n1;
        z.n[FB_RRANGE] = 2;
        z.n[FB_LNG] = (size_t)T * z.lmax;
        z.n[FB_LNGN] = (size_t)T;
        z.n[FB_FLAGS] = 16;
    }
    return z;
}

int ctx_forest_bufs(rfxp_ctx* ctx, const ForestSizes& z, DevBuf<int32_t>& off, DevBuf<uint32_t>& mem,
                    ForestBufs& fb) {
    fb = ForestBufs();
    fb.ldr = z.ldr;
    fb.lmax = z.lmax;
    fb.ms = z.ms;
#define RFXP_FB(K, buf, field)                                  \
    if (z.n[K]) {                                               \
        RFXP_HIP(ctx, (buf).ensure(z.n[K]));                    \
        fb.field = (buf).p;                                     \
    }
    RFXP_FB(FB_OFF, off, off)
    RFXP_FB(FB_BEND, ctx->bkt_end, bend)
    RFXP_FB(FB_MEM, mem, mem)
    RFXP_FB(FB_ROFF, ctx->roff, roff)
    RFXP_FB(FB_RLEN, ctx->rlen, rlen)
    RFXP_FB(FB_ROFFT, ctx->roffT, roffT)
    RFXP_FB(FB_RLENT, ctx->rlenT, rlenT)
    RFXP_FB(FB_SCRATCH, ctx->scratch, scratch)
    RFXP_FB(FB_SCRATCH2, ctx->scratch2, scratch2)
    RFXP_FB(FB_KEY16, ctx->key16, key16)
    RFXP_FB(FB_NOUT, ctx->nout, nout)
    RFXP_FB(FB_RINV, ctx->rinv, rinv)
    RFXP_FB(FB_RRANGE, ctx->rrange, rrange)
    RFXP_FB(FB_LNG, ctx->lng, lng)
    RFXP_FB(FB_LNGN, ctx->lngn, lngn)
    RFXP_FB(FB_FLAGS, ctx->flags, flags)
#undef RFXP_FB
    return RFXP_OK;
}

size_t forest_elem_bytes(int k) {
    switch (k) {
        case FB_OFF: case FB_BEND: case FB_NOUT: case FB_LNGN: case FB_FLAGS: return 4;
        case FB_MEM: case FB_ROFF: case FB_ROFFT: case FB_SCRATCH: case FB_SCRATCH2: return 4;
        case FB_RLEN: case FB_RLENT: case FB_KEY16: return 2;
        case FB_RINV: case FB_RRANGE: case FB_LNG: return 8;
        default: return 0;
    }
}

static int pack_forest_parts(rfxp_ctx* ctx, const LeafView& v, const int32_t* nout_in, const ForestBufs& fb);
static int pack_nout(rfxp_ctx* ctx, const LeafView& v, const int32_t* nout_in, const ForestBufs& fb);

// Reference-set path (see k_seg_hist).
static int pack_reference_segments(rfxp_ctx* ctx, const LeafView& v, const ForestBufs& fb) {
    hipStream_t s = ctx->stream;
    const int32_t nb = view_buckets(v);
    const unsigned grid = (unsigned)(8 * cdiv(v.T, 8) * v.nseg);
    const size_t lds = (size_t)v.L * 4;
    if (lds > 32768) {
        RFXP_HIP(ctx, hipFuncSetAttribute((const void*)k_seg_hist, hipFuncAttributeMaxDynamicSharedMemorySize,
                                          (int)lds));
        RFXP_HIP(ctx, hipFuncSetAttribute((const void*)k_seg_scatter, hipFuncAttributeMaxDynamicSharedMemorySize,
                                          (int)lds));
    }
    {
        LaunchTimer tm(ctx, "pack_hist");
        hipLaunchKernelGGL(k_seg_hist, dim3(grid), dim3(PACK_THREADS), lds, s, v, fb.scratch);
    }
    if (int rc = check_launch(ctx, "k_seg_hist")) return rc;
    {
        LaunchTimer tm(ctx, "pack_scan");
        hipLaunchKernelGGL(k_seg_scan, dim3((unsigned)v.T), dim3(PACK_THREADS), 0, s, nb, v.T, fb.scratch, fb.off);
    }
    if (int rc = check_launch(ctx, "k_seg_scan")) return rc;
    // leaf-ordered writes with the largest sub-chunk (at most 8 samples per
    // thread, at least 2) that keeps two workgroups per CU; with more leaves
    // than that allows (L above about 8,000) the direct writes, which at one
    // workgroup per CU and short sub-chunks were faster (measured at
    // N = 200,000, L = 16,384: 1.8 against 7.6 ms)
    int32_t sc = SEG_SORT_KR * PACK_THREADS;
    while (sc > 2048 && seg_sorted_lds(v.L, sc) * 2 > (size_t)ctx->max_lds) sc /= 2;
    const bool sorted = seg_sorted_lds(v.L, sc) * 2 <= (size_t)ctx->max_lds;
    if (sorted) {
        const size_t lds2 = seg_sorted_lds(v.L, sc);
        if (lds2 > 32768)
            RFXP_HIP(ctx, hipFuncSetAttribute((const void*)k_seg_scatter_sorted,
                                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds2));
        LaunchTimer tm(ctx, "pack_scatter");
        hipLaunchKernelGGL(k_seg_scatter_sorted, dim3(grid), dim3(PACK_THREADS), lds2, s, v, (const int32_t*)fb.off,
                           fb.mem, sc);
    } else {
        LaunchTimer tm(ctx, "pack_scatter");
        hipLaunchKernelGGL(k_seg_scatter, dim3(grid), dim3(PACK_THREADS), lds, s, v, (const int32_t*)fb.off, fb.mem);
    }
    return check_launch(ctx, "k_seg_scatter");
}

// The table of long buckets (forest mode), once the offsets are known.
static int pack_long_runs(rfxp_ctx* ctx, const LeafView& v, const ForestBufs& fb) {
    const int32_t nb = view_buckets(v);
    const int64_t n = (int64_t)v.T * nb;
    hipLaunchKernelGGL(k_long_runs, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, ctx->stream, (const int32_t*)fb.off,
                       nb, v.T, v.N, fb.lng, fb.lngn, fb.lmax);
    return check_launch(ctx, "k_long_runs");
}

int pack_forest(rfxp_ctx* ctx, const LeafView& v, const int32_t* nout_in, const ForestBufs& fb) {
    hipStream_t s = ctx->stream;
    const int64_t N = v.N;
    const int32_t T = v.T;
    const int32_t nb = view_buckets(v);
    const bool forest = v.nseg == 0;
    const ForestSizes z = forest_sizes(v, nout_in == nullptr, ctx->max_lds);
    if (forest) {
        const int64_t n1 = std::max<int64_t>(N, 1);
        ForestInit fi{fb.roff + n1 * fb.ldr, (uint32_t*)(fb.rlen + n1 * fb.ldr), (uint32_t*)fb.flags,
                      (uint32_t*)fb.lngn, T, nout_in ? nullptr : fb.scratch2, N, fb.rrange};
        const int64_t work = std::max<int64_t>({N, (int64_t)T, (int64_t)REC_PAD});
        LaunchTimer tm(ctx, "rr_init");
        hipLaunchKernelGGL(k_forest_init, dim3((unsigned)std::min<int64_t>(cdiv(work, 256), 1024)), dim3(256), 0, s,
                           fi);
    }
    if (int rc = check_launch(ctx, "k_forest_init")) return rc;
    if (N == 0) return RFXP_OK;
    if (z.part_path) {
        if (int rc = pack_forest_parts(ctx, v, nout_in, fb)) return rc;  // long runs listed by k_part_scan
        return pack_nout(ctx, v, nout_in, fb);
    }
    if (z.seg_path) return pack_reference_segments(ctx, v, fb);
    // trees -> workgroups in XCD-sized groups of 128 (8 XCDs x 16 trees)
    const unsigned grid = (unsigned)(cdiv(T, 128) * 128);
    const size_t lds_bytes = (size_t)2 * (nb + 1) * 4;
    // compact bucket ids for the second pass when they fit 16 bits
    uint16_t* k16 = z.n[FB_KEY16] ? fb.key16 : nullptr;
    const int64_t ldk = cdiv(N, 8) * 8;
    if (z.lds_path) {
        if (lds_bytes > 32768)
            RFXP_HIP(ctx, hipFuncSetAttribute((const void*)k_pack_hist,
                                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes));
        LaunchTimer tm(ctx, "pack_hist");
        hipLaunchKernelGGL(k_pack_hist, dim3(grid), dim3(PACK_THREADS), lds_bytes, s, v, fb.off, k16, ldk);
    } else {
        const int32_t nrange = (int32_t)cdiv(nb, TREE_HR);
        const size_t lds_r = (size_t)std::min<int32_t>(nb, TREE_HR) * 4;
        RFXP_HIP(ctx, hipFuncSetAttribute((const void*)k_tree_hist, hipFuncAttributeMaxDynamicSharedMemorySize,
                                          (int)lds_r));
        {
            LaunchTimer tm(ctx, "pack_hist");
            hipLaunchKernelGGL(k_tree_hist, dim3((unsigned)(cdiv((int64_t)T * nrange, 8) * 8)), dim3(PACK_THREADS),
                               lds_r, s, v, nrange, fb.scratch, k16, ldk);
        }
        if (int rc = check_launch(ctx, "k_tree_hist")) return rc;
        LaunchTimer tm(ctx, "pack_scan");
        hipLaunchKernelGGL(k_seg_scan, dim3((unsigned)T), dim3(PACK_THREADS), 0, s, nb, T, fb.scratch, fb.off);
    }
    if (int rc = check_launch(ctx, "k_pack_hist")) return rc;
    if (forest && z.tree_rec) {
        const int32_t nchunk = (int32_t)cdiv(N, TREE_REC_CHUNK);
        const size_t lds_t = (size_t)(nb + 1) * 4;
        const bool in_lds = lds_t <= (size_t)ctx->max_lds;
        if (in_lds && lds_t > 32768)
            RFXP_HIP(ctx, hipFuncSetAttribute((const void*)k_tree_records<true>,
                                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_t));
        LaunchTimer tm(ctx, "records");
        const dim3 grid_r((unsigned)(cdiv((int64_t)T * nchunk, 8) * 8));
        if (in_lds)
            hipLaunchKernelGGL(k_tree_records<true>, grid_r, dim3(PACK_THREADS), lds_t, s, v, (const uint16_t*)k16, ldk,
                               (const int32_t*)fb.off, nchunk, fb.roffT, fb.rlenT);
        else
            hipLaunchKernelGGL(k_tree_records<false>, grid_r, dim3(PACK_THREADS), 0, s, v, (const uint16_t*)k16, ldk,
                               (const int32_t*)fb.off, nchunk, fb.roffT, fb.rlenT);
        if (int rc = check_launch(ctx, "k_tree_records")) return rc;
        hipLaunchKernelGGL(k_rec_transpose, dim3((unsigned)cdiv(N, 64), (unsigned)cdiv(fb.ldr, 64)), dim3(256), 0, s,
                           fb.roffT, fb.rlenT, N, T, fb.ldr, fb.roff, fb.rlen, v.oob, v.old,
                           nout_in ? nullptr : fb.scratch2);
    }
    if (int rc = check_launch(ctx, "k_rec_transpose")) return rc;
    {
        // windows of win members, plus one for the slack a window can gain
        // from keeping bucket pairs whole; ncur = 1.5 * win * nb / N cursors
        const int64_t w0 = (int64_t)PACK_STAGE_WORDS * 2 * N / (2 * N + 3 * (int64_t)nb);
        const int32_t win = (int32_t)std::min<int64_t>(std::max<int64_t>(w0 & ~15LL, 4096), 16384);
        const int32_t nwin = (int32_t)cdiv(N, win) + 1;
        const int64_t nwg = cdiv((int64_t)T * nwin, 8) * 8;
        const size_t lds2 = (size_t)PACK_STAGE_WORDS * 4;
        RFXP_HIP(ctx, hipFuncSetAttribute((const void*)k_pack_scatter, hipFuncAttributeMaxDynamicSharedMemorySize,
                                          (int)lds2));
        LaunchTimer tm(ctx, "pack_scatter");
        hipLaunchKernelGGL(k_pack_scatter, dim3((unsigned)nwg), dim3(PACK_THREADS), lds2, s, v, fb.off, fb.mem,
                           fb.scratch, nwin, win, (const uint16_t*)k16, ldk);
    }
    if (int rc = check_launch(ctx, "k_pack_scatter")) return rc;
    if (!forest) return RFXP_OK;
    if (int rc = pack_long_runs(ctx, v, fb)) return rc;
    return pack_nout(ctx, v, nout_in, fb);
}

// Member scatter of the per-part path (RFXP_PACK_PARTS_*).  Bucket-ordered
// writes for forests whose member regions outgrow the L2 (8 trees x 4N bytes
// in flight per XCD), when the part's staging fits in LDS: of the two sorted
// kernels, the one with more workgroups per CU (at most two), the 4-byte
// staging on a tie; the 2-byte one only up to PART_SORT_MAX_NB buckets (its
// search gets slower with more).  Measured at T = 500 and N = 50,000-400,000
// they are up to 2.6x faster than k_part_scatter; below N = 32,768 the
// direct writes merge in L2.
static int part_scatter_kind(int64_t N, int32_t nb, int max_lds) {
    const int64_t part = cdiv(N, PACK_PARTS);
    if (N < PART_SORT_MIN_N) return RFXP_PACK_PARTS_DIRECT;
    auto wgs_per_cu = [&](size_t lds) { return lds * 2 <= (size_t)max_lds ? 2 : lds <= (size_t)max_lds ? 1 : 0; };
    const int occ4 = part <= PART_SORT4_MAX ? wgs_per_cu(part_sorted4_lds(nb, part)) : 0;
    const int occ2 = nb <= PART_SORT_MAX_NB && part <= PART_SORT_MAX ? wgs_per_cu(part_sorted_lds(nb, part)) : 0;
    if (occ4 > 0 && occ4 >= occ2) return RFXP_PACK_PARTS_SORTED4;
    return occ2 > 0 ? RFXP_PACK_PARTS_SORTED2 : RFXP_PACK_PARTS_DIRECT;
}

// Forest path for 2L <= PART_MAX_NB (see k_part_hist).
static int pack_forest_parts(rfxp_ctx* ctx, const LeafView& v, const int32_t* nout_in, const ForestBufs& fb) {
    hipStream_t s = ctx->stream;
    const int64_t N = v.N;
    const int32_t T = v.T;
    const int32_t nb = view_buckets(v);
    // every buffer these kernels write must have been sized by forest_sizes
    if (!fb.off || !fb.bend || !fb.mem || !fb.roff || !fb.rlen || !fb.scratch || !fb.key16 || !fb.lng ||
        !fb.lngn || (!nout_in && !fb.scratch2))
        return set_error(ctx, RFXP_ERR_STATE, "per-part packing: a forest index buffer was not allocated");
    const int64_t ldk = cdiv(N, 8) * 8;
    // (tree, part) blocks: 8 XCDs x ceil(T/8) trees x PACK_PARTS parts
    const unsigned grid = (unsigned)(8 * cdiv(T, 8) * PACK_PARTS);
    const size_t lds_h = (size_t)nb * 4;
    const int64_t part = cdiv(N, PACK_PARTS);
    const int kind = part_scatter_kind(N, nb, ctx->max_lds);
    const bool sorted4 = kind == RFXP_PACK_PARTS_SORTED4, sorted = kind == RFXP_PACK_PARTS_SORTED2;
    const void* scatter = sorted4  ? (const void*)k_part_scatter_sorted4
                          : sorted ? (const void*)k_part_scatter_sorted
                                   : (const void*)k_part_scatter;
    const size_t lds_s = sorted4  ? part_sorted4_lds(nb, part)
                         : sorted ? part_sorted_lds(nb, part)
                                  : (size_t)(2 * nb) * 4;
    if (lds_h > 32768)
        RFXP_HIP(ctx, hipFuncSetAttribute((const void*)k_part_hist, hipFuncAttributeMaxDynamicSharedMemorySize,
                                          (int)lds_h));
    if (lds_s > 32768)
        RFXP_HIP(ctx, hipFuncSetAttribute(scatter, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_s));
    {
        LaunchTimer tm(ctx, "pack_hist");
        hipLaunchKernelGGL(k_part_hist, dim3(grid), dim3(PACK_THREADS), lds_h, s, v, fb.scratch, fb.key16, ldk);
    }
    if (int rc = check_launch(ctx, "k_part_hist")) return rc;
    {
        LaunchTimer tm(ctx, "pack_scan");
        // fit: the line-fit layout (the tree stride exceeds N exactly then)
        hipLaunchKernelGGL(k_part_scan, dim3((unsigned)T), dim3(PACK_THREADS), 0, s, nb, T, fb.ms,
                           (int32_t)(fb.ms != N), fb.scratch, fb.off, fb.bend, fb.lng, fb.lngn, fb.lmax);
    }
    if (int rc = check_launch(ctx, "k_part_scan")) return rc;
    {
        LaunchTimer tm(ctx, "pack_scatter");
        if (sorted4)
            hipLaunchKernelGGL(k_part_scatter_sorted4, dim3(grid), dim3(PACK_THREADS), lds_s, s, v,
                               (const uint32_t*)fb.scratch, (const int32_t*)fb.bend, fb.ms, (const uint16_t*)fb.key16,
                               ldk, fb.mem);
        else if (sorted)
            hipLaunchKernelGGL(k_part_scatter_sorted, dim3(grid), dim3(PACK_THREADS), lds_s, s, v,
                               (const uint32_t*)fb.scratch, (const int32_t*)fb.bend, fb.ms, (const uint16_t*)fb.key16,
                               ldk, fb.mem);
        else
            hipLaunchKernelGGL(k_part_scatter, dim3(grid), dim3(PACK_THREADS), lds_s, s, v,
                               (const uint32_t*)fb.scratch, (const int32_t*)fb.bend, fb.ms, (const uint16_t*)fb.key16,
                               ldk, fb.mem);
    }
    if (int rc = check_launch(ctx, "k_part_scatter")) return rc;
    {
        LaunchTimer tm(ctx, "records");
        hipLaunchKernelGGL(k_part_records, dim3((unsigned)cdiv(N, PREC_S), (unsigned)cdiv(fb.ldr, PREC_T)), dim3(256),
                           0, s, (const uint16_t*)fb.key16, ldk, (const uint32_t*)fb.scratch,
                           (const int32_t*)fb.bend, nb, N, T, fb.ms, fb.ldr, fb.roff, fb.rlen, v.oob, v.old,
                           nout_in ? nullptr : fb.scratch2);
    }
    return check_launch(ctx, "k_part_records");
}

// nout, 1/nout and its range (forest mode).
static int pack_nout(rfxp_ctx* ctx, const LeafView& v, const int32_t* nout_in, const ForestBufs& fb) {
    hipStream_t s = ctx->stream;
    const int64_t N = v.N;
    // without nout_in, the records kernel (k_part_records or k_rec_transpose)
    // has summed the OOB bits into fb.scratch2
    {
        LaunchTimer tm(ctx, "nout_final");
        hipLaunchKernelGGL(k_nout_final, dim3((unsigned)cdiv(N, 256)), dim3(256), 0, s, N, nout_in,
                           nout_in ? (const uint32_t*)nullptr : fb.scratch2, fb.nout, fb.rinv, fb.rrange);
    }
    return check_launch(ctx, "k_nout_final");
}

}  // namespace rfxp

extern "C" int rfxp_pack_plan(int64_t N, int32_t T, int32_t nleaf, int32_t max_lds) {
    using namespace rfxp;
    if (N < 1 || N > MAX_FOREST_N || T < 1 || nleaf < 1 || nleaf > 0x3fffffff || max_lds < 1) return -1;
    LeafView v{};
    v.N = N;
    v.T = T;
    v.L = nleaf;
    const ForestSizes z = forest_sizes(v, true, max_lds);
    if (z.part_path) return part_scatter_kind(N, view_buckets(v), max_lds);
    return z.lds_path ? RFXP_PACK_TREE_LDS : RFXP_PACK_TREE_RANGES;
}
