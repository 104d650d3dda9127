// Host check of the line-fit bucket layout of the per-part packing path
// (rfx-fuse_amd/csrc/rfxp_pack.hip: k_part_hist, k_part_scan, the member
// scatters' slots and the run records), with the placement rule and the
// stride bound the kernels use (fit_start, fit_stride, FIT_GROUP).
//
// For a seeded forest of the given shape it rebuilds, per tree, every
// bucket's start and end, every part's slot range and every sample's run
// record, and asserts that:
//   - buckets lie in order inside [0, ms) of their tree, T * ms + MEM_PAD
//     stays below 2^30 (32-bit byte offsets, the triangle's buffer range);
//   - a bucket of at most 32 members lies in one 128-byte line, a larger one
//     ends on a line boundary;
//   - every member slot of every part lies inside its bucket;
//   - every run [off, off + len) lies inside its bucket, so inside mem;
//   - long buckets' table entries lie inside mem.
// It prints the mean number of 128-byte lines a run touches and ms / N.
//
// usage: layout_check N T L [p_invalid] [seed]
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include "rfxp_forest.hpp"

using namespace rfxp;

static int fail(const char* what, long long a, long long b, long long c) {
    std::printf("FAIL %s: %lld %lld %lld\n", what, a, b, c);
    return 1;
}

int main(int argc, char** argv) {
    if (argc < 4) {
        std::printf("usage: layout_check N T L [p_invalid] [seed]\n");
        return 2;
    }
    const int64_t N = std::atoll(argv[1]);
    const int32_t T = std::atoi(argv[2]), L = std::atoi(argv[3]);
    const double p_invalid = argc > 4 ? std::atof(argv[4]) : 0.0;
    const uint64_t seed = argc > 5 ? std::strtoull(argv[5], nullptr, 10) : 1;
    const int32_t nb = 2 * L;
    const int P = 8;  // PACK_PARTS
    const int64_t ms = fit_stride(N, nb);
    if (ms % LINE_IDS) return fail("stride not a whole number of lines", ms, 0, 0);
    if ((int64_t)T * ms + MEM_PAD >= (1LL << 30)) return fail("T * ms above 2^30", T, ms, 0);
    const uint64_t mem_bytes = ((uint64_t)T * ms + MEM_PAD) * 4;
    const int64_t chunk = (N + P - 1) / P;
    auto part_begin = [&](int p) { return std::min<int64_t>(N, (int64_t)p * chunk); };
    std::mt19937_64 rng(seed);
    std::uniform_int_distribution<int32_t> leaf_d(0, L - 1);
    std::uniform_real_distribution<double> u01(0.0, 1.0);
    std::vector<int32_t> key(N);
    std::vector<uint32_t> cnt((size_t)P * nb), ps((size_t)P * nb), sz(nb), start(nb), end(nb);
    double lines = 0.0, runs = 0.0, used = 0.0;
    int64_t max_used = 0;
    for (int32_t t = 0; t < T; ++t) {
        std::fill(cnt.begin(), cnt.end(), 0u);
        for (int64_t i = 0; i < N; ++i) {
            const bool bad = p_invalid > 0 && u01(rng) < p_invalid;
            const int32_t l = leaf_d(rng);
            const uint32_t o = u01(rng) < 0.368 ? 1u : 0u;
            key[i] = bad ? -1 : 2 * l + (int32_t)o;
            if (key[i] >= 0) ++cnt[(size_t)(i / chunk) * nb + key[i]];
        }
        // k_part_scan: groups of FIT_GROUP buckets from line-aligned starts
        uint32_t gbase = 0;
        for (int32_t b0 = 0; b0 < nb; b0 += FIT_GROUP) {
            uint32_t pos = 0;
            for (int32_t b = b0; b < std::min(nb, b0 + FIT_GROUP); ++b) {
                uint32_t s = 0;
                for (int q = 0; q < P; ++q) s += cnt[(size_t)q * nb + b];
                sz[b] = s;
                const uint32_t st = fit_start(pos, s);
                if (st < pos) return fail("placement moved back", b, st, pos);
                start[b] = gbase + st;
                end[b] = start[b] + s;
                pos = st + s;
            }
            gbase += (pos + LINE_IDS - 1) & ~(LINE_IDS - 1);
        }
        if ((int64_t)gbase > ms) return fail("tree length above the stride bound", t, gbase, ms);
        used += gbase;
        max_used = std::max<int64_t>(max_used, gbase);
        for (int32_t b = 0; b < nb; ++b) {
            if (b > 0 && start[b] < end[b - 1]) return fail("buckets overlap", t, b, start[b]);
            if (end[b] > (uint32_t)ms) return fail("bucket past the stride", t, b, end[b]);
            if (sz[b] > 0 && sz[b] <= LINE_IDS && start[b] / LINE_IDS != (end[b] - 1) / LINE_IDS)
                return fail("small bucket straddles a line", t, b, start[b]);
            if (sz[b] > LINE_IDS && end[b] % LINE_IDS) return fail("large bucket not line-ended", t, b, end[b]);
            if (sz[b] >= REC_LONG) {
                const uint64_t lo = 4ull * ((uint64_t)t * ms + start[b]), hi = 4ull * ((uint64_t)t * ms + end[b]);
                if (hi > mem_bytes || lo > hi) return fail("long-bucket entry outside mem", t, b, (long long)hi);
            }
            uint32_t run = start[b];
            for (int q = 0; q < P; ++q) {
                ps[(size_t)q * nb + b] = run;
                run += cnt[(size_t)q * nb + b];
                // the scatter writes part q's members of b to [ps, ps + cnt)
                if (run > end[b]) return fail("part slots past the bucket end", t, b, q);
            }
        }
        // records: the run of (i, t) in the opposite bucket from i's part on
        for (int64_t i = 0; i < N; ++i) {
            if (key[i] < 0) continue;
            const int32_t ob = key[i] ^ 1;
            const int q = (int)(i / chunk);
            if (part_begin(q) > i || part_begin(q + 1) <= i) return fail("part of sample", i, q, 0);
            const uint32_t rs = ps[(size_t)q * nb + ob], rem = end[ob] - rs;
            if (rs < start[ob] || rs > end[ob]) return fail("run start outside its bucket", t, i, rs);
            const uint64_t off = 4ull * ((uint64_t)t * ms + rs);
            const uint64_t len4 = 4ull * std::min<uint32_t>(rem, REC_LONG);
            if (off + len4 > mem_bytes) return fail("run past mem", t, i, (long long)(off + len4));
            if (rem > 0) {
                const uint64_t e = 4ull * ((uint64_t)t * ms + end[ob]);
                lines += (double)((e - 1) / 128 - off / 128 + 1);
                runs += 1.0;
            }
        }
    }
    std::printf("ok N=%lld T=%d L=%d ms=%lld (%.3f x N) used=%.3f x N max_used=%lld lines_per_run=%.4f runs=%.0f\n",
                (long long)N, T, L, (long long)ms, (double)ms / N, used / T / N, (long long)max_used,
                runs > 0 ? lines / runs : 0.0, runs);
    return 0;
}
