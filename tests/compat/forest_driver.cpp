// Test driver of rfx::ForestProximity (include/rfx_forest.hpp), the object
// RandomForest's proximity queries forward to.  Reads (little-endian):
//   int32 N, T, K; int16 leaf[T*N]; per sample: int32 count, tree ids;
//   int32 npairs, pairs[2*npairs]; int32 nq, int16 new_leaves[nq*T];
//   int32 classes[N].
// Writes: float pair proximities; per sample q: int32 m, m x (int32 idx,
// float score) of get_top_k_similar(q, K, true), then of (q, K, false) for
// q < 5; predict idx[nq*K], score[nq*K]; proximity matrix N*N float;
// outlier scores without and with classes (2 x N float).
#include <stdio.h>
#include <stdlib.h>

#include <vector>

#include "rfx_compat.hpp"
#include "rfx_forest.hpp"

static void rd(FILE* f, void* p, size_t n) {
    if (fread(p, 1, n, f) != n) {
        fprintf(stderr, "short read\n");
        exit(2);
    }
}

int main(int argc, char** argv) {
    if (argc != 3) return 2;
    FILE* f = fopen(argv[1], "rb");
    if (!f) return 2;
    int32_t hdr[3];
    rd(f, hdr, sizeof(hdr));
    const int32_t N = hdr[0], T = hdr[1], K = hdr[2];
    std::vector<int16_t> leaf((size_t)T * N);
    rd(f, leaf.data(), 2 * leaf.size());
    std::vector<std::vector<int32_t>> oob(N);
    for (int32_t i = 0; i < N; ++i) {
        int32_t c;
        rd(f, &c, 4);
        oob[i].resize(c);
        rd(f, oob[i].data(), 4 * (size_t)c);
    }
    int32_t np_;
    rd(f, &np_, 4);
    std::vector<int32_t> pairs(2 * (size_t)np_);
    rd(f, pairs.data(), 4 * pairs.size());
    int32_t nq;
    rd(f, &nq, 4);
    std::vector<int16_t> qleaf((size_t)nq * T);
    rd(f, qleaf.data(), 2 * qleaf.size());
    std::vector<int32_t> classes(N);
    rd(f, classes.data(), 4 * (size_t)N);
    fclose(f);

    rfx::ForestProximity fp(leaf.data(), N, T, oob, 0);
    if (!fp.ok()) {
        fprintf(stderr, "ForestProximity: %s\n", rfx_compat_last_error());
        return 3;
    }
    FILE* o = fopen(argv[2], "wb");
    if (!o) return 2;
    for (int32_t p = 0; p < np_; ++p) {
        const float v = fp.compute_proximity_from_leaves(pairs[2 * p], pairs[2 * p + 1]);
        fwrite(&v, 4, 1, o);
    }
    auto dump = [&](const std::vector<std::pair<int32_t, float>>& r) {
        const int32_t m = (int32_t)r.size();
        fwrite(&m, 4, 1, o);
        for (auto& e : r) {
            fwrite(&e.first, 4, 1, o);
            fwrite(&e.second, 4, 1, o);
        }
    };
    for (int32_t q = 0; q < N; ++q) dump(fp.get_top_k_similar(q, K, true));
    for (int32_t q = 0; q < 5 && q < N; ++q) dump(fp.get_top_k_similar(q, K, false));
    std::vector<int32_t> pi((size_t)nq * K);
    std::vector<float> ps((size_t)nq * K);
    if (!fp.predict_top_k_similar(qleaf.data(), nq, K, pi.data(), ps.data())) return 4;
    fwrite(pi.data(), 4, pi.size(), o);
    fwrite(ps.data(), 4, ps.size(), o);
    std::vector<float> P((size_t)N * N);
    if (!fp.get_proximity_matrix(P.data())) return 4;
    fwrite(P.data(), 4, P.size(), o);
    std::vector<float> s0 = fp.compute_outlier_scores(nullptr), s1 = fp.compute_outlier_scores(classes.data());
    if ((int32_t)s0.size() != N || (int32_t)s1.size() != N) return 4;
    fwrite(s0.data(), 4, N, o);
    fwrite(s1.data(), 4, N, o);
    fclose(o);
    if (rfx_compat_last_error()[0]) {
        fprintf(stderr, "error: %s\n", rfx_compat_last_error());
        return 4;
    }
    printf("forest_driver ok N=%d T=%d K=%d\n", N, T, K);
    return 0;
}
