/*
 * rfx_oracle.c -- CPU restatement of RFX-Fuse's proximity path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product): loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
 * Written from the reference's algorithm, not from its code; each function
 * names the reference lines it restates.  Built with -ffp-contract=off and
 * without fast-math so that every double/float operation is the IEEE
 * operation the reference performs.
 */
#include "rfx_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define UNUSED_LABEL (-1)

static inline int64_t tri_idx(int64_t N, int64_t i, int64_t j) {
    return i * N - i * (i + 1) / 2 + j;
}

/* ------------------------------------------------------------------------ */
/* a1: src/rf_proximity.cpp:99-231                                           */
/* ------------------------------------------------------------------------ */
void orc_cpu_proximity(const int32_t* nodestatus, const int32_t* nodextr, const int32_t* nin,
                       int32_t nsample, int32_t nnode, int use_casewise, double* prox) {
    const int64_t N = nsample;
    int32_t* nod = (int32_t*)malloc(sizeof(int32_t) * (size_t)(nnode > 0 ? nnode : 1));
    int32_t* term = (int32_t*)malloc(sizeof(int32_t) * (size_t)(N > 0 ? N : 1));
    int32_t nterm = 0;
    /* terminal nodes get ordinals (src/rf_proximity.cpp:110-119) */
    for (int32_t k = 0; k < nnode; ++k) nod[k] = (nodestatus[k] == -1) ? nterm++ : -1;
    /* sample -> terminal ordinal or -1 (src/rf_proximity.cpp:126-135) */
    for (int64_t n = 0; n < N; ++n) {
        int32_t node = nodextr[n];
        term[n] = (node >= 0 && node < nnode) ? nod[node] : -1;
    }
    /* CSR of members per terminal ordinal, in sample order (:138-171) */
    int32_t* start = (int32_t*)calloc((size_t)nterm + 1, sizeof(int32_t));
    int32_t* members = (int32_t*)malloc(sizeof(int32_t) * (size_t)(N > 0 ? N : 1));
    int32_t* fill = (int32_t*)calloc((size_t)nterm + 1, sizeof(int32_t));
    for (int64_t n = 0; n < N; ++n)
        if (term[n] >= 0) start[term[n] + 1]++;
    for (int32_t k = 0; k < nterm; ++k) start[k + 1] += start[k];
    for (int64_t n = 0; n < N; ++n)
        if (term[n] >= 0) members[start[term[n]] + fill[term[n]]++] = (int32_t)n;
    /* OOB n x in-bag kk of the same terminal node (:179-230) */
    for (int64_t n = 0; n < N; ++n) {
        if (nin[n] != 0) continue;
        int32_t k = term[n];
        if (k < 0) continue;
        int32_t nodesize = 0;
        for (int32_t p = start[k]; p < start[k + 1]; ++p)
            if (nin[members[p]] > 0) nodesize += nin[members[p]];
        if (!(nodesize > 0 || !use_casewise)) continue;
        for (int32_t p = start[k]; p < start[k + 1]; ++p) {
            int32_t kk = members[p];
            if (nin[kk] <= 0) continue;
            double w = (use_casewise && nodesize > 0) ? (double)nin[kk] / (double)nodesize : 1.0;
            prox[n + (int64_t)kk * N] += w;
        }
    }
    free(nod);
    free(term);
    free(start);
    free(members);
    free(fill);
}

/* ------------------------------------------------------------------------ */
/* a2: src/rf_finishprox.cpp:12-74                                           */
/* ------------------------------------------------------------------------ */
void orc_finishprox(int32_t nsample, const int32_t* nout, const double* prox, double* proxsym) {
    const int64_t N = nsample;
    for (int64_t e = 0; e < N * N; ++e) proxsym[e] = prox[e];               /* :19-21 */
    for (int64_t i = 0; i < N; ++i) proxsym[i + i * N] = (double)nout[i];   /* :26-28 */
    for (int64_t i = 0; i < N; ++i)                                         /* :33-42 */
        for (int64_t j = i + 1; j < N; ++j) {
            double avg = (prox[i + j * N] + prox[j + i * N]) / 2.0;
            proxsym[i + j * N] = avg;
            proxsym[j + i * N] = avg;
        }
    for (int64_t i = 0; i < N; ++i) {                                       /* :47-55 */
        if (nout[i] <= 0) continue;
        double inv = 1.0 / (double)nout[i];
        for (int64_t j = 0; j < N; ++j) proxsym[i + j * N] *= inv;
    }
    for (int64_t i = 0; i < N; ++i) {                                       /* :61-73 */
        proxsym[i + i * N] = 1.0;
        for (int64_t j = i + 1; j < N; ++j) {
            double avg = 0.5 * (proxsym[i + j * N] + proxsym[j + i * N]);
            proxsym[i + j * N] = avg;
            proxsym[j + i * N] = avg;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* a10: src/rf_proximity.cpp:238-397 (RF-GAP)                                */
/* ------------------------------------------------------------------------ */
void orc_rfgap(int32_t ntree, int32_t nsample, const int32_t* nin_flat,
               const int32_t* nodextr_flat, double* prox) {
    const int64_t N = nsample;
    memset(prox, 0, sizeof(double) * (size_t)(N * N));
    for (int64_t i = 0; i < N; ++i) {
        int32_t n_oob = 0;
        for (int32_t t = 0; t < ntree; ++t)
            if (nin_flat[(int64_t)t * N + i] == 0) n_oob++;
        if (n_oob == 0) {                       /* :314-318 */
            prox[i + i * N] = 1.0;
            continue;
        }
        for (int32_t t = 0; t < ntree; ++t) {   /* trees in ascending order (:321) */
            const int32_t* nin = nin_flat + (int64_t)t * N;
            const int32_t* ndx = nodextr_flat + (int64_t)t * N;
            if (nin[i] != 0) continue;
            int32_t node = ndx[i];
            if (node < 0) continue;
            int32_t mult = 0;
            for (int64_t j = 0; j < N; ++j)
                if (nin[j] > 0 && ndx[j] == node) mult += nin[j];
            if (mult == 0) continue;
            double inv = 1.0 / (double)mult;
            for (int64_t j = 0; j < N; ++j)
                if (nin[j] > 0 && ndx[j] == node) prox[i + j * N] += (double)nin[j] * inv;
        }
        double norm = 1.0 / (double)n_oob;       /* :370-375 */
        for (int64_t j = 0; j < N; ++j) prox[i + j * N] *= norm;
    }
    for (int64_t i = 0; i < N; ++i)              /* :383-396 */
        for (int64_t j = i + 1; j < N; ++j) {
            double avg = (prox[i + j * N] + prox[j + i * N]) / 2.0;
            prox[i + j * N] = avg;
            prox[j + i * N] = avg;
        }
}

void orc_terminal_leaf(const int32_t* nodestatus, int32_t nnode, const int32_t* nodextr,
                       int32_t nsample, int32_t* leaf_out) {
    int32_t* nod = (int32_t*)malloc(sizeof(int32_t) * (size_t)(nnode > 0 ? nnode : 1));
    int32_t nterm = 0;
    for (int32_t k = 0; k < nnode; ++k) nod[k] = (nodestatus[k] == -1) ? nterm++ : -1;
    for (int32_t n = 0; n < nsample; ++n) {
        int32_t node = nodextr[n];
        leaf_out[n] = (node >= 0 && node < nnode) ? nod[node] : UNUSED_LABEL;
    }
    free(nod);
}

/* ------------------------------------------------------------------------ */
/* normalisation + quantizers                                                */
/* ------------------------------------------------------------------------ */

/* For i != j with integer counts c_ij, c_ji (U = c_ij + c_ji) the finishprox
 * steps reduce to this sequence of IEEE double operations
 * (src/rf_finishprox.cpp:38, :49-52, :69). */
double orc_p(uint32_t U, int32_t n_i, int32_t n_j) {
    double s = (double)U / 2.0;
    double a = (n_i > 0) ? s * (1.0 / (double)n_i) : s;
    double b = (n_j > 0) ? s * (1.0 / (double)n_j) : s;
    return 0.5 * (a + b);
}

/* IEEE-754 binary32 -> binary16, round to nearest even. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ex = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (ex == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
    int32_t e = (int32_t)ex - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t h = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

int8_t orc_q_i8(float v, float scale, float zp) {
    float r = v / scale + zp;
    r = fmaxf(-128.0f, fminf(127.0f, r));
    return (int8_t)r;
}

uint8_t orc_q_nf4(float v) {
    if (v >= 0.0f) return (uint8_t)fminf(7.0f, roundf(v * 7.0f));
    return (uint8_t)fmaxf(8.0f, roundf(8.0f - v * 7.0f));
}

uint8_t orc_q_u8(float v, float scale, float zp) {
    float r = v / scale + zp;
    r = fmaxf(0.0f, fminf(255.0f, r));
    return (uint8_t)r;
}

void orc_u8_scale_from_minmax(float vmin, float vmax, float* scale, float* zp) {
    float s = (vmax - vmin) / 255.0f;
    *scale = s;
    *zp = -vmin / s;
}

/* Writes the entry for (U, n_i, n_j) -- or the diagonal when diag -- into
 * a packed output at element e. NF4 entries are OR-ed into a zeroed byte. */
static inline void put_entry(int fmt, void* out, int64_t e, int diag, uint32_t U, int32_t ni,
                             int32_t nj, float scale, float zp) {
    double P = diag ? 1.0 : orc_p(U, ni, nj);
    float pf = (float)P;
    switch (fmt) {
        case 0: ((float*)out)[e] = pf; break;
        case 1: ((uint16_t*)out)[e] = orc_f32_to_f16(pf); break;
        case 2: ((int8_t*)out)[e] = orc_q_i8(pf, scale, zp); break;
        case 3: ((uint8_t*)out)[e >> 1] |= (uint8_t)((orc_q_nf4(pf) & 0xfu) << ((e & 1) * 4)); break;
        case 4: ((uint8_t*)out)[e] = orc_q_u8(pf, scale, zp); break;
        case 5: ((uint16_t*)out)[e] = diag ? 0 : (uint16_t)U; break;
        default: break;
    }
}

void orc_nout(const uint8_t* oob, int64_t N, int32_t T, int32_t* nout) {
    for (int64_t i = 0; i < N; ++i) nout[i] = 0;
    for (int32_t t = 0; t < T; ++t)
        for (int64_t i = 0; i < N; ++i) nout[i] += oob[(int64_t)t * N + i] ? 1 : 0;
}

/* ------------------------------------------------------------------------ */
/* counts, reference-shaped                                                  */
/* ------------------------------------------------------------------------ */

/* CSR of one tree's members grouped by label, in ascending sample order. */
typedef struct {
    int32_t* start; /* nleaf + 1 */
    int32_t* mem;   /* N */
} tree_csr;

static void csr_build(const int32_t* lab, int64_t N, int32_t nleaf, tree_csr* c) {
    c->start = (int32_t*)calloc((size_t)nleaf + 1, sizeof(int32_t));
    c->mem = (int32_t*)malloc(sizeof(int32_t) * (size_t)(N > 0 ? N : 1));
    int32_t* fill = (int32_t*)calloc((size_t)nleaf + 1, sizeof(int32_t));
    for (int64_t n = 0; n < N; ++n)
        if (lab[n] >= 0 && lab[n] < nleaf) c->start[lab[n] + 1]++;
    for (int32_t l = 0; l < nleaf; ++l) c->start[l + 1] += c->start[l];
    for (int64_t n = 0; n < N; ++n)
        if (lab[n] >= 0 && lab[n] < nleaf) c->mem[c->start[lab[n]] + fill[lab[n]]++] = (int32_t)n;
    free(fill);
}

static void csr_free(tree_csr* c) {
    free(c->start);
    free(c->mem);
}

void orc_upper_counts_scatter(const int32_t* leaf, const uint8_t* oob, int64_t N, int32_t T,
                              int32_t nleaf, uint16_t* U) {
    memset(U, 0, sizeof(uint16_t) * (size_t)(N * (N + 1) / 2));
    for (int32_t t = 0; t < T; ++t) {
        const int32_t* lab = leaf + (int64_t)t * N;
        const uint8_t* ob = oob + (int64_t)t * N;
        tree_csr c;
        csr_build(lab, N, nleaf, &c);
        for (int64_t n = 0; n < N; ++n) {
            if (!ob[n]) continue;                       /* OOB sample n */
            int32_t l = lab[n];
            if (l < 0 || l >= nleaf) continue;
            for (int32_t p = c.start[l]; p < c.start[l + 1]; ++p) {
                int32_t kk = c.mem[p];
                if (ob[kk]) continue;                   /* in-bag partner only */
                int64_t i = n < kk ? n : kk, j = n < kk ? kk : n;
                U[tri_idx(N, i, j)]++;
            }
        }
        csr_free(&c);
    }
}

/* ------------------------------------------------------------------------ */
/* counts, row-oriented (same count, used for row ranges and the baseline)   */
/* ------------------------------------------------------------------------ */
struct orc_index {
    const int32_t* leaf;
    const uint8_t* oob;
    int64_t N;
    int32_t T;
    int32_t nleaf;
    int32_t* nout;
    tree_csr* csr;
};

orc_index* orc_index_build(const int32_t* leaf, const uint8_t* oob, int64_t N, int32_t T,
                           int32_t nleaf, const int32_t* nout_in, int threads) {
    orc_index* x = (orc_index*)calloc(1, sizeof(orc_index));
    x->leaf = leaf;
    x->oob = oob;
    x->N = N;
    x->T = T;
    x->nleaf = nleaf;
    x->csr = (tree_csr*)malloc(sizeof(tree_csr) * (size_t)(T > 0 ? T : 1));
    x->nout = (int32_t*)malloc(sizeof(int32_t) * (size_t)(N > 0 ? N : 1));
    if (nout_in) memcpy(x->nout, nout_in, sizeof(int32_t) * (size_t)N);
    else orc_nout(oob, N, T, x->nout);
#ifdef _OPENMP
    int nth = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nth)
#endif
    for (int32_t t = 0; t < T; ++t) csr_build(leaf + (int64_t)t * N, N, nleaf, &x->csr[t]);
    return x;
}

void orc_index_free(orc_index* x) {
    if (!x) return;
    for (int32_t t = 0; t < x->T; ++t) csr_free(&x->csr[t]);
    free(x->csr);
    free(x->nout);
    free(x);
}

int orc_index_rows(const orc_index* x, int fmt, float scale, float zp, int64_t r0, int64_t r1,
                   void* out, int threads) {
    const int64_t N = x->N;
    const int32_t T = x->T;
    const int32_t nleaf = x->nleaf;
    const int32_t* leaf = x->leaf;
    const uint8_t* oob = x->oob;
    const int32_t* nout = x->nout;
    const tree_csr* csr = x->csr;
    if (r0 < 0 || r1 > N || r0 > r1) return -1;
#ifdef _OPENMP
    int nth = threads > 0 ? threads : omp_get_max_threads();
#endif
    const int64_t base = tri_idx(N, r0, r0);
    if (fmt == 3) { /* NF4: zero the bytes we own before OR-ing nibbles in */
        int64_t e0 = base, e1 = tri_idx(N, r1, r1);
        if (e1 > e0) memset((uint8_t*)out, 0, (size_t)(((e1 - 1) >> 1) - (e0 >> 1) + 1));
    }
#ifdef _OPENMP
#pragma omp parallel num_threads(nth)
#endif
    {
        uint16_t* cnt = (uint16_t*)calloc((size_t)(N > 0 ? N : 1), sizeof(uint16_t));
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 8)
#endif
        for (int64_t i = r0; i < r1; ++i) {
            for (int32_t t = 0; t < T; ++t) {
                int32_t l = leaf[(int64_t)t * N + i];
                if (l < 0 || l >= nleaf) continue;
                const uint8_t* ob = oob + (int64_t)t * N;
                uint8_t oi = ob[i] ? 1 : 0;
                const tree_csr* c = &csr[t];
                for (int32_t p = c->start[l + 1] - 1; p >= c->start[l]; --p) {
                    int32_t j = c->mem[p];
                    if (j <= i) break;                   /* members ascend */
                    if ((ob[j] ? 1 : 0) != oi) cnt[j]++;
                }
            }
            int64_t rowe = tri_idx(N, i, i) - base;
            for (int64_t j = i; j < N; ++j) {
                int64_t e = rowe + (j - i);
                if (fmt == 3) {
                    /* NF4 bytes straddling two rows are shared between
                     * threads: compose atomically */
                    double P = (j == i) ? 1.0 : orc_p(cnt[j], nout[i], nout[j]);
                    uint8_t v = (uint8_t)((orc_q_nf4((float)P) & 0xfu) << (((e + base) & 1) * 4));
                    if (v) {
#ifdef _OPENMP
#pragma omp atomic
#endif
                        ((uint8_t*)out)[((e + base) >> 1) - (base >> 1)] |= v;
                    }
                } else {
                    put_entry(fmt, out, e, j == i, cnt[j], nout[i], nout[j], scale, zp);
                }
                cnt[j] = 0;
            }
        }
        free(cnt);
    }
    return 0;
}

int orc_upper_rows(const int32_t* leaf, const uint8_t* oob, int64_t N, int32_t T, int32_t nleaf,
                   const int32_t* nout_in, int fmt, float scale, float zp, int64_t r0, int64_t r1,
                   void* out, int threads) {
    if (r0 < 0 || r1 > N || r0 > r1) return -1;
    orc_index* x = orc_index_build(leaf, oob, N, T, nleaf, nout_in, threads);
    int rc = orc_index_rows(x, fmt, scale, zp, r0, r1, out, threads);
    orc_index_free(x);
    return rc;
}

int orc_both_oob_rows(const int32_t* leaf, const uint8_t* oob, int64_t N, int32_t T, int32_t nleaf, int fmt,
                      int64_t r0, int64_t r1, void* out, int threads) {
    if (r0 < 0 || r1 > N || r0 > r1 || (fmt != 0 && fmt != 5)) return -1;
    const int64_t e0 = tri_idx(N, r0, r0);
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 4)
    for (int64_t i = r0; i < r1; ++i) {
        for (int64_t j = i; j < N; ++j) {
            uint32_t num = 0, den = 0;
            if (j != i) {
                for (int32_t t = 0; t < T; ++t) {
                    if (!oob[(int64_t)t * N + i] || !oob[(int64_t)t * N + j]) continue;
                    ++den;
                    const int32_t a = leaf[(int64_t)t * N + i], b = leaf[(int64_t)t * N + j];
                    if (a == b && a >= 0 && a < nleaf) ++num;
                }
            }
            const int64_t e = tri_idx(N, i, j) - e0;
            if (fmt == 5) ((uint16_t*)out)[e] = (uint16_t)num;
            else ((float*)out)[e] = (j == i) ? 1.0f : (den > 0 ? (float)num / (float)den : 0.0f);
        }
    }
    return 0;
}

void orc_upper_from_counts(const uint16_t* U, const int32_t* nout, int64_t N, int fmt, float scale,
                           float zp, void* out) {
    if (fmt == 3) memset(out, 0, (size_t)((N * (N + 1) / 2 + 1) / 2));
    for (int64_t i = 0; i < N; ++i)
        for (int64_t j = i; j < N; ++j) {
            int64_t e = tri_idx(N, i, j);
            put_entry(fmt, out, e, i == j, U[e], nout[i], nout[j], scale, zp);
        }
}

/* ------------------------------------------------------------------------ */
/* top-K                                                                     */
/* ------------------------------------------------------------------------ */

/* Keep the K best (count desc, index asc) in a sorted array. */
static inline void topk_insert(int32_t K, int32_t* n_have, int32_t* bi, uint16_t* bc, int32_t j,
                               uint16_t c) {
    int32_t n = *n_have;
    if (n == K) {
        uint16_t lc = bc[K - 1];
        int32_t li = bi[K - 1];
        if (c < lc || (c == lc && j > li)) return;
        n = K - 1;
    }
    int32_t p = n;
    while (p > 0 && (bc[p - 1] < c || (bc[p - 1] == c && bi[p - 1] > j))) {
        bc[p] = bc[p - 1];
        bi[p] = bi[p - 1];
        --p;
    }
    bc[p] = c;
    bi[p] = j;
    *n_have = n + 1;
}

void orc_topk_all(const int32_t* ref_leaf, int64_t N, int32_t T, int32_t nleaf, const int32_t* qleaf, int64_t Q,
                  int32_t K, const int32_t* exclude, int32_t* idx_out, uint16_t* cnt_out,
                  int threads) {
#ifdef _OPENMP
    int nth = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel num_threads(nth)
#endif
    {
        uint16_t* cnt = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(N > 0 ? N : 1));
        int32_t* bi = (int32_t*)malloc(sizeof(int32_t) * (size_t)(K > 0 ? K : 1));
        uint16_t* bc = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(K > 0 ? K : 1));
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 4)
#endif
        for (int64_t q = 0; q < Q; ++q) {
            memset(cnt, 0, sizeof(uint16_t) * (size_t)N);
            for (int32_t t = 0; t < T; ++t) {
                int32_t ql = qleaf[q * T + t];
                if (ql < 0 || ql >= nleaf) continue;   /* an invalid label matches nothing */
                const int32_t* rl = ref_leaf + (int64_t)t * N;
                for (int64_t j = 0; j < N; ++j) cnt[j] += (rl[j] == ql);
            }
            int32_t have = 0;
            int32_t ex = exclude ? exclude[q] : -1;
            for (int64_t j = 0; j < N; ++j)
                if (j != ex) topk_insert(K, &have, bi, bc, (int32_t)j, cnt[j]);
            for (int32_t k = 0; k < K; ++k) {
                idx_out[q * K + k] = k < have ? bi[k] : -1;
                cnt_out[q * K + k] = k < have ? bc[k] : 0;
            }
        }
        free(cnt);
        free(bi);
        free(bc);
    }
}

int32_t orc_topk_oob(const int32_t* leaf, const uint8_t* oob, int64_t N, int32_t T, int32_t nleaf, int64_t q,
                     int32_t K, int exclude_self, int32_t* idx_out, uint16_t* cnt_out,
                     float* score_out) {
    uint16_t* cnt = (uint16_t*)calloc((size_t)(N > 0 ? N : 1), sizeof(uint16_t));
    int32_t n_oob = 0;
    for (int32_t t = 0; t < T; ++t) {
        if (!oob[(int64_t)t * N + q]) continue;
        n_oob++;
        int32_t ql = leaf[(int64_t)t * N + q];
        if (ql < 0 || ql >= nleaf) continue;   /* the tree counts in |OOB(q)|, its label matches nothing */
        const int32_t* rl = leaf + (int64_t)t * N;
        for (int64_t j = 0; j < N; ++j)
            if (rl[j] == ql && !(exclude_self && j == q)) cnt[j]++;
    }
    int32_t have = 0;
    if (n_oob > 0) {
        int32_t* bi = (int32_t*)malloc(sizeof(int32_t) * (size_t)(K > 0 ? K : 1));
        uint16_t* bc = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(K > 0 ? K : 1));
        for (int64_t j = 0; j < N; ++j)
            if (cnt[j] > 0 && !(exclude_self && j == q)) topk_insert(K, &have, bi, bc, (int32_t)j, cnt[j]);
        float norm = 1.0f / (float)n_oob;   /* src/rf_random_forest.cpp:4744 */
        for (int32_t k = 0; k < have; ++k) {
            idx_out[k] = bi[k];
            cnt_out[k] = bc[k];
            score_out[k] = (float)bc[k] * norm;
        }
        free(bi);
        free(bc);
    }
    free(cnt);
    return have;
}

/* ------------------------------------------------------------------------ */
/* low rank: P V with P = A A^T / T                                          */
/* ------------------------------------------------------------------------ */
void orc_lowrank_pv(const int32_t* leaf, int64_t N, int32_t T, int32_t nleaf, const double* V,
                    int32_t r, double* Y, int threads) {
    /* W_t[l] = sum over j ascending of V_j (one tree per thread), then
     * Y_i = sum over t ascending of W_t[leaf_i(t)] (rows split over threads):
     * the same additions in the same order for any thread count. */
    const int nth = threads > 0 ? threads : omp_get_max_threads();
    double* W = (double*)calloc((size_t)T * (size_t)nleaf * (size_t)r, sizeof(double));
#pragma omp parallel for num_threads(nth) schedule(dynamic, 1)
    for (int32_t t = 0; t < T; ++t) {
        const int32_t* lab = leaf + (int64_t)t * N;
        double* Wt = W + (size_t)t * (size_t)nleaf * (size_t)r;
        for (int64_t j = 0; j < N; ++j) {
            int32_t l = lab[j];
            if (l < 0 || l >= nleaf) continue;
            for (int32_t c = 0; c < r; ++c) Wt[(int64_t)l * r + c] += V[j * r + c];
        }
    }
#pragma omp parallel for num_threads(nth) schedule(static)
    for (int64_t i = 0; i < N; ++i) {
        double* y = Y + i * r;
        for (int32_t c = 0; c < r; ++c) y[c] = 0.0;
        for (int32_t t = 0; t < T; ++t) {
            int32_t l = leaf[(int64_t)t * N + i];
            if (l < 0 || l >= nleaf) continue;
            const double* w = W + ((size_t)t * (size_t)nleaf + (size_t)l) * (size_t)r;
            for (int32_t c = 0; c < r; ++c) y[c] += w[c];
        }
        for (int32_t c = 0; c < r; ++c) y[c] /= (double)T;
    }
    free(W);
}

/* ------------------------------------------------------------------------ */
/* a4: per-tree triangles, cuda/rf_proximity_upper_triangle.cu              */
/* ------------------------------------------------------------------------ */

static float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const int32_t ex = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (ex == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal half -> normal float */
            int32_t e = -1;
            do {
                man <<= 1;
                ++e;
            } while (!(man & 0x400u));
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (ex == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((uint32_t)(ex - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* include/rf_quantization_kernels.hpp:53-65 */
static float orc_nf4_to_f32(uint8_t q) {
    if (q <= 7) return (float)q / 7.0f;
    return -((float)(q - 8)) / 7.0f;
}

static int64_t tri_index64(int64_t n, int64_t i, int64_t j) { return i * n - i * (i + 1) / 2 + j; }

void orc_tree_upper(int fmt, const int32_t* nodestatus, const int32_t* nodextr, const int32_t* nin, int32_t nsample,
                    int32_t nnode, int casewise, int32_t n_real, float scale, float zp, void* out) {
    const int64_t N = nsample;
    const int64_t np = (n_real > 0 && n_real < nsample) ? n_real : nsample;
    const int64_t ne = np * (np + 1) / 2;
    if (fmt == 1) memset(out, 0, (size_t)(2 * ne));
    else if (fmt == 2) memset(out, 0, (size_t)ne);
    else memset(out, 0, (size_t)((ne + 1) / 2));
    /* members of each node (node index as key), in sample order */
    for (int64_t n = 0; n < np; ++n) {
        if (fmt != 2 && nin[n] > 0) continue; /* F16 / NF4: OOB samples only */
        const int32_t k = nodextr[n];
        if (k < 0 || k >= nnode || nodestatus[k] != -1) continue;
        int32_t nodesize = 0;
        for (int64_t j = 0; j < N; ++j)
            if (nodextr[j] == k && nin[j] > 0) nodesize += nin[j];
        if (fmt == 2 ? !(nodesize > 0) : !(nodesize > 0 || !casewise)) continue;
        for (int64_t kk = 0; kk < N; ++kk) {
            if (nodextr[kk] != k || nin[kk] <= 0 || kk >= np) continue;
            const int64_t e = tri_index64(np, n < kk ? n : kk, n < kk ? kk : n);
            if (fmt == 1) {
                const float w = casewise ? (float)nin[kk] / (float)nodesize : 1.0f;
                uint16_t* o = (uint16_t*)out;
                o[e] = orc_f32_to_f16(orc_f16_to_f32(o[e]) + w);
            } else if (fmt == 3) {
                const float w = casewise ? (float)nin[kk] / (float)nodesize : 1.0f;
                uint8_t* o = (uint8_t*)out;
                const int sh = (int)(e & 1) * 4;
                const uint8_t old = (uint8_t)((o[e >> 1] >> sh) & 0xf);
                const uint8_t nw = (uint8_t)(orc_q_nf4(orc_nf4_to_f32(old) + w) & 0xf);
                o[e >> 1] = (uint8_t)((o[e >> 1] & ~(0xf << sh)) | (nw << sh));
            } else {
                const float w = (float)nin[kk] / (float)nodesize;
                int8_t* o = (int8_t*)out;
                o[e] = (int8_t)(uint8_t)((uint8_t)o[e] + (uint8_t)orc_q_i8(w, scale, zp));
            }
        }
    }
}

void orc_rfgap_tree_upper(const int32_t* nin, const int32_t* nodextr, int32_t nsample, int32_t n_real,
                          uint16_t* out) {
    const int64_t N = nsample;
    const int64_t np = (n_real > 0 && n_real < nsample) ? n_real : nsample;
    memset(out, 0, sizeof(uint16_t) * (size_t)(np * (np + 1) / 2));
    for (int64_t i = 0; i < np; ++i) {
        if (nin[i] != 0) continue;
        const int32_t node = nodextr[i];
        if (node < 0) continue;
        int32_t mult = 0;
        for (int64_t j = 0; j < N; ++j)
            if (nin[j] > 0 && nodextr[j] == node) mult += nin[j];
        if (mult == 0) continue;
        const float inv = 1.0f / (float)mult;
        for (int64_t j = i; j < np; ++j) {
            if (!(nin[j] > 0 && nodextr[j] == node)) continue;
            const int64_t e = tri_index64(np, i, j);
            out[e] = orc_f32_to_f16(orc_f16_to_f32(out[e]) + (float)nin[j] * inv);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* a5: QuantizationDispatcher::launch_proximity_kernel,                       */
/* cuda/rf_quantization_kernels.cu:195-355 (one launch)                      */
/* ------------------------------------------------------------------------ */
void orc_dispatch_prox(int level, const int32_t* nodexb, const int32_t* nin, int32_t nsample,
                       const int32_t* ndbegin, const int32_t* npcase, void* out) {
    /* every sample n with a terminal ordinal k = nodexb[n] >= 0: nodesize =
     * sum of nin over the in-bag members of k (first pass, :207-213); then
     * each in-bag member kk with n <= kk adds its weight at n + kk*N
     * (second pass, :216-227).  The reference adds through type-punned
     * 32-bit atomics; the entries here take the width of the level. */
    const int64_t N = nsample;
    for (int64_t n = 0; n < N; ++n) {
        const int32_t k = nodexb[n];
        if (k < 0) continue;
        int32_t nsz = 0;
        for (int32_t j = ndbegin[k]; j < ndbegin[k + 1]; ++j)
            if (nin[npcase[j]] > 0) nsz += nin[npcase[j]];
        if (nsz <= 0) continue;
        for (int32_t j = ndbegin[k]; j < ndbegin[k + 1]; ++j) {
            const int32_t kk = npcase[j];
            if (nin[kk] <= 0 || n > kk) continue;
            const int64_t e = n + (int64_t)kk * N;
            if (level == 0) {          /* FP32: double weight (:236-270) */
                ((double*)out)[e] += (double)nin[kk] / (double)nsz;
            } else if (level == 1) {   /* FP16: half(weight) (:195-231) */
                uint16_t* o = (uint16_t*)out;
                const float w = orc_f16_to_f32(orc_f32_to_f16((float)nin[kk] / (float)nsz));
                o[e] = orc_f32_to_f16(orc_f16_to_f32(o[e]) + w);
            } else if (level == 2) {   /* INT8: fp32_to_int8(w, 1/127, 0) (:273-310, dispatcher :372-378) */
                uint8_t* o = (uint8_t*)out;
                o[e] = (uint8_t)(o[e] + (uint8_t)orc_q_i8((float)nin[kk] / (float)nsz, 1.0f / 127.0f, 0.0f));
            } else {                   /* NF4: one byte per entry, + fp32_to_nf4(w) (:313-355) */
                uint8_t* o = (uint8_t*)out;
                o[e] = (uint8_t)(o[e] + orc_q_nf4((float)nin[kk] / (float)nsz));
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* a8: compute_proximity_from_leaves, src/rf_random_forest.cpp:4605-4642     */
/* ------------------------------------------------------------------------ */
float orc_pair_proximity(const int32_t* leaf, const uint8_t* oob, int64_t N, int32_t T, int32_t nleaf, int64_t i,
                         int64_t j) {
    if (i < 0 || i >= N || j < 0 || j >= N) return 0.0f;            /* :4610-4613 */
    int32_t matches = 0, noob = 0;
    for (int32_t t = 0; t < T; ++t) {                                /* oob_trees_[i], ascending */
        if (!oob[(int64_t)t * N + i]) continue;
        ++noob;
        const int32_t li = leaf[(int64_t)t * N + i], lj = leaf[(int64_t)t * N + j];
        if (li == lj && li >= 0 && li < nleaf) ++matches;            /* :4628-4636 */
    }
    if (noob == 0) return 0.0f;                                      /* :4619-4621 */
    return (float)matches / (float)noob;                             /* :4641 */
}

/* ------------------------------------------------------------------------ */
/* f2: outlier scores, src/rf_random_forest.cpp:4100-4273                    */
/* ------------------------------------------------------------------------ */
void orc_outlier_raw(const int32_t* ref_leaf, int64_t N, int32_t T, int32_t nleaf, const int32_t* qleaf, int64_t Q,
                     const int32_t* exclude, float numerator, float isolated, float* raw_out, int threads) {
    const int nth = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel num_threads(nth)
    {
        uint16_t* cnt = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(N > 0 ? N : 1));
#pragma omp for schedule(dynamic, 4)
        for (int64_t q = 0; q < Q; ++q) {
            memset(cnt, 0, sizeof(uint16_t) * (size_t)N);
            for (int32_t t = 0; t < T; ++t) {   /* the query's leaf members in every tree (:4167-4178) */
                const int32_t ql = qleaf[q * T + t];
                if (ql < 0 || ql >= nleaf) continue;
                const int32_t* rl = ref_leaf + (int64_t)t * N;
                for (int64_t j = 0; j < N; ++j) cnt[j] += (uint16_t)(rl[j] == ql);
            }
            const int64_t ex = exclude ? exclude[q] : -1;
            double s = 0.0;                     /* prox = count / ntree, squared, summed (:4179-4183) */
            for (int64_t j = 0; j < N; ++j) {
                if (j == ex || cnt[j] == 0) continue;
                const float p = (float)cnt[j] / (float)T;
                s += (double)(p * p);
            }
            const float sq = (float)s;
            raw_out[q] = sq > 1e-10f ? numerator / sq : isolated; /* :4184-4188 */
        }
        free(cnt);
    }
}

static int cmp_f32(const void* a, const void* b) {
    const float x = *(const float*)a, y = *(const float*)b;
    return (x > y) - (x < y);
}

void orc_outlier_normalize(const float* raw, int64_t N, const int32_t* classes, float* scores) {
    /* groups: ascending class values (std::map order, :4198-4203), or all */
    int32_t* keys = (int32_t*)malloc(sizeof(int32_t) * (size_t)N);
    int64_t ng = 0;
    if (classes) {
        for (int64_t n = 0; n < N; ++n) {
            int found = 0;
            for (int64_t g = 0; g < ng; ++g) found |= keys[g] == classes[n];
            if (!found) keys[ng++] = classes[n];
        }
        /* insertion sort of the class keys */
        for (int64_t a = 1; a < ng; ++a)
            for (int64_t b = a; b > 0 && keys[b - 1] > keys[b]; --b) {
                const int32_t t = keys[b];
                keys[b] = keys[b - 1];
                keys[b - 1] = t;
            }
    } else {
        ng = 1;
    }
    float* v = (float*)malloc(sizeof(float) * (size_t)N);
    float* d = (float*)malloc(sizeof(float) * (size_t)N);
    for (int64_t g = 0; g < ng; ++g) {
        int64_t m = 0;
        for (int64_t n = 0; n < N; ++n)
            if (!classes || classes[n] == keys[g]) v[m++] = raw[n];
        qsort(v, (size_t)m, sizeof(float), cmp_f32);
        const float median = v[m / 2];                             /* :4218-4219, :4249-4250 */
        int64_t k = 0;
        for (int64_t n = 0; n < N; ++n)
            if (!classes || classes[n] == keys[g]) d[k++] = fabsf(raw[n] - median);
        qsort(d, (size_t)m, sizeof(float), cmp_f32);
        float mad = d[m / 2];                                      /* :4221-4228 */
        if (mad < 1e-10f) mad = 1.0f;
        for (int64_t n = 0; n < N; ++n)
            if (!classes || classes[n] == keys[g]) scores[n] = (raw[n] - median) / mad;
    }
    free(v);
    free(d);
    free(keys);
}

/* ------------------------------------------------------------------------ */
/* f1: leaf assignments on a forest (tree walks)                             */
/* ------------------------------------------------------------------------ */
typedef struct {
    const int32_t *ns, *bv, *tm, *cg, *cat;
    const float* sp;
    int32_t maxnode, maxcat, mdim;
} orc_tree;

/* (int)(f + 0.5) with f + 0.5 in double; values whose truncation leaves
 * int32 give -1 (an invalid category) */
static int32_t orc_round_cat(float f) {
    const double d = (double)f + 0.5;
    if (!(d > -2147483649.0 && d < 2147483648.0)) return -1;
    return (int32_t)d;
}
static int32_t orc_trunc_cat(float f) {
    if (!(f > -2147483649.0f && f < 2147483648.0f)) return -1;
    return (int32_t)f;
}
static int orc_node_ok(const orc_tree* t, int32_t k) { return k >= 0 && k < t->maxnode; }

/* predict_leaf_assignments, src/rf_random_forest.cpp:4800-4845 */
static int32_t orc_walk_predict(const orc_tree* t, const float* x) {
    int32_t cur = 0;
    for (int32_t k = 0; k < t->maxnode; ++k) {
        if (t->ns[cur] == -1) break;
        const int32_t v = t->bv[cur];
        int32_t nxt = cur;
        if (v >= 0 && v < t->mdim) {
            const float f = x[v];
            const int32_t c = t->cat ? t->cat[v] : 1;
            if (c == 1) {
                nxt = f <= t->sp[cur] ? t->tm[2 * cur] : t->tm[2 * cur + 1];
            } else {
                const int32_t j = orc_round_cat(f);
                if (j >= 0 && j < c && j < t->maxcat)
                    nxt = t->cg[cur * t->maxcat + j] == 1 ? t->tm[2 * cur] : t->tm[2 * cur + 1];
            }
        }
        if (!orc_node_ok(t, nxt)) break; /* a child outside the tree ends the walk */
        cur = nxt;
    }
    return cur;
}

/* RandomForest::find_terminal_node, src/rf_random_forest.cpp:3724-3774 */
static int32_t orc_walk_inbag(const orc_tree* t, const float* x) {
    int32_t cur = 0;
    for (int32_t k = 0; k < t->maxnode; ++k) {
        if (t->ns[cur] == -1) return cur;
        const int32_t v = t->bv[cur];
        if (!(v >= 0 && v < t->mdim)) return 0;
        const float f = x[v];
        const int32_t c = t->cat ? t->cat[v] : 1;
        int32_t nxt;
        if (c == 1) {
            nxt = f <= t->sp[cur] ? t->tm[2 * cur] : t->tm[2 * cur + 1];
        } else {
            const int32_t j = orc_round_cat(f);
            if (!(j >= 0 && j < c && j < t->maxcat)) return 0;
            nxt = t->cg[cur * t->maxcat + j] == 1 ? t->tm[2 * cur] : t->tm[2 * cur + 1];
        }
        if (!orc_node_ok(t, nxt)) return 0;
        cur = nxt;
    }
    return 0;
}

/* cpu_testreebag's walk of an OOB sample, src/rf_testreebag.cpp:43-119 */
static int32_t orc_walk_oob(const orc_tree* t, const float* x) {
    int32_t kt = 0, count = 0;
    while (t->ns[kt] == 1 && count < 1000) {
        count++;
        const int32_t mvar = t->bv[kt];
        if (!(mvar >= 0 && mvar < t->mdim)) break; /* (the reference reads outside x here) */
        int32_t nxt;
        if (!t->cat || t->cat[mvar] <= 2) {
            nxt = x[mvar] <= t->sp[kt] ? t->tm[2 * kt] : t->tm[2 * kt + 1];
        } else {
            const int32_t cv = orc_trunc_cat(x[mvar]);
            if (cv >= 0 && cv < t->cat[mvar] && cv < t->maxcat)
                nxt = t->cg[cv + kt * t->maxcat] == 1 ? t->tm[2 * kt] : t->tm[2 * kt + 1];
            else nxt = t->tm[2 * kt + 1];
        }
        if (!orc_node_ok(t, nxt)) break;
        kt = nxt;
        if (t->ns[kt] != 1) break;
    }
    return (t->ns[kt] == -1 || t->ns[kt] == 2) ? kt : 0;
}

void orc_forest_leaves(int mode, const int32_t* nodestatus, const int32_t* bestvar, const float* xbestsplit,
                       const int32_t* treemap, const int32_t* catgoleft, const int32_t* cat, int32_t T, int32_t maxnode,
                       int32_t maxcat, int32_t mdim, const float* X, int64_t N, const int32_t* nin, int32_t* leaf_out) {
#pragma omp parallel for schedule(static)
    for (int32_t tr = 0; tr < T; ++tr) {
        orc_tree t;
        t.ns = nodestatus + (int64_t)tr * maxnode;
        t.bv = bestvar + (int64_t)tr * maxnode;
        t.sp = xbestsplit + (int64_t)tr * maxnode;
        t.tm = treemap + (int64_t)tr * maxnode * 2;
        t.cg = catgoleft ? catgoleft + (int64_t)tr * maxnode * maxcat : NULL;
        t.cat = cat;
        t.maxnode = maxnode;
        t.maxcat = maxcat;
        t.mdim = mdim;
        for (int64_t n = 0; n < N; ++n) {
            const float* x = X + n * mdim;
            int32_t leaf;
            if (mode == 0) leaf = orc_walk_predict(&t, x);
            else leaf = nin[(int64_t)tr * N + n] == 0 ? orc_walk_oob(&t, x) : orc_walk_inbag(&t, x);
            leaf_out[(int64_t)tr * N + n] = leaf;
        }
    }
}
