// Test infrastructure only: a C shim over the reference's own CPU proximity
// sources, compiled in place from /root/reference (src/rf_proximity.cpp,
// src/rf_finishprox.cpp, src/rf_config.cpp) into oracle/_ref/libref.so.
// It is used to generate and check golden fixtures in the build container;
// nothing in the product links it, and it never runs on the GPU box.
//
// Entry points wrapped (reference declarations):
//   rf::cpu_proximity        include/rf_proximity.hpp:10-14
//   rf::cpu_proximity_rfgap  include/rf_proximity.hpp:34-38
//   rf::cpu_finishprox       include/rf_finishprox.hpp:9
//   rf::cpu_testreebag       include/rf_testreebag.hpp:9-15
//   rf::g_config             include/rf_config.hpp:156 (fields use_casewise,
//                            use_sparse, n_threads_cpu)
#include <cstdint>
#include <vector>

#include "rf_config.hpp"
#include "rf_finishprox.hpp"
#include "rf_proximity.hpp"
#include "rf_testreebag.hpp"

extern "C" {

void ref_set_config(int use_casewise, int use_sparse, int n_threads_cpu) {
    rf::g_config.use_casewise = use_casewise != 0;
    rf::g_config.use_sparse = use_sparse != 0;
    rf::g_config.n_threads_cpu = n_threads_cpu;
}

// One tree: accumulates into the column-major nsample x nsample double matrix.
// Workspaces are sized as the forest sizes them (src/rf_random_forest.cpp:1959-1967).
void ref_cpu_proximity(const int32_t* nodestatus, const int32_t* nodextr, const int32_t* nin,
                       int32_t nsample, int32_t nnode, double* prox) {
    std::vector<int32_t> nod(nnode > 0 ? nnode : 1), ncount(nsample), ncn(nsample), nodexb(nsample),
        ndbegin(nnode + 2), npcase(nsample);
    rf::cpu_proximity(nodestatus, nodextr, nin, nsample, nnode, prox, nod.data(), ncount.data(),
                      ncn.data(), nodexb.data(), ndbegin.data(), npcase.data());
}

void ref_cpu_finishprox(int32_t nsample, const int32_t* nout, double* prox, double* proxsym) {
    rf::cpu_finishprox(nsample, nout, prox, proxsym);
}

// nin_flat / nodextr_flat are tree-major [t * nsample + i].
void ref_cpu_proximity_rfgap(int32_t ntree, int32_t nsample, const int32_t* nin_flat,
                             const int32_t* nodextr_flat, double* prox) {
    std::vector<std::vector<int32_t>> nin(ntree), ndx(ntree);
    for (int32_t t = 0; t < ntree; ++t) {
        nin[t].assign(nin_flat + (size_t)t * nsample, nin_flat + (size_t)(t + 1) * nsample);
        ndx[t].assign(nodextr_flat + (size_t)t * nsample, nodextr_flat + (size_t)(t + 1) * nsample);
    }
    rf::cpu_proximity_rfgap(ntree, nsample, nin, ndx, prox);
}

// One tree: nodextr of the OOB samples (0 for the others), x row-major N x mdim.
void ref_cpu_testreebag(const float* x, const float* xbestsplit, const int32_t* nin, const int32_t* treemap,
                        const int32_t* bestvar, const int32_t* cat, const int32_t* nodestatus, const int32_t* catgoleft,
                        int32_t nsample, int32_t mdim, int32_t nnode, int32_t maxcat, int32_t* nodextr) {
    std::vector<int32_t> nodeclass(nnode > 0 ? nnode : 1, 0), jtr(nsample > 0 ? nsample : 1);
    rf::cpu_testreebag(x, xbestsplit, nin, treemap, bestvar, nodeclass.data(), cat, nodestatus, catgoleft, nsample,
                       mdim, nnode, maxcat, jtr.data(), nodextr);
}

}  // extern "C"
