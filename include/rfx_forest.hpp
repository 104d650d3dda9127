// rfx_forest.hpp -- the proximity queries of RFX-Fuse's RandomForest object
// (src/rf_random_forest.cpp, python/randomforest_py.cpp) as one object over
// the forest's own state, run on the GPU through librfxprox's C ABI.
//
// RandomForest keeps leaf_assignments_ (int16, tree-major [t*N + i]) and
// oob_trees_ (per sample, the trees where it is out-of-bag).  A
// ForestProximity built from them answers the same questions as the methods
// named below, with their argument meaning and results; RandomForest and the
// Python binding forward to it without changing their signatures (each
// method's body becomes one call on a ForestProximity member).  Leaf labels
// are compared as node indices; a negative label never matches (the
// reference's labels are node indices >= 0).  Top-K ties are broken by the
// lower index.
// Failures print one line to stderr and are readable with
// rfx_compat_last_error(); results are then empty / false.
#ifndef RFX_FOREST_HPP
#define RFX_FOREST_HPP

#include <stdint.h>

#include <utility>
#include <vector>

namespace rfx {

class ForestProximity {
   public:
    // leaf_assignments: host int16 [t*nsample + i]; oob_trees: host, one tree
    // list per sample (RandomForest::oob_trees_).  The data are copied.
    ForestProximity(const int16_t* leaf_assignments, int32_t nsample, int32_t ntree,
                    const std::vector<std::vector<int32_t>>& oob_trees, int device = 0);
    ~ForestProximity();
    ForestProximity(const ForestProximity&) = delete;
    ForestProximity& operator=(const ForestProximity&) = delete;

    bool ok() const;  // the forest reached the device

    // RandomForest::compute_proximity_from_leaves (src/rf_random_forest.cpp:4605-4642)
    float compute_proximity_from_leaves(int32_t sample_i, int32_t sample_j) const;
    // RandomForest::get_top_k_similar (src/rf_random_forest.cpp:4677-4782): at most
    // k (<= 64) samples with counts > 0 over the query's OOB trees, with
    // (float)count * (1.0f / |OOB(query)|)
    std::vector<std::pair<int32_t, float>> get_top_k_similar(int32_t query_idx, int32_t k,
                                                             bool exclude_self = true) const;
    // predict_top_k_similar (python/randomforest_py.cpp:2496-2568): for nq new
    // samples (new_leaves [q*ntree + t], predict_leaf_assignments' layout) the k
    // (<= 64) most similar training samples over all trees, zeros included, into
    // idx_out / score_out [q*k + c] (score = count / ntree)
    bool predict_top_k_similar(const int16_t* new_leaves, int32_t nq, int32_t k, int32_t* idx_out,
                               float* score_out) const;
    // get_proximity_matrix (python/randomforest_py.cpp:2129-2150): the N x N
    // float32 matrix of cpu_finishprox over the OOB co-occurrence counts
    // (src/rf_proximity.cpp:99-231, src/rf_finishprox.cpp:12-74), nout =
    // |oob_trees[i]|, into host `out` (symmetric, so row- or column-major)
    bool get_proximity_matrix(float* out) const;
    // RandomForest::compute_outlier_scores, full mode (src/rf_random_forest.cpp:4100-4273);
    // classes (host int32[N]) or NULL
    std::vector<float> compute_outlier_scores(const int32_t* classes = nullptr) const;

    struct Impl;  // opaque

   private:
    Impl* p_;
};

}  // namespace rfx

#endif  // RFX_FOREST_HPP
