// rfx_compat.hpp -- the reference's C++ entry points of the proximity path,
// with their original signatures, as exported by librfxprox.so.
//
// A program built against RFX-Fuse's own headers (include/rf_proximity.hpp,
// rf_finishprox.hpp, rf_proximity_upper_triangle.hpp,
// rf_quantization_kernels.hpp) links these definitions unchanged; this
// header declares the same functions for code built without those headers.
// The low-rank class (rf_proximity_lowrank.hpp) keeps its public interface
// but not the reference's private members, so its callers compile against
// this header; the helpers of rf_lowrank_helpers.hpp are declared here too.
// The declarations follow the reference's (file:line at each group); the
// definitions run on the GPU through the C ABI of rfx_prox.h.
//
// Conventions kept from the reference: void functions, caller-allocated
// outputs, column-major N x N double matrices, device 0 and the null
// stream.  A failure (no HIP device, bad arguments) leaves the output as it
// was, prints one line to stderr and is readable with rfx_compat_last_error;
// nothing falls back to a CPU implementation.
#ifndef RFX_COMPAT_HPP
#define RFX_COMPAT_HPP

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <vector>

// Settings the reference reads from its global configuration
// (include/rf_config.hpp:62, :106): case-wise weights and the number of real
// samples (> 0: only the first n_real samples form the triangle outputs).
extern "C" void rfx_compat_configure(int use_casewise, int32_t n_real_samples);
// Message of the last failure of a compat function on this thread ("" if none).
extern "C" const char* rfx_compat_last_error(void);

#ifndef RF_TYPES_HPP
namespace rf {
using integer_t = int32_t;  // include/rf_types.hpp:15-19
using dp_t = double;
using real_t = float;
}  // namespace rf
#endif

namespace rf {

// include/rf_proximity.hpp:10-21: one tree, accumulating
// prox[n + kk*nsample] += w for OOB n and in-bag kk of a terminal node.
// The workspace arguments are accepted and not used.
void cpu_proximity(const integer_t* nodestatus, const integer_t* nodextr, const integer_t* nin, integer_t nsample,
                   integer_t nnode, dp_t* prox, integer_t* nod, integer_t* ncount, integer_t* ncn, integer_t* nodexb,
                   integer_t* ndbegin, integer_t* npcase);
void gpu_proximity(const integer_t* nodestatus, const integer_t* nodextr, const integer_t* nin, integer_t nsample,
                   integer_t nnode, dp_t* prox, integer_t* nod, integer_t* ncount, integer_t* ncn, integer_t* nodexb,
                   integer_t* ndbegin, integer_t* npcase);

// include/rf_proximity.hpp:34-46: RF-GAP proximity, N x N, symmetrised.
void cpu_proximity_rfgap(integer_t ntree, integer_t nsample, const std::vector<std::vector<integer_t>>& tree_nin,
                         const std::vector<std::vector<integer_t>>& tree_nodextr, dp_t* prox);
void gpu_proximity_rfgap(integer_t ntree, integer_t nsample, const integer_t* tree_nin_flat,
                         const integer_t* tree_nodextr_flat, dp_t* prox);

// include/rf_finishprox.hpp:9-12
void cpu_finishprox(integer_t nsample, const integer_t* nout, dp_t* prox, dp_t* proxsym);
void gpu_finishprox(integer_t nsample, const integer_t* nout, dp_t* prox, dp_t* proxsym);

namespace cuda {

#ifndef RF_QUANTIZATION_KERNELS_HPP
// include/rf_quantization_kernels.hpp:13-18
enum class QuantizationLevel { FP32 = 0, FP16 = 1, INT8 = 2, NF4 = 3 };

// include/rf_quantization_kernels.hpp:21-66: the converters (same
// formulas) and the two scaling helpers.
class QuantizationUtils {
   public:
    static __device__ __forceinline__ int8_t fp32_to_int8(float value, float scale, float zero_point) {
        float r = value / scale + zero_point;
        r = fmaxf(-128.0f, fminf(127.0f, r));
        return static_cast<int8_t>(r);
    }
    static __device__ __forceinline__ float int8_to_fp32(int8_t value, float scale, float zero_point) {
        return (static_cast<float>(value) - zero_point) * scale;
    }
    static __device__ __forceinline__ uint8_t fp32_to_nf4(float value) {
        if (value >= 0.0f) return static_cast<uint8_t>(fminf(7.0f, roundf(value * 7.0f)));
        return static_cast<uint8_t>(fmaxf(8.0f, roundf(8.0f - value * 7.0f)));
    }
    static __device__ __forceinline__ float nf4_to_fp32(uint8_t value) {
        if (value <= 7) return static_cast<float>(value) / 7.0f;
        return -(static_cast<float>(value - 8)) / 7.0f;
    }
    // scale = (max - min) / 255, zero_point = -min / scale over host data
    static void compute_int8_scaling(const float* data, size_t count, float& scale, float& zero_point);
    // the same over device doubles (as floats), results left in device memory;
    // scale 1/127 when (max - min)/255 < 1e-10, and (1/127, 127) for count 0
    static void compute_int8_scaling_gpu(const dp_t* data_gpu, size_t count, float* d_scale, float* d_zero_point);
};

// include/rf_quantization_kernels.hpp:69-107: per-tree dense kernels over a
// node CSR (nodexb: terminal ordinal per sample, ndbegin/npcase: members),
// entry (n, kk) of an N x N column-major matrix for n <= kk, weight
// nin[kk] / nodesize.
__global__ void cuda_proximity_fp16_kernel(const integer_t* nodexb, const integer_t* nin, integer_t nsample,
                                           const integer_t* ndbegin, const integer_t* npcase, __half* prox_fp16);
__global__ void cuda_proximity_kernel(const integer_t* nodexb, const integer_t* nin, integer_t nsample,
                                      const integer_t* ndbegin, const integer_t* npcase, dp_t* prox);
__global__ void cuda_proximity_int8_kernel(const integer_t* nodexb, const integer_t* nin, integer_t nsample,
                                           const integer_t* ndbegin, const integer_t* npcase, int8_t* prox_int8,
                                           float scale, float zero_point);
__global__ void cuda_proximity_nf4_kernel(const integer_t* nodexb, const integer_t* nin, integer_t nsample,
                                          const integer_t* ndbegin, const integer_t* npcase, uint8_t* prox_nf4);

// include/rf_quantization_kernels.hpp:110-121
class QuantizationDispatcher {
   public:
    static void launch_proximity_kernel(QuantizationLevel level, const integer_t* nodexb, const integer_t* nin,
                                        integer_t nsample, const integer_t* ndbegin, const integer_t* npcase,
                                        void* prox_data, int blocks, int threads);
    static size_t get_quantized_size(QuantizationLevel level, size_t base_size);
};
#endif

// include/rf_proximity_upper_triangle.hpp:42-156: one tree's packed upper
// triangle (zeroed first).  FP16 needs a device output; INT8 and NF4 take
// host or device outputs.
void gpu_proximity_upper_triangle_fp16(const integer_t* nodestatus, const integer_t* nodextr, const integer_t* nin,
                                       integer_t nsample, integer_t nnode, __half* prox_upper_fp16, integer_t* nod,
                                       integer_t* ncount, integer_t* ncn, integer_t* nodexb, integer_t* ndbegin,
                                       integer_t* npcase);
void gpu_proximity_upper_triangle_int8(const integer_t* nodestatus, const integer_t* nodextr, const integer_t* nin,
                                       integer_t nsample, integer_t nnode, int8_t* prox_upper_int8, float scale,
                                       float zero_point, integer_t* nod, integer_t* ncount, integer_t* ncn,
                                       integer_t* nodexb, integer_t* ndbegin, integer_t* npcase);
void gpu_proximity_upper_triangle_nf4(const integer_t* nodestatus, const integer_t* nodextr, const integer_t* nin,
                                      integer_t nsample, integer_t nnode, uint8_t* prox_upper_nf4, integer_t* nod,
                                      integer_t* ncount, integer_t* ncn, integer_t* nodexb, integer_t* ndbegin,
                                      integer_t* npcase);
void gpu_proximity_upper_triangle(const integer_t* nodestatus, const integer_t* nodextr, const integer_t* nin,
                                  integer_t nsample, integer_t nnode, QuantizationLevel quant_level,
                                  void* prox_upper_output, integer_t* nod, integer_t* ncount, integer_t* ncn,
                                  integer_t* nodexb, integer_t* ndbegin, integer_t* npcase);

// include/rf_proximity_upper_triangle.hpp:177-182: one tree's RF-GAP
// contributions as an FP16 triangle (host output).
void gpu_proximity_rfgap_upper_triangle_fp16(const integer_t* nin_tree, const integer_t* nodextr_tree,
                                             integer_t nsample, __half* prox_upper_fp16);

// The reference's include guards: whichever of this header and the
// reference's rf_proximity_lowrank.hpp / rf_lowrank_helpers.hpp comes first
// provides the declarations.  Code that creates the object must see this
// declaration (its private layout is the library's), so such code includes
// this header first, or the reference header is reduced to an include of it.
#ifndef RF_PROXIMITY_LOWRANK_HPP
#define RF_PROXIMITY_LOWRANK_HPP
// include/rf_proximity_lowrank.hpp:27-433: the low-rank proximity object.
// Public interface as the reference's; the private state is this build's.
// Contributions (per-tree packed triangles in FP16 / INT8 / NF4, FP32 read
// as FP16 as the reference does, or dense N x N doubles) are accumulated
// exactly as a sparse symmetric matrix M on the device; the factor A (N x
// rank, column-major double, B = A) is the rank-`rank` positive part of M
// from block subspace iteration with power_iterations products
// (rfxp_symacc_factor), computed when first needed after new
// contributions.  With final_call, finalize_accumulation stores the factors
// at the object's quantization level (FP16 / INT8 / NF4); get_factors then
// returns their dequantised values, as the reference's does.
class LowRankProximityMatrix {
   public:
    LowRankProximityMatrix(integer_t nsample, integer_t initial_rank = 100,
                           QuantizationLevel quant_level = QuantizationLevel::FP16, integer_t max_rank = 1000,
                           integer_t power_iterations = 30);
    ~LowRankProximityMatrix();
    LowRankProximityMatrix(const LowRankProximityMatrix&) = delete;
    LowRankProximityMatrix& operator=(const LowRankProximityMatrix&) = delete;

    // false when no HIP device can be used (the reference always says true)
    bool initialize();
    void add_tree_contribution(const dp_t* tree_proximity, integer_t nsample, bool use_incremental = false);
    void add_tree_contribution_incremental(const dp_t* tree_proximity, integer_t nsample);
    void add_tree_contribution_incremental_upper_triangle(const void* tree_proximity_upper, integer_t nsample,
                                                          QuantizationLevel quant_level,
                                                          float int8_scale = 1.0f / 127.0f,
                                                          float int8_zero_point = 0.0f);
    void add_tree_contribution_incremental_upper_triangle_fp16(const __half* tree_proximity_upper_fp16,
                                                               integer_t nsample);
    void finalize_accumulation(integer_t n_trees_processed = 0, bool final_call = false);
    void get_accumulated_proximity(dp_t* output_prox, integer_t nsample);
    void reconstruct_full_matrix(dp_t* output_prox, integer_t nsample,
                                 QuantizationLevel quant_level = QuantizationLevel::FP32);
    void quantize_factors(QuantizationLevel quant_level);
    void dequantize_factors();
    bool is_quantized() const { return current_quant_level_ != QuantizationLevel::FP32; }
    QuantizationLevel get_quantization_level() const { return current_quant_level_; }
    void get_factors(dp_t** A_gpu, dp_t** B_gpu, integer_t* rank);
    void compute_distances_from_factors(dp_t* output_distances, integer_t nsample);
    void set_oob_counts_for_rfgap(const integer_t* oob_counts);
    std::vector<double> compute_mds_from_factors(integer_t k = 3);
    std::vector<double> compute_mds_3d_from_factors() { return compute_mds_from_factors(3); }
    integer_t auto_adjust_rank(double target_variance = 0.95);
    size_t get_memory_usage() const;
    size_t get_memory_usage(QuantizationLevel quant_level) const;
    static bool should_use_incremental(integer_t nsample, size_t available_memory = 0);

    struct State;  // opaque: the library's device state of the object

   private:
    State* st_;
    integer_t nsample_;
    integer_t rank_;
    integer_t max_rank_;
    integer_t power_iterations_;
    QuantizationLevel current_quant_level_;
};

// include/rf_proximity_lowrank.hpp:433: min(max_rank, floor(sqrt(nsample))), at least 1
integer_t estimate_optimal_rank(integer_t nsample, integer_t max_rank = 1000);
#endif  // RF_PROXIMITY_LOWRANK_HPP

#ifndef RF_LOWRANK_HELPERS_HPP
#define RF_LOWRANK_HELPERS_HPP

// include/rf_lowrank_helpers.hpp:13-34 (lowrank_proximity_ptr is a
// LowRankProximityMatrix*): host copies of the factors (new[], the caller
// deletes), MDS coordinates (empty on failure), and the reconstructed
// N x N matrix (new[], refused above 50000 samples).
bool get_lowrank_factors_host(void* lowrank_proximity_ptr, dp_t** A_host, dp_t** B_host, integer_t* rank,
                              integer_t nsamples);
std::vector<double> compute_mds_from_factors_host(void* lowrank_proximity_ptr, integer_t k);
inline std::vector<double> compute_mds_3d_from_factors_host(void* lowrank_proximity_ptr) {
    return compute_mds_from_factors_host(lowrank_proximity_ptr, 3);
}
bool reconstruct_proximity_matrix_host(void* lowrank_proximity_ptr, dp_t** output_prox, integer_t nsamples);
#endif  // RF_LOWRANK_HELPERS_HPP

}  // namespace cuda
}  // namespace rf

#endif  // RFX_COMPAT_HPP
