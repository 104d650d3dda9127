// Device-side building blocks shared by the proximity kernels (gfx950).
//
// Numerics: every function here performs the same IEEE operations, in the
// same order, as the reference CPU path it cites.  The translation units
// that include this header are compiled with -ffp-contract=off and with
// correctly rounded fp32 division, so no multiply-add is fused and no
// division is replaced by a reciprocal.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rfxp {

// Output formats of the packed triangle (values of RFXP_FMT_* in rfx_prox.h).
enum Fmt : int { F32 = 0, F16 = 1, I8 = 2, NF4 = 3, U8 = 4, U16 = 5 };

// Row-wise packed upper triangle with the diagonal, 64-bit
// (cuda/rf_proximity_upper_triangle.cu:34-39 uses int32, which overflows
// beyond N ~ 65k).
__host__ __device__ __forceinline__ int64_t tri_idx(int64_t n, int64_t i, int64_t j) {
    return i * n - i * (i + 1) / 2 + j;
}

// Reciprocal used by the row normalisation of src/rf_finishprox.cpp:47-55:
// rows with nout == 0 are left unscaled, which is a multiply by exactly 1.0.
__host__ __device__ __forceinline__ double nout_recip(int32_t n) {
    return n > 0 ? 1.0 / (double)n : 1.0;
}

// Normalised proximity of an off-diagonal pair with co-occurrence count U:
// s = (c_ij + c_ji)/2 (src/rf_finishprox.cpp:38), a = s / n_i and
// b = s / n_j as multiplies by the reciprocals (:49-52), P = 0.5 (a + b)
// (:69).  ri, rj come from nout_recip().
__device__ __forceinline__ double pair_p(uint32_t U, double ri, double rj) {
    double s = (double)U / 2.0;
    double a = s * ri;
    double b = s * rj;
    return 0.5 * (a + b);
}

// include/rf_quantization_kernels.hpp:24-29 (fp32_to_int8).
__device__ __forceinline__ int8_t q_i8(float v, float scale, float zp) {
    float r = v / scale + zp;
    r = fmaxf(-128.0f, fminf(127.0f, r));
    return (int8_t)r;
}

// Unsigned 8-bit code of a normalised proximity: the reference's affine
// rule (value / scale + zero_point, truncated) clamped to [0, 255].
__device__ __forceinline__ uint8_t q_u8(float v, float scale, float zp) {
    float r = v / scale + zp;
    r = fmaxf(0.0f, fminf(255.0f, r));
    return (uint8_t)r;
}

// include/rf_quantization_kernels.hpp:37-50 (fp32_to_nf4, a linear 4-bit code).
__device__ __forceinline__ uint8_t q_nf4(float v) {
    if (v >= 0.0f) return (uint8_t)fminf(7.0f, roundf(v * 7.0f));
    return (uint8_t)fmaxf(8.0f, roundf(8.0f - v * 7.0f));
}

// IEEE binary16 bits of v, round to nearest even.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
    _Float16 h = (_Float16)v;
    return __builtin_bit_cast(uint16_t, h);
}

// One-byte code of P in format F (I8, U8, NF4 nibble); the integer formats
// that the epilogue table-drives.
template <int F>
__device__ __forceinline__ uint32_t code_of(double P, float scale, float zp) {
    float pf = (float)P;
    if constexpr (F == I8) return (uint32_t)(uint8_t)q_i8(pf, scale, zp);
    else if constexpr (F == U8) return (uint32_t)q_u8(pf, scale, zp);
    else return (uint32_t)(q_nf4(pf) & 0xfu);
}

}  // namespace rfxp
