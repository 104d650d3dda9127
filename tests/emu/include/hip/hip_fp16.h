// Host-side stand-in for <hip/hip_fp16.h> (CPU emulation build only, see
// hip_runtime.h in this directory): binary16 through _Float16, whose
// conversions round to nearest even as the GPU's do.
#pragma once
#include <stdint.h>
#include <string.h>

struct __half {
    _Float16 v;
};
inline __half __float2half(float f) { return __half{(_Float16)f}; }
inline float __half2float(__half h) { return (float)h.v; }
inline uint16_t __half_as_ushort(__half h) { uint16_t u; memcpy(&u, &h.v, 2); return u; }
inline __half __ushort_as_half(uint16_t u) { __half h; memcpy(&h.v, &u, 2); return h; }
