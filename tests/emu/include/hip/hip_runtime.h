// Host-side stand-in for <hip/hip_runtime.h> used ONLY by the CPU emulation
// build of the library's kernels (tests/emu).  It maps the HIP kernel
// language onto plain C++ running under a coroutine scheduler
// (tests/emu/emu_rt.cpp): every GPU thread of a workgroup is a coroutine,
// __syncthreads is a workgroup barrier, and the wave-wide builtins
// (readfirstlane, ballot, shuffles, DPP moves) are resolved when every live
// lane of the 64-lane wave has reached them.  Device memory is host memory
// from malloc, so an AddressSanitizer build reports any access outside an
// allocation or outside a workgroup's LDS.  Nothing in the product library
// or its GPU build includes this file.
#pragma once

#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include <tuple>
#include <type_traits>
#include <utility>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __shared__ static
#define __align__(n) __attribute__((aligned(n)))
#define __noinline__ __attribute__((noinline))

// ---- runtime types -------------------------------------------------------
typedef enum hipError_t {
    hipSuccess = 0,
    hipErrorInvalidValue = 1,
    hipErrorOutOfMemory = 2,
    hipErrorMemoryAllocation = 2,
    hipErrorInvalidDevice = 101,
    hipErrorNoDevice = 100,
    hipErrorIllegalAddress = 700,
    hipErrorLaunchFailure = 719,
    hipErrorUnknown = 999
} hipError_t;

typedef struct emu_stream* hipStream_t;
typedef struct emu_event* hipEvent_t;

typedef enum hipMemcpyKind {
    hipMemcpyHostToHost = 0,
    hipMemcpyHostToDevice = 1,
    hipMemcpyDeviceToHost = 2,
    hipMemcpyDeviceToDevice = 3,
    hipMemcpyDefault = 4
} hipMemcpyKind;

typedef enum hipMemoryType {
    hipMemoryTypeHost = 0,
    hipMemoryTypeDevice = 1,
    hipMemoryTypeArray = 2,
    hipMemoryTypeUnified = 3,
    hipMemoryTypeManaged = 4
} hipMemoryType;

typedef struct hipPointerAttribute_t {
    hipMemoryType type;
    int device;
    void* devicePointer;
    void* hostPointer;
    int isManaged;
    unsigned allocationFlags;
} hipPointerAttribute_t;

typedef enum hipDeviceAttribute_t {
    hipDeviceAttributeMaxSharedMemoryPerBlock = 1,
    hipDeviceAttributeMultiprocessorCount = 2
} hipDeviceAttribute_t;

typedef enum hipFuncAttribute {
    hipFuncAttributeMaxDynamicSharedMemorySize = 8
} hipFuncAttribute;

#define hipStreamNonBlocking 0x01

struct dim3 {
    uint32_t x, y, z;
    constexpr dim3(uint32_t a = 1, uint32_t b = 1, uint32_t c = 1) : x(a), y(b), z(c) {}
};

// ---- vector types --------------------------------------------------------
// aligned as HIP aligns them (the size of the whole vector), so that layouts
// match the device's and the alignment sanitizer sees misaligned accesses
struct alignas(8) uint2 { uint32_t x, y; };
struct alignas(16) uint4 { uint32_t x, y, z, w; };
struct alignas(8) int2 { int32_t x, y; };
struct alignas(16) int4 { int32_t x, y, z, w; };
struct alignas(8) float2 { float x, y; };
struct alignas(16) float4 { float x, y, z, w; };
struct alignas(16) double2 { double x, y; };
inline uint2 make_uint2(uint32_t a, uint32_t b) { return uint2{a, b}; }
inline uint4 make_uint4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) { return uint4{a, b, c, d}; }
inline int2 make_int2(int32_t a, int32_t b) { return int2{a, b}; }
inline int4 make_int4(int32_t a, int32_t b, int32_t c, int32_t d) { return int4{a, b, c, d}; }
inline float2 make_float2(float a, float b) { return float2{a, b}; }
inline float4 make_float4(float a, float b, float c, float d) { return float4{a, b, c, d}; }
inline double2 make_double2(double a, double b) { return double2{a, b}; }

// ---- the scheduler's view (tests/emu/emu_rt.cpp) -------------------------
namespace emu {
struct Idx {
    uint32_t x, y, z;
};
struct ThreadView {
    Idx tid, bid, bdim, gdim;
    int lane;
};
const ThreadView& view();
char* lds_base();
void barrier(const char* file, int line);
enum WaveOp {
    W_READFIRST = 1, W_READLANE, W_BALLOT, W_SHFL, W_SHFL_UP, W_SHFL_DOWN, W_SHFL_XOR, W_DPP
};
uint64_t wave(int op, uint64_t v, int64_t arg, int64_t width, const char* file, int line);

// A build-time constant of the library that the emulation lets a test set:
// the environment variable `name` as an integer, else dflt.
long long knob(const char* name, long long dflt);

typedef void (*Body)(void* closure);
void launch_raw(const void* kernel, const char* name, dim3 grid, dim3 block, size_t lds, hipStream_t s, Body body,
                void* closure, const void* args, size_t args_bytes);

template <class T>
inline uint64_t to_bits(T v) {
    uint64_t b = 0;
    static_assert(sizeof(T) <= 8, "wave values up to 8 bytes");
    memcpy(&b, &v, sizeof(T));
    return b;
}
template <class T>
inline T from_bits(uint64_t b) {
    T v;
    memcpy(&v, &b, sizeof(T));
    return v;
}

template <class... P, class... A>
inline void launch(void (*kernel)(P...), const char* name, dim3 grid, dim3 block, size_t lds, hipStream_t s,
                   A&&... args) {
    std::tuple<std::decay_t<P>...> t(static_cast<std::decay_t<P>>(std::forward<A>(args))...);
    struct C {
        void (*k)(P...);
        std::tuple<std::decay_t<P>...>* t;
    } c{kernel, &t};
    launch_raw((const void*)kernel, name, grid, block, lds, s,
               [](void* p) {
                   C* cc = (C*)p;
                   std::apply(cc->k, *cc->t);
               },
               &c, (const void*)&t, sizeof(t));
}
}  // namespace emu

#define threadIdx (::emu::view().tid)
#define blockIdx (::emu::view().bid)
#define blockDim (::emu::view().bdim)
#define gridDim (::emu::view().gdim)
#define hipLaunchKernelGGL(kernel, grid, block, lds, stream, ...) \
    ::emu::launch(kernel, #kernel, dim3(grid), dim3(block), (size_t)(lds), stream, ##__VA_ARGS__)

// the call site of each barrier and wave builtin is recorded for the scheduler's checks
#define EMU_AT const char* emu_file = __builtin_FILE(), int emu_line = __builtin_LINE()
inline void __syncthreads(EMU_AT) { ::emu::barrier(emu_file, emu_line); }
inline void __threadfence() {}
inline void __threadfence_block() {}

// ---- wave-wide operations ------------------------------------------------
template <class T>
inline T __shfl(T v, int src, int width = 64, EMU_AT) {
    return ::emu::from_bits<T>(::emu::wave(::emu::W_SHFL, ::emu::to_bits(v), src, width,
                                                emu_file, emu_line));
}
template <class T>
inline T __shfl_up(T v, unsigned d, int width = 64, EMU_AT) {
    return ::emu::from_bits<T>(::emu::wave(::emu::W_SHFL_UP, ::emu::to_bits(v), (int64_t)d, width,
                                                emu_file, emu_line));
}
template <class T>
inline T __shfl_down(T v, unsigned d, int width = 64, EMU_AT) {
    return ::emu::from_bits<T>(::emu::wave(::emu::W_SHFL_DOWN, ::emu::to_bits(v), (int64_t)d, width,
                                                emu_file, emu_line));
}
template <class T>
inline T __shfl_xor(T v, int m, int width = 64, EMU_AT) {
    return ::emu::from_bits<T>(::emu::wave(::emu::W_SHFL_XOR, ::emu::to_bits(v), m, width,
                                                emu_file, emu_line));
}
inline unsigned long long __ballot(int pred, EMU_AT) {
    return ::emu::wave(::emu::W_BALLOT, pred != 0, 0, 64, emu_file, emu_line);
}
inline uint32_t emu_readfirstlane(uint32_t v, EMU_AT) {
    return (uint32_t)::emu::wave(::emu::W_READFIRST, v, 0, 64, emu_file, emu_line);
}
inline int32_t emu_readfirstlane(int32_t v, EMU_AT) {
    return (int32_t)::emu::wave(::emu::W_READFIRST, (uint32_t)v, 0, 64, emu_file, emu_line);
}
inline uint32_t emu_readlane(uint32_t v, int lane, EMU_AT) {
    return (uint32_t)::emu::wave(::emu::W_READLANE, v, lane, 64, emu_file, emu_line);
}
inline int32_t emu_readlane(int32_t v, int lane, EMU_AT) {
    return (int32_t)::emu::wave(::emu::W_READLANE, (uint32_t)v, lane, 64, emu_file, emu_line);
}
inline int emu_mov_dpp(int v, int ctrl, int, int, bool, EMU_AT) {
    return (int)::emu::wave(::emu::W_DPP, (uint32_t)v, ctrl, 64, emu_file, emu_line);
}
inline uint32_t emu_mbcnt_lo(uint32_t m, uint32_t acc) {
    const int l = ::emu::view().lane;
    const uint32_t below = l >= 32 ? m : (l == 0 ? 0u : (m & ((1u << l) - 1u)));
    return acc + (uint32_t)__builtin_popcount(below);
}
inline uint32_t emu_mbcnt_hi(uint32_t m, uint32_t acc) {
    const int l = ::emu::view().lane;
    const uint32_t below = l < 32 ? 0u : (l == 32 ? 0u : (m & ((1u << (l - 32)) - 1u)));
    return acc + (uint32_t)__builtin_popcount(below);
}
#define __builtin_amdgcn_readfirstlane emu_readfirstlane
#define __builtin_amdgcn_readlane emu_readlane
#define __builtin_amdgcn_mov_dpp emu_mov_dpp
#define __builtin_amdgcn_mbcnt_lo emu_mbcnt_lo
#define __builtin_amdgcn_mbcnt_hi emu_mbcnt_hi
#define __builtin_amdgcn_sched_barrier(x) ((void)0)

// v_perm_b32: byte k of the result is byte sel_k of {s0 (bytes 4..7), s1 (bytes 0..3)};
// selectors 8..11 and 12 give sign / 0x00 / 0xff patterns (only 0..7 are used here)
inline uint32_t emu_perm(uint32_t s0, uint32_t s1, uint32_t sel) {
    const uint64_t v = ((uint64_t)s0 << 32) | s1;
    uint32_t r = 0;
    for (int k = 0; k < 4; ++k) {
        const uint32_t s = (sel >> (8 * k)) & 0xffu;
        uint32_t b;
        if (s < 8) b = (uint32_t)(v >> (8 * s)) & 0xffu;
        else if (s == 12) b = 0x00u;
        else if (s >= 13) b = 0xffu;
        else {  // 8..11: sign bits of bytes 1, 3, 5, 7 replicated
            const int src = 2 * (int)(s - 8) + 1;
            b = ((v >> (8 * src + 7)) & 1u) ? 0xffu : 0x00u;
        }
        r |= b << (8 * k);
    }
    return r;
}
// v_sad_u8: acc + sum over the four bytes of |a_k - b_k|
inline uint32_t emu_sad_u8(uint32_t a, uint32_t b, uint32_t acc) {
    for (int k = 0; k < 4; ++k) {
        const int x = (int)((a >> (8 * k)) & 0xffu), y = (int)((b >> (8 * k)) & 0xffu);
        acc += (uint32_t)(x > y ? x - y : y - x);
    }
    return acc;
}
#define __builtin_amdgcn_perm emu_perm
#define __builtin_amdgcn_sad_u8 emu_sad_u8

// buffer resources: base, range in bytes; loads past the range read 0
struct emu_rsrc {
    const char* base;
    uint32_t num;
};
typedef emu_rsrc __amdgpu_buffer_rsrc_t;
inline emu_rsrc emu_make_rsrc(void* p, short, int num, int) { return emu_rsrc{(const char*)p, (uint32_t)num}; }
inline uint32_t emu_raw_load_b32(emu_rsrc r, uint32_t voff, uint32_t soff, int) {
    const uint64_t o = (uint64_t)voff + soff;
    if (o + 4 > r.num) return 0u;
    uint32_t v;
    memcpy(&v, r.base + o, 4);
    return v;
}
inline uint16_t emu_raw_load_b16(emu_rsrc r, uint32_t voff, uint32_t soff, int) {
    const uint64_t o = (uint64_t)voff + soff;
    if (o + 2 > r.num) return 0u;
    uint16_t v;
    memcpy(&v, r.base + o, 2);
    return v;
}
#define __builtin_amdgcn_make_buffer_rsrc emu_make_rsrc
#define __builtin_amdgcn_raw_buffer_load_b32 emu_raw_load_b32
#define __builtin_amdgcn_raw_buffer_load_b16 emu_raw_load_b16

// ---- atomics (one OS thread runs every coroutine: plain read-modify-write)
#define __HIP_MEMORY_SCOPE_WORKGROUP 2
#define __HIP_MEMORY_SCOPE_AGENT 3
template <class T, class U>
inline T emu_atomic_fetch_add(T* p, U v, int, int) {
    T o = *p;
    *p = (T)(o + (T)v);
    return o;
}
#define __hip_atomic_fetch_add emu_atomic_fetch_add
template <class T, class U>
inline T atomicAdd(T* p, U v) {
    T o = *p;
    *p = (T)(o + (T)v);
    return o;
}
template <class T, class U>
inline T atomicSub(T* p, U v) {
    T o = *p;
    *p = (T)(o - (T)v);
    return o;
}
template <class T, class U>
inline T atomicAnd(T* p, U v) {
    T o = *p;
    *p = (T)(o & (T)v);
    return o;
}
template <class T, class U>
inline T atomicOr(T* p, U v) {
    T o = *p;
    *p = (T)(o | (T)v);
    return o;
}
template <class T, class U>
inline T atomicMin(T* p, U v) {
    T o = *p;
    if ((T)v < o) *p = (T)v;
    return o;
}
template <class T, class U>
inline T atomicMax(T* p, U v) {
    T o = *p;
    if ((T)v > o) *p = (T)v;
    return o;
}
template <class T, class U, class W>
inline T atomicCAS(T* p, U cmp, W v) {
    T o = *p;
    if (o == (T)cmp) *p = (T)v;
    return o;
}
template <class T, class U>
inline T atomicExch(T* p, U v) {
    T o = *p;
    *p = (T)v;
    return o;
}

// ---- device min / max of the HIP headers (integer and mixed arguments) ----
template <class A, class B>
inline typename std::common_type<A, B>::type min(A a, B b) {
    typedef typename std::common_type<A, B>::type C;
    return (C)a < (C)b ? (C)a : (C)b;
}
template <class A, class B>
inline typename std::common_type<A, B>::type max(A a, B b) {
    typedef typename std::common_type<A, B>::type C;
    return (C)a > (C)b ? (C)a : (C)b;
}

// ---- bit and type helpers ------------------------------------------------
inline int __popc(uint32_t x) { return __builtin_popcount(x); }
inline int __popcll(unsigned long long x) { return __builtin_popcountll(x); }
inline int __clz(int x) { return x == 0 ? 32 : __builtin_clz((unsigned)x); }
inline int __clzll(long long x) { return x == 0 ? 64 : __builtin_clzll((unsigned long long)x); }
inline int __ffs(int x) { return __builtin_ffs(x); }
inline int __ffsll(long long x) { return __builtin_ffsll(x); }
inline long long __double_as_longlong(double d) { long long v; memcpy(&v, &d, 8); return v; }
inline double __longlong_as_double(long long v) { double d; memcpy(&d, &v, 8); return d; }
inline uint32_t __float_as_uint(float f) { uint32_t v; memcpy(&v, &f, 4); return v; }
inline float __uint_as_float(uint32_t v) { float f; memcpy(&f, &v, 4); return f; }
inline int __float_as_int(float f) { int v; memcpy(&v, &f, 4); return v; }
inline float __int_as_float(int v) { float f; memcpy(&f, &v, 4); return f; }

// ---- runtime API ---------------------------------------------------------
hipError_t hipMalloc(void** p, size_t n);
template <class T>
inline hipError_t hipMalloc(T** p, size_t n) { return hipMalloc((void**)p, n); }
hipError_t hipFree(void* p);
hipError_t hipMemGetInfo(size_t* free_b, size_t* total_b);
hipError_t hipMemcpy(void* d, const void* s, size_t n, hipMemcpyKind k);
hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind k, hipStream_t st = nullptr);
hipError_t hipMemset(void* d, int v, size_t n);
hipError_t hipMemsetAsync(void* d, int v, size_t n, hipStream_t st = nullptr);
hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned flags);
hipError_t hipStreamCreate(hipStream_t* s);
hipError_t hipStreamDestroy(hipStream_t s);
hipError_t hipStreamSynchronize(hipStream_t s);
hipError_t hipDeviceSynchronize();
hipError_t hipEventCreate(hipEvent_t* e);
hipError_t hipEventDestroy(hipEvent_t e);
hipError_t hipEventRecord(hipEvent_t e, hipStream_t s = nullptr);
hipError_t hipEventSynchronize(hipEvent_t e);
hipError_t hipEventElapsedTime(float* ms, hipEvent_t a, hipEvent_t b);
hipError_t hipSetDevice(int d);
hipError_t hipGetDevice(int* d);
hipError_t hipGetDeviceCount(int* n);
hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t a, int d);
hipError_t hipPointerGetAttributes(hipPointerAttribute_t* a, const void* p);
hipError_t hipFuncSetAttribute(const void* f, hipFuncAttribute a, int v);
hipError_t hipGetLastError();
hipError_t hipPeekAtLastError();
const char* hipGetErrorString(hipError_t e);
hipError_t hipGetSymbolAddress(void** p, const void* sym);
#define HIP_SYMBOL(x) ((const void*)&(x))
