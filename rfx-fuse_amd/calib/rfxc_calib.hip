// Calibration kernels: the two traffic streams of the batched triangle,
// timed alone and together on synthetic data of the triangle's shape.
//
// The triangle (rfxp_triangle.hip) runs one 1024-thread workgroup per row
// item; each wave loads row i's run records (scalar loads), then one buffer
// load per run (a run is ~12 member ids at a random place of the id array),
// bumps an LDS byte counter per member, and the epilogue streams the row's
// N - i output bytes with 16-byte non-temporal stores.  These kernels keep
// exactly that shape and drop everything else (formats, normalisation,
// exactness checks), so their times are the floor of that formulation on
// this GPU:
//   gather: records + run loads + LDS counting, no output;
//   store:  counter zeroing + the row's LDS reads + stores, no run loads;
//   both:   one workgroup does both, in the triangle's order.
// Rows i = 0 .. N-1 are one item each (widths N - i: the whole triangle,
// N(N+1)/2 bytes).  Records are random: the run of (i, t) starts at a
// uniformly drawn id of an array of mem_bytes bytes and holds 0..24 ids
// (mean 12); ids are 4 bytes (as in the library) or 2 bytes.
//
// Used only by bench.py --calibrate; not part of the proximity library.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int CAL_THREADS = 1024;
constexpr int CAL_WAVES = CAL_THREADS / 64;
constexpr uint32_t CAL_COUNTERS = 65536;                         // counter bytes
constexpr uint32_t CAL_LDS = CAL_COUNTERS + CAL_THREADS * 4;     // + one dummy word per thread
constexpr int CAL_MAX_LEN = 24;                                   // ids per run: 0..24

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) uint32_t lds_u32;

__host__ __device__ inline uint32_t mix32(uint64_t x) {
    x ^= x >> 33;
    x *= 0xff51afd7ed558ccdull;
    x ^= x >> 33;
    x *= 0xc4ceb9fe1a85ec53ull;
    x ^= x >> 33;
    return (uint32_t)x;
}

__host__ __device__ inline int64_t tri_idx(int64_t n, int64_t i, int64_t j) { return i * n - i * (i + 1) / 2 + j; }

// ids: uniform on [1, 65535] (0 marks "no member", as in the library)
__global__ void k_cal_fill(void* mem, int64_t nid, int idb, uint32_t seed) {
    for (int64_t k = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; k < nid; k += (int64_t)gridDim.x * blockDim.x) {
        const uint32_t v = 1u + mix32(((uint64_t)seed << 40) ^ (uint64_t)k) % 65535u;
        if (idb == 4) ((uint32_t*)mem)[k] = v;
        else ((uint16_t*)mem)[k] = (uint16_t)v;
    }
}

// records of (i, t): byte offset of the run, its length in bytes; trees
// t >= T (row padding to ldr) are empty
__global__ void k_cal_records(uint32_t* roff, uint16_t* rlen, int64_t n, int32_t T, int64_t ldr, int64_t nid,
                              int idb, uint32_t seed) {
    const int64_t total = n * ldr;
    for (int64_t k = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; k < total; k += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = k % ldr;
        const uint32_t h = mix32(((uint64_t)(seed + 1) << 40) ^ (uint64_t)k);
        const uint32_t h2 = mix32(((uint64_t)(seed + 2) << 40) ^ (uint64_t)k);
        const uint32_t start = h % (uint32_t)(nid - CAL_MAX_LEN);
        roff[k] = start * (uint32_t)idb;
        rlen[k] = t < T ? (uint16_t)((h2 % (CAL_MAX_LEN + 1)) * (uint32_t)idb) : (uint16_t)0;
    }
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* mem, uint32_t nbytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)mem, (short)0, (int)nbytes, 0x00020000);
}

__device__ __forceinline__ void lds_add(uint32_t addr, uint32_t val) {
    __hip_atomic_fetch_add((lds_u32*)(uintptr_t)addr, val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void count(uint32_t m, uint32_t xlim) {
    const uint32_t c = min(m - 1u, xlim);
    lds_add(c & ~3u, 1u << ((c << 3) & 31u));
}

template <int IDB>
struct Grp {
    uint32_t m[16];
};

// The 16 run loads of one record group.  REC 0: the group's records by
// scalar loads (row index uniform in an SGPR); REC 1: by one vector load of
// 16 offsets and 8 length words (lanes 0..15) and readlane.
template <int IDB, int REC>
__device__ __forceinline__ void load_grp(const void* mem, const uint32_t* ro, const uint16_t* rl, uint32_t lane_off,
                                         Grp<IDB>& G) {
    uint32_t off[16], lw[8];
    if constexpr (REC == 0) {
#pragma unroll
        for (int u = 0; u < 16; ++u) off[u] = __builtin_amdgcn_readfirstlane(ro[u]);
#pragma unroll
        for (int k = 0; k < 8; ++k) lw[k] = __builtin_amdgcn_readfirstlane(((const uint32_t*)rl)[k]);
    } else {
        const uint32_t lane = threadIdx.x & 15u;
        const uint32_t vo = ro[lane];
        const uint32_t vl = ((const uint32_t*)rl)[lane & 7u];
#pragma unroll
        for (int u = 0; u < 16; ++u) off[u] = __builtin_amdgcn_readlane(vo, u);
#pragma unroll
        for (int k = 0; k < 8; ++k) lw[k] = __builtin_amdgcn_readlane(vl, k);
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const uint32_t len = (lw[u >> 1] >> (16 * (u & 1))) & 0xffffu;
        if constexpr (IDB == 4)
            G.m[u] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rsrc(mem, off[u] + len), lane_off, off[u], 0);
        else
            G.m[u] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rsrc(mem, off[u] + len), lane_off, off[u], 0);
    }
}

template <int IDB, int REC>
__device__ __forceinline__ void gather_row(const void* mem, const uint32_t* roff, const uint16_t* rlen, int64_t ldr, int32_t T,
                           int64_t i, uint32_t xlim) {
    const uint32_t lane_off = (threadIdx.x & 63) * (uint32_t)IDB;
    const int32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int32_t ng = (T + 15) >> 4;
    const int32_t g0 = (ng * wave) / CAL_WAVES, g1 = (ng * (wave + 1)) / CAL_WAVES;
    if (g0 >= g1) return;
    const uint32_t* ro = roff + i * ldr;
    const uint16_t* rl = rlen + i * ldr;
    Grp<IDB> A, B;
    load_grp<IDB, REC>(mem, ro + 16 * g0, rl + 16 * g0, lane_off, A);
    if (g0 + 1 < g1) load_grp<IDB, REC>(mem, ro + 16 * (g0 + 1), rl + 16 * (g0 + 1), lane_off, B);
    for (int32_t g = g0;; g += 2) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 16; ++u) count(A.m[u], xlim);
        if (g + 2 < g1) load_grp<IDB, REC>(mem, ro + 16 * (g + 2), rl + 16 * (g + 2), lane_off, A);
        if (g + 1 >= g1) break;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 16; ++u) count(B.m[u], xlim);
        if (g + 3 < g1) load_grp<IDB, REC>(mem, ro + 16 * (g + 3), rl + 16 * (g + 3), lane_off, B);
        if (g + 2 >= g1) break;
    }
}

// MODE bit 1: gather, bit 2: store.  One workgroup per row.
template <int MODE, int IDB, int REC>
__global__ __launch_bounds__(CAL_THREADS) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_cal(
    const void* mem, const uint32_t* roff, const uint16_t* rlen, int64_t ldr, int32_t T, int64_t n, char* out,
    uint32_t* sink) {
    extern __shared__ uint32_t cnt[];
    const int64_t i = blockIdx.x;
    {
        uint4* c4 = (uint4*)cnt;
        for (uint32_t w = threadIdx.x; w < CAL_LDS / 16; w += CAL_THREADS) c4[w] = make_uint4(0u, 0u, 0u, 0u);
    }
    __syncthreads();
    if constexpr (MODE & 1) gather_row<IDB, REC>(mem, roff, rlen, ldr, T, i, CAL_COUNTERS + 4u * threadIdx.x);
    __syncthreads();
    if constexpr (MODE & 2) {
        // the 16-byte chunks that lie wholly inside row i's bytes
        const int64_t e0 = tri_idx(n, i, i), e1 = e0 + (n - i);
        const int64_t c0 = (e0 + 15) >> 4, c1 = e1 >> 4;
        const uint4* c4 = (const uint4*)cnt;
        for (int64_t ck = c0 + threadIdx.x; ck < c1; ck += CAL_THREADS) {
            const uint4 w = c4[(uint32_t)(ck - c0) & (CAL_COUNTERS / 16 - 1)];
            u32x4 v = {w.x, w.y, w.z, w.w};
            __builtin_nontemporal_store(v, (u32x4*)(out + ck * 16));
        }
    } else {
        // keep the counts observable: one word per row
        if (threadIdx.x == 0) sink[i] = cnt[(uint32_t)i & (CAL_COUNTERS / 4 - 1)];
    }
}

template <int MODE, int IDB, int REC>
hipError_t launch(const void* mem, const uint32_t* roff, const uint16_t* rlen, int64_t ldr, int32_t T, int64_t n,
                  void* out, uint32_t* sink, hipStream_t s) {
    hipError_t e = hipFuncSetAttribute((const void*)k_cal<MODE, IDB, REC>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)CAL_LDS);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((k_cal<MODE, IDB, REC>), dim3((unsigned)n), dim3(CAL_THREADS), CAL_LDS, s, mem, roff, rlen, ldr, T,
                       n, (char*)out, sink);
    return hipGetLastError();
}

}  // namespace

extern "C" {

// Fills the id array (mem_bytes / idb ids) and the records ([n][ldr] u32
// offsets and u16 lengths, ldr >= T) on `stream`.  Returns a hipError_t.
int rfxc_setup(void* mem, int64_t mem_bytes, int idb, uint32_t* roff, uint16_t* rlen, int64_t n, int32_t T,
               int64_t ldr, uint32_t seed, void* stream) {
    if ((idb != 2 && idb != 4) || mem_bytes < 4096 || mem_bytes >= (1ll << 31) || n < 1 || T < 1 || ldr < T ||
        ldr % 16)
        return (int)hipErrorInvalidValue;
    const int64_t nid = mem_bytes / idb;
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(k_cal_fill, dim3(4096), dim3(256), 0, s, mem, nid, idb, seed);
    hipLaunchKernelGGL(k_cal_records, dim3(4096), dim3(256), 0, s, roff, rlen, n, T, ldr, nid, idb, seed);
    return (int)hipGetLastError();
}

// One launch of mode 1 (gather), 2 (store) or 3 (both) over rows [0, n):
// mem / roff / rlen from rfxc_setup, out = N(N+1)/2 bytes (modes 2, 3),
// sink = n words (mode 1).  Returns a hipError_t.
int rfxc_run(int mode, int idb, const void* mem, const uint32_t* roff, const uint16_t* rlen, int64_t ldr, int32_t T,
             int64_t n, void* out, uint32_t* sink, void* stream) {
    hipStream_t s = (hipStream_t)stream;
    if (n < 1 || n >= (1ll << 31) || ldr < T || ldr % 16) return (int)hipErrorInvalidValue;
    if ((mode & 2) ? out == nullptr : sink == nullptr) return (int)hipErrorInvalidValue;
    mode &= 7;
    // mode bit 4: records by vector loads (REC 1)
    hipError_t e;
    switch (mode * 8 + idb) {
        case 1 * 8 + 4: e = launch<1, 4, 0>(mem, roff, rlen, ldr, T, n, out, sink, s); break;
        case 2 * 8 + 4: e = launch<2, 4, 0>(mem, roff, rlen, ldr, T, n, out, sink, s); break;
        case 3 * 8 + 4: e = launch<3, 4, 0>(mem, roff, rlen, ldr, T, n, out, sink, s); break;
        case 1 * 8 + 2: e = launch<1, 2, 0>(mem, roff, rlen, ldr, T, n, out, sink, s); break;
        case 3 * 8 + 2: e = launch<3, 2, 0>(mem, roff, rlen, ldr, T, n, out, sink, s); break;
        case 5 * 8 + 4: e = launch<1, 4, 1>(mem, roff, rlen, ldr, T, n, out, sink, s); break;
        case 7 * 8 + 4: e = launch<3, 4, 1>(mem, roff, rlen, ldr, T, n, out, sink, s); break;
        case 5 * 8 + 2: e = launch<1, 2, 1>(mem, roff, rlen, ldr, T, n, out, sink, s); break;
        case 7 * 8 + 2: e = launch<3, 2, 1>(mem, roff, rlen, ldr, T, n, out, sink, s); break;
        default: return (int)hipErrorInvalidValue;
    }
    return (int)e;
}

}  // extern "C"
