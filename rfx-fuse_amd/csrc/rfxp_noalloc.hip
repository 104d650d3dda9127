// Allocation-free one-shot triangle (rfxp_upper_noalloc): rfxp_set_forest +
// rfxp_upper in one call, with the whole forest index (buckets, records,
// histograms, nout) in a static device workspace instead of context buffers.
// For callers that may not allocate device memory: code under stream
// capture, tight loops over many small forests, harnesses that forbid
// hipMalloc.  It launches the same kernels as the two calls it combines.
//
// The workspace is one file-scope __device__ array per GPU, NOALLOC_BYTES
// long, held by every GPU the library runs on until the process ends.  Its
// device address is taken once per device with hipGetSymbolAddress when a
// context is created on that device (rfxp_ctx_create) and used from then on;
// the array's host-side name is never passed to a kernel.  Every call on a
// GPU shares that GPU's workspace: calls that overlap on one GPU (other
// streams, other host threads) race and must be serialised by the caller.
#include <mutex>
#include <string>

#include "rfxp_device.hpp"
#include "rfxp_forest.hpp"
#include "rfxp_internal.hpp"

namespace rfxp {

constexpr size_t NOALLOC_BYTES = (size_t)RFXP_UPPER_NOALLOC_MAX_BYTES;
constexpr int NOALLOC_MAX_DEVICES = 64;
constexpr size_t NOALLOC_ALIGN = 256;

static __device__ __align__(256) unsigned char scratch[NOALLOC_BYTES];

static std::mutex g_noalloc_mu;
static void* g_noalloc_ptr[NOALLOC_MAX_DEVICES];  // device address of `scratch`, per device
static int g_noalloc_err[NOALLOC_MAX_DEVICES];    // hipError_t of the set-up, per device

// Called by rfxp_ctx_create with `device` current.
void noalloc_setup(int device) {
    if (device < 0 || device >= NOALLOC_MAX_DEVICES) return;
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (g_noalloc_ptr[device]) return;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        g_noalloc_err[device] = e != hipSuccess ? (int)e : (int)hipErrorUnknown;
        return;
    }
    g_noalloc_ptr[device] = p;
    g_noalloc_err[device] = 0;
}

static void* noalloc_ptr(int device) {
    if (device < 0 || device >= NOALLOC_MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    return g_noalloc_ptr[device];
}

// Bytes of workspace the forest index of a view takes (every buffer
// 256-byte aligned), and its carving out of base (when base is not NULL).
static size_t noalloc_layout(const ForestSizes& z, unsigned char* base, ForestBufs& fb) {
    size_t off = 0;
    void* at[FB_COUNT] = {};
    for (int k = 0; k < FB_COUNT; ++k) {
        if (!z.n[k]) continue;
        off = (off + NOALLOC_ALIGN - 1) & ~(NOALLOC_ALIGN - 1);
        at[k] = base ? (void*)(base + off) : nullptr;
        off += z.n[k] * forest_elem_bytes(k);
    }
    fb = ForestBufs();
    fb.off = (int32_t*)at[FB_OFF];
    fb.bend = (int32_t*)at[FB_BEND];
    fb.mem = (uint32_t*)at[FB_MEM];
    fb.roff = (uint32_t*)at[FB_ROFF];
    fb.rlen = (uint16_t*)at[FB_RLEN];
    fb.roffT = (uint32_t*)at[FB_ROFFT];
    fb.rlenT = (uint16_t*)at[FB_RLENT];
    fb.scratch = (uint32_t*)at[FB_SCRATCH];
    fb.scratch2 = (uint32_t*)at[FB_SCRATCH2];
    fb.key16 = (uint16_t*)at[FB_KEY16];
    fb.nout = (int32_t*)at[FB_NOUT];
    fb.rinv = (double*)at[FB_RINV];
    fb.rrange = (unsigned long long*)at[FB_RRANGE];
    fb.lng = (uint2*)at[FB_LNG];
    fb.lngn = (int32_t*)at[FB_LNGN];
    fb.flags = (int32_t*)at[FB_FLAGS];
    fb.ldr = z.ldr;
    fb.lmax = z.lmax;
    fb.ms = z.ms;
    return off;
}

}  // namespace rfxp

using namespace rfxp;

extern "C" int64_t rfxp_upper_noalloc_workspace(int64_t N, int32_t T, int32_t nleaf, int nout_given) {
    if (N < 0 || T < 1 || T > 65535 || nleaf < 1 || nleaf > (1 << 29) || N > MAX_FOREST_N) return -1;
    const LeafView v{nullptr, 1, N, nullptr, (N + 31) / 32, N, T, nleaf, 0, 0};
    ForestBufs fb;
    return (int64_t)noalloc_layout(forest_sizes(v, nout_given == 0, 65536), nullptr, fb);
}

extern "C" int rfxp_upper_noalloc(rfxp_ctx* ctx, const int32_t* leaf, int64_t stride_i, int64_t stride_t,
                                  const uint32_t* oob_words, int64_t oob_ld, int64_t N, int32_t T, int32_t nleaf,
                                  const int32_t* nout, int fmt, float scale, float zp, int64_t r0, int64_t r1,
                                  void* out) {
    if (!ctx) return RFXP_ERR_INVALID;
    if (N < 0 || T < 1 || T > 65535 || nleaf < 1 || nleaf > (1 << 29))
        return set_error(ctx, RFXP_ERR_INVALID,
                         "rfxp_upper_noalloc: need N >= 0, 1 <= T <= 65535, 1 <= nleaf <= 2^29");
    if (N > MAX_FOREST_N || (int64_t)N * T + MEM_PAD > (1LL << 30) - 1)
        return set_error(ctx, RFXP_ERR_UNSUPPORTED, "rfxp_upper_noalloc: N or N*T too large");
    if (N > 0 && (!leaf || !oob_words))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_upper_noalloc: leaf / oob_words are NULL");
    if (oob_ld < (N + 31) / 32) return set_error(ctx, RFXP_ERR_INVALID, "rfxp_upper_noalloc: oob_ld < ceil(N/32)");
    if (N > 0 && (!is_device_pointer(leaf) || !is_device_pointer(oob_words) || (nout && !is_device_pointer(nout))))
        return set_error(ctx, RFXP_ERR_INVALID, "rfxp_upper_noalloc: inputs must be device pointers");
    if (int rc = upper_check_args(ctx, "rfxp_upper_noalloc", N, fmt, scale, zp, r0, r1, out)) return rc;
    const LeafView v{leaf, stride_i, stride_t, oob_words, oob_ld, N, T, nleaf, 0, 0};
    const ForestSizes z = forest_sizes(v, nout == nullptr, ctx->max_lds);
    ForestBufs fb;
    const size_t need = noalloc_layout(z, nullptr, fb);
    if (need > NOALLOC_BYTES)
        return set_error(ctx, RFXP_ERR_UNSUPPORTED,
                         "rfxp_upper_noalloc: this forest needs " + std::to_string(need) +
                             " bytes of workspace, above the maximum of " + std::to_string(NOALLOC_BYTES) +
                             " (use rfxp_set_forest + rfxp_upper)");
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    unsigned char* base = (unsigned char*)noalloc_ptr(ctx->device);
    if (!base)
        return set_error(ctx, RFXP_ERR_HIP,
                         "rfxp_upper_noalloc: the device workspace was not set up for device " +
                             std::to_string(ctx->device));
    noalloc_layout(z, base, fb);
    // no launch timing here: its events are created on demand
    const bool timing = ctx->timing;
    ctx->timing = false;
    int rc = pack_forest(ctx, v, nout, fb);
    if (rc == RFXP_OK) rc = upper_launch(ctx, fb, N, T, fmt, scale, zp, r0, r1, out);
    ctx->timing = timing;
    return rc;
}
