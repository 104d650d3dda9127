// Context lifecycle, error reporting, streams and launch timing of the
// C ABI (include/rfx_prox.h).
#include <string.h>

#include <string>

#include "rfxp_internal.hpp"

static thread_local std::string g_create_error;
static thread_local int g_create_status = RFXP_OK;

namespace rfxp {

int set_error(rfxp_ctx* ctx, int status, const std::string& msg) {
    if (ctx) {
        ctx->last_status = status;
        ctx->last_error = msg;
    } else {
        g_create_status = status;
        g_create_error = msg;
    }
    return status;
}

int hip_error(rfxp_ctx* ctx, hipError_t e, const char* what) {
    int st = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? RFXP_ERR_NOMEM : RFXP_ERR_HIP;
    (void)hipGetLastError();
    return set_error(ctx, st, std::string(what) + ": " + hipGetErrorString(e));
}

int check_launch(rfxp_ctx* ctx, const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(ctx, e, what);
    return RFXP_OK;
}

bool is_device_pointer(const void* p) {
    if (!p) return false;
    hipPointerAttribute_t attr;
    hipError_t e = hipPointerGetAttributes(&attr, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}

static hipEvent_t take_event(rfxp_ctx* ctx) {
    if (!ctx->event_pool.empty()) {
        hipEvent_t e = ctx->event_pool.back();
        ctx->event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return e;
}

// Folds completed event pairs into the per-kernel totals.
static void drain_timing(rfxp_ctx* ctx, bool wait) {
    std::vector<std::pair<std::string, std::pair<hipEvent_t, hipEvent_t>>> keep;
    for (auto& it : ctx->pending) {
        hipEvent_t a = it.second.first, b = it.second.second;
        if (wait) (void)hipEventSynchronize(b);
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, a, b) == hipSuccess) {
            KernelTiming& k = ctx->times[it.first];
            k.ms += ms;
            k.launches += 1;
            ctx->event_pool.push_back(a);
            ctx->event_pool.push_back(b);
        } else {
            (void)hipGetLastError();
            keep.push_back(it);
        }
    }
    ctx->pending.swap(keep);
}

LaunchTimer::LaunchTimer(rfxp_ctx* c, const char* n) : ctx(c), name(n) {
    if (!ctx->timing) return;
    a = take_event(ctx);
    b = take_event(ctx);
    if (a && b) (void)hipEventRecord(a, ctx->stream);
}

LaunchTimer::~LaunchTimer() {
    if (!ctx->timing || !a || !b) return;
    (void)hipEventRecord(b, ctx->stream);
    ctx->pending.push_back({name, {a, b}});
    if (ctx->pending.size() > 256) drain_timing(ctx, true);
}

}  // namespace rfxp

extern "C" {

int rfxp_ctx_create(int device, rfxp_ctx** out) {
    if (!out) return rfxp::set_error(nullptr, RFXP_ERR_INVALID, "rfxp_ctx_create: out is NULL");
    *out = nullptr;
    int ndev = 0;
    hipError_t e = hipGetDeviceCount(&ndev);
    if (e != hipSuccess || ndev <= 0) {
        (void)hipGetLastError();
        return rfxp::set_error(nullptr, RFXP_ERR_HIP, "rfxp_ctx_create: no HIP device visible");
    }
    if (device < 0 || device >= ndev)
        return rfxp::set_error(nullptr, RFXP_ERR_INVALID, "rfxp_ctx_create: device index out of range");
    rfxp_ctx* ctx = new rfxp_ctx();
    ctx->device = device;
    if ((e = hipSetDevice(device)) != hipSuccess ||
        (e = hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking)) != hipSuccess) {
        delete ctx;
        (void)hipGetLastError();
        return rfxp::set_error(nullptr, RFXP_ERR_HIP, std::string("rfxp_ctx_create: ") + hipGetErrorString(e));
    }
    ctx->stream = ctx->own_stream;
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, device) == hipSuccess && v > 0)
        ctx->max_lds = v;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess)
        ctx->n_cu = v;
    (void)hipGetLastError();
    rfxp::noalloc_setup(device);  // the static workspace's address on this device
    *out = ctx;
    return RFXP_OK;
}

int rfxp_ctx_destroy(rfxp_ctx* ctx) {
    if (!ctx) return RFXP_OK;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    for (auto& it : ctx->pending) {
        (void)hipEventDestroy(it.second.first);
        (void)hipEventDestroy(it.second.second);
    }
    for (hipEvent_t ev : ctx->event_pool) (void)hipEventDestroy(ev);
    ctx->bkt_off.release();
    ctx->bkt_end.release();
    ctx->bkt_mem.release();
    ctx->roffT.release();
    ctx->rlenT.release();
    ctx->scratch.release();
    ctx->scratch2.release();
    ctx->key16.release();
    ctx->roff.release();
    ctx->rlen.release();
    ctx->lng.release();
    ctx->lngn.release();
    ctx->nout.release();
    ctx->rinv.release();
    ctx->rrange.release();
    ctx->flags.release();
    ctx->mm_ws.release();
    ctx->mm_part.release();
    ctx->ref_off.release();
    ctx->ref_mem.release();
    ctx->lr_start.release();
    ctx->lr_tot.release();
    ctx->lr_pmap.release();
    ctx->lr_w.release();
    ctx->lr_z.release();
    ctx->lr_tmp.release();
    ctx->lr_part.release();
    ctx->lr_rinv.release();
    for (auto* b : {&ctx->tr_status, &ctx->tr_nodextr, &ctx->tr_nin, &ctx->tr_term, &ctx->tr_members, &ctx->tr_node,
                    &ctx->tr_pofs, &ctx->dn_nout})
        b->release();
    ctx->tr_idx.release();
    ctx->tr_w.release();
    ctx->tr_out.release();
    ctx->dn_prox.release();
    ctx->dn_out.release();
    for (auto* b : {&ctx->sa_i, &ctx->sa_j, &ctx->sa_col, &ctx->sa_sv}) b->release();
    ctx->sa_v.release();
    ctx->sa_val.release();
    ctx->sa_cnt.release();
    ctx->sa_rowptr.release();
    ctx->sa_deg.release();
    for (auto* b : {&ctx->sa_tri, &ctx->sa_stage, &ctx->sa_x, &ctx->sa_y, &ctx->sa_z, &ctx->sa_part, &ctx->sa_g,
                    &ctx->sa_w, &ctx->sa_wv})
        b->release();
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
    (void)hipGetLastError();
    delete ctx;
    return RFXP_OK;
}

int rfxp_ctx_set_stream(rfxp_ctx* ctx, void* hip_stream) {
    if (!ctx) return RFXP_ERR_INVALID;
    ctx->stream = (hipStream_t)hip_stream;
    return RFXP_OK;
}

void* rfxp_ctx_stream(rfxp_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

void* rfxp_ctx_own_stream(rfxp_ctx* ctx) { return ctx ? (void*)ctx->own_stream : nullptr; }

int rfxp_sync(rfxp_ctx* ctx) {
    if (!ctx) return RFXP_ERR_INVALID;
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    RFXP_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return RFXP_OK;
}

int rfxp_last_error(rfxp_ctx* ctx, char* buf, size_t n) {
    const std::string& m = ctx ? ctx->last_error : g_create_error;
    if (buf && n > 0) {
        size_t k = m.size() < n - 1 ? m.size() : n - 1;
        memcpy(buf, m.data(), k);
        buf[k] = '\0';
    }
    return ctx ? ctx->last_status : g_create_status;
}

int rfxp_set_timing(rfxp_ctx* ctx, int on) {
    if (!ctx) return RFXP_ERR_INVALID;
    ctx->timing = on != 0;
    return RFXP_OK;
}

int rfxp_kernel_time(rfxp_ctx* ctx, const char* name, double* ms, int64_t* launches) {
    if (!ctx || !name) return RFXP_ERR_INVALID;
    RFXP_HIP(ctx, hipSetDevice(ctx->device));
    rfxp::drain_timing(ctx, true);
    auto it = ctx->times.find(name);
    if (ms) *ms = it == ctx->times.end() ? 0.0 : it->second.ms;
    if (launches) *launches = it == ctx->times.end() ? 0 : it->second.launches;
    return RFXP_OK;
}

int rfxp_reset_timing(rfxp_ctx* ctx) {
    if (!ctx) return RFXP_ERR_INVALID;
    rfxp::drain_timing(ctx, true);
    ctx->times.clear();
    return RFXP_OK;
}

}  // extern "C"
