// Context management for the C ABI declared in include/aq_mi355x.h.
#include "aq_internal.hpp"

#include <mutex>
#include <unordered_map>

size_t aq_static_lds(const void *fn) {
    static std::mutex mu;
    static std::unordered_map<const void *, size_t> cache;
    std::lock_guard<std::mutex> lock(mu);
    const auto it = cache.find(fn);
    if (it != cache.end()) return it->second;
    hipFuncAttributes attr{};
    const size_t v = hipFuncGetAttributes(&attr, fn) == hipSuccess ? attr.sharedSizeBytes : kAqLdsBytes + 1;
    cache.emplace(fn, v);
    return v;
}

aq_status aq_ctx_scratch(aq_ctx *ctx, int slot, size_t bytes, void **out) {
    if (!ctx || !out || slot < 0 || slot >= aq_ctx::kScratchSlots) return AQ_E_INVALID_ARG;
    if (bytes > ctx->scratch_bytes[slot]) {
        aq_device_guard g(ctx->device);
        AQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (ctx->scratch[slot]) (void)hipFree(ctx->scratch[slot]);
        ctx->scratch[slot] = nullptr;
        ctx->scratch_bytes[slot] = 0;
        if (hipMalloc(&ctx->scratch[slot], bytes) != hipSuccess)
            return aq_fail(ctx, AQ_E_NOMEM, "work buffer of %zu bytes could not be allocated", bytes);
        ctx->scratch_bytes[slot] = bytes;
    }
    *out = ctx->scratch[slot];
    return AQ_OK;
}

bool aq_timing_events(aq_ctx *ctx, hipEvent_t *start, hipEvent_t *stop) {
    if (!ctx || !ctx->timing) return false;
    if (ctx->ev_used == ctx->ev_start.size()) {
        hipEvent_t a = nullptr, b = nullptr;
        if (hipEventCreate(&a) != hipSuccess) return false;
        if (hipEventCreate(&b) != hipSuccess) {
            (void)hipEventDestroy(a);
            return false;
        }
        ctx->ev_start.push_back(a);
        ctx->ev_stop.push_back(b);
    }
    const size_t slot = ctx->ev_used++;
    *start = ctx->ev_start[slot];
    *stop = ctx->ev_stop[slot];
    return true;
}

aq_status aq_launch_lds(aq_ctx *ctx, const void *fn, size_t dynamic, const char *what) {
    if (!aq_lds_fits(fn, dynamic))
        return aq_fail(ctx, AQ_E_SHAPE, "%s: %zu bytes of LDS (%zu dynamic) exceed a CU's %zu", what,
                       dynamic + aq_static_lds(fn), dynamic, kAqLdsBytes);
    static std::mutex mu;
    static std::unordered_map<const void *, size_t> raised[64];
    const int dev = ctx->device >= 0 && ctx->device < 64 ? ctx->device : 0;
    std::lock_guard<std::mutex> lock(mu);
    size_t &have = raised[dev][fn];
    if (dynamic > have) {
        const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(dynamic));
        if (e != hipSuccess)
            return aq_fail(ctx, AQ_E_DEVICE, "%s: hipFuncSetAttribute failed: %s", what, hipGetErrorString(e));
        have = dynamic;
    }
    return AQ_OK;
}

extern "C" {

int aq_abi_version(void) { return AQ_ABI_VERSION; }

aq_status aq_ctx_set_timing(aq_ctx *ctx, int enable) {
    if (!ctx) return AQ_E_INVALID_ARG;
    ctx->timing = enable != 0;
    ctx->ev_used = 0;
    return AQ_OK;
}

aq_status aq_ctx_read_timing(aq_ctx *ctx, float *ms, int capacity, int *count) {
    if (!ctx || !count || (capacity > 0 && !ms)) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_ctx_read_timing: null argument");
    aq_device_guard g(ctx->device);
    AQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    const int n = static_cast<int>(ctx->ev_used);
    for (int i = 0; i < n && i < capacity; ++i)
        AQ_HIP(ctx, hipEventElapsedTime(&ms[i], ctx->ev_start[static_cast<size_t>(i)], ctx->ev_stop[static_cast<size_t>(i)]));
    *count = n;
    ctx->ev_used = 0;
    return AQ_OK;
}

aq_status aq_ctx_create(int device, void *hip_stream, aq_ctx **out) {
    if (!out) return AQ_E_INVALID_ARG;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) return AQ_E_DEVICE;
    if (device < 0 || device >= count) return AQ_E_INVALID_ARG;
    aq_ctx *ctx = new (std::nothrow) aq_ctx();
    if (!ctx) return AQ_E_NOMEM;
    ctx->device = device;
    ctx->stream = static_cast<hipStream_t>(hip_stream);
    aq_device_guard g(device);
    hipDeviceProp_t prop{};
    if (hipGetDeviceProperties(&prop, device) != hipSuccess ||
        hipMalloc(&ctx->d_flags, sizeof(int32_t) * AQ_FLAG_COUNT) != hipSuccess ||
        hipMemset(ctx->d_flags, 0, sizeof(int32_t) * AQ_FLAG_COUNT) != hipSuccess) {
        if (ctx->d_flags) (void)hipFree(ctx->d_flags);
        delete ctx;
        return AQ_E_DEVICE;
    }
    ctx->num_cus = prop.multiProcessorCount;
    *out = ctx;
    return AQ_OK;
}

aq_status aq_ctx_destroy(aq_ctx *ctx) {
    if (!ctx) return AQ_E_INVALID_ARG;
    {
        aq_device_guard g(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
        if (ctx->d_flags) (void)hipFree(ctx->d_flags);
        for (int i = 0; i < aq_ctx::kScratchSlots; ++i)
            if (ctx->scratch[i]) (void)hipFree(ctx->scratch[i]);
        for (hipEvent_t e : ctx->ev_start) (void)hipEventDestroy(e);
        for (hipEvent_t e : ctx->ev_stop) (void)hipEventDestroy(e);
    }
    delete ctx;
    return AQ_OK;
}

aq_status aq_ctx_set_stream(aq_ctx *ctx, void *hip_stream) {
    if (!ctx) return AQ_E_INVALID_ARG;
    ctx->stream = static_cast<hipStream_t>(hip_stream);
    return AQ_OK;
}

aq_status aq_ctx_synchronize(aq_ctx *ctx) {
    if (!ctx) return AQ_E_INVALID_ARG;
    aq_device_guard g(ctx->device);
    AQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return AQ_OK;
}

const char *aq_last_error(const aq_ctx *ctx) {
    return ctx ? ctx->err.c_str() : "null context";
}

}  // extern "C"
