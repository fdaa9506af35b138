// Context management for the C ABI declared in include/aq_mi355x.h.
#include "aq_internal.hpp"

extern "C" {

int aq_abi_version(void) { return AQ_ABI_VERSION; }

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
        if (ctx->d_flags) (void)hipFree(ctx->d_flags);
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
