// Internal definitions shared by the C-ABI translation units.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "aq_mi355x.h"

struct aq_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string err;
    int32_t *d_flags = nullptr;   // device status words written by kernels (vector stores only)
    int num_cus = 0;
    // Work buffers owned by the context, grown on demand (slot 0: residual
    // cascade, 1: per-stage failure counters and lists, 2: projected queries,
    // 3: refine-pass keys, 4: sweep keys and frame norms, 5: gathered
    // strided input rows of a DAC encode, 6: exact values of the frames an
    // exact scan takes).
    static constexpr int kScratchSlots = 7;
    // Per-stage counters of the last Euclidean encode on this context (in
    // slot 1, or in the no-allocation scratch).
    int32_t *euclid_counts = nullptr;
    void *scratch[kScratchSlots] = {};
    size_t scratch_bytes[kScratchSlots] = {};
    // Kernel timing (aq_ctx_set_timing): event pairs around each main kernel.
    bool timing = false;
    std::vector<hipEvent_t> ev_start, ev_stop;
    size_t ev_used = 0;
};

// The event pair of the next timed launch (false when timing is off or the
// events cannot be created).
bool aq_timing_events(aq_ctx *ctx, hipEvent_t *start, hipEvent_t *stop);

// Launch of one of the timed kernels on ctx's stream.  With timing on (and
// `may_time`), the dispatch itself records the kernel's start and end
// (hipExtLaunchKernelGGL), so no event packets sit between the launches and
// the durations are the kernels' own; otherwise a plain launch.
template <typename F, typename... Args>
inline void aq_launch_timed(aq_ctx *ctx, bool may_time, F kernel, dim3 grid, dim3 block, uint32_t lds, Args... args) {
    hipEvent_t a = nullptr, b = nullptr;
    if (may_time && aq_timing_events(ctx, &a, &b))
        hipExtLaunchKernelGGL(kernel, grid, block, lds, ctx->stream, a, b, 0, args...);
    else
        hipLaunchKernelGGL(kernel, grid, block, lds, ctx->stream, args...);
}

// Device buffer `slot` of at least `bytes` (grows it, waiting for the stream
// first; bytes == 0 returns the current buffer, possibly null).
aq_status aq_ctx_scratch(aq_ctx *ctx, int slot, size_t bytes, void **out);

// LDS of a gfx950 compute unit: a block's static and dynamic LDS together
// must fit in it.  HIP does not reject a launch whose total exceeds it (the
// queue aborts instead), so every launch with dynamic LDS is checked first.
constexpr size_t kAqLdsBytes = 160 * 1024;
// Static LDS of kernel `fn` (hipFuncGetAttributes, cached per kernel; an
// unreadable attribute counts as the whole LDS, so the check fails).
size_t aq_static_lds(const void *fn);
// True when `dynamic` bytes of dynamic LDS fit next to fn's static LDS.
inline bool aq_lds_fits(const void *fn, size_t dynamic) {
    const size_t st = aq_static_lds(fn);
    return st <= kAqLdsBytes && dynamic <= kAqLdsBytes - st;
}

// LDS left for dynamic allocation next to fn's static LDS.
inline size_t aq_lds_budget(const void *fn) {
    const size_t st = aq_static_lds(fn);
    return st < kAqLdsBytes ? kAqLdsBytes - st : 0;
}
// Before a launch of fn with `dynamic` bytes of dynamic LDS on ctx's device:
// AQ_E_SHAPE (naming `what`) when it does not fit next to the kernel's
// static LDS, else raises the kernel's dynamic-LDS limit if needed (once
// per device and size, not per call).
aq_status aq_launch_lds(aq_ctx *ctx, const void *fn, size_t dynamic, const char *what);

// Sets `ctx->err` and returns `st`.
inline aq_status aq_fail(aq_ctx *ctx, aq_status st, const char *fmt, ...) {
    if (ctx) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        std::vsnprintf(buf, sizeof(buf), fmt, ap);
        va_end(ap);
        ctx->err = buf;
    }
    return st;
}

#define AQ_HIP(ctx, call)                                                                  \
    do {                                                                                   \
        hipError_t e_ = (call);                                                            \
        if (e_ != hipSuccess)                                                              \
            return aq_fail((ctx), AQ_E_DEVICE, "%s failed: %s", #call, hipGetErrorString(e_)); \
    } while (0)

// Makes ctx->device current for the lifetime of the guard, restoring the
// caller's device afterwards.  It also clears the thread's last-error slot,
// so that the hipGetLastError checks after this call's launches report
// this call's errors, not one the caller's own HIP calls left behind (a
// fault of earlier work stays visible: the launches and copies fail).
class aq_device_guard {
public:
    explicit aq_device_guard(int device) {
        (void)hipGetLastError();
        if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
        if (prev_ != device) (void)hipSetDevice(device);
    }
    ~aq_device_guard() {
        int cur = -1;
        if (prev_ >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev_) (void)hipSetDevice(prev_);
    }
    aq_device_guard(const aq_device_guard &) = delete;
    aq_device_guard &operator=(const aq_device_guard &) = delete;

private:
    int prev_ = -1;
};

// Indices of the device status words in ctx->d_flags.
enum aq_flag_slot : int {
    AQ_FLAG_BAD_INDEX = 0,   // a forced / decoded code outside [0, N)
    AQ_FLAG_COUNT = 8
};

// Host-loop DAC quantizers (aq_hostloop.hip).  Device pointers throughout.
struct aq_outetts_args {
    const float *x;        // [M, D]
    int64_t M;
    int D, N, Q;
    const float *w_in;     // [Q, 8, D]
    const float *b_in;     // [Q, 8]
    const float *chat;     // [Q, N, 8] normalised codes
    const float *cb;       // [Q, N, 8] raw codes
    const float *w_out;    // [Q, D, 8]
    const float *b_out;    // [Q, D]
    const int32_t *force_idx;
    int32_t *idx;          // [M, Q]
    float *residual;       // [M, D] or null
    int32_t *flags;
    int win_lds, chat_lds;   // set by aq_outetts_launch: stage tables staged in LDS
};
// chat[n] = c[n] / (sqrt(|c[n]|^2) + 1e-12) for `rows` codes of dim 8.
aq_status aq_outetts_prepare(aq_ctx *ctx, const float *d_cb, int64_t rows, float *d_chat);
aq_status aq_outetts_launch(aq_ctx *ctx, const aq_outetts_args &a);

struct aq_moss_args {
    double *res;           // [M, R] in / out
    int64_t M;
    int R, N, Q;
    const float *w_in;     // [Q, 8, R]
    const float *b_in;     // [Q, 8]
    const float *tn;       // [Q, N, 8] normalised codes
    const float *cb;       // [Q, N, 8] raw codes
    const float *w_out;    // [Q, R, 8]
    const float *b_out;    // [Q, R]
    const int32_t *force_idx;
    int32_t *idx;          // [M, Q]
    int32_t *flags;
    int write_res;
    int win_lds, tn_lds;     // set at launch: stage tables staged in LDS
};
