// Euclidean VQ / RVQ: host side of the C ABI (upload, encode, decode,
// gather) and the kernels that do not depend on the codebook width.  The
// kernels, the certificate and the reference recipes are described in
// aq_euclid_kernels.hpp.
#include "aq_euclid_kernels.hpp"
#include "aq_projected.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <vector>

namespace {

using namespace aq_euclid;

// --------------------------------------------------------------- gather, sum

// out[m] = cbf[stage][idx[m]] (get_rows; Q8_0 rows dequantised).
// Zeroes a[0, na) and b[0, nb) (the encode's counters and status words).  A
// kernel rather than hipMemsetAsync, so that a caller may capture the encode
// in a HIP graph: memset nodes have given wrong results on graph replays.
__global__ void zero2_kernel(int32_t *__restrict__ a, int na, int32_t *__restrict__ b, int nb) {
    for (int i = threadIdx.x; i < na; i += blockDim.x) a[i] = 0;
    for (int i = threadIdx.x; i < nb; i += blockDim.x) b[i] = 0;
}

// Per-stage counters of an any-width encode: no frame goes through a
// certificate ([0, 64) stay 0) and the exact scan decides all M ([64, 128)).
__global__ void any_counts_kernel(int32_t *__restrict__ c, int32_t m) {
    const int i = threadIdx.x;
    if (i < 128) c[i] = i < 64 ? 0 : m;
}

__global__ void gather_kernel(const float *__restrict__ cbf, int64_t N, int64_t K, const int32_t *__restrict__ idx,
                              int64_t M, float *__restrict__ out, int32_t *__restrict__ flags) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= M * K) return;
    const int64_t m = t / K, k = t % K;
    int32_t c = idx[m];
    if (c < 0 || c >= N) {
        flags[AQ_FLAG_BAD_INDEX] = 1;
        c = 0;
    }
    out[t] = cbf[static_cast<int64_t>(c) * K + k];
}

// out[m] = sum over stages of cbf[s][idx[m, s]] in stage order (-0 start).
__global__ void decode_sum_kernel(const float *__restrict__ cbf, int Q, int64_t N, int64_t K,
                                  const int32_t *__restrict__ idx, int64_t M, float *__restrict__ out,
                                  int32_t *__restrict__ flags) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= M * K) return;
    const int64_t m = t / K, k = t % K;
    float acc = -0.0f;
    for (int s = 0; s < Q; ++s) {
        int32_t c = idx[m * Q + s];
        if (c < 0 || c >= N) {
            flags[AQ_FLAG_BAD_INDEX] = 1;
            c = 0;
        }
        acc = __fadd_rn(acc, cbf[(static_cast<int64_t>(s) * N + c) * K + k]);
    }
    out[t] = acc;
}

// codebook[q,n,k] = embedding_sum[q,n,k] / std::max(usage[q,n], eps): the
// max is (u < eps) ? eps : u, so a NaN usage stays NaN; IEEE division.
__global__ void ema_codebook_kernel(const float *__restrict__ esum, const float *__restrict__ usage, int64_t QN,
                                    int64_t K, float eps, float *__restrict__ out) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= QN * K) return;
    const float u = usage[t / K];
    const float denom = u < eps ? eps : u;
    out[t] = __fdiv_rn(esum[t], denom);
}

// ------------------------------------------------------ codebook preparation

// block_q8_0 rows {fp16 d; int8 qs[32]} (ggml-common.h:241-246) -> quants,
// scales and the dequantised codebook q * d (ggml-quants.c:491-505; the
// product is exact in fp32).  One thread per element.
__global__ void q8_unpack_kernel(const unsigned char *__restrict__ raw, int64_t nblocks, int8_t *__restrict__ qs,
                                 float *__restrict__ qd, float *__restrict__ cbf) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= nblocks * 32) return;
    const int64_t b = t / 32;
    const int j = static_cast<int>(t % 32);
    const unsigned char *p = raw + b * 34;
    const uint16_t h = static_cast<uint16_t>(p[0] | (p[1] << 8));
    const float d = static_cast<float>(__builtin_bit_cast(_Float16, h));
    const int8_t q = static_cast<int8_t>(p[2 + j]);
    qs[t] = q;
    cbf[t] = __fmul_rn(static_cast<float>(q), d);
    if (j == 0) qd[b] = d;
}

// F32 rows quantised to Q8_0 the way the reference's weight store does at
// load (ggml_quantize_chunk -> quantize_row_q8_0_ref, ggml-quants.c:236-256;
// backend_weight_store.h:343-392, tensor_source.cpp:173-200): per 32-block
// amax = MAX(amax, |x|) (C's MAX: a NaN is passed over by the next value),
// d = amax / 127, id = d ? 1 / d : 0 in fp32, q = roundf(x * id), the scale
// stored as fp16(d).  Writes the quants, the scales and q * d.  One thread
// per block.
__global__ void q8_quantize_kernel(const float *__restrict__ x, int64_t nblocks, int8_t *__restrict__ qs,
                                   float *__restrict__ qd, float *__restrict__ cbf) {
    const int64_t b = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const float *xb = x + b * 32;
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) {
        const float a = fabsf(xb[j]);
        amax = amax > a ? amax : a;
    }
    const float d = __fdiv_rn(amax, 127.0f);
    const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    const float ds = static_cast<float>(static_cast<_Float16>(d));
    qd[b] = ds;
    for (int j = 0; j < 32; ++j) {
        const int8_t q = static_cast<int8_t>(static_cast<int>(roundf(__fmul_rn(xb[j], id))));
        qs[b * 32 + j] = q;
        cbf[b * 32 + j] = __fmul_rn(static_cast<float>(q), ds);
    }
}

// fp16 images, round to nearest even.
__device__ inline uint16_t img_half(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f)); }
__device__ inline float img_float(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }

// Per code row (one thread each): the matrix-core images c_h = fp16(c) and
// c_l = fp16(c - c_h), the per-code
// constants -|c|^2 / 2 (sweep), -|c|^2 (OmniVoice bias, double sum of double
// products) and sum_rows(c * c) (Higgs: fp32 squares summed in double), and
// per stage the largest |c|, |c_h - c|, |c_h|, |c_l| and |c - c_h - c_l|
// (as double bit patterns, atomicMax over non-negative values; NaN skipped)
// for the certificate's bounds.  nonfinite[0] = 1 on any non-finite entry
// or one beyond fp16's range (the stage is then scanned exactly).
__global__ void euclid_prep_kernel(const float *__restrict__ cbf, int64_t QN, int64_t N, int K,
                                   uint16_t *__restrict__ cbh, uint16_t *__restrict__ cbl, float *__restrict__ hh,
                                   float *__restrict__ bias, float *__restrict__ e2,
                                   unsigned long long *__restrict__ smax, int32_t *__restrict__ nonfinite) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r >= QN) return;
    const int64_t row = r * K;
    double sq = 0.0, dq = 0.0, hq = 0.0, e2d = 0.0, lq = 0.0, rq = 0.0;
    bool nf = false;
    for (int k = 0; k < K; ++k) {
        const float c = cbf[row + k];
        const uint16_t h = img_half(c);
        cbh[row + k] = h;
        const float hf = img_float(h);
        nf |= !__builtin_isfinite(hf);
        // c - c_h and c - c_h - c_l are exact in fp32 (finite c)
        const float dl = __fsub_rn(c, hf);
        const uint16_t l = __builtin_isfinite(dl) ? img_half(dl) : 0;
        cbl[row + k] = l;
        const double ld = img_float(l), rd = __dsub_rn(static_cast<double>(dl), ld);
        const double cd = c, hd = hf, dd = __dsub_rn(hd, cd);
        sq = __dadd_rn(sq, __dmul_rn(cd, cd));
        e2d = __dadd_rn(e2d, static_cast<double>(__fmul_rn(c, c)));
        dq = __dadd_rn(dq, __dmul_rn(dd, dd));
        hq = __dadd_rn(hq, __dmul_rn(hd, hd));
        lq = __dadd_rn(lq, __dmul_rn(ld, ld));
        rq = __dadd_rn(rq, __dmul_rn(rd, rd));
    }
    hh[r] = static_cast<float>(__dmul_rn(-0.5, sq));
    bias[r] = static_cast<float>(-sq);
    e2[r] = static_cast<float>(e2d);
    const int64_t s = r / N;
    const double norms[5] = {sqrt(sq), sqrt(dq), sqrt(hq), sqrt(lq), sqrt(rq)};
    for (int i = 0; i < 5; ++i)
        if (norms[i] == norms[i]) atomicMax(&smax[s * 5 + i], static_cast<unsigned long long>(__double_as_longlong(norms[i])));
    if (nf) nonfinite[0] = 1;
}

// --------------------------------------------------------------- dispatch

const KsKernels *kernels_for(int ks) {
    switch (ks) {
        case 2: return kernels_ks2();
        case 8: return kernels_ks8();
        case 16: return kernels_ks16();
        case 24: return kernels_ks24();
        default: return nullptr;
    }
}

// Recipe variant index of KsKernels.
int variant_of(int recipe, bool q8) { return q8 ? 3 : recipe; }

float round_up(double v) {
    float f = static_cast<float>(v);
    if (static_cast<double>(f) < v) f = std::nextafter(f, INFINITY);
    return f;
}

}  // namespace

struct aq_codebooks {
    // device of the creating context (the handle keeps no pointer to it, so
    // it may be released after that context is destroyed)
    int device = -1;
    int64_t Q = 0, N = 0, K = 0;
    int recipe = 0;
    bool q8 = false;
    bool exact_only = false;
    // A width or size outside the fast kernels' (K in {64, 256, 512, 768},
    // N a multiple of their chunk): every frame is scanned exactly.
    bool any = false;
    uint16_t *d_cbh = nullptr;   // [Q][N][K] fp16(c)
    uint16_t *d_cbl = nullptr;   // [Q][N][K] fp16(c - fp16(c)) (refine pass)
    float *d_hh = nullptr;       // [Q][N] -|c|^2 / 2 (fp32 of the double sum)
    float *d_cbf = nullptr;      // [Q][N][K]
    float *d_bias = nullptr;     // [Q][N] (OMNI)
    float *d_e2 = nullptr;       // [Q][N] (HIGGS)
    int8_t *d_q8 = nullptr;      // [Q][N][K]
    float *d_q8d = nullptr;      // [Q][N][K/32]
    float *d_bounds = nullptr;   // [Q][3] max |c|, max |c~ - c|, max |c~| (the cascade kernel's certificate)
    std::vector<float> cmax, dcmax, chmax;
    std::vector<float> clmax, crmax;   // max |c_l|, max |c - c_h - c_l| (refine bound)
    aq_proj_weights *proj = nullptr;   // project_in / project_out (projected cascades)
};

namespace {

// Largest codebook width of the any-width path (the exact scan stages the
// frame, its Q8_0 image and scales in LDS) and largest codebook size of
// either path (codes are int32; the fast path keys carry 20 index bits).
constexpr int64_t kAnyMaxK = 16384;
constexpr int64_t kAnyMaxN = int64_t{1} << 24;
constexpr int64_t kFastMaxN = int64_t{1} << 20;

// Shape and type checks shared by the uploads.  *any: the shape takes the
// any-width exact path (every width and size the reference accepts; GGUF
// Q8_0 rows are whole 32-element blocks).
aq_status check_upload(aq_ctx *ctx, const char *fn, int64_t Q, int64_t N, int64_t K, int cb_type, int recipe,
                       bool *any) {
    if (recipe < AQ_EUCLID_OMNIVOICE || recipe > AQ_EUCLID_DIRECT)
        return aq_fail(ctx, AQ_E_INVALID_ARG, "%s: unknown recipe %d", fn, recipe);
    if (cb_type != AQ_CB_F32 && cb_type != AQ_CB_Q8_0 && cb_type != AQ_CB_F32_AS_Q8_0)
        return aq_fail(ctx, AQ_E_INVALID_ARG, "%s: unknown codebook type %d", fn, cb_type);
    if (cb_type != AQ_CB_F32 && recipe != AQ_EUCLID_HIGGS)
        return aq_fail(ctx, AQ_E_UNSUPPORTED, "%s: Q8_0 codebooks follow the Higgs recipe only", fn);
    if (Q <= 0 || N <= 0 || K <= 0)
        return aq_fail(ctx, AQ_E_SHAPE, "%s: empty shape Q=%lld N=%lld K=%lld", fn, (long long)Q, (long long)N,
                       (long long)K);
    if (cb_type != AQ_CB_F32 && K % 32 != 0)
        return aq_fail(ctx, AQ_E_SHAPE, "%s: Q8_0 rows of K=%lld are not whole 32-element blocks", fn, (long long)K);
    const KsKernels *kk = K % 32 == 0 ? kernels_for(static_cast<int>(K / 32)) : nullptr;
    *any = !kk || N % kk->cc != 0 || N > kFastMaxN;
    if (*any && (K > kAnyMaxK || N > kAnyMaxN))
        return aq_fail(ctx, AQ_E_SHAPE, "%s: K=%lld N=%lld exceed the supported %lld x %lld", fn, (long long)K,
                       (long long)N, (long long)kAnyMaxK, (long long)kAnyMaxN);
    return AQ_OK;
}

// A codebook set with its device buffers allocated, not yet filled.
aq_status euclid_alloc(aq_ctx *ctx, int64_t Q, int64_t N, int64_t K, bool q8, int recipe, aq_codebooks **out) {
    aq_codebooks *cb = new (std::nothrow) aq_codebooks();
    if (!cb) return aq_fail(ctx, AQ_E_NOMEM, "aq_euclid_upload: host allocation failed");
    cb->device = ctx->device;
    cb->Q = Q;
    cb->N = N;
    cb->K = K;
    cb->recipe = recipe;
    cb->q8 = q8;
    const size_t QNK = static_cast<size_t>(Q * N * K), QN = static_cast<size_t>(Q * N);
    bool ok = hipMalloc(&cb->d_cbh, QNK * 2) == hipSuccess && hipMalloc(&cb->d_cbl, QNK * 2) == hipSuccess &&
              hipMalloc(&cb->d_hh, QN * 4) == hipSuccess && hipMalloc(&cb->d_cbf, QNK * 4) == hipSuccess &&
              hipMalloc(&cb->d_bias, QN * 4) == hipSuccess && hipMalloc(&cb->d_e2, QN * 4) == hipSuccess;
    if (ok && q8) ok = hipMalloc(&cb->d_q8, QNK) == hipSuccess && hipMalloc(&cb->d_q8d, QNK / 32 * 4) == hipSuccess;
    if (!ok) {
        aq_euclid_release(cb);
        return aq_fail(ctx, AQ_E_NOMEM, "aq_euclid_upload: device allocation failed");
    }
    *out = cb;
    return AQ_OK;
}

// Fills the codebook (d_cbf; for Q8_0 also the quants and scales) from
// `data` in host or device memory (F32 [Q][N][K], or block_q8_0 rows; F32
// rows for AQ_CB_F32_AS_Q8_0, quantised here).
aq_status euclid_fill(aq_ctx *ctx, aq_codebooks *cb, int cb_type, const void *data, hipMemcpyKind kind) {
    const size_t QNK = static_cast<size_t>(cb->Q * cb->N * cb->K);
    if (!cb->q8) {
        AQ_HIP(ctx, hipMemcpyAsync(cb->d_cbf, data, QNK * 4, kind, ctx->stream));
        return AQ_OK;
    }
    if (cb_type == AQ_CB_F32_AS_Q8_0) {
        float *f = nullptr;
        if (hipMalloc(&f, QNK * 4) != hipSuccess) return aq_fail(ctx, AQ_E_NOMEM, "aq_euclid_upload: device allocation failed");
        aq_status st = AQ_OK;
        if (hipMemcpyAsync(f, data, QNK * 4, kind, ctx->stream) != hipSuccess) {
            st = aq_fail(ctx, AQ_E_DEVICE, "aq_euclid_upload: copy of the codebook failed");
        } else {
            hipLaunchKernelGGL(q8_quantize_kernel, dim3(static_cast<unsigned>((QNK / 32 + 127) / 128)), dim3(128), 0,
                               ctx->stream, f, static_cast<int64_t>(QNK / 32), cb->d_q8, cb->d_q8d, cb->d_cbf);
            if (hipGetLastError() != hipSuccess || hipStreamSynchronize(ctx->stream) != hipSuccess)
                st = aq_fail(ctx, AQ_E_DEVICE, "aq_euclid_upload: Q8_0 quantisation failed");
        }
        (void)hipFree(f);
        return st;
    }
    const size_t nblocks = QNK / 32;
    unsigned char *raw = nullptr;
    if (hipMalloc(&raw, nblocks * 34) != hipSuccess)
        return aq_fail(ctx, AQ_E_NOMEM, "aq_euclid_upload: device allocation failed");
    aq_status st = AQ_OK;
    if (hipMemcpyAsync(raw, data, nblocks * 34, kind, ctx->stream) != hipSuccess) {
        st = aq_fail(ctx, AQ_E_DEVICE, "aq_euclid_upload: copy of the Q8_0 blocks failed");
    } else {
        hipLaunchKernelGGL(q8_unpack_kernel, dim3(static_cast<unsigned>((QNK + 255) / 256)), dim3(256), 0, ctx->stream,
                           raw, static_cast<int64_t>(nblocks), cb->d_q8, cb->d_q8d, cb->d_cbf);
        if (hipGetLastError() != hipSuccess || hipStreamSynchronize(ctx->stream) != hipSuccess)
            st = aq_fail(ctx, AQ_E_DEVICE, "aq_euclid_upload: Q8_0 unpack failed");
    }
    (void)hipFree(raw);
    return st;
}

// Builds the matrix-core images, the per-code constants and the
// certificate's per-stage bounds from d_cbf on the device; only the 5 * Q
// stage maxima and the non-finite flag come back to the host.
aq_status euclid_prepare(aq_ctx *ctx, aq_codebooks *cb) {
    const int64_t QN = cb->Q * cb->N;
    unsigned long long *smax = nullptr;
    if (hipMalloc(&smax, sizeof(unsigned long long) * (5 * cb->Q + 1)) != hipSuccess)
        return aq_fail(ctx, AQ_E_NOMEM, "aq_euclid_upload: device allocation failed");
    int32_t *nonfinite = reinterpret_cast<int32_t *>(smax + 5 * cb->Q);
    std::vector<unsigned long long> host(5 * cb->Q + 1, 0);
    aq_status st = AQ_OK;
    const char *step = "memset";
    hipError_t e = hipMemsetAsync(smax, 0, sizeof(unsigned long long) * (5 * cb->Q + 1), ctx->stream);
    if (e == hipSuccess) {
        const dim3 grid(static_cast<unsigned>((QN + 127) / 128)), block(128);
        hipLaunchKernelGGL(euclid_prep_kernel, grid, block, 0, ctx->stream, cb->d_cbf, QN, cb->N,
                           static_cast<int>(cb->K), cb->d_cbh, cb->d_cbl, cb->d_hh, cb->d_bias, cb->d_e2, smax,
                           nonfinite);
        step = "launch";
        e = hipGetLastError();
        if (e == hipSuccess) {
            step = "copy";
            e = hipMemcpyAsync(host.data(), smax, sizeof(unsigned long long) * host.size(), hipMemcpyDeviceToHost,
                               ctx->stream);
        }
        if (e == hipSuccess) {
            step = "synchronize";
            e = hipStreamSynchronize(ctx->stream);
        }
    }
    (void)hipFree(smax);
    if (e != hipSuccess)
        return aq_fail(ctx, AQ_E_DEVICE, "aq_euclid_upload: codebook preparation failed (%s: %s)", step,
                       hipGetErrorString(e));
    auto bound = [&](int64_t s, int i) {
        double v;
        std::memcpy(&v, &host[s * 5 + i], 8);
        return round_up(v * (1.0 + 1e-6));
    };
    cb->cmax.resize(cb->Q);
    cb->dcmax.resize(cb->Q);
    cb->chmax.resize(cb->Q);
    cb->clmax.resize(cb->Q);
    cb->crmax.resize(cb->Q);
    for (int64_t s = 0; s < cb->Q; ++s) {
        cb->cmax[s] = bound(s, 0);
        cb->dcmax[s] = bound(s, 1);
        cb->chmax[s] = bound(s, 2);
        cb->clmax[s] = bound(s, 3);
        cb->crmax[s] = bound(s, 4);
    }
    int32_t nf;
    std::memcpy(&nf, &host[5 * cb->Q], 4);
    cb->exact_only = nf != 0;
    // the per-stage bounds on the device, for the one-launch cascade
    std::vector<float> b3(static_cast<size_t>(3 * cb->Q));
    for (int64_t s = 0; s < cb->Q; ++s) {
        b3[3 * s] = cb->cmax[s];
        b3[3 * s + 1] = cb->dcmax[s];
        b3[3 * s + 2] = cb->chmax[s];
    }
    if (!cb->d_bounds && hipMalloc(&cb->d_bounds, b3.size() * sizeof(float)) != hipSuccess)
        return aq_fail(ctx, AQ_E_NOMEM, "aq_euclid_upload: device allocation failed");
    AQ_HIP(ctx, hipMemcpyAsync(cb->d_bounds, b3.data(), b3.size() * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
    AQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return st;
}

aq_status euclid_upload_from(aq_ctx *ctx, const char *fn, int64_t Q, int64_t N, int64_t K, int cb_type,
                             const void *data, hipMemcpyKind kind, int recipe, aq_codebooks **out) {
    if (!ctx || !out || !data) return aq_fail(ctx, AQ_E_INVALID_ARG, "%s: null argument", fn);
    *out = nullptr;
    bool any = false;
    aq_status st = check_upload(ctx, fn, Q, N, K, cb_type, recipe, &any);
    if (st != AQ_OK) return st;
    aq_device_guard g(ctx->device);
    aq_codebooks *cb = nullptr;
    st = euclid_alloc(ctx, Q, N, K, cb_type != AQ_CB_F32, recipe, &cb);
    if (st == AQ_OK) cb->any = any;
    if (st == AQ_OK) st = euclid_fill(ctx, cb, cb_type, data, kind);
    if (st == AQ_OK) st = euclid_prepare(ctx, cb);
    if (st != AQ_OK) {
        if (cb) aq_euclid_release(cb);
        return st;
    }
    *out = cb;
    return AQ_OK;
}

}  // namespace

extern "C" {

aq_status aq_euclid_upload(aq_ctx *ctx, int64_t Q, int64_t N, int64_t K, int cb_type, const void *data, int recipe,
                           aq_codebooks **out) {
    return euclid_upload_from(ctx, "aq_euclid_upload", Q, N, K, cb_type, data, hipMemcpyHostToDevice, recipe, out);
}

aq_status aq_euclid_upload_device(aq_ctx *ctx, int64_t Q, int64_t N, int64_t K, int cb_type, const void *data,
                                  int recipe, aq_codebooks **out) {
    return euclid_upload_from(ctx, "aq_euclid_upload_device", Q, N, K, cb_type, data, hipMemcpyDeviceToDevice, recipe,
                              out);
}

aq_status aq_ema_codebook(aq_ctx *ctx, const float *embedding_sum, const float *cluster_usage, int64_t Q, int64_t N,
                          int64_t K, float eps, float *codebook) {
    if (!ctx || !embedding_sum || !cluster_usage || !codebook)
        return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_ema_codebook: null argument");
    if (Q <= 0 || N <= 0 || K <= 0) return aq_fail(ctx, AQ_E_SHAPE, "aq_ema_codebook: empty shape");
    aq_device_guard g(ctx->device);
    const int64_t total = Q * N * K;
    hipLaunchKernelGGL(ema_codebook_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, ctx->stream,
                       embedding_sum, cluster_usage, Q * N, K, eps, codebook);
    AQ_HIP(ctx, hipGetLastError());
    return AQ_OK;
}

aq_status aq_euclid_upload_ema(aq_ctx *ctx, int64_t Q, int64_t N, int64_t K, const float *embedding_sum,
                               const float *cluster_usage, float eps, int recipe, aq_codebooks **out) {
    if (!ctx || !out || !embedding_sum || !cluster_usage)
        return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_euclid_upload_ema: null argument");
    *out = nullptr;
    bool any = false;
    aq_status st = check_upload(ctx, "aq_euclid_upload_ema", Q, N, K, AQ_CB_F32, recipe, &any);
    if (st != AQ_OK) return st;
    aq_device_guard g(ctx->device);
    const size_t QNK = static_cast<size_t>(Q * N * K), QN = static_cast<size_t>(Q * N);
    aq_codebooks *cb = nullptr;
    st = euclid_alloc(ctx, Q, N, K, false, recipe, &cb);
    if (st != AQ_OK) return st;
    cb->any = any;
    // the inputs go to the device once; the codebook is materialised straight
    // into the set's fp32 buffer and prepared there
    float *d = nullptr;
    if (hipMalloc(&d, (QNK + QN) * sizeof(float)) != hipSuccess) {
        aq_euclid_release(cb);
        return aq_fail(ctx, AQ_E_NOMEM, "aq_euclid_upload_ema: device allocation failed");
    }
    if (hipMemcpyAsync(d, embedding_sum, QNK * 4, hipMemcpyHostToDevice, ctx->stream) != hipSuccess ||
        hipMemcpyAsync(d + QNK, cluster_usage, QN * 4, hipMemcpyHostToDevice, ctx->stream) != hipSuccess)
        st = aq_fail(ctx, AQ_E_DEVICE, "aq_euclid_upload_ema: host to device copy failed");
    if (st == AQ_OK) st = aq_ema_codebook(ctx, d, d + QNK, Q, N, K, eps, cb->d_cbf);
    if (st == AQ_OK) st = euclid_prepare(ctx, cb);
    (void)hipFree(d);
    if (st != AQ_OK) {
        aq_euclid_release(cb);
        return st;
    }
    *out = cb;
    return AQ_OK;
}

aq_status aq_euclid_upload_projected(aq_ctx *ctx, int64_t Q, int64_t N, int64_t K, int64_t H, int cb_type,
                                     const void *codebook, int proj_type, const void *w_in, const float *b_in,
                                     const void *w_out, const float *b_out, int recipe, aq_codebooks **out) {
    if (!ctx || !out || !codebook || !w_in || !w_out)
        return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_euclid_upload_projected: null argument");
    *out = nullptr;
    if (recipe != AQ_EUCLID_OMNIVOICE && recipe != AQ_EUCLID_HIGGS)
        return aq_fail(ctx, AQ_E_UNSUPPORTED, "aq_euclid_upload_projected: projections follow the OmniVoice and Higgs recipes");
    if (proj_type != AQ_CB_F32 && proj_type != AQ_CB_Q8_0)
        return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_euclid_upload_projected: unknown weight type %d", proj_type);
    if (H <= 0 || H % 64 != 0)
        return aq_fail(ctx, AQ_E_SHAPE, "aq_euclid_upload_projected: hidden size H=%lld (a multiple of 64 up to %d)",
                       (long long)H, proj_type == AQ_CB_Q8_0 ? 1984 : 2496);
    {
        // the projection block keeps 16 residual rows of H + 1 floats in LDS
        // (plus their Q8_0 image for Q8_0 weights)
        aq_status ls = aq_proj_check_lds(ctx, H, proj_type == AQ_CB_Q8_0, "aq_euclid_upload_projected");
        if (ls != AQ_OK) return ls;
    }
    aq_codebooks *cb = nullptr;
    aq_status st = aq_euclid_upload(ctx, Q, N, K, cb_type, codebook, recipe, &cb);
    if (st != AQ_OK) return st;
    if (cb->any) {
        aq_euclid_release(cb);
        return aq_fail(ctx, AQ_E_SHAPE,
                       "aq_euclid_upload_projected: codebook shape N=%lld K=%lld (K in {64,256,512,768}, N a multiple of "
                       "the chunk)", (long long)N, (long long)K);
    }
    aq_device_guard g(ctx->device);
    st = aq_proj_create(ctx, Q, N, K, H, cb->d_cbf, proj_type, w_in, b_in, w_out, b_out, &cb->proj);
    if (st != AQ_OK) {
        aq_euclid_release(cb);
        return st;
    }
    *out = cb;
    return AQ_OK;
}

aq_status aq_euclid_release(aq_codebooks *cb) {
    if (!cb) return AQ_E_INVALID_ARG;
    {
        aq_device_guard g(cb->device);
        aq_proj_release(cb->proj);
        for (void *p : {static_cast<void *>(cb->d_cbh), static_cast<void *>(cb->d_cbl), static_cast<void *>(cb->d_hh),
                        static_cast<void *>(cb->d_cbf),
                        static_cast<void *>(cb->d_bias), static_cast<void *>(cb->d_e2), static_cast<void *>(cb->d_q8),
                        static_cast<void *>(cb->d_q8d), static_cast<void *>(cb->d_bounds)})
            if (p) (void)hipFree(p);
    }
    delete cb;
    return AQ_OK;
}

}  // extern "C"

namespace {

// Work buffers of one encode: the context's growable buffers (base null), or
// consecutive 256-byte aligned pieces of a fixed device region (the
// no-allocation entry point).
struct Arena {
    aq_ctx *ctx;
    unsigned char *base;
    size_t cap, used;
    aq_status get(int slot, size_t bytes, void **out) {
        if (!base) return aq_ctx_scratch(ctx, slot, bytes, out);
        const size_t off = (used + 255) & ~size_t{255};
        if (off > cap || bytes > cap - off)
            return aq_fail(ctx, AQ_E_SHAPE,
                           "aq_euclid_encode_noalloc: the encode needs more than the %zu bytes of scratch "
                           "(pass a residual buffer or encode fewer frames per call)", cap);
        *out = base + off;
        used = off + bytes;
        return AQ_OK;
    }
    // bytes still free (for the growable buffers: unbounded)
    size_t left() const {
        if (!base) return ~size_t{0};
        const size_t off = (used + 255) & ~size_t{255};
        return off < cap ? cap - off : 0;
    }
};

// Scratch of aq_euclid_encode_noalloc: every call on a device uses this one
// region (the device holds it until the process ends), so calls that overlap
// on one device race.  Host code never uses the name `scratch` as an
// address: each device's address comes from hipGetSymbolAddress.
constexpr size_t kNoAllocBytes = size_t{32} << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];
constexpr int kNoAllocDevices = 64;
std::mutex g_noalloc_mu;
void *g_noalloc_ptr[kNoAllocDevices];
// Calls on one device are ordered through one event per device: each call's
// stream waits for the previous call's work, which records the event after
// it (the host enqueues one call at a time per device).  Calls captured
// into a HIP graph are not ordered by it.
std::mutex g_noalloc_call_mu[kNoAllocDevices];
hipEvent_t g_noalloc_done[kNoAllocDevices];

// The device address of `scratch` on ctx's device (current when called),
// looked up on the first call on that device.
aq_status noalloc_region(aq_ctx *ctx, unsigned char **out) {
    if (ctx->device < 0 || ctx->device >= kNoAllocDevices)
        return aq_fail(ctx, AQ_E_UNSUPPORTED, "aq_euclid_encode_noalloc: device %d out of range", ctx->device);
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc_ptr[ctx->device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return aq_fail(ctx, AQ_E_DEVICE, "aq_euclid_encode_noalloc: hipGetSymbolAddress failed: %s",
                           hipGetErrorString(e));
        hipEvent_t ev = nullptr;
        const hipError_t e2 = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e2 != hipSuccess)
            return aq_fail(ctx, AQ_E_DEVICE, "aq_euclid_encode_noalloc: hipEventCreate failed: %s", hipGetErrorString(e2));
        g_noalloc_done[ctx->device] = ev;
        g_noalloc_ptr[ctx->device] = p;
    }
    *out = static_cast<unsigned char *>(g_noalloc_ptr[ctx->device]);
    return AQ_OK;
}

// Encode on an any-width codebook set: per stage, the exact scan of every
// frame in the recipe's arithmetic (the run-time-width exact scan, one block
// per frame), with the residual cascade r -= c[code] in between.
aq_status euclid_encode_any(aq_ctx *ctx, const aq_codebooks *cb, const aq_frames_desc &in, int64_t M, int32_t *idx,
                            float *residual, float *dist, int topk, int32_t *topk_idx, float *topk_dist,
                            const int32_t *force_idx, Arena &arena) {
    const int64_t K = cb->K;
    StageFn scan = kernels_any()->exact_scan[variant_of(cb->recipe, cb->q8)];
    const size_t lds = scan_lds_bytes(K);
    {
        aq_status ls = aq_launch_lds(ctx, reinterpret_cast<const void *>(scan), lds, "aq_euclid_encode (exact scan)");
        if (ls != AQ_OK) return ls;
    }
    float *work = residual;
    if (!work) {
        aq_status st = arena.get(0, static_cast<size_t>(M) * K * sizeof(float), reinterpret_cast<void **>(&work));
        if (st != AQ_OK) return st;
    }
    int32_t *counts = nullptr;
    {
        aq_status st = arena.get(1, 128 * sizeof(int32_t), reinterpret_cast<void **>(&counts));
        if (st != AQ_OK) return st;
    }
    ctx->euclid_counts = counts;
    hipLaunchKernelGGL(any_counts_kernel, dim3(1), dim3(128), 0, ctx->stream, counts, static_cast<int32_t>(M));
    AQ_HIP(ctx, hipGetLastError());
    hipLaunchKernelGGL(zero2_kernel, dim3(1), dim3(64), 0, ctx->stream, ctx->d_flags, static_cast<int>(AQ_FLAG_COUNT),
                       ctx->d_flags, 0);
    AQ_HIP(ctx, hipGetLastError());
    const float *x0 = in.x;
    const bool row_major = in.frame_stride == K && in.chan_stride == 1 && (in.clip_len >= M || in.clip_stride == in.clip_len * K);
    if (!row_major) {
        aq_status st = aq_gather_frames(ctx, in, M, K, work);
        if (st != AQ_OK) return st;
        x0 = work;
    }
    const int cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>(M, int64_t{8} * cus));
    for (int64_t s = 0; s < cb->Q; ++s) {
        StageArgs a{};
        a.xin = s == 0 ? x0 : work;
        a.xout = (s + 1 < cb->Q || residual) ? work : nullptr;
        a.M = M;
        a.N = static_cast<int>(cb->N);
        a.K = static_cast<int>(K);
        a.cbf = cb->d_cbf + s * cb->N * K;
        a.bias = cb->d_bias + s * cb->N;
        a.e2 = cb->d_e2 + s * cb->N;
        a.q8 = cb->q8 ? cb->d_q8 + s * cb->N * K : nullptr;
        a.q8d = cb->q8 ? cb->d_q8d + s * cb->N * (K / 32) : nullptr;
        // ggml's choice between tinyBLAS and ggml_vec_dot_f32 (see run_stage)
        a.order = (M >= 2 && K % 16 == 0 && cb->N % 4 == 0) ? 0 : 1;
        a.Q = static_cast<int>(cb->Q);
        a.s = static_cast<int>(s);
        a.idx = idx;
        a.dist = dist;
        a.topk = topk;
        a.topk_idx = topk_idx;
        a.topk_dist = topk_dist;
        a.force_idx = force_idx;
        a.flags = ctx->d_flags;
        aq_launch_timed(ctx, !arena.base, scan, dim3(grid), dim3(kScanThreads), static_cast<uint32_t>(lds), a);
        AQ_HIP(ctx, hipGetLastError());
    }
    if (force_idx) {
        int32_t flag = 0;
        AQ_HIP(ctx, hipMemcpyAsync(&flag, ctx->d_flags + AQ_FLAG_BAD_INDEX, sizeof(int32_t), hipMemcpyDeviceToHost, ctx->stream));
        AQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (flag) return aq_fail(ctx, AQ_E_INDEX_RANGE, "aq_euclid_encode: force_idx holds a code outside [0, %lld)", (long long)cb->N);
    }
    return AQ_OK;
}

// The encode pipeline of a plain codebook: the register-resident one-launch
// cascade where it exists (K = 256), else the per-stage pipeline.  The
// one-launch cascade that keeps the residual in memory measured no faster
// than the per-stage pipeline at K = 256 and slower for Q8_0 codebooks (its
// verification then scans 2-3 % of the frames); it runs when
// AQ_EUCLID_PIPELINE=cascade asks for it (comparisons and tests), as
// AQ_EUCLID_PIPELINE=stages asks for the per-stage pipeline.
enum class Pipeline { kStages, kCascade, kResident };
Pipeline pipeline_for(const aq_codebooks *cb, const KsKernels *kk, int var, int topl) {
    if (cb->proj || cb->exact_only || !kk->cascade[var][topl - 3]) return Pipeline::kStages;
    const char *e = std::getenv("AQ_EUCLID_PIPELINE");
    if (e && std::strcmp(e, "stages") == 0) return Pipeline::kStages;
    if (e && std::strcmp(e, "cascade") == 0) return Pipeline::kCascade;
    return kk->resident[var][topl - 3] ? Pipeline::kResident : Pipeline::kStages;
}

// Encode with a one-launch cascade: every stage of every frame in
// euclid_resident_kernel (resident) or euclid_cascade_kernel (frames the
// certificate cannot settle continue with their best exact candidate and
// are listed), the exact verification of the listed (frame, stage) pairs
// (their values spread over the grid, then the selections), and the fix-up
// of frames whose continuation was wrong.  Five launches per encode,
// whatever the number of stages.
aq_status euclid_encode_cascade(aq_ctx *ctx, const aq_codebooks *cb, const aq_frames_desc &in, int64_t M, int32_t *idx,
                                float *residual, float *dist, int topk, int32_t *topk_idx, float *topk_dist,
                                const int32_t *force_idx, Arena &arena, const KsKernels *kk, int var, int topl,
                                bool resident) {
    const int K = static_cast<int>(cb->K);
    CascadeFn casc = kk->cascade[var][topl - 3], ver = kk->verify[var], fix = kk->fixup[var];
    CascadeFn vvals = kk->verify_values[var];
    size_t clds = static_cast<size_t>(kk->cascade_lds);
    int frames = kk->cascade_frames, threads = kCThreads;
    if (resident) {
        casc = kk->resident[var][topl - 3];
        clds = static_cast<size_t>(kk->resident_lds);
        frames = kk->resident_frames;
        threads = kRsThreads;
    }
    const size_t slds = scan_lds_bytes(K);
    {
        aq_status ls = aq_launch_lds(ctx, reinterpret_cast<const void *>(casc), clds, "aq_euclid_encode (cascade)");
        if (ls == AQ_OK) ls = aq_launch_lds(ctx, reinterpret_cast<const void *>(ver), slds, "aq_euclid_encode (verify)");
        if (ls == AQ_OK)
            ls = aq_launch_lds(ctx, reinterpret_cast<const void *>(vvals), slds, "aq_euclid_encode (verify values)");
        if (ls == AQ_OK) ls = aq_launch_lds(ctx, reinterpret_cast<const void *>(fix), slds, "aq_euclid_encode (fix-up)");
        if (ls != AQ_OK) return ls;
    }
    float *work = residual;
    if (!work) {
        aq_status st = arena.get(0, static_cast<size_t>(M) * K * sizeof(float), reinterpret_cast<void **>(&work));
        if (st != AQ_OK) return st;
    }
    // the stage-0 input stays intact for the verification: a strided input
    // is gathered into a buffer of its own
    const float *x0 = in.x;
    const bool row_major = in.frame_stride == K && in.chan_stride == 1 && (in.clip_len >= M || in.clip_stride == in.clip_len * K);
    if (!row_major) {
        float *g = nullptr;
        aq_status st = arena.get(2, static_cast<size_t>(M) * K * sizeof(float), reinterpret_cast<void **>(&g));
        if (st == AQ_OK) st = aq_gather_frames(ctx, in, M, K, g);
        if (st != AQ_OK) return st;
        x0 = g;
    }
    // counters: [0, 128) per stage, 128 listed pairs, 129 frames to fix;
    // then the pair list [2 M Q], bad_stage [M] and the frames to fix [M]
    constexpr int kZeroInts = 130;
    constexpr int kHead = 256;
    int32_t *ints = nullptr;
    {
        const size_t n = kHead + 2 * static_cast<size_t>(M) * cb->Q + 2 * static_cast<size_t>(M);
        aq_status st = arena.get(1, n * sizeof(int32_t), reinterpret_cast<void **>(&ints));
        if (st != AQ_OK) return st;
    }
    ctx->euclid_counts = ints;
    hipLaunchKernelGGL(zero2_kernel, dim3(1), dim3(256), 0, ctx->stream, ints, kZeroInts, ctx->d_flags,
                       static_cast<int>(AQ_FLAG_COUNT));
    AQ_HIP(ctx, hipGetLastError());
    // Exact values of up to kVerifySpread verified pairs ([pairs, N], at most
    // 64 MiB), spread over the grid by euclid_verify_values_kernel; a fixed
    // region too small for them leaves a block per pair computing its own.
    constexpr int kVerifySpread = 256;
    float *svals = nullptr;
    int scap = 0;
    {
        const int64_t fit = (int64_t{64} << 20) / (cb->N * static_cast<int64_t>(sizeof(float)));
        const int want = static_cast<int>(std::min<int64_t>(kVerifySpread, fit));
        const size_t bytes = static_cast<size_t>(want) * cb->N * sizeof(float);
        if (want > 0 && (!arena.base || arena.left() >= bytes + (size_t{4} << 20))) {
            void *w = nullptr;
            aq_status st = arena.get(6, bytes, &w);
            if (st != AQ_OK) return st;
            svals = static_cast<float *>(w);
            scap = want;
        }
    }
    CascadeArgs c{};
    StageArgs &a = c.a;
    a.M = M;
    a.N = static_cast<int>(cb->N);
    a.K = K;
    a.cbh = cb->d_cbh;
    a.nhh = cb->d_hh;
    a.cbf = cb->d_cbf;
    a.bias = cb->d_bias;
    a.e2 = cb->d_e2;
    a.q8 = cb->q8 ? cb->d_q8 : nullptr;
    a.q8d = cb->q8 ? cb->d_q8d : nullptr;
    // ggml's choice between tinyBLAS and ggml_vec_dot_f32 (see run_stage)
    a.order = (M >= 2 && K % 16 == 0 && cb->N % 4 == 0) ? 0 : 1;
    a.Q = static_cast<int>(cb->Q);
    a.idx = idx;
    a.dist = dist;
    a.topk = topk;
    a.topk_idx = topk_idx;
    a.topk_dist = topk_dist;
    a.force_idx = force_idx;
    a.flags = ctx->d_flags;
    a.spec_count = ints + 128;
    a.spec_list = ints + kHead;
    a.svals = svals;
    a.scap = scap;
    {
        // test hooks: every frame speculates, on a wrong code (1: the
        // verification and fix-up then decide all of them), or with its best
        // code and distances one bit off (2: the verification corrects them)
        const char *e = std::getenv("AQ_EUCLID_TEST_MISSPECULATE");
        a.misspeculate = e && (e[0] == '1' || e[0] == '2') ? e[0] - '0' : 0;
    }
    c.x0 = x0;
    c.work = work;
    c.bounds = cb->d_bounds;
    c.counts = ints;
    c.bad_count = ints + 129;
    c.bad_stage = ints + kHead + 2 * M * cb->Q;
    c.bad_list = c.bad_stage + M;
    c.write_last = residual ? 1 : 0;
    const int cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
    const int64_t blocks = (M + frames - 1) / frames;
    aq_launch_timed(ctx, !arena.base, casc, dim3(static_cast<unsigned>(blocks)), dim3(threads),
                    static_cast<uint32_t>(clds), c);
    AQ_HIP(ctx, hipGetLastError());
    hipLaunchKernelGGL(vvals, dim3(static_cast<unsigned>(2 * cus)), dim3(kScanThreads), slds, ctx->stream, c);
    AQ_HIP(ctx, hipGetLastError());
    hipLaunchKernelGGL(ver, dim3(static_cast<unsigned>(2 * cus)), dim3(kScanThreads), slds, ctx->stream, c);
    AQ_HIP(ctx, hipGetLastError());
    hipLaunchKernelGGL(fix, dim3(static_cast<unsigned>(cus)), dim3(kScanThreads), slds, ctx->stream, c);
    AQ_HIP(ctx, hipGetLastError());
    if (force_idx) {
        int32_t flag = 0;
        AQ_HIP(ctx, hipMemcpyAsync(&flag, ctx->d_flags + AQ_FLAG_BAD_INDEX, sizeof(int32_t), hipMemcpyDeviceToHost, ctx->stream));
        AQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (flag) return aq_fail(ctx, AQ_E_INDEX_RANGE, "aq_euclid_encode: force_idx holds a code outside [0, %lld)", (long long)cb->N);
    }
    return AQ_OK;
}

// Encode M frames (strided input `in`) through every stage of cb.  Plain
// codebooks: the residual cascade in codebook space, r -= c[code].
// Projected codebooks: per stage p = project_in(r), the stage pipeline on p,
// and r -= project_out(c[code]) in hidden space, fused into the next stage's
// projection.
aq_status euclid_encode_impl(aq_ctx *ctx, const aq_codebooks *cb, const aq_frames_desc &in, int64_t M, int32_t *idx,
                             float *residual, float *dist, int topk, int32_t *topk_idx, float *topk_dist,
                             const int32_t *force_idx, Arena arena) {
    if (!ctx || !cb || (M > 0 && (!idx || !in.x))) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_euclid_encode: null argument");
    if (cb->device != ctx->device)
        return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_euclid_encode: codebooks belong to another device");
    if (M < 0 || M > (int64_t{1} << 31) - 1) return aq_fail(ctx, AQ_E_SHAPE, "aq_euclid_encode: M=%lld out of range", (long long)M);
    if (in.clip_len <= 0) return aq_fail(ctx, AQ_E_SHAPE, "aq_euclid_encode: clip_len must be positive");
    if (topk < 0 || topk > 4 || topk > cb->N)
        return aq_fail(ctx, AQ_E_SHAPE, "aq_euclid_encode: topk=%d (supported 0..4, at most N)", topk);
    if (topk > 0 && M > 0 && (!topk_idx || !topk_dist))
        return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_euclid_encode: topk outputs missing");
    if (M == 0) return AQ_OK;
    aq_device_guard g(ctx->device);
    if (cb->any) return euclid_encode_any(ctx, cb, in, M, idx, residual, dist, topk, topk_idx, topk_dist, force_idx, arena);
    const int K = static_cast<int>(cb->K);
    const int ks = K / 32;
    const aq_proj_weights *pw = cb->proj;
    const int64_t H = pw ? pw->H : K;   // width of the input and of the residual
    // Keys per lane: 4 for top-4, 3 otherwise (one med3 less per score in
    // the sweep).  On k-means (16 384 x 768) three keys leave 328 frames to
    // the split-fp16 refine pass instead of 10, and the step is still 1 %
    // faster (the sweep 2.5 %).
    const int topl = topk >= 4 ? 4 : 3;
    const KsKernels *kk = kernels_for(ks);
    const int var = variant_of(cb->recipe, cb->q8);
    const Pipeline pipe = pipeline_for(cb, kk, var, topl);
    if (pipe != Pipeline::kStages)
        return euclid_encode_cascade(ctx, cb, in, M, idx, residual, dist, topk, topk_idx, topk_dist, force_idx, arena, kk,
                                     var, topl, pipe == Pipeline::kResident);
    StageFn sweep = kk->sweep[cb->q8 ? 1 : 0][topl - 3];
    StageFn select = kk->select[var][topl - 3];
    StageFn scan = kk->exact_scan[var];
    const int lds = kk->lds;
    const size_t scan_lds = scan_lds_bytes(K);
    {
        aq_status ls = aq_launch_lds(ctx, reinterpret_cast<const void *>(sweep), static_cast<size_t>(lds), "aq_euclid_encode (sweep)");
        if (ls == AQ_OK) ls = aq_launch_lds(ctx, reinterpret_cast<const void *>(scan), scan_lds, "aq_euclid_encode (exact scan)");
        if (ls != AQ_OK) return ls;
    }
    const int cus = ctx->num_cus > 0 ? ctx->num_cus : 256;

    // Sweep launch: tiles of kWaves * FG * 16 frames; the codebook is split
    // over blockIdx.y so that there are about two sweep waves per SIMD (each
    // split a whole number of LDS chunks, at most 4 splits).
    const int FG = groups_for(ks);
    const int64_t frames_per_block = static_cast<int64_t>(kWaves) * FG * 16;
    const int64_t tiles = (M + frames_per_block - 1) / frames_per_block;
    const int nch = static_cast<int>(cb->N / kk->cc);
    const int64_t tiles8 = (tiles + 7) / 8 * 8;
    int nsplit = 1;
    for (int sp = 1; sp <= 4; ++sp)
        if (nch % sp == 0 && tiles * sp <= 2 * cus) nsplit = sp;
    int nsplit2 = nsplit;
    int64_t tile2 = tiles8;   // no second part
    // Grids of several rounds of blocks: the tiles that fill whole rounds
    // take nsplit splits, the rest (the last, partial round) nsplit2 >=
    // nsplit, so that the last round's blocks are short; both chosen to
    // minimise the estimated time in whole-codebook block times, at a small
    // price per split (each split loads its frames again and the select
    // merges one more key list: about 6 %; k-means took the same time with
    // 2 and 4 splits throughout).
    if (tiles > 2 * cus) {
        const int64_t slots = static_cast<int64_t>(cus) * sweep_blocks_per_cu(ks);
        auto cost = [&](int64_t blocks, int sp) {
            return static_cast<double>((blocks + slots - 1) / slots) / sp * (1.0 + 0.06 * (sp - 1));
        };
        double best = 1e30;
        for (int sp : {1, 2, 4}) {
            if (nch % sp != 0) continue;
            const double one = cost(tiles8 * sp, sp);
            if (one < best) {
                best = one;
                nsplit = nsplit2 = sp;
                tile2 = tiles8;
            }
            const int64_t t1 = (tiles8 * sp / slots) * slots / sp / 8 * 8;   // tiles of the whole rounds
            if (t1 <= 0 || t1 >= tiles) continue;
            for (int sp2 : {2, 4, 8, 16}) {
                if (sp2 <= sp || nch % sp2 != 0) continue;
                const double two = cost(t1 * sp, sp) + cost((tiles - t1 + 7) / 8 * 8 * sp2, sp2);
                if (two < best) {
                    best = two;
                    nsplit = sp;
                    nsplit2 = sp2;
                    tile2 = t1;
                }
            }
        }
    }
    {
        // test hook: one split count for every tile (the results are the
        // same bits either way)
        const char *e = std::getenv("AQ_EUCLID_TEST_SPLIT");
        if (e && std::strcmp(e, "uniform") == 0) {
            nsplit2 = nsplit;
            tile2 = tiles8;
        }
    }
    const int maxsplit = nsplit2 > nsplit ? nsplit2 : nsplit;
    const int64_t sweep_blocks = tile2 * nsplit + (tiles8 - tile2) * nsplit2;
    const int64_t ngroups = (M + 15) / 16;

    // Work buffers: the residual (the caller's buffer when given; [M, H]),
    // the projected queries of a projected cascade ([M, K]), the sweep's keys
    // and frame norms, and the per-stage failure lists.
    float *work = residual;
    if (!work) {
        aq_status st = arena.get(0, static_cast<size_t>(M) * H * sizeof(float), reinterpret_cast<void **>(&work));
        if (st != AQ_OK) return st;
    }
    float *pbuf = nullptr;
    if (pw) {
        aq_status st = arena.get(2, static_cast<size_t>(M) * K * sizeof(float), reinterpret_cast<void **>(&pbuf));
        if (st != AQ_OK) return st;
    }
    float *keys = nullptr;
    {
        const size_t key_bytes = static_cast<size_t>(maxsplit) * ngroups * topl * kWave * sizeof(float);
        void *w = nullptr;
        aq_status st = arena.get(4, key_bytes + 3 * static_cast<size_t>(M) * sizeof(float), &w);
        if (st != AQ_OK) return st;
        keys = static_cast<float *>(w);
    }
    // Counters (per stage, modulo 64): [0, 64) frames the fp16 certificate
    // left open, [64, 128) frames sent on to the exact scan, [128, 128 +
    // kScanSplitFrames) the exact scan's chunks done per frame; then the two
    // frame lists.
    constexpr int kCounters = 128 + kScanSplitFrames;
    int32_t *fails = nullptr;
    {
        aq_status st = arena.get(1, (2 * static_cast<size_t>(M) + kCounters) * sizeof(int32_t),
                                 reinterpret_cast<void **>(&fails));
        if (st != AQ_OK) return st;
    }
    ctx->euclid_counts = fails;   // read by aq_euclid_failures / aq_euclid_exact_scans
    int32_t *counts = fails;
    int32_t *counts2 = fails + 64;
    int32_t *slot_done = fails + 128;
    int32_t *list = fails + kCounters;
    int32_t *list2 = list + M;
    RefArgs rf{};
    // Refine-pass keys: the largest of the slicings' needs (short slices for
    // up to kRSmallFrames open frames, middle ones for up to kRMidFrames,
    // long slices for all M), at most
    // 64 MiB; frames beyond the capacity go straight to the exact scan (a
    // buffer too small for short slices of the open frames takes long ones).
    {
        const int64_t per_small =   // floats per frame
            cb->N <= kRSmallCodes ? ((cb->N + kRSSmall - 1) / kRSSmall) * 4 * kTopR : ((cb->N + kRS - 1) / kRS) * 4 * kTopR;
        const int64_t per_mid = ((cb->N + kRSMid - 1) / kRSMid) * 4 * kTopR;
        const int64_t per_big = ((cb->N + kRS - 1) / kRS) * 4 * kTopR;
        int64_t floats = std::max({std::min<int64_t>(M, kRSmallFrames) * per_small,
                                   std::min<int64_t>(M, kRMidFrames) * per_mid, M * per_big});
        floats = std::min<int64_t>(floats, (int64_t{64} << 20) / 4);
        // Test hook: AQ_EUCLID_REFINE_KEY_FLOATS caps the buffer, so that the
        // path from the capacity limit to the exact scan runs at small sizes.
        if (const char *cap = std::getenv("AQ_EUCLID_REFINE_KEY_FLOATS")) {
            const long long v = std::atoll(cap);
            if (v > 0) floats = std::min<int64_t>(floats, v);
        }
        // in a fixed region, whatever is left after the other buffers
        floats = std::min<int64_t>(floats, static_cast<int64_t>(std::min<size_t>(arena.left() / 4, size_t{1} << 40)));
        floats = std::max(floats, per_small);
        void *w = nullptr;
        aq_status st = arena.get(3, static_cast<size_t>(floats) * 4, &w);
        if (st != AQ_OK) return st;
        rf.keys = static_cast<float *>(w);
        rf.key_floats = floats;
    }
    // Exact values of the scanned frames' codes ([kScanSplitFrames, N]); a
    // fixed region too small for them leaves every scan on one CU per frame.
    float *svals = nullptr;
    int scap = 0;
    {
        const size_t bytes = static_cast<size_t>(kScanSplitFrames) * cb->N * sizeof(float);
        if (!arena.base || arena.left() >= bytes + (size_t{8} << 20)) {
            void *w = nullptr;
            aq_status st = arena.get(6, bytes, &w);
            if (st != AQ_OK) return st;
            svals = static_cast<float *>(w);
            scap = kScanSplitFrames;
        }
    }
    rf.list2 = list2;
    RefineFn rvals = kk->refine_values[var];
    RefineFn rsel = kk->refine_select[var];
    hipLaunchKernelGGL(zero2_kernel, dim3(1), dim3(256), 0, ctx->stream, counts, kCounters, ctx->d_flags,
                       static_cast<int>(AQ_FLAG_COUNT));
    AQ_HIP(ctx, hipGetLastError());

    // Stage s of the pipeline: queries xin [M, K], residual out xout (null:
    // not needed), teacher forcing `force` of the codebook-space update.
    auto run_stage = [&](int64_t s, const float *xin, float *xout, const int32_t *force) -> aq_status {
        StageArgs a{};
        a.xin = xin;
        a.xout = xout;
        a.M = M;
        a.N = static_cast<int>(cb->N);
        a.K = K;
        a.cbh = cb->d_cbh + s * cb->N * K;
        a.nhh = cb->d_hh + s * cb->N;
        a.cbf = cb->d_cbf + s * cb->N * K;
        a.bias = cb->d_bias + s * cb->N;
        a.e2 = cb->d_e2 + s * cb->N;
        a.q8 = cb->q8 ? cb->d_q8 + s * cb->N * K : nullptr;
        a.q8d = cb->q8 ? cb->d_q8d + s * cb->N * (K / 32) : nullptr;
        a.cmax = cb->cmax[s];
        a.dcmax = cb->dcmax[s];
        a.chmax = cb->chmax[s];
        // ggml hands an F32 x F32 mul_mat to tinyBLAS when the query batch has
        // >= 2 rows, k % 16 == 0 and the codebook has a multiple of 4 rows
        // (ggml-cpu.c:1285-1306, sgemm.cpp:3705-3725); else ggml_vec_dot_f32.
        a.order = (M >= 2 && K % 16 == 0 && cb->N % 4 == 0) ? 0 : 1;
        a.Q = static_cast<int>(cb->Q);
        a.s = static_cast<int>(s);
        a.idx = idx;
        a.dist = dist;
        a.topk = topk;
        a.topk_idx = topk_idx;
        a.topk_dist = topk_dist;
        a.force_idx = force;
        a.fail_count = counts + (s % 64);
        a.fail_list = list;
        a.flags = ctx->d_flags;
        a.exact_only = cb->exact_only ? 1 : 0;
        a.keys = keys;
        a.norms = keys + static_cast<size_t>(maxsplit) * ngroups * topl * kWave;
        a.nsplit = nsplit;
        a.nsplit2 = nsplit2;
        a.tile2 = tile2;
        a.svals = svals;
        a.scap = scap;
        a.slot_done = slot_done;
        if (s >= 64 && s % 64 == 0) {
            hipLaunchKernelGGL(zero2_kernel, dim3(1), dim3(256), 0, ctx->stream, counts, 128, counts, 0);
            AQ_HIP(ctx, hipGetLastError());
        }
        // (the no-allocation entry point creates no timing events)
        aq_launch_timed(ctx, !arena.base, sweep, dim3(static_cast<unsigned>(sweep_blocks)), dim3(kThreads),
                        static_cast<uint32_t>(lds), a);
        AQ_HIP(ctx, hipGetLastError());
        hipLaunchKernelGGL(select, dim3(static_cast<unsigned>((ngroups + kWaves - 1) / kWaves)), dim3(kThreads), 0,
                           ctx->stream, a);
        AQ_HIP(ctx, hipGetLastError());
        // refine pass over the frames the stage kernel left open
        RefArgs r = rf;
        r.cbl = cb->d_cbl + s * cb->N * K;
        r.clmax = cb->clmax[s];
        r.crmax = cb->crmax[s];
        r.count2 = counts2 + (s % 64);
        hipLaunchKernelGGL(rvals, dim3(static_cast<unsigned>(2 * cus)), dim3(kWave * kRWaves), 0, ctx->stream, a, r);
        AQ_HIP(ctx, hipGetLastError());
        hipLaunchKernelGGL(rsel, dim3(static_cast<unsigned>(16 * cus)), dim3(kWave), 0, ctx->stream, a, r);
        AQ_HIP(ctx, hipGetLastError());
        // exact scan of what the refine pass left open
        StageArgs a2 = a;
        a2.fail_count = r.count2;
        a2.fail_list = list2;
        a2.open_count = a.fail_count;
        hipLaunchKernelGGL(scan, dim3(static_cast<unsigned>(cus)), dim3(kScanThreads), scan_lds, ctx->stream, a2);
        AQ_HIP(ctx, hipGetLastError());
        return AQ_OK;
    };

    const bool row_major = in.frame_stride == H && in.chan_stride == 1 && (in.clip_len >= M || in.clip_stride == in.clip_len * H);
    if (!pw) {
        // A strided input is gathered into the residual buffer first.
        const float *x0 = in.x;
        if (!row_major) {
            aq_status st = aq_gather_frames(ctx, in, M, H, work);
            if (st != AQ_OK) return st;
            x0 = work;
        }
        for (int64_t s = 0; s < cb->Q; ++s) {
            // the last stage's residual is only written when the caller asks for it
            aq_status st = run_stage(s, s == 0 ? x0 : work, (s + 1 < cb->Q || residual) ? work : nullptr, force_idx);
            if (st != AQ_OK) return st;
        }
    } else {
        // Stage s reads the input (s <= 1) or the residual buffer, subtracts
        // the table row of stage s - 1's code (teacher-forced when asked) and
        // projects.
        const int32_t *codes = force_idx ? force_idx : idx;
        const int ld = static_cast<int>(cb->Q);
        const aq_frames_desc wdesc = aq_frames_row_major(work, M, H);
        for (int64_t s = 0; s < cb->Q; ++s) {
            aq_status st = aq_proj_step(ctx, pw, static_cast<int>(s), static_cast<int>(s) - 1, s <= 1 ? in : wdesc,
                                        s >= 1 ? work : nullptr, codes, ld, pbuf, M);
            if (st != AQ_OK) return st;
            st = run_stage(s, pbuf, nullptr, nullptr);
            if (st != AQ_OK) return st;
        }
        if (residual) {
            aq_status st = aq_proj_step(ctx, pw, -1, static_cast<int>(cb->Q) - 1, cb->Q == 1 ? in : wdesc, residual,
                                        codes, ld, nullptr, M);
            if (st != AQ_OK) return st;
        }
    }
    if (force_idx) {
        int32_t flag = 0;
        AQ_HIP(ctx, hipMemcpyAsync(&flag, ctx->d_flags + AQ_FLAG_BAD_INDEX, sizeof(int32_t), hipMemcpyDeviceToHost, ctx->stream));
        AQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (flag) return aq_fail(ctx, AQ_E_INDEX_RANGE, "aq_euclid_encode: force_idx holds a code outside [0, %lld)", (long long)cb->N);
    }
    return AQ_OK;
}

}  // namespace

extern "C" {

aq_status aq_euclid_encode(aq_ctx *ctx, const aq_codebooks *cb, const float *x, int64_t M, int32_t *idx,
                           float *residual, float *dist, int topk, int32_t *topk_idx, float *topk_dist,
                           const int32_t *force_idx) {
    if (!cb) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_euclid_encode: null argument");
    const int64_t H = cb->proj ? cb->proj->H : cb->K;
    return euclid_encode_impl(ctx, cb, aq_frames_row_major(x, M, H), M, idx, residual, dist, topk, topk_idx, topk_dist,
                              force_idx, Arena{ctx, nullptr, 0, 0});
}

aq_status aq_euclid_encode_noalloc(aq_ctx *ctx, const aq_codebooks *cb, const float *x, int64_t M, int32_t *idx,
                                   float *residual, float *dist, int topk, int32_t *topk_idx, float *topk_dist,
                                   const int32_t *force_idx) {
    if (!ctx || !cb) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_euclid_encode_noalloc: null argument");
    aq_device_guard g(ctx->device);
    unsigned char *base = nullptr;
    aq_status st = noalloc_region(ctx, &base);
    if (st != AQ_OK) return st;
    const int64_t H = cb->proj ? cb->proj->H : cb->K;
    // One call at a time per device on the host; on the device, this call's
    // stream waits for the previous call's work (any context, any stream).
    std::lock_guard<std::mutex> order(g_noalloc_call_mu[ctx->device]);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    AQ_HIP(ctx, hipStreamIsCapturing(ctx->stream, &cap));
    const bool ordered = cap == hipStreamCaptureStatusNone;
    if (ordered) AQ_HIP(ctx, hipStreamWaitEvent(ctx->stream, g_noalloc_done[ctx->device], 0));
    st = euclid_encode_impl(ctx, cb, aq_frames_row_major(x, M, H), M, idx, residual, dist, topk, topk_idx, topk_dist,
                            force_idx, Arena{ctx, base, kNoAllocBytes, 0});
    if (ordered) {
        const hipError_t e = hipEventRecord(g_noalloc_done[ctx->device], ctx->stream);
        if (e != hipSuccess && st == AQ_OK)
            return aq_fail(ctx, AQ_E_DEVICE, "aq_euclid_encode_noalloc: hipEventRecord failed: %s", hipGetErrorString(e));
    }
    return st;
}

aq_status aq_euclid_encode_strided(aq_ctx *ctx, const aq_codebooks *cb, const float *x, int64_t M, int64_t clip_len,
                                   int64_t clip_stride, int64_t frame_stride, int64_t chan_stride, int32_t *idx,
                                   float *residual, float *dist, int topk, int32_t *topk_idx, float *topk_dist,
                                   const int32_t *force_idx) {
    return euclid_encode_impl(ctx, cb, aq_frames_desc{x, clip_len, clip_stride, frame_stride, chan_stride}, M, idx,
                              residual, dist, topk, topk_idx, topk_dist, force_idx, Arena{ctx, nullptr, 0, 0});
}

aq_status aq_euclid_failures(aq_ctx *ctx, const aq_codebooks *cb, int32_t *host_counts) {
    if (!ctx || !cb || !host_counts) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_euclid_failures: null argument");
    int32_t *fails = ctx->euclid_counts;
    if (!fails) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_euclid_failures: no encode has run");
    aq_device_guard g(ctx->device);
    const int64_t n = std::min<int64_t>(cb->Q, 64);
    AQ_HIP(ctx, hipMemcpyAsync(host_counts, fails, sizeof(int32_t) * n, hipMemcpyDeviceToHost, ctx->stream));
    AQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return AQ_OK;
}

aq_status aq_euclid_exact_scans(aq_ctx *ctx, const aq_codebooks *cb, int32_t *host_counts) {
    if (!ctx || !cb || !host_counts) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_euclid_exact_scans: null argument");
    int32_t *fails = ctx->euclid_counts;
    if (!fails) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_euclid_exact_scans: no encode has run");
    aq_device_guard g(ctx->device);
    const int64_t n = std::min<int64_t>(cb->Q, 64);
    AQ_HIP(ctx, hipMemcpyAsync(host_counts, fails + 64, sizeof(int32_t) * n, hipMemcpyDeviceToHost, ctx->stream));
    AQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return AQ_OK;
}

aq_status aq_codebook_gather(aq_ctx *ctx, const aq_codebooks *cb, int64_t stage, const int32_t *idx, int64_t M, float *out) {
    if (!ctx || !cb || (M > 0 && (!idx || !out))) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_codebook_gather: null argument");
    if (stage < 0 || stage >= cb->Q || M < 0) return aq_fail(ctx, AQ_E_SHAPE, "aq_codebook_gather: stage or M out of range");
    if (M == 0) return AQ_OK;
    aq_device_guard g(ctx->device);
    hipLaunchKernelGGL(zero2_kernel, dim3(1), dim3(256), 0, ctx->stream, ctx->d_flags, static_cast<int>(AQ_FLAG_COUNT),
                       ctx->d_flags, 0);
    AQ_HIP(ctx, hipGetLastError());
    const int64_t total = M * cb->K;
    hipLaunchKernelGGL(gather_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, ctx->stream,
                       cb->d_cbf + stage * cb->N * cb->K, cb->N, cb->K, idx, M, out, ctx->d_flags);
    AQ_HIP(ctx, hipGetLastError());
    int32_t flag = 0;
    AQ_HIP(ctx, hipMemcpyAsync(&flag, ctx->d_flags + AQ_FLAG_BAD_INDEX, sizeof(int32_t), hipMemcpyDeviceToHost, ctx->stream));
    AQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (flag) return aq_fail(ctx, AQ_E_INDEX_RANGE, "aq_codebook_gather: code outside [0, %lld)", (long long)cb->N);
    return AQ_OK;
}

aq_status aq_euclid_decode(aq_ctx *ctx, const aq_codebooks *cb, const int32_t *idx, int64_t M, float *out) {
    if (!ctx || !cb || (M > 0 && (!idx || !out))) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_euclid_decode: null argument");
    if (M < 0) return aq_fail(ctx, AQ_E_SHAPE, "aq_euclid_decode: negative M");
    if (M == 0) return AQ_OK;
    aq_device_guard g(ctx->device);
    hipLaunchKernelGGL(zero2_kernel, dim3(1), dim3(256), 0, ctx->stream, ctx->d_flags, static_cast<int>(AQ_FLAG_COUNT),
                       ctx->d_flags, 0);
    AQ_HIP(ctx, hipGetLastError());
    const int64_t total = M * cb->K;
    if (cb->proj) {
        aq_status st = aq_proj_decode(ctx, cb->proj, idx, M, out);
        if (st != AQ_OK) return st;
    } else {
        hipLaunchKernelGGL(decode_sum_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, ctx->stream,
                           cb->d_cbf, static_cast<int>(cb->Q), cb->N, cb->K, idx, M, out, ctx->d_flags);
    }
    AQ_HIP(ctx, hipGetLastError());
    int32_t flag = 0;
    AQ_HIP(ctx, hipMemcpyAsync(&flag, ctx->d_flags + AQ_FLAG_BAD_INDEX, sizeof(int32_t), hipMemcpyDeviceToHost, ctx->stream));
    AQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (flag) return aq_fail(ctx, AQ_E_INDEX_RANGE, "aq_euclid_decode: code outside [0, %lld)", (long long)cb->N);
    return AQ_OK;
}

}  // extern "C"
