// DAC-style cosine RVQ on gfx950: fused multi-stage encode, decode and the
// upload-time preparation of per-stage weights.
//
// Reference recipe (audio.cpp, Fish Audio codec; paths relative to the
// audio.cpp tree):
//   quantize_one        src/models/fish_audio/codec.cpp:587-605
//   normalized_rows     src/models/fish_audio/codec.cpp:171-189
//   l2_normalize_last   src/models/fish_audio/codec.cpp:323-334
//   build_quantizer_out src/models/fish_audio/codec.cpp:542-550
//   decode sum          src/models/fish_audio/codec.cpp:552-568
// and the ggml CPU arithmetic it runs on (external/ggml/src/ggml-cpu):
//   in-projection  mul_mat -> ggml_vec_dot_f32 (vec.cpp:11-135) when the clip
//                  length T is not a multiple of 4 (tinyBLAS otherwise,
//                  llamafile/sgemm.cpp:527-545)
//   score          mul_mat with k = 8 -> scalar leftovers of ggml_vec_dot_f32
//   argmax         ggml_vec_argmax_f32 (vec.h:1576-1584), last index of the max
//   out-projection mul_mat with k = 8 -> scalar leftovers, then the bias add.
//
// Design (one kernel for all stages):
//  * A wave owns FW frames.  Lane L holds residual elements d = L + 64*i of
//    each of its frames in registers for the whole cascade, so the residual
//    is read from HBM once and written once per frame (not once per stage).
//  * ggml_vec_dot_f32 keeps 4 x 16 fp32 accumulators; accumulator (j, l)
//    takes elements k = 64*i + 16*j + l, i.e. exactly lane L = 16*j + l here.
//    Each lane runs its FMA chain over i, then an xor butterfly with lane
//    distances 32, 16, 8, 4, 2, 1 reproduces ggml's reduction tree (every
//    pairing is the same pair of partial sums; IEEE addition is commutative),
//    so the projection is bit-identical.
//  * The stage's in-projection weights and L2-normalised codebook are staged
//    in LDS in a lane-major float4 layout (conflict-free ds_read_b128); each
//    LDS read feeds FW frames.
//  * The out-projection z = W_out c[code] + b_out depends only on the code, so
//    it is tabulated per stage at upload time with the reference's arithmetic
//    (sequential non-fused 8-term sum, then the bias) and gathered per frame:
//    a coalesced 4*D-byte row read from L2/MALL instead of 2*8*D flops.
#include "aq_internal.hpp"

#include <cmath>
#include <cstdlib>
#include <new>
#include <vector>

namespace {

constexpr int kWave = 64;
constexpr int kBlock = 256;

// Values that are identical in every lane (after a full butterfly) are moved
// to scalar registers; VALU instructions then read them as SGPR operands.
__device__ inline float uniform_f(float v) {
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}
__device__ inline int uniform_i(int v) { return __builtin_amdgcn_readfirstlane(v); }
constexpr int kWavesPerBlock = kBlock / kWave;

// Per-stage LDS image (units of float4):
//   [0, 2*DI*64)           W_in : float4 (i*2 + q)*64 + L = W_in[4q .. 4q+3][64 i + L]
//   [.., + 2*(N/64)*64)    c_hat: float4 (c*2 + q)*64 + L = c_hat[64 c + L][4q .. 4q+3]
//   [.., + 2)              b_in[0..7]
inline int64_t image_f4(int64_t D, int64_t N) { return 2 * D + 2 * N + 2; }

template <int DI, int FW, bool RECON>
__global__ __launch_bounds__(kBlock, 2) void dac_encode_vecdot_kernel(
    const float *__restrict__ x, int64_t M, int Q, int N, const float4 *__restrict__ images, int64_t img_f4,
    const float *__restrict__ tables, int32_t *__restrict__ idx, float *__restrict__ residual,
    float *__restrict__ recon, const int32_t *__restrict__ force_idx, int32_t *__restrict__ flags, int has_bin) {
    extern __shared__ float4 lds[];
    constexpr int D = DI * kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int64_t m_first = (static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave) * FW;

    int64_t mrow[FW];
    bool active[FW];
    float r[FW][DI];
    float rc[FW][DI];
#pragma unroll
    for (int f = 0; f < FW; ++f) {
        active[f] = (m_first + f) < M;
        mrow[f] = active[f] ? (m_first + f) : (M - 1);
#pragma unroll
        for (int i = 0; i < DI; ++i) {
            r[f][i] = x[mrow[f] * D + i * kWave + lane];
            rc[f][i] = 0.0f;
        }
    }

    const float4 *win = lds;
    const float4 *chat = lds + 2 * DI * kWave;
    const float *bin = reinterpret_cast<const float *>(lds + 2 * DI * kWave + 2 * N);
    const int NC = N / kWave;

    for (int s = 0; s < Q; ++s) {
        __syncthreads();
        const float4 *img = images + static_cast<int64_t>(s) * img_f4;
        for (int64_t t = threadIdx.x; t < img_f4; t += kBlock) lds[t] = img[t];
        __syncthreads();

        // ---- in-projection: one FMA chain per lane and output, ggml order ----
        float acc[FW][8];
#pragma unroll
        for (int f = 0; f < FW; ++f)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[f][j] = 0.0f;
#pragma unroll
        for (int i = 0; i < DI; ++i) {
            const float4 wa = win[(i * 2 + 0) * kWave + lane];
            const float4 wb = win[(i * 2 + 1) * kWave + lane];
#pragma unroll
            for (int f = 0; f < FW; ++f) {
                const float v = r[f][i];
                acc[f][0] = __fmaf_rn(v, wa.x, acc[f][0]);
                acc[f][1] = __fmaf_rn(v, wa.y, acc[f][1]);
                acc[f][2] = __fmaf_rn(v, wa.z, acc[f][2]);
                acc[f][3] = __fmaf_rn(v, wa.w, acc[f][3]);
                acc[f][4] = __fmaf_rn(v, wb.x, acc[f][4]);
                acc[f][5] = __fmaf_rn(v, wb.y, acc[f][5]);
                acc[f][6] = __fmaf_rn(v, wb.z, acc[f][6]);
                acc[f][7] = __fmaf_rn(v, wb.w, acc[f][7]);
            }
        }
        // xor butterfly = GGML_F32x16_REDUCE (0+=2, 1+=3, 0+=1) then
        // _mm512_reduce_add_ps (distances 8, 4, 2, 1).
        float pn[FW][8];
#pragma unroll
        for (int f = 0; f < FW; ++f) {
            float p[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float v = acc[f][j];
#pragma unroll
                for (int off = 32; off >= 1; off >>= 1) v = __fadd_rn(v, __shfl_xor(v, off));
                p[j] = has_bin ? __fadd_rn(v, bin[j]) : v;
            }
            // l2_normalize_last: fp32 squares, double row sum, + 1e-12, sqrt, divide.
            double ss = 0.0;
#pragma unroll
            for (int j = 0; j < 8; ++j) ss += static_cast<double>(__fmul_rn(p[j], p[j]));
            const float den = __fsqrt_rn(__fadd_rn(static_cast<float>(ss), 1.0e-12f));
#pragma unroll
            for (int j = 0; j < 8; ++j) pn[f][j] = uniform_f(__fdiv_rn(p[j], den));
        }

        // ---- scores against the normalised codebook, argmax (last index) ----
        float bv[FW];
        int bn[FW];
        bool bad[FW];
#pragma unroll
        for (int f = 0; f < FW; ++f) {
            bv[f] = -INFINITY;
            bn[f] = 0;
            bad[f] = false;
        }
        for (int c = 0; c < NC; ++c) {
            const float4 a = chat[(c * 2 + 0) * kWave + lane];
            const float4 b = chat[(c * 2 + 1) * kWave + lane];
            const int n = c * kWave + lane;
#pragma unroll
            for (int f = 0; f < FW; ++f) {
                float sc = 0.0f;
                sc = __fadd_rn(sc, __fmul_rn(a.x, pn[f][0]));
                sc = __fadd_rn(sc, __fmul_rn(a.y, pn[f][1]));
                sc = __fadd_rn(sc, __fmul_rn(a.z, pn[f][2]));
                sc = __fadd_rn(sc, __fmul_rn(a.w, pn[f][3]));
                sc = __fadd_rn(sc, __fmul_rn(b.x, pn[f][4]));
                sc = __fadd_rn(sc, __fmul_rn(b.y, pn[f][5]));
                sc = __fadd_rn(sc, __fmul_rn(b.z, pn[f][6]));
                sc = __fadd_rn(sc, __fmul_rn(b.w, pn[f][7]));
                bad[f] |= (sc != sc);
                if (sc >= bv[f]) {
                    bv[f] = sc;
                    bn[f] = n;
                }
            }
        }
        int code[FW];
#pragma unroll
        for (int f = 0; f < FW; ++f) {
#pragma unroll
            for (int off = 1; off <= 32; off <<= 1) {
                const float ov = __shfl_xor(bv[f], off);
                const int on = __shfl_xor(bn[f], off);
                if (ov > bv[f] || (ov == bv[f] && on > bn[f])) {
                    bv[f] = ov;
                    bn[f] = on;
                }
            }
            code[f] = uniform_i(bn[f]);
            if (__any(bad[f])) {
                // A NaN score changes ggml's sequential running max; replay the
                // exact loop (rare: only for NaN/Inf inputs).
                float mx = -INFINITY;
                int id = 0;
                for (int n = 0; n < N; ++n) {
                    const float4 a = chat[((n / kWave) * 2 + 0) * kWave + (n % kWave)];
                    const float4 b = chat[((n / kWave) * 2 + 1) * kWave + (n % kWave)];
                    float sc = 0.0f;
                    sc = __fadd_rn(sc, __fmul_rn(a.x, pn[f][0]));
                    sc = __fadd_rn(sc, __fmul_rn(a.y, pn[f][1]));
                    sc = __fadd_rn(sc, __fmul_rn(a.z, pn[f][2]));
                    sc = __fadd_rn(sc, __fmul_rn(a.w, pn[f][3]));
                    sc = __fadd_rn(sc, __fmul_rn(b.x, pn[f][4]));
                    sc = __fadd_rn(sc, __fmul_rn(b.y, pn[f][5]));
                    sc = __fadd_rn(sc, __fmul_rn(b.z, pn[f][6]));
                    sc = __fadd_rn(sc, __fmul_rn(b.w, pn[f][7]));
                    mx = mx > sc ? mx : sc;
                    if (mx == sc) id = n;
                }
                code[f] = uniform_i(id);
            }
        }

        // ---- out-projection by table gather, residual update ----
#pragma unroll
        for (int f = 0; f < FW; ++f) {
            if (lane == 0 && active[f]) idx[mrow[f] * Q + s] = code[f];
            int use = code[f];
            if (force_idx) {
                use = force_idx[mrow[f] * Q + s];
                if (use < 0 || use >= N) {
                    if (lane == 0) flags[AQ_FLAG_BAD_INDEX] = 1;
                    use = 0;
                }
            }
            const float *zrow = tables + (static_cast<int64_t>(s) * N + use) * D;
#pragma unroll
            for (int i = 0; i < DI; ++i) {
                const float z = zrow[i * kWave + lane];
                r[f][i] = __fsub_rn(r[f][i], z);
                if (RECON) rc[f][i] = (s == 0) ? z : __fadd_rn(rc[f][i], z);
            }
        }
    }

#pragma unroll
    for (int f = 0; f < FW; ++f) {
        if (!active[f]) continue;
#pragma unroll
        for (int i = 0; i < DI; ++i) {
            if (residual) residual[mrow[f] * D + i * kWave + lane] = r[f][i];
            if (RECON) recon[mrow[f] * D + i * kWave + lane] = rc[f][i];
        }
    }
}

// z[s][n][d] = ((0 + c0*w0) + c1*w1 + ... + c7*w7) (+ b_out[d]): the k = 8
// mul_mat of the out-projection (scalar leftovers of ggml_vec_dot_f32: each
// product rounded, then added) followed by the bias add.
__global__ void dac_table_kernel(const float *__restrict__ cb, const float *__restrict__ w_out,
                                 const float *__restrict__ b_out, int64_t N, int64_t D, float *__restrict__ table) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= N * D) return;
    const int64_t n = t / D;
    const int64_t d = t % D;
    float z = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) z = __fadd_rn(z, __fmul_rn(cb[n * 8 + k], w_out[d * 8 + k]));
    if (b_out) z = __fadd_rn(z, b_out[d]);
    table[t] = z;
}

// recon[m][d] = sum over stages of z[s][idx[m][s]][d] (decode recipe).
__global__ void dac_decode_kernel(const int32_t *__restrict__ idx, int64_t M, int Q, int64_t N, int64_t D,
                                  const float *__restrict__ tables, float *__restrict__ out,
                                  int32_t *__restrict__ flags) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= M * D) return;
    const int64_t m = t / D;
    const int64_t d = t % D;
    float acc = 0.0f;
    for (int s = 0; s < Q; ++s) {
        int32_t code = idx[m * Q + s];
        if (code < 0 || code >= N) {
            flags[AQ_FLAG_BAD_INDEX] = 1;
            code = 0;
        }
        const float z = tables[(static_cast<int64_t>(s) * N + code) * D + d];
        acc = (s == 0) ? z : __fadd_rn(acc, z);
    }
    out[t] = acc;
}

using EncodeFn = void (*)(const float *, int64_t, int, int, const float4 *, int64_t, const float *, int32_t *,
                          float *, float *, const int32_t *, int32_t *, int);

template <int DI, int FW>
EncodeFn pick_recon(bool recon) {
    return recon ? dac_encode_vecdot_kernel<DI, FW, true> : dac_encode_vecdot_kernel<DI, FW, false>;
}

template <int DI>
EncodeFn pick_fw(int fw, bool recon) {
    switch (fw) {
        case 1: return pick_recon<DI, 1>(recon);
        case 2: return pick_recon<DI, 2>(recon);
        default: return pick_recon<DI, 4>(recon);
    }
}

EncodeFn pick_kernel(int64_t D, int fw, bool recon) {
    switch (D / kWave) {
        case 1: return pick_fw<1>(fw, recon);
        case 2: return pick_fw<2>(fw, recon);
        case 4: return pick_fw<4>(fw, recon);
        case 8: return pick_fw<8>(fw, recon);
        case 12: return pick_fw<12>(fw, recon);
        case 16: return pick_fw<16>(fw, recon);
        default: return nullptr;
    }
}

int frames_per_wave() {
    const char *e = std::getenv("AQ_DAC_FW");
    if (e) {
        const int v = std::atoi(e);
        if (v == 1 || v == 2 || v == 4) return v;
    }
    return 2;
}

}  // namespace

struct aq_dac_stages {
    aq_ctx *ctx = nullptr;
    int64_t Q = 0, D = 0, N = 0;
    bool has_bin = false;
    int64_t img_f4 = 0;
    float4 *d_images = nullptr;   // [Q][img_f4]
    float *d_tables = nullptr;    // [Q][N][D]
};

extern "C" {

aq_status aq_dac_upload(aq_ctx *ctx, int64_t Q, int64_t D, int64_t N, const float *w_in, const float *b_in,
                        const float *codebook, const float *w_out, const float *b_out, aq_dac_stages **out) {
    if (!ctx || !out || !w_in || !codebook || !w_out) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_dac_upload: null argument");
    *out = nullptr;
    if (Q <= 0 || D <= 0 || N <= 0 || D % kWave != 0 || N % kWave != 0 || !pick_kernel(D, 4, false))
        return aq_fail(ctx, AQ_E_SHAPE, "aq_dac_upload: unsupported shape Q=%lld D=%lld N=%lld (D in {64,128,256,512,768,1024}, N multiple of 64)",
                       (long long)Q, (long long)D, (long long)N);
    const int64_t img = image_f4(D, N);
    if (img * 16 > 160 * 1024)
        return aq_fail(ctx, AQ_E_SHAPE, "aq_dac_upload: D=%lld N=%lld exceeds the LDS budget", (long long)D, (long long)N);
    aq_device_guard g(ctx->device);

    // Host-side layout of the per-stage LDS images.  c_hat follows
    // normalized_rows (codec.cpp:171-189): double sum of squares, float
    // inverse 1/sqrt, float product.
    std::vector<float> images(static_cast<size_t>(Q * img * 4), 0.0f);
    for (int64_t s = 0; s < Q; ++s) {
        float *im = images.data() + s * img * 4;
        const float *Wi = w_in + s * 8 * D;
        for (int64_t i = 0; i < D / kWave; ++i)
            for (int q = 0; q < 2; ++q)
                for (int L = 0; L < kWave; ++L)
                    for (int t = 0; t < 4; ++t)
                        im[((i * 2 + q) * kWave + L) * 4 + t] = Wi[(4 * q + t) * D + i * kWave + L];
        float *ch = im + 2 * D * 4;
        const float *C = codebook + s * N * 8;
        for (int64_t n = 0; n < N; ++n) {
            double sum = 0.0;
            for (int k = 0; k < 8; ++k) sum += static_cast<double>(C[n * 8 + k]) * static_cast<double>(C[n * 8 + k]);
            const float inv = sum > 0.0 ? static_cast<float>(1.0 / std::sqrt(sum)) : 0.0f;
            const int64_t c = n / kWave, L = n % kWave;
            for (int q = 0; q < 2; ++q)
                for (int t = 0; t < 4; ++t) ch[((c * 2 + q) * kWave + L) * 4 + t] = C[n * 8 + 4 * q + t] * inv;
        }
        float *bi = im + (2 * D + 2 * N) * 4;
        for (int j = 0; j < 8; ++j) bi[j] = b_in ? b_in[s * 8 + j] : 0.0f;
    }

    aq_dac_stages *st = new (std::nothrow) aq_dac_stages();
    if (!st) return aq_fail(ctx, AQ_E_NOMEM, "aq_dac_upload: host allocation failed");
    st->ctx = ctx;
    st->Q = Q;
    st->D = D;
    st->N = N;
    st->has_bin = b_in != nullptr;
    st->img_f4 = img;
    float *d_cb = nullptr, *d_wout = nullptr, *d_bout = nullptr;
    auto cleanup = [&]() {
        if (d_cb) (void)hipFree(d_cb);
        if (d_wout) (void)hipFree(d_wout);
        if (d_bout) (void)hipFree(d_bout);
    };
    if (hipMalloc(&st->d_images, images.size() * sizeof(float)) != hipSuccess ||
        hipMalloc(&st->d_tables, sizeof(float) * static_cast<size_t>(Q * N * D)) != hipSuccess ||
        hipMalloc(&d_cb, sizeof(float) * static_cast<size_t>(Q * N * 8)) != hipSuccess ||
        hipMalloc(&d_wout, sizeof(float) * static_cast<size_t>(Q * D * 8)) != hipSuccess ||
        (b_out && hipMalloc(&d_bout, sizeof(float) * static_cast<size_t>(Q * D)) != hipSuccess)) {
        cleanup();
        aq_dac_release(st);
        return aq_fail(ctx, AQ_E_NOMEM, "aq_dac_upload: device allocation failed");
    }
    bool ok = hipMemcpyAsync(st->d_images, images.data(), images.size() * sizeof(float), hipMemcpyHostToDevice, ctx->stream) == hipSuccess &&
              hipMemcpyAsync(d_cb, codebook, sizeof(float) * static_cast<size_t>(Q * N * 8), hipMemcpyHostToDevice, ctx->stream) == hipSuccess &&
              hipMemcpyAsync(d_wout, w_out, sizeof(float) * static_cast<size_t>(Q * D * 8), hipMemcpyHostToDevice, ctx->stream) == hipSuccess &&
              (!b_out || hipMemcpyAsync(d_bout, b_out, sizeof(float) * static_cast<size_t>(Q * D), hipMemcpyHostToDevice, ctx->stream) == hipSuccess);
    for (int64_t s = 0; ok && s < Q; ++s) {
        const int64_t total = N * D;
        const unsigned blocks = static_cast<unsigned>((total + 255) / 256);
        hipLaunchKernelGGL(dac_table_kernel, dim3(blocks), dim3(256), 0, ctx->stream, d_cb + s * N * 8, d_wout + s * D * 8,
                           d_bout ? d_bout + s * D : nullptr, N, D, st->d_tables + s * N * D);
        ok = hipGetLastError() == hipSuccess;
    }
    ok = ok && hipStreamSynchronize(ctx->stream) == hipSuccess;
    cleanup();
    if (!ok) {
        aq_dac_release(st);
        return aq_fail(ctx, AQ_E_DEVICE, "aq_dac_upload: device copy or table preparation failed");
    }
    *out = st;
    return AQ_OK;
}

aq_status aq_dac_release(aq_dac_stages *st) {
    if (!st) return AQ_E_INVALID_ARG;
    {
        aq_device_guard g(st->ctx->device);
        if (st->d_images) (void)hipFree(st->d_images);
        if (st->d_tables) (void)hipFree(st->d_tables);
    }
    delete st;
    return AQ_OK;
}

aq_status aq_dac_encode(aq_ctx *ctx, const aq_dac_stages *st, const float *x, int64_t M, int64_t clip_len,
                        int32_t *idx, float *residual, float *recon, const int32_t *force_idx) {
    if (!ctx || !st || !idx || (!x && M > 0)) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_dac_encode: null argument");
    if (st->ctx->device != ctx->device) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_dac_encode: stages belong to another device");
    if (M < 0 || clip_len <= 0 || M % clip_len != 0)
        return aq_fail(ctx, AQ_E_SHAPE, "aq_dac_encode: M=%lld must be a non-negative multiple of clip_len=%lld",
                       (long long)M, (long long)clip_len);
    if (M == 0) return AQ_OK;
    if (clip_len % 4 == 0)
        return aq_fail(ctx, AQ_E_UNSUPPORTED,
                       "aq_dac_encode: clip_len %% 4 == 0 selects ggml's tinyBLAS in-projection order, not built yet");
    aq_device_guard g(ctx->device);
    const int fw = frames_per_wave();
    EncodeFn fn = pick_kernel(st->D, fw, recon != nullptr);
    const size_t lds_bytes = static_cast<size_t>(st->img_f4) * sizeof(float4);
    AQ_HIP(ctx, hipFuncSetAttribute(reinterpret_cast<const void *>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                    static_cast<int>(lds_bytes)));
    if (force_idx) AQ_HIP(ctx, hipMemsetAsync(ctx->d_flags, 0, sizeof(int32_t) * AQ_FLAG_COUNT, ctx->stream));
    const int64_t frames_per_block = static_cast<int64_t>(kWavesPerBlock) * fw;
    const unsigned blocks = static_cast<unsigned>((M + frames_per_block - 1) / frames_per_block);
    hipLaunchKernelGGL(fn, dim3(blocks), dim3(kBlock), lds_bytes, ctx->stream, x, M, static_cast<int>(st->Q),
                       static_cast<int>(st->N), st->d_images, st->img_f4, st->d_tables, idx, residual, recon, force_idx,
                       ctx->d_flags, st->has_bin ? 1 : 0);
    AQ_HIP(ctx, hipGetLastError());
    if (force_idx) {
        int32_t flag = 0;
        AQ_HIP(ctx, hipMemcpyAsync(&flag, ctx->d_flags + AQ_FLAG_BAD_INDEX, sizeof(int32_t), hipMemcpyDeviceToHost, ctx->stream));
        AQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (flag) return aq_fail(ctx, AQ_E_INDEX_RANGE, "aq_dac_encode: force_idx holds a code outside [0, %lld)", (long long)st->N);
    }
    return AQ_OK;
}

aq_status aq_dac_decode(aq_ctx *ctx, const aq_dac_stages *st, const int32_t *idx, int64_t M, float *out) {
    if (!ctx || !st || (M > 0 && (!idx || !out))) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_dac_decode: null argument");
    if (M < 0) return aq_fail(ctx, AQ_E_SHAPE, "aq_dac_decode: negative M");
    if (M == 0) return AQ_OK;
    aq_device_guard g(ctx->device);
    AQ_HIP(ctx, hipMemsetAsync(ctx->d_flags, 0, sizeof(int32_t) * AQ_FLAG_COUNT, ctx->stream));
    const int64_t total = M * st->D;
    hipLaunchKernelGGL(dac_decode_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, ctx->stream, idx,
                       M, static_cast<int>(st->Q), st->N, st->D, st->d_tables, out, ctx->d_flags);
    AQ_HIP(ctx, hipGetLastError());
    int32_t flag = 0;
    AQ_HIP(ctx, hipMemcpyAsync(&flag, ctx->d_flags + AQ_FLAG_BAD_INDEX, sizeof(int32_t), hipMemcpyDeviceToHost, ctx->stream));
    AQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (flag) return aq_fail(ctx, AQ_E_INDEX_RANGE, "aq_dac_decode: code outside [0, %lld)", (long long)st->N);
    return AQ_OK;
}

}  // extern "C"
