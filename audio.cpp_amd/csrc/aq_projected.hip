// Projected Euclidean RVQ kernels (OmniVoice / Higgs acoustic quantizers).
//
// The reference runs, per stage s (omnivoice/audio_tokenizer.cpp:1886-1927,
// higgs_audio_tts/codec.cpp:958-1016):
//   p = LinearModule(project_in)(r)                     H -> K, + bias
//   code = argmax of the recipe's logits of p           (the Euclidean stage)
//   r -= LinearModule(project_out)(get_rows(c, code))   K -> H, + bias
// with LinearModule = ggml_mul_mat then ggml_add (linear_module.cpp:73-108).
//
// Here:
//  * project_out(c[n]) + b depends only on the code, so each stage's values
//    for all N codes are a table built once at upload with ggml's arithmetic;
//    the residual update is a row gather and one subtraction per element,
//    fused into the next stage's projection block.
//  * project_in is computed exactly in ggml's order, because the codes (and
//    the reported logits) are taken from its bits: for F32 weights tinyBLAS's
//    16 FMA lanes over k = 16u + t, then _mm512_reduce_add_ps's pairing tree
//    (sgemm.cpp:523-580), which are a 16-lane DPP row here; for Q8_0 weights
//    x86 quantize_row_q8_0 of the residual and the block dot of
//    tinyBLAS_Q0_AVX / ggml_vec_dot_q8_0_q8_0 (8 exact int lanes per block
//    scaled by d_w * d_x and FMA-accumulated, then an 8-lane tree).  A single
//    frame (M = 1) takes ggml_vec_dot_f32 for F32 weights, as ggml does.
//  * Each projection block holds 16 frames' residuals in LDS; each thread
//    owns one of the 16 tinyBLAS lanes of 8 outputs x 8 frames, i.e. 64
//    independent FMA chains fed by 8 weight and 8 residual loads per step.
#include "aq_euclid_kernels.hpp"
#include "aq_projected.hpp"

#include <algorithm>
#include <cstring>
#include <new>
#include <vector>

namespace {

constexpr int kPF = 16;     // frames per projection block
constexpr int kPT = 256;    // threads per projection block

// Dynamic LDS of the batched projection kernels: kPF residual rows of H + 1
// floats (channel-major reads spread over the banks), and for Q8_0 weights
// their quantised image (H bytes and H / 32 scales per row).
inline size_t proj_rows_lds(int64_t H, bool q8) {
    size_t b = static_cast<size_t>(kPF) * static_cast<size_t>(H + 1) * sizeof(float);
    if (q8) b += static_cast<size_t>(kPF) * static_cast<size_t>(H) + static_cast<size_t>(kPF) * static_cast<size_t>(H / 32) * sizeof(float);
    return b;
}

struct ProjArgs {
    aq_frames_desc in;
    float *rout;            // [M, H] or null
    const float *table;     // [N, H] of the stage being subtracted, or null
    const int32_t *codes;   // codes[m * ld] of that stage (pointer offset by its column)
    int ld;
    int N;
    int32_t *flags;
    const float *w;         // [K, H] F32 project_in
    const int8_t *wq;       // [K, H] Q8_0 quants
    const float *wd;        // [K, H/32] Q8_0 scales
    const float *bias;      // [K] or null
    float *p;               // [M, K] or null
    int64_t M;
    int H, K;
};

__device__ inline float load_frame(const aq_frames_desc &in, int64_t base, int h) {
    return in.x[base + static_cast<int64_t>(h) * in.chan_stride];
}

// Phase shared by both weight types: residual rows of the block's frames into
// LDS (rows of H + 1 floats: a channel-major read writes 16 frames of one
// channel, which then fall in 16 different banks), the table update, the
// write-back.  Returns the number of frames the block owns.
__device__ int stage_rows(const ProjArgs &a, float *rs, int HP, int64_t m0) {
    __shared__ int64_t base[kPF];
    __shared__ int use[kPF];
    const int H = a.H;
    const int nf = static_cast<int>(a.M - m0 < kPF ? a.M - m0 : kPF);
    if (threadIdx.x < kPF) {
        const int f = threadIdx.x;
        const int64_t m = m0 + (f < nf ? f : 0);
        base[f] = (m / a.in.clip_len) * a.in.clip_stride + (m % a.in.clip_len) * a.in.frame_stride;
        if (a.table) {
            int c = f < nf ? a.codes[m * a.ld] : 0;
            if (c < 0 || c >= a.N) {
                a.flags[AQ_FLAG_BAD_INDEX] = 1;
                c = 0;
            }
            use[f] = c;
        }
    }
    __syncthreads();
    // Channel-adjacent frames (ggml's [C, T] layout) are read frame-fastest so
    // that a wave's loads are contiguous; frame-major rows channel-fastest.
    const bool frames_adjacent = a.in.frame_stride == 1 && a.in.chan_stride != 1;
    for (int e = threadIdx.x; e < kPF * H; e += kPT) {
        int f, h;
        if (frames_adjacent) {
            f = e % kPF;
            h = e / kPF;
        } else {
            f = e / H;
            h = e % H;
        }
        float v = 0.0f;
        if (f < nf) v = load_frame(a.in, base[f], h);
        if (a.table && f < nf) v = __fsub_rn(v, a.table[static_cast<int64_t>(use[f]) * H + h]);
        rs[f * HP + h] = v;
    }
    __syncthreads();
    if (a.rout)
        for (int e = threadIdx.x; e < nf * H; e += kPT) {
            const int f = e / H, h = e % H;
            a.rout[(m0 + f) * H + h] = rs[f * HP + h];
        }
    return nf;
}

// F32 project_in in tinyBLAS order for a block of kPF frames.
__global__ __launch_bounds__(kPT) void proj_in_f32_kernel(ProjArgs a) {
    extern __shared__ float rs[];
    const int H = a.H, HP = H + 1;
    const int64_t m0 = static_cast<int64_t>(blockIdx.x) * kPF;
    const int nf = stage_rows(a, rs, HP, m0);
    if (!a.p) return;
    const int t = threadIdx.x & 15;          // tinyBLAS lane: k = 16 u + t
    const int slot = threadIdx.x >> 4;       // 16 slots: 8 output groups x 2 frame groups
    const int jg = slot & 7, fg = slot >> 3;
    const int nu = H / 16;
    for (int j0 = 0; j0 < a.K; j0 += 64) {
        float acc[8][8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int f = 0; f < 8; ++f) acc[i][f] = 0.0f;
        const float *wrow = a.w + static_cast<int64_t>(j0 + jg * 8) * H + t;
        const float *rrow = rs + (fg * 8) * HP + t;
        float wn[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) wn[i] = wrow[i * H];
        for (int u = 0; u < nu; ++u) {
            float wv[8], rv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) wv[i] = wn[i];
            if (u + 1 < nu) {   // the next step's weights are loaded ahead of this step's chains
#pragma unroll
                for (int i = 0; i < 8; ++i) wn[i] = wrow[i * H + 16 * (u + 1)];
            }
#pragma unroll
            for (int f = 0; f < 8; ++f) rv[f] = rrow[f * HP + 16 * u];
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int f = 0; f < 8; ++f) acc[i][f] = __fmaf_rn(wv[i], rv[f], acc[i][f]);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int f = 0; f < 8; ++f) {
                float v = row_ror_add<8>(acc[i][f]);
                v = row_ror_add<4>(v);
                v = row_ror_add<2>(v);
                v = row_ror_add<1>(v);
                const int j = j0 + jg * 8 + i, ff = fg * 8 + f;
                if (t == 0 && ff < nf) {
                    if (a.bias) v = __fadd_rn(v, a.bias[j]);
                    a.p[(m0 + ff) * a.K + j] = v;
                }
            }
    }
}

// Q8_0 project_in: the block's residual rows quantised with x86
// quantize_row_q8_0 into LDS, then per (output, frame) 8 lanes of exact
// 4-element int8 dots, each FMA-accumulated over the blocks with d_w * d_x.
__global__ __launch_bounds__(kPT) void proj_in_q8_kernel(ProjArgs a) {
    extern __shared__ float rs[];
    const int H = a.H, HP = H + 1, NB = H / 32;
    const int64_t m0 = static_cast<int64_t>(blockIdx.x) * kPF;
    const int nf = stage_rows(a, rs, HP, m0);
    if (!a.p) return;
    int8_t *xq = reinterpret_cast<int8_t *>(rs + kPF * HP);              // [kPF][H]
    float *xd = reinterpret_cast<float *>(xq + kPF * H);                 // [kPF][NB]
    for (int b = threadIdx.x; b < kPF * NB; b += kPT) {
        const int f = b / NB, ib = b % NB;
        quantize_block_q8(rs + f * HP + 32 * ib, xq + f * H + 32 * ib, xd + f * NB + ib);
    }
    __syncthreads();
    const int l = threadIdx.x & 7;           // int lane of the block dot: bytes 4l .. 4l+3
    const int slot = threadIdx.x >> 3;       // 32 slots: 16 output groups x 2 frame groups
    const int jg = slot & 15, fg = slot >> 4;
    for (int j0 = 0; j0 < a.K; j0 += 64) {
        float acc[4][8];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int f = 0; f < 8; ++f) acc[i][f] = 0.0f;
        const int jb = j0 + jg * 4;
        for (int ib = 0; ib < NB; ++ib) {
            int wv[4], xv[8];
            float wdv[4], xdv[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                wv[i] = *reinterpret_cast<const int *>(a.wq + static_cast<int64_t>(jb + i) * H + 32 * ib + 4 * l);
                wdv[i] = a.wd[static_cast<int64_t>(jb + i) * NB + ib];
            }
#pragma unroll
            for (int f = 0; f < 8; ++f) {
                xv[f] = *reinterpret_cast<const int *>(xq + (fg * 8 + f) * H + 32 * ib + 4 * l);
                xdv[f] = xd[(fg * 8 + f) * NB + ib];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int f = 0; f < 8; ++f) {
                    const int s = __builtin_amdgcn_sdot4(wv[i], xv[f], 0, false);
                    acc[i][f] = __fmaf_rn(__fmul_rn(wdv[i], xdv[f]), static_cast<float>(s), acc[i][f]);
                }
        }
        // hsum of the 8 lanes: i + 4, then 2, then 1 (addition commutes).
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int f = 0; f < 8; ++f) {
                float v = acc[i][f];
                v = __fadd_rn(v, __shfl_xor(v, 4));
                v = __fadd_rn(v, __shfl_xor(v, 2));
                v = __fadd_rn(v, __shfl_xor(v, 1));
                const int j = jb + i, ff = fg * 8 + f;
                if (l == 0 && ff < nf) {
                    if (a.bias) v = __fadd_rn(v, a.bias[j]);
                    a.p[(m0 + ff) * a.K + j] = v;
                }
            }
    }
}

// A single frame with F32 weights: ggml_vec_dot_f32 order for both
// products (mul_mat with one src1 row declines tinyBLAS).  The residual
// update recomputes project_out of the previous stage's code in that order.
struct OneArgs {
    ProjArgs a;
    const float *w_out_prev;   // [H, K] of the stage being subtracted
    const float *b_out_prev;   // [H] or null
    const float *cbf_prev;     // [N, K] its fp32 codebook
};

__global__ __launch_bounds__(kPT) void proj_one_kernel(OneArgs o) {
    extern __shared__ float rs[];
    const ProjArgs &a = o.a;
    const int H = a.H;
    float *cs = rs + H;        // [K] code row
    const int64_t base = 0;    // frame 0 of clip 0
    __shared__ int use;
    if (threadIdx.x == 0 && a.table) {
        int c = a.codes[0];
        if (c < 0 || c >= a.N) {
            a.flags[AQ_FLAG_BAD_INDEX] = 1;
            c = 0;
        }
        use = c;
    }
    __syncthreads();
    const int Kc = a.K;
    if (a.table)
        for (int k = threadIdx.x; k < Kc; k += kPT) cs[k] = o.cbf_prev[static_cast<int64_t>(use) * Kc + k];
    __syncthreads();
    for (int h = threadIdx.x; h < H; h += kPT) {
        float v = load_frame(a.in, base, h);
        if (a.table) {
            float z = dot_vecdot(o.w_out_prev + static_cast<int64_t>(h) * Kc, cs, Kc, 1.0f);
            if (o.b_out_prev) z = __fadd_rn(z, o.b_out_prev[h]);
            v = __fsub_rn(v, z);
        }
        rs[h] = v;
        if (a.rout) a.rout[h] = v;
    }
    __syncthreads();
    if (!a.p) return;
    for (int j = threadIdx.x; j < Kc; j += kPT) {
        float v = dot_vecdot(a.w + static_cast<int64_t>(j) * H, rs, H, 1.0f);
        if (a.bias) v = __fadd_rn(v, a.bias[j]);
        a.p[j] = v;
    }
}

// table[n][h] = project_out(c[n])[h] + b[h] for a batch of >= 2 rows: F32
// weights in tinyBLAS order over k = K, Q8_0 weights as the quantised block
// dot of x86 quantize_row_q8_0(c[n]).  One block per code.
template <bool Q8W>
__global__ __launch_bounds__(kPT) void proj_table_kernel(const float *__restrict__ cbf, int K, int H,
                                                         const float *__restrict__ w, const int8_t *__restrict__ wq,
                                                         const float *__restrict__ wd, const float *__restrict__ b,
                                                         float *__restrict__ table) {
    __shared__ float c[1024];
    __shared__ __align__(16) int8_t cq[1024];
    __shared__ float cd[32];
    const int64_t n = blockIdx.x;
    for (int k = threadIdx.x; k < K; k += kPT) c[k] = cbf[n * K + k];
    __syncthreads();
    if (Q8W) {
        for (int ib = threadIdx.x; ib < K / 32; ib += kPT) quantize_block_q8(c + 32 * ib, cq + 32 * ib, cd + ib);
        __syncthreads();
    }
    for (int h = threadIdx.x; h < H; h += kPT) {
        float v;
        if (Q8W) v = dot_q8(wq + static_cast<int64_t>(h) * K, wd + static_cast<int64_t>(h) * (K / 32), cq, cd, K / 32);
        else v = dot_tinyblas(w + static_cast<int64_t>(h) * K, c, K, 1.0f);
        if (b) v = __fadd_rn(v, b[h]);
        table[n * H + h] = v;
    }
}

// out[m][h] = sum over stages of table[s][idx[m, s]][h], in stage order from
// -0 (so the first term is exact).
__global__ void proj_decode_kernel(const float *__restrict__ table, int Q, int64_t N, int64_t H,
                                   const int32_t *__restrict__ idx, int64_t M, float *__restrict__ out,
                                   int32_t *__restrict__ flags) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= M * H) return;
    const int64_t m = t / H, h = t % H;
    float acc = -0.0f;
    for (int s = 0; s < Q; ++s) {
        int32_t c = idx[m * Q + s];
        if (c < 0 || c >= N) {
            flags[AQ_FLAG_BAD_INDEX] = 1;
            c = 0;
        }
        acc = __fadd_rn(acc, table[(static_cast<int64_t>(s) * N + c) * H + h]);
    }
    out[t] = acc;
}

// The decode of a single frame with F32 weights (vec_dot order).
__global__ void proj_decode_one_kernel(const float *__restrict__ cbf, const float *__restrict__ w_out,
                                       const float *__restrict__ b_out, int Q, int64_t N, int K, int H,
                                       const int32_t *__restrict__ idx, float *__restrict__ out,
                                       int32_t *__restrict__ flags) {
    const int h = blockIdx.x * blockDim.x + threadIdx.x;
    if (h >= H) return;
    float acc = -0.0f;
    for (int s = 0; s < Q; ++s) {
        int32_t c = idx[s];
        if (c < 0 || c >= N) {
            flags[AQ_FLAG_BAD_INDEX] = 1;
            c = 0;
        }
        float z = dot_vecdot(w_out + (static_cast<int64_t>(s) * H + h) * K, cbf + (s * N + c) * K, K, 1.0f);
        if (b_out) z = __fadd_rn(z, b_out[static_cast<int64_t>(s) * H + h]);
        acc = __fadd_rn(acc, z);
    }
    out[h] = acc;
}

// Strided frames -> frame-major rows, through a 64 x 64 LDS tile so that both
// the reads (along whichever axis is contiguous) and the writes coalesce.
__global__ __launch_bounds__(256) void gather_frames_kernel(aq_frames_desc in, int64_t M, int64_t C,
                                                            float *__restrict__ out) {
    __shared__ float tile[64][65];
    const int64_t m0 = static_cast<int64_t>(blockIdx.x) * 64, c0 = static_cast<int64_t>(blockIdx.y) * 64;
    const bool frames_adjacent = in.frame_stride == 1 && in.chan_stride != 1;
    for (int e = threadIdx.x; e < 64 * 64; e += 256) {
        const int i = e % 64, j = e / 64;   // i runs along the contiguous axis
        const int fm = frames_adjacent ? i : j, fc = frames_adjacent ? j : i;
        const int64_t m = m0 + fm, c = c0 + fc;
        float v = 0.0f;
        if (m < M && c < C)
            v = in.x[(m / in.clip_len) * in.clip_stride + (m % in.clip_len) * in.frame_stride + c * in.chan_stride];
        tile[fm][fc] = v;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < 64 * 64; e += 256) {
        const int fc = e % 64, fm = e / 64;
        const int64_t m = m0 + fm, c = c0 + fc;
        if (m < M && c < C) out[m * C + c] = tile[fm][fc];
    }
}

float fp16_bits_to_float(uint16_t h) {
    const uint32_t sign = (static_cast<uint32_t>(h) & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, mant = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            const float v = std::ldexp(static_cast<float>(mant), -24);
            std::memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (mant << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (mant << 13);
    }
    float out;
    std::memcpy(&out, &bits, 4);
    return out;
}

// block_q8_0 rows -> int8 quants and fp32 scales.
void split_q8(const void *data, size_t blocks, std::vector<int8_t> &qs, std::vector<float> &ds) {
    qs.resize(blocks * 32);
    ds.resize(blocks);
    const unsigned char *p = static_cast<const unsigned char *>(data);
    for (size_t b = 0; b < blocks; ++b) {
        uint16_t h;
        std::memcpy(&h, p + b * 34, 2);
        ds[b] = fp16_bits_to_float(h);
        std::memcpy(qs.data() + b * 32, p + b * 34 + 2, 32);
    }
}

template <typename T>
bool upload(T **dst, const T *src, size_t count) {
    if (hipMalloc(reinterpret_cast<void **>(dst), count * sizeof(T)) != hipSuccess) return false;
    return hipMemcpy(*dst, src, count * sizeof(T), hipMemcpyHostToDevice) == hipSuccess;
}

}  // namespace

aq_status aq_proj_create(aq_ctx *ctx, int64_t Q, int64_t N, int64_t K, int64_t H, const float *d_cbf,
                         int proj_type, const void *w_in, const float *b_in, const void *w_out,
                         const float *b_out, aq_proj_weights **out) {
    aq_proj_weights *pw = new (std::nothrow) aq_proj_weights();
    if (!pw) return aq_fail(ctx, AQ_E_NOMEM, "aq_euclid_upload_projected: host allocation failed");
    pw->Q = Q;
    pw->N = N;
    pw->K = K;
    pw->H = H;
    pw->q8 = proj_type == AQ_CB_Q8_0;
    pw->cbf = d_cbf;
    const size_t QKH = static_cast<size_t>(Q * K * H);
    bool ok = true;
    std::vector<int8_t> wq_in, wq_out;
    std::vector<float> wd_in, wd_out;
    int8_t *d_wq_out = nullptr;
    float *d_wd_out = nullptr;
    if (pw->q8) {
        split_q8(w_in, QKH / 32, wq_in, wd_in);
        split_q8(w_out, QKH / 32, wq_out, wd_out);
        ok = upload(&pw->w_in_q, wq_in.data(), QKH) && upload(&pw->w_in_d, wd_in.data(), QKH / 32) &&
             upload(&d_wq_out, wq_out.data(), QKH) && upload(&d_wd_out, wd_out.data(), QKH / 32);
    } else {
        ok = upload(&pw->w_in, static_cast<const float *>(w_in), QKH) &&
             upload(&pw->w_out, static_cast<const float *>(w_out), QKH);
    }
    if (ok && b_in) ok = upload(&pw->b_in, b_in, static_cast<size_t>(Q * K));
    if (ok && b_out) ok = upload(&pw->b_out, b_out, static_cast<size_t>(Q * H));
    if (ok) ok = hipMalloc(&pw->table, static_cast<size_t>(Q * N * H) * sizeof(float)) == hipSuccess;
    if (!ok) {
        (void)hipFree(d_wq_out);
        (void)hipFree(d_wd_out);
        aq_proj_release(pw);
        return aq_fail(ctx, AQ_E_NOMEM, "aq_euclid_upload_projected: device allocation or copy failed");
    }
    for (int64_t s = 0; s < Q; ++s) {
        const float *cb_s = d_cbf + s * N * K;
        const float *b_s = pw->b_out ? pw->b_out + s * H : nullptr;
        float *t_s = pw->table + s * N * H;
        if (pw->q8)
            hipLaunchKernelGGL(proj_table_kernel<true>, dim3(static_cast<unsigned>(N)), dim3(kPT), 0, ctx->stream, cb_s,
                               static_cast<int>(K), static_cast<int>(H), nullptr, d_wq_out + s * H * K,
                               d_wd_out + s * H * (K / 32), b_s, t_s);
        else
            hipLaunchKernelGGL(proj_table_kernel<false>, dim3(static_cast<unsigned>(N)), dim3(kPT), 0, ctx->stream, cb_s,
                               static_cast<int>(K), static_cast<int>(H), pw->w_out + s * H * K, nullptr, nullptr, b_s,
                               t_s);
    }
    const hipError_t e = hipGetLastError();
    const hipError_t e2 = hipStreamSynchronize(ctx->stream);
    (void)hipFree(d_wq_out);
    (void)hipFree(d_wd_out);
    if (e != hipSuccess || e2 != hipSuccess) {
        aq_proj_release(pw);
        return aq_fail(ctx, AQ_E_DEVICE, "aq_euclid_upload_projected: table kernel failed: %s",
                       hipGetErrorString(e != hipSuccess ? e : e2));
    }
    *out = pw;
    return AQ_OK;
}

aq_status aq_proj_create_linear(aq_ctx *ctx, int64_t O, int64_t I, int w_type, const void *w, const float *b,
                                aq_proj_weights **out) {
    aq_proj_weights *pw = new (std::nothrow) aq_proj_weights();
    if (!pw) return aq_fail(ctx, AQ_E_NOMEM, "aq_linear_upload: host allocation failed");
    pw->Q = 1;
    pw->N = 0;
    pw->K = O;
    pw->H = I;
    pw->q8 = w_type == AQ_CB_Q8_0;
    const size_t OI = static_cast<size_t>(O * I);
    bool ok;
    if (pw->q8) {
        std::vector<int8_t> wq;
        std::vector<float> wd;
        split_q8(w, OI / 32, wq, wd);
        ok = upload(&pw->w_in_q, wq.data(), OI) && upload(&pw->w_in_d, wd.data(), OI / 32);
    } else {
        ok = upload(&pw->w_in, static_cast<const float *>(w), OI);
    }
    if (ok && b) ok = upload(&pw->b_in, b, static_cast<size_t>(O));
    if (!ok) {
        aq_proj_release(pw);
        return aq_fail(ctx, AQ_E_NOMEM, "aq_linear_upload: device allocation or copy failed");
    }
    *out = pw;
    return AQ_OK;
}

void aq_proj_release(aq_proj_weights *pw) {
    if (!pw) return;
    for (void *p : {static_cast<void *>(pw->w_in), static_cast<void *>(pw->w_in_q), static_cast<void *>(pw->w_in_d),
                    static_cast<void *>(pw->b_in), static_cast<void *>(pw->w_out), static_cast<void *>(pw->b_out),
                    static_cast<void *>(pw->table)})
        if (p) (void)hipFree(p);
    delete pw;
}

aq_status aq_proj_step(aq_ctx *ctx, const aq_proj_weights *pw, int s, int prev, const aq_frames_desc &in,
                       float *rout, const int32_t *codes, int ld, float *p, int64_t M) {
    if (M <= 0) return AQ_OK;
    const int H = static_cast<int>(pw->H), K = static_cast<int>(pw->K);
    ProjArgs a{};
    a.in = in;
    a.rout = rout;
    a.table = prev >= 0 ? pw->table + prev * pw->N * pw->H : nullptr;
    a.codes = prev >= 0 ? codes + prev : nullptr;
    a.ld = ld;
    a.N = static_cast<int>(pw->N);
    a.flags = ctx->d_flags;
    a.p = s >= 0 ? p : nullptr;
    a.M = M;
    a.H = H;
    a.K = K;
    if (s >= 0) {
        a.w = pw->w_in ? pw->w_in + s * pw->K * pw->H : nullptr;
        a.wq = pw->w_in_q ? pw->w_in_q + s * pw->K * pw->H : nullptr;
        a.wd = pw->w_in_d ? pw->w_in_d + s * pw->K * (pw->H / 32) : nullptr;
        a.bias = pw->b_in ? pw->b_in + s * pw->K : nullptr;
    }
    if (M == 1 && !pw->q8) {
        OneArgs o{};
        o.a = a;
        if (prev >= 0) {
            o.w_out_prev = pw->w_out + prev * pw->H * pw->K;
            o.b_out_prev = pw->b_out ? pw->b_out + prev * pw->H : nullptr;
            o.cbf_prev = pw->cbf + prev * pw->N * pw->K;
        }
        // the frame's H floats, and the previous stage's K-float code row
        // when a table row is subtracted
        const size_t lds = (static_cast<size_t>(H) + (prev >= 0 ? static_cast<size_t>(K) : 0)) * sizeof(float);
        aq_status ls = aq_launch_lds(ctx, reinterpret_cast<const void *>(proj_one_kernel), lds, "projection of one frame");
        if (ls != AQ_OK) return ls;
        hipLaunchKernelGGL(proj_one_kernel, dim3(1), dim3(kPT), lds, ctx->stream, o);
        AQ_HIP(ctx, hipGetLastError());
        return AQ_OK;
    }
    const size_t lds = proj_rows_lds(H, pw->q8);
    const void *fn = pw->q8 ? reinterpret_cast<const void *>(proj_in_q8_kernel)
                            : reinterpret_cast<const void *>(proj_in_f32_kernel);
    aq_status ls = aq_launch_lds(ctx, fn, lds, "projection");
    if (ls != AQ_OK) return ls;
    const unsigned grid = static_cast<unsigned>((M + kPF - 1) / kPF);
    if (pw->q8) hipLaunchKernelGGL(proj_in_q8_kernel, dim3(grid), dim3(kPT), lds, ctx->stream, a);
    else hipLaunchKernelGGL(proj_in_f32_kernel, dim3(grid), dim3(kPT), lds, ctx->stream, a);
    AQ_HIP(ctx, hipGetLastError());
    return AQ_OK;
}

aq_status aq_proj_check_lds(aq_ctx *ctx, int64_t H, bool q8, const char *fn) {
    const void *k = q8 ? reinterpret_cast<const void *>(proj_in_q8_kernel)
                       : reinterpret_cast<const void *>(proj_in_f32_kernel);
    if (H <= 0 || !aq_lds_fits(k, proj_rows_lds(H, q8)) ||
        !aq_lds_fits(reinterpret_cast<const void *>(proj_one_kernel), static_cast<size_t>(H) * sizeof(float)))
        return aq_fail(ctx, AQ_E_SHAPE, "%s: hidden size H=%lld needs more LDS than a CU has (up to %d)", fn,
                       (long long)H, q8 ? 1984 : 2496);
    return AQ_OK;
}

aq_status aq_proj_decode(aq_ctx *ctx, const aq_proj_weights *pw, const int32_t *idx, int64_t M, float *out) {
    if (M == 1 && !pw->q8) {
        hipLaunchKernelGGL(proj_decode_one_kernel, dim3(static_cast<unsigned>((pw->H + 255) / 256)), dim3(256), 0,
                           ctx->stream, pw->cbf, pw->w_out, pw->b_out, static_cast<int>(pw->Q), pw->N,
                           static_cast<int>(pw->K), static_cast<int>(pw->H), idx, out, ctx->d_flags);
    } else {
        const int64_t total = M * pw->H;
        hipLaunchKernelGGL(proj_decode_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                           ctx->stream, pw->table, static_cast<int>(pw->Q), pw->N, pw->H, idx, M, out, ctx->d_flags);
    }
    AQ_HIP(ctx, hipGetLastError());
    return AQ_OK;
}

aq_status aq_gather_frames(aq_ctx *ctx, const aq_frames_desc &in, int64_t M, int64_t C, float *out) {
    if (M <= 0) return AQ_OK;
    hipLaunchKernelGGL(gather_frames_kernel, dim3(static_cast<unsigned>((M + 63) / 64), static_cast<unsigned>((C + 63) / 64)),
                       dim3(256), 0, ctx->stream, in, M, C, out);
    AQ_HIP(ctx, hipGetLastError());
    return AQ_OK;
}

// ---------------------------------------------------------------- C ABI

struct aq_linear {
    // device of the creating context (the handle keeps no pointer to it, so
    // it may be released after that context is destroyed)
    int device = -1;
    aq_proj_weights *pw = nullptr;
};

extern "C" {

aq_status aq_linear_upload(aq_ctx *ctx, int64_t out_features, int64_t in_features, int w_type, const void *w,
                           const float *bias, aq_linear **out) {
    if (!ctx || !w || !out) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_linear_upload: null argument");
    *out = nullptr;
    if (w_type != AQ_CB_F32 && w_type != AQ_CB_Q8_0)
        return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_linear_upload: unknown weight type %d", w_type);
    if (out_features <= 0 || out_features % 64 != 0 || out_features > (int64_t{1} << 16) || in_features <= 0 ||
        in_features % 64 != 0)
        return aq_fail(ctx, AQ_E_SHAPE,
                       "aq_linear_upload: out_features=%lld in_features=%lld (multiples of 64; in_features up to %d)",
                       (long long)out_features, (long long)in_features, w_type == AQ_CB_Q8_0 ? 1984 : 2496);
    {
        aq_status ls = aq_proj_check_lds(ctx, in_features, w_type == AQ_CB_Q8_0, "aq_linear_upload");
        if (ls != AQ_OK) return ls;
    }
    aq_device_guard g(ctx->device);
    aq_linear *lin = new (std::nothrow) aq_linear();
    if (!lin) return aq_fail(ctx, AQ_E_NOMEM, "aq_linear_upload: host allocation failed");
    lin->device = ctx->device;
    aq_status st = aq_proj_create_linear(ctx, out_features, in_features, w_type, w, bias, &lin->pw);
    if (st != AQ_OK) {
        delete lin;
        return st;
    }
    *out = lin;
    return AQ_OK;
}

aq_status aq_linear_forward(aq_ctx *ctx, const aq_linear *lin, const float *x, int64_t M, int64_t clip_len,
                            int64_t clip_stride, int64_t frame_stride, int64_t chan_stride, float *out) {
    if (!ctx || !lin || (M > 0 && (!x || !out))) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_linear_forward: null argument");
    if (lin->device != ctx->device)
        return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_linear_forward: weights belong to another device");
    if (M < 0 || M > (int64_t{1} << 31) - 1 || clip_len <= 0)
        return aq_fail(ctx, AQ_E_SHAPE, "aq_linear_forward: M=%lld clip_len=%lld", (long long)M, (long long)clip_len);
    if (M == 0) return AQ_OK;
    aq_device_guard g(ctx->device);
    const aq_frames_desc in{x, clip_len, clip_stride, frame_stride, chan_stride};
    return aq_proj_step(ctx, lin->pw, 0, -1, in, nullptr, nullptr, 0, out, M);
}

aq_status aq_linear_release(aq_linear *lin) {
    if (!lin) return AQ_E_INVALID_ARG;
    {
        aq_device_guard g(lin->device);
        aq_proj_release(lin->pw);
    }
    delete lin;
    return AQ_OK;
}

}  // extern "C"
