// Host-loop members of the DAC quantizer family on the MI355X.
//
//   OuteTTS  quantize_reference (community_models/outetts/dac.cpp:376-456):
//            fp32, every product rounded before it is added, bias first,
//            first index of the minimum squared distance between the
//            normalised projection and the normalised code.
//   MOSS     MossAudioTokenizerQuantizer (models/moss/shared/
//            audio_tokenizer_quantizer.cpp): fp64 input projection, per
//            stage an fp64 in-projection, max(|e|, 1e-12) normalisation,
//            first index of the maximum dot, fp64 residual update; fp32
//            latent tables for decode.
//
// The reference builds this code without FMA (x86-64 baseline), so the exact
// arithmetic below is written as separate multiplies and adds (the library
// is compiled with -ffp-contract=off).  Where a product of two floats is
// formed in double it is exact, and a fused multiply-add gives the same
// result as the reference's multiply then add; those places use __fma_rn.
//
// Layout of one encode: a wave owns 4 frames and keeps their residuals in
// LDS (row stride padded by 16 bytes so the frames fall in different
// banks).  Lane (f, j) = (lane / 16, lane % 16): lanes j < 8 run the
// in-projection chain of code dimension j of frame f -- the reference's
// sequential sum over the latent channels; lanes j >= 8 repeat it -- and
// all 16 then score codes j, j + 16, ... of the frame and merge their
// winners with the reference's tie rule.  The residual update then sweeps
// each frame's channels across the wave.  The chains are latency-bound, so
// a block holds six such waves (24 frames; the residuals and the stage
// tables fill the LDS, so one block per CU): two SIMDs of each CU run two
// waves, whose chains interleave.  The stage's in-projection weights and
// normalised codebook are staged in LDS when they fit (an L2 round trip per
// few elements otherwise), and the residual update reads each channel's
// out-projection row once for the wave's frames.
#include "aq_device_math.hpp"
#include "aq_internal.hpp"

#include <algorithm>
#include <cmath>
#include <vector>

namespace {

constexpr int kWave = 64;
constexpr int kHF = 4;               // frames per wave
constexpr int kLPF = kWave / kHF;    // lanes per frame: 16 (in-projection: dims of lanes j < 8)
constexpr int kOtW = 6;  // waves per block (OuteTTS: 24 frames share the staged in-projection)
constexpr int kMsW = 6;  // waves per block (MOSS)

// ------------------------------------------------------------------ OuteTTS

__global__ void outetts_chat_kernel(const float *__restrict__ cb, int64_t rows, float *__restrict__ chat) {
    const int64_t n = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (n >= rows) return;
    const float *c = cb + n * 8;
    float e2 = 0.0f;   // dac.cpp:417-421
    for (int d = 0; d < 8; ++d) e2 = e2 + c[d] * c[d];
    const float en = aq_math::sqrt_rn(e2) + 1.0e-12f;
    for (int d = 0; d < 8; ++d) chat[n * 8 + d] = c[d] / en;   // dac.cpp:426-427
}

__global__ __launch_bounds__(kWave *kOtW) void outetts_encode_kernel(aq_outetts_args a) {
    extern __shared__ float lds_ot[];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int D = a.D;
    const int stride = D + 4;
    float *r = lds_ot + wave * kHF * stride;
    const int nw = blockDim.x / kWave;                      // waves per block (up to kOtW)
    // [8][D + 4] (a.win_lds; rows padded so that the 8 rows read at one k
    // fall in different banks)
    float *win_s = lds_ot + nw * kHF * stride;
    float *chat_s = win_s + (a.win_lds ? 8 * stride : 0);  // [N][8] (a.chat_lds)
    const int64_t m0 = (static_cast<int64_t>(blockIdx.x) * nw + wave) * kHF;
    for (int f = 0; f < kHF; ++f) {
        const int64_t m = m0 + f;
        for (int e = lane * 4; e < D; e += kWave * 4) {
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (m < a.M) v = *reinterpret_cast<const float4 *>(a.x + m * D + e);
            *reinterpret_cast<float4 *>(r + f * stride + e) = v;
        }
    }
    const int f = lane / kLPF;
    const int j = lane % kLPF;
    const int jd = j & 7;   // in-projection output (lanes j >= 8 repeat it)
    const int64_t mf = m0 + f;
    const bool live = mf < a.M;
    for (int s = 0; s < a.Q; ++s) {
        // the stage's tables into LDS (the previous stage's readers are past
        // its closing barrier)
        if (a.win_lds) {
            const float4 *src = reinterpret_cast<const float4 *>(a.w_in + static_cast<int64_t>(s) * 8 * D);
            for (int i = threadIdx.x; i < 2 * D; i += blockDim.x) {
                const int row = i / (D / 4), c4 = i % (D / 4);
                reinterpret_cast<float4 *>(win_s + row * stride)[c4] = src[i];
            }
        }
        if (a.chat_lds) {
            const float4 *src = reinterpret_cast<const float4 *>(a.chat + static_cast<int64_t>(s) * a.N * 8);
            for (int i = threadIdx.x; i < 2 * a.N; i += blockDim.x) reinterpret_cast<float4 *>(chat_s)[i] = src[i];
        }
        __syncthreads();
        // in-projection chain of (frame f, dim j), dac.cpp:402-410
        const float *W = a.win_lds ? win_s + jd * stride : a.w_in + (static_cast<int64_t>(s) * 8 + jd) * D;
        const float *rf = r + f * stride;
        float v = a.b_in[s * 8 + jd];
        // unrolled: the weight loads of 8 steps are in flight ahead of the chain
#pragma unroll 8
        for (int h = 0; h < D; h += 4) {
            const float4 w4 = *reinterpret_cast<const float4 *>(W + h);
            const float4 r4 = *reinterpret_cast<const float4 *>(rf + h);
            v = v + w4.x * r4.x;
            v = v + w4.y * r4.y;
            v = v + w4.z * r4.z;
            v = v + w4.w * r4.w;
        }
        // |p| and p / (|p| + 1e-12), dac.cpp:409-412,425-426
        float p[8];
        float nsq = 0.0f;
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            p[d] = __shfl(v, f * kLPF + d);
            nsq = nsq + p[d] * p[d];
        }
        const float pn = aq_math::sqrt_rn(nsq) + 1.0e-12f;
#pragma unroll
        for (int d = 0; d < 8; ++d) p[d] = p[d] / pn;
        // distances to codes j, j + 8, ... (dac.cpp:415-434), strict < keeps
        // the first index of the minimum; NaN distances never win
        float bd = INFINITY;
        int bn = -1;
        const float *Ch = a.chat_lds ? chat_s : a.chat + static_cast<int64_t>(s) * a.N * 8;
        // eight codes per step, their distance chains interleaved (the
        // compares stay in code order)
        for (int n0 = j; n0 < a.N; n0 += 8 * kLPF) {
            float dist[8];
            float cv[8][8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int n = n0 + kLPF * q < a.N ? n0 + kLPF * q : 0;
                const float4 c0 = *reinterpret_cast<const float4 *>(Ch + static_cast<int64_t>(n) * 8);
                const float4 c1 = *reinterpret_cast<const float4 *>(Ch + static_cast<int64_t>(n) * 8 + 4);
                cv[q][0] = c0.x; cv[q][1] = c0.y; cv[q][2] = c0.z; cv[q][3] = c0.w;
                cv[q][4] = c1.x; cv[q][5] = c1.y; cv[q][6] = c1.z; cv[q][7] = c1.w;
                dist[q] = 0.0f;
            }
#pragma unroll
            for (int d = 0; d < 8; ++d)
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const float diff = p[d] - cv[q][d];
                    dist[q] = dist[q] + diff * diff;
                }
#pragma unroll
            for (int q = 0; q < 8; ++q)
                if (n0 + kLPF * q < a.N && dist[q] < bd) {
                    bd = dist[q];
                    bn = n0 + kLPF * q;
                }
        }
#pragma unroll
        for (int o = 1; o < kLPF; o <<= 1) {
            const float od = __shfl_xor(bd, o);
            const int on = __shfl_xor(bn, o);
            if (on >= 0 && (bn < 0 || od < bd || (od == bd && on < bn))) {
                bd = od;
                bn = on;
            }
        }
        const int code = bn < 0 ? 0 : bn;
        int use = code;
        if (live) {
            if (j == 0) a.idx[mf * a.Q + s] = code;
            if (a.force_idx) {
                use = a.force_idx[mf * a.Q + s];
                if (use < 0 || use >= a.N) {
                    if (j == 0) a.flags[AQ_FLAG_BAD_INDEX] = 1;
                    use = 0;
                }
            }
        }
        __syncthreads();
        // residual -= b_out + W_out c[use], dac.cpp:438-453: the frames'
        // code rows first, then 4 channels at a time, each channel's
        // out-projection row read once for the wave's frames
        float4 cr0[kHF], cr1[kHF];
#pragma unroll
        for (int g = 0; g < kHF; ++g) {
            const int ug = __shfl(use, g * kLPF);
            const float *c = a.cb + (static_cast<int64_t>(s) * a.N + ug) * 8;
            cr0[g] = *reinterpret_cast<const float4 *>(c);
            cr1[g] = *reinterpret_cast<const float4 *>(c + 4);
        }
        for (int o0 = lane; o0 < D; o0 += 4 * kWave) {
            float4 w0[4], w1[4];
            float bo[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int o = o0 + t * kWave < D ? o0 + t * kWave : o0;
                const float *wo = a.w_out + (static_cast<int64_t>(s) * D + o) * 8;
                w0[t] = *reinterpret_cast<const float4 *>(wo);
                w1[t] = *reinterpret_cast<const float4 *>(wo + 4);
                bo[t] = a.b_out[static_cast<int64_t>(s) * D + o];
            }
#pragma unroll
            for (int g = 0; g < kHF; ++g) {
                float *rg = r + g * stride;
                const float4 c0 = cr0[g], c1 = cr1[g];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int o = o0 + t * kWave;
                    if (o >= D) continue;
                    float val = bo[t];
                    val = val + w0[t].x * c0.x;
                    val = val + w0[t].y * c0.y;
                    val = val + w0[t].z * c0.z;
                    val = val + w0[t].w * c0.w;
                    val = val + w1[t].x * c1.x;
                    val = val + w1[t].y * c1.y;
                    val = val + w1[t].z * c1.z;
                    val = val + w1[t].w * c1.w;
                    rg[o] = rg[o] - val;
                }
            }
        }
        __syncthreads();
    }
    if (a.residual) {
        for (int g = 0; g < kHF; ++g) {
            const int64_t m = m0 + g;
            if (m >= a.M) break;
            for (int e = lane * 4; e < D; e += kWave * 4)
                *reinterpret_cast<float4 *>(a.residual + m * D + e) = *reinterpret_cast<const float4 *>(r + g * stride + e);
        }
    }
}

// --------------------------------------------------------------------- MOSS

constexpr int kIpF = 64;   // input projection tile: frames
constexpr int kIpO = 64;   //                         outputs
constexpr int kIpK = 32;   //                         channels per LDS chunk

// residual[m, o] = b[o] + sum_k w[o, k] h[m, k] in fp64, k in order
// (audio_tokenizer_quantizer.cpp:193-201).  256 threads, 4 frames x 4
// outputs each.
__global__ __launch_bounds__(256) void moss_input_kernel(const float *__restrict__ h, int64_t M, int C, int R,
                                                         const float *__restrict__ w, const float *__restrict__ b,
                                                         double *__restrict__ res) {
    // staged as doubles: each element is converted once, not once per use
    __shared__ double hs[kIpK][kIpF + 2];
    __shared__ double ws[kIpK][kIpO + 2];
    const int tid = threadIdx.x;
    const int tx = tid & 15;
    const int ty = tid >> 4;
    const int64_t m0 = static_cast<int64_t>(blockIdx.x) * kIpF;
    const int o0 = blockIdx.y * kIpO;
    // outputs 2 tx, 2 tx + 1, 32 + 2 tx, 33 + 2 tx: the 16 lanes of a row
    // read 256 contiguous bytes of ws per 16-byte load (no bank conflicts)
    auto oq = [&](int q) { return (q < 2 ? 0 : kIpO / 2 - 2) + 2 * tx + q; };
    double acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[i][q] = static_cast<double>(b[o0 + oq(q)]);
    // The next chunk's inputs are loaded into registers while this chunk
    // computes (kIpF * kIpK / 256 = 8 elements of each per thread).
    constexpr int kPer = kIpF * kIpK / 256;
    float hn[kPer], wn[kPer];
    auto fetch = [&](int k0) {
        const int kn = min(kIpK, C - k0);
#pragma unroll
        for (int t = 0; t < kPer; ++t) {
            const int e = tid + t * 256;
            const int rr = e / kIpK, cc = e % kIpK;
            const int64_t m = m0 + rr;
            hn[t] = (m < M && cc < kn) ? h[m * C + k0 + cc] : 0.0f;
            wn[t] = cc < kn ? w[static_cast<int64_t>(o0 + rr) * C + k0 + cc] : 0.0f;
        }
    };
    fetch(0);
    for (int k0 = 0; k0 < C; k0 += kIpK) {
        const int kn = min(kIpK, C - k0);
#pragma unroll
        for (int t = 0; t < kPer; ++t) {
            const int e = tid + t * 256;
            const int rr = e / kIpK, cc = e % kIpK;
            hs[cc][rr] = static_cast<double>(hn[t]);
            ws[cc][rr] = static_cast<double>(wn[t]);
        }
        __syncthreads();
        if (k0 + kIpK < C) fetch(k0 + kIpK);
        for (int kk = 0; kk < kn; ++kk) {
            const double2 xa0 = *reinterpret_cast<const double2 *>(&hs[kk][ty * 4]);
            const double2 xa1 = *reinterpret_cast<const double2 *>(&hs[kk][ty * 4 + 2]);
            const double2 wb0 = *reinterpret_cast<const double2 *>(&ws[kk][2 * tx]);
            const double2 wb1 = *reinterpret_cast<const double2 *>(&ws[kk][kIpO / 2 + 2 * tx]);
            const double xv[4] = {xa0.x, xa0.y, xa1.x, xa1.y};
            const double wv[4] = {wb0.x, wb0.y, wb1.x, wb1.y};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q) acc[i][q] = __fma_rn(wv[q], xv[i], acc[i][q]);   // exact product
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t m = m0 + ty * 4 + i;
        if (m >= M) break;
#pragma unroll
        for (int q = 0; q < 4; ++q) res[m * R + o0 + oq(q)] = acc[i][q];
    }
}

__global__ __launch_bounds__(kWave *kMsW) void moss_cascade_kernel(aq_moss_args a) {
    extern __shared__ double lds_ms[];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int R = a.R;
    const int stride = R + 2;
    double *r = lds_ms + wave * kHF * stride;
    const int nw = blockDim.x / kWave;   // waves per block (up to kMsW)
    // the stage's in-projection [8][R + 4] (rows padded so that the 8 rows
    // read at one k fall in different banks) and normalised codebook [N][8]
    float *win_s = reinterpret_cast<float *>(lds_ms + nw * kHF * stride);
    float *tn_s = win_s + (a.win_lds ? 8 * (R + 4) : 0);
    const int64_t m0 = (static_cast<int64_t>(blockIdx.x) * nw + wave) * kHF;
    for (int f = 0; f < kHF; ++f) {
        const int64_t m = m0 + f;
        for (int e = lane * 2; e < R; e += kWave * 2) {
            double2 v = make_double2(0.0, 0.0);
            if (m < a.M) v = *reinterpret_cast<const double2 *>(a.res + m * R + e);
            *reinterpret_cast<double2 *>(r + f * stride + e) = v;
        }
    }
    const int f = lane / kLPF;
    const int j = lane % kLPF;
    const int jd = j & 7;   // in-projection output (lanes j >= 8 repeat it)
    const int64_t mf = m0 + f;
    const bool live = mf < a.M;
    for (int s = 0; s < a.Q; ++s) {
        // the stage's tables into LDS (the previous stage's readers are past
        // its closing barrier)
        if (a.win_lds) {
            const float4 *src = reinterpret_cast<const float4 *>(a.w_in + static_cast<int64_t>(s) * 8 * R);
            for (int i = threadIdx.x; i < 2 * R; i += blockDim.x) {
                const int row = i / (R / 4), c4 = i % (R / 4);
                reinterpret_cast<float4 *>(win_s + row * (R + 4))[c4] = src[i];
            }
        }
        if (a.tn_lds) {
            const float4 *src = reinterpret_cast<const float4 *>(a.tn + static_cast<int64_t>(s) * a.N * 8);
            for (int i = threadIdx.x; i < 2 * a.N; i += blockDim.x) reinterpret_cast<float4 *>(tn_s)[i] = src[i];
        }
        __syncthreads();
        // in_proj of (frame f, dim j): float weight times fp64 residual,
        // rounded, then added (:207-216)
        const float *W = a.win_lds ? win_s + jd * (R + 4) : a.w_in + (static_cast<int64_t>(s) * 8 + jd) * R;
        const double *rf = r + f * stride;
        double v = a.b_in[s * 8 + jd];
        // unrolled: the weight loads of 8 steps are in flight ahead of the chain
#pragma unroll 8
        for (int k = 0; k < R; k += 4) {
            const float4 w4 = *reinterpret_cast<const float4 *>(W + k);
            const double2 r01 = *reinterpret_cast<const double2 *>(rf + k);
            const double2 r23 = *reinterpret_cast<const double2 *>(rf + k + 2);
            v = v + static_cast<double>(w4.x) * r01.x;
            v = v + static_cast<double>(w4.y) * r01.y;
            v = v + static_cast<double>(w4.z) * r23.x;
            v = v + static_cast<double>(w4.w) * r23.y;
        }
        // encoding * (1 / std::max(sqrt(|e|^2), 1e-12)) (:210-221)
        double e[8];
        double nrm = 0.0;
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            e[d] = __shfl(v, f * kLPF + d);
            nrm = nrm + e[d] * e[d];
        }
        const double sq = aq_math::sqrt_rn(nrm);
        const double scale = 1.0 / ((sq < 1.0e-12) ? 1.0e-12 : sq);
#pragma unroll
        for (int d = 0; d < 8; ++d) e[d] = e[d] * scale;
        // first index of the maximum dot with the normalised codebook (:225-237)
        double bd = -INFINITY;
        int bn = -1;
        const float *T = a.tn_lds ? tn_s : a.tn + static_cast<int64_t>(s) * a.N * 8;
        // eight codes per step, their dot chains interleaved (the compares
        // stay in code order)
        for (int n0 = j; n0 < a.N; n0 += 8 * kLPF) {
            double dot[8];
            float tv[8][8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int n = n0 + kLPF * q < a.N ? n0 + kLPF * q : 0;
                const float4 t0 = *reinterpret_cast<const float4 *>(T + static_cast<int64_t>(n) * 8);
                const float4 t1 = *reinterpret_cast<const float4 *>(T + static_cast<int64_t>(n) * 8 + 4);
                tv[q][0] = t0.x; tv[q][1] = t0.y; tv[q][2] = t0.z; tv[q][3] = t0.w;
                tv[q][4] = t1.x; tv[q][5] = t1.y; tv[q][6] = t1.z; tv[q][7] = t1.w;
                dot[q] = 0.0;
            }
#pragma unroll
            for (int c = 0; c < 8; ++c)
#pragma unroll
                for (int q = 0; q < 8; ++q) dot[q] = dot[q] + static_cast<double>(tv[q][c]) * e[c];
#pragma unroll
            for (int q = 0; q < 8; ++q)
                if (n0 + kLPF * q < a.N && dot[q] > bd) {
                    bd = dot[q];
                    bn = n0 + kLPF * q;
                }
        }
#pragma unroll
        for (int o = 1; o < kLPF; o <<= 1) {
            const double od = __shfl_xor(bd, o);
            const int on = __shfl_xor(bn, o);
            if (on >= 0 && (bn < 0 || od > bd || (od == bd && on < bn))) {
                bd = od;
                bn = on;
            }
        }
        const int code = bn < 0 ? 0 : bn;
        int use = code;
        if (live) {
            if (j == 0) a.idx[mf * a.Q + s] = code;
            if (a.force_idx) {
                use = a.force_idx[mf * a.Q + s];
                if (use < 0 || use >= a.N) {
                    if (j == 0) a.flags[AQ_FLAG_BAD_INDEX] = 1;
                    use = 0;
                }
            }
        }
        __syncthreads();
        // residual -= b_out + W_out c[use] in fp64 (:240-248): the frames'
        // code rows first, then 4 channels at a time, each channel's
        // out-projection row read once for the wave's frames
        float4 cr0[kHF], cr1[kHF];
#pragma unroll
        for (int g = 0; g < kHF; ++g) {
            const int ug = __shfl(use, g * kLPF);
            const float *c = a.cb + (static_cast<int64_t>(s) * a.N + ug) * 8;
            cr0[g] = *reinterpret_cast<const float4 *>(c);
            cr1[g] = *reinterpret_cast<const float4 *>(c + 4);
        }
        for (int o0 = lane; o0 < R; o0 += 4 * kWave) {
            float4 w0[4], w1[4];
            float bo[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int o = o0 + t * kWave < R ? o0 + t * kWave : o0;
                const float *wo = a.w_out + (static_cast<int64_t>(s) * R + o) * 8;
                w0[t] = *reinterpret_cast<const float4 *>(wo);
                w1[t] = *reinterpret_cast<const float4 *>(wo + 4);
                bo[t] = a.b_out[static_cast<int64_t>(s) * R + o];
            }
#pragma unroll
            for (int g = 0; g < kHF; ++g) {
                double *rg = r + g * stride;
                const double cv[8] = {cr0[g].x, cr0[g].y, cr0[g].z, cr0[g].w, cr1[g].x, cr1[g].y, cr1[g].z, cr1[g].w};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int o = o0 + t * kWave;
                    if (o >= R) continue;
                    const double wv[8] = {w0[t].x, w0[t].y, w0[t].z, w0[t].w, w1[t].x, w1[t].y, w1[t].z, w1[t].w};
                    double z = bo[t];
#pragma unroll
                    for (int k = 0; k < 8; ++k) z = __fma_rn(wv[k], cv[k], z);   // exact product
                    rg[o] = rg[o] - z;
                }
            }
        }
        __syncthreads();
    }
    if (a.write_res) {
        for (int g = 0; g < kHF; ++g) {
            const int64_t m = m0 + g;
            if (m >= a.M) break;
            for (int e = lane * 2; e < R; e += kWave * 2)
                *reinterpret_cast<double2 *>(a.res + m * R + e) = *reinterpret_cast<const double2 *>(r + g * stride + e);
        }
    }
}

// Constructor tables (:77-115): per stage, comb[o][0..7] = sum_j w_op[o][j]
// w_out[j][k] and comb[o][8] = sum_j w_op[o][j] b_out[j] (fp32, from 0, in
// order), then table[n][o] = comb[o][8] + sum_k comb[o][k] c[n][k].
// Weight-norm folding w = g v / |v| per output row (one thread per row, the
// reference's sequential double sum of double squares):
//   AQ_WN_OUTETTS  scale = g / (float)sqrt(norm2), fp32 division
//                  (fold_weight_norm, community_models/outetts/dac.cpp:91-110)
//   AQ_WN_MOSS     scale = (float)(g / sqrt(norm)), double division
//                  (reconstruct_weight_norm, audio_tokenizer_quantizer.cpp:17-39)
// then w = v * scale in fp32.
__global__ void weight_norm_fold_kernel(const float *v, const float *__restrict__ g, int64_t rows,
                                        int64_t cols, int rule, float *w) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const float *vr = v + r * cols;
    double norm = 0.0;
    for (int64_t k = 0; k < cols; ++k) {
        const double x = vr[k];
        norm = __dadd_rn(norm, __dmul_rn(x, x));
    }
    const double root = aq_math::sqrt_rn(norm);
    const float scale = rule == AQ_WN_OUTETTS ? __fdiv_rn(g[r], static_cast<float>(root))
                                              : static_cast<float>(__ddiv_rn(static_cast<double>(g[r]), root));
    for (int64_t k = 0; k < cols; ++k) w[r * cols + k] = __fmul_rn(vr[k], scale);
}

// Codebook rows normalised once, in double (audio_tokenizer_quantizer.cpp
// :116-130): scale = 1 / std::max(sqrt(sum c*c), 1e-12), tn = (float)(c *
// scale).  One thread per row.
__global__ void moss_normalize_kernel(const float *__restrict__ cb, int64_t rows, float *__restrict__ tn) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    double norm = 0.0;
    for (int k = 0; k < 8; ++k) {
        const double c = cb[r * 8 + k];
        norm = __dadd_rn(norm, __dmul_rn(c, c));
    }
    const double n = aq_math::sqrt_rn(norm);
    const double scale = __ddiv_rn(1.0, n < 1.0e-12 ? 1.0e-12 : n);   // std::max: NaN stays
    for (int k = 0; k < 8; ++k) tn[r * 8 + k] = static_cast<float>(__dmul_rn(static_cast<double>(cb[r * 8 + k]), scale));
}

__global__ void moss_combine_kernel(const float *__restrict__ w_op, const float *__restrict__ w_out,
                                    const float *__restrict__ b_out, int Q, int C, int R, float *__restrict__ comb) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= static_cast<int64_t>(Q) * C * 9) return;
    const int s = static_cast<int>(t / (static_cast<int64_t>(C) * 9));
    const int rem = static_cast<int>(t % (static_cast<int64_t>(C) * 9));
    const int o = rem / 9;
    const int k = rem % 9;
    const float *orow = w_op + static_cast<int64_t>(o) * R;
    float sum = 0.0f;
    if (k < 8) {
        for (int q = 0; q < R; ++q) sum = sum + orow[q] * w_out[(static_cast<int64_t>(s) * R + q) * 8 + k];
    } else {
        for (int q = 0; q < R; ++q) sum = sum + orow[q] * b_out[static_cast<int64_t>(s) * R + q];
    }
    comb[t] = sum;
}

__global__ void moss_table_kernel(const float *__restrict__ comb, const float *__restrict__ cb, int Q, int64_t N,
                                  int C, float *__restrict__ tables) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= static_cast<int64_t>(Q) * N * C) return;
    const int64_t sn = t / C;
    const int o = static_cast<int>(t % C);
    const int s = static_cast<int>(sn / N);
    const float *cw = comb + (static_cast<int64_t>(s) * C + o) * 9;
    const float *e = cb + sn * 8;
    float sum = cw[8];
    for (int k = 0; k < 8; ++k) sum = sum + cw[k] * e[k];
    tables[t] = sum;
}

// latent[m][o] = b_op[o] + sum over stages of table[s][idx[m][s]][o] (:160-171)
__global__ void moss_decode_kernel(const int32_t *__restrict__ idx, int64_t M, int Q, int64_t N, int C,
                                   const float *__restrict__ tables, const float *__restrict__ b_op,
                                   float *__restrict__ out, int32_t *__restrict__ flags) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= M * C) return;
    const int64_t m = t / C;
    const int o = static_cast<int>(t % C);
    float v = b_op[o];
    for (int s = 0; s < Q; ++s) {
        int32_t code = idx[m * Q + s];
        if (code < 0 || code >= N) {
            flags[AQ_FLAG_BAD_INDEX] = 1;
            code = 0;
        }
        v = v + tables[(static_cast<int64_t>(s) * N + code) * C + o];
    }
    out[t] = v;
}

}  // namespace

// ---------------------------------------------------------------- OuteTTS host


aq_status aq_outetts_prepare(aq_ctx *ctx, const float *d_cb, int64_t rows, float *d_chat) {
    hipLaunchKernelGGL(outetts_chat_kernel, dim3(static_cast<unsigned>((rows + 255) / 256)), dim3(256), 0, ctx->stream,
                       d_cb, rows, d_chat);
    AQ_HIP(ctx, hipGetLastError());
    return AQ_OK;
}

aq_status aq_outetts_launch(aq_ctx *ctx, const aq_outetts_args &args) {
    // the residuals, then the stage tables while they fit the CU's LDS
    // (kOtW waves per block while they and the in-projection fit, fewer for
    // wide latents)
    aq_outetts_args a = args;
    const void *fn = reinterpret_cast<const void *>(outetts_encode_kernel);
    const size_t budget = aq_lds_budget(fn);
    const size_t per_wave = static_cast<size_t>(kHF) * (a.D + 4) * sizeof(float);
    const size_t win = static_cast<size_t>(8) * (a.D + 4) * sizeof(float), chat = static_cast<size_t>(8) * a.N * sizeof(float);
    int nw = kOtW;
    while (nw > 1 && nw * per_wave + win > budget) --nw;
    size_t lds = nw * per_wave;
    a.win_lds = lds + win <= budget ? 1 : 0;
    if (a.win_lds) lds += win;
    a.chat_lds = lds + chat <= budget ? 1 : 0;
    if (a.chat_lds) lds += chat;
    {
        aq_status ls = aq_launch_lds(ctx, fn, lds, "aq_dac_encode (OuteTTS)");
        if (ls != AQ_OK) return ls;
    }
    const int64_t per_block = static_cast<int64_t>(nw) * kHF;
    const unsigned blocks = static_cast<unsigned>((a.M + per_block - 1) / per_block);
    aq_launch_timed(ctx, true, outetts_encode_kernel, dim3(blocks), dim3(kWave * nw), static_cast<uint32_t>(lds), a);
    AQ_HIP(ctx, hipGetLastError());
    return AQ_OK;
}

// ------------------------------------------------------------------- MOSS host

struct aq_moss_quantizer {
    // device of the creating context (the handle keeps no pointer to it, so
    // it may be released after that context is destroyed)
    int device = -1;
    int64_t Q = 0, N = 0, C = 0, R = 0;
    float *d_mem = nullptr;      // one allocation holding the arrays below
    float *d_wip = nullptr;      // [R][C]
    float *d_bip = nullptr;      // [R]
    float *d_win = nullptr;      // [Q][8][R]
    float *d_bin = nullptr;      // [Q][8]
    float *d_cb = nullptr;       // [Q][N][8] raw
    float *d_tn = nullptr;       // [Q][N][8] normalised
    float *d_wout = nullptr;     // [Q][R][8]
    float *d_bout = nullptr;     // [Q][R]
    float *d_bop = nullptr;      // [C]
    float *d_tables = nullptr;   // [Q][N][C] decode latent tables (null: encode only)
};

namespace {
constexpr int64_t kMossMaxR = 1024;
}

extern "C" {

aq_status aq_weight_norm_fold(aq_ctx *ctx, const float *v, const float *g, int64_t rows, int64_t cols, int rule,
                              float *w) {
    if (!ctx || !v || !g || !w) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_weight_norm_fold: null argument");
    if (rule != AQ_WN_OUTETTS && rule != AQ_WN_MOSS)
        return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_weight_norm_fold: unknown rule %d", rule);
    if (rows <= 0 || cols <= 0 || rows > (int64_t{1} << 31) - 1)
        return aq_fail(ctx, AQ_E_SHAPE, "aq_weight_norm_fold: rows=%lld cols=%lld", (long long)rows, (long long)cols);
    aq_device_guard gd(ctx->device);
    hipLaunchKernelGGL(weight_norm_fold_kernel, dim3(static_cast<unsigned>((rows + 63) / 64)), dim3(64), 0, ctx->stream,
                       v, g, rows, cols, rule, w);
    AQ_HIP(ctx, hipGetLastError());
    return AQ_OK;
}

aq_status aq_moss_upload(aq_ctx *ctx, int64_t Q, int64_t N, int64_t code_dim, int64_t rvq_dim, const float *input_w,
                         const float *input_b, const float *in_w, const float *in_b, const float *codebook,
                         const float *out_w, const float *out_b, const float *output_w, const float *output_b,
                         aq_moss_quantizer **out) {
    if (!ctx || !out || !input_w || !input_b || !in_w || !in_b || !codebook || !out_w || !out_b)
        return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_moss_upload: null argument");
    *out = nullptr;
    if ((output_w == nullptr) != (output_b == nullptr))
        return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_moss_upload: output_w and output_b come together (both or neither)");
    if (Q <= 0)
        return aq_fail(ctx, AQ_E_SHAPE, "aq_moss_upload: MOSS codec dequantizer requires a positive quantizer count");
    if (N <= 0 || N % 8 != 0 || N > (int64_t{1} << 20) || code_dim <= 0 || code_dim > (int64_t{1} << 16) ||
        rvq_dim <= 0 || rvq_dim % kIpO != 0 || rvq_dim > kMossMaxR)
        return aq_fail(ctx, AQ_E_SHAPE,
                       "aq_moss_upload: unsupported shape N=%lld code_dim=%lld rvq_dim=%lld (N a multiple of 8, "
                       "rvq_dim a multiple of 64 up to 1024)",
                       (long long)N, (long long)code_dim, (long long)rvq_dim);
    aq_device_guard g(ctx->device);
    const int64_t C = code_dim, R = rvq_dim;
    const int64_t sizes[] = {R * C, R, Q * 8 * R, Q * 8, Q * N * 8, Q * N * 8, Q * R * 8, Q * R, C};
    int64_t total = 0;
    for (int64_t s : sizes) total += (s + 63) / 64 * 64;
    auto *q = new aq_moss_quantizer();
    q->device = ctx->device;
    q->Q = Q;
    q->N = N;
    q->C = C;
    q->R = R;
    if (hipMalloc(&q->d_mem, static_cast<size_t>(total) * sizeof(float)) != hipSuccess) {
        delete q;
        return aq_fail(ctx, AQ_E_DEVICE, "aq_moss_upload: device allocation of %lld bytes failed",
                       (long long)(total * 4));
    }
    float **slots[] = {&q->d_wip, &q->d_bip, &q->d_win, &q->d_bin, &q->d_cb, &q->d_tn, &q->d_wout, &q->d_bout, &q->d_bop};
    // the normalised codebook (slot 5) is built on the device below
    const float *srcs[] = {input_w, input_b, in_w, in_b, codebook, nullptr, out_w, out_b, output_b};
    int64_t off = 0;
    bool ok = true;
    for (int i = 0; i < 9; ++i) {
        *slots[i] = q->d_mem + off;
        if (srcs[i])
            ok = ok && hipMemcpyAsync(*slots[i], srcs[i], static_cast<size_t>(sizes[i]) * sizeof(float),
                                      hipMemcpyHostToDevice, ctx->stream) == hipSuccess;
        off += (sizes[i] + 63) / 64 * 64;
    }
    if (ok) {
        hipLaunchKernelGGL(moss_normalize_kernel, dim3(static_cast<unsigned>((Q * N + 255) / 256)), dim3(256), 0,
                           ctx->stream, q->d_cb, Q * N, q->d_tn);
        ok = hipGetLastError() == hipSuccess;
    }
    float *d_wop = nullptr;
    float *d_comb = nullptr;
    if (ok && output_w) {
        ok = hipMalloc(&q->d_tables, static_cast<size_t>(Q * N * C) * sizeof(float)) == hipSuccess &&
             hipMalloc(&d_wop, static_cast<size_t>(C * R) * sizeof(float)) == hipSuccess &&
             hipMalloc(&d_comb, static_cast<size_t>(Q * C * 9) * sizeof(float)) == hipSuccess;
        ok = ok && hipMemcpyAsync(d_wop, output_w, static_cast<size_t>(C * R) * sizeof(float), hipMemcpyHostToDevice,
                                  ctx->stream) == hipSuccess;
        if (ok) {
            const int64_t nc = Q * C * 9;
            hipLaunchKernelGGL(moss_combine_kernel, dim3(static_cast<unsigned>((nc + 255) / 256)), dim3(256), 0,
                               ctx->stream, d_wop, q->d_wout, q->d_bout, static_cast<int>(Q), static_cast<int>(C),
                               static_cast<int>(R), d_comb);
            const int64_t nt = Q * N * C;
            hipLaunchKernelGGL(moss_table_kernel, dim3(static_cast<unsigned>((nt + 255) / 256)), dim3(256), 0,
                               ctx->stream, d_comb, q->d_cb, static_cast<int>(Q), N, static_cast<int>(C), q->d_tables);
            ok = hipGetLastError() == hipSuccess;
        }
    }
    ok = hipStreamSynchronize(ctx->stream) == hipSuccess && ok;
    if (d_wop) (void)hipFree(d_wop);
    if (d_comb) (void)hipFree(d_comb);
    if (!ok) {
        aq_moss_release(q);
        return aq_fail(ctx, AQ_E_DEVICE, "aq_moss_upload: device copy or table preparation failed");
    }
    *out = q;
    return AQ_OK;
}

aq_status aq_moss_release(aq_moss_quantizer *q) {
    if (!q) return AQ_E_INVALID_ARG;
    {
        aq_device_guard g(q->device);
        if (q->d_mem) (void)hipFree(q->d_mem);
        if (q->d_tables) (void)hipFree(q->d_tables);
    }
    delete q;
    return AQ_OK;
}

aq_status aq_moss_encode(aq_ctx *ctx, const aq_moss_quantizer *q, const float *hidden, int64_t M, int32_t *idx,
                         double *residual, const int32_t *force_idx) {
    if (!ctx || !q) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_moss_encode: null argument");
    if (q->device != ctx->device)
        return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_moss_encode: quantizer belongs to another device");
    // the shape first, as the reference rejects an empty latent before use
    if (M <= 0 || M > (int64_t{1} << 31) - 1)
        return aq_fail(ctx, AQ_E_SHAPE, "aq_moss_encode: MOSS codec quantizer requires a non-empty encoder latent");
    if (!hidden || !idx) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_moss_encode: null argument");
    aq_device_guard g(ctx->device);
    double *res = residual;
    if (!res) {
        aq_status st = aq_ctx_scratch(ctx, 0, static_cast<size_t>(M * q->R) * sizeof(double), reinterpret_cast<void **>(&res));
        if (st != AQ_OK) return st;
    }
    if (force_idx) AQ_HIP(ctx, hipMemsetAsync(ctx->d_flags, 0, sizeof(int32_t) * AQ_FLAG_COUNT, ctx->stream));
    aq_launch_timed(ctx, true, moss_input_kernel,
                    dim3(static_cast<unsigned>((M + kIpF - 1) / kIpF), static_cast<unsigned>(q->R / kIpO)), dim3(256), 0u,
                    hidden, M, static_cast<int>(q->C), static_cast<int>(q->R), static_cast<const float *>(q->d_wip),
                    static_cast<const float *>(q->d_bip), res);
    AQ_HIP(ctx, hipGetLastError());
    aq_moss_args a{};
    a.res = res;
    a.M = M;
    a.R = static_cast<int>(q->R);
    a.N = static_cast<int>(q->N);
    a.Q = static_cast<int>(q->Q);
    a.w_in = q->d_win;
    a.b_in = q->d_bin;
    a.tn = q->d_tn;
    a.cb = q->d_cb;
    a.w_out = q->d_wout;
    a.b_out = q->d_bout;
    a.force_idx = force_idx;
    a.idx = idx;
    a.flags = ctx->d_flags;
    a.write_res = residual ? 1 : 0;
    // the residuals, then the stage tables while they fit the CU's LDS
    // (kMsW waves per block while they and the in-projection fit)
    const void *fn = reinterpret_cast<const void *>(moss_cascade_kernel);
    const size_t budget = aq_lds_budget(fn);
    const size_t per_wave = static_cast<size_t>(kHF) * (q->R + 2) * sizeof(double);
    const size_t win = static_cast<size_t>(8) * (q->R + 4) * sizeof(float), tn = static_cast<size_t>(8) * q->N * sizeof(float);
    int nw = kMsW;
    while (nw > 1 && nw * per_wave + win > budget) --nw;
    size_t lds = nw * per_wave;
    a.win_lds = lds + win <= budget ? 1 : 0;
    if (a.win_lds) lds += win;
    a.tn_lds = lds + tn <= budget ? 1 : 0;
    if (a.tn_lds) lds += tn;
    {
        aq_status ls = aq_launch_lds(ctx, fn, lds, "aq_moss_encode");
        if (ls != AQ_OK) return ls;
    }
    const int64_t per_block = static_cast<int64_t>(nw) * kHF;
    aq_launch_timed(ctx, true, moss_cascade_kernel, dim3(static_cast<unsigned>((M + per_block - 1) / per_block)),
                    dim3(kWave * nw), static_cast<uint32_t>(lds), a);
    AQ_HIP(ctx, hipGetLastError());
    if (force_idx) {
        int32_t flag = 0;
        AQ_HIP(ctx, hipMemcpyAsync(&flag, ctx->d_flags + AQ_FLAG_BAD_INDEX, sizeof(int32_t), hipMemcpyDeviceToHost, ctx->stream));
        AQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (flag)
            return aq_fail(ctx, AQ_E_INDEX_RANGE, "aq_moss_encode: force_idx holds a code outside [0, %lld)", (long long)q->N);
    }
    return AQ_OK;
}

aq_status aq_moss_decode(aq_ctx *ctx, const aq_moss_quantizer *q, const int32_t *idx, int64_t M, float *latent) {
    if (!ctx || !q) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_moss_decode: null argument");
    if (q->device != ctx->device)
        return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_moss_decode: quantizer belongs to another device");
    if (M <= 0) return aq_fail(ctx, AQ_E_SHAPE, "aq_moss_decode: MOSS codec dequantizer requires a non-empty code sequence");
    if (!idx || !latent) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_moss_decode: null argument");
    if (!q->d_tables)
        return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_moss_decode: no output projection was uploaded (encode only)");
    aq_device_guard g(ctx->device);
    AQ_HIP(ctx, hipMemsetAsync(ctx->d_flags, 0, sizeof(int32_t) * AQ_FLAG_COUNT, ctx->stream));
    const int64_t total = M * q->C;
    hipLaunchKernelGGL(moss_decode_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, ctx->stream, idx, M,
                       static_cast<int>(q->Q), q->N, static_cast<int>(q->C), q->d_tables, q->d_bop, latent, ctx->d_flags);
    AQ_HIP(ctx, hipGetLastError());
    int32_t flag = 0;
    AQ_HIP(ctx, hipMemcpyAsync(&flag, ctx->d_flags + AQ_FLAG_BAD_INDEX, sizeof(int32_t), hipMemcpyDeviceToHost, ctx->stream));
    AQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (flag) return aq_fail(ctx, AQ_E_INDEX_RANGE, "aq_moss_decode: MOSS codec code index out of range");
    return AQ_OK;
}

}  // extern "C"
