// Reference harness (test infrastructure, never shipped): runs the
// reference's quantizer op graphs on the reference's own ggml CPU backend,
// compiled from /root/reference/external/ggml by oracle/Makefile into
// oracle/_ref/libaqref-*.so.  It is the ground truth that the plain-C
// restatement (oracle/aq_oracle.c) and the golden fixtures are pinned to.
//
// Each entry point builds the same ggml op sequence as one reference recipe:
//   aqref_dac_rvq     Fish Audio encode quantizer
//                     src/models/fish_audio/codec.cpp:570-611 (quantize_one
//                     587-605), normalized_rows 171-189, l2_normalize_last
//                     323-334, build_quantizer_out 542-550, decode sum 552-568;
//                     Conv1dModule per-batch conv_1d (conv_modules.cpp:284-341)
//                     plus add_bias_if_needed (conv_modules.cpp:152-166).
//   aqref_euclid_rvq  OmniVoice encode quantizer without projections:
//                     score = Linear(2c, -|c|^2) -> argmax -> lookup -> sub
//                     src/models/omnivoice/audio_tokenizer.cpp:1227-1253
//                     (score weights), 1897-1927 (graph).
//   aqref_higgs_rvq   Higgs-style logits = 2*dot - |x|^2 - |c|^2 with an F32
//                     or Q8_0 codebook, argmax, optional top_k, lookup, sub
//                     src/models/higgs_audio_tts/codec.cpp:958-1016.
//
// Data layouts at this C boundary (all row-major, frame-major):
//   x          [M, D]                 M = B*T frames
//   codebooks  [Q, N, K]  (F32)  or   [Q, N, K/32] block_q8_0 (34 B each)
//   idx_out    [M, Q] int32
// All timings cover ggml_graph_compute only (graph build/alloc excluded).

#include "ggml.h"
#include "ggml-cpu.h"
#include "engine/framework/runtime/host_ops.h"

#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

namespace {

struct Ctx {
    ggml_context * ctx = nullptr;
    explicit Ctx(size_t bytes) {
        ggml_init_params p{bytes, nullptr, false};
        ctx = ggml_init(p);
    }
    ~Ctx() { if (ctx) ggml_free(ctx); }
};

double run_graph(ggml_context * ctx, ggml_tensor * out, int n_threads, ggml_cgraph ** gf_out = nullptr,
                 ggml_tensor * out2 = nullptr, ggml_tensor * out3 = nullptr, ggml_tensor * out4 = nullptr) {
    ggml_cgraph * gf = ggml_new_graph_custom(ctx, 8192, false);
    ggml_build_forward_expand(gf, out);
    if (out2) ggml_build_forward_expand(gf, out2);
    if (out3) ggml_build_forward_expand(gf, out3);
    if (out4) ggml_build_forward_expand(gf, out4);
    auto t0 = std::chrono::steady_clock::now();
    ggml_graph_compute_with_ctx(ctx, gf, n_threads);
    auto t1 = std::chrono::steady_clock::now();
    if (gf_out) *gf_out = gf;
    return std::chrono::duration<double, std::milli>(t1 - t0).count();
}

// Fish normalized_rows (codec.cpp:171-189): double sum of squares, float inverse.
std::vector<float> fish_normalized_rows(const float * v, int64_t rows, int64_t cols) {
    std::vector<float> out(static_cast<size_t>(rows * cols), 0.0f);
    for (int64_t r = 0; r < rows; ++r) {
        double sum = 0.0;
        for (int64_t c = 0; c < cols; ++c) {
            const double d = static_cast<double>(v[r * cols + c]);
            sum += d * d;
        }
        const float inv = sum > 0.0 ? static_cast<float>(1.0 / std::sqrt(sum)) : 0.0f;
        for (int64_t c = 0; c < cols; ++c) out[r * cols + c] = v[r * cols + c] * inv;
    }
    return out;
}

// IndexTTS2 normalized_codebook (index_tts2/semantic_codec.cpp:43-58): double
// sum, inv_norm = 1.0F / (float)sqrt(norm), float product (no zero guard).
std::vector<float> indextts2_normalized_rows(const float * v, int64_t rows, int64_t cols) {
    std::vector<float> out(static_cast<size_t>(rows * cols), 0.0f);
    for (int64_t r = 0; r < rows; ++r) {
        double norm = 0.0;
        for (int64_t c = 0; c < cols; ++c) norm += static_cast<double>(v[r * cols + c]) * static_cast<double>(v[r * cols + c]);
        const float inv_norm = 1.0F / static_cast<float>(std::sqrt(norm));
        for (int64_t c = 0; c < cols; ++c) out[r * cols + c] = v[r * cols + c] * inv_norm;
    }
    return out;
}

// Vevo2 l2_normalized_rows (vevo2/components.cpp:566-590): double sum, norm =
// sqrt, inv = (float)(1.0 / norm), float product; a zero row is an error there
// (returns false here).
bool vevo2_normalized_rows(const float * v, int64_t rows, int64_t cols, std::vector<float> & out) {
    out.assign(static_cast<size_t>(rows * cols), 0.0f);
    for (int64_t r = 0; r < rows; ++r) {
        double sum = 0.0;
        for (int64_t c = 0; c < cols; ++c) sum += static_cast<double>(v[r * cols + c]) * static_cast<double>(v[r * cols + c]);
        const double norm = std::sqrt(sum);
        if (norm == 0.0) return false;
        const float inv = static_cast<float>(1.0 / norm);
        for (int64_t c = 0; c < cols; ++c) out[r * cols + c] = v[r * cols + c] * inv;
    }
    return true;
}

// Conv1dModule with kernel 1 (conv_modules.cpp:284-341): one ggml_conv_1d per
// batch element, concatenated along the batch axis, then the repeated bias add.
// input ne = [T, IC, B], weight ne = [1, IC, OC], bias ne = [OC] or null.
ggml_tensor * conv1d_k1(ggml_context * ctx, ggml_tensor * input, ggml_tensor * weight, ggml_tensor * bias) {
    const int64_t T = input->ne[0], IC = input->ne[1], B = input->ne[2];
    const int64_t OC = weight->ne[2];
    ggml_tensor * in = ggml_is_contiguous(input) ? input : ggml_cont(ctx, input);
    ggml_tensor * out = nullptr;
    if (B == 1) {
        out = ggml_conv_1d(ctx, weight, in, 1, 0, 1);
    } else {
        for (int64_t b = 0; b < B; ++b) {
            ggml_tensor * mat = ggml_view_2d(ctx, in, T, IC, in->nb[1], static_cast<size_t>(b) * in->nb[2]);
            ggml_tensor * o = ggml_conv_1d(ctx, weight, mat, 1, 0, 1);
            o = ggml_reshape_3d(ctx, o, T, OC, 1);
            out = out ? ggml_concat(ctx, out, o, 2) : o;
        }
    }
    if (bias) {
        ggml_tensor * bv = ggml_reshape_3d(ctx, bias, 1, OC, 1);
        ggml_tensor * rep = ggml_repeat(ctx, bv, out);
        out = ggml_add(ctx, out, rep);
    }
    return out;
}

// l2_normalize_last (fish codec.cpp:323-334) on ne = [C, T, B].  MulModule
// makes its operands contiguous (primitive_modules.cpp:243-254); ggml_div gets
// `x` as passed in.
// recipe 1 (IndexTTS2 normalize_code_latents, index_tts2/semantic_codec.cpp:110-115)
// takes ggml_sqr, no bias; recipe 2 (Vevo2 build_l2_normalized_rows,
// vevo2/components.cpp:848-863) adds 1e-20 with ggml_scale_bias.
ggml_tensor * l2_normalize_last(ggml_context * ctx, ggml_tensor * x, int recipe = 0) {
    ggml_tensor * xc = ggml_is_contiguous(x) ? x : ggml_cont(ctx, x);
    ggml_tensor * sq = recipe == 1 ? ggml_sqr(ctx, xc) : ggml_mul(ctx, xc, xc);
    ggml_tensor * sum = ggml_sum_rows(ctx, sq);
    ggml_tensor * shifted = recipe == 1 ? sum : ggml_scale_bias(ctx, sum, 1.0f, recipe == 2 ? 1.0e-20f : 1.0e-12f);
    ggml_tensor * denom = ggml_sqrt(ctx, shifted);
    ggml_tensor * rep = ggml_repeat(ctx, denom, x);
    return ggml_div(ctx, x, rep);
}

void to_channel_major(const float * x, int64_t B, int64_t T, int64_t D, float * dst) {
    for (int64_t b = 0; b < B; ++b)
        for (int64_t t = 0; t < T; ++t)
            for (int64_t d = 0; d < D; ++d)
                dst[(b * D + d) * T + t] = x[(b * T + t) * D + d];
}

void from_channel_major(const float * src, int64_t B, int64_t T, int64_t D, float * x) {
    for (int64_t b = 0; b < B; ++b)
        for (int64_t t = 0; t < T; ++t)
            for (int64_t d = 0; d < D; ++d)
                x[(b * T + t) * D + d] = src[(b * D + d) * T + t];
}

}  // namespace

extern "C" {

int aqref_version(void) { return 1; }

// DAC/Fish cosine RVQ.  Weights per stage s:
//   w_in  [Q, 8, D]   b_in  [Q, 8]   (may be null -> no bias add)
//   cb    [Q, N, 8]
//   w_out [Q, D, 8]   b_out [Q, D]  (may be null)
// Outputs: idx [M, Q]; residual [M, D] (final); recon [M, D] = sum_s z_s
// (decode recipe codec.cpp:552-568); stage_res optional [Q, M, D] = residual
// after each stage.  Returns compute milliseconds.
// recipe: 0 Fish, 1 IndexTTS2, 2 Vevo2 (query and codebook normalisation).
// Returns compute milliseconds, or -1 when the recipe rejects the codebook.
// N0 / cb0: the first stage's codebook size and codebook (the Fish semantic
// quantizer, codec.cpp:606); the other stages take N and cb[s - 1].
static double dac_rvq_core(const float * x, int64_t B, int64_t T, int64_t D, int64_t Q, int64_t N0, const float * cb0,
                           int64_t N1, const float * cb1,
                           const float * w_in, const float * b_in,
                           const float * w_out, const float * b_out,
                           int32_t * idx, float * residual, float * recon, float * stage_res,
                           int n_threads, int materialize, int recipe) {
    ggml_cpu_init();
    const int64_t M = B * T;
    double ms = 0.0;
    std::vector<float> res_cm(static_cast<size_t>(M * D));
    std::vector<float> rec_cm(static_cast<size_t>(M * D), 0.0f);
    to_channel_major(x, B, T, D, res_cm.data());
    std::vector<float> tmp(static_cast<size_t>(M * D));
    for (int64_t s = 0; s < Q; ++s) {
        const int64_t N = s == 0 ? N0 : N1;
        const float * cb = s == 0 ? cb0 : cb1 + (s - 1) * N1 * 8;
        const size_t bytes = static_cast<size_t>(M) * static_cast<size_t>(D + N + 64) * 4 * 12 + (64u << 20);
        Ctx c(bytes);
        ggml_context * ctx = c.ctx;
        ggml_tensor * R = ggml_new_tensor_3d(ctx, GGML_TYPE_F32, T, D, B);
        std::memcpy(R->data, res_cm.data(), res_cm.size() * 4);
        ggml_tensor * Win = ggml_new_tensor_3d(ctx, GGML_TYPE_F32, 1, D, 8);
        std::memcpy(Win->data, w_in + s * 8 * D, static_cast<size_t>(8 * D) * 4);
        ggml_tensor * Bin = nullptr;
        if (b_in) {
            Bin = ggml_new_tensor_1d(ctx, GGML_TYPE_F32, 8);
            std::memcpy(Bin->data, b_in + s * 8, 8 * 4);
        }
        ggml_tensor * CB = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, 8, N);
        std::memcpy(CB->data, cb, static_cast<size_t>(N * 8) * 4);
        ggml_tensor * CBn = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, 8, N);
        {
            std::vector<float> nr;
            if (recipe == 1) nr = indextts2_normalized_rows(cb, N, 8);
            else if (recipe == 2) { if (!vevo2_normalized_rows(cb, N, 8, nr)) return -1.0; }
            else nr = fish_normalized_rows(cb, N, 8);
            std::memcpy(CBn->data, nr.data(), nr.size() * 4);
        }
        ggml_tensor * Wout = ggml_new_tensor_3d(ctx, GGML_TYPE_F32, 1, 8, D);
        std::memcpy(Wout->data, w_out + s * D * 8, static_cast<size_t>(D * 8) * 4);
        ggml_tensor * Bout = nullptr;
        if (b_out) {
            Bout = ggml_new_tensor_1d(ctx, GGML_TYPE_F32, D);
            std::memcpy(Bout->data, b_out + s * D, static_cast<size_t>(D) * 4);
        }
        // quantize_one (codec.cpp:587-605)
        ggml_tensor * projected = conv1d_k1(ctx, R, Win, Bin);                  // [T, 8, B]
        ggml_tensor * proj_btd = ggml_permute(ctx, projected, 1, 0, 2, 3);     // [8, T, B] view
        // materialize != 0: the contiguous copy that codec.cpp:324-327 makes on
        // Metal.  materialize == 0: the view as the CPU branch passes it; ggml's
        // CPU binary ops read src0 rows as contiguous (binary-ops.cpp:120-136),
        // so ggml_div then reads the wrong elements (kept only to document it).
        if (materialize) proj_btd = ggml_cont(ctx, proj_btd);
        ggml_tensor * pn = l2_normalize_last(ctx, proj_btd, recipe);           // [8, T, B]
        ggml_tensor * pn2 = ggml_reshape_2d(ctx, ggml_cont(ctx, pn), 8, M);
        ggml_tensor * logits = ggml_mul_mat(ctx, CBn, pn2);                    // [N, M]
        ggml_mul_mat_set_prec(logits, GGML_PREC_F32);
        ggml_tensor * ids = ggml_argmax(ctx, logits);                          // [M]
        ggml_tensor * emb = ggml_get_rows(ctx, CB, ids);                       // [8, M]
        ggml_tensor * emb_btd = ggml_reshape_3d(ctx, emb, 8, T, B);
        ggml_tensor * emb_bdt = ggml_permute(ctx, emb_btd, 1, 0, 2, 3);        // [T, 8, B] view
        ggml_tensor * z = conv1d_k1(ctx, emb_bdt, Wout, Bout);                 // [T, D, B]
        ggml_tensor * Rn = ggml_sub(ctx, R, z);
        ggml_tensor * Rec = ggml_new_tensor_3d(ctx, GGML_TYPE_F32, T, D, B);
        std::memcpy(Rec->data, rec_cm.data(), rec_cm.size() * 4);
        ggml_tensor * RecN = s == 0 ? z : ggml_add(ctx, Rec, z);
        ms += run_graph(ctx, Rn, n_threads, nullptr, ids, RecN);
        std::memcpy(res_cm.data(), Rn->data, res_cm.size() * 4);
        std::memcpy(rec_cm.data(), RecN->data, rec_cm.size() * 4);
        const int32_t * ip = static_cast<const int32_t *>(ids->data);
        for (int64_t m = 0; m < M; ++m) idx[m * Q + s] = ip[m];
        if (stage_res) from_channel_major(res_cm.data(), B, T, D, stage_res + s * M * D);
    }
    if (residual) from_channel_major(res_cm.data(), B, T, D, residual);
    if (recon) from_channel_major(rec_cm.data(), B, T, D, recon);
    return ms;
}

double aqref_dac_rvq_ex(const float * x, int64_t B, int64_t T, int64_t D, int64_t Q, int64_t N,
                        const float * w_in, const float * b_in, const float * cb,
                        const float * w_out, const float * b_out,
                        int32_t * idx, float * residual, float * recon, float * stage_res,
                        int n_threads, int materialize, int recipe) {
    return dac_rvq_core(x, B, T, D, Q, N, cb, N, cb + N * 8, w_in, b_in, w_out, b_out, idx, residual, recon,
                        stage_res, n_threads, materialize, recipe);
}

// The Fish cascade of build_encode_quantizer (codec.cpp:606-608): a semantic
// quantizer of N0 codes (cb0 [N0, 8]) and Q - 1 residual quantizers of N codes
// (cb [Q - 1, N, 8]); recon is the decoder's sum.
double aqref_dac_rvq_mixed(const float * x, int64_t B, int64_t T, int64_t D, int64_t Q, int64_t N0, int64_t N,
                           const float * w_in, const float * b_in, const float * cb0, const float * cb,
                           const float * w_out, const float * b_out,
                           int32_t * idx, float * residual, float * recon, int n_threads) {
    return dac_rvq_core(x, B, T, D, Q, N0, cb0, N, cb, w_in, b_in, w_out, b_out, idx, residual, recon, nullptr,
                        n_threads, 1, 0);
}

double aqref_dac_rvq(const float * x, int64_t B, int64_t T, int64_t D, int64_t Q, int64_t N,
                     const float * w_in, const float * b_in, const float * cb,
                     const float * w_out, const float * b_out,
                     int32_t * idx, float * residual, float * recon, float * stage_res,
                     int n_threads, int materialize) {
    return aqref_dac_rvq_ex(x, B, T, D, Q, N, w_in, b_in, cb, w_out, b_out, idx, residual, recon, stage_res,
                            n_threads, materialize, 0);
}

// OmniVoice-style Euclidean RVQ (no projections): logits = (2c)·x + (-|c|^2).
// x [M, K]; cb [Q, N, K]; idx [M, Q]; residual [M, K]; logit_best [M, Q] (optional).
double aqref_euclid_rvq(const float * x, int64_t M, int64_t K, int64_t Q, int64_t N, const float * cb,
                        int32_t * idx, float * residual, float * logit_best, int n_threads) {
    ggml_cpu_init();
    double ms = 0.0;
    std::vector<float> res(x, x + M * K);
    for (int64_t s = 0; s < Q; ++s) {
        const size_t bytes = static_cast<size_t>(M) * static_cast<size_t>(2 * N + 4 * K) * 4 + static_cast<size_t>(N * K) * 12 + (64u << 20);
        Ctx c(bytes);
        ggml_context * ctx = c.ctx;
        const float * cbs = cb + s * N * K;
        ggml_tensor * R = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, K, M);
        std::memcpy(R->data, res.data(), res.size() * 4);
        ggml_tensor * W = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, K, N);
        ggml_tensor * Bs = ggml_new_tensor_1d(ctx, GGML_TYPE_F32, N);
        ggml_tensor * CB = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, K, N);
        std::memcpy(CB->data, cbs, static_cast<size_t>(N * K) * 4);
        float * wp = static_cast<float *>(W->data);
        float * bp = static_cast<float *>(Bs->data);
        for (int64_t r = 0; r < N; ++r) {   // audio_tokenizer.cpp:1227-1237
            double norm = 0.0;
            for (int64_t k = 0; k < K; ++k) {
                const float v = cbs[r * K + k];
                wp[r * K + k] = 2.0f * v;
                norm += static_cast<double>(v) * static_cast<double>(v);
            }
            bp[r] = static_cast<float>(-norm);
        }
        ggml_tensor * lg = ggml_mul_mat(ctx, W, R);                           // [N, M]
        ggml_mul_mat_set_prec(lg, GGML_PREC_F32);
        lg = ggml_add(ctx, lg, Bs);
        ggml_tensor * ids = ggml_argmax(ctx, lg);
        ggml_tensor * q = ggml_get_rows(ctx, CB, ids);
        ggml_tensor * Rn = ggml_sub(ctx, R, q);
        ms += run_graph(ctx, Rn, n_threads, nullptr, ids, lg);
        std::memcpy(res.data(), Rn->data, res.size() * 4);
        const int32_t * ip = static_cast<const int32_t *>(ids->data);
        const float * lp = static_cast<const float *>(lg->data);
        for (int64_t m = 0; m < M; ++m) {
            idx[m * Q + s] = ip[m];
            if (logit_best) logit_best[m * Q + s] = lp[m * N + ip[m]];
        }
    }
    if (residual) std::memcpy(residual, res.data(), res.size() * 4);
    return ms;
}

// Higgs-style Euclidean RVQ: logits = scale(dot,2) - |x|^2 - |c|^2 (codec.cpp:975-999).
// cb_type 0 = F32 codebook [Q, N, K]; 1 = Q8_0 blocks [Q, N, K/32] (34 B each).
// Outputs: idx [M, Q]; residual [M, K]; dist [M, Q] = -logit[idx] (optional);
// topk_idx / topk_logit [M, Q, topk] in ggml_top_k order (optional, topk > 0).
double aqref_higgs_rvq(const float * x, int64_t M, int64_t K, int64_t Q, int64_t N,
                       const void * cb, int cb_type, int topk,
                       int32_t * idx, float * residual, float * dist,
                       int32_t * topk_idx, float * topk_logit, int n_threads) {
    ggml_cpu_init();
    double ms = 0.0;
    std::vector<float> res(x, x + M * K);
    const ggml_type t = cb_type == 1 ? GGML_TYPE_Q8_0 : GGML_TYPE_F32;
    const size_t cb_bytes = ggml_row_size(t, K) * static_cast<size_t>(N);
    for (int64_t s = 0; s < Q; ++s) {
        const size_t bytes = static_cast<size_t>(M) * static_cast<size_t>(N * 6 + 6 * K) * 4 + static_cast<size_t>(N * K) * 16 + (64u << 20);
        Ctx c(bytes);
        ggml_context * ctx = c.ctx;
        ggml_tensor * R = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, K, M);
        std::memcpy(R->data, res.data(), res.size() * 4);
        ggml_tensor * CB = ggml_new_tensor_2d(ctx, t, K, N);
        std::memcpy(CB->data, static_cast<const char *>(cb) + s * cb_bytes, cb_bytes);
        // MatMulModule(flat, codebook_t) -> ggml_mul_mat(codebook, flat) (primitive_modules.cpp:186-212)
        ggml_tensor * dot = ggml_mul_mat(ctx, CB, R);                           // [N, M]
        ggml_tensor * x2 = ggml_sum_rows(ctx, ggml_mul(ctx, R, R));              // [1, M]
        x2 = ggml_repeat(ctx, x2, dot);
        ggml_tensor * cbf = t == GGML_TYPE_F32 ? CB : ggml_cast(ctx, CB, GGML_TYPE_F32);
        ggml_tensor * e2 = ggml_sum_rows(ctx, ggml_mul(ctx, cbf, cbf));          // [1, N]
        e2 = ggml_reshape_2d(ctx, e2, N, 1);
        e2 = ggml_repeat(ctx, e2, dot);
        ggml_tensor * lg = ggml_scale(ctx, dot, 2.0f);
        lg = ggml_sub(ctx, lg, x2);
        lg = ggml_sub(ctx, lg, e2);
        ggml_tensor * ids = ggml_argmax(ctx, lg);
        ggml_tensor * tk = topk > 0 ? ggml_top_k(ctx, lg, topk) : nullptr;
        ggml_tensor * q = ggml_get_rows(ctx, CB, ids);                          // dequantized rows
        ggml_tensor * Rn = ggml_sub(ctx, R, q);
        ms += run_graph(ctx, Rn, n_threads, nullptr, ids, lg, tk);
        std::memcpy(res.data(), Rn->data, res.size() * 4);
        const int32_t * ip = static_cast<const int32_t *>(ids->data);
        const float * lp = static_cast<const float *>(lg->data);
        for (int64_t m = 0; m < M; ++m) {
            idx[m * Q + s] = ip[m];
            if (dist) dist[m * Q + s] = -lp[m * N + ip[m]];
            if (tk) {
                const int32_t * tp = static_cast<const int32_t *>(tk->data) + m * topk;
                for (int k = 0; k < topk; ++k) {
                    topk_idx[(m * Q + s) * topk + k] = tp[k];
                    topk_logit[(m * Q + s) * topk + k] = lp[m * N + tp[k]];
                }
            }
        }
    }
    if (residual) std::memcpy(residual, res.data(), res.size() * 4);
    return ms;
}

// OmniVoice / Higgs RVQ with the per-stage projections
// (omnivoice/audio_tokenizer.cpp:1886-1927; higgs_audio_tts/codec.cpp:958-1016).
// The residual is kept frame-major [H, M] (ne order): the graphs' bct <-> btc
// transposes only move data, and LinearModule makes its input contiguous
// (ensure_backend_addressable_layout, src/framework/core/module.cpp:199-210)
// before mul_mat + bias add (linear_module.cpp:73-108).
// recipe 0 OmniVoice (score = Linear(2c, -|c|^2)), 1 Higgs (2*dot - x2 - e2).
// cb_type / proj_type: 0 F32, 1 Q8_0 blocks.  w_in [Q, K, H], w_out [Q, H, K]
// (row-major: ne = [H, K] and [K, H]); b_in [Q, K], b_out [Q, H] nullable.
// Outputs idx [M, Q]; residual [M, H]; dist [M, Q] = -logit[idx] (nullable);
// topk_idx / topk_logit [M, Q, topk] (Higgs, topk > 0).
double aqref_projected_rvq(const float * x, int64_t M, int64_t H, int64_t K, int64_t Q, int64_t N, int recipe,
                           const void * cb, int cb_type, const void * w_in, const float * b_in,
                           const void * w_out, const float * b_out, int proj_type, int topk,
                           int32_t * idx, float * residual, float * dist,
                           int32_t * topk_idx, float * topk_logit, int n_threads) {
    ggml_cpu_init();
    double ms = 0.0;
    std::vector<float> res(x, x + M * H);
    const ggml_type tc = cb_type == 1 ? GGML_TYPE_Q8_0 : GGML_TYPE_F32;
    const ggml_type tp = proj_type == 1 ? GGML_TYPE_Q8_0 : GGML_TYPE_F32;
    const size_t cb_bytes = ggml_row_size(tc, K) * static_cast<size_t>(N);
    const size_t wi_bytes = ggml_row_size(tp, H) * static_cast<size_t>(K);
    const size_t wo_bytes = ggml_row_size(tp, K) * static_cast<size_t>(H);
    for (int64_t s = 0; s < Q; ++s) {
        const size_t bytes = static_cast<size_t>(M) * static_cast<size_t>(N * 8 + 6 * H + 8 * K) * 4 +
                             static_cast<size_t>(N * K) * 16 + static_cast<size_t>(H * K) * 12 + (64u << 20);
        Ctx c(bytes);
        ggml_context * ctx = c.ctx;
        ggml_tensor * R = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, H, M);
        std::memcpy(R->data, res.data(), res.size() * 4);
        ggml_tensor * CB = ggml_new_tensor_2d(ctx, tc, K, N);
        std::memcpy(CB->data, static_cast<const char *>(cb) + s * cb_bytes, cb_bytes);
        ggml_tensor * Wi = ggml_new_tensor_2d(ctx, tp, H, K);
        std::memcpy(Wi->data, static_cast<const char *>(w_in) + s * wi_bytes, wi_bytes);
        ggml_tensor * Wo = ggml_new_tensor_2d(ctx, tp, K, H);
        std::memcpy(Wo->data, static_cast<const char *>(w_out) + s * wo_bytes, wo_bytes);
        ggml_tensor * p = ggml_mul_mat(ctx, Wi, R);                              // [K, M]
        ggml_mul_mat_set_prec(p, GGML_PREC_F32);
        if (b_in) {
            ggml_tensor * Bi = ggml_new_tensor_1d(ctx, GGML_TYPE_F32, K);
            std::memcpy(Bi->data, b_in + s * K, static_cast<size_t>(K) * 4);
            p = ggml_add(ctx, p, Bi);
        }
        ggml_tensor * lg = nullptr;
        if (recipe == 0) {   // audio_tokenizer.cpp:1227-1237 score weights
            ggml_tensor * W = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, K, N);
            ggml_tensor * Bs = ggml_new_tensor_1d(ctx, GGML_TYPE_F32, N);
            const float * cbs = static_cast<const float *>(cb) + s * N * K;
            float * wp = static_cast<float *>(W->data);
            float * bp = static_cast<float *>(Bs->data);
            for (int64_t r = 0; r < N; ++r) {
                double norm = 0.0;
                for (int64_t k = 0; k < K; ++k) {
                    const float v = cbs[r * K + k];
                    wp[r * K + k] = 2.0f * v;
                    norm += static_cast<double>(v) * static_cast<double>(v);
                }
                bp[r] = static_cast<float>(-norm);
            }
            lg = ggml_mul_mat(ctx, W, p);
            ggml_mul_mat_set_prec(lg, GGML_PREC_F32);
            lg = ggml_add(ctx, lg, Bs);
        } else {             // codec.cpp:975-999
            ggml_tensor * dot = ggml_mul_mat(ctx, CB, p);                        // [N, M]
            ggml_tensor * x2 = ggml_repeat(ctx, ggml_sum_rows(ctx, ggml_mul(ctx, p, p)), dot);
            ggml_tensor * cbf = tc == GGML_TYPE_F32 ? CB : ggml_cast(ctx, CB, GGML_TYPE_F32);
            ggml_tensor * e2 = ggml_reshape_2d(ctx, ggml_sum_rows(ctx, ggml_mul(ctx, cbf, cbf)), N, 1);
            e2 = ggml_repeat(ctx, e2, dot);
            lg = ggml_sub(ctx, ggml_sub(ctx, ggml_scale(ctx, dot, 2.0f), x2), e2);
        }
        ggml_tensor * ids = ggml_argmax(ctx, lg);
        ggml_tensor * tk = topk > 0 ? ggml_top_k(ctx, lg, topk) : nullptr;
        ggml_tensor * emb = ggml_get_rows(ctx, CB, ids);                         // [K, M] F32
        ggml_tensor * z = ggml_mul_mat(ctx, Wo, emb);                            // [H, M]
        ggml_mul_mat_set_prec(z, GGML_PREC_F32);
        if (b_out) {
            ggml_tensor * Bo = ggml_new_tensor_1d(ctx, GGML_TYPE_F32, H);
            std::memcpy(Bo->data, b_out + s * H, static_cast<size_t>(H) * 4);
            z = ggml_add(ctx, z, Bo);
        }
        ggml_tensor * Rn = ggml_sub(ctx, R, z);
        ms += run_graph(ctx, Rn, n_threads, nullptr, ids, lg, tk);
        std::memcpy(res.data(), Rn->data, res.size() * 4);
        const int32_t * ip = static_cast<const int32_t *>(ids->data);
        const float * lp = static_cast<const float *>(lg->data);
        for (int64_t m = 0; m < M; ++m) {
            idx[m * Q + s] = ip[m];
            if (dist) dist[m * Q + s] = -lp[m * N + ip[m]];
            if (tk) {
                const int32_t * tkp = static_cast<const int32_t *>(tk->data) + m * topk;
                for (int k = 0; k < topk; ++k) {
                    topk_idx[(m * Q + s) * topk + k] = tkp[k];
                    topk_logit[(m * Q + s) * topk + k] = lp[m * N + tkp[k]];
                }
            }
        }
    }
    if (residual) std::memcpy(residual, res.data(), res.size() * 4);
    return ms;
}

// LinearModule::forward (linear_module.cpp:73-108) on M frame-major rows:
// out = mul_mat(W, x) (+ ggml_add bias).  W [n_out, k] F32 (w_type 0) or
// Q8_0 rows (1); x [M, k]; out [M, n_out].
double aqref_linear(const void * w, int w_type, const float * bias, int64_t n_out, int64_t k, int64_t M,
                    const float * x, float * out, int n_threads) {
    ggml_cpu_init();
    const ggml_type tp = w_type == 1 ? GGML_TYPE_Q8_0 : GGML_TYPE_F32;
    const size_t w_bytes = ggml_row_size(tp, k) * static_cast<size_t>(n_out);
    Ctx c(w_bytes + static_cast<size_t>(M) * static_cast<size_t>(k + 3 * n_out) * 4 + (64u << 20));
    ggml_context * ctx = c.ctx;
    ggml_tensor * W = ggml_new_tensor_2d(ctx, tp, k, n_out);
    std::memcpy(W->data, w, w_bytes);
    ggml_tensor * X = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, k, M);
    std::memcpy(X->data, x, static_cast<size_t>(M * k) * 4);
    ggml_tensor * y = ggml_mul_mat(ctx, W, X);
    ggml_mul_mat_set_prec(y, GGML_PREC_F32);
    if (bias) {
        ggml_tensor * B = ggml_new_tensor_1d(ctx, GGML_TYPE_F32, n_out);
        std::memcpy(B->data, bias, static_cast<size_t>(n_out) * 4);
        y = ggml_add(ctx, y, B);
    }
    const double ms = run_graph(ctx, y, n_threads);
    std::memcpy(out, y->data, static_cast<size_t>(M * n_out) * 4);
    return ms;
}

// Their decode (omnivoice/audio_tokenizer.cpp:1745-1771; higgs codec.cpp:
// 1040-1065): latent = z_0, then latent = latent + z_s, z_s =
// Linear(project_out)(get_rows(c_s, idx[:, s])).  idx [M, Q]; out [M, H].
double aqref_projected_decode(const int32_t * idx, int64_t M, int64_t H, int64_t K, int64_t Q, int64_t N,
                              const void * cb, int cb_type, const void * w_out, const float * b_out, int proj_type,
                              float * out, int n_threads) {
    ggml_cpu_init();
    const ggml_type tc = cb_type == 1 ? GGML_TYPE_Q8_0 : GGML_TYPE_F32;
    const ggml_type tp = proj_type == 1 ? GGML_TYPE_Q8_0 : GGML_TYPE_F32;
    const size_t cb_bytes = ggml_row_size(tc, K) * static_cast<size_t>(N);
    const size_t wo_bytes = ggml_row_size(tp, K) * static_cast<size_t>(H);
    const size_t bytes = static_cast<size_t>(Q) * (cb_bytes + wo_bytes + static_cast<size_t>(M) * (3 * H + 2 * K + 4) * 4) +
                         (64u << 20);
    Ctx c(bytes);
    ggml_context * ctx = c.ctx;
    ggml_tensor * latent = nullptr;
    for (int64_t s = 0; s < Q; ++s) {
        ggml_tensor * ids = ggml_new_tensor_1d(ctx, GGML_TYPE_I32, M);
        int32_t * ip = static_cast<int32_t *>(ids->data);
        for (int64_t m = 0; m < M; ++m) ip[m] = idx[m * Q + s];
        ggml_tensor * CB = ggml_new_tensor_2d(ctx, tc, K, N);
        std::memcpy(CB->data, static_cast<const char *>(cb) + s * cb_bytes, cb_bytes);
        ggml_tensor * Wo = ggml_new_tensor_2d(ctx, tp, K, H);
        std::memcpy(Wo->data, static_cast<const char *>(w_out) + s * wo_bytes, wo_bytes);
        ggml_tensor * z = ggml_mul_mat(ctx, Wo, ggml_get_rows(ctx, CB, ids));
        if (b_out) {
            ggml_tensor * Bo = ggml_new_tensor_1d(ctx, GGML_TYPE_F32, H);
            std::memcpy(Bo->data, b_out + s * H, static_cast<size_t>(H) * 4);
            z = ggml_add(ctx, z, Bo);
        }
        latent = latent ? ggml_add(ctx, latent, z) : z;
    }
    const double ms = run_graph(ctx, latent, n_threads);
    std::memcpy(out, latent->data, static_cast<size_t>(M * H) * 4);
    return ms;
}

// ggml_top_k alone (ops.cpp:8423-8456) on rows of n values: v [rows, n],
// dst [rows, k] in ggml's order.
void aqref_top_k(const float * v, int64_t rows, int64_t n, int k, int32_t * dst, int n_threads) {
    ggml_cpu_init();
    Ctx c(static_cast<size_t>(rows) * static_cast<size_t>(n + k) * 8 + (16u << 20));
    ggml_tensor * V = ggml_new_tensor_2d(c.ctx, GGML_TYPE_F32, n, rows);
    std::memcpy(V->data, v, static_cast<size_t>(rows * n) * 4);
    ggml_tensor * tk = ggml_top_k(c.ctx, V, k);
    run_graph(c.ctx, tk, n_threads);
    std::memcpy(dst, tk->data, static_cast<size_t>(rows * k) * 4);
}

// The reference's framework host quantizer, engine::runtime::VectorQuantizer
// (src/framework/runtime/host_ops.cpp:236-273, compiled from the reference
// sources): x_len floats of input and cb_len floats of codebook as given, so
// the reference's own size check sees the true lengths.  Writes the nearest
// codewords (x_len floats) and returns 0, or -1 when the reference throws.
int aqref_vector_quantizer(const float * x, int64_t x_len, int64_t batch, int64_t steps, int64_t dim,
                           const float * cb, int64_t cb_len, int64_t N, float * out) {
    try {
        std::vector<float> in(x, x + x_len);
        std::vector<float> code(cb, cb + cb_len);
        const auto res = engine::runtime::VectorQuantizer().compute(in, code, batch, steps, dim, N);
        std::memcpy(out, res.values.data(), res.values.size() * sizeof(float));
        return 0;
    } catch (...) {
        return -1;
    }
}

// x86 query quantisation as ggml applies it inside mul_mat (quantize_row_q8_0,
// ggml-cpu/arch/x86/quants.c:302), exposed for known-answer checks.
void aqref_quantize_row_q8_0(const float * x, void * y, int64_t k) {
    ggml_cpu_init();
    const auto * tr = ggml_get_type_traits_cpu(GGML_TYPE_Q8_0);
    tr->from_float(x, y, k);
}

// ggml_vec_dot_f32 (ggml-cpu/vec.cpp:11-135) through the CPU type traits:
// one dot product of n floats in the arithmetic of mul_mat's non-tinyBLAS
// path, as this build's compiler laid out its scalar leftover loop.
float aqref_vec_dot_f32(int n, const float * x, const float * y) {
    ggml_cpu_init();
    const auto * tr = ggml_get_type_traits_cpu(GGML_TYPE_F32);
    float s = 0.0f;
    tr->vec_dot(n, &s, 0, x, 0, y, 0, 1);
    return s;
}

// Reference-rounding quantisation (ggml_quantize_chunk -> quantize_row_q8_0_ref,
// ggml-quants.c:236-256), used by the reference's weight store for Q8_0 weights.
void aqref_quantize_chunk_q8_0(const float * x, void * y, int64_t rows, int64_t k) {
    ggml_cpu_init();
    ggml_quantize_chunk(GGML_TYPE_Q8_0, x, y, 0, rows, k, nullptr);
}

}  // extern "C"
