/*
 * aq_oracle.h -- CPU restatement of the reference quantizer path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or as the labelled CPU baseline), never as the thing measured or shipped.
 *
 * Every function restates, in plain C, the arithmetic that the reference's
 * ggml CPU backend (vendored at external/ggml, v0.12.0) performs for the op
 * it names, on an AVX-512 x86 host built with the reference's defaults
 * (-O3 -march=native, GCC, -ffp-contract=fast by GNU dialect).  Operation
 * order, fused multiply-adds, double accumulations and tie rules follow the
 * cited lines so results are bit-identical, which the CPU tests check against
 * oracle/_ref (ggml itself) and the golden fixtures.
 */
#ifndef AQ_ORACLE_H
#define AQ_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    uint16_t d;      /* fp16 scale */
    int8_t qs[32];
} aqo_block_q8_0;    /* ggml-common.h:241-246 (34 bytes, packed) */

/* ---- primitives ---------------------------------------------------------- */
float aqo_vec_dot_f32(int n, const float *x, const float *y);
float aqo_vec_dot_f32_tail(int n, const float *x, const float *y, int tail_mod);
float aqo_tinyblas_dot_f32(int k, const float *a, const float *b);
int   aqo_mul_mat_f32_uses_tinyblas(int64_t m, int64_t n, int64_t k);
int   aqo_argmax_f32(int n, const float *x);
float aqo_sum_f32(int n, const float *x);
uint16_t aqo_fp32_to_fp16(float f);
float aqo_fp16_to_fp32(uint16_t h);
void  aqo_quantize_row_q8_0_x86(const float *x, aqo_block_q8_0 *y, int k);
void  aqo_quantize_row_q8_0_ref(const float *x, aqo_block_q8_0 *y, int k);
void  aqo_dequantize_row_q8_0(const aqo_block_q8_0 *x, float *y, int k);
float aqo_dot_q8_0(int nb, const aqo_block_q8_0 *a, const aqo_block_q8_0 *b);

/* ---- whole-path restatements -------------------------------------------- */
/* DAC cosine RVQ (Fish recipe).  x [B*T, D] frame-major; weights per stage:
 * w_in [Q,8,D], b_in [Q,8] (nullable), cb [Q,N,8], w_out [Q,D,8],
 * b_out [Q,D] (nullable).  force_idx [M,Q] (nullable) teacher-forces the code
 * used for the residual update; idx always receives the computed argmax. */
int aqo_dac_rvq(const float *x, int64_t B, int64_t T, int64_t D, int64_t Q, int64_t N,
                const float *w_in, const float *b_in, const float *cb,
                const float *w_out, const float *b_out, const int32_t *force_idx,
                int32_t *idx, float *residual, float *recon);
/* Same with the normalisation recipe: 0 Fish, 1 IndexTTS2, 2 Vevo2; w_out may
 * be NULL (codes only; the residual stays the input). */
int aqo_dac_rvq_ex(const float *x, int64_t B, int64_t T, int64_t D, int64_t Q, int64_t N,
                   const float *w_in, const float *b_in, const float *cb,
                   const float *w_out, const float *b_out, const int32_t *force_idx,
                   int32_t *idx, float *residual, float *recon, int recipe);

/* The Fish cascade with a semantic stage of N0 codes (cb0 [N0,8]) before
 * Q-1 residual stages of N codes (cb [Q-1,N,8]); weights [Q,...] as above. */
int aqo_dac_rvq_mixed(const float *x, int64_t B, int64_t T, int64_t D, int64_t Q, int64_t N0, int64_t N,
                      const float *w_in, const float *b_in, const float *cb0, const float *cb,
                      const float *w_out, const float *b_out, const int32_t *force_idx,
                      int32_t *idx, float *residual, float *recon);
/* OmniVoice-style Euclidean RVQ: logit = dot(2c, r) + (-|c|^2). x [M,K],
 * cb [Q,N,K].  logit_best [M,Q] nullable. */
int aqo_euclid_rvq(const float *x, int64_t M, int64_t K, int64_t Q, int64_t N,
                   const float *cb, const int32_t *force_idx,
                   int32_t *idx, float *residual, float *logit_best);

/* Higgs-style Euclidean RVQ: logit = ((2*dot) - |x|^2) - |c|^2, F32 codebook
 * (cb_type 0, [Q,N,K] floats) or Q8_0 (cb_type 1, [Q,N,K/32] blocks).
 * dist [M,Q] = -logit[idx]; topk_idx/topk_logit [M,Q,topk] as ggml_top_k
 * leaves them (aqo_top_k_f32: the same set and the same order). */
int aqo_higgs_rvq(const float *x, int64_t M, int64_t K, int64_t Q, int64_t N,
                  const void *cb, int cb_type, int topk, const int32_t *force_idx,
                  int32_t *idx, float *residual, float *dist,
                  int32_t *topk_idx, float *topk_logit);

/* OmniVoice / Higgs RVQ with per-stage project_in (H -> K) and project_out
 * (K -> H) around the score, the residual kept in hidden space
 * (omnivoice/audio_tokenizer.cpp:1886-1927, higgs_audio_tts/codec.cpp:958-1016).
 * recipe 0 OmniVoice, 1 Higgs; cb [Q,N,K] F32 (cb_type 0) or [Q,N,K/32] Q8_0
 * blocks (cb_type 1); w_in [Q,K,H] and w_out [Q,H,K] F32 (proj_type 0) or
 * Q8_0 blocks (proj_type 1); b_in [Q,K], b_out [Q,H] nullable.  x [M,H];
 * idx [M,Q]; residual [M,H]; dist [M,Q] nullable; topk outputs [M,Q,topk]. */
int aqo_projected_rvq(const float *x, int64_t M, int64_t H, int64_t K, int64_t Q, int64_t N, int recipe,
                      const void *cb, int cb_type, const void *w_in, const float *b_in, const void *w_out,
                      const float *b_out, int proj_type, int topk, const int32_t *force_idx, int32_t *idx,
                      float *residual, float *dist, int32_t *topk_idx, float *topk_logit);
/* Their decode: out[m] = sum over stages, in order, of project_out(c_s[idx]). */
int aqo_projected_decode(const int32_t *idx, int64_t M, int64_t H, int64_t K, int64_t Q, int64_t N,
                         const void *cb, int cb_type, const void *w_out, const float *b_out, int proj_type,
                         float *out);
/* ggml_top_k of one row: the k indices std::partial_sort (libstdc++) keeps
 * with comp(a, b) = v[a] > v[b], in its order, dst[0] and dst[1] swapped. */
void aqo_top_k_f32(const float *v, int64_t n, int k, int32_t *dst);

/* Direct-distance RVQ (VectorQuantizer::compute / Qwen3 nearest_code):
 * rounded squares added in order, first index of the minimum.  dist [M,Q]
 * (nullable) receives the winner's distance. */
int aqo_direct_rvq(const float *x, int64_t M, int64_t K, int64_t Q, int64_t N, const float *cb,
                   const int32_t *force_idx, int32_t *idx, float *residual, float *dist);

/* Codebook gather (get_rows, ops.cpp:4923-4962 / 4797-4840). Returns -1 on an
 * out-of-range index (the reference asserts). */
int aqo_gather_f32(const float *cb, int64_t N, int64_t K, const int32_t *idx, int64_t M, float *out);

/* EMA codebook materialisation (Mimi / Qwen3 speech tokenizer):
 * cb[q,n,k] = embedding_sum[q,n,k] / std::max(cluster_usage[q,n], eps). */
int aqo_ema_codebook(const float *embedding_sum, const float *cluster_usage, int64_t Q, int64_t N, int64_t K,
                     float eps, float *cb);
/* OuteTTS DAC host quantizer (quantize_reference,
 * src/community_models/outetts/dac.cpp:376-456), generalised to Q stages,
 * D latent channels, N codes of dim 8: fp32, every product rounded before it
 * is added (the reference's engine code is built without FMA), bias first,
 * first index of the minimum of |p/|p|' - c/|c|'|^2 with |v|' = sqrt(.)+1e-12.
 * b_in / b_out may be NULL (zeros).  x [M,D], w_in [Q,8,D], cb [Q,N,8],
 * w_out [Q,D,8]; idx [M,Q]; residual [M,D] (required). */
int aqo_outetts_rvq(const float *x, int64_t M, int64_t D, int64_t Q, int64_t N,
                    const float *w_in, const float *b_in, const float *cb,
                    const float *w_out, const float *b_out, const int32_t *force_idx,
                    int32_t *idx, float *residual);

/* MOSS weight-norm reconstruction (reconstruct_weight_norm,
 * src/models/moss/shared/audio_tokenizer_quantizer.cpp:17-39):
 * w[o,k] = v[o,k] * (float)(g[o] / sqrt(sum_k (double)v[o,k]^2)). */
void aqo_moss_weight_norm(const float *g, const float *v, int64_t out_ch, int64_t in_ch, float *w);
void aqo_outetts_weight_norm(const float *v, const float *g, int64_t rows, int64_t cols, float *w);
int aqo_linear(const void *w, int w_type, const float *bias, int64_t n_out, int64_t k, int64_t M, const float *x,
               float *out);

/* MOSS codebook row normalisation (constructor, :116-130):
 * row * (1 / max(sqrt(sum (double)c^2), 1e-12)) in double, stored as float. */
void aqo_moss_normalize_rows(const float *cb, int64_t rows, int64_t dim, float *out);

/* MOSS RLFQ encode (MossAudioTokenizerQuantizer::encode, :174-271): fp64
 * input projection [C -> R], then per stage an fp64 in-projection [R -> 8],
 * L2 normalisation with max(|e|, 1e-12), the first index of the maximum dot
 * with the normalised codebook, and the fp64 residual update by the
 * out-projection of the raw codebook row.  hidden [M,C], w_ip [R,C], b_ip [R],
 * w_in [Q,8,R], b_in [Q,8], cb [Q,N,8] (raw), w_out [Q,R,8], b_out [Q,R];
 * idx [M,Q]; residual [M,R] doubles (nullable). */
int aqo_moss_rvq(const float *hidden, int64_t M, int64_t C, int64_t R, int64_t Q, int64_t N,
                 const float *w_ip, const float *b_ip, const float *w_in, const float *b_in,
                 const float *cb, const float *w_out, const float *b_out, const int32_t *force_idx,
                 int32_t *idx, double *residual);

/* MOSS dequantisation (MossAudioTokenizerQuantizer::decode, :139-172 with the
 * constructor's latent tables, :77-115): latent[m,c] = b_op[c] + sum over
 * stages of table_q[idx[m,q], c] in fp32, frame-major [M,C].  w_op [C,R].
 * Returns -1 on an out-of-range code. */
int aqo_moss_decode(const int32_t *idx, int64_t M, int64_t C, int64_t R, int64_t Q, int64_t N,
                    const float *cb, const float *w_out, const float *b_out,
                    const float *w_op, const float *b_op, float *latent);
int aqo_gather_q8_0(const aqo_block_q8_0 *cb, int64_t N, int64_t K, const int32_t *idx, int64_t M, float *out);

#ifdef __cplusplus
}
#endif
#endif
