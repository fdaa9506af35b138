/*
 * aq_oracle.c -- plain-C restatement of the reference quantizer arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (see aq_oracle.h).  The product path never links
 * or calls this file; it is the checker for the HIP path and the labelled
 * "port" CPU baseline.
 *
 * Compiled with -ffp-contract=off: every fused multiply-add below is an
 * explicit fmaf() standing for an FMA intrinsic of the reference build
 * (_mm512_fmadd_ps / _mm256_fmadd_ps); every other product is rounded before
 * it is added, as in the reference build (checked bit for bit against
 * oracle/_ref).
 *
 * Reference paths are relative to /root/reference/external/ggml/src unless
 * they start with src/ (the audio.cpp tree).
 */
#include "aq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------------
 * _mm512_reduce_add_ps as GCC 11 implements it (avx512fintrin.h
 * __MM512_REDUCE_OP): halves 256 -> 128 -> 64 -> 32, i.e. pairwise sums at
 * distances 8, 4, 2, 1.  Used by hsum(__m512) (ggml-cpu/llamafile/sgemm.cpp:
 * 274-278) and GGML_F32x16_REDUCE (ggml-cpu/simd-mappings.h:451-476).
 */
static float reduce16(const float a[16]) {
    float t3[8], t6[4], t8[2];
    for (int i = 0; i < 8; ++i) t3[i] = a[i + 8] + a[i];
    for (int i = 0; i < 4; ++i) t6[i] = t3[i + 4] + t3[i];
    for (int i = 0; i < 2; ++i) t8[i] = t6[i] + t6[i + 2];
    return t8[0] + t8[1];
}

/* hsum(__m256) (sgemm.cpp:267-271 -> 252-264) and hsum_float_8
 * (ggml-cpu/arch/x86/quants.c:43-49): lanes i+4 added to i, then distance 2,
 * then 1. */
static float reduce8(const float a[8]) {
    float v[4];
    for (int i = 0; i < 4; ++i) v[i] = a[i + 4] + a[i];
    const float y0 = v[0] + v[2];
    const float y1 = v[1] + v[3];
    return y0 + y1;
}

/* ggml_vec_dot_f32, GGML_SIMD AVX-512 branch (ggml-cpu/vec.cpp:11-135;
 * GGML_F32_STEP 64, GGML_F32_EPR 16, GGML_F32_ARR 4 at simd-mappings.h:
 * 439-478).  Four 16-lane accumulators take elements i+16j+l with FMA
 * (GGML_F32x16_FMA = _mm512_fmadd_ps), are combined 0+=2, 1+=3, 0+=1, then
 * reduced by reduce16.  The scalar leftovers `sumf += x[i]*y[i]` (n % 64 of
 * them, vec.cpp:125-128) are compiled by GCC 11 with -O3 -march=native on
 * the reference's AVX-512 build host as: the products of the first
 * rem - rem % 4 leftovers computed 8 (then 4) at a time and added to sumf in
 * order (a rounded multiply, then an add), the last rem % 4 contracted to
 * scalar fused multiply-adds.  That is the reference's default build
 * (GGML_NATIVE); an x86-64-v4 build of the same source fuses the last
 * rem % 8 instead (tests/test_oracle.py pins both against oracle/_ref). */
float aqo_vec_dot_f32(int n, const float *x, const float *y) {
    return aqo_vec_dot_f32_tail(n, x, y, 4);
}

/* aqo_vec_dot_f32 with the last rem % tail_mod leftovers fused (4: the
 * native build, 8: x86-64-v4). */
float aqo_vec_dot_f32_tail(int n, const float *x, const float *y, int tail_mod) {
    const int np = n & ~63;
    float sum[4][16];
    memset(sum, 0, sizeof(sum));
    for (int i = 0; i < np; i += 64)
        for (int j = 0; j < 4; ++j)
            for (int l = 0; l < 16; ++l)
                sum[j][l] = fmaf(x[i + 16 * j + l], y[i + 16 * j + l], sum[j][l]);
    for (int l = 0; l < 16; ++l) {
        sum[0][l] = sum[0][l] + sum[2][l];
        sum[1][l] = sum[1][l] + sum[3][l];
    }
    for (int l = 0; l < 16; ++l) sum[0][l] = sum[0][l] + sum[1][l];
    float sumf = reduce16(sum[0]);
    const int fused_from = n - (n - np) % tail_mod;
    for (int i = np; i < n; ++i) {
        if (i >= fused_from) {
            sumf = fmaf(x[i], y[i], sumf);
        } else {
            const float prod = x[i] * y[i];
            sumf = sumf + prod;
        }
    }
    return sumf;
}

/* One output element of tinyBLAS<16, __m512, __m512, float, float, float>
 * (sgemm.cpp:523-580, dispatched at 3716-3725): a 16-lane FMA accumulator
 * over k in steps of 16 (madd = _mm512_fmadd_ps, sgemm.cpp:145-149), then
 * hsum = _mm512_reduce_add_ps. */
float aqo_tinyblas_dot_f32(int k, const float *a, const float *b) {
    float acc[16];
    memset(acc, 0, sizeof(acc));
    for (int l = 0; l < k; l += 16)
        for (int j = 0; j < 16; ++j) acc[j] = fmaf(a[l + j], b[l + j], acc[j]);
    return reduce16(acc);
}

/* When ggml_compute_forward_mul_mat hands an F32 x F32 product to tinyBLAS
 * (ggml-cpu/ggml-cpu.c:1285-1306 -> sgemm.cpp:3705-3725 -> matmul 527-545,
 * VECTOR_REGISTERS == 32): n >= 2, k % 16 == 0 and m % 4 == 0 (m = src0 rows,
 * n = src1 rows).  Otherwise ggml_vec_dot_f32 computes each element. */
int aqo_mul_mat_f32_uses_tinyblas(int64_t m, int64_t n, int64_t k) {
    return n >= 2 && (k % 16) == 0 && (m % 4) == 0;
}

/* ggml_vec_argmax_f32 (ggml-cpu/vec.h:1576-1584): running MAX(max, x[i]) with
 * MAX(a,b) = a > b ? a : b, index updated whenever max == x[i].  Keeps the
 * last index of the maximum; NaN restarts the running max (see the loop). */
int aqo_argmax_f32(int n, const float *x) {
    float max = -INFINITY;
    int idx = 0;
    for (int i = 0; i < n; ++i) {
        max = max > x[i] ? max : x[i];
        if (max == x[i]) idx = i;
    }
    return idx;
}

/* ggml_vec_sum_f32 (ggml-cpu/vec.h:1513-1523): double accumulation, one
 * final rounding to float; used by sum_rows (ops.cpp:1457-1489). */
float aqo_sum_f32(int n, const float *x) {
    double s = 0.0;
    for (int i = 0; i < n; ++i) s += (double)x[i];
    return (float)s;
}

/* IEEE binary16 round-to-nearest-even, as F16C _cvtss_sh(x, 0) which
 * GGML_CPU_FP32_TO_FP16 maps to on x86 (simd-mappings.h). */
uint16_t aqo_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t absx = x & 0x7FFFFFFFu;
    if (absx > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((absx >> 13) & 0x3FFu)); /* NaN */
    if (absx >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);                           /* overflow */
    if (absx < 0x38800000u) {                                                              /* subnormal / zero */
        if (absx < 0x33000000u) return (uint16_t)sign;
        const uint32_t e = absx >> 23;
        const uint32_t mant = (absx & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126u - e;           /* 14 .. 24 */
        uint32_t q = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q += 1u;
        return (uint16_t)(sign | q);
    }
    uint32_t h = ((absx - 0x38000000u) >> 13);
    const uint32_t rem = absx & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

float aqo_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            float v = ldexpf((float)m, -24);
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

/* quantize_row_q8_0 for x86 AVX2 (ggml-cpu/arch/x86/quants.c:302-393): the
 * from_float that mul_mat applies to the F32 operand of a Q8_0 product
 * (ggml-cpu.c:1309-1340).  amax by max-tree, d = amax/127 stored as fp16,
 * id = 127/amax, q = round-half-even(x*id), saturating packs to int8. */
static int8_t sat_q(float v) {
    if (isnan(v) || v >= 2147483648.0f || v < -2147483648.0f) return -128;
    long q = (long)v;
    if (q > 127) q = 127;
    if (q < -128) q = -128;
    return (int8_t)q;
}

void aqo_quantize_row_q8_0_x86(const float *x, aqo_block_q8_0 *y, int k) {
    const int nb = k / 32;
    for (int i = 0; i < nb; ++i) {
        const float *xb = x + 32 * i;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const float a = fabsf(xb[j]);
            amax = amax > a ? amax : a;
        }
        const float d = amax / 127.f;
        y[i].d = aqo_fp32_to_fp16(d);
        const float id = (amax != 0.0f) ? 127.f / amax : 0.0f;
        for (int j = 0; j < 32; ++j) y[i].qs[j] = sat_q(nearbyintf(xb[j] * id));
    }
}

/* quantize_row_q8_0_ref (ggml-quants.c:236-256): the weight-side rounding
 * used by ggml_quantize_chunk (roundf, id = 1/d). */
void aqo_quantize_row_q8_0_ref(const float *x, aqo_block_q8_0 *y, int k) {
    const int nb = k / 32;
    for (int i = 0; i < nb; ++i) {
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const float v = fabsf(x[32 * i + j]);
            amax = amax > v ? amax : v;
        }
        const float d = amax / ((1 << 7) - 1);
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = aqo_fp32_to_fp16(d);
        for (int j = 0; j < 32; ++j) y[i].qs[j] = (int8_t)roundf(x[32 * i + j] * id);
    }
}

/* dequantize_row_q8_0 (ggml-quants.c:491-505): y = q * d. */
void aqo_dequantize_row_q8_0(const aqo_block_q8_0 *x, float *y, int k) {
    const int nb = k / 32;
    for (int i = 0; i < nb; ++i) {
        const float d = aqo_fp16_to_fp32(x[i].d);
        for (int j = 0; j < 32; ++j) y[32 * i + j] = (float)x[i].qs[j] * d;
    }
}

/* One element of tinyBLAS_Q0_AVX<block_q8_0, block_q8_0, float>
 * (sgemm.cpp:1353-1680, dispatched at 3928-3938) and of
 * ggml_vec_dot_q8_0_q8_0 (ggml-cpu/arch/x86/quants.c:1170-1216), which share
 * the arithmetic: per block, 8 lanes of exact 4-byte int8 dot products
 * (updot / mul_sum_i8_pairs_float), scaled by fp32(d_a)*fp32(d_b) and
 * accumulated with FMA; then reduce8. */
float aqo_dot_q8_0(int nb, const aqo_block_q8_0 *a, const aqo_block_q8_0 *b) {
    float acc[8];
    memset(acc, 0, sizeof(acc));
    for (int ib = 0; ib < nb; ++ib) {
        const float dd = aqo_fp16_to_fp32(a[ib].d) * aqo_fp16_to_fp32(b[ib].d);
        for (int l = 0; l < 8; ++l) {
            int32_t s = 0;
            for (int t = 0; t < 4; ++t) s += (int32_t)a[ib].qs[4 * l + t] * (int32_t)b[ib].qs[4 * l + t];
            acc[l] = fmaf(dd, (float)s, acc[l]);
        }
    }
    return reduce8(acc);
}

/* ------------------------------------------------------------------------- */

static float dot_f32(int64_t m_rows, int64_t n_rows, int k, const float *src0_row, const float *src1_row) {
    return aqo_mul_mat_f32_uses_tinyblas(m_rows, n_rows, k) ? aqo_tinyblas_dot_f32(k, src0_row, src1_row)
                                                            : aqo_vec_dot_f32(k, src0_row, src1_row);
}

/* Fish Audio encode quantizer, one stage per codebook
 * (src/models/fish_audio/codec.cpp:570-611, quantize_one 587-605):
 *   projected = Conv1d(k=1)(residual) + b_in       conv_modules.cpp:284-341,152-166
 *     (ggml_conv_1d = im2col + mul_mat(im2col, W), ggml.c:4554-4571; one
 *     conv per clip, so m = T decides tinyBLAS vs vec_dot)
 *   pn = projected / sqrt(sum(projected^2) + 1e-12)  codec.cpp:323-334
 *   logits = mul_mat(normalized_codebook, pn)        k = 8 -> vec_dot_f32
 *   code = argmax(logits)                            (last index of max)
 *   z = Conv1d(k=1)(codebook[code]) + b_out          k = 8 -> vec_dot_f32
 *   residual -= z ; recon += z (decode sum, codec.cpp:552-568)
 * normalized_codebook = normalized_rows(codebook)    codec.cpp:171-189. */
/* recipe: 0 Fish (normalized_rows codec.cpp:171-189, l2_normalize_last
 * 323-334: +1e-12 by ggml_scale_bias), 1 IndexTTS2 (normalized_codebook
 * semantic_codec.cpp:43-58: 1.0F / (float)sqrt; normalize_code_latents
 * 110-115: no bias), 2 Vevo2 (l2_normalized_rows components.cpp:566-590:
 * zero rows rejected; build_l2_normalized_rows 848-863: +1e-20).  Returns -2
 * when the recipe rejects the codebook. */
/* One stage of the cascade on the residual r [M, D] (codes into
 * idx[m * ld + s]; recon[m] = z when first, else recon[m] + z). */
static int dac_stage(float *r, int64_t M, int64_t T, int64_t D, int64_t N, const float *Wi, const float *bi,
                     const float *C, const float *Wo, const float *bo, const int32_t *force_idx, int32_t *idx,
                     int64_t ld, int64_t s, float *recon, int first, int recipe) {
    float *cbn = (float *)malloc((size_t)(N * 8) * sizeof(float));
    float *scores = (float *)malloc((size_t)N * sizeof(float));
    if (!cbn || !scores) { free(cbn); free(scores); return -1; }
    const int inproj_tiny = aqo_mul_mat_f32_uses_tinyblas(T, 8, D);
    for (int64_t n = 0; n < N; ++n) {
        double sum = 0.0;
        for (int k = 0; k < 8; ++k) sum += (double)C[n * 8 + k] * (double)C[n * 8 + k];
        float inv;
        if (recipe == 1) {
            inv = 1.0f / (float)sqrt(sum);
        } else if (recipe == 2) {
            const double norm = sqrt(sum);
            if (norm == 0.0) { free(cbn); free(scores); return -2; }
            inv = (float)(1.0 / norm);
        } else {
            inv = sum > 0.0 ? (float)(1.0 / sqrt(sum)) : 0.0f;
        }
        for (int k = 0; k < 8; ++k) cbn[n * 8 + k] = C[n * 8 + k] * inv;
    }
    for (int64_t m = 0; m < M; ++m) {
        float *rm = r + m * D;
        float p[8], pn[8], sq[8];
        for (int j = 0; j < 8; ++j) {
            p[j] = inproj_tiny ? aqo_tinyblas_dot_f32((int)D, rm, Wi + j * D) : aqo_vec_dot_f32((int)D, rm, Wi + j * D);
            if (bi) p[j] = p[j] + bi[j];
        }
        for (int j = 0; j < 8; ++j) sq[j] = p[j] * p[j];
        float ss = aqo_sum_f32(8, sq);
        if (recipe != 1) ss = fmaf(ss, 1.0f, recipe == 2 ? 1.0e-20f : 1.0e-12f);   /* ggml_scale_bias, vec.h:708-710 */
        const float den = sqrtf(ss);
        for (int j = 0; j < 8; ++j) pn[j] = p[j] / den;
        for (int64_t n = 0; n < N; ++n) scores[n] = aqo_vec_dot_f32(8, cbn + n * 8, pn);
        const int code = aqo_argmax_f32((int)N, scores);
        idx[m * ld + s] = code;
        const int use = force_idx ? force_idx[m * ld + s] : code;
        const float *q = C + (int64_t)use * 8;
        if (!Wo) continue;   /* codes only (no out-projection given) */
        for (int64_t d = 0; d < D; ++d) {
            float z = aqo_vec_dot_f32(8, q, Wo + d * 8);
            if (bo) z = z + bo[d];
            rm[d] = rm[d] - z;
            if (recon) recon[m * D + d] = first ? z : recon[m * D + d] + z;
        }
    }
    free(cbn);
    free(scores);
    return 0;
}

int aqo_dac_rvq_ex(const float *x, int64_t B, int64_t T, int64_t D, int64_t Q, int64_t N,
                   const float *w_in, const float *b_in, const float *cb,
                   const float *w_out, const float *b_out, const int32_t *force_idx,
                   int32_t *idx, float *residual, float *recon, int recipe) {
    const int64_t M = B * T;
    memcpy(residual, x, (size_t)(M * D) * sizeof(float));
    for (int64_t s = 0; s < Q; ++s) {
        const int rc = dac_stage(residual, M, T, D, N, w_in + s * 8 * D, b_in ? b_in + s * 8 : NULL, cb + s * N * 8,
                                 w_out ? w_out + s * D * 8 : NULL, b_out ? b_out + s * D : NULL, force_idx, idx, Q, s,
                                 recon, s == 0, recipe);
        if (rc != 0) return rc;
    }
    return 0;
}

/* The Fish cascade as build_encode_quantizer runs it (fish_audio/codec.cpp:
 * 606-608): the semantic quantizer of N0 codes (cb0 [N0, 8]), then Q - 1
 * residual quantizers of N codes (cb [Q-1, N, 8]); the recon is the
 * decoder's sum z_0 + z_1 + ... (codec.cpp:552-568).  Weights as
 * aqo_dac_rvq with Q stages. */
int aqo_dac_rvq_mixed(const float *x, int64_t B, int64_t T, int64_t D, int64_t Q, int64_t N0, int64_t N,
                      const float *w_in, const float *b_in, const float *cb0, const float *cb,
                      const float *w_out, const float *b_out, const int32_t *force_idx,
                      int32_t *idx, float *residual, float *recon) {
    const int64_t M = B * T;
    memcpy(residual, x, (size_t)(M * D) * sizeof(float));
    for (int64_t s = 0; s < Q; ++s) {
        const int rc = dac_stage(residual, M, T, D, s == 0 ? N0 : N, w_in + s * 8 * D, b_in ? b_in + s * 8 : NULL,
                                 s == 0 ? cb0 : cb + (s - 1) * N * 8, w_out + s * D * 8, b_out ? b_out + s * D : NULL,
                                 force_idx, idx, Q, s, recon, s == 0, 0);
        if (rc != 0) return rc;
    }
    return 0;
}

/* OmniVoice encode quantizer without projections
 * (src/models/omnivoice/audio_tokenizer.cpp:1227-1237 score weights,
 * 1897-1927 graph): logits = mul_mat(2c, r) + (float)(-sum_double(c^2)),
 * argmax, get_rows(codebook), residual -= q. */
int aqo_euclid_rvq(const float *x, int64_t M, int64_t K, int64_t Q, int64_t N,
                   const float *cb, const int32_t *force_idx,
                   int32_t *idx, float *residual, float *logit_best) {
    float *r = residual;
    memcpy(r, x, (size_t)(M * K) * sizeof(float));
    float *w2 = (float *)malloc((size_t)(N * K) * sizeof(float));
    float *bias = (float *)malloc((size_t)N * sizeof(float));
    float *lg = (float *)malloc((size_t)N * sizeof(float));
    if (!w2 || !bias || !lg) { free(w2); free(bias); free(lg); return -1; }
    for (int64_t s = 0; s < Q; ++s) {
        const float *C = cb + s * N * K;
        for (int64_t n = 0; n < N; ++n) {
            double norm = 0.0;
            for (int64_t k = 0; k < K; ++k) {
                const float v = C[n * K + k];
                w2[n * K + k] = 2.0f * v;
                norm += (double)v * (double)v;
            }
            bias[n] = (float)(-norm);
        }
        for (int64_t m = 0; m < M; ++m) {
            float *rm = r + m * K;
            for (int64_t n = 0; n < N; ++n) lg[n] = dot_f32(N, M, (int)K, w2 + n * K, rm) + bias[n];
            const int code = aqo_argmax_f32((int)N, lg);
            idx[m * Q + s] = code;
            if (logit_best) logit_best[m * Q + s] = lg[code];
            const int use = force_idx ? force_idx[m * Q + s] : code;
            for (int64_t k = 0; k < K; ++k) rm[k] = rm[k] - C[(int64_t)use * K + k];
        }
    }
    free(w2);
    free(bias);
    free(lg);
    return 0;
}

/* ggml_top_k on the CPU (ops.cpp:8423-8456) is std::partial_sort over the
 * index sequence 0..N-1 with comp(a, b) = v[a] > v[b], then dst[0] and
 * dst[1] swapped.  Which of several equal values survive at the k-th place
 * is decided by the heap inside std::partial_sort, so the heap is restated
 * here as libstdc++ (GCC 11.4, the toolchain the reference build uses)
 * implements it: std::__heap_select = make_heap over the first k, then every
 * later element strictly better than the root replaces it (pop_heap), then
 * std::__sort_heap.  Textbook binary heap with the hole-sifting adjust_heap
 * followed by push_heap. */
static void heap_adjust(int32_t *h, const float *v, int64_t hole, int64_t len, int32_t val) {
    const int64_t top = hole;
    int64_t child = hole;
    while (child < (len - 1) / 2) {
        child = 2 * (child + 1);
        if (v[h[child]] > v[h[child - 1]]) child--;
        h[hole] = h[child];
        hole = child;
    }
    if ((len & 1) == 0 && child == (len - 2) / 2) {
        child = 2 * (child + 1);
        h[hole] = h[child - 1];
        hole = child - 1;
    }
    int64_t parent = (hole - 1) / 2;
    while (hole > top && v[h[parent]] > v[val]) {
        h[hole] = h[parent];
        hole = parent;
        parent = (hole - 1) / 2;
    }
    h[hole] = val;
}

void aqo_top_k_f32(const float *v, int64_t n, int k, int32_t *dst) {
    int32_t *h = dst;
    for (int i = 0; i < k; ++i) h[i] = i;
    if (k >= 2)
        for (int64_t parent = (k - 2) / 2;; --parent) {
            heap_adjust(h, v, parent, k, h[parent]);
            if (parent == 0) break;
        }
    for (int64_t i = k; i < n; ++i)
        if (v[i] > v[h[0]]) heap_adjust(h, v, 0, k, (int32_t)i);
    for (int64_t last = k - 1; last > 0; --last) {   /* sort_heap */
        const int32_t val = h[last];
        h[last] = h[0];
        heap_adjust(h, v, 0, last, val);
    }
    if (k > 1) { const int32_t t = dst[0]; dst[0] = dst[1]; dst[1] = t; }
}

/* Higgs encode quantizer without projections
 * (src/models/higgs_audio_tts/codec.cpp:975-1013): dot = mul_mat(codebook, r)
 * (MatMulModule, src/framework/modules/primitive_modules.cpp:186-212),
 * x2 = sum_rows(r*r), e2 = sum_rows(c*c) on the F32 (dequantised) codebook,
 * logits = ((scale(dot, 2) - x2) - e2), argmax, optional top_k
 * (ops.cpp:8423-8456), get_rows(codebook) (dequantised for Q8_0), sub.
 * For a Q8_0 codebook the F32 operand is quantised by x86
 * quantize_row_q8_0 before the integer product (ggml-cpu.c:1309-1340). */
int aqo_higgs_rvq(const float *x, int64_t M, int64_t K, int64_t Q, int64_t N,
                  const void *cb, int cb_type, int topk, const int32_t *force_idx,
                  int32_t *idx, float *residual, float *dist,
                  int32_t *topk_idx, float *topk_logit) {
    const int64_t nb = K / 32;
    float *r = residual;
    memcpy(r, x, (size_t)(M * K) * sizeof(float));
    float *cbf = (float *)malloc((size_t)(N * K) * sizeof(float));
    float *e2 = (float *)malloc((size_t)N * sizeof(float));
    float *lg = (float *)malloc((size_t)N * sizeof(float));
    float *tmp = (float *)malloc((size_t)(K > N ? K : N) * sizeof(float));
    aqo_block_q8_0 *xq = (aqo_block_q8_0 *)malloc((size_t)(nb > 0 ? nb : 1) * sizeof(aqo_block_q8_0));
    if (!cbf || !e2 || !lg || !tmp || !xq) {
        free(cbf); free(e2); free(lg); free(tmp); free(xq);
        return -1;
    }
    for (int64_t s = 0; s < Q; ++s) {
        const float *Cf = cb_type == 0 ? (const float *)cb + s * N * K : NULL;
        const aqo_block_q8_0 *Cq = cb_type == 1 ? (const aqo_block_q8_0 *)cb + s * N * nb : NULL;
        for (int64_t n = 0; n < N; ++n) {
            if (Cq) aqo_dequantize_row_q8_0(Cq + n * nb, cbf + n * K, (int)K);
            else memcpy(cbf + n * K, Cf + n * K, (size_t)K * sizeof(float));
            for (int64_t k = 0; k < K; ++k) tmp[k] = cbf[n * K + k] * cbf[n * K + k];
            e2[n] = aqo_sum_f32((int)K, tmp);
        }
        for (int64_t m = 0; m < M; ++m) {
            float *rm = r + m * K;
            for (int64_t k = 0; k < K; ++k) tmp[k] = rm[k] * rm[k];
            const float x2 = aqo_sum_f32((int)K, tmp);
            if (Cq) aqo_quantize_row_q8_0_x86(rm, xq, (int)K);
            for (int64_t n = 0; n < N; ++n) {
                const float dot = Cq ? aqo_dot_q8_0((int)nb, Cq + n * nb, xq) : dot_f32(N, M, (int)K, Cf + n * K, rm);
                lg[n] = ((dot * 2.0f) - x2) - e2[n];
            }
            const int code = aqo_argmax_f32((int)N, lg);
            idx[m * Q + s] = code;
            if (dist) dist[m * Q + s] = -lg[code];
            if (topk > 0) {
                int32_t *ti = topk_idx + (m * Q + s) * topk;
                aqo_top_k_f32(lg, N, topk, ti);
                for (int k = 0; k < topk; ++k) topk_logit[(m * Q + s) * topk + k] = lg[ti[k]];
            }
            const int use = force_idx ? force_idx[m * Q + s] : code;
            for (int64_t k = 0; k < K; ++k) rm[k] = rm[k] - cbf[(int64_t)use * K + k];
        }
    }
    free(cbf); free(e2); free(lg); free(tmp); free(xq);
    return 0;
}

/* Direct-distance RVQ: VectorQuantizer::compute
 * (src/framework/runtime/host_ops.cpp:236-273) per stage, and the Qwen3
 * cascade quantize_projected (src/models/qwen3_tts/tokenizer_speech_encoder.cpp:
 * 287-349): distance = sum_k (x_k - c_k)^2 with each square rounded and added
 * in order (the reference is built as ISO C++17, so GCC does not contract),
 * first index of the minimum (strict <, NaN never wins, start at index 0),
 * residual -= c[code]. */
int aqo_direct_rvq(const float *x, int64_t M, int64_t K, int64_t Q, int64_t N, const float *cb,
                   const int32_t *force_idx, int32_t *idx, float *residual, float *dist) {
    float *r = residual;
    memcpy(r, x, (size_t)(M * K) * sizeof(float));
    for (int64_t s = 0; s < Q; ++s) {
        const float *C = cb + s * N * K;
        for (int64_t m = 0; m < M; ++m) {
            float *rm = r + m * K;
            int32_t best = 0;
            float best_d = INFINITY;
            for (int64_t n = 0; n < N; ++n) {
                float d = 0.0f;
                for (int64_t k = 0; k < K; ++k) {
                    const float diff = rm[k] - C[n * K + k];
                    const float sq = diff * diff;
                    d = d + sq;
                }
                if (d < best_d) { best_d = d; best = (int32_t)n; }
            }
            idx[m * Q + s] = best;
            if (dist) dist[m * Q + s] = best_d;
            const int64_t use = force_idx ? force_idx[m * Q + s] : best;
            for (int64_t k = 0; k < K; ++k) rm[k] = rm[k] - C[use * K + k];
        }
    }
    return 0;
}

/* One row of LinearModule (src/framework/modules/linear_module.cpp:73-108):
 * out[o] = mul_mat(W, x)[o] (+ bias[o] by ggml_add), for a weight of n_out
 * rows of k values (F32, or Q8_0 blocks whose product quantises x with x86
 * quantize_row_q8_0 first, ggml-cpu.c:1309-1340) applied to a batch of
 * n_rows input rows (the batch size decides tinyBLAS vs vec_dot for F32).
 * xq: scratch of k/32 blocks. */
static void linear_row(const void *w, int w_type, const float *bias, int64_t n_out, int64_t k, int64_t n_rows,
                       const float *x, aqo_block_q8_0 *xq, float *out) {
    if (w_type == 1) aqo_quantize_row_q8_0_x86(x, xq, (int)k);
    for (int64_t o = 0; o < n_out; ++o) {
        float v = w_type == 1 ? aqo_dot_q8_0((int)(k / 32), (const aqo_block_q8_0 *)w + o * (k / 32), xq)
                              : dot_f32(n_out, n_rows, (int)k, (const float *)w + o * k, x);
        if (bias) v = v + bias[o];
        out[o] = v;
    }
}

/* LinearModule over a batch: out [M, n_out] = linear_row of each of the M
 * input rows x [M, k] (the batch size M is the mul_mat's, which picks the
 * F32 summation order). */
int aqo_linear(const void *w, int w_type, const float *bias, int64_t n_out, int64_t k, int64_t M, const float *x,
               float *out) {
    aqo_block_q8_0 *xq = (aqo_block_q8_0 *)malloc((size_t)(k / 32 + 1) * sizeof(aqo_block_q8_0));
    if (!xq) return -1;
    for (int64_t m = 0; m < M; ++m) linear_row(w, w_type, bias, n_out, k, M, x + m * k, xq, out + m * n_out);
    free(xq);
    return 0;
}

/* OmniVoice and Higgs acoustic RVQ with the projections of the reference
 * (omnivoice/audio_tokenizer.cpp:1886-1927; higgs_audio_tts/codec.cpp:958-1016):
 * per stage, on the residual r of hidden size H (frame-major after the
 * graphs' transposes, which only move data):
 *   p      = project_in(r)                 LinearModule H -> K (+ bias)
 *   logits = OmniVoice: mul_mat(2c, p) + (float)(-sum_double c^2)
 *            Higgs:     ((2*mul_mat(c, p)) - sum_rows(p*p)) - sum_rows(c*c)
 *   code   = argmax (last index), optional top_k (Higgs)
 *   z      = project_out(get_rows(c, code)) LinearModule K -> H (+ bias)
 *   r     -= z
 * recipe 0 OmniVoice (F32 codebook), 1 Higgs (F32 or Q8_0 codebook);
 * w_in [Q,K,H] and w_out [Q,H,K] are F32 (type 0) or Q8_0 blocks (type 1).
 * x [M,H]; idx [M,Q]; residual [M,H]; dist [M,Q] = -logit[code] (nullable);
 * topk_idx / topk_logit [M,Q,topk] (Higgs only). */
int aqo_projected_rvq(const float *x, int64_t M, int64_t H, int64_t K, int64_t Q, int64_t N, int recipe,
                      const void *cb, int cb_type, const void *w_in, const float *b_in, const void *w_out,
                      const float *b_out, int proj_type, int topk, const int32_t *force_idx, int32_t *idx,
                      float *residual, float *dist, int32_t *topk_idx, float *topk_logit) {
    const int64_t nbk = K / 32;
    float *r = residual;
    memcpy(r, x, (size_t)(M * H) * sizeof(float));
    float *cbf = (float *)malloc((size_t)(N * K) * sizeof(float));
    float *w2 = (float *)malloc((size_t)(N * K) * sizeof(float));
    float *cterm = (float *)malloc((size_t)N * sizeof(float));
    float *lg = (float *)malloc((size_t)N * sizeof(float));
    float *p = (float *)malloc((size_t)K * sizeof(float));
    float *z = (float *)malloc((size_t)H * sizeof(float));
    float *tmp = (float *)malloc((size_t)K * sizeof(float));
    aqo_block_q8_0 *xq = (aqo_block_q8_0 *)malloc((size_t)(H / 32 + nbk + 1) * sizeof(aqo_block_q8_0));
    if (!cbf || !w2 || !cterm || !lg || !p || !z || !tmp || !xq) {
        free(cbf); free(w2); free(cterm); free(lg); free(p); free(z); free(tmp); free(xq);
        return -1;
    }
    const size_t win_stage = proj_type == 1 ? (size_t)(K * (H / 32)) * sizeof(aqo_block_q8_0) : (size_t)(K * H) * 4;
    const size_t wout_stage = proj_type == 1 ? (size_t)(H * nbk) * sizeof(aqo_block_q8_0) : (size_t)(H * K) * 4;
    for (int64_t s = 0; s < Q; ++s) {
        const aqo_block_q8_0 *Cq = cb_type == 1 ? (const aqo_block_q8_0 *)cb + s * N * nbk : NULL;
        const void *Wi = (const char *)w_in + s * win_stage;
        const void *Wo = (const char *)w_out + s * wout_stage;
        const float *bi = b_in ? b_in + s * K : NULL;
        const float *bo = b_out ? b_out + s * H : NULL;
        for (int64_t n = 0; n < N; ++n) {
            if (Cq) aqo_dequantize_row_q8_0(Cq + n * nbk, cbf + n * K, (int)K);
            else memcpy(cbf + n * K, (const float *)cb + (s * N + n) * K, (size_t)K * sizeof(float));
            if (recipe == 0) {   /* audio_tokenizer.cpp:1227-1237 */
                double norm = 0.0;
                for (int64_t k = 0; k < K; ++k) {
                    const float v = cbf[n * K + k];
                    w2[n * K + k] = 2.0f * v;
                    norm += (double)v * (double)v;
                }
                cterm[n] = (float)(-norm);
            } else {             /* sum_rows(c*c) */
                for (int64_t k = 0; k < K; ++k) tmp[k] = cbf[n * K + k] * cbf[n * K + k];
                cterm[n] = aqo_sum_f32((int)K, tmp);
            }
        }
        for (int64_t m = 0; m < M; ++m) {
            float *rm = r + m * H;
            linear_row(Wi, proj_type, bi, K, H, M, rm, xq, p);
            if (recipe == 0) {
                for (int64_t n = 0; n < N; ++n) lg[n] = dot_f32(N, M, (int)K, w2 + n * K, p) + cterm[n];
            } else {
                for (int64_t k = 0; k < K; ++k) tmp[k] = p[k] * p[k];
                const float x2 = aqo_sum_f32((int)K, tmp);
                if (Cq) aqo_quantize_row_q8_0_x86(p, xq, (int)K);
                for (int64_t n = 0; n < N; ++n) {
                    const float dot = Cq ? aqo_dot_q8_0((int)nbk, Cq + n * nbk, xq) : dot_f32(N, M, (int)K, cbf + n * K, p);
                    lg[n] = ((dot * 2.0f) - x2) - cterm[n];
                }
            }
            const int code = aqo_argmax_f32((int)N, lg);
            idx[m * Q + s] = code;
            if (dist) dist[m * Q + s] = -lg[code];
            if (topk > 0) {
                int32_t *ti = topk_idx + (m * Q + s) * topk;
                aqo_top_k_f32(lg, N, topk, ti);
                for (int k = 0; k < topk; ++k) topk_logit[(m * Q + s) * topk + k] = lg[ti[k]];
            }
            const int64_t use = force_idx ? force_idx[m * Q + s] : code;
            linear_row(Wo, proj_type, bo, H, K, M, cbf + use * K, xq, z);
            for (int64_t h = 0; h < H; ++h) rm[h] = rm[h] - z[h];
        }
    }
    free(cbf); free(w2); free(cterm); free(lg); free(p); free(z); free(tmp); free(xq);
    return 0;
}

/* Decode of the projected cascades (omnivoice/audio_tokenizer.cpp:1745-1771,
 * higgs_audio_tts/codec.cpp:1040-1065): out[m] = z_0 + z_1 + ... in stage
 * order, z_s = project_out(get_rows(c_s, idx[m,s])).  Returns -1 on an
 * out-of-range code. */
int aqo_projected_decode(const int32_t *idx, int64_t M, int64_t H, int64_t K, int64_t Q, int64_t N,
                         const void *cb, int cb_type, const void *w_out, const float *b_out, int proj_type,
                         float *out) {
    const int64_t nbk = K / 32;
    float *c = (float *)malloc((size_t)K * sizeof(float));
    float *z = (float *)malloc((size_t)H * sizeof(float));
    aqo_block_q8_0 *xq = (aqo_block_q8_0 *)malloc((size_t)(nbk + 1) * sizeof(aqo_block_q8_0));
    if (!c || !z || !xq) { free(c); free(z); free(xq); return -1; }
    const size_t wout_stage = proj_type == 1 ? (size_t)(H * nbk) * sizeof(aqo_block_q8_0) : (size_t)(H * K) * 4;
    int rc = 0;
    for (int64_t m = 0; m < M && rc == 0; ++m) {
        float *om = out + m * H;
        for (int64_t s = 0; s < Q; ++s) {
            const int32_t code = idx[m * Q + s];
            if (code < 0 || code >= N) { rc = -1; break; }
            if (cb_type == 1) aqo_dequantize_row_q8_0((const aqo_block_q8_0 *)cb + (s * N + code) * nbk, c, (int)K);
            else memcpy(c, (const float *)cb + (s * N + code) * K, (size_t)K * sizeof(float));
            linear_row((const char *)w_out + s * wout_stage, proj_type, b_out ? b_out + s * H : NULL, H, K, M, c, xq, z);
            for (int64_t h = 0; h < H; ++h) om[h] = s == 0 ? z[h] : om[h] + z[h];
        }
    }
    free(c); free(z); free(xq);
    return rc;
}

int aqo_gather_f32(const float *cb, int64_t N, int64_t K, const int32_t *idx, int64_t M, float *out) {
    for (int64_t m = 0; m < M; ++m) {
        if (idx[m] < 0 || idx[m] >= N) return -1;
        memcpy(out + m * K, cb + (int64_t)idx[m] * K, (size_t)K * sizeof(float));
    }
    return 0;
}

int aqo_gather_q8_0(const aqo_block_q8_0 *cb, int64_t N, int64_t K, const int32_t *idx, int64_t M, float *out) {
    for (int64_t m = 0; m < M; ++m) {
        if (idx[m] < 0 || idx[m] >= N) return -1;
        aqo_dequantize_row_q8_0(cb + (int64_t)idx[m] * (K / 32), out + m * K, (int)K);
    }
    return 0;
}

/* codebook_embedding (src/models/qwen3_tts/tokenizer_speech_encoder.cpp:271-285;
 * the decoder's copy at tokenizer_speech_decoder.cpp:205-212): per code,
 * denom = std::max(usage, eps), i.e. (usage < eps) ? eps : usage (a NaN usage
 * stays NaN), then one fp32 division per element. */
int aqo_ema_codebook(const float *embedding_sum, const float *cluster_usage, int64_t Q, int64_t N, int64_t K,
                     float eps, float *cb) {
    for (int64_t qn = 0; qn < Q * N; ++qn) {
        const float u = cluster_usage[qn];
        const float denom = (u < eps) ? eps : u;
        for (int64_t k = 0; k < K; ++k) cb[qn * K + k] = embedding_sum[qn * K + k] / denom;
    }
    return 0;
}

int aqo_dac_rvq(const float *x, int64_t B, int64_t T, int64_t D, int64_t Q, int64_t N,
                const float *w_in, const float *b_in, const float *cb,
                const float *w_out, const float *b_out, const int32_t *force_idx,
                int32_t *idx, float *residual, float *recon) {
    return aqo_dac_rvq_ex(x, B, T, D, Q, N, w_in, b_in, cb, w_out, b_out, force_idx, idx, residual, recon, 0);
}

/* ------------------------------------------------------------------------
 * Host-loop DAC quantizers.  The reference builds its engine code without
 * -march (reference CMakeLists.txt: only ggml gets the native ISA flags), so
 * x86-64 has no FMA there and every product below is rounded before it is
 * added; this file is compiled with -ffp-contract=off to match.
 * ------------------------------------------------------------------------ */

/* quantize_reference, src/community_models/outetts/dac.cpp:376-456. */
int aqo_outetts_rvq(const float *x, int64_t M, int64_t D, int64_t Q, int64_t N,
                    const float *w_in, const float *b_in, const float *cb,
                    const float *w_out, const float *b_out, const int32_t *force_idx,
                    int32_t *idx, float *residual) {
    float *r = residual;
    memcpy(r, x, (size_t)(M * D) * sizeof(float));
    for (int64_t s = 0; s < Q; ++s) {
        const float *W = w_in + s * 8 * D;
        const float *C = cb + s * N * 8;
        const float *Wo = w_out + s * D * 8;
        for (int64_t m = 0; m < M; ++m) {
            float *rm = r + m * D;
            float p[8];
            float nsq = 0.0f;                              /* :399-411 */
            for (int d = 0; d < 8; ++d) {
                float v = b_in ? b_in[s * 8 + d] : 0.0f;
                for (int64_t h = 0; h < D; ++h) v = v + W[d * D + h] * rm[h];
                p[d] = v;
                nsq = nsq + v * v;
            }
            const float pn = sqrtf(nsq) + 1.0e-12f;        /* :412 */
            int32_t best = 0;
            float best_d = INFINITY;
            for (int64_t n = 0; n < N; ++n) {              /* :415-434 */
                float e2 = 0.0f;
                for (int d = 0; d < 8; ++d) e2 = e2 + C[n * 8 + d] * C[n * 8 + d];
                const float en = sqrtf(e2) + 1.0e-12f;
                float dist = 0.0f;
                for (int d = 0; d < 8; ++d) {
                    const float diff = p[d] / pn - C[n * 8 + d] / en;
                    dist = dist + diff * diff;
                }
                if (dist < best_d) { best_d = dist; best = (int32_t)n; }
            }
            idx[m * Q + s] = best;
            const int64_t use = force_idx ? force_idx[m * Q + s] : best;
            for (int64_t o = 0; o < D; ++o) {              /* :438-453 */
                float v = b_out ? b_out[s * D + o] : 0.0f;
                for (int d = 0; d < 8; ++d) v = v + Wo[o * 8 + d] * C[use * 8 + d];
                rm[o] = rm[o] - v;
            }
        }
    }
    return 0;
}

/* fold_weight_norm, src/community_models/outetts/dac.cpp:91-110: per output
   row (dim1 * kernel weights) the double sum of double squares, then
   scale = g / (float)sqrt(norm2) in fp32 and w = v * scale. */
void aqo_outetts_weight_norm(const float *v, const float *g, int64_t rows, int64_t cols, float *w) {
    for (int64_t i = 0; i < rows; ++i) {
        double norm2 = 0.0;
        for (int64_t j = 0; j < cols; ++j) {
            const double x = v[i * cols + j];
            norm2 += x * x;
        }
        const float scale = g[i] / (float)sqrt(norm2);
        for (int64_t j = 0; j < cols; ++j) w[i * cols + j] = v[i * cols + j] * scale;
    }
}

/* reconstruct_weight_norm, src/models/moss/shared/audio_tokenizer_quantizer.cpp:17-39. */
void aqo_moss_weight_norm(const float *g, const float *v, int64_t out_ch, int64_t in_ch, float *w) {
    for (int64_t o = 0; o < out_ch; ++o) {
        double norm = 0.0;
        for (int64_t k = 0; k < in_ch; ++k) {
            const double value = v[o * in_ch + k];
            norm = norm + value * value;
        }
        const float scale = (float)(g[o] / sqrt(norm));
        for (int64_t k = 0; k < in_ch; ++k) w[o * in_ch + k] = v[o * in_ch + k] * scale;
    }
}

/* std::max(a, b) for doubles: (a < b) ? b : a (a NaN stays). */
static double aqo_std_max_d(double a, double b) { return (a < b) ? b : a; }

/* MossAudioTokenizerQuantizer constructor, :116-130. */
void aqo_moss_normalize_rows(const float *cb, int64_t rows, int64_t dim, float *out) {
    for (int64_t n = 0; n < rows; ++n) {
        double norm = 0.0;
        for (int64_t k = 0; k < dim; ++k) norm = norm + (double)cb[n * dim + k] * (double)cb[n * dim + k];
        const double scale = 1.0 / aqo_std_max_d(sqrt(norm), 1.0e-12);
        for (int64_t k = 0; k < dim; ++k) out[n * dim + k] = (float)(cb[n * dim + k] * scale);
    }
}

/* MossAudioTokenizerQuantizer::encode, :174-271. */
int aqo_moss_rvq(const float *hidden, int64_t M, int64_t C, int64_t R, int64_t Q, int64_t N,
                 const float *w_ip, const float *b_ip, const float *w_in, const float *b_in,
                 const float *cb, const float *w_out, const float *b_out, const int32_t *force_idx,
                 int32_t *idx, double *residual) {
    float *tn = (float *)malloc((size_t)(Q * N * 8) * sizeof(float));
    double *r = (double *)malloc((size_t)R * sizeof(double));
    if (!tn || !r) { free(tn); free(r); return -1; }
    aqo_moss_normalize_rows(cb, Q * N, 8, tn);
    for (int64_t m = 0; m < M; ++m) {
        const float *h = hidden + m * C;
        for (int64_t o = 0; o < R; ++o) {                  /* input_proj, :193-201 */
            double sum = b_ip[o];
            for (int64_t k = 0; k < C; ++k) sum = sum + (double)w_ip[o * C + k] * (double)h[k];
            r[o] = sum;
        }
        for (int64_t s = 0; s < Q; ++s) {
            double enc[8];
            double enc_norm = 0.0;                         /* in_proj + norm, :207-221 */
            for (int c = 0; c < 8; ++c) {
                double sum = b_in[s * 8 + c];
                const float *row = w_in + (s * 8 + c) * R;
                for (int64_t k = 0; k < R; ++k) sum = sum + (double)row[k] * r[k];
                enc[c] = sum;
                enc_norm = enc_norm + sum * sum;
            }
            const double enc_scale = 1.0 / aqo_std_max_d(sqrt(enc_norm), 1.0e-12);
            for (int c = 0; c < 8; ++c) enc[c] = enc[c] * enc_scale;
            int32_t best = 0;                              /* :225-237 */
            double best_dot = -INFINITY;
            const float *T = tn + s * N * 8;
            for (int64_t n = 0; n < N; ++n) {
                double dot = 0.0;
                for (int c = 0; c < 8; ++c) dot = dot + (double)T[n * 8 + c] * enc[c];
                if (dot > best_dot) { best_dot = dot; best = (int32_t)n; }
            }
            idx[m * Q + s] = best;
            const int64_t use = force_idx ? force_idx[m * Q + s] : best;
            const float *emb = cb + (s * N + use) * 8;     /* :240-248 */
            for (int64_t o = 0; o < R; ++o) {
                double sum = b_out[s * R + o];
                const float *row = w_out + (s * R + o) * 8;
                for (int k = 0; k < 8; ++k) sum = sum + (double)row[k] * (double)emb[k];
                r[o] = r[o] - sum;
            }
        }
        if (residual) memcpy(residual + m * R, r, (size_t)R * sizeof(double));
    }
    free(tn); free(r);
    return 0;
}

/* MossAudioTokenizerQuantizer::decode, :139-172, with the constructor's
 * combined out-projection and latent tables, :77-115. */
int aqo_moss_decode(const int32_t *idx, int64_t M, int64_t C, int64_t R, int64_t Q, int64_t N,
                    const float *cb, const float *w_out, const float *b_out,
                    const float *w_op, const float *b_op, float *latent) {
    for (int64_t i = 0; i < M * Q; ++i)
        if (idx[i] < 0 || idx[i] >= N) return -1;
    float *cbias = (float *)malloc((size_t)C * sizeof(float));
    float *cw = (float *)malloc((size_t)(C * 8) * sizeof(float));
    float *table = (float *)malloc((size_t)(Q * N * C) * sizeof(float));
    if (!cbias || !cw || !table) { free(cbias); free(cw); free(table); return -2; }
    for (int64_t s = 0; s < Q; ++s) {
        const float *Wo = w_out + s * R * 8;
        const float *bo = b_out + s * R;
        for (int64_t o = 0; o < C; ++o) {
            const float *orow = w_op + o * R;
            float bsum = 0.0f;
            for (int64_t k = 0; k < R; ++k) bsum = bsum + orow[k] * bo[k];
            cbias[o] = bsum;
            for (int k = 0; k < 8; ++k) {
                float sum = 0.0f;
                for (int64_t j = 0; j < R; ++j) sum = sum + orow[j] * Wo[j * 8 + k];
                cw[o * 8 + k] = sum;
            }
        }
        for (int64_t n = 0; n < N; ++n) {
            const float *e = cb + (s * N + n) * 8;
            for (int64_t o = 0; o < C; ++o) {
                float sum = cbias[o];
                for (int k = 0; k < 8; ++k) sum = sum + cw[o * 8 + k] * e[k];
                table[(s * N + n) * C + o] = sum;
            }
        }
    }
    for (int64_t m = 0; m < M; ++m)
        for (int64_t o = 0; o < C; ++o) {
            float v = b_op[o];
            for (int64_t s = 0; s < Q; ++s) v = v + table[(s * N + idx[m * Q + s]) * C + o];
            latent[m * C + o] = v;
        }
    free(cbias); free(cw); free(table);
    return 0;
}
