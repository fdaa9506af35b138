/*
 * aq_mi355x.h -- C ABI of the MI355X (gfx950) codec-quantizer library.
 *
 * The library replaces audio.cpp's codec-quantizer hot path: the VQ/RVQ
 * encode that maps latent frames to codebook indices by nearest-neighbour
 * search, the residual cascade across codebooks, and the codebook-gather
 * decode.  Results are bit-identical to the reference's ggml CPU backend on
 * the same inputs (same fp32 operation order, fused multiply-adds, double
 * accumulations and tie rules), with one documented exception: the Fish
 * recipe (AQ_DAC_FISH) gives the exact cosine argmax, which is what the
 * reference computes on its Metal branch (fish_audio/codec.cpp:324-327, a
 * contiguous copy of the transposed projection before ggml_div).  On the CPU
 * backend the reference hands ggml_div the transposed view itself
 * (codec.cpp:323-334 with the transpose at :589), and ggml's CPU binary ops
 * read src0 rows as contiguous (external/ggml/src/ggml-cpu/binary-ops.cpp:
 * 120-136), so the reference's CPU Fish codes are not the cosine argmax and
 * differ from this library's (tests/test_oracle.py
 * test_reference_cpu_view_bug_is_real shows it on ggml itself).
 *
 * Conventions
 *  - Plain C types only.  Every entry point returns aq_status; a message for
 *    the last failure on a context is available from aq_last_error().
 *  - "host" pointers are ordinary CPU memory; "device" pointers are HIP device
 *    memory of the context's device (allocated by the caller).  Nothing the
 *    library allocates escapes the ABI except opaque handles.
 *  - Work is enqueued on the context's stream and is asynchronous with respect
 *    to the host unless a function says otherwise.  One context per calling
 *    thread; a context performs no internal locking (the reference also runs
 *    one session per model under its own lock).
 *  - Matrices are row-major.  Frames are rows: x[m, d] at x + m*D + d.
 *  - An empty batch (M = 0) enqueues nothing and returns AQ_OK whatever its
 *    data pointers hold, except for MOSS, whose reference rejects it.
 *  - A handle (stages, codebooks, quantizer, linear) records its device,
 *    not its creating context: it may be released after that context is
 *    destroyed, and is used with any context on the same device.
 *
 * Reference interfaces replaced (paths relative to the audio.cpp tree):
 *  - engine::runtime::VectorQuantizer::compute
 *      include/engine/framework/runtime/host_ops.h:87-96,
 *      src/framework/runtime/host_ops.cpp:236-273
 *  - the inline encode quantizers of the codec models:
 *      Fish DAC cosine   src/models/fish_audio/codec.cpp:570-611
 *      OmniVoice         src/models/omnivoice/audio_tokenizer.cpp:1886-1927 (with projections)
 *      Higgs             src/models/higgs_audio_tts/codec.cpp:958-1016 (with projections)
 *      Qwen3 / VieNeu    src/models/qwen3_tts/tokenizer_speech_encoder.cpp:287-349
 *      MOSS RLFQ         src/models/moss/shared/audio_tokenizer_quantizer.cpp:174-271
 *  - engine::modules::CodebookLookupModule / EmbeddingModule (ggml_get_rows)
 *      include/engine/framework/modules/lookup_modules.h:69-82,
 *      src/framework/modules/lookup_modules.cpp:88-112,182-187
 */
#ifndef AQ_MI355X_H
#define AQ_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AQ_ABI_VERSION 1

typedef enum aq_status {
    AQ_OK = 0,
    AQ_E_INVALID_ARG = 1,   /* null handle/pointer, bad enum value            */
    AQ_E_SHAPE = 2,         /* sizes inconsistent or outside supported range  */
    AQ_E_INDEX_RANGE = 3,   /* a code index outside [0, N)                    */
    AQ_E_DEVICE = 4,        /* a HIP runtime call failed                      */
    AQ_E_UNSUPPORTED = 5,   /* valid request this build does not implement    */
    AQ_E_NOMEM = 6          /* device or host allocation failed               */
} aq_status;

typedef struct aq_ctx aq_ctx;             /* device + stream + scratch       */
typedef struct aq_dac_stages aq_dac_stages;   /* uploaded DAC RVQ weights    */
typedef struct aq_codebooks aq_codebooks; /* uploaded Euclidean codebooks    */

/* ---- context -------------------------------------------------------------- */

/* Create a context on HIP device `device`; `hip_stream` is a hipStream_t (NULL
 * = the null stream).  Replaces backend/session setup
 * (src/framework/core/backend.cpp:94 init_backend). */
aq_status aq_ctx_create(int device, void *hip_stream, aq_ctx **out);
aq_status aq_ctx_destroy(aq_ctx *ctx);
aq_status aq_ctx_set_stream(aq_ctx *ctx, void *hip_stream);
/* Blocks until all work enqueued on the context's stream has finished. */
aq_status aq_ctx_synchronize(aq_ctx *ctx);
/* Message of the last failure on ctx ("" if none).  Valid until the next call. */
const char *aq_last_error(const aq_ctx *ctx);
int aq_abi_version(void);

/* Kernel timing, a measurement aid with no counterpart in the reference: when
 * enabled, the library brackets each launch of its main kernels (the DAC
 * encode kernel, each Euclidean stage's score kernel) with HIP events on the
 * context's stream.  aq_ctx_read_timing synchronises the stream, writes up to
 * `capacity` durations in milliseconds (launch order) and the number
 * recorded to *count, and starts a new record. */
aq_status aq_ctx_set_timing(aq_ctx *ctx, int enable);
aq_status aq_ctx_read_timing(aq_ctx *ctx, float *ms, int capacity, int *count);

/* ---- DAC-style cosine RVQ (Fish Audio recipe) --------------------------------
 *
 * Per stage s (codec.cpp:587-605):
 *   p    = W_in[s] r + b_in[s]                 (1x1 conv D -> 8)
 *   pn   = p / sqrt(sum(p*p) + 1e-12)
 *   code = argmax_n <normalize(c[s][n]), pn>   (last index among equal maxima)
 *   z    = W_out[s] c[s][code] + b_out[s]      (1x1 conv 8 -> D)
 *   r   -= z ;  recon += z
 * Codebook rows are L2-normalised at upload exactly as codec.cpp:171-189
 * (double sum of squares, float inverse).
 */

/* Upload Q stages of DAC weights from host memory (upload once, reuse).
 *   w_in  [Q, 8, D]   b_in  [Q, 8]   (NULL = no bias)
 *   codebook [Q, N, 8]
 *   w_out [Q, D, 8]   b_out [Q, D]   (NULL = no bias)
 * Supported: codebook dim 8, any D >= 1 (up to 40000) and N >= 1 (up to
 * 2^24), as the reference's graphs accept.  D in {64, 128, 256, 512, 768,
 * 1024} with N a multiple of 64 up to 2^20 runs the fused kernel (residual
 * in registers, certified approximate scores); other shapes run a cascade
 * kernel with run-time D and N (residual in LDS, every score exact), with
 * the same results.
 * Replaces load_quantizer_unit (codec.cpp:693-720) / BackendWeightStore. */
aq_status aq_dac_upload(aq_ctx *ctx, int64_t Q, int64_t D, int64_t N,
                        const float *w_in, const float *b_in, const float *codebook,
                        const float *w_out, const float *b_out, aq_dac_stages **out);

/* The same cosine quantizer with another model family's normalisation
 * (the variants of the query and codebook L2 normalisation in the model
 * code):
 *   AQ_DAC_FISH       pn = p / sqrt(sum(p*p) + 1e-12); rows c * (float)(1/|c|),
 *                     zero rows -> 0 (fish_audio/codec.cpp:171-189,323-334)
 *   AQ_DAC_INDEXTTS2  pn = p / sqrt(sum(p*p)) (normalize_code_latents,
 *                     index_tts2/semantic_codec.cpp:110-115); rows
 *                     c * (1.0F / (float)|c|) (normalized_codebook, :43-58)
 *   AQ_DAC_VEVO2      pn = p / sqrt(sum(p*p) + 1e-20) (build_l2_normalized_rows,
 *                     vevo2/components.cpp:848-863); rows c * (float)(1/|c|),
 *                     a zero row is an error (l2_normalized_rows, :566-590)
 * These three take the ggml arithmetic of the Fish path otherwise (1x1 conv,
 * k = 8 mul_mat scores, argmax keeping the last maximum).  w_out (and b_out)
 * may be NULL for a single stage (Q = 1): codes only, as the IndexTTS2 and
 * Vevo2 tokenisers use them; encode then takes no residual / recon and decode
 * is unavailable.  Codebooks too large for LDS next to W_in (e.g. IndexTTS2's
 * 8192 x 8 with D = 1024) are read from device memory.
 *   AQ_DAC_OUTETTS    the OuteTTS host loop (quantize_reference,
 *                     community_models/outetts/dac.cpp:376-456): fp32, each
 *                     product rounded before it is added, bias first;
 *                     p / (sqrt(sum p*p) + 1e-12) against c / (sqrt(sum c*c)
 *                     + 1e-12), first index of the minimum squared distance;
 *                     residual -= b_out + W_out c.  w_out is required; D a
 *                     multiple of 64 up to 2048, N a multiple of 8; clip_len
 *                     does not change the arithmetic; encode takes no recon
 *                     (aq_dac_decode gives it, with the ggml 1x1-conv
 *                     arithmetic of the OuteTTS decoder graph, dac.cpp:596-611). */
typedef enum aq_dac_recipe {
    AQ_DAC_FISH = 0,
    AQ_DAC_INDEXTTS2 = 1,
    AQ_DAC_VEVO2 = 2,
    AQ_DAC_OUTETTS = 3
} aq_dac_recipe;
aq_status aq_dac_upload_ex(aq_ctx *ctx, int64_t Q, int64_t D, int64_t N,
                           const float *w_in, const float *b_in, const float *codebook,
                           const float *w_out, const float *b_out, int recipe, aq_dac_stages **out);
aq_status aq_dac_release(aq_dac_stages *stages);

/* Encode M frames through all Q stages (codec.cpp:570-611).
 *   x         device [M, D]  (frame-major; not modified)
 *   clip_len  frames per clip T (M must be a multiple of T).  The reference
 *             runs one 1x1 conv per clip, and ggml picks the in-projection
 *             summation order from T (tinyBLAS when T % 4 == 0, vec_dot
 *             otherwise); the library reproduces whichever applies.
 *   idx       device [M, Q] int32 (frame-major codes)
 *   residual  device [M, D] or NULL: residual after the last stage
 *   recon     device [M, D] or NULL: sum over stages of z (decode recipe,
 *             codec.cpp:552-568)
 *   force_idx device [M, Q] or NULL: teacher forcing -- the residual update of
 *             stage s uses force_idx[m, s] instead of the computed code (idx
 *             still receives the computed code); used for per-stage parity. */
aq_status aq_dac_encode(aq_ctx *ctx, const aq_dac_stages *stages, const float *x, int64_t M,
                        int64_t clip_len, int32_t *idx, float *residual, float *recon,
                        const int32_t *force_idx);

/* aq_dac_encode with a strided input, a row stride for the codes and a
 * recon that continues an earlier cascade.  For a cascade whose stages do
 * not share one codebook size, such as Fish's semantic quantizer of 4096
 * codes followed by residual quantizers of 1024 (fish_audio/codec.cpp:
 * 606-608), upload each group as its own stages object and chain them:
 *   encode_ex(semantic, x, ..., idx, idx_ld = Q_total, residual = r, recon, 0)
 *   encode_ex(rest, r, ..., idx + 1, idx_ld = Q_total, residual, recon, 1)
 * gives the codes, residual and recon (the decoder's sum z_0 + z_1 + ...,
 * codec.cpp:552-568) of the single cascade, bit for bit.
 *   x            frame m, channel d at x + (m / clip_len) * clip_stride +
 *                (m % clip_len) * frame_stride + d * chan_stride (channel-major
 *                [B, D, T]: clip_stride = D*T, frame_stride = 1, chan_stride = T)
 *   idx_ld       row stride of idx and force_idx (>= Q); codes at idx[m*idx_ld + s]
 *   recon_accumulate  nonzero: recon holds the sum of earlier stages on entry
 * The OuteTTS recipe takes idx_ld = Q and no recon. */
aq_status aq_dac_encode_ex(aq_ctx *ctx, const aq_dac_stages *stages, const float *x, int64_t M, int64_t clip_len,
                           int64_t clip_stride, int64_t frame_stride, int64_t chan_stride, int32_t *idx,
                           int64_t idx_ld, float *residual, float *recon, int recon_accumulate,
                           const int32_t *force_idx);

/* Decode: recon[m] = sum_s (W_out[s] c[s][idx[m, s]] + b_out[s])
 * (build_decode_quantizer, codec.cpp:552-568).  idx device [M, Q], out device
 * [M, D].  Out-of-range codes -> AQ_E_INDEX_RANGE (checked on device; the call
 * synchronises the stream to report it). */
aq_status aq_dac_decode(aq_ctx *ctx, const aq_dac_stages *stages, const int32_t *idx, int64_t M,
                        float *out);
/* aq_dac_decode with codes at idx[m*idx_ld + s]; accumulate nonzero adds the
 * stages' z to what out holds (the decode of a chained cascade, as above). */
aq_status aq_dac_decode_ex(aq_ctx *ctx, const aq_dac_stages *stages, const int32_t *idx, int64_t idx_ld, int64_t M,
                           float *out, int accumulate);

/* ---- Euclidean VQ / RVQ (Mimi-style codecs, k-means tokenisers) ------------
 *
 * Nearest codeword by squared Euclidean distance, with the residual cascade
 * r <- r - c[code] across Q stages in codebook space (Qwen3 / VieNeu,
 * VectorQuantizer, k-means tokenisers).  The OmniVoice and Higgs acoustic
 * quantizers project the residual in and out of each stage's codebook space
 * and keep it in hidden space: aq_euclid_upload_projected below uploads them
 * as one cascade; aq_euclid_upload without projections reproduces one of
 * their stages on already projected queries.  `recipe` selects the reference
 * arithmetic the results are identical to:
 *   AQ_EUCLID_OMNIVOICE  logit = mul_mat(2c, r) + (float)(-(double)|c|^2),
 *                        argmax, last index among equal maxima
 *                        (omnivoice/audio_tokenizer.cpp:1227-1237,1897-1927)
 *   AQ_EUCLID_HIGGS      logit = ((2*mul_mat(c, r)) - sum_rows(r*r)) -
 *                        sum_rows(c*c), argmax (higgs_audio_tts/codec.cpp:975-1013);
 *                        F32 or Q8_0 codebooks (a Q8_0 mul_mat quantises r to
 *                        Q8_0 with x86 rounding first)
 *   AQ_EUCLID_DIRECT     distance = sum (x-c)^2 (rounded products added in
 *                        order), first index of the minimum
 *                        (VectorQuantizer::compute, host_ops.cpp:236-273;
 *                        Qwen3 nearest_code, tokenizer_speech_encoder.cpp:287-303)
 * Scores are contracted in fp16 on the matrix cores; every code that could
 * win is re-ranked in the recipe's fp32 arithmetic under a rigorous error
 * bound, and frames the bound cannot settle are rescanned exactly, so the
 * outputs equal the reference's. */
typedef enum aq_euclid_recipe {
    AQ_EUCLID_OMNIVOICE = 0,
    AQ_EUCLID_HIGGS = 1,
    AQ_EUCLID_DIRECT = 2
} aq_euclid_recipe;

typedef enum aq_codebook_type {
    AQ_CB_F32 = 0,    /* float [Q][N][K]                                       */
    AQ_CB_Q8_0 = 1,   /* GGUF block_q8_0 {fp16 d; int8 qs[32]} [Q][N][K/32],
                         34 bytes per block (ggml-common.h:241-246)             */
    AQ_CB_F32_AS_Q8_0 = 2  /* float [Q][N][K] stored as Q8_0, quantised on the
                         device at upload as the reference's weight store does
                         for a Q8_0 storage type (ggml_quantize_chunk ->
                         quantize_row_q8_0_ref: d = amax/127, q = roundf(x/d);
                         backend_weight_store.h:272-287,343-392,
                         tensor_source.cpp:173-200)                             */
} aq_codebook_type;

/* Upload Q codebooks of N codes of dimension K from host memory (upload
 * once; replaces BackendWeightStore loads, backend_weight_store.h:272-392,
 * and the per-call codebook set-up of the host loops).  The data goes to
 * the device as given; Q8_0 blocks are unpacked and every derived image and
 * constant is built there (only 5 bounds per stage come back).
 * Supported: any K >= 1 (up to 16384) and N >= 1 (up to 2^24), as the
 * reference's VectorQuantizer and mul_mat graphs accept; Q8_0 rows are whole
 * 32-element blocks (K % 32 == 0) and follow AQ_EUCLID_HIGGS only.  K in
 * {64, 256, 512, 768} with N a multiple of 256, 64, 32, 16 respectively (up
 * to 2^20) runs the matrix-core sweep with its certificate; other shapes
 * scan every frame exactly in the recipe's arithmetic (same results).  For
 * a codebook width that is not a multiple of 64 in ggml_vec_dot_f32's order
 * (one query, or K % 16 != 0, or N % 4 != 0), the results are those of the
 * reference's default native x86 build (its leftover products: the last
 * n % 4 fused, the others rounded then added). */
aq_status aq_euclid_upload(aq_ctx *ctx, int64_t Q, int64_t N, int64_t K, int cb_type, const void *data,
                           int recipe, aq_codebooks **out);
/* aq_euclid_upload from device memory (a codebook already resident, e.g.
 * loaded by the caller's weight store or produced by a graph): data is a
 * device pointer of the same layout, copied on the context's stream. */
aq_status aq_euclid_upload_device(aq_ctx *ctx, int64_t Q, int64_t N, int64_t K, int cb_type, const void *data,
                                  int recipe, aq_codebooks **out);
aq_status aq_euclid_release(aq_codebooks *cb);

/* Encode M frames through all stages.
 *   x          device [M, K] (frame-major; not modified)
 *   idx        device [M, Q] int32 codes
 *   residual   device [M, K] or NULL: residual after the last stage
 *   dist       device [M, Q] or NULL: the winner's distance in the recipe's
 *              arithmetic (DIRECT: the distance; OMNIVOICE / HIGGS: -logit)
 *   topk       0..4: also the topk best codes per stage, best first (ties
 *              by index; ggml_top_k's order is unspecified, compare as sets)
 *   topk_idx   device [M, Q, topk];  topk_dist device [M, Q, topk]
 *   force_idx  device [M, Q] or NULL: teacher forcing of the residual update */
aq_status aq_euclid_encode(aq_ctx *ctx, const aq_codebooks *cb, const float *x, int64_t M, int32_t *idx,
                           float *residual, float *dist, int topk, int32_t *topk_idx, float *topk_dist,
                           const int32_t *force_idx);

/* aq_euclid_encode without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The work
 * buffers (the residual when `residual` is NULL, sweep keys, frame lists,
 * refine keys, projected queries) live in one 32 MiB device region that the
 * library holds on each device it runs on until the process ends; refine
 * keys get what the other buffers leave (frames past that go to the exact
 * scan, same results).  A call that needs more of the region fails with
 * AQ_E_SHAPE (e.g. a 48 000 x 256 Mimi batch needs a caller residual buffer).
 * Every call on a device shares the region.  Calls are ordered on the device
 * through one HIP event per device (created with the region's address at
 * the first call): each call's stream waits for the previous call's work,
 * from any context and stream, and the host enqueues one call at a time per
 * device.  Calls captured into a HIP graph are not ordered by the event:
 * graph launches that contain this call must not overlap each other or
 * other calls on the device.  The counters of aq_euclid_failures /
 * aq_euclid_exact_scans refer to the region, i.e. to the last no-allocation
 * call on the device.  Results equal aq_euclid_encode's. */
aq_status aq_euclid_encode_noalloc(aq_ctx *ctx, const aq_codebooks *cb, const float *x, int64_t M, int32_t *idx,
                                   float *residual, float *dist, int topk, int32_t *topk_idx, float *topk_dist,
                                   const int32_t *force_idx);

/* aq_euclid_encode on a strided input, e.g. the channel-major [B, C, T]
 * latent of a ggml encoder graph (qwen3_tts/tokenizer_speech_encoder.cpp:
 * 330-335 reads it that way; outetts/dac.cpp:565-571 and
 * higgs_audio_tts/codec.cpp:965 transpose it first): frame m, channel c at
 *   x + (m / clip_len) * clip_stride + (m % clip_len) * frame_stride + c * chan_stride.
 * Channel-major [B, C, T]: clip_len = T, clip_stride = C*T, frame_stride = 1,
 * chan_stride = T.  Frame-major [M, C]: clip_len = M, frame_stride = C,
 * chan_stride = 1 (= aq_euclid_encode).  The outputs stay frame-major. */
aq_status aq_euclid_encode_strided(aq_ctx *ctx, const aq_codebooks *cb, const float *x, int64_t M, int64_t clip_len,
                                   int64_t clip_stride, int64_t frame_stride, int64_t chan_stride, int32_t *idx,
                                   float *residual, float *dist, int topk, int32_t *topk_idx, float *topk_dist,
                                   const int32_t *force_idx);

/* Projected Euclidean RVQ: the OmniVoice and Higgs acoustic quantizers
 * (omnivoice/audio_tokenizer.cpp:1886-1927; higgs_audio_tts/codec.cpp:958-1016).
 * Per stage s, on the residual r of hidden size H (x at stage 0):
 *   p    = W_in[s] r + b_in[s]              (LinearModule H -> K)
 *   code = argmax of the recipe's logits of p against codebook s
 *   r   -= W_out[s] c[s][code] + b_out[s]   (LinearModule K -> H)
 * in ggml's arithmetic (tinyBLAS or ggml_vec_dot_f32 for F32 weights as ggml
 * picks them, the quantised block dot for Q8_0 weights).  Replaces the
 * quantizer loops of those two graphs and their weight loads
 * (audio_tokenizer.cpp:1223-1271; higgs codec.cpp:544-568).
 *   codebook  [Q, N, K] as cb_type (Q8_0 with AQ_EUCLID_HIGGS only)
 *   w_in      [Q, K, H] and w_out [Q, H, K] as proj_type (AQ_CB_F32, or
 *             AQ_CB_Q8_0 block rows), b_in [Q, K] and b_out [Q, H] float or NULL
 * recipe AQ_EUCLID_OMNIVOICE or AQ_EUCLID_HIGGS; K as aq_euclid_upload; H a
 * multiple of 64 (up to 2496 for F32 weights, 1984 for Q8_0).  The handle
 * works with aq_euclid_encode / aq_euclid_encode_strided (x and residual
 * [M, H]), aq_euclid_decode (out [M, H] = sum over stages of
 * W_out c + b_out, the decoders' sum, audio_tokenizer.cpp:1745-1771 and
 * higgs codec.cpp:1040-1065) and aq_codebook_gather (codebook rows, [M, K]). */
aq_status aq_euclid_upload_projected(aq_ctx *ctx, int64_t Q, int64_t N, int64_t K, int64_t H, int cb_type,
                                     const void *codebook, int proj_type, const void *w_in, const float *b_in,
                                     const void *w_out, const float *b_out, int recipe, aq_codebooks **out);

/* Frames per stage (first min(Q, 64) stages) of the last encode on ctx that
 * the fp16 error certificate could not settle: the split-fp16 refine pass
 * took them or, when no more than 64 were open, the exact scan; in the
 * one-launch cascade (codebooks at K = 256) the frames that continued
 * with their best exactly evaluated candidate and were verified by the
 * exact scan afterwards (host int32 array; synchronises the stream).  A
 * measurement aid with no reference counterpart. */
aq_status aq_euclid_failures(aq_ctx *ctx, const aq_codebooks *cb, int32_t *host_counts);

/* Frames per stage (first min(Q, 64) stages) of the last encode on ctx that
 * the exact scan decided: those the refine pass left open, or all open
 * frames when no more than 64 were; in the one-launch cascade the frames
 * whose verified continuation was wrong, recomputed from that stage on and
 * counted at each recomputed stage (host int32 array; synchronises the
 * stream).  A measurement aid with no reference counterpart. */
aq_status aq_euclid_exact_scans(aq_ctx *ctx, const aq_codebooks *cb, int32_t *host_counts);

/* EMA codebook materialisation, once at load (Mimi-style codecs store
 * embedding_sum and cluster_usage): codebook[q,n,k] = embedding_sum[q,n,k] /
 * std::max(cluster_usage[q,n], eps).  Replaces codebook_embedding
 * (qwen3_tts/tokenizer_speech_encoder.cpp:271-285, called per encode there;
 * also tokenizer_speech_decoder.cpp:205-212), whose eps is 1e-5.
 * Device pointers: embedding_sum [Q,N,K], cluster_usage [Q,N], codebook
 * [Q,N,K] (may not alias the inputs). */
aq_status aq_ema_codebook(aq_ctx *ctx, const float *embedding_sum, const float *cluster_usage, int64_t Q, int64_t N,
                          int64_t K, float eps, float *codebook);

/* aq_euclid_upload of an EMA codebook: host embedding_sum [Q,N,K] and
 * cluster_usage [Q,N] are materialised on the device with aq_ema_codebook's
 * arithmetic, straight into the set's buffer, and prepared there as an F32
 * codebook for `recipe` (no copy back to the host). */
aq_status aq_euclid_upload_ema(aq_ctx *ctx, int64_t Q, int64_t N, int64_t K, const float *embedding_sum,
                               const float *cluster_usage, float eps, int recipe, aq_codebooks **out);

/* ---- Weight-norm folding on the device -----------------------------------
 *
 * w[r, :] = v[r, :] * scale_r for a weight-normalised conv (rows = output
 * channels, cols = in_channels * kernel), scale_r from g[r] and the double
 * sum of squares of v's row, as the model loaders fold them:
 *   AQ_WN_OUTETTS  scale = g / (float)sqrt(norm2), fp32 division
 *                  (fold_weight_norm, community_models/outetts/dac.cpp:91-110)
 *   AQ_WN_MOSS     scale = (float)(g / sqrt(norm)), double division
 *                  (reconstruct_weight_norm,
 *                  models/moss/shared/audio_tokenizer_quantizer.cpp:17-39)
 * Device pointers v [rows, cols], g [rows], w [rows, cols] (w may be v).
 * Replaces those host loops; the folded weights then go to aq_dac_upload_ex
 * (AQ_DAC_OUTETTS) or aq_moss_upload. */
typedef enum aq_wn_rule { AQ_WN_OUTETTS = 0, AQ_WN_MOSS = 1 } aq_wn_rule;
aq_status aq_weight_norm_fold(aq_ctx *ctx, const float *v, const float *g, int64_t rows, int64_t cols, int rule,
                              float *w);

/* ---- MOSS RLFQ quantizer (fp64 host loop) ---------------------------------
 *
 * MossAudioTokenizerQuantizer (models/moss/shared/audio_tokenizer_quantizer.cpp):
 *   encode (:174-271)  residual = b_ip + W_ip h in fp64 (W_ip [R, C]); per
 *                      stage e = b_in + W_in residual in fp64 (each float
 *                      weight times the double residual rounded, then added),
 *                      e *= 1 / std::max(|e|, 1e-12), code = first index of
 *                      the maximum fp64 dot with the normalised codebook,
 *                      residual -= b_out + W_out c[code] in fp64.
 *   decode (:139-172)  latent = b_op + sum over stages of the constructor's
 *                      fp32 latent tables (:77-115).
 * Weight-normalised convs are passed folded (w = g v / |v|, as
 * reconstruct_weight_norm builds them, :17-39).  Host weights:
 *   input_w [R, C], input_b [R]               (quantizer.input_proj)
 *   in_w [Q, 8, R], in_b [Q, 8]               (quantizers.s.in_proj)
 *   codebook [Q, N, 8]                        (quantizers.s.codebook, raw)
 *   out_w [Q, R, 8], out_b [Q, R]             (quantizers.s.out_proj)
 *   output_w [C, R], output_b [C] or both NULL (quantizer.output_proj; decode)
 * with C = code_dim, R = rvq_dim.  Supported: N a multiple of 8, R a multiple
 * of 64 up to 1024.  Replaces the MossAudioTokenizerQuantizer constructor. */
typedef struct aq_moss_quantizer aq_moss_quantizer;
aq_status aq_moss_upload(aq_ctx *ctx, int64_t Q, int64_t N, int64_t code_dim, int64_t rvq_dim,
                         const float *input_w, const float *input_b, const float *in_w, const float *in_b,
                         const float *codebook, const float *out_w, const float *out_b,
                         const float *output_w, const float *output_b, aq_moss_quantizer **out);
aq_status aq_moss_release(aq_moss_quantizer *q);

/* Encode (MossAudioTokenizerQuantizer::encode): hidden device [M, C]
 * frame-major; idx device [M, Q] (the reference returns [Q][M]); residual
 * device [M, R] doubles or NULL (the fp64 residual after the last stage);
 * force_idx device [M, Q] or NULL (teacher forcing, as aq_dac_encode).
 * M = 0 is AQ_E_SHAPE with the reference's message. */
aq_status aq_moss_encode(aq_ctx *ctx, const aq_moss_quantizer *q, const float *hidden, int64_t M, int32_t *idx,
                         double *residual, const int32_t *force_idx);

/* Decode (MossAudioTokenizerQuantizer::decode): idx device [M, Q], latent
 * device [M, C] frame-major (the reference returns [C, M]).  Out-of-range
 * codes -> AQ_E_INDEX_RANGE with the reference's message (checked on device;
 * the call synchronises the stream). */
aq_status aq_moss_decode(aq_ctx *ctx, const aq_moss_quantizer *q, const int32_t *idx, int64_t M, float *latent);

/* Codebook gather of one stage: out[m] = codebook[stage][idx[m]] (ggml_get_rows,
 * lookup_modules.cpp:88-112,182-187; Q8_0 rows dequantised as q*d).
 * idx device [M], out device [M, K].  Out-of-range codes -> AQ_E_INDEX_RANGE. */
aq_status aq_codebook_gather(aq_ctx *ctx, const aq_codebooks *cb, int64_t stage, const int32_t *idx, int64_t M,
                             float *out);

/* Decode: out[m] = sum over stages of codebook[s][idx[m, s]], in stage order.
 * idx device [M, Q], out device [M, K]. */
aq_status aq_euclid_decode(aq_ctx *ctx, const aq_codebooks *cb, const int32_t *idx, int64_t M, float *out);

/* ---- Encoder output projection in the CPU's arithmetic --------------------
 *
 * The layer in front of the quantizer (an encoder's output Linear / 1x1
 * conv, LinearModule::forward, src/framework/modules/linear_module.cpp:73-108)
 * with ggml's CPU arithmetic, deterministic on the device:
 *   out[m, o] = mul_mat(W, x_m)[o] (+ bias[o], ggml_add)
 * F32 weights: tinyBLAS order for a batch of M >= 2 frames (16 FMA lanes
 * over k = 16u + t, then _mm512_reduce_add_ps's pairing; sgemm.cpp), the
 * ggml_vec_dot_f32 order for one frame (ggml-cpu.c:1245-1443); Q8_0 weights:
 * x quantised by x86 quantize_row_q8_0, then int8 block dots scaled by
 * d_w * d_x and FMA-accumulated over 8 lanes (tinyBLAS_Q0 /
 * ggml_vec_dot_q8_0_q8_0).  The reference pins voice-prompt encoding to the
 * CPU because its CUDA path runs TF32 (qwen3_tts/session.cpp:101-107); this
 * gives the CPU's bits on the GPU.  The input is read through the frame
 * descriptor of aq_euclid_encode_strided (channel-major [B, C, T] taken
 * as is); the output is frame-major [M, out_features].
 *   w     host [out_features, in_features] F32, or block_q8_0 rows (w_type
 *         AQ_CB_Q8_0); bias host [out_features] or NULL.
 * Supported: out_features a multiple of 64; in_features a multiple of 64 up
 * to 2496 (F32) / 1984 (Q8_0). */
typedef struct aq_linear aq_linear;
aq_status aq_linear_upload(aq_ctx *ctx, int64_t out_features, int64_t in_features, int w_type, const void *w,
                           const float *bias, aq_linear **out);
aq_status aq_linear_forward(aq_ctx *ctx, const aq_linear *lin, const float *x, int64_t M, int64_t clip_len,
                            int64_t clip_stride, int64_t frame_stride, int64_t chan_stride, float *out);
aq_status aq_linear_release(aq_linear *lin);

#ifdef __cplusplus
}
#endif
#endif /* AQ_MI355X_H */
