/*
 * aq_mi355x.h -- C ABI of the MI355X (gfx950) codec-quantizer library.
 *
 * The library replaces audio.cpp's codec-quantizer hot path: the VQ/RVQ
 * encode that maps latent frames to codebook indices by nearest-neighbour
 * search, the residual cascade across codebooks, and the codebook-gather
 * decode.  Results are bit-identical to the reference's ggml CPU backend on
 * the same inputs (same fp32 operation order, fused multiply-adds, double
 * accumulations and tie rules).
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
 *
 * Reference interfaces replaced (paths relative to the audio.cpp tree):
 *  - engine::runtime::VectorQuantizer::compute
 *      include/engine/framework/runtime/host_ops.h:87-96,
 *      src/framework/runtime/host_ops.cpp:236-273
 *  - the inline encode quantizers of the codec models:
 *      Fish DAC cosine   src/models/fish_audio/codec.cpp:570-611
 *      OmniVoice         src/models/omnivoice/audio_tokenizer.cpp:1886-1927
 *      Higgs             src/models/higgs_audio_tts/codec.cpp:958-1016
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
 * Supported: codebook dim 8, D in {64, 128, ..., 1024} (multiple of 64),
 * N a multiple of 64 up to 8192.
 * Replaces load_quantizer_unit (codec.cpp:693-720) / BackendWeightStore. */
aq_status aq_dac_upload(aq_ctx *ctx, int64_t Q, int64_t D, int64_t N,
                        const float *w_in, const float *b_in, const float *codebook,
                        const float *w_out, const float *b_out, aq_dac_stages **out);
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

/* Decode: recon[m] = sum_s (W_out[s] c[s][idx[m, s]] + b_out[s])
 * (build_decode_quantizer, codec.cpp:552-568).  idx device [M, Q], out device
 * [M, D].  Out-of-range codes -> AQ_E_INDEX_RANGE (checked on device; the call
 * synchronises the stream to report it). */
aq_status aq_dac_decode(aq_ctx *ctx, const aq_dac_stages *stages, const int32_t *idx, int64_t M,
                        float *out);

#ifdef __cplusplus
}
#endif
#endif /* AQ_MI355X_H */
