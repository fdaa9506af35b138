// Projected Euclidean RVQ (OmniVoice / Higgs acoustic quantizers): the
// per-stage project_in / project_out around the codebook search, with the
// residual kept in hidden space.  Internal interface between aq_euclid.hip
// (ABI, stage pipeline) and aq_projected.hip (projection kernels).
#pragma once

#include "aq_internal.hpp"

// Frames of a possibly strided input: frame m, channel h at
//   x + (m / clip_len) * clip_stride + (m % clip_len) * frame_stride + h * chan_stride.
// Frame-major [M, C]: clip_len = M, frame_stride = C, chan_stride = 1.
// ggml's channel-major [B, C, T]: clip_len = T, clip_stride = C * T,
// frame_stride = 1, chan_stride = T.
struct aq_frames_desc {
    const float *x;
    int64_t clip_len, clip_stride, frame_stride, chan_stride;
};

inline aq_frames_desc aq_frames_row_major(const float *x, int64_t M, int64_t C) {
    return aq_frames_desc{x, M > 0 ? M : 1, M * C, C, 1};
}

// Device images of the projections of Q stages.
struct aq_proj_weights {
    int64_t Q = 0, N = 0, K = 0, H = 0;
    bool q8 = false;            // Q8_0 projection weights
    float *w_in = nullptr;      // [Q][K][H] (F32)
    int8_t *w_in_q = nullptr;   // [Q][K][H] quants (Q8_0)
    float *w_in_d = nullptr;    // [Q][K][H/32] scales (Q8_0)
    float *b_in = nullptr;      // [Q][K] or null
    float *w_out = nullptr;     // [Q][H][K] (F32; the single-frame path)
    float *b_out = nullptr;     // [Q][H] or null
    float *table = nullptr;     // [Q][N][H]: project_out(c[n]) + b_out
    const float *cbf = nullptr; // [Q][N][K] the fp32 codebooks (owned by the aq_codebooks)
};

// Upload the projections and build the project_out tables from the device
// fp32 codebooks d_cbf [Q][N][K].  proj_type: AQ_CB_F32 or AQ_CB_Q8_0 (host
// data: F32 [Q][K][H] / [Q][H][K], or block_q8_0 rows of the same shapes).
aq_status aq_proj_create(aq_ctx *ctx, int64_t Q, int64_t N, int64_t K, int64_t H, const float *d_cbf,
                         int proj_type, const void *w_in, const float *b_in, const void *w_out,
                         const float *b_out, aq_proj_weights **out);
void aq_proj_release(aq_proj_weights *pw);

// A single F32 / Q8_0 linear layer (Q = 1, no codebook, no out-projection):
// w [O][I] (F32) or block_q8_0 rows, b [O] or null; run with aq_proj_step
// (s = 0, prev = -1).
aq_status aq_proj_create_linear(aq_ctx *ctx, int64_t O, int64_t I, int w_type, const void *w, const float *b,
                                aq_proj_weights **out);

// One projection step over M frames:
//   r = in (frame m's hidden vector);
//   if prev >= 0: r -= table[prev][code(m)], code(m) = codes[m * ld + prev]
//                 (AQ_FLAG_BAD_INDEX and code 0 when out of range);
//   if rout: rout[m] = r (frame-major [M, H]; may alias in.x when in is
//            frame-major);
//   if s >= 0: p[m] = project_in[s](r) (frame-major [M, K]).
// The arithmetic is ggml's LinearModule for a batch of M frames (tinyBLAS
// for F32 weights when M >= 2, ggml_vec_dot_f32 for M = 1; the Q8_0 product
// for Q8_0 weights).
aq_status aq_proj_step(aq_ctx *ctx, const aq_proj_weights *pw, int s, int prev, const aq_frames_desc &in,
                       float *rout, const int32_t *codes, int ld, float *p, int64_t M);

// Decode: out[m] = sum over stages, in order, of project_out[s](c_s[idx[m, s]])
// (frame-major [M, H]); AQ_FLAG_BAD_INDEX on an out-of-range code.
aq_status aq_proj_decode(aq_ctx *ctx, const aq_proj_weights *pw, const int32_t *idx, int64_t M, float *out);

// AQ_OK when the projection kernels' LDS (16 frames of H + 1 floats, plus
// their Q8_0 image for Q8_0 weights; one H-float row for a single frame)
// fits a CU next to their static LDS; else AQ_E_SHAPE with `fn` in the
// message.
aq_status aq_proj_check_lds(aq_ctx *ctx, int64_t H, bool q8, const char *fn);

// Gather of a strided input into frame-major rows: out[m, c] for c < C.
aq_status aq_gather_frames(aq_ctx *ctx, const aq_frames_desc &in, int64_t M, int64_t C, float *out);
