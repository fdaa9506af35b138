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
//    Each lane runs its FMA chain over i.  The reduction then pairs the same
//    partial sums as ggml's tree (j with j+2, j with j+1, then lanes 8, 4, 2,
//    1 apart inside each 16-lane row), so the projection is bit-identical;
//    IEEE addition is commutative, so which lane of a pair adds is free.
//    The two cross-row levels are transposed (each lane finishes 2 of the 8
//    outputs) and the in-row levels are DPP row rotations.
//  * The stage's in-projection weights and L2-normalised codebook are staged
//    in LDS in a lane-major float4 layout (conflict-free ds_read_b128); each
//    LDS read feeds FW frames.  Two blocks share a CU, so one block's stage
//    load overlaps the other's compute.
//  * Scores: every lane scores codes n = 64*c + L with an FMA chain (8 ops)
//    and keeps its two best keys (score with the chunk index c in the low
//    mantissa bits; max / med3).  A margin certificate proves the winner:
//    if the best key is unique and beats every other code's key by more than
//    the worst-case gap between these scores and ggml's (product-rounded,
//    sequential) scores plus the key truncation, ggml's argmax is the same
//    code.  Frames that fail it (near-ties, zero or non-finite projections)
//    are rescored with ggml's exact arithmetic and tie rule (last index).
//  * The out-projection z = W_out c[code] + b_out depends only on the code, so
//    it is tabulated per stage at upload time with the reference's arithmetic
//    (sequential non-fused 8-term sum, then the bias) and gathered per frame:
//    a coalesced 4*D-byte row read from L2/MALL instead of 2*8*D flops.
#include "aq_device_math.hpp"
#include "aq_internal.hpp"
#include "aq_projected.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <new>
#include <vector>

namespace {

constexpr int kWave = 64;
constexpr int kMaxBlock = 512;   // threads; the launch picks 4, 6 or 8 waves per block

// Values that are identical in every lane (after a full reduction) are moved
// to scalar registers; VALU instructions then read them as SGPR operands.
__device__ inline float uniform_f(float v) {
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}
__device__ inline int uniform_i(int v) { return __builtin_amdgcn_readfirstlane(v); }

using aq_math::sqrt_rn;   // correctly rounded fp32 square root

// v + v[lane rotated by N inside its 16-lane row] (DPP row_ror).
template <int N>
__device__ inline float row_ror_add(float v) {
    const int o = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + N, 0xF, 0xF, false);
    return __fadd_rn(v, __int_as_float(o));
}
// v from lane + N of its 16-lane row (DPP row_shl; lanes past the row end read 0).
template <int N>
__device__ inline float row_shl(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + N, 0xF, 0xF, false));
}

// +inf in a scalar register the compiler cannot see through.  With a literal
// +inf, fmed3(x, y, +inf) is folded to maxnum, which in IEEE mode costs a
// canonicalising v_max per operand; v_med3_f32 needs none.  The max of the
// score keys never sees a NaN (a query or codebook row that is not finite
// takes the exact path).
__device__ inline float opaque_inf() {
    float v;
    asm volatile("s_mov_b32 %0, 0x7f800000" : "=s"(v));
    return v;
}

// A wave-uniform value copied to a vector register by an instruction the
// compiler cannot rematerialise, so the copy is made once, outside the loop
// that reads it, and bit selects against it stay single v_bfi_b32.
__device__ inline int in_vgpr(int v) {
    int r;
    asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "s"(v));
    return r;
}

// gfx950 permlane swaps: {a, b} -> {lo, hi} where lo holds, in each pair of
// rows (16 lanes for permlane16, 32 for permlane32), the even row of a then
// the even row of b, and hi the odd row of a then the odd row of b.  Lane L of
// an even row therefore sees a(L) and a(L + row) and lane L of an odd row
// b(L - row) and b(L): the cross-row half of a butterfly in one VALU op.
__device__ inline void swap16(float a, float b, float &lo, float &hi) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    lo = __uint_as_float(s[0]);
    hi = __uint_as_float(s[1]);
}
__device__ inline void swap32(float a, float b, float &lo, float &hi) {
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    lo = __uint_as_float(s[0]);
    hi = __uint_as_float(s[1]);
}

template <int N>
__device__ inline float row_ror_max(float v, float pinf) {
    const int o = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + N, 0xF, 0xF, false);
    return __builtin_amdgcn_fmed3f(v, __int_as_float(o), pinf);
}
// Maximum over the wave, in every lane (NaN-free inputs).
__device__ inline float wave_max(float v, float pinf) {
    v = row_ror_max<8>(v, pinf);
    v = row_ror_max<4>(v, pinf);
    v = row_ror_max<2>(v, pinf);
    v = row_ror_max<1>(v, pinf);
    float lo, hi;
    swap16(v, v, lo, hi);
    v = __builtin_amdgcn_fmed3f(lo, hi, pinf);
    swap32(v, v, lo, hi);
    return __builtin_amdgcn_fmed3f(lo, hi, pinf);
}

// Per-stage image (units of float4), staged in LDS:
//   [0, 2*DI*64)           W_in : float4 (i*2 + q)*64 + L = W_in[4q .. 4q+3][64 i + L]
//   [.., + 2)              b_in[0..7]
//   [.., + 2*(N/64)*64)    c_hat: float4 (c*2 + q)*64 + L = c_hat[64 c + L][4q .. 4q+3]
// When W_in and c_hat do not fit in LDS together (large codebooks), only the
// prefix W_in + b_in is staged and c_hat is read from global memory (L2), in
// the same lane-major layout (coalesced 1 KB per wave load).
inline int64_t image_f4(int64_t D, int64_t N) { return 2 * D + 2 + 2 * N; }
inline int64_t image_prefix_f4(int64_t D) { return 2 * D + 2; }

// ggml's cosine score of code n (scalar leftovers of ggml_vec_dot_f32 with
// k = 8: each product rounded, then added in order).
__device__ inline float exact_score(const float4 a, const float4 b, const float *pn) {
    float sc = 0.0f;
    sc = __fadd_rn(sc, __fmul_rn(a.x, pn[0]));
    sc = __fadd_rn(sc, __fmul_rn(a.y, pn[1]));
    sc = __fadd_rn(sc, __fmul_rn(a.z, pn[2]));
    sc = __fadd_rn(sc, __fmul_rn(a.w, pn[3]));
    sc = __fadd_rn(sc, __fmul_rn(b.x, pn[4]));
    sc = __fadd_rn(sc, __fmul_rn(b.y, pn[5]));
    sc = __fadd_rn(sc, __fmul_rn(b.z, pn[6]));
    sc = __fadd_rn(sc, __fmul_rn(b.w, pn[7]));
    return sc;
}

// argmax over all N codes with ggml's arithmetic and tie rule
// (ggml_vec_argmax_f32: running max, index of the last element equal to it;
// a NaN score restarts the running max, replayed sequentially).
__device__ int exact_argmax(const float4 *chat, int N, const float *pn, int lane) {
    float bv = -INFINITY;
    int bn = 0;
    bool bad = false;
    const int NC = N / kWave;
#pragma unroll 1
    for (int c = 0; c < NC; ++c) {
        const float sc = exact_score(chat[(c * 2 + 0) * kWave + lane], chat[(c * 2 + 1) * kWave + lane], pn);
        bad |= (sc != sc);
        if (sc >= bv) {
            bv = sc;
            bn = c * kWave + lane;
        }
    }
#pragma unroll
    for (int off = 1; off <= 32; off <<= 1) {
        const float ov = __shfl_xor(bv, off);
        const int on = __shfl_xor(bn, off);
        if (ov > bv || (ov == bv && on > bn)) {
            bv = ov;
            bn = on;
        }
    }
    int code = uniform_i(bn);
    if (__any(bad)) {
        float mx = -INFINITY;
        int id = 0;
        for (int n = 0; n < N; ++n) {
            const float sc = exact_score(chat[((n / kWave) * 2 + 0) * kWave + (n % kWave)],
                                         chat[((n / kWave) * 2 + 1) * kWave + (n % kWave)], pn);
            mx = mx > sc ? mx : sc;
            if (mx == sc) id = n;
        }
        code = uniform_i(id);
    }
    return code;
}

// PF > 0: each thread keeps up to PF float4 of the next stage's image in
// registers (loaded while the current stage computes).  PF == 0: the image is
// copied in batches of kCopyBatch loads per thread at the stage start.
constexpr int kCopyBatch = 8;

typedef float f32x4 __attribute__((ext_vector_type(4)));   // native vector: stays in VGPRs

template <int PF>
__device__ inline void fetch_image(f32x4 (&pre)[PF > 0 ? PF : 1], const float4 *__restrict__ img, int64_t img_f4) {
    // img_f4: the float4 staged in LDS (a prefix of the stage image)
    const f32x4 *src = reinterpret_cast<const f32x4 *>(img);
#pragma unroll
    for (int k = 0; k < PF; ++k) {
        const int64_t t = threadIdx.x + static_cast<int64_t>(k) * blockDim.x;
        pre[k] = src[t < img_f4 ? t : img_f4 - 1];   // unconditional load keeps pre[] in registers
    }
}

// The tinyBLAS image's W_in: float4 ((j * 16 + t) * DI + sw(u4, t)) holds
// W_in[j][16 * (4 u4 + c) + t], c = 0..3 -- accumulator t of output j walks
// u = 0, 1, 2, ... in order.  The XOR swizzle keeps the 16 lanes of a row on
// distinct banks when DI is a power of two.
template <int DI>
__device__ __host__ inline int tb_sw(int u4, int t) {
    return (DI & (DI - 1)) == 0 ? (u4 ^ (t & (DI - 1))) : u4;
}

// In-projection of a wave's FW frames in one of ggml's summation orders:
// afterwards lane 16 g holds outputs 2 g and 2 g + 1 of each frame in wred.
// win: the stage's W_in in LDS (the order's layout); rt: the wave's D-float
// LDS area for the transposed frame (tinyBLAS order only).
template <int DI, int FW, int ORDER>
__device__ __forceinline__ void project_frames(const float (&r)[FW][DI], const float4 *win, float *rt, int lane,
                                               float (&wred)[FW][2]) {
    constexpr int D = DI * kWave;
    if (ORDER == 1) {
        // ---- in-projection, tinyBLAS order (sgemm.cpp:527-545: 16 FMA
        // accumulators over k = 16 u + t, then _mm512_reduce_add_ps) ----
        // Lane L = 16 g + t runs accumulator t of outputs 2g and 2g+1 over
        // the frame's elements k = 16 u + t, read from a transposed copy
        // of the residual in LDS (the cascade keeps k = L + 64 i per lane).
        const int t = lane & 15, g = lane >> 4;
        const float4 *w0 = win + (2 * g * 16 + t) * DI;
        const float4 *w1 = win + ((2 * g + 1) * 16 + t) * DI;
#pragma unroll
        for (int f = 0; f < FW; ++f) {
#pragma unroll
            for (int i = 0; i < DI; ++i) rt[t * (D / 16) + tb_sw<DI>(i, t) * 4 + g] = r[f][i];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
            for (int u4 = 0; u4 < DI; ++u4) {
                const int sw = tb_sw<DI>(u4, t);
                const float4 rv = *reinterpret_cast<const float4 *>(rt + t * (D / 16) + sw * 4);
                const float4 x0 = w0[sw], x1 = w1[sw];
                a0 = __fmaf_rn(x0.x, rv.x, a0);
                a0 = __fmaf_rn(x0.y, rv.y, a0);
                a0 = __fmaf_rn(x0.z, rv.z, a0);
                a0 = __fmaf_rn(x0.w, rv.w, a0);
                a1 = __fmaf_rn(x1.x, rv.x, a1);
                a1 = __fmaf_rn(x1.y, rv.y, a1);
                a1 = __fmaf_rn(x1.z, rv.z, a1);
                a1 = __fmaf_rn(x1.w, rv.w, a1);
            }
            a0 = row_ror_add<8>(a0);
            a0 = row_ror_add<4>(a0);
            a0 = row_ror_add<2>(a0);
            a0 = row_ror_add<1>(a0);
            a1 = row_ror_add<8>(a1);
            a1 = row_ror_add<4>(a1);
            a1 = row_ror_add<2>(a1);
            a1 = row_ror_add<1>(a1);
            wred[f][0] = a0;
            wred[f][1] = a1;
            // the next frame overwrites rt
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    } else {
        // ---- in-projection: one FMA chain per lane and output, ggml order ----
        float acc[FW][8];
#pragma unroll
        for (int f = 0; f < FW; ++f)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[f][j] = 0.0f;
        // Weights are loaded one step ahead.
        float4 wa = win[lane];
        float4 wb = win[kWave + lane];
#pragma unroll
        for (int i = 0; i < DI; ++i) {
            float4 na = wa, nb = wb;
            if (i + 1 < DI) {
                na = win[((i + 1) * 2 + 0) * kWave + lane];
                nb = win[((i + 1) * 2 + 1) * kWave + lane];
            }
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
            wa = na;
            wb = nb;
            // Pin this step's accumulators here: otherwise LLVM sinks the
            // later frames' FMA chains below the first frame's reduction and
            // keeps every step's weights live.
#pragma unroll
            for (int f = 0; f < FW; ++f)
#pragma unroll
                for (int j = 0; j < 8; ++j) __asm__ volatile("" : "+v"(acc[f][j]));
        }
        // Reduction = GGML_F32x16_REDUCE (0+=2, 1+=3, 0+=1) then
        // _mm512_reduce_add_ps (distances 8, 4, 2, 1), transposed: after the
        // two cross-row levels lane L holds outputs 2*(L/16) and 2*(L/16)+1.
        // Each level is one permlane swap: lanes 0-31 add acc[q] of lanes L
        // and L + 32, lanes 32-63 acc[q + 4] of lanes L - 32 and L; then
        // rows 0 and 2 add v[q] of lanes L and L + 16, rows 1 and 3 v[q + 2]
        // of lanes L - 16 and L.
#pragma unroll
        for (int f = 0; f < FW; ++f) {
            float v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float lo, hi;
                swap32(acc[f][q], acc[f][q + 4], lo, hi);
                v[q] = __fadd_rn(lo, hi);
            }
            float w[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                float lo, hi;
                swap16(v[q], v[q + 2], lo, hi);
                w[q] = __fadd_rn(lo, hi);
            }
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                w[q] = row_ror_add<8>(w[q]);
                w[q] = row_ror_add<4>(w[q]);
                w[q] = row_ror_add<2>(w[q]);
                w[q] = row_ror_add<1>(w[q]);
            }
            wred[f][0] = w[0];
            wred[f][1] = w[1];
        }
    }
}

// The stage's queries, normalised as l2_normalize_last does, for all FW
// frames of a wave at once: lane 8 f + o returns output o of frame f (lanes
// 8 FW .. 63 carry don't-care values).  bias: b_in[lane & 7] when has_bin.
template <int FW>
__device__ __forceinline__ float normalise_queries(const float (&wred)[FW][2], int lane, bool has_bin, float bias,
                                                   float qeps) {
    // Output o of frame f moves to lane 8 f + o: in row g, lane 16 g + j
    // (j < 2 FW) offers wred[j / 2][j % 2], i.e. output 2 g + j % 2 of
    // frame j / 2.  Lanes 8 FW .. 63 carry don't-care values.
    const int jrow = lane & 15;
    float offer = wred[0][0];
#pragma unroll
    for (int f = 0; f < FW; ++f) {
        if (jrow == 2 * f) offer = wred[f][0];
        if (jrow == 2 * f + 1) offer = wred[f][1];
    }
    const int ol = lane & 7;
    float p = __shfl(offer, 16 * (ol >> 1) + 2 * (lane >> 3) + (ol & 1));
    if (has_bin) p = __fadd_rn(p, bias);
    // l2_normalize_last: fp32 squares, double row sum in output order,
    // + eps, sqrt, divide.  Lane 8 f sums ((sq_0 + sq_1) + sq_2) + ... of
    // frame f, reading sq_k from lane 8 f + k (the leading 0.0 + sq_0 of
    // the reference is sq_0 exactly: a square is +0 or more, or NaN).
    const float sq = __fmul_rn(p, p);
    double ss = static_cast<double>(sq);
    ss += static_cast<double>(row_shl<1>(sq));
    ss += static_cast<double>(row_shl<2>(sq));
    ss += static_cast<double>(row_shl<3>(sq));
    ss += static_cast<double>(row_shl<4>(sq));
    ss += static_cast<double>(row_shl<5>(sq));
    ss += static_cast<double>(row_shl<6>(sq));
    ss += static_cast<double>(row_shl<7>(sq));
    // ggml_scale_bias(sum, 1, eps): 1e-12 (Fish), 1e-20 (Vevo2), none
    // (IndexTTS2: qeps = 0, and sum + 0 == sum for a sum >= +0)
    const float den8 = sqrt_rn(__fadd_rn(static_cast<float>(ss), qeps));
    return __fdiv_rn(p, __shfl(den8, lane & ~7));
}

// Frame f's normalised query in scalar registers (pn[f][o] from lane 8 f + o)
// and whether all of its outputs are finite.
template <int FW>
__device__ __forceinline__ void query_scalars(float qv, float (&pn)[FW][8], bool (&finite)[FW]) {
    const uint64_t good = __ballot((qv - qv) == 0.0f);
#pragma unroll
    for (int f = 0; f < FW; ++f) {
        finite[f] = ((good >> (8 * f)) & 0xffull) == 0xffull;
#pragma unroll
        for (int o = 0; o < 8; ++o) pn[f][o] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qv), 8 * f + o));
    }
}

// The wave's frames: residual rows into registers (rc: -0, or the recon
// rows that this cascade adds to), and out again at the end.
template <int DI, int FW, bool RECON>
__device__ __forceinline__ void load_frames(const float *__restrict__ x, int64_t M, int64_t m_first, int lane,
                                            const float *__restrict__ recon, int recon_acc, int64_t (&mrow)[FW],
                                            bool (&active)[FW], float (&r)[FW][DI], float (&rc)[FW][DI]) {
    constexpr int D = DI * kWave;
#pragma unroll
    for (int f = 0; f < FW; ++f) {
        active[f] = (m_first + f) < M;
        mrow[f] = active[f] ? (m_first + f) : (M - 1);
#pragma unroll
        for (int i = 0; i < DI; ++i) {
            r[f][i] = x[mrow[f] * D + i * kWave + lane];
            rc[f][i] = -0.0f;   // -0 + z == z exactly, for every z
            if (RECON && recon_acc) rc[f][i] = recon[mrow[f] * D + i * kWave + lane];
        }
    }
}

template <int DI, int FW, bool RECON>
__device__ __forceinline__ void store_frames(const int64_t (&mrow)[FW], const bool (&active)[FW], int lane,
                                             const float (&r)[FW][DI], const float (&rc)[FW][DI],
                                             float *__restrict__ residual, float *__restrict__ recon) {
    constexpr int D = DI * kWave;
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

// Codes out, then the out-projection by table gather and the residual update
// of a wave's FW frames at stage s (force_idx: teacher forcing, checked).
template <int DI, int FW, bool RECON>
__device__ __forceinline__ void apply_codes(const int (&code)[FW], int s, int N, const int64_t (&mrow)[FW],
                                            const bool (&active)[FW], int lane, int ld, int32_t *__restrict__ idx,
                                            const int32_t *__restrict__ force_idx, int32_t *__restrict__ flags,
                                            const float *__restrict__ tables, float (&r)[FW][DI], float (&rc)[FW][DI]) {
    constexpr int D = DI * kWave;
    int use[FW];
#pragma unroll
    for (int f = 0; f < FW; ++f) {
        if (lane == 0 && active[f]) idx[mrow[f] * ld + s] = code[f];
        use[f] = code[f];
        if (force_idx) {
            use[f] = force_idx[mrow[f] * ld + s];
            if (use[f] < 0 || use[f] >= N) {
                if (lane == 0) flags[AQ_FLAG_BAD_INDEX] = 1;
                use[f] = 0;
            }
        }
    }
    if (tables) {   // (codes only: no out-projection was uploaded)
        // Every row load of the wave's frames is issued before the first
        // use, so the gathers overlap instead of waiting one by one.
        float z[FW][DI];
#pragma unroll
        for (int f = 0; f < FW; ++f) {
            const float *zrow = tables + (static_cast<int64_t>(s) * N + use[f]) * D;
#pragma unroll
            for (int i = 0; i < DI; ++i) z[f][i] = zrow[i * kWave + lane];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int f = 0; f < FW; ++f)
#pragma unroll
            for (int i = 0; i < DI; ++i) {
                r[f][i] = __fsub_rn(r[f][i], z[f][i]);
                if (RECON) rc[f][i] = __fadd_rn(rc[f][i], z[f][i]);
            }
    }
}

template <int DI, int FW, bool RECON, int PF, bool CBG, int ORDER>
__global__ __launch_bounds__(kMaxBlock, 1) void dac_encode_kernel(
    const float *__restrict__ x, int64_t M, int Q, int N, const float4 *__restrict__ images, int64_t stride_f4,
    int64_t img_f4, const float *__restrict__ tables, int32_t *__restrict__ idx, float *__restrict__ residual,
    float *__restrict__ recon, const int32_t *__restrict__ force_idx, int32_t *__restrict__ flags, int has_bin,
    int key_bits, float margin, int exact_only, float qeps, int64_t dbuf_f4, int ld, int recon_acc) {
    // ld: row stride of idx and force_idx; recon_acc: recon holds the sum of
    // earlier stages' z (another stage set's), which this cascade adds to.
    // stride_f4: float4 per stage image; img_f4: the prefix staged in LDS
    // (the whole image, or W_in + b_in when CBG reads c_hat from memory).
    extern __shared__ float4 lds[];
    constexpr int D = DI * kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int waves_per_block = blockDim.x / kWave;
    const int64_t m_first = (static_cast<int64_t>(blockIdx.x) * waves_per_block + wave) * FW;

    int64_t mrow[FW];
    bool active[FW];
    float r[FW][DI];
    float rc[FW][DI];
    load_frames<DI, FW, RECON>(x, M, m_first, lane, recon, recon_acc, mrow, active, r, rc);

    const int NC = N / kWave;
    const int key_mask = (1 << key_bits) - 1;

    f32x4 pre[PF > 0 ? PF : 1];
    if (PF > 0) fetch_image<PF>(pre, images, img_f4);

    for (int s = 0; s < Q; ++s) {
        // dbuf_f4 > 0: two LDS images, stage s in the one at (s & 1) * dbuf_f4.
        // The image written here was last read two stages ago, and every wave
        // has finished that stage once it passed the previous stage's barrier,
        // so one barrier per stage suffices.
        float4 *img_lds = lds + ((s & 1) ? dbuf_f4 : 0);
        if (dbuf_f4 == 0) __syncthreads();
        if (PF > 0) {
            f32x4 *lds4 = reinterpret_cast<f32x4 *>(img_lds);
#pragma unroll
            for (int k = 0; k < PF; ++k) {
                const int64_t t = threadIdx.x + static_cast<int64_t>(k) * blockDim.x;
                if (t < img_f4) lds4[t] = pre[k];
            }
        } else {
            const float4 *img = images + static_cast<int64_t>(s) * stride_f4;
            for (int64_t t0 = 0; t0 < img_f4; t0 += static_cast<int64_t>(kCopyBatch) * blockDim.x) {
                float4 buf[kCopyBatch];
#pragma unroll
                for (int k = 0; k < kCopyBatch; ++k) {
                    const int64_t t = t0 + threadIdx.x + static_cast<int64_t>(k) * blockDim.x;
                    buf[k] = img[t < img_f4 ? t : img_f4 - 1];
                }
#pragma unroll
                for (int k = 0; k < kCopyBatch; ++k) {
                    const int64_t t = t0 + threadIdx.x + static_cast<int64_t>(k) * blockDim.x;
                    if (t < img_f4) img_lds[t] = buf[k];
                }
            }
        }
        __syncthreads();
        if (PF > 0 && s + 1 < Q) fetch_image<PF>(pre, images + static_cast<int64_t>(s + 1) * stride_f4, img_f4);
        const float4 *win = img_lds;
        const float *bin = reinterpret_cast<const float *>(img_lds + 2 * DI * kWave);
        const float4 *chat = CBG ? images + static_cast<int64_t>(s) * stride_f4 + 2 * DI * kWave + 2
                                 : img_lds + 2 * DI * kWave + 2;

        float wred[FW][2];   // lane 16 g holds outputs 2 g and 2 g + 1 of each frame
        project_frames<DI, FW, ORDER>(r, win, ORDER == 1 ? reinterpret_cast<float *>(lds + img_f4 + dbuf_f4) + wave * D : nullptr,
                                      lane, wred);
        // ---- query normalisation, every frame of the wave at once ----
        const float qv = normalise_queries<FW>(wred, lane, has_bin != 0, has_bin ? bin[lane & 7] : 0.0f, qeps);
        float pn[FW][8];
        bool finite[FW];
        query_scalars<FW>(qv, pn, finite);
        // ---- approximate scores, two best keys per lane ----
        const float pinf = opaque_inf();
        const int vmask = in_vgpr(key_mask);
        float k1[FW], k2[FW];
#pragma unroll
        for (int f = 0; f < FW; ++f) {
            k1[f] = -INFINITY;
            k2[f] = -INFINITY;
        }
#pragma unroll 2
        for (int c = 0; c < NC; ++c) {
            const float4 a = chat[(c * 2 + 0) * kWave + lane];
            const float4 b = chat[(c * 2 + 1) * kWave + lane];
#pragma unroll
            for (int f = 0; f < FW; ++f) {
                float sc = a.x * pn[f][0];
                sc = __fmaf_rn(a.y, pn[f][1], sc);
                sc = __fmaf_rn(a.z, pn[f][2], sc);
                sc = __fmaf_rn(a.w, pn[f][3], sc);
                sc = __fmaf_rn(b.x, pn[f][4], sc);
                sc = __fmaf_rn(b.y, pn[f][5], sc);
                sc = __fmaf_rn(b.z, pn[f][6], sc);
                sc = __fmaf_rn(b.w, pn[f][7], sc);
                const float key = __int_as_float((__float_as_int(sc) & ~vmask) | (c & vmask));
                k2[f] = __builtin_amdgcn_fmed3f(k1[f], k2[f], key);
                k1[f] = __builtin_amdgcn_fmed3f(k1[f], key, pinf);
            }
        }
        int code[FW];
#pragma unroll
        for (int f = 0; f < FW; ++f) {
            const float best = wave_max(k1[f], pinf);
            const bool mine = k1[f] == best;
            const uint64_t owners = __ballot(mine);
            const float second = wave_max(mine ? k2[f] : k1[f], pinf);
            const bool pass = finite[f] && !exact_only && __popcll(owners) == 1 && (best - second) > margin;
            if (pass) {
                const int owner = __ffsll(static_cast<unsigned long long>(owners)) - 1;
                code[f] = uniform_i(((__float_as_int(best) & key_mask) * kWave) + owner);
            } else {
                code[f] = exact_argmax(chat, N, pn[f], lane);
            }
        }

        apply_codes<DI, FW, RECON>(code, s, N, mrow, active, lane, ld, idx, force_idx, flags, tables, r, rc);
    }

    store_frames<DI, FW, RECON>(mrow, active, lane, r, rc, residual, recon);
}

// ------------------------------------------------ scores on matrix cores
// A variant of dac_encode_kernel for blocks of 8 waves x 3 frames, N a
// multiple of 128 up to 1024 and D up to 1024.  The in-projection, the query
// normalisation, the exact rescoring and the out-projection are the same;
// the approximate scores run on fp16 matrix cores over the block's 24 frames:
//  * Codes and queries are scaled by 2^12 and split into fp16 pairs
//    (hi = fp16(v), lo = fp16(v - hi)), so one v_mfma_f32_16x16x32_f16 with
//    k-slices (c_hi, c_lo, c_hi, c_lo) x (q_hi, q_hi, q_lo, q_lo) gives
//    2^24 c.q for 16 codes x 16 frames.  The scaling keeps every operand that
//    matters out of fp16's subnormal range.
//  * Wave w scores codes [w N/8, (w+1) N/8) for all 24 frames (two 16-frame
//    column tiles; frames 24-31 are zero) and keeps two keys per lane and
//    frame; keys carry the code's index inside the wave's range.  The four
//    lanes of a frame merge theirs by lane swaps, the block's eight waves
//    through LDS.
//  * The certificate bound covers the split (2^-22 relative per operand), the
//    matrix core's fp32 accumulation of 32 products (taken as 2u per add),
//    the fp16 flush of operands below 2^-14 (2^-26 after scaling back),
//    ggml's own rounding and the key truncation.
// Stage images hold W_in, b_in, c_hat and the split codebook (c16); each
// part has one LDS copy, rewritten at a point where every wave has finished
// reading it and made visible by the next barrier:
//   W_in(s+1)  after barrier B_s (in-projections done), read after C_s
//   c_hat(s)   after B_s (stage s - 1's selects done), read after C_s
//   c16(s+1)   after C_s (scores done), read after B_{s+1}
// with B_s after the queries are written and C_s after the keys are.
constexpr int kMsWaves = 8;
constexpr int kMsFw = 3;
constexpr int kMsFrames = kMsWaves * kMsFw;   // frames per block (<= 32)
constexpr int kMsPart = 4;                    // float4 per thread of each image part
constexpr float kMsScale = 4096.0f;           // 2^12 before the fp16 split

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// c16 region of a stage image: code n, part h (0 hi, 1 lo) at float4
// (n / 16) * 32 + h * 16 + n % 16 (16 codes' parts contiguous: the MFMA
// operand reads of a row of lanes are conflict-free).
__host__ __device__ inline int64_t c16_at(int64_t n, int h) { return (n >> 4) * 32 + h * 16 + (n & 15); }

template <int CTRL>
__device__ inline float dpp_max(float v, float pinf) {
    const int o = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false);
    return __builtin_amdgcn_fmed3f(v, __int_as_float(o), pinf);
}
// Maximum over each group of 8 lanes (xor 1, xor 2, half-row mirror).
__device__ inline float max8(float v, float pinf) {
    v = dpp_max<0xB1>(v, pinf);
    v = dpp_max<0x4E>(v, pinf);
    return dpp_max<0x141>(v, pinf);
}
// Two best keys of a lane pair given as {own, partner} (swap16 / swap32
// results): best = max, second = the larger of the other best and the
// better second.
__device__ inline void merge_top2(float lo1, float hi1, float lo2, float hi2, float pinf, float &k1, float &k2) {
    k1 = __builtin_amdgcn_fmed3f(lo1, hi1, pinf);
    k2 = __builtin_amdgcn_fmed3f(lo1, hi1, __builtin_amdgcn_fmed3f(lo2, hi2, pinf));
}

template <int DI, bool RECON, int ORDER>
__global__ __launch_bounds__(kMsWaves * kWave, 1) void dac_encode_ms_kernel(
    const float *__restrict__ x, int64_t M, int Q, int N, const float4 *__restrict__ images, int64_t stride_f4,
    const float *__restrict__ tables, int32_t *__restrict__ idx, float *__restrict__ residual,
    float *__restrict__ recon, const int32_t *__restrict__ force_idx, int32_t *__restrict__ flags, int has_bin,
    int key_bits, float margin, int exact_only, float qeps, int ld, int recon_acc) {
    // margin: in units of the scaled scores (2^24 c.q); key_bits: bits of a
    // code's index inside a wave's range of N / 8 codes.
    extern __shared__ float4 lds[];
    constexpr int FW = kMsFw;
    constexpr int D = DI * kWave;
    constexpr int kThreads = kMsWaves * kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int64_t m_first = (static_cast<int64_t>(blockIdx.x) * kMsWaves + wave) * FW;
    const int n2 = 2 * N;                    // float4 of c_hat, and of c16
    const int64_t ch_off = 2 * D + 2;        // c_hat in the stage image (after W_in, b_in)
    const int64_t c16_off = ch_off + n2;
    float4 *w_lds = lds;                     // [2D]
    float4 *ch_lds = lds + 2 * D;            // [2N]
    float4 *c16_lds = ch_lds + n2;           // [2N]
    float4 *qb = c16_lds + n2;               // [32 frames][hi, lo] of fp16 x 8
    float2 *kb = reinterpret_cast<float2 *>(qb + 64);   // [8 waves][32 frames] two keys
    float *rt = reinterpret_cast<float *>(qb + 64 + kMsWaves * 16) + wave * D;   // tinyBLAS order only

    int64_t mrow[FW];
    bool active[FW];
    float r[FW][DI];
    float rc[FW][DI];
    load_frames<DI, FW, RECON>(x, M, m_first, lane, recon, recon_acc, mrow, active, r, rc);
    if (threadIdx.x < (32 - kMsFrames) * 2) qb[kMsFrames * 2 + threadIdx.x] = float4{0.0f, 0.0f, 0.0f, 0.0f};

    f32x4 pw[kMsPart], pch[kMsPart], pc16[kMsPart];
    auto fetch = [&](f32x4 (&dst)[kMsPart], const float4 *src, int cnt) {
        const f32x4 *v = reinterpret_cast<const f32x4 *>(src);
#pragma unroll
        for (int k = 0; k < kMsPart; ++k) {
            const int t = static_cast<int>(threadIdx.x) + k * kThreads;
            dst[k] = v[t < cnt ? t : cnt - 1];
        }
    };
    auto put = [&](float4 *dst, const f32x4 (&src)[kMsPart], int cnt) {
        f32x4 *v = reinterpret_cast<f32x4 *>(dst);
#pragma unroll
        for (int k = 0; k < kMsPart; ++k) {
            const int t = static_cast<int>(threadIdx.x) + k * kThreads;
            if (t < cnt) v[t] = src[k];
        }
    };
    auto image = [&](int s) { return images + static_cast<int64_t>(s) * stride_f4; };
    fetch(pw, image(0), 2 * D);
    fetch(pch, image(0) + ch_off, n2);
    fetch(pc16, image(0) + c16_off, n2);
    put(w_lds, pw, 2 * D);
    put(c16_lds, pc16, n2);
    if (Q > 1) {
        fetch(pw, image(1), 2 * D);
        fetch(pc16, image(1) + c16_off, n2);
    }
    __syncthreads();

    const int cpw = N / kMsWaves;            // codes per wave, a multiple of 16
    const int key_mask = (1 << key_bits) - 1;
    const int g = lane >> 4, j = lane & 15;
    for (int s = 0; s < Q; ++s) {
        const float bias = has_bin ? reinterpret_cast<const float *>(image(s) + 2 * D)[lane & 7] : 0.0f;
        float wred[FW][2];
        project_frames<DI, FW, ORDER>(r, w_lds, rt, lane, wred);
        const float qv = normalise_queries<FW>(wred, lane, has_bin != 0, bias, qeps);
        // The wave's queries into the block's B operands.
        if (lane < 8 * FW) {
            const float qs = qv * kMsScale;
            const _Float16 hi = static_cast<_Float16>(qs);
            const _Float16 lo = static_cast<_Float16>(qs - static_cast<float>(hi));
            _Float16 *qh = reinterpret_cast<_Float16 *>(qb) + (wave * FW + (lane >> 3)) * 16 + (lane & 7);
            qh[0] = hi;
            qh[8] = lo;
        }
        __syncthreads();   // B_s

        // ---- scores of this wave's codes for the block's frames ----
        const float pinf = opaque_inf();
        const int vmask = in_vgpr(key_mask);
        float k1[2] = {-INFINITY, -INFINITY}, k2[2] = {-INFINITY, -INFINITY};
        {
            const f16x8 bq0 = *reinterpret_cast<const f16x8 *>(qb + j * 2 + (g >> 1));
            const f16x8 bq1 = *reinterpret_cast<const f16x8 *>(qb + (16 + j) * 2 + (g >> 1));
            const f16x8 *ca = reinterpret_cast<const f16x8 *>(c16_lds) + c16_at(static_cast<int64_t>(wave) * cpw + j, g & 1);
            const int lane_id = in_vgpr(0) + 4 * g;   // rows 4 g + i of each 16-code tile
            const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 2
            for (int t = 0; t < cpw / 16; ++t) {
                const f16x8 a = ca[t * 32];
                const f32x4 s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq0, zero, 0, 0, 0);
                const f32x4 s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq1, zero, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int id = lane_id + (t * 16 + i);
                    const float key0 = __int_as_float((__float_as_int(s0[i]) & ~vmask) | id);
                    k2[0] = __builtin_amdgcn_fmed3f(k1[0], k2[0], key0);
                    k1[0] = __builtin_amdgcn_fmed3f(k1[0], key0, pinf);
                    const float key1 = __int_as_float((__float_as_int(s1[i]) & ~vmask) | id);
                    k2[1] = __builtin_amdgcn_fmed3f(k1[1], k2[1], key1);
                    k1[1] = __builtin_amdgcn_fmed3f(k1[1], key1, pinf);
                }
            }
        }
        // the four lanes of a frame (16 apart), then the block's waves
#pragma unroll
        for (int ft = 0; ft < 2; ++ft) {
            float lo1, hi1, lo2, hi2;
            swap16(k1[ft], k1[ft], lo1, hi1);
            swap16(k2[ft], k2[ft], lo2, hi2);
            merge_top2(lo1, hi1, lo2, hi2, pinf, k1[ft], k2[ft]);
            swap32(k1[ft], k1[ft], lo1, hi1);
            swap32(k2[ft], k2[ft], lo2, hi2);
            merge_top2(lo1, hi1, lo2, hi2, pinf, k1[ft], k2[ft]);
        }
        // W_in(s+1) and c_hat(s), stored after the scores so that their
        // operand reads do not queue behind these stores
        if (s + 1 < Q) {
            put(w_lds, pw, 2 * D);
            if (s + 2 < Q) fetch(pw, image(s + 2), 2 * D);
        }
        put(ch_lds, pch, n2);
        if (s + 1 < Q) fetch(pch, image(s + 1) + ch_off, n2);
        if (g == 0) kb[wave * 32 + j] = float2{k1[0], k2[0]};
        if (g == 1 && 16 + j < kMsFrames) kb[wave * 32 + 16 + j] = float2{k1[1], k2[1]};
        __syncthreads();   // C_s
        if (s + 1 < Q) {
            put(c16_lds, pc16, n2);
            if (s + 2 < Q) fetch(pc16, image(s + 2) + c16_off, n2);
        }

        // ---- this wave's frames: lane 8 f + w reads wave w's keys ----
        const int fl = lane >> 3;
        float a1 = -INFINITY, a2 = -INFINITY;
        if (fl < FW) {
            const float2 kv = kb[(lane & 7) * 32 + wave * FW + fl];
            a1 = kv.x;
            a2 = kv.y;
        }
        const float best8 = max8(a1, pinf);
        const bool mine = a1 == best8;
        const uint64_t owners = __ballot(mine);
        const float second8 = max8(mine ? a2 : a1, pinf);
        const uint64_t good = __ballot((qv - qv) == 0.0f);
        int code[FW];
#pragma unroll
        for (int f = 0; f < FW; ++f) {
            const unsigned grp = static_cast<unsigned>(owners >> (8 * f)) & 0xffu;
            const float best = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(best8), 8 * f));
            const float second = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(second8), 8 * f));
            const bool finite = ((good >> (8 * f)) & 0xffull) == 0xffull;
            const bool pass = finite && !exact_only && __popc(grp) == 1 && (best - second) > margin;
            if (pass) {
                code[f] = (__ffs(grp) - 1) * cpw + (__float_as_int(best) & key_mask);
            } else {
                // the query in scalar registers, for the exact rescoring only
                float pn[8];
#pragma unroll
                for (int o = 0; o < 8; ++o) pn[o] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qv), 8 * f + o));
                code[f] = exact_argmax(ch_lds, N, pn, lane);
            }
        }
        apply_codes<DI, FW, RECON>(code, s, N, mrow, active, lane, ld, idx, force_idx, flags, tables, r, rc);
    }
    store_frames<DI, FW, RECON>(mrow, active, lane, r, rc, residual, recon);
}

// Stage images of the cosine quantizer, built on the device at upload.
// W_in [Q][8][D] goes to both images: the vec_dot order's layout (element
// (r, d) at ((d/64 * 2 + r/4) * 64 + d%64) * 4 + r%4) and the tinyBLAS
// order's (row r, d = 16 * (4 * u4 + c) + t at ((r * 16 + t) * DI + sw) * 4
// + c, DI = D / 64, sw = u4 ^ (t & (DI - 1)) for a power-of-two DI).
__global__ void dac_image_win_kernel(const float *__restrict__ w_in, int64_t Q, int64_t D, int64_t img_f,
                                     float *__restrict__ images, float *__restrict__ images_tb) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= Q * 8 * D) return;
    const int64_t s = t / (8 * D), e = t % (8 * D);
    const int r = static_cast<int>(e / D);
    const int64_t d = e % D;
    const float w = w_in[t];
    images[s * img_f + ((d / kWave * 2 + r / 4) * kWave + d % kWave) * 4 + r % 4] = w;
    const int64_t DI = D / kWave;
    const int64_t tt = d % 16, u4 = (d / 16) / 4, c = (d / 16) % 4;
    const int64_t sw = (DI & (DI - 1)) == 0 ? (u4 ^ (tt & (DI - 1))) : u4;
    images_tb[s * img_f + ((r * 16 + tt) * DI + sw) * 4 + c] = w;
}

// The recipe's inverse norm of codebook row C (8 floats; t: the row's index
// over all stages, reported in flags[0] for a zero Vevo2 row).
__device__ inline float dac_row_inv(const float *__restrict__ C, int recipe, int64_t t,
                                    unsigned long long *__restrict__ flags) {
    double sum = 0.0;
    for (int k = 0; k < 8; ++k) sum = __dadd_rn(sum, __dmul_rn(static_cast<double>(C[k]), static_cast<double>(C[k])));
    if (recipe == AQ_DAC_INDEXTTS2) return __fdiv_rn(1.0f, static_cast<float>(sqrt_rn(sum)));
    if (recipe == AQ_DAC_VEVO2) {
        const double norm = sqrt_rn(sum);
        if (norm == 0.0) atomicMin(&flags[0], static_cast<unsigned long long>(t));
        return static_cast<float>(__ddiv_rn(1.0, norm));
    }
    return sum > 0.0 ? static_cast<float>(__ddiv_rn(1.0, sqrt_rn(sum))) : 0.0f;
}

// b_in and the recipe's normalised codebook rows, the same in both images
// (all recipes: double sum of squares, float products):
//   Fish      inv = sum > 0 ? (float)(1 / sqrt(sum)) : 0   (fish_audio/codec.cpp:171-189)
//   IndexTTS2 inv = 1.0F / (float)sqrt(sum)               (index_tts2/semantic_codec.cpp:43-58)
//   Vevo2     inv = (float)(1 / sqrt(sum)), a zero row is an error (vevo2/components.cpp:566-590)
// Code n's element 4q + t sits at ((n/64 * 2 + q) * 64 + n%64) * 4 + t after
// the 2D + 2 float4 of W_in and b_in.  flags[0]: lowest s * N + n of a zero
// Vevo2 row (atomicMin); flags[1] = 1 on a non-finite normalised entry.
__global__ void dac_image_cb_kernel(const float *__restrict__ codebook, const float *__restrict__ b_in, int64_t Q,
                                    int64_t N, int64_t D, int64_t img_f, int recipe, float *__restrict__ images,
                                    float *__restrict__ images_tb, unsigned long long *__restrict__ flags) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t < Q * 8) {
        const int64_t s = t / 8;
        const float b = b_in ? b_in[t] : 0.0f;
        images[s * img_f + 8 * D + t % 8] = b;
        images_tb[s * img_f + 8 * D + t % 8] = b;
    }
    if (t >= Q * N) return;
    const int64_t s = t / N, n = t % N;
    const float *C = codebook + t * 8;
    const float inv = dac_row_inv(C, recipe, t, flags);
    const int64_t base = s * img_f + 8 * D + 8, c = n / kWave, L = n % kWave;
    bool nf = false;
    for (int q = 0; q < 2; ++q)
        for (int k = 0; k < 4; ++k) {
            const float v = __fmul_rn(C[4 * q + k], inv);
            nf |= !__builtin_isfinite(v);
            images[base + ((c * 2 + q) * kWave + L) * 4 + k] = v;
            images_tb[base + ((c * 2 + q) * kWave + L) * 4 + k] = v;
        }
    if (nf) flags[1] = 1;
}

// The split codebook of each stage image (after c_hat, read from it): code
// n's normalised row scaled by 2^12, as fp16 hi = fp16(v) and lo =
// fp16(v - hi), at c16_at(n, 0) and c16_at(n, 1); the same in both images.
__global__ void dac_image_c16_kernel(int64_t Q, int64_t N, int64_t D, int64_t img_f, float *__restrict__ images,
                                     float *__restrict__ images_tb) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= Q * N) return;
    const int64_t s = t / N, n = t % N, c = n / kWave, L = n % kWave;
    const int64_t chat = s * img_f + 8 * D + 8;
    const int64_t c16 = (chat + 8 * N) * 2;   // in halves
    for (int q = 0; q < 2; ++q)
        for (int k = 0; k < 4; ++k) {
            const float v = images[chat + ((c * 2 + q) * kWave + L) * 4 + k] * kMsScale;
            const _Float16 hi = static_cast<_Float16>(v);
            const _Float16 lo = static_cast<_Float16>(v - static_cast<float>(hi));
            for (float *img : {images, images_tb}) {
                _Float16 *h = reinterpret_cast<_Float16 *>(img) + c16;
                h[c16_at(n, 0) * 8 + 4 * q + k] = hi;
                h[c16_at(n, 1) * 8 + 4 * q + k] = lo;
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
// (accumulate: out already holds the sum of earlier stages, which the z of
// these stages are added to in order.)
__global__ void dac_decode_kernel(const int32_t *__restrict__ idx, int64_t ld, int64_t M, int Q, int64_t N, int64_t D,
                                  const float *__restrict__ tables, float *__restrict__ out,
                                  int32_t *__restrict__ flags, int accumulate) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= M * D) return;
    const int64_t m = t / D;
    const int64_t d = t % D;
    float acc = accumulate ? out[t] : 0.0f;
    for (int s = 0; s < Q; ++s) {
        int32_t code = idx[m * ld + s];
        if (code < 0 || code >= N) {
            flags[AQ_FLAG_BAD_INDEX] = 1;
            code = 0;
        }
        const float z = tables[(static_cast<int64_t>(s) * N + code) * D + d];
        acc = (s == 0 && !accumulate) ? z : __fadd_rn(acc, z);
    }
    out[t] = acc;
}

// ----------------------------------------------------------- any shape
// Latent widths D and codebook sizes N outside the fused kernel's (D in
// {64, ..., 1024} by its register tiles, N a multiple of 64) take a cascade
// kernel with run-time D and N and the same ggml arithmetic, at the cost of
// rescoring every code exactly (no certificate) and of a residual in LDS.

// Plain normalised codebook rows [Q][N][8] of the recipe.
__global__ void dac_any_chat_kernel(const float *__restrict__ codebook, int64_t QN, int recipe, float *__restrict__ chat,
                                    unsigned long long *__restrict__ flags) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= QN) return;
    const float *C = codebook + t * 8;
    const float inv = dac_row_inv(C, recipe, t, flags);
    bool nf = false;
    for (int k = 0; k < 8; ++k) {
        const float v = __fmul_rn(C[k], inv);
        nf |= !__builtin_isfinite(v);
        chat[t * 8 + k] = v;
    }
    if (nf) flags[1] = 1;
}

struct DacAnyArgs {
    const float *x;          // [M, D] frame-major
    int64_t M;
    int D, N, Q;
    const float *w_in;       // [Q][8][D]
    const float *b_in;       // [Q][8] or null
    const float *chat;       // [Q][N][8] normalised codes
    const float *tables;     // [Q][N][D] out-projection (+ bias) per code, or null (codes only)
    int32_t *idx;            // [M, ld]
    int ld;
    float *residual;         // [M, D] or null
    float *recon;            // [M, D] or null
    int recon_acc;
    const int32_t *force_idx;
    int32_t *flags;
    float qeps;
    int order;               // 0 ggml_vec_dot_f32, 1 tinyBLAS
};

// Orders this wave's LDS stores before its other lanes' loads.
__device__ inline void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One wave per frame; its residual row (D floats) in LDS for all stages.
__global__ __launch_bounds__(256) void dac_any_kernel(DacAnyArgs a) {
    extern __shared__ float any_lds[];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int64_t m = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + wave;
    if (m >= a.M) return;   // wave-uniform
    const int D = a.D;
    float *r = any_lds + static_cast<int64_t>(wave) * D;
    for (int d = lane; d < D; d += kWave) r[d] = a.x[m * D + d];
    wave_lds_sync();
    const int np = D & ~(kWave - 1);
    const int fused_from = D - (D - np) % 4;
    for (int s = 0; s < a.Q; ++s) {
        const float *W = a.w_in + static_cast<int64_t>(s) * 8 * D;
        float p[8];
        if (a.order == 1) {
            // tinyBLAS (sgemm.cpp:527-545): lane 16 g + t runs accumulator t
            // (k = 16 u + t) of outputs 2g and 2g+1, then _mm512_reduce_add_ps
            // (pairs 8, 4, 2, 1 apart) inside the 16-lane row
            const int t = lane & 15, g = lane >> 4;
            float a0 = 0.0f, a1 = 0.0f;
            for (int k = t; k < D; k += 16) {
                const float v = r[k];
                a0 = __fmaf_rn(v, W[(2 * g) * D + k], a0);
                a1 = __fmaf_rn(v, W[(2 * g + 1) * D + k], a1);
            }
            for (int off = 8; off >= 1; off >>= 1) {
                a0 = __fadd_rn(a0, __shfl_xor(a0, off));
                a1 = __fadd_rn(a1, __shfl_xor(a1, off));
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                p[2 * q] = __shfl(a0, 16 * q);
                p[2 * q + 1] = __shfl(a1, 16 * q);
            }
        } else {
            // ggml_vec_dot_f32 (vec.cpp:11-135): accumulator (j, l) = lane
            // 16 j + l over 64-element steps, GGML_F32_VEC_REDUCE's pairing
            // (lanes 32 apart, then 16, then 8, 4, 2, 1), then the leftovers:
            // rounded products added in order, the last rem % 4 fused (the
            // reference's native build)
            float acc[8];
#pragma unroll
            for (int o = 0; o < 8; ++o) acc[o] = 0.0f;
            for (int k = lane; k < np; k += kWave) {
                const float v = r[k];
#pragma unroll
                for (int o = 0; o < 8; ++o) acc[o] = __fmaf_rn(v, W[o * D + k], acc[o]);
            }
#pragma unroll
            for (int o = 0; o < 8; ++o)
                for (int off = 32; off >= 1; off >>= 1) acc[o] = __fadd_rn(acc[o], __shfl_xor(acc[o], off));
            float sum = acc[0];
#pragma unroll
            for (int o = 1; o < 8; ++o)
                if ((lane & 7) == o) sum = acc[o];
            if (lane < 8) {
                const float *w = W + lane * D;
                for (int k = np; k < D; ++k)
                    sum = k >= fused_from ? __fmaf_rn(r[k], w[k], sum) : __fadd_rn(sum, __fmul_rn(r[k], w[k]));
            }
#pragma unroll
            for (int o = 0; o < 8; ++o) p[o] = __shfl(sum, o);
        }
        if (a.b_in) {
#pragma unroll
            for (int o = 0; o < 8; ++o) p[o] = __fadd_rn(p[o], a.b_in[s * 8 + o]);
        }
        // l2 normalisation: fp32 squares summed in double in output order,
        // + eps (ggml_scale_bias), correctly rounded sqrt, IEEE division
        double ss = 0.0;
#pragma unroll
        for (int o = 0; o < 8; ++o) ss += static_cast<double>(__fmul_rn(p[o], p[o]));
        const float den = sqrt_rn(__fadd_rn(static_cast<float>(ss), a.qeps));
        float pn[8];
#pragma unroll
        for (int o = 0; o < 8; ++o) pn[o] = __fdiv_rn(p[o], den);
        // exact scores (k = 8 mul_mat: rounded products added in order) and
        // ggml_vec_argmax_f32 (last index of the maximum; a NaN restarts it)
        const float *C = a.chat + static_cast<int64_t>(s) * a.N * 8;
        float bv = -INFINITY;
        int bn = -1;
        bool bad = false;
        for (int n = lane; n < a.N; n += kWave) {
            const float4 c0 = *reinterpret_cast<const float4 *>(C + static_cast<int64_t>(n) * 8);
            const float4 c1 = *reinterpret_cast<const float4 *>(C + static_cast<int64_t>(n) * 8 + 4);
            const float sc = exact_score(c0, c1, pn);
            bad |= sc != sc;
            if (sc >= bv) {
                bv = sc;
                bn = n;
            }
        }
#pragma unroll
        for (int off = 1; off <= 32; off <<= 1) {
            const float ov = __shfl_xor(bv, off);
            const int on = __shfl_xor(bn, off);
            if (ov > bv || (ov == bv && on > bn)) {
                bv = ov;
                bn = on;
            }
        }
        int code = uniform_i(bn < 0 ? 0 : bn);
        if (__any(bad)) {
            float mx = -INFINITY;
            int id = 0;
            for (int n = 0; n < a.N; ++n) {
                const float4 c0 = *reinterpret_cast<const float4 *>(C + static_cast<int64_t>(n) * 8);
                const float4 c1 = *reinterpret_cast<const float4 *>(C + static_cast<int64_t>(n) * 8 + 4);
                const float sc = exact_score(c0, c1, pn);
                mx = mx > sc ? mx : sc;
                if (mx == sc) id = n;
            }
            code = uniform_i(id);
        }
        if (lane == 0) a.idx[m * a.ld + s] = code;
        int use = code;
        if (a.force_idx) {
            use = a.force_idx[m * a.ld + s];
            if (use < 0 || use >= a.N) {
                if (lane == 0) a.flags[AQ_FLAG_BAD_INDEX] = 1;
                use = 0;
            }
        }
        if (a.tables) {
            // r -= z; recon += z (each lane its own elements)
            const float *z = a.tables + (static_cast<int64_t>(s) * a.N + use) * D;
            for (int d = lane; d < D; d += kWave) {
                const float zd = z[d];
                r[d] = __fsub_rn(r[d], zd);
                if (a.recon) {
                    const float prev = (s == 0 && !a.recon_acc) ? -0.0f : a.recon[m * D + d];
                    a.recon[m * D + d] = __fadd_rn(prev, zd);
                }
            }
            wave_lds_sync();
        }
    }
    if (a.residual)
        for (int d = lane; d < D; d += kWave) a.residual[m * D + d] = r[d];
}

using EncodeFn = void (*)(const float *, int64_t, int, int, const float4 *, int64_t, int64_t, const float *, int32_t *,
                          float *, float *, const int32_t *, int32_t *, int, int, float, int, float, int64_t, int, int);

constexpr int kPrefetch = 12;   // float4 per thread in the prefetching variant

// Variants: image copied at each stage start, prefetched a stage ahead, or
// (large codebooks) the W_in + b_in prefix prefetched with c_hat in memory.
// ORDER: the in-projection's summation order, 0 ggml_vec_dot_f32, 1 tinyBLAS.
template <int DI, int FW, bool RECON, int ORDER>
EncodeFn pick_pf(bool prefetch, bool cbg) {
    if (cbg) return dac_encode_kernel<DI, FW, RECON, kPrefetch, true, ORDER>;
    return prefetch ? dac_encode_kernel<DI, FW, RECON, kPrefetch, false, ORDER>
                    : dac_encode_kernel<DI, FW, RECON, 0, false, ORDER>;
}

template <int DI, int FW, int ORDER>
EncodeFn pick_recon(bool recon, bool prefetch, bool cbg) {
    return recon ? pick_pf<DI, FW, true, ORDER>(prefetch, cbg) : pick_pf<DI, FW, false, ORDER>(prefetch, cbg);
}

template <int DI, int ORDER>
EncodeFn pick_fw(int fw, bool recon, bool prefetch, bool cbg) {
    switch (fw) {
        case 1: return pick_recon<DI, 1, ORDER>(recon, prefetch, cbg);
        case 2: return pick_recon<DI, 2, ORDER>(recon, prefetch, cbg);
        default: return pick_recon<DI, 3, ORDER>(recon, prefetch, cbg);
    }
}

template <int ORDER>
EncodeFn pick_kernel_o(int64_t D, int fw, bool recon, bool prefetch, bool cbg) {
    switch (D / kWave) {
        case 1: return pick_fw<1, ORDER>(fw, recon, prefetch, cbg);
        case 2: return pick_fw<2, ORDER>(fw, recon, prefetch, cbg);
        case 4: return pick_fw<4, ORDER>(fw, recon, prefetch, cbg);
        case 8: return pick_fw<8, ORDER>(fw, recon, prefetch, cbg);
        case 12: return pick_fw<12, ORDER>(fw, recon, prefetch, cbg);
        case 16: return pick_fw<16, ORDER>(fw, recon, prefetch, cbg);
        default: return nullptr;
    }
}

EncodeFn pick_kernel(int64_t D, int fw, bool recon, bool prefetch, bool cbg, int order = 0) {
    return order == 1 ? pick_kernel_o<1>(D, fw, recon, prefetch, cbg) : pick_kernel_o<0>(D, fw, recon, prefetch, cbg);
}

using MsFn = void (*)(const float *, int64_t, int, int, const float4 *, int64_t, const float *, int32_t *, float *,
                      float *, const int32_t *, int32_t *, int, int, float, int, float, int, int);

template <int DI, int ORDER>
MsFn pick_ms_recon(bool recon) {
    return recon ? dac_encode_ms_kernel<DI, true, ORDER> : dac_encode_ms_kernel<DI, false, ORDER>;
}

template <int ORDER>
MsFn pick_ms_o(int64_t D, bool recon) {
    switch (D / kWave) {
        case 1: return pick_ms_recon<1, ORDER>(recon);
        case 2: return pick_ms_recon<2, ORDER>(recon);
        case 4: return pick_ms_recon<4, ORDER>(recon);
        case 8: return pick_ms_recon<8, ORDER>(recon);
        case 12: return pick_ms_recon<12, ORDER>(recon);
        case 16: return pick_ms_recon<16, ORDER>(recon);
        default: return nullptr;
    }
}

MsFn pick_ms(int64_t D, bool recon, int order) {
    return order == 1 ? pick_ms_o<1>(D, recon) : pick_ms_o<0>(D, recon);
}

// Launch shape.  A wave keeps its frames' residuals in registers for the
// whole cascade, so work cannot be rebalanced after launch.  The shape is
// ranked by
//   1. frames on the busiest SIMD: ceil(blocks / CUs) blocks per CU, each
//      spreading waves_per_block * FW frames over the 4 SIMDs;
//   2. stage-image prefetch (the next stage's image is loaded into registers
//      while the current stage computes, so no wave waits on the copy);
//   3. 8-wave blocks (one image copy per CU and stage feeds 8 waves);
//   4. more frames per wave (each LDS read of the image feeds FW frames).
// Measured on MI355X (6000 frames, D = N = 1024, 12 stages): FW = 3 in 8-wave
// blocks with prefetch 113 us; the same without prefetch 134 us; FW = 1 in
// 8-wave blocks with prefetch 148 us; FW = 3 in 4-wave blocks 148 us.
struct Shape {
    int fw = 1;
    int waves_per_block = 4;
    bool prefetch = false;
};

Shape launch_shape(int64_t M, int64_t D, int64_t img_f4, bool recon, int num_cus, size_t lds_bytes, bool cbg,
                   int order) {
    const int64_t cus = num_cus > 0 ? num_cus : 256;
    int env_fw = 0, env_wpb = 0;
    if (const char *e = std::getenv("AQ_DAC_FW")) env_fw = std::atoi(e);
    if (const char *e = std::getenv("AQ_DAC_WPB")) env_wpb = std::atoi(e);
    Shape best;
    int64_t best_rank = INT64_MAX;
    for (int fw = 1; fw <= 3; ++fw) {
        if (env_fw >= 1 && env_fw <= 3 && fw != env_fw) continue;
        for (int wpb : {4, 6, 8}) {
            if (env_wpb && wpb != env_wpb) continue;
            bool prefetch = (img_f4 + wpb * kWave - 1) / (wpb * kWave) <= kPrefetch;
            if (const char *e = std::getenv("AQ_DAC_PF")) prefetch = prefetch && std::atoi(e) != 0;
            if (cbg && !prefetch) continue;   // the in-memory codebook variant always prefetches
            hipFuncAttributes attr{};
            int64_t simd_waves = 8;
            const void *kfn = reinterpret_cast<const void *>(pick_kernel(D, fw, recon, prefetch, cbg, order));
            if (hipFuncGetAttributes(&attr, kfn) == hipSuccess && attr.numRegs > 0)
                simd_waves = std::min<int64_t>(8, 512 / ((attr.numRegs + 7) / 8 * 8));
            // The block must fit on a CU at all (waves per SIMD by registers,
            // one stage image in LDS next to the kernel's static LDS).
            // order 1 adds a transposed copy of one frame per wave to LDS
            const size_t lds_total = lds_bytes + (order == 1 ? static_cast<size_t>(wpb) * D * 4 : 0);
            if (simd_waves < (wpb + 3) / 4 || lds_total > aq_lds_budget(kfn)) continue;
            const int64_t waves = (M + fw - 1) / fw;
            const int64_t blocks = (waves + wpb - 1) / wpb;
            const int64_t per_simd = ((blocks + cus - 1) / cus) * ((wpb * fw + 3) / 4);
            const int64_t rank = per_simd * 64 + (prefetch ? 0 : 16) + (wpb == 8 ? 0 : 8) + (3 - fw);
            if (std::getenv("AQ_DEBUG"))
                std::fprintf(stderr, "aq_dac shape fw=%d wpb=%d pf=%d regs=%d blocks=%lld per_simd=%lld rank=%lld\n", fw,
                             wpb, prefetch ? 1 : 0, attr.numRegs, (long long)blocks, (long long)per_simd,
                             (long long)rank);
            if (rank < best_rank) {
                best_rank = rank;
                best.fw = fw;
                best.waves_per_block = wpb;
                best.prefetch = prefetch;
            }
        }
    }
    return best;
}

}  // namespace

struct aq_dac_stages {
    // device of the creating context (the handle keeps no pointer to it, so
    // it may be released after that context is destroyed)
    int device = -1;
    int64_t Q = 0, D = 0, N = 0;
    int recipe = AQ_DAC_FISH;
    float qeps = 1.0e-12f;        // ggml_scale_bias bias before the query norm's sqrt
    bool cbg = false;             // c_hat read from memory (does not fit in LDS with W_in)
    int64_t lds_f4 = 0;           // float4 of each stage image staged in LDS
    bool has_bin = false;
    bool exact_only = false;      // a normalised codebook entry is not finite
    int key_bits = 0;             // chunk-index bits in the score keys
    float margin = 0.0f;          // score-certificate margin
    // Matrix-core scores (dac_encode_ms_kernel) where the shape allows them:
    // their key bits and margin (in units of 2^24 c.q)
    bool ms = false;
    int ms_key_bits = 0;
    float ms_margin = 0.0f;
    int64_t img_f4 = 0;           // float4 per stage image (W_in, b_in, c_hat, c16)
    float4 *d_images = nullptr;   // [Q][img_f4]
    float4 *d_images_tb = nullptr;   // the same with W_in in the tinyBLAS layout
    float *d_tables = nullptr;    // [Q][N][D]
    // Shapes outside the fused kernel's (dac_any_kernel): W_in [Q][8][D],
    // b_in [Q][8], normalised codes [Q][N][8], one allocation
    bool any = false;
    float *d_any = nullptr;
    // OuteTTS host-loop recipe: raw weights, one allocation
    float *d_ot = nullptr;
    aq_outetts_args ot{};         // the weight pointers into d_ot
    // Launch-shape cache: the shape depends on M, recon and the summation
    // order only, and finding it queries the attributes of up to nine kernel
    // variants.  Calls that overlap on one stages object from several host
    // threads race on it (as they would on the context's stream).
    mutable int64_t shape_m = -1;
    mutable int shape_key = -1;
    mutable Shape shape{};
    mutable const void *lds_fn = nullptr;   // the kernel whose dynamic-LDS limit was last raised
    mutable size_t lds_limit = 0;
};

namespace {

// The OuteTTS recipe keeps the raw weights: its host loop recomputes
// everything per frame in sequential fp32 (aq_hostloop.hip).  The decode
// tables are the Fish ones (its decoder graph is the same 1x1 conv).
aq_status upload_outetts(aq_ctx *ctx, int64_t Q, int64_t D, int64_t N, const float *w_in, const float *b_in,
                         const float *codebook, const float *w_out, const float *b_out, aq_dac_stages **out) {
    if (!w_out) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_dac_upload: the OuteTTS recipe needs the out-projection");
    if (Q <= 0 || D <= 0 || D % kWave != 0 || D > 2048 || N <= 0 || N % 8 != 0 || N > (int64_t{1} << 20))
        return aq_fail(ctx, AQ_E_SHAPE,
                       "aq_dac_upload: unsupported OuteTTS shape Q=%lld D=%lld N=%lld (D a multiple of 64 up to 2048, "
                       "N a multiple of 8)",
                       (long long)Q, (long long)D, (long long)N);
    aq_device_guard g(ctx->device);
    const int64_t sizes[] = {Q * 8 * D, Q * 8, Q * N * 8, Q * N * 8, Q * D * 8, Q * D};
    int64_t total = 0;
    for (int64_t v : sizes) total += (v + 63) / 64 * 64;
    auto *st = new aq_dac_stages();
    st->device = ctx->device;
    st->Q = Q;
    st->D = D;
    st->N = N;
    st->recipe = AQ_DAC_OUTETTS;
    st->has_bin = b_in != nullptr;
    bool ok = hipMalloc(&st->d_ot, static_cast<size_t>(total) * sizeof(float)) == hipSuccess &&
              hipMalloc(&st->d_tables, static_cast<size_t>(Q * N * D) * sizeof(float)) == hipSuccess;
    std::vector<float> zeros;
    if (ok) {
        float *slot[6];
        int64_t off = 0;
        for (int i = 0; i < 6; ++i) {
            slot[i] = st->d_ot + off;
            off += (sizes[i] + 63) / 64 * 64;
        }
        zeros.assign(static_cast<size_t>(std::max(Q * 8, Q * D)), 0.0f);
        const float *src[6] = {w_in, b_in ? b_in : zeros.data(), codebook, nullptr, w_out, b_out ? b_out : zeros.data()};
        for (int i = 0; i < 6 && ok; ++i)
            if (src[i])
                ok = hipMemcpyAsync(slot[i], src[i], static_cast<size_t>(sizes[i]) * sizeof(float), hipMemcpyHostToDevice,
                                    ctx->stream) == hipSuccess;
        ok = ok && aq_outetts_prepare(ctx, slot[2], Q * N, slot[3]) == AQ_OK;
        for (int64_t s = 0; s < Q && ok; ++s) {
            const unsigned blocks = static_cast<unsigned>((N * D + 255) / 256);
            hipLaunchKernelGGL(dac_table_kernel, dim3(blocks), dim3(256), 0, ctx->stream, slot[2] + s * N * 8,
                               slot[4] + s * D * 8, b_out ? slot[5] + s * D : nullptr, N, D, st->d_tables + s * N * D);
            ok = hipGetLastError() == hipSuccess;
        }
        st->ot.w_in = slot[0];
        st->ot.b_in = slot[1];
        st->ot.cb = slot[2];
        st->ot.chat = slot[3];
        st->ot.w_out = slot[4];
        st->ot.b_out = slot[5];
        st->ot.D = static_cast<int>(D);
        st->ot.N = static_cast<int>(N);
        st->ot.Q = static_cast<int>(Q);
    }
    ok = hipStreamSynchronize(ctx->stream) == hipSuccess && ok;
    if (!ok) {
        aq_dac_release(st);
        return aq_fail(ctx, AQ_E_DEVICE, "aq_dac_upload: device copy or OuteTTS preparation failed");
    }
    *out = st;
    return AQ_OK;
}

// Largest latent of the any-shape kernel (one frame's residual in LDS) and
// largest codebook of either kernel.
constexpr int64_t kAnyMaxD = 40000;
constexpr int64_t kMaxN = int64_t{1} << 24;

// Upload for dac_any_kernel: the weights as given, the recipe's normalised
// codebook rows and the out-projection tables, built on the device.
aq_status upload_any(aq_ctx *ctx, int64_t Q, int64_t D, int64_t N, const float *w_in, const float *b_in,
                     const float *codebook, const float *w_out, const float *b_out, int recipe, aq_dac_stages **out) {
    if (D > kAnyMaxD || N > kMaxN)
        return aq_fail(ctx, AQ_E_SHAPE, "aq_dac_upload: D=%lld N=%lld exceed the supported %lld x %lld", (long long)D,
                       (long long)N, (long long)kAnyMaxD, (long long)kMaxN);
    aq_device_guard g(ctx->device);
    aq_dac_stages *st = new (std::nothrow) aq_dac_stages();
    if (!st) return aq_fail(ctx, AQ_E_NOMEM, "aq_dac_upload: host allocation failed");
    st->device = ctx->device;
    st->Q = Q;
    st->D = D;
    st->N = N;
    st->recipe = recipe;
    st->any = true;
    st->has_bin = b_in != nullptr;
    st->qeps = recipe == AQ_DAC_INDEXTTS2 ? 0.0f : (recipe == AQ_DAC_VEVO2 ? 1.0e-20f : 1.0e-12f);
    const size_t nwin = static_cast<size_t>(Q * 8 * D), nbin = static_cast<size_t>(Q * 8),
                 nchat = static_cast<size_t>(Q * N * 8);
    float *d_cb = nullptr, *d_wout = nullptr, *d_bout = nullptr;
    unsigned long long *d_flags = nullptr;
    auto cleanup = [&]() {
        for (void *p : {static_cast<void *>(d_cb), static_cast<void *>(d_wout), static_cast<void *>(d_bout),
                        static_cast<void *>(d_flags)})
            if (p) (void)hipFree(p);
    };
    if (hipMalloc(&st->d_any, sizeof(float) * (nwin + nbin + nchat)) != hipSuccess ||
        hipMalloc(&d_cb, sizeof(float) * nchat) != hipSuccess ||
        hipMalloc(&d_flags, 2 * sizeof(unsigned long long)) != hipSuccess ||
        (w_out && (hipMalloc(&st->d_tables, sizeof(float) * static_cast<size_t>(Q * N * D)) != hipSuccess ||
                   hipMalloc(&d_wout, sizeof(float) * static_cast<size_t>(Q * D * 8)) != hipSuccess ||
                   (b_out && hipMalloc(&d_bout, sizeof(float) * static_cast<size_t>(Q * D)) != hipSuccess)))) {
        cleanup();
        aq_dac_release(st);
        return aq_fail(ctx, AQ_E_NOMEM, "aq_dac_upload: device allocation failed");
    }
    float *win = st->d_any, *bin = st->d_any + nwin, *chat = st->d_any + nwin + nbin;
    const unsigned long long flags_init[2] = {~0ull, 0ull};
    bool ok = hipMemcpyAsync(win, w_in, sizeof(float) * nwin, hipMemcpyHostToDevice, ctx->stream) == hipSuccess &&
              (!b_in || hipMemcpyAsync(bin, b_in, sizeof(float) * nbin, hipMemcpyHostToDevice, ctx->stream) == hipSuccess) &&
              hipMemcpyAsync(d_cb, codebook, sizeof(float) * nchat, hipMemcpyHostToDevice, ctx->stream) == hipSuccess &&
              hipMemcpyAsync(d_flags, flags_init, sizeof(flags_init), hipMemcpyHostToDevice, ctx->stream) == hipSuccess;
    if (ok) {
        hipLaunchKernelGGL(dac_any_chat_kernel, dim3(static_cast<unsigned>((Q * N + 255) / 256)), dim3(256), 0,
                           ctx->stream, d_cb, Q * N, recipe, chat, d_flags);
        ok = hipGetLastError() == hipSuccess;
    }
    if (w_out)
        ok = ok &&
             hipMemcpyAsync(d_wout, w_out, sizeof(float) * static_cast<size_t>(Q * D * 8), hipMemcpyHostToDevice, ctx->stream) == hipSuccess &&
             (!b_out || hipMemcpyAsync(d_bout, b_out, sizeof(float) * static_cast<size_t>(Q * D), hipMemcpyHostToDevice, ctx->stream) == hipSuccess);
    for (int64_t s = 0; ok && w_out && s < Q; ++s) {
        hipLaunchKernelGGL(dac_table_kernel, dim3(static_cast<unsigned>((N * D + 255) / 256)), dim3(256), 0, ctx->stream,
                           d_cb + s * N * 8, d_wout + s * D * 8, d_bout ? d_bout + s * D : nullptr, N, D,
                           st->d_tables + s * N * D);
        ok = hipGetLastError() == hipSuccess;
    }
    unsigned long long flags[2] = {~0ull, 0ull};
    ok = ok && hipMemcpyAsync(flags, d_flags, sizeof(flags), hipMemcpyDeviceToHost, ctx->stream) == hipSuccess &&
         hipStreamSynchronize(ctx->stream) == hipSuccess;
    cleanup();
    if (!ok) {
        aq_dac_release(st);
        return aq_fail(ctx, AQ_E_DEVICE, "aq_dac_upload: device copy or codebook preparation failed");
    }
    if (flags[0] != ~0ull) {
        const long long n = static_cast<long long>(flags[0] % static_cast<unsigned long long>(N)),
                        s = static_cast<long long>(flags[0] / static_cast<unsigned long long>(N));
        aq_dac_release(st);
        return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_dac_upload: codebook row %lld of stage %lld has zero norm", n, s);
    }
    *out = st;
    return AQ_OK;
}

// Launch of dac_any_kernel on frame-major rows x [M, D].
aq_status encode_any(aq_ctx *ctx, const aq_dac_stages *st, const float *x, int64_t M, int64_t clip_len, int32_t *idx,
                     int64_t idx_ld, float *residual, float *recon, int recon_accumulate, const int32_t *force_idx) {
    const int64_t D = st->D;
    int wpb = 4;
    while (wpb > 1 && static_cast<size_t>(wpb) * D * sizeof(float) > aq_lds_budget(reinterpret_cast<const void *>(dac_any_kernel)))
        wpb /= 2;
    const size_t lds = static_cast<size_t>(wpb) * D * sizeof(float);
    {
        aq_status ls = aq_launch_lds(ctx, reinterpret_cast<const void *>(dac_any_kernel), lds, "aq_dac_encode");
        if (ls != AQ_OK) return ls;
    }
    DacAnyArgs a{};
    a.x = x;
    a.M = M;
    a.D = static_cast<int>(D);
    a.N = static_cast<int>(st->N);
    a.Q = static_cast<int>(st->Q);
    const float *win = st->d_any;
    a.w_in = win;
    a.b_in = st->has_bin ? win + st->Q * 8 * D : nullptr;
    a.chat = win + st->Q * 8 * D + st->Q * 8;
    a.tables = st->d_tables;
    a.idx = idx;
    a.ld = static_cast<int>(idx_ld);
    a.residual = residual;
    a.recon = recon;
    a.recon_acc = recon_accumulate ? 1 : 0;
    a.force_idx = force_idx;
    a.flags = ctx->d_flags;
    a.qeps = st->qeps;
    // tinyBLAS takes the in-projection when the clip length is a multiple of
    // 4 and D of 16 (ggml-cpu.c:1285-1306, sgemm.cpp:3705-3725)
    a.order = (clip_len % 4 == 0 && D % 16 == 0) ? 1 : 0;
    aq_launch_timed(ctx, true, dac_any_kernel, dim3(static_cast<unsigned>((M + wpb - 1) / wpb)), dim3(wpb * kWave),
                    static_cast<uint32_t>(lds), a);
    AQ_HIP(ctx, hipGetLastError());
    return AQ_OK;
}

// After a teacher-forced encode: AQ_E_INDEX_RANGE when force_idx held a code
// outside [0, N) (the kernels flag it and use code 0 instead).
aq_status dac_check_forced(aq_ctx *ctx, const aq_dac_stages *st, const int32_t *force_idx) {
    if (!force_idx) return AQ_OK;
    int32_t flag = 0;
    AQ_HIP(ctx, hipMemcpyAsync(&flag, ctx->d_flags + AQ_FLAG_BAD_INDEX, sizeof(int32_t), hipMemcpyDeviceToHost, ctx->stream));
    AQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (flag) return aq_fail(ctx, AQ_E_INDEX_RANGE, "aq_dac_encode: force_idx holds a code outside [0, %lld)", (long long)st->N);
    return AQ_OK;
}

}  // namespace

extern "C" {

aq_status aq_dac_upload(aq_ctx *ctx, int64_t Q, int64_t D, int64_t N, const float *w_in, const float *b_in,
                        const float *codebook, const float *w_out, const float *b_out, aq_dac_stages **out) {
    return aq_dac_upload_ex(ctx, Q, D, N, w_in, b_in, codebook, w_out, b_out, AQ_DAC_FISH, out);
}

aq_status aq_dac_upload_ex(aq_ctx *ctx, int64_t Q, int64_t D, int64_t N, const float *w_in, const float *b_in,
                           const float *codebook, const float *w_out, const float *b_out, int recipe,
                           aq_dac_stages **out) {
    if (!ctx || !out || !w_in || !codebook) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_dac_upload: null argument");
    *out = nullptr;
    if (recipe == AQ_DAC_OUTETTS) return upload_outetts(ctx, Q, D, N, w_in, b_in, codebook, w_out, b_out, out);
    if (recipe < AQ_DAC_FISH || recipe > AQ_DAC_VEVO2)
        return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_dac_upload: unknown recipe %d", recipe);
    if (!w_out && Q != 1)
        return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_dac_upload: a residual cascade (Q=%lld) needs the out-projection",
                       (long long)Q);
    if (Q <= 0 || D <= 0 || N <= 0)
        return aq_fail(ctx, AQ_E_SHAPE, "aq_dac_upload: empty shape Q=%lld D=%lld N=%lld", (long long)Q, (long long)D,
                       (long long)N);
    // The fused kernel's shapes: D a multiple of 64 with a register tile
    // (64 ... 1024), N a multiple of 64 up to 2^20; anything else takes the
    // any-shape kernel.
    if (D % kWave != 0 || N % kWave != 0 || N > (int64_t{1} << 20) || !pick_kernel(D, 1, false, false, false))
        return upload_any(ctx, Q, D, N, w_in, b_in, codebook, w_out, b_out, recipe, out);
    int64_t img = image_f4(D, N);
    // c_hat read from memory when the whole stage image does not fit in LDS
    // next to the kernel's static LDS
    const bool cbg = static_cast<size_t>(img) * 16 >
                     aq_lds_budget(reinterpret_cast<const void *>(pick_kernel(D, 1, false, false, false)));
    aq_device_guard g(ctx->device);

    aq_dac_stages *st = new (std::nothrow) aq_dac_stages();
    if (!st) return aq_fail(ctx, AQ_E_NOMEM, "aq_dac_upload: host allocation failed");
    st->device = ctx->device;
    st->Q = Q;
    st->D = D;
    st->N = N;
    st->has_bin = b_in != nullptr;
    st->recipe = recipe;
    st->qeps = recipe == AQ_DAC_INDEXTTS2 ? 0.0f : (recipe == AQ_DAC_VEVO2 ? 1.0e-20f : 1.0e-12f);
    st->cbg = cbg;
    st->lds_f4 = cbg ? image_prefix_f4(D) : img;
    // Certificate margin: each approximate score (FMA chain) and ggml's score
    // (rounded products, sequential sum) are within 8u and 15u of the exact
    // dot of two vectors of norm <= 1 (u = 2^-24): 2 * 23u = 2.8e-6 for the
    // pair compared, plus the truncation of two keys (2^(bits-23) relative
    // each, |score| <= 1) and the rounding of their difference.
    {
        int bits = 0;
        while ((int64_t{1} << bits) < N / kWave) ++bits;
        st->key_bits = bits;
        st->margin = 5.0e-6f + std::ldexp(1.001f, bits - 22);
    }
    // Matrix-core scores: each score is within 4.3e-6 of the exact dot
    // (split 2^-21 + accumulation 62u + flushed operands 1e-7) and ggml's
    // within 15u: 1.2e-5 for the pair, plus the keys' truncation; scaled by
    // 2^24 like the scores.
    st->ms = !cbg && N % (16 * kMsWaves) == 0 && N <= kMsPart * kMsWaves * kWave / 2 &&
             D <= kMsPart * kMsWaves * kWave / 2;
    {
        int bits = 0;
        while ((int64_t{1} << bits) < N / kMsWaves) ++bits;
        st->ms_key_bits = bits;
        st->ms_margin = std::ldexp(1.2e-5f + std::ldexp(1.001f, bits - 22), 24);
    }
    img += 2 * N;   // the split codebook (c16) after c_hat
    st->img_f4 = img;
    // The host arrays go to the device as given; the stage images and the
    // out-projection tables are built there.
    const size_t img_bytes = sizeof(float) * static_cast<size_t>(Q * img * 4);
    float *d_cb = nullptr, *d_win = nullptr, *d_bin = nullptr, *d_wout = nullptr, *d_bout = nullptr;
    unsigned long long *d_flags = nullptr;
    auto cleanup = [&]() {
        for (void *p : {static_cast<void *>(d_cb), static_cast<void *>(d_win), static_cast<void *>(d_bin),
                        static_cast<void *>(d_wout), static_cast<void *>(d_bout), static_cast<void *>(d_flags)})
            if (p) (void)hipFree(p);
    };
    if (hipMalloc(&st->d_images, img_bytes) != hipSuccess || hipMalloc(&st->d_images_tb, img_bytes) != hipSuccess ||
        hipMalloc(&d_cb, sizeof(float) * static_cast<size_t>(Q * N * 8)) != hipSuccess ||
        hipMalloc(&d_win, sizeof(float) * static_cast<size_t>(Q * 8 * D)) != hipSuccess ||
        hipMalloc(&d_flags, 2 * sizeof(unsigned long long)) != hipSuccess ||
        (b_in && hipMalloc(&d_bin, sizeof(float) * static_cast<size_t>(Q * 8)) != hipSuccess) ||
        (w_out && (hipMalloc(&st->d_tables, sizeof(float) * static_cast<size_t>(Q * N * D)) != hipSuccess ||
                   hipMalloc(&d_wout, sizeof(float) * static_cast<size_t>(Q * D * 8)) != hipSuccess ||
                   (b_out && hipMalloc(&d_bout, sizeof(float) * static_cast<size_t>(Q * D)) != hipSuccess)))) {
        cleanup();
        aq_dac_release(st);
        return aq_fail(ctx, AQ_E_NOMEM, "aq_dac_upload: device allocation failed");
    }
    const unsigned long long flags_init[2] = {~0ull, 0ull};
    bool ok = hipMemcpyAsync(d_cb, codebook, sizeof(float) * static_cast<size_t>(Q * N * 8), hipMemcpyHostToDevice, ctx->stream) == hipSuccess &&
              hipMemcpyAsync(d_win, w_in, sizeof(float) * static_cast<size_t>(Q * 8 * D), hipMemcpyHostToDevice, ctx->stream) == hipSuccess &&
              (!b_in || hipMemcpyAsync(d_bin, b_in, sizeof(float) * static_cast<size_t>(Q * 8), hipMemcpyHostToDevice, ctx->stream) == hipSuccess) &&
              hipMemcpyAsync(d_flags, flags_init, sizeof(flags_init), hipMemcpyHostToDevice, ctx->stream) == hipSuccess &&
              hipMemsetAsync(st->d_images, 0, img_bytes, ctx->stream) == hipSuccess &&
              hipMemsetAsync(st->d_images_tb, 0, img_bytes, ctx->stream) == hipSuccess;
    if (ok) {
        hipLaunchKernelGGL(dac_image_win_kernel, dim3(static_cast<unsigned>((Q * 8 * D + 255) / 256)), dim3(256), 0,
                           ctx->stream, d_win, Q, D, img * 4, reinterpret_cast<float *>(st->d_images), reinterpret_cast<float *>(st->d_images_tb));
        hipLaunchKernelGGL(dac_image_cb_kernel, dim3(static_cast<unsigned>((Q * N + 255) / 256)), dim3(256), 0,
                           ctx->stream, d_cb, d_bin, Q, N, D, img * 4, recipe, reinterpret_cast<float *>(st->d_images), reinterpret_cast<float *>(st->d_images_tb), d_flags);
        hipLaunchKernelGGL(dac_image_c16_kernel, dim3(static_cast<unsigned>((Q * N + 255) / 256)), dim3(256), 0,
                           ctx->stream, Q, N, D, img * 4, reinterpret_cast<float *>(st->d_images), reinterpret_cast<float *>(st->d_images_tb));
        ok = hipGetLastError() == hipSuccess;
    }
    if (w_out)
        ok = ok &&
             hipMemcpyAsync(d_wout, w_out, sizeof(float) * static_cast<size_t>(Q * D * 8), hipMemcpyHostToDevice, ctx->stream) == hipSuccess &&
             (!b_out || hipMemcpyAsync(d_bout, b_out, sizeof(float) * static_cast<size_t>(Q * D), hipMemcpyHostToDevice, ctx->stream) == hipSuccess);
    for (int64_t s = 0; ok && w_out && s < Q; ++s) {
        const int64_t total = N * D;
        const unsigned blocks = static_cast<unsigned>((total + 255) / 256);
        hipLaunchKernelGGL(dac_table_kernel, dim3(blocks), dim3(256), 0, ctx->stream, d_cb + s * N * 8, d_wout + s * D * 8,
                           d_bout ? d_bout + s * D : nullptr, N, D, st->d_tables + s * N * D);
        ok = hipGetLastError() == hipSuccess;
    }
    unsigned long long flags[2] = {~0ull, 0ull};
    ok = ok && hipMemcpyAsync(flags, d_flags, sizeof(flags), hipMemcpyDeviceToHost, ctx->stream) == hipSuccess &&
         hipStreamSynchronize(ctx->stream) == hipSuccess;
    cleanup();
    if (!ok) {
        aq_dac_release(st);
        return aq_fail(ctx, AQ_E_DEVICE, "aq_dac_upload: device copy or image preparation failed");
    }
    if (flags[0] != ~0ull) {
        const long long n = static_cast<long long>(flags[0] % static_cast<unsigned long long>(N)),
                        s = static_cast<long long>(flags[0] / static_cast<unsigned long long>(N));
        aq_dac_release(st);
        return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_dac_upload: codebook row %lld of stage %lld has zero norm", n, s);
    }
    st->exact_only = flags[1] != 0;
    *out = st;
    return AQ_OK;
}

aq_status aq_dac_release(aq_dac_stages *st) {
    if (!st) return AQ_E_INVALID_ARG;
    {
        aq_device_guard g(st->device);
        if (st->d_images) (void)hipFree(st->d_images);
        if (st->d_images_tb) (void)hipFree(st->d_images_tb);
        if (st->d_tables) (void)hipFree(st->d_tables);
        if (st->d_ot) (void)hipFree(st->d_ot);
        if (st->d_any) (void)hipFree(st->d_any);
    }
    delete st;
    return AQ_OK;
}

aq_status aq_dac_encode(aq_ctx *ctx, const aq_dac_stages *st, const float *x, int64_t M, int64_t clip_len,
                        int32_t *idx, float *residual, float *recon, const int32_t *force_idx) {
    const int64_t D = st ? st->D : 0;
    return aq_dac_encode_ex(ctx, st, x, M, clip_len, clip_len * D, D, 1, idx, st ? st->Q : 0, residual, recon, 0,
                            force_idx);
}

aq_status aq_dac_encode_ex(aq_ctx *ctx, const aq_dac_stages *st, const float *x, int64_t M, int64_t clip_len,
                           int64_t clip_stride, int64_t frame_stride, int64_t chan_stride, int32_t *idx,
                           int64_t idx_ld, float *residual, float *recon, int recon_accumulate,
                           const int32_t *force_idx) {
    if (!ctx || !st || (M > 0 && (!idx || !x))) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_dac_encode: null argument");
    if (st->device != ctx->device) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_dac_encode: stages belong to another device");
    if (M < 0 || clip_len <= 0 || M % clip_len != 0)
        return aq_fail(ctx, AQ_E_SHAPE, "aq_dac_encode: M=%lld must be a non-negative multiple of clip_len=%lld",
                       (long long)M, (long long)clip_len);
    if (idx_ld < st->Q || idx_ld > (int64_t{1} << 20))
        return aq_fail(ctx, AQ_E_SHAPE, "aq_dac_encode: idx_ld=%lld must be at least Q=%lld", (long long)idx_ld,
                       (long long)st->Q);
    if (recon_accumulate && !recon)
        return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_dac_encode: recon_accumulate needs a recon buffer");
    if (M == 0) return AQ_OK;
    // A strided input (e.g. the encoder's channel-major [B, D, T] latent) is
    // gathered into frame-major rows first.
    if (!(frame_stride == st->D && chan_stride == 1 && clip_stride == clip_len * st->D)) {
        aq_device_guard g(ctx->device);
        float *rows = nullptr;
        aq_status gs = aq_ctx_scratch(ctx, 5, static_cast<size_t>(M) * st->D * sizeof(float), reinterpret_cast<void **>(&rows));
        if (gs != AQ_OK) return gs;
        gs = aq_gather_frames(ctx, aq_frames_desc{x, clip_len, clip_stride, frame_stride, chan_stride}, M, st->D, rows);
        if (gs != AQ_OK) return gs;
        x = rows;
    }
    if (st->recipe == AQ_DAC_OUTETTS) {
        if (recon)
            return aq_fail(ctx, AQ_E_INVALID_ARG,
                           "aq_dac_encode: the OuteTTS recipe gives no recon (aq_dac_decode of the codes does)");
        if (idx_ld != st->Q)
            return aq_fail(ctx, AQ_E_UNSUPPORTED, "aq_dac_encode: the OuteTTS recipe writes codes [M, Q] (idx_ld = Q)");
        aq_device_guard g(ctx->device);
        if (force_idx) AQ_HIP(ctx, hipMemsetAsync(ctx->d_flags, 0, sizeof(int32_t) * AQ_FLAG_COUNT, ctx->stream));
        aq_outetts_args a = st->ot;
        a.x = x;
        a.M = M;
        a.force_idx = force_idx;
        a.idx = idx;
        a.residual = residual;
        a.flags = ctx->d_flags;
        aq_status rs = aq_outetts_launch(ctx, a);
        if (rs != AQ_OK) return rs;
        if (force_idx) {
            int32_t flag = 0;
            AQ_HIP(ctx, hipMemcpyAsync(&flag, ctx->d_flags + AQ_FLAG_BAD_INDEX, sizeof(int32_t), hipMemcpyDeviceToHost,
                                       ctx->stream));
            AQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
            if (flag)
                return aq_fail(ctx, AQ_E_INDEX_RANGE, "aq_dac_encode: force_idx holds a code outside [0, %lld)", (long long)st->N);
        }
        return AQ_OK;
    }
    // ggml hands the in-projection (m = T rows, n = 8, k = D) to tinyBLAS when
    // T % 4 == 0 (ggml-cpu.c:1285-1306, sgemm.cpp:3705-3725), otherwise each
    // element is a ggml_vec_dot_f32.
    const int order = clip_len % 4 == 0 ? 1 : 0;
    if (!st->d_tables && (residual || recon))
        return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_dac_encode: no out-projection was uploaded (codes only)");
    aq_device_guard g(ctx->device);
    if (st->any) {
        if (force_idx) AQ_HIP(ctx, hipMemsetAsync(ctx->d_flags, 0, sizeof(int32_t) * AQ_FLAG_COUNT, ctx->stream));
        aq_status as = encode_any(ctx, st, x, M, clip_len, idx, idx_ld, residual, recon, recon_accumulate, force_idx);
        if (as != AQ_OK) return as;
        if (force_idx) {
            int32_t flag = 0;
            AQ_HIP(ctx, hipMemcpyAsync(&flag, ctx->d_flags + AQ_FLAG_BAD_INDEX, sizeof(int32_t), hipMemcpyDeviceToHost,
                                       ctx->stream));
            AQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
            if (flag)
                return aq_fail(ctx, AQ_E_INDEX_RANGE, "aq_dac_encode: force_idx holds a code outside [0, %lld)", (long long)st->N);
        }
        return AQ_OK;
    }
    const size_t img_bytes = static_cast<size_t>(st->lds_f4) * sizeof(float4);
    const int shape_key = (recon != nullptr ? 1 : 0) | (order << 1);
    if (st->shape_m != M || st->shape_key != shape_key) {
        st->shape = launch_shape(M, st->D, st->lds_f4, recon != nullptr, ctx->num_cus, img_bytes, st->cbg, order);
        st->shape_m = M;
        st->shape_key = shape_key;
    }
    const Shape shape = st->shape;
    const int fw = shape.fw;
    // Matrix-core scores where the shape allows them and the launch shape is
    // the one they use (8 waves x 3 frames); AQ_DAC_MS=0 / 1 turns them off /
    // takes them whenever the codebook allows (tests of both paths).
    {
        const char *e = std::getenv("AQ_DAC_MS");
        const bool want = st->ms && !st->exact_only &&
                          (e && e[0] == '1' ? true
                           : e && e[0] == '0' ? false
                                               : fw == kMsFw && shape.waves_per_block == kMsWaves);
        MsFn mfn = want ? pick_ms(st->D, recon != nullptr, order) : nullptr;
        const size_t ms_lds = static_cast<size_t>(2 * st->D + 4 * st->N + 64 + kMsWaves * 16) * sizeof(float4) +
                              (order == 1 ? static_cast<size_t>(kMsWaves) * st->D * sizeof(float) : 0);
        if (mfn && ms_lds <= aq_lds_budget(reinterpret_cast<const void *>(mfn))) {
            if (st->lds_fn != reinterpret_cast<const void *>(mfn) || st->lds_limit != ms_lds) {
                aq_status ls = aq_launch_lds(ctx, reinterpret_cast<const void *>(mfn), ms_lds, "aq_dac_encode");
                if (ls != AQ_OK) return ls;
                st->lds_fn = reinterpret_cast<const void *>(mfn);
                st->lds_limit = ms_lds;
            }
            if (force_idx) AQ_HIP(ctx, hipMemsetAsync(ctx->d_flags, 0, sizeof(int32_t) * AQ_FLAG_COUNT, ctx->stream));
            const unsigned blocks = static_cast<unsigned>((M + kMsFrames - 1) / kMsFrames);
            if (std::getenv("AQ_DEBUG")) std::fprintf(stderr, "aq_dac matrix scores blocks=%u\n", blocks);
            aq_launch_timed(ctx, true, mfn, dim3(blocks), dim3(kMsWaves * kWave), static_cast<uint32_t>(ms_lds), x, M,
                            static_cast<int>(st->Q), static_cast<int>(st->N), order == 1 ? st->d_images_tb : st->d_images,
                            st->img_f4, static_cast<const float *>(st->d_tables), idx, residual, recon, force_idx,
                            ctx->d_flags, st->has_bin ? 1 : 0, st->ms_key_bits, st->ms_margin, 0, st->qeps,
                            static_cast<int>(idx_ld), recon_accumulate ? 1 : 0);
            AQ_HIP(ctx, hipGetLastError());
            return dac_check_forced(ctx, st, force_idx);
        }
    }
    EncodeFn fn = pick_kernel(st->D, fw, recon != nullptr, shape.prefetch, st->cbg, order);
    const size_t rt_bytes = order == 1 ? static_cast<size_t>(shape.waves_per_block) * static_cast<size_t>(st->D) * 4 : 0;
    // A second stage image in LDS when it fits: one barrier per stage.
    const size_t budget = aq_lds_budget(reinterpret_cast<const void *>(fn));
    const int64_t dbuf_f4 = 2 * img_bytes + rt_bytes <= budget ? st->lds_f4 : 0;
    const size_t lds_bytes = img_bytes * (dbuf_f4 > 0 ? 2 : 1) + rt_bytes;
    if (st->lds_fn != reinterpret_cast<const void *>(fn) || st->lds_limit != lds_bytes) {
        aq_status ls = aq_launch_lds(ctx, reinterpret_cast<const void *>(fn), lds_bytes, "aq_dac_encode");
        if (ls != AQ_OK) return ls;
        st->lds_fn = reinterpret_cast<const void *>(fn);
        st->lds_limit = lds_bytes;
    }
    if (force_idx) AQ_HIP(ctx, hipMemsetAsync(ctx->d_flags, 0, sizeof(int32_t) * AQ_FLAG_COUNT, ctx->stream));
    const int64_t frames_per_block = static_cast<int64_t>(shape.waves_per_block) * fw;
    const unsigned blocks = static_cast<unsigned>((M + frames_per_block - 1) / frames_per_block);
    aq_launch_timed(ctx, true, fn, dim3(blocks), dim3(shape.waves_per_block * kWave), static_cast<uint32_t>(lds_bytes), x, M,
                    static_cast<int>(st->Q), static_cast<int>(st->N), order == 1 ? st->d_images_tb : st->d_images,
                    st->img_f4, st->lds_f4, static_cast<const float *>(st->d_tables), idx, residual, recon, force_idx,
                    ctx->d_flags, st->has_bin ? 1 : 0, st->key_bits, st->margin, st->exact_only ? 1 : 0, st->qeps,
                    dbuf_f4, static_cast<int>(idx_ld), recon_accumulate ? 1 : 0);
    AQ_HIP(ctx, hipGetLastError());
    return dac_check_forced(ctx, st, force_idx);
}

aq_status aq_dac_decode(aq_ctx *ctx, const aq_dac_stages *st, const int32_t *idx, int64_t M, float *out) {
    return aq_dac_decode_ex(ctx, st, idx, st ? st->Q : 0, M, out, 0);
}

aq_status aq_dac_decode_ex(aq_ctx *ctx, const aq_dac_stages *st, const int32_t *idx, int64_t idx_ld, int64_t M,
                           float *out, int accumulate) {
    if (!ctx || !st || (M > 0 && (!idx || !out))) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_dac_decode: null argument");
    if (M < 0) return aq_fail(ctx, AQ_E_SHAPE, "aq_dac_decode: negative M");
    if (idx_ld < st->Q) return aq_fail(ctx, AQ_E_SHAPE, "aq_dac_decode: idx_ld must be at least Q");
    if (M == 0) return AQ_OK;
    if (!st->d_tables) return aq_fail(ctx, AQ_E_INVALID_ARG, "aq_dac_decode: no out-projection was uploaded");
    aq_device_guard g(ctx->device);
    AQ_HIP(ctx, hipMemsetAsync(ctx->d_flags, 0, sizeof(int32_t) * AQ_FLAG_COUNT, ctx->stream));
    const int64_t total = M * st->D;
    hipLaunchKernelGGL(dac_decode_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, ctx->stream, idx,
                       idx_ld, M, static_cast<int>(st->Q), st->N, st->D, st->d_tables, out, ctx->d_flags,
                       accumulate ? 1 : 0);
    AQ_HIP(ctx, hipGetLastError());
    int32_t flag = 0;
    AQ_HIP(ctx, hipMemcpyAsync(&flag, ctx->d_flags + AQ_FLAG_BAD_INDEX, sizeof(int32_t), hipMemcpyDeviceToHost, ctx->stream));
    AQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (flag) return aq_fail(ctx, AQ_E_INDEX_RANGE, "aq_dac_decode: code outside [0, %lld)", (long long)st->N);
    return AQ_OK;
}

}  // extern "C"
