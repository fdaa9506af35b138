// Euclidean VQ / RVQ kernels for gfx950, shared by the per-width translation
// units (aq_euclid_ks*.hip) and the host code (aq_euclid.hip).
//
// Euclidean VQ / RVQ encode on gfx950: nearest codeword by fp16 MFMA
// distance contraction, a per-lane top-L epilogue, a rigorous error
// certificate, and exact re-ranking in the reference recipe's own fp32
// arithmetic.  Also the codebook gather and the multi-stage decode sum.
//
// Reference recipes (paths relative to the audio.cpp tree):
//   OMNIVOICE  score weight 2c, bias -(double)|c|^2 cast to float
//              (src/models/omnivoice/audio_tokenizer.cpp:1227-1237); logits =
//              mul_mat(2c, r) + bias; ggml_argmax; get_rows; r -= c[code]
//              (audio_tokenizer.cpp:1897-1927)
//   HIGGS      logits = ((2 * mul_mat(c, r)) - sum_rows(r*r)) - sum_rows(c*c)
//              (src/models/higgs_audio_tts/codec.cpp:975-1013), F32 or Q8_0
//              codebook (a Q8_0 mul_mat quantises r to Q8_0 first)
//   DIRECT     distance = sum_k (x_k - c_k)^2, rounded products added in
//              order, first index of the minimum: VectorQuantizer::compute
//              (src/framework/runtime/host_ops.cpp:236-273) and Qwen3
//              nearest_code (src/models/qwen3_tts/tokenizer_speech_encoder.cpp:287-303)
// on the ggml CPU arithmetic (external/ggml/src/ggml-cpu): tinyBLAS F32
// (llamafile/sgemm.cpp:523-580: 16 FMA lanes, then _mm512_reduce_add_ps),
// ggml_vec_dot_f32 (vec.cpp:11-135) when tinyBLAS declines, tinyBLAS_Q0 /
// ggml_vec_dot_q8_0_q8_0 (sgemm.cpp:1353-, arch/x86/quants.c:1170-), x86
// quantize_row_q8_0 (arch/x86/quants.c:302-), ggml_vec_sum_f32 (vec.h, double
// accumulation), ggml_vec_argmax_f32 (vec.h:1576-1584, last index of the max).
//
// Design
//  * Scores: v(n) = x~ . c~_n - |c_n|^2/2 with x~, c~ rounded to fp16, from
//    v_mfma_f32_16x16x32_f16 with codes as A and frames as B.  Each wave
//    keeps FG groups of 16 frames of x~ in registers for the whole sweep over
//    the codebook, which streams through double-buffered, XOR-swizzled LDS
//    (conflict-free 16-byte reads).  Output lane l owns frame l%16 and codes
//    4*(l/16)+i of each 16-code block.
//  * Epilogue per score: key = v with the lane-local code index in the low
//    mantissa bits; the lane keeps its TOPL best keys (one max + med3 per
//    level).  The full score matrix never leaves the CU.
//  * Certificate: for every code, |v(n) - S'(n)| <= E, where S' is the
//    recipe's value (ggml's fp32 arithmetic) in the same units.  E is built
//    from the actual rounding residuals (|x~| |c~_n - c_n| + |x~ - x| |c_n|,
//    Cauchy-Schwarz), the fp32 accumulation bounds and the key truncation.
//    Kept candidates that could still be in the top T are re-ranked exactly;
//    the result is certified when the T-th exact value beats every unkept
//    code's bound.  Otherwise the frame is scored again with split fp16
//    operands (a bound about 2^-11 of the first) and, if that certificate
//    fails too, by an exact full scan, so results never depend on fp16
//    rounding.  A few open frames (up to the exact scan's spread capacity)
//    skip the split pass and go to the exact scan at once.
//  * Residual cascade: per stage the sweep, the select (re-rank, update
//    r -= c), the refine pair and the exact scan; the last three exit at
//    once when no frame is left for them.
#pragma once

#include "aq_internal.hpp"

#include <cmath>
#include <cstdint>

namespace aq_euclid {

constexpr int kWave = 64;
constexpr int kWaves = 4;
constexpr int kThreads = kWave * kWaves;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Matrix-core operand type of the sweep and the refine pass: fp16.  Its
// 11-bit mantissa makes the certificate's bound 8x tighter than bf16's
// (about 30x fewer frames left open on Mimi-shaped data; Q8_0's dequantised
// codes q * d carry up to 18 significant bits, and top-4 needs the 4th/5th
// gap), at the same matrix-core rate.  The matrix cores keep fp16 subnormal
// inputs, so the images' rounding errors, which the bounds measure, are the
// errors the products see.  Values beyond fp16's range become infinite:
// such a frame fails its certificate and is scanned exactly, and a codebook
// with such an entry is scanned exactly for every frame.
struct Mx {
    using E = _Float16;
    using V8 = f16x8;
    typedef _Float16 V2 __attribute__((ext_vector_type(2)));
    __device__ static f32x4 mfma(V8 a, V8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
    // the two values of a packed pair as fp32
    __device__ static float lo(unsigned w) { return static_cast<float>(__builtin_bit_cast(V2, w)[0]); }
    __device__ static float hi(unsigned w) { return static_cast<float>(__builtin_bit_cast(V2, w)[1]); }
};

enum Recipe : int { OMNI = 0, HIGGS = 1, DIRECT = 2 };

constexpr int kRS = 256;       // most codes per refine slice (64 per lane: 6 index bits)
constexpr int kTopR = 4;       // keys per lane and slice
constexpr int kRCand = 256;    // exact candidates per frame in refine_select
constexpr int kRKeyLds = 1024; // keys per frame refine_select stages in LDS
constexpr int kRWaves = 4;     // refine_values waves per block

template <int KS>
struct Tile {
    static constexpr int K = KS * 32;
    static constexpr int ROWB = K * 2;                         // bytes per fp16 code row
    static constexpr int CH16 = K / 8;                         // 16-byte chunks per row
    static constexpr int SWZ = CH16 >= 16 ? 15 : CH16 - 1;     // XOR swizzle mask
    static constexpr int CC = (32768 / ROWB) >= 16 ? ((32768 / ROWB) / 16) * 16 : 16;   // codes per LDS chunk
    static constexpr int CHUNKB = CC * ROWB;                   // codebook bytes per chunk
    static constexpr int BUFB = CHUNKB + kThreads * 4;         // + |c|^2/2 of the chunk (one slot per thread)
    static constexpr int STAGE16 = CHUNKB / 16 / kThreads;     // 16-byte loads per thread per chunk
    static constexpr int LDS = 2 * BUFB;
};

// The byte offsets, within a codebook chunk, of a thread's 16-byte staging
// pieces: piece k of thread t is row r = (t + THREADS k) / CH16, 16-byte
// column ((t + THREADS k) % CH16) ^ (r & SWZ).  Where THREADS is a multiple
// of CH16 and the rows per piece index (RPK) and the swizzle period divide
// one another, piece k's offset is k RPK ROWB (uniform) plus one of NVO
// per-thread values, which is all a thread keeps (the general form holds an
// address per piece across the sweep).
template <typename T, int THREADS>
struct StageOffsets {
    static constexpr int RPK0 = THREADS / T::CH16;
    static constexpr bool kAffine = THREADS % T::CH16 == 0 &&
                                    ((T::SWZ + 1) % RPK0 == 0 || RPK0 % (T::SWZ + 1) == 0);
    static constexpr int RPK = kAffine ? RPK0 : 1;
    static constexpr int NVO = kAffine && T::SWZ + 1 > RPK ? (T::SWZ + 1) / RPK : 1;
    unsigned v[NVO];
    __device__ StageOffsets() {
        if constexpr (kAffine) {
            const int br = threadIdx.x / T::CH16, c16 = threadIdx.x % T::CH16;
#pragma unroll
            for (int i = 0; i < NVO; ++i) v[i] = br * T::ROWB + 16 * (c16 ^ ((br + RPK * i) & T::SWZ));
        }
    }
    // piece k's offset = uni(k) (the same for every thread) + lane(k)
    __device__ int uni(int k) const { return kAffine ? k * RPK * T::ROWB : 0; }
    __device__ unsigned lane(int k) const {
        if constexpr (kAffine) {
            return v[k % NVO];
        } else {
            const int q = threadIdx.x + k * THREADS;
            const int r = q / T::CH16, j = (q % T::CH16) ^ (r & T::SWZ);
            return static_cast<unsigned>(r * T::ROWB + j * 16);
        }
    }
};

struct StageArgs {
    const float *xin;        // [M, K] residual entering the stage
    float *xout;             // [M, K] residual leaving the stage (may alias xin; null: not needed)
    int64_t M;
    int N;
    const uint16_t *cbh;     // [N, K] fp16 codebook (scores)
    const float *nhh;        // [N] -|c|^2 / 2 (the score accumulators start from it)
    const float *cbf;        // [N, K] fp32 codebook (dequantised for Q8_0)
    const float *bias;       // [N] OmniVoice score bias
    const float *e2;         // [N] Higgs sum_rows(c*c)
    const int8_t *q8;        // [N, K] Q8_0 quants
    const float *q8d;        // [N, K/32] Q8_0 scales (fp32 of fp16)
    float cmax, dcmax, chmax;   // max |c_n|, max |c~_n - c_n|, max |c~_n|
    int order;               // exact dot order: 0 tinyBLAS, 1 ggml_vec_dot_f32
    int Q, s;
    int32_t *idx;            // [M, Q]
    float *dist;             // [M, Q] or null
    int topk;                // 0..4
    int32_t *topk_idx;       // [M, Q, topk]
    float *topk_dist;        // [M, Q, topk]
    const int32_t *force_idx;   // [M, Q] or null
    int32_t *fail_count;     // this stage's counter
    int32_t *fail_list;      // [M]
    int32_t *spec_count;     // speculative (frame, stage) pairs listed (cascade)
    int32_t *spec_list;      // [2 * M * Q] the pairs, for the exact verification
    int misspeculate;        // test hook (cascade): every frame speculates, on a wrong code (1) or with
                             // its best code and perturbed distances (2)
    int32_t *flags;
    int exact_only;
    float *keys;             // sweep -> select: [nsplit][M/16][TOPL][64] score keys
    float *norms;            // sweep -> select: [3][M] |x~|^2, |x - x~|^2, |x|^2
    int nsplit;              // code splits of the sweep (tiles before tile2)
    int nsplit2;             // code splits of the tiles from tile2 on (a finer last round)
    int64_t tile2;           // first tile of the second part (a multiple of 8)
    float *svals;            // [scap, N] exact values of the scanned frames, by list slot
    int scap;                // frames whose values the exact scan spreads over its grid
    int32_t *slot_done;      // [scap] chunks done per slot (zero between stages)
    const int32_t *open_count;   // exact scan: the frames the select left open (null: not known)
    int K;                   // codebook width (read by the any-width exact scan, KS = 0)
};

struct RefArgs {
    const uint16_t *cbl;       // [N, K] fp16(c - fp16(c))
    float *keys;               // [cap][nslices][4][kTopR] (RefShape)
    int64_t key_floats;        // capacity of the key buffer
    int32_t *count2;           // exact-scan counter of this stage
    int32_t *list2;            // exact-scan frame list
    float clmax, crmax;        // max |c_l|, max |c_r| over the stage's codes
};

// Slicing of the refine pass, chosen on the device from the number of open
// frames (both refine kernels derive the same shape): a few hundred open
// frames of a codebook of up to kRSmallCodes codes fill the GPU only with
// short slices (kRSSmall codes, two 16-code blocks per work item), when the
// key buffer holds their keys; many open frames, or larger codebooks, take
// long slices (kRS codes), which keep the per-item set-up and the keys per
// frame low (short slices for 1 300 open Q8_0 frames measured 30 % slower;
// up to kRMidFrames take kRSMid-code slices).
// Frames past the key buffer's capacity go to the exact scan.
constexpr int kRSSmall = 32;
constexpr int kRSmallFrames = 512;
constexpr int kRSMid = 128;         // middle slices: up to kRMidFrames open frames
constexpr int kRMidFrames = 4096;
constexpr int kRSmallCodes = 4096;
struct RefShape {
    int rs, nslices, cap;
};
__device__ inline RefShape ref_shape(const RefArgs &rf, int N, int count) {
    RefShape r;
    auto fits = [&](int rs) { return static_cast<int64_t>((N + rs - 1) / rs) * 4 * kTopR * count <= rf.key_floats; };
    if (count <= kRSmallFrames && N <= kRSmallCodes && fits(kRSSmall)) r.rs = kRSSmall;
    else if (count <= kRMidFrames && fits(kRSMid)) r.rs = kRSMid;
    else r.rs = kRS;
    r.nslices = (N + r.rs - 1) / r.rs;
    const int64_t cap = rf.key_floats / (static_cast<int64_t>(r.nslices) * 4 * kTopR);
    r.cap = static_cast<int>(cap < count ? cap : count);
    return r;
}

// The whole residual cascade in one launch (euclid_cascade_kernel): per
// stage s the kernel takes `a` with the stage's codebook pointers
// (cbh / nhh / cbf / bias / e2 / q8 / q8d advanced by s codebooks), bounds
// (bounds[3 s .. 3 s + 2] = max |c|, max |c~ - c|, max |c~|), xin = x0 at
// stage 0 and the residual buffer after, xout = the residual buffer.
struct CascadeArgs {
    StageArgs a;             // stage 0's pointers; spec_count / spec_list set
    const float *x0;         // [M, K] stage 0's input (frame-major; kept for the verification)
    float *work;             // [M, K] the residual
    const float *bounds;     // [Q][3] certificate bounds per stage
    int32_t *counts;         // [128]: [0, 64) frames speculated per stage, [64, 128) frames the fix-up recomputed
    int32_t *bad_stage;      // [M] the earliest stage whose speculation was wrong (Q: none)
    int32_t *bad_count;      // frames listed in bad_list
    int32_t *bad_list;       // [M]
    int write_last;          // the last stage writes the residual
};

using StageFn = void (*)(StageArgs);
using RefineFn = void (*)(StageArgs, RefArgs);
using CascadeFn = void (*)(CascadeArgs);

// 16-frame groups per sweep wave: the fp16 frames of a wave stay in
// registers (4 * KS registers per group), so wider codebooks take fewer;
// K = 768 takes three again, its fragments partly in AGPRs (one wave per
// SIMD), for one A-fragment read per three MFMAs.
constexpr int groups_for(int ks) { return ks <= 2 ? 4 : (ks <= 8 ? 3 : (ks <= 16 ? 2 : 3)); }
// Sweep blocks resident per CU (the launch bound the register budget follows).
constexpr int sweep_blocks_per_cu(int ks) { return ks <= 8 ? 2 : 1; }
// LDS chunk buffers of the sweep: two where two blocks share a CU; four for
// one block per CU, so that a chunk's codebook loads are issued two chunks
// before it is read (a chunk of the widest codebooks is a single 16-code
// block, too short to hide a global load behind).
constexpr int sweep_buffers(int ks) { return sweep_blocks_per_cu(ks) == 1 ? 4 : 2; }
template <int KS>
constexpr int sweep_lds_bytes() { return sweep_buffers(KS) * Tile<KS>::BUFB; }

// Kernels of one codebook width (K = 32 * KS), built in their own
// translation unit (aq_euclid_ks<KS>.hip).  Recipe variants: 0 OmniVoice,
// 1 Higgs, 2 direct, 3 Higgs with a Q8_0 codebook.  [.][0] keeps 3 keys per
// lane, [.][1] keeps 4.
struct KsKernels {
    StageFn sweep[2][2];      // [q8][topl]
    StageFn select[4][2];     // [variant][topl]
    RefineFn refine_values[4];
    RefineFn refine_select[4];
    StageFn exact_scan[4];
    int lds;                  // sweep dynamic LDS bytes
    int cc;                   // codes per LDS chunk
    // One-launch cascade (widths whose frame tiles keep two waves per SIMD;
    // null otherwise), its verification and fix-up.
    CascadeFn cascade[4][2];  // [variant][topl]
    CascadeFn verify[4];
    CascadeFn verify_values[4];
    CascadeFn fixup[4];
    int cascade_lds;          // cascade dynamic LDS bytes (TOPL 4)
    int cascade_frames;       // frames per cascade block
    // The register-resident cascade (the widths whose residual fits the
    // registers; null otherwise).
    CascadeFn resident[4][2]; // [variant][topl]
    int resident_lds;         // its dynamic LDS bytes (TOPL 4)
    int resident_frames;      // frames per block
};
const KsKernels *kernels_ks2();
const KsKernels *kernels_ks8();
const KsKernels *kernels_ks16();
const KsKernels *kernels_ks24();

// The exact scan at a run-time width (any K; K % 32 == 0 for Q8_0), built in
// aq_euclid_any.hip: codebooks outside the fast widths and tile sizes scan
// every frame exactly in the recipe's arithmetic.  Variants as KsKernels.
struct AnyKernels {
    StageFn exact_scan[4];
};
const AnyKernels *kernels_any();
// Dynamic LDS of the exact scan: the frame (K floats), its Q8_0 quants (K
// bytes) and scales (K / 32 floats).
constexpr size_t scan_lds_bytes(int64_t K) { return static_cast<size_t>(K) * 5 + static_cast<size_t>(K / 32) * 4 + 64; }

}  // namespace aq_euclid

namespace {

using namespace aq_euclid;




// --------------------------------------------------------------- exact math

// _mm512_reduce_add_ps order (pairs 8, 4, 2, 1).
__device__ inline float reduce16(const float (&a)[16]) {
    float t3[8], t6[4];
#pragma unroll
    for (int i = 0; i < 8; ++i) t3[i] = __fadd_rn(a[i + 8], a[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) t6[i] = __fadd_rn(t3[i + 4], t3[i]);
    const float t80 = __fadd_rn(t6[0], t6[2]);
    const float t81 = __fadd_rn(t6[1], t6[3]);
    return __fadd_rn(t80, t81);
}

// hsum of 8 lanes (hsum(__m256) / hsum_float_8): i+4, then 2, then 1.
__device__ inline float reduce8(const float (&a)[8]) {
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __fadd_rn(a[i + 4], a[i]);
    return __fadd_rn(__fadd_rn(v[0], v[2]), __fadd_rn(v[1], v[3]));
}

// One tinyBLAS<16> element: sa*a . b with 16 FMA accumulators over k = 16l + j.
// sa is 1 or 2 (exact scaling, OmniVoice's 2c).
__device__ float dot_tinyblas(const float *__restrict__ a, const float *__restrict__ b, int K, float sa) {
    float acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
    for (int l = 0; l < K; l += 16) {
        const f32x4 *pa = reinterpret_cast<const f32x4 *>(a + l);
        const f32x4 *pb = reinterpret_cast<const f32x4 *>(b + l);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const f32x4 va = pa[q], vb = pb[q];
#pragma unroll
            for (int t = 0; t < 4; ++t) acc[4 * q + t] = __fmaf_rn(va[t] * sa, vb[t], acc[4 * q + t]);
        }
    }
    return reduce16(acc);
}

// ggml_vec_dot_f32, AVX-512 branch: 4 x 16 accumulators over 64-element
// steps, combined 0+=2, 1+=3, 0+=1, reduced, then the scalar leftovers.
__device__ float dot_vecdot(const float *__restrict__ a, const float *__restrict__ b, int K, float sa) {
    float s[4][16];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int l = 0; l < 16; ++l) s[j][l] = 0.0f;
    const int np = K & ~63;
    for (int i = 0; i < np; i += 64) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int l = 0; l < 16; ++l) s[j][l] = __fmaf_rn(a[i + 16 * j + l] * sa, b[i + 16 * j + l], s[j][l]);
    }
    float r[16];
#pragma unroll
    for (int l = 0; l < 16; ++l) r[l] = __fadd_rn(__fadd_rn(s[0][l], s[2][l]), __fadd_rn(s[1][l], s[3][l]));
    float sum = reduce16(r);
    // The leftover loop `sumf += x[i]*y[i]` as GCC 11 compiles it for the
    // reference's native AVX-512 build: the products of the first
    // rem - rem % 4 leftovers rounded and added in order, the last rem % 4
    // fused (vec.cpp:125-128).
    const int fused_from = K - (K - np) % 4;
    for (int i = np; i < K; ++i)
        sum = i >= fused_from ? __fmaf_rn(a[i] * sa, b[i], sum) : __fadd_rn(sum, __fmul_rn(a[i] * sa, b[i]));
    return sum;
}

// Direct squared distance: rounded (x - c)^2 added in order.
__device__ float dist_direct(const float *__restrict__ x, const float *__restrict__ c, int K) {
    float d = 0.0f;
    for (int k = 0; k < K; ++k) {
        const float diff = __fsub_rn(x[k], c[k]);
        d = __fadd_rn(d, __fmul_rn(diff, diff));
    }
    return d;
}

// x86 quantize_row_q8_0 on one 32-element block: d = amax/127 stored as fp16,
// id = 127/amax, q = round-half-even(x*id) with int8 saturation.
// One quant of x86 quantize_row_q8_0: round half to even of x * id (the
// conversion of _mm256_cvtps_epi32, whose out-of-range result packs to -128),
// saturated to int8 by the packs.
__device__ inline int q8_quant(float x, float id) {
    const float v = __builtin_rintf(__fmul_rn(x, id));
    if (!(v >= -2147483648.0f && v < 2147483648.0f)) return -128;
    const int qi = static_cast<int>(v);
    return qi < -128 ? -128 : (qi > 127 ? 127 : qi);
}
// The block's scale d = fp16(amax / 127) (as fp32) and 127 / amax.
__device__ inline void q8_scale(float amax, float &d, float &id) {
    d = static_cast<float>(static_cast<_Float16>(__fdiv_rn(amax, 127.0f)));
    id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
}
// Four quants in [-128, 127] packed into a dword, first in the low byte
// (two saturating 16-bit packs, then a byte select).
__device__ inline int q8_pack4(int q0, int q1, int q2, int q3) {
    const auto lo = __builtin_amdgcn_cvt_pk_i16(q0, q1);
    const auto hi = __builtin_amdgcn_cvt_pk_i16(q2, q3);
    return static_cast<int>(__builtin_amdgcn_perm(__builtin_bit_cast(unsigned, hi), __builtin_bit_cast(unsigned, lo),
                                                  0x06040200u));
}
__device__ inline void quantize_block_q8(const float *__restrict__ x, int8_t *__restrict__ q, float *__restrict__ d) {
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[j]));
    float id;
    q8_scale(amax, *d, id);
    for (int j = 0; j < 32; ++j) q[j] = static_cast<int8_t>(q8_quant(x[j], id));
}

// tinyBLAS_Q0 / ggml_vec_dot_q8_0_q8_0: per block, 8 exact 4-element int
// dots scaled by d_c*d_x and accumulated with FMA, then an 8-lane hsum.
__device__ float dot_q8(const int8_t *__restrict__ qc, const float *__restrict__ dc, const int8_t *__restrict__ qx,
                        const float *__restrict__ dx, int nb) {
    float acc[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
    for (int ib = 0; ib < nb; ++ib) {
        const float dd = __fmul_rn(dc[ib], dx[ib]);
        // the code's 32 quants as two 16-byte loads (rows are 32-byte aligned)
        const u32x4 *pc = reinterpret_cast<const u32x4 *>(qc + 32 * ib);
        const u32x4 c0 = pc[0], c1 = pc[1];
        const int cw[8] = {static_cast<int>(c0[0]), static_cast<int>(c0[1]), static_cast<int>(c0[2]),
                           static_cast<int>(c0[3]), static_cast<int>(c1[0]), static_cast<int>(c1[1]),
                           static_cast<int>(c1[2]), static_cast<int>(c1[3])};
        const int *px = reinterpret_cast<const int *>(qx + 32 * ib);
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            const int s = __builtin_amdgcn_sdot4(cw[l], px[l], 0, false);
            acc[l] = __fmaf_rn(dd, static_cast<float>(s), acc[l]);
        }
    }
    return reduce8(acc);
}

// dot_q8 for a compile-time width: the code row's quants are loaded four
// blocks (128 bytes) at a time before any of them is used, so a code costs
// K / 128 memory round trips instead of K / 32.
template <int K>
__device__ float dot_q8_k(const int8_t *__restrict__ qc, const float *__restrict__ dc, const int8_t *__restrict__ qx,
                          const float *__restrict__ dx) {
    constexpr int NB = K / 32;
    constexpr int G = NB < 4 ? NB : 4;
    static_assert(NB % G == 0, "blocks per group");
    float acc[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
    const u32x4 *pc = reinterpret_cast<const u32x4 *>(qc);
#pragma unroll
    for (int b0 = 0; b0 < NB; b0 += G) {
        u32x4 c[2 * G];
        float d[G];
#pragma unroll
        for (int j = 0; j < 2 * G; ++j) c[j] = pc[2 * b0 + j];
#pragma unroll
        for (int j = 0; j < G; ++j) d[j] = dc[b0 + j];
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const int ib = b0 + j;
            const float dd = __fmul_rn(d[j], dx[ib]);
            const int *px = reinterpret_cast<const int *>(qx + 32 * ib);
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                const int cw = static_cast<int>(c[2 * j + l / 4][l % 4]);
                acc[l] = __fmaf_rn(dd, static_cast<float>(__builtin_amdgcn_sdot4(cw, px[l], 0, false)), acc[l]);
            }
        }
    }
    return reduce8(acc);
}

// Compile-time-K forms for the stage kernel: the loops unroll, so the loads
// of later steps are issued ahead of the FMA chains that consume them.
template <int K>
__device__ float dot_tinyblas_k(const float *__restrict__ a, const float *__restrict__ b, float sa) {
    float acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
#pragma unroll 4
    for (int l = 0; l < K; l += 16) {
        const f32x4 *pa = reinterpret_cast<const f32x4 *>(a + l);
        const f32x4 *pb = reinterpret_cast<const f32x4 *>(b + l);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const f32x4 va = pa[q], vb = pb[q];
#pragma unroll
            for (int t = 0; t < 4; ++t) acc[4 * q + t] = __fmaf_rn(va[t] * sa, vb[t], acc[4 * q + t]);
        }
    }
    return reduce16(acc);
}

// ggml_vec_sum_f32 of the fp32 squares (sum_rows(mul(x, x))): double
// accumulation in order, one rounding to float.
template <int K>
__device__ float sum_squares_k(const float *__restrict__ x) {
    double s = 0.0;
#pragma unroll 8
    for (int k = 0; k < K; k += 4) {
        const f32x4 v = *reinterpret_cast<const f32x4 *>(x + k);
#pragma unroll
        for (int t = 0; t < 4; ++t) s += static_cast<double>(__fmul_rn(v[t], v[t]));
    }
    return static_cast<float>(s);
}

template <int K>
__device__ float dist_direct_k(const float *__restrict__ x, const float *__restrict__ c) {
    float d = 0.0f;
#pragma unroll 4
    for (int k = 0; k < K; k += 4) {
        const f32x4 xv = *reinterpret_cast<const f32x4 *>(x + k);
        const f32x4 cv = *reinterpret_cast<const f32x4 *>(c + k);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float diff = __fsub_rn(xv[t], cv[t]);
            d = __fadd_rn(d, __fmul_rn(diff, diff));
        }
    }
    return d;
}

// dot_q8 with the query block quantised on the fly (quantize_block_q8's
// arithmetic, block by block), so no per-lane copy of the quantised row.
template <int K>
__device__ float dot_q8_fused(const int8_t *__restrict__ qc, const float *__restrict__ dc, const float *__restrict__ x) {
    float acc[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
#pragma unroll 2
    for (int ib = 0; ib < K / 32; ++ib) {
        float v[32];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const f32x4 t = *reinterpret_cast<const f32x4 *>(x + 32 * ib + 4 * q);
            v[4 * q] = t[0]; v[4 * q + 1] = t[1]; v[4 * q + 2] = t[2]; v[4 * q + 3] = t[3];
        }
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
        const float dx = static_cast<float>(static_cast<_Float16>(__fdiv_rn(amax, 127.0f)));
        const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
        int qw[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            unsigned w = 0;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float r = __builtin_rintf(__fmul_rn(v[4 * l + t], id));
                int qi;
                if (!(r >= -2147483648.0f && r < 2147483648.0f)) qi = -128;
                else qi = static_cast<int>(r) < -128 ? -128 : (static_cast<int>(r) > 127 ? 127 : static_cast<int>(r));
                w |= (static_cast<unsigned>(qi) & 0xFFu) << (8 * t);
            }
            qw[l] = static_cast<int>(w);
        }
        const float dd = __fmul_rn(dc[ib], dx);
        const u32x4 *pc = reinterpret_cast<const u32x4 *>(qc + 32 * ib);
        const u32x4 c0 = pc[0], c1 = pc[1];
        const int cw[8] = {static_cast<int>(c0[0]), static_cast<int>(c0[1]), static_cast<int>(c0[2]),
                           static_cast<int>(c0[3]), static_cast<int>(c1[0]), static_cast<int>(c1[1]),
                           static_cast<int>(c1[2]), static_cast<int>(c1[3])};
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            const int s = __builtin_amdgcn_sdot4(cw[l], qw[l], 0, false);
            acc[l] = __fmaf_rn(dd, static_cast<float>(s), acc[l]);
        }
    }
    return reduce8(acc);
}

template <int RECIPE, bool Q8, int K>
__device__ float exact_value_k(const StageArgs &a, const float *__restrict__ x, int n, float x2) {
    const float *c = a.cbf + static_cast<int64_t>(n) * K;
    if (RECIPE == DIRECT) return dist_direct_k<K>(x, c);
    float dot;
    if (Q8) {
        dot = dot_q8_fused<K>(a.q8 + static_cast<int64_t>(n) * K, a.q8d + static_cast<int64_t>(n) * (K / 32), x);
    } else {
        const float sa = RECIPE == OMNI ? 2.0f : 1.0f;
        dot = a.order == 0 ? dot_tinyblas_k<K>(c, x, sa) : dot_vecdot(c, x, K, sa);
    }
    if (RECIPE == OMNI) return __fadd_rn(dot, a.bias[n]);
    return __fsub_rn(__fsub_rn(__fmul_rn(dot, 2.0f), x2), a.e2[n]);
}

// exact_value_k with the query's Q8_0 blocks already quantised (xq, xd).
template <int RECIPE, bool Q8, int K>
__device__ float exact_value_kq(const StageArgs &a, const float *__restrict__ x, int n, float x2,
                                const int8_t *__restrict__ xq, const float *__restrict__ xd) {
    if (!Q8) return exact_value_k<RECIPE, Q8, K>(a, x, n, x2);
    const float dot = dot_q8_k<K>(a.q8 + static_cast<int64_t>(n) * K, a.q8d + static_cast<int64_t>(n) * (K / 32), xq, xd);
    return __fsub_rn(__fsub_rn(__fmul_rn(dot, 2.0f), x2), a.e2[n]);
}

// Recipe value of code n ("larger is better" for OMNI/HIGGS: the logit;
// DIRECT returns the distance, smaller is better).  x2 is sum_rows(x*x)
// (HIGGS); xq/xd the quantised query (HIGGS with a Q8_0 codebook).
template <int RECIPE, bool Q8>
__device__ float exact_value(const StageArgs &a, int K, const float *__restrict__ x, int n, float x2,
                             const int8_t *xq, const float *xd) {
    const float *c = a.cbf + static_cast<int64_t>(n) * K;
    if (RECIPE == DIRECT) return dist_direct(x, c, K);
    float dot;
    if (Q8) {
        dot = dot_q8(a.q8 + static_cast<int64_t>(n) * K, a.q8d + static_cast<int64_t>(n) * (K / 32), xq, xd, K / 32);
    } else {
        const float sa = RECIPE == OMNI ? 2.0f : 1.0f;
        dot = a.order == 0 ? dot_tinyblas(c, x, K, sa) : dot_vecdot(c, x, K, sa);
    }
    if (RECIPE == OMNI) return __fadd_rn(dot, a.bias[n]);
    return __fsub_rn(__fsub_rn(__fmul_rn(dot, 2.0f), x2), a.e2[n]);
}

// True if (va, na) ranks before (vb, nb): ggml recipes take the larger logit
// and, on equality, the larger index (argmax keeps the last maximum);
// DIRECT takes the smaller distance and, on equality, the smaller index.
template <int RECIPE>
__device__ inline bool ranks_before(float va, int na, float vb, int nb) {
    if (RECIPE == DIRECT) return va < vb || (va == vb && na < nb);
    return va > vb || (va == vb && na > nb);
}
// Top-k order for ggml recipes (a set in ggml): value desc, index asc.
template <int RECIPE>
__device__ inline bool topk_before(float va, int na, float vb, int nb) {
    if (RECIPE == DIRECT) return va < vb || (va == vb && na < nb);
    return va > vb || (va == vb && na < nb);
}

// (va, na) before (vb, nb) in top-k order, an empty place (n < 0) last.
template <int RECIPE>
__device__ inline bool topk_first(float va, int na, float vb, int nb) {
    return na >= 0 && (nb < 0 || topk_before<RECIPE>(va, na, vb, nb));
}
// Compare-exchange of places i < k of a ranked list.
template <int RECIPE>
__device__ inline void topk_cx(float (&v)[5], int (&n)[5], int i, int k) {
    const bool s = topk_first<RECIPE>(v[k], n[k], v[i], n[i]);
    const float vi = v[i], vk = v[k];
    const int ni = n[i], nk = n[k];
    v[i] = s ? vk : vi;
    n[i] = s ? nk : ni;
    v[k] = s ? vi : vk;
    n[k] = s ? ni : nk;
}
// x of the lane in the partner row (row r ^ X, X = 1 or 2) of the lane's
// column, by one gfx950 lane swap (kq: the lane's row).
template <int X>
__device__ inline unsigned row_partner(unsigned x, int kq) {
    if constexpr (X == 1) {
        const auto ab = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        return (kq & 1) ? ab[0] : ab[1];
    } else {
        const auto ab = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        return (kq & 2) ? ab[0] : ab[1];
    }
}
// The better (ranks_before; an empty place, n < 0, last) of the lane's
// candidate and its partner row's.
template <int RECIPE, int X>
__device__ inline void best_rows(float &v, int &n, int kq) {
    const float pv = __uint_as_float(row_partner<X>(__float_as_uint(v), kq));
    const int pn = static_cast<int>(row_partner<X>(static_cast<unsigned>(n), kq));
    const bool s = pn >= 0 && (n < 0 || ranks_before<RECIPE>(pv, pn, v, n));
    v = s ? pv : v;
    n = s ? pn : n;
}
// The top 5 of the union of the lane's ranked list of 5 and its partner
// row's (disjoint codes): the better of L_i and R_{4-i} gives the union's
// top 5 (the first half of a bitonic merge), which a 5-input sorting
// network (9 compare-exchanges) ranks.  Both partners end with the same list.
template <int RECIPE, int X>
__device__ inline void merge_rows5(float (&v)[5], int (&n)[5], int kq) {
    float pv[5];
    int pn[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) {
        pv[i] = __uint_as_float(row_partner<X>(__float_as_uint(v[i]), kq));
        pn[i] = static_cast<int>(row_partner<X>(static_cast<unsigned>(n[i]), kq));
    }
#pragma unroll
    for (int i = 0; i < 5; ++i) {
        const bool s = topk_first<RECIPE>(pv[4 - i], pn[4 - i], v[i], n[i]);
        v[i] = s ? pv[4 - i] : v[i];
        n[i] = s ? pn[4 - i] : n[i];
    }
    topk_cx<RECIPE>(v, n, 0, 1);
    topk_cx<RECIPE>(v, n, 3, 4);
    topk_cx<RECIPE>(v, n, 2, 4);
    topk_cx<RECIPE>(v, n, 2, 3);
    topk_cx<RECIPE>(v, n, 0, 3);
    topk_cx<RECIPE>(v, n, 0, 2);
    topk_cx<RECIPE>(v, n, 1, 4);
    topk_cx<RECIPE>(v, n, 1, 3);
    topk_cx<RECIPE>(v, n, 1, 2);
}

// --------------------------------------------------------------- score kernel

// v + v[lane rotated by N inside its 16-lane row] (DPP row_ror).  IEEE
// addition is commutative, so each lane's sum is the pair the reference adds.
template <int N>
__device__ inline float row_ror_add(float v) {
    const int o = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + N, 0xF, 0xF, false);
    return __fadd_rn(v, __int_as_float(o));
}

// ggml's hsum_float_8 ((a0+a4) + (a2+a6)) + ((a1+a5) + (a3+a7)) of eight
// accumulators held by 8 neighbouring lanes, lane j holding a_{q8_lane_word(j)}
// (words 0, 1, 2, 3, 7, 6, 5, 4): the half-row mirror pairs a_i with a_{i+4},
// the quad permutations [2,3,0,1] and [1,0,3,2] then add as the reference
// does (IEEE addition is commutative), all as DPP moves.  Lane 0 of the 8
// holds the sum.
__device__ inline int q8_lane_word(int j) { return j < 4 ? j : 11 - j; }
__device__ inline float hsum8_dpp(float a) {
    float v = __fadd_rn(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x141, 0xF, 0xF, false)));
    v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
    return __fadd_rn(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
}

// The values of x at the lane's column in each of the wave's four 16-lane
// rows (out[q] = x of lane col + 16 q), by three gfx950 lane-swap
// instructions instead of LDS permutes: permlane16_swap(x, x) gives rows
// (r & 2) and (r & 2) + 1 at a lane of row r, permlane32_swap of each then
// rows 0, 2 and 1, 3.
__device__ inline void rows4_u(unsigned x, unsigned (&out)[4]) {
    const auto ab = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    const auto a = __builtin_amdgcn_permlane32_swap(ab[0], ab[0], false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(ab[1], ab[1], false, false);
    out[0] = a[0];
    out[1] = b[0];
    out[2] = a[1];
    out[3] = b[1];
}
__device__ inline void rows4(float x, float (&out)[4]) {
    unsigned u[4];
    rows4_u(__float_as_uint(x), u);
#pragma unroll
    for (int q = 0; q < 4; ++q) out[q] = __uint_as_float(u[q]);
}
__device__ inline void rows4(int x, int (&out)[4]) {
    unsigned u[4];
    rows4_u(static_cast<unsigned>(x), u);
#pragma unroll
    for (int q = 0; q < 4; ++q) out[q] = static_cast<int>(u[q]);
}
__device__ inline double row_bcast(double x, int q) {
    unsigned lo[4], hi[4];
    const uint64_t b = __double_as_longlong(x);
    rows4_u(static_cast<unsigned>(b), lo);
    rows4_u(static_cast<unsigned>(b >> 32), hi);
    return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi[q]) << 32) | lo[q]));
}
// max and sum over the four rows (every lane of a column gets the same value)
__device__ inline float rows_max(float x) {
    float r[4];
    rows4(x, r);
    return fmaxf(fmaxf(r[0], r[1]), fmaxf(r[2], r[3]));
}
__device__ inline float rows_sum(float x) {
    float r[4];
    rows4(x, r);
    return (r[0] + r[1]) + (r[2] + r[3]);
}

// The query's Q8_0 image x_q = q * d of one 32-wide block (x86
// quantize_row_q8_0: d = fp16(amax/127), q = round-half-even(x * 127/amax)),
// held by 4 lanes 16 apart with 8 elements each.  x_q is exact in fp32
// (a 7-bit integer times an fp16 scale).
__device__ inline void q8_image_block(float (&v)[8]) {
    float am = 0.0f;
#pragma unroll
    for (int t = 0; t < 8; ++t) am = fmaxf(am, fabsf(v[t]));
    am = rows_max(am);
    const float dq = static_cast<float>(static_cast<_Float16>(__fdiv_rn(am, 127.0f)));
    const float id = am != 0.0f ? __fdiv_rn(127.0f, am) : 0.0f;
#pragma unroll
    for (int t = 0; t < 8; ++t) v[t] = __fmul_rn(__builtin_rintf(__fmul_rn(v[t], id)), dq);
}

// Score key: the score's bits with the low ones replaced by the lane-local
// code index.  `keep` is the complement of the index mask, held in a VGPR so
// that the bit select is one v_and_or_b32 with the (wave-uniform) index.
__device__ inline float key_of(float v, unsigned local, unsigned keep) {
    return __uint_as_float((__float_as_uint(v) & keep) | local);
}


// Sweep of one stage: every frame of a tile against the codes of one split.
// Up to K = 256 two blocks share a CU (256 VGPRs per lane at most), so the
// matrix pipe of a SIMD is fed by two waves; wider frames need the whole
// register file of one wave.  The frames' certificate and re-ranking run in
// the select kernel, at higher occupancy.
template <bool Q8, int KS, int FG, int TOPL>
__global__ __launch_bounds__(kThreads, sweep_blocks_per_cu(KS)) void euclid_sweep_kernel(StageArgs a) {
    using T = Tile<KS>;
    constexpr int K = T::K;
    static_assert(T::CHUNKB % (16 * kThreads) == 0, "chunk must split evenly over the block");
    extern __shared__ __align__(16) unsigned char lds[];

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int col = lane & 15;      // frame within a 16-frame group
    const int kq = lane >> 4;       // which 8-element quarter of each 32-wide K slice
    // Block order: the nsplit blocks of a frame tile have ids 8 apart, so
    // the round-robin dispatch over the 8 XCDs puts them on one XCD and the
    // second read of the tile's frames is served by that XCD's L2.  Tiles
    // from tile2 on (the grid's last, partial round) take nsplit2 splits
    // with the same order after the first part's blocks.  Ids past the last
    // tile (each part is a whole number of 8-tile groups) exit.
    int64_t bi = blockIdx.x;
    int nsp = a.nsplit;
    int64_t tbase = 0;
    if (bi >= a.tile2 * a.nsplit) {
        bi -= a.tile2 * a.nsplit;
        nsp = a.nsplit2;
        tbase = a.tile2;
    }
    const int per = 8 * nsp;
    const int split = static_cast<int>(bi % per) / 8;
    const int64_t tile = tbase + (bi / per) * 8 + (bi % per) % 8;
    if (tile * (kWaves * FG * 16) >= a.M) return;
    const int64_t m_base = (tile * kWaves + wave) * (FG * 16);
    const int N = a.N;
    const int cps = (N / T::CC) / nsp;   // chunks per split
    const int c0 = split * cps, c1 = c0 + cps;

    using MX = Mx;
    // ---- phase 0: frames -> fp16 fragments in registers, rounding norms ----
    // x~ fragments stay packed (2 fp16 per register) for the whole sweep.
    u32x4 xb[FG][KS];
    float nx2[FG], nd2[FG], nxx2[FG];
#pragma unroll
    for (int g = 0; g < FG; ++g) {
        const int64_t m = m_base + g * 16 + col;
        const int64_t mc = m < a.M ? m : a.M - 1;
        const float *xr = a.xin + mc * K;
        float sx = 0.0f, sd = 0.0f, sxx = 0.0f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const f32x4 lo = *reinterpret_cast<const f32x4 *>(xr + ks * 32 + kq * 8);
            const f32x4 hi = *reinterpret_cast<const f32x4 *>(xr + ks * 32 + kq * 8 + 4);
            float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            // A Q8_0 mul_mat scores the query's Q8_0 image x_q = q * d, so
            // the matrix cores contract fp16(x_q) and the bound only has to
            // cover fp16 rounding.
            if (Q8) q8_image_block(v);
            u32x4 packed;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const typename MX::V2 pr = {static_cast<typename MX::E>(v[2 * t]),
                                            static_cast<typename MX::E>(v[2 * t + 1])};
                const unsigned w = __builtin_bit_cast(unsigned, pr);
                packed[t] = w;
                const float r0 = MX::lo(w), r1 = MX::hi(w);
                sx = __fmaf_rn(r0, r0, sx);
                sx = __fmaf_rn(r1, r1, sx);
                const float d0 = v[2 * t] - r0, d1 = v[2 * t + 1] - r1;
                sd = __fmaf_rn(d0, d0, sd);
                sd = __fmaf_rn(d1, d1, sd);
                sxx = __fmaf_rn(v[2 * t], v[2 * t], sxx);
                sxx = __fmaf_rn(v[2 * t + 1], v[2 * t + 1], sxx);
            }
            xb[g][ks] = packed;
        }
        sx = rows_sum(sx);
        sd = rows_sum(sd);
        sxx = rows_sum(sxx);
        nx2[g] = sx;
        nd2[g] = sd;
        nxx2[g] = sxx;
    }

    // ---- phase 1: sweep the codebook ----
    float top[FG][TOPL];
#pragma unroll
    for (int g = 0; g < FG; ++g)
#pragma unroll
        for (int j = 0; j < TOPL; ++j) top[g][j] = -INFINITY;

    int lbits = 0;   // bits of the lane-local code index (N/4 codes per lane)
    while ((1 << lbits) < N / 4) ++lbits;
    const unsigned kmask = (1u << lbits) - 1u;
    unsigned vkeep;   // ~kmask in a VGPR (one scalar operand per VOP3 on gfx950)
    asm volatile("v_mov_b32 %0, %1" : "=v"(vkeep) : "s"(~kmask));

    // Software pipeline over 16-code blocks (chunk c holds blocks b = 0 ..
    // BPC-1; the block loop is unrolled so that a chunk is one basic block):
    //  * A fragments live in a ring of R registers, loaded L = R-1 K-slices
    //    ahead (across the block boundary inside a chunk); scheduling
    //    barriers between the slices keep the loads there;
    //  * each K-slice's MFMAs carry a share of the previous block's
    //    epilogue (the VALU work costs issue cycles of the SIMD either way;
    //    spread out, it waits on no MFMA result);
    //  * chunk c + NB - 1 is staged into the buffer chunk c - 1 left, a few
    //    16-byte pieces per block, straight from global memory to LDS
    //    (global_load_lds: no registers); at the chunk's end only chunk
    //    c + 1's loads are waited for, then one barrier.  Chunks past the
    //    last re-stage the last into the idle buffer, which keeps the loop
    //    free of branches.
    constexpr int NB = sweep_buffers(KS);
    constexpr int BPC = T::CC / 16;
    // ring depth: fewer frame groups per wave give fewer MFMAs per slice,
    // so the loads run more slices ahead; where one block holds a CU (no
    // second block's waves cover the LDS latency) eight slices ahead too
    // (K = 768: the sweep 1.5 % faster than with four)
    constexpr int R = KS % 4 != 0 ? 2 : (FG <= 2 || sweep_blocks_per_cu(KS) == 1 ? 8 : 4);
    constexpr int L = R - 1;
    constexpr int PPB = (T::STAGE16 + BPC - 1) / BPC;   // staged pieces per block

    auto lds_a = [&](int buf, int blk, int ks) -> typename MX::V8 {
        const int r = blk * 16 + col;
        const int j = ks * 4 + kq;
        return *reinterpret_cast<const typename MX::V8 *>(lds + buf * T::BUFB + r * T::ROWB + ((j ^ (r & T::SWZ)) * 16));
    };
    auto lds_h = [&](int buf, int blk) -> f32x4 {
        return *reinterpret_cast<const f32x4 *>(lds + buf * T::BUFB + T::CHUNKB + (blk * 16 + kq * 4) * 4);
    };
    // Every thread stages one |c|^2/2 slot (threads >= CC write a slot past
    // the chunk's, which nothing reads): no divergent branch.
    const int hsrc = threadIdx.x < T::CC ? threadIdx.x : 0;
    // Direct staging: the 16 bytes of lane l of wave w land at LDS piece
    // q = k * kThreads + 64 w + l (a wave's 64 pieces are contiguous, as the
    // instruction requires), so piece q fetches code row q / CH16, k-piece
    // (q % CH16) ^ (row & SWZ): the XOR swizzle that lds_a reads.  The
    // |c|^2/2 slots follow the same per-thread layout as h_dst.
    const unsigned char *cbb = reinterpret_cast<const unsigned char *>(a.cbh);
    const StageOffsets<T, kThreads> so;
    auto stage_piece = [&](int buf, int chunk, int k) {
        const unsigned char *g = cbb + (static_cast<int64_t>(chunk) * T::CHUNKB + so.uni(k)) + so.lane(k);
        unsigned char *d = lds + buf * T::BUFB + (k * kThreads + wave * kWave) * 16;
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)g,
                                         (__attribute__((address_space(3))) void *)d, 16, 0, 0);
    };
    auto stage_h = [&](int buf, int chunk) {
        const float *g = a.nhh + static_cast<int64_t>(chunk) * T::CC + hsrc;
        unsigned char *d = lds + buf * T::BUFB + T::CHUNKB + wave * kWave * 4;
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)g,
                                         (__attribute__((address_space(3))) void *)d, 4, 0, 0);
    };
    // s_waitcnt vmcnt(n) (no other counter): at most n of this wave's
    // global loads still in flight; a chunk is STAGE16 + 1 of them
    constexpr int kPerChunk = T::STAGE16 + 1;
    constexpr int kWaitNext = ((kPerChunk * (NB - 2)) & 15) | (((kPerChunk * (NB - 2)) >> 4) << 14) | 0x0070 | 0x0F00;
    static_assert(kPerChunk * (NB - 2) < 64, "vmcnt holds 6 bits");

    // prologue: chunks c0 .. c0 + NB - 2, and wait for the first
#pragma unroll
    for (int q = 0; q < NB - 1; ++q) {
        const int cq = c0 + q < c1 ? c0 + q : c1 - 1;
#pragma unroll
        for (int k = 0; k < T::STAGE16; ++k) stage_piece(q, cq, k);
        stage_h(q, cq);
    }
    __builtin_amdgcn_s_waitcnt(kWaitNext);
    __syncthreads();

    typename MX::V8 ring[R];
#pragma unroll
    for (int l = 0; l < L; ++l) ring[l] = lds_a(0, 0, l);
    f32x4 hcur = lds_h(0, 0);
    // The first epilogue sees a dummy block of -FLT_MAX scores: finite keys
    // below every real score, displaced from each lane's list by the N/4 >=
    // TOPL real codes that follow (frames whose scores are not finite fail
    // the certificate).
    f32x4 accp[FG];
#pragma unroll
    for (int g = 0; g < FG; ++g) accp[g] = f32x4{-3.40282347e38f, -3.40282347e38f, -3.40282347e38f, -3.40282347e38f};
    unsigned lprev = 0;

    // Per score: key (1 op), TOPL-1 med3 and one max-by-med3.  The upper
    // clamp is FLT_MAX rather than +inf so the compiler keeps a plain med3
    // (an fmax would need NaN canonicalisation of both operands); frames with
    // a key of +inf or NaN fail the certificate in any case.
    // key e (< 4 FG) of a block's sums into its group's list
    auto insert_key = [&](const f32x4 (&acc)[FG], unsigned local0, int e) {
        const int g = e / 4, i = e % 4;
        const float key = key_of(acc[g][i], local0 + i, vkeep);
#pragma unroll
        for (int j = TOPL - 1; j > 0; --j) top[g][j] = __builtin_amdgcn_fmed3f(top[g][j - 1], top[g][j], key);
        top[g][0] = __builtin_amdgcn_fmed3f(top[g][0], key, 3.40282347e38f);
    };
    auto epilogue = [&](const f32x4 (&acc)[FG], unsigned local0) {
#pragma unroll
        for (int e = 0; e < 4 * FG; ++e) insert_key(acc, local0, e);
    };

    for (int c = c0; c < c1; ++c) {
        const int buf = (c - c0) % NB;
        const int sbuf = (buf + NB - 1) % NB;   // left by chunk c - 1
        const int cs = c + NB - 1 < c1 ? c + NB - 1 : c1 - 1;
#pragma unroll
        for (int b = 0; b < BPC; ++b) {
            // this block's share of chunk cs, straight into LDS
#pragma unroll
            for (int i = 0; i < PPB; ++i) {
                const int k = b + i * BPC;
                if (k < T::STAGE16) stage_piece(sbuf, cs, k);
            }
            if (b == 0) stage_h(sbuf, cs);

            // the accumulators start from -|c|^2/2 of the block's codes
            const f32x4 hnext = b + 1 < BPC ? lds_h(buf, b + 1) : hcur;
            f32x4 acc[FG];
#pragma unroll
            for (int g = 0; g < FG; ++g) acc[g] = hcur;
            // Scheduling barriers keep each K-slice's fragment load L slices
            // ahead of its MFMAs (the compiler would sink it next to them);
            // each slice takes its share of the previous block's epilogue.
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const int pk = ks + L;
                if (pk < KS) ring[pk % R] = lds_a(buf, b, pk);
                else if (b + 1 < BPC) ring[pk % R] = lds_a(buf, b + 1, pk - KS);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int g = 0; g < FG; ++g)
                    acc[g] = MX::mfma(ring[ks % R], __builtin_bit_cast(typename MX::V8, xb[g][ks]), acc[g]);
#pragma unroll
                for (int e = ks * 4 * FG / KS; e < (ks + 1) * 4 * FG / KS; ++e) insert_key(accp, lprev, e);
                __builtin_amdgcn_sched_barrier(0);
            }
            hcur = hnext;
#pragma unroll
            for (int g = 0; g < FG; ++g) accp[g] = acc[g];
            lprev = static_cast<unsigned>((c * BPC + b) * 4);
        }
        __builtin_amdgcn_s_waitcnt(kWaitNext);   // chunk c + 1 has landed (this wave's part)
        __syncthreads();
        const int nbuf = (buf + 1) % NB;
#pragma unroll
        for (int l = 0; l < L; ++l) ring[l] = lds_a(nbuf, 0, l);
        hcur = lds_h(nbuf, 0);
    }
    epilogue(accp, lprev);

    // ---- keys and norms for the select kernel ----
    const int64_t ngroups = (a.M + 15) / 16;
#pragma unroll
    for (int g = 0; g < FG; ++g) {
        const int64_t gi = m_base / 16 + g;
        if (gi < ngroups) {
#pragma unroll
            for (int j = 0; j < TOPL; ++j)
                a.keys[((static_cast<int64_t>(split) * ngroups + gi) * TOPL + j) * kWave + lane] = top[g][j];
        }
        const int64_t m = m_base + g * 16 + col;
        if (split == 0 && kq == 0 && m < a.M) {
            a.norms[m] = nx2[g];
            a.norms[a.M + m] = nd2[g];
            a.norms[2 * a.M + m] = nxx2[g];
        }
    }
}

// Per-wave LDS of the select: the queue of (frame, code) pairs evaluated
// exactly, the frames' sum_rows(x*x) and (Q8_0) their query blocks, XQS
// bytes apart: the 8 lane groups of a pass read 8 frames' blocks, which a
// stride of K + 32 bytes puts in different LDS banks.
template <bool Q8, int K, int TOPL>
struct SelLds {
    static constexpr int QCAP = 16 * 4 * TOPL;
    static constexpr int XQS = K + 32;
    alignas(16) int8_t q_xq[Q8 ? 16 * XQS : 16];
    float q_xd[Q8 ? 16 * (K / 32) : 1];
    int32_t q_n[QCAP], q_f[QCAP];
    float q_v[QCAP], q_x2[16];
};

// Certificate, exact re-ranking, outputs and residual update of one group of
// 16 frames (m_base ...) in one wave, 4 lanes per frame (the sweep's lane
// layout): top / taul are the lane's merged keys and the bound of the keys it
// dropped, nx2 / nd2 / nxx2 the frame's |x~|^2, |x - x~|^2, |x|^2; the
// frames' fp32 rows are read at xrows + f * xstride (f < 16; global memory
// or LDS).  Frames the certificate cannot settle go to a.fail_list for the
// refine pass, or, with `speculate`, take the best exactly evaluated
// candidate (outputs and residual update as if certified) and are listed in
// a.spec_list as (frame, stage) for the exact verification after the
// cascade.  With `update` the residual a.xout = a.xin - c[code] is written
// for the settled frames; the lane's frame's code is returned (-1: frame
// not settled or past M).
template <int RECIPE, bool Q8, int KS, int TOPL>
__device__ int select_group(const StageArgs &a, int64_t m_base, const float (&top_in)[TOPL], float taul_in,
                            float nx2_in, float nd2_in, float nxx2_in, SelLds<Q8, KS * 32, TOPL> &sl,
                            bool speculate, const float *xrows, int xstride, bool update) {
    constexpr int K = KS * 32;
    constexpr int FG = 1;
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 15;
    const int kq = lane >> 4;
    const int N = a.N;
    int lbits = 0;
    while ((1 << lbits) < N / 4) ++lbits;
    const unsigned kmask = (1u << lbits) - 1u;
    float top[FG][TOPL], taul[FG], nx2[FG], nd2[FG], nxx2[FG];
#pragma unroll
    for (int j = 0; j < TOPL; ++j) top[0][j] = top_in[j];
    taul[0] = taul_in;
    nx2[0] = nx2_in;
    nd2[0] = nd2_in;
    nxx2[0] = nxx2_in;

    // ---- phase 2: per-frame certificate and exact re-ranking ----
    // 2a bounds and candidates per frame; 2b the frames' |x|^2 (Higgs);
    // 2c every candidate (frame, code) pair of the wave evaluated exactly, one
    // pair per lane, through a queue in LDS (the codebook tiles are dead);
    // 2d per-frame selection, certificate and outputs.
    const float u = 5.9604645e-8f;   // 2^-24
    const int Tk = a.topk > 0 ? a.topk : 1;
    const int Tsel = a.topk > 0 ? a.topk + 1 : 1;
    const bool want_value = a.dist != nullptr || a.topk > 0;
    constexpr int XQS = SelLds<Q8, K, TOPL>::XQS;
    int32_t *q_n = sl.q_n;
    int32_t *q_f = sl.q_f;
    float *q_v = sl.q_v;
    float *q_x2 = sl.q_x2;
    int8_t *q_xq = sl.q_xq;
    float *q_xd = sl.q_xd;

    float Eg[FG], taug[FG], best0g[FG];
    bool okg[FG], needg[FG];
    int cand_n[FG][TOPL], qpos[FG][TOPL];
    int qcount = 0;
#pragma unroll
    for (int g = 0; g < FG; ++g) {
        const int64_t m = m_base + g * 16 + col;
        const bool live = m < a.M;

        // Bound E (in units of v = x.c - |c|^2/2) on |v(n) - S'(n)| for every n.
        const float nx = sqrtf(nx2[g]) * 1.0001f, nd = sqrtf(nd2[g]) * 1.0001f;
        const float nxe = nx + nd;                           // >= |x|
        const float e_half = nx * a.dcmax + nd * a.cmax;
        // fp32 accumulation from -|c|^2/2: partial sums stay below
        // |x~||c~| + |c|^2/2
        const float e_acc = (K + 4) * u * (nx * a.chmax + 0.5f * a.cmax * a.cmax);
        const float e_rec = (K + 16) * u * (nxe * a.cmax + nxe * nxe + a.cmax * a.cmax);
        const float vmax = nx * a.chmax + 0.5f * a.cmax * a.cmax + e_rec;
        const float trunc = ldexpf(vmax, lbits - 23);
        const float E = 1.02f * (e_half + e_acc + e_rec + 4.0f * u * vmax) + trunc + 1e-30f;

        // Keys of the frame's 4 lanes, gathered in every one of them.
        float all[4 * TOPL];
#pragma unroll
        for (int j = 0; j < TOPL; ++j) {
            float kr[4];
            rows4(top[g][j], kr);
#pragma unroll
            for (int q = 0; q < 4; ++q) all[4 * j + q] = kr[q];
        }
        // tau bounds every key a lane dropped; vT is the T-th largest kept key.
        float tau = taul[g];
        tau = rows_max(tau);
        float best[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
        for (int t = 0; t < 4 * TOPL; ++t) {
            float v = all[t];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float hi = fmaxf(best[r], v);
                v = fminf(best[r], v);
                best[r] = hi;
            }
        }
        const float vT = best[Tk - 1];
        const bool ok = live && !a.exact_only && (E < INFINITY) && (vT - vT == 0.0f);
        const float thr = vT - 2.0f * E;
        int nabove = 0;
#pragma unroll
        for (int t = 0; t < 4 * TOPL; ++t) nabove += all[t] >= thr ? 1 : 0;
        const bool need = ok && (want_value || nabove > 1);
        Eg[g] = E;
        taug[g] = tau;
        best0g[g] = best[0];
        okg[g] = ok;
        needg[g] = need;
        // enqueue this lane's candidates
#pragma unroll
        for (int j = 0; j < TOPL; ++j) {
            const float key = top[g][j];
            const bool c = need && key >= thr && key > -INFINITY;
            const unsigned local = __float_as_uint(key) & kmask;
            const int n = static_cast<int>((local >> 2) * 16 + kq * 4 + (local & 3));
            const unsigned long long bal = __ballot(c);
            const int pos = qcount + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                                         static_cast<unsigned>(bal >> 32),
                                         __builtin_amdgcn_mbcnt_lo(static_cast<unsigned>(bal), 0u)));
            if (c) {
                q_n[pos] = n;
                q_f[pos] = g * 16 + col;
            }
            cand_n[g][j] = c ? n : -1;
            qpos[g][j] = pos;
            qcount += __popcll(bal);
        }
    }
    // 2b: sum_rows(x*x) of each frame that has candidates, and (Q8_0) each
    // frame's query blocks quantised once (x86 quantize_row_q8_0).  For
    // K % 256 == 0 the frame's 4 lanes load it in one round trip per 256
    // elements (lane kq the 64 from 64 kq), add their squares in order in
    // turn (the double running sum handed on from lane to lane) and quantise
    // their two blocks from registers.
    if (RECIPE == HIGGS && K % 256 == 0) {
        if (__any(needg[0])) {
            static_assert(FG == 1, "one frame group per select wave");
            const int fq = m_base + col < a.M ? col : static_cast<int>(a.M - 1 - m_base);
            const float *xr = xrows + static_cast<int64_t>(fq) * xstride;
            double sq = 0.0;
#pragma unroll
            for (int c = 0; c < K / 256; ++c) {
                f32x4 v[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) v[i] = *reinterpret_cast<const f32x4 *>(xr + 256 * c + 64 * kq + 4 * i);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if (kq == q)
#pragma unroll
                        for (int i = 0; i < 16; ++i)
#pragma unroll
                            for (int t = 0; t < 4; ++t) sq += static_cast<double>(__fmul_rn(v[i][t], v[i][t]));
                    sq = row_bcast(sq, q);
                }
                if (Q8) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const int blk = 8 * c + 2 * kq + h;
                        float amax = 0.0f, fin = 0.0f;   // fin: 0 unless a value is inf or NaN
#pragma unroll
                        for (int i = 0; i < 8; ++i)
#pragma unroll
                            for (int t = 0; t < 4; ++t) {
                                amax = fmaxf(amax, fabsf(v[8 * h + i][t]));
                                fin = __fmaf_rn(v[8 * h + i][t], 0.0f, fin);
                            }
                        float d, id;
                        q8_scale(amax, d, id);
                        int *qw = reinterpret_cast<int *>(q_xq + col * XQS + 32 * blk);
                        if (fin == 0.0f && id < INFINITY) {
                            // finite values and |v * id| <= 127 (1 + 2^-23)^2:
                            // the rounded values are integers in [-127, 127],
                            // where q8_quant's range test and clamp are idle
#pragma unroll
                            for (int i = 0; i < 8; ++i) {
                                const f32x4 x = v[8 * h + i];
                                qw[i] = q8_pack4(static_cast<int>(__builtin_rintf(__fmul_rn(x[0], id))),
                                                 static_cast<int>(__builtin_rintf(__fmul_rn(x[1], id))),
                                                 static_cast<int>(__builtin_rintf(__fmul_rn(x[2], id))),
                                                 static_cast<int>(__builtin_rintf(__fmul_rn(x[3], id))));
                            }
                        } else {
#pragma unroll
                            for (int i = 0; i < 8; ++i) {
                                unsigned w = 0;
#pragma unroll
                                for (int t = 0; t < 4; ++t)
                                    w |= (static_cast<unsigned>(q8_quant(v[8 * h + i][t], id)) & 0xFFu) << (8 * t);
                                qw[i] = static_cast<int>(w);
                            }
                        }
                        q_xd[col * (K / 32) + blk] = d;
                    }
                }
            }
            if (kq == 0) q_x2[col] = static_cast<float>(sq);
        }
    } else {
        if (RECIPE == HIGGS) {
            int needmask = 0;   // bit g: frame (g, lane % 16) has candidates
#pragma unroll
            for (int g = 0; g < FG; ++g) needmask |= (__shfl(needg[g] ? 1 : 0, lane % 16) & 1) << g;
            if (lane < FG * 16) {
                const bool need = ((needmask >> (lane / 16)) & 1) != 0;
                q_x2[lane] = need ? sum_squares_k<K>(xrows + static_cast<int64_t>(lane) * xstride) : 0.0f;
            }
        }
        // Q8_0: the 4 lanes of a frame taking every 4th block.
        if (Q8 && qcount > 0) {
            const int fq = m_base + col < a.M ? col : static_cast<int>(a.M - 1 - m_base);
#pragma unroll
            for (int ib = kq; ib < K / 32; ib += 4)
                quantize_block_q8(xrows + static_cast<int64_t>(fq) * xstride + 32 * ib, q_xq + col * XQS + 32 * ib,
                                  q_xd + col * (K / 32) + ib);
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // 2c: exact values of the queued pairs, in the reference's arithmetic.
    if (!Q8 && RECIPE != DIRECT && a.order == 0) {
        // tinyBLAS: 16 accumulators over k = 16 l + j, one per lane of a
        // 16-lane row (coalesced row reads), then _mm512_reduce_add_ps's
        // pairing tree as DPP row rotations 8, 4, 2, 1; 4 pairs per pass.
        // Several pairs per row and pass (four up to K = 256, else two), so
        // that their row reads are in flight together.
        constexpr int P = K <= 256 ? 4 : 2;
        const int j = lane & 15, grp = lane >> 4;
        const float sa = RECIPE == OMNI ? 2.0f : 1.0f;
        for (int e0 = grp; e0 < qcount; e0 += 4 * P) {
            int fs[P], n[P];
            float acc[P], off[P];
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const int e = e0 + 4 * p;
                fs[p] = e < qcount ? q_f[e] : 0;
                n[p] = e < qcount ? q_n[e] : 0;
                acc[p] = 0.0f;
            }
            // the code's bias (OmniVoice) or |c|^2 (Higgs) is loaded with
            // its row, not after the sum
#pragma unroll
            for (int p = 0; p < P; ++p) off[p] = RECIPE == OMNI ? a.bias[n[p]] : a.e2[n[p]];
#pragma unroll
            for (int l = 0; l < K / 16; ++l)
#pragma unroll
                for (int p = 0; p < P; ++p)
                    acc[p] = __fmaf_rn(a.cbf[static_cast<int64_t>(n[p]) * K + 16 * l + j] * sa,
                                       xrows[static_cast<int64_t>(fs[p]) * xstride + 16 * l + j], acc[p]);
#pragma unroll
            for (int p = 0; p < P; ++p) {
                float v = row_ror_add<8>(acc[p]);
                v = row_ror_add<4>(v);
                v = row_ror_add<2>(v);
                v = row_ror_add<1>(v);
                const int e = e0 + 4 * p;
                if (j == 0 && e < qcount) {
                    if (RECIPE == OMNI) q_v[e] = __fadd_rn(v, off[p]);
                    else q_v[e] = __fsub_rn(__fsub_rn(__fmul_rn(v, 2.0f), q_x2[fs[p]]), off[p]);
                }
            }
        }
    } else if (Q8) {
        // ggml_vec_dot_q8_0_q8_0: 8 accumulators over the 4-element groups
        // of every block, one per lane of an 8-lane group, then hsum_float_8
        // by DPP (hsum8_dpp); 8 pairs per pass.  Several pairs per group and
        // pass (as registers allow): the queue entries are read first, then
        // every memory operand of the pass (code rows, scales, |c|^2, the
        // frames' query blocks) is issued before the first is used, so a
        // pass costs one memory round trip.
        constexpr int P = K <= 256 ? 4 : (K <= 512 ? 2 : 1);
        const int j = lane & 7, grp = lane >> 3;
        const int jw = q8_lane_word(j);
        for (int e0 = grp; e0 < qcount; e0 += 8 * P) {
            int cq[P][K / 32], xw[P][K / 32], fs[P], n[P];
            float cd[P][K / 32], xd[P][K / 32], e2v[P], x2v[P];
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const int e = e0 + 8 * p < qcount ? e0 + 8 * p : e0;
                fs[p] = q_f[e];
                n[p] = q_n[e];
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const int *cqp = reinterpret_cast<const int *>(a.q8 + static_cast<int64_t>(n[p]) * K) + jw;
                const float *cdp = a.q8d + static_cast<int64_t>(n[p]) * (K / 32);
#pragma unroll
                for (int ib = 0; ib < K / 32; ++ib) {
                    cq[p][ib] = cqp[8 * ib];
                    cd[p][ib] = cdp[ib];
                }
                e2v[p] = a.e2[n[p]];
            }
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const int *xq = reinterpret_cast<const int *>(q_xq + fs[p] * XQS) + jw;
#pragma unroll
                for (int ib = 0; ib < K / 32; ++ib) {
                    xw[p][ib] = xq[8 * ib];
                    xd[p][ib] = q_xd[fs[p] * (K / 32) + ib];
                }
                x2v[p] = q_x2[fs[p]];
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int p = 0; p < P; ++p) {
                float acc = 0.0f;
#pragma unroll
                for (int ib = 0; ib < K / 32; ++ib) {
                    const float dd = __fmul_rn(cd[p][ib], xd[p][ib]);
                    acc = __fmaf_rn(dd, static_cast<float>(__builtin_amdgcn_sdot4(cq[p][ib], xw[p][ib], 0, false)), acc);
                }
                acc = hsum8_dpp(acc);
                const int e = e0 + 8 * p;
                if (j == 0 && e < qcount) q_v[e] = __fsub_rn(__fsub_rn(__fmul_rn(acc, 2.0f), x2v[p]), e2v[p]);
            }
        }
    } else {
        for (int e0 = 0; e0 < qcount; e0 += kWave) {
            const int e = e0 + lane;
            if (e < qcount) {
                const int fs = q_f[e];
                const int n = q_n[e];
                const float x2 = RECIPE == HIGGS ? q_x2[fs] : 0.0f;
                q_v[e] = exact_value_k<RECIPE, Q8, K>(a, xrows + static_cast<int64_t>(fs) * xstride, n, x2);
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // 2d: selection, certificate, outputs
    int win_code[FG];
    bool win_ok[FG];
#pragma unroll
    for (int g = 0; g < FG; ++g) {
        const int64_t m = m_base + g * 16 + col;
        const bool live = m < a.M;
        bool ok = okg[g];
        const float E = Eg[g], tau = taug[g];
        const float x2 = RECIPE == HIGGS ? q_x2[g * 16 + col] : 0.0f;
        float cand_val[TOPL];
#pragma unroll
        for (int j = 0; j < TOPL; ++j) cand_val[j] = cand_n[g][j] >= 0 ? q_v[qpos[g][j]] : 0.0f;
        // Exact top-T over the frame's evaluated candidates (all 4 lanes agree).
        // With top-k the list holds one entry more than reported, so that a
        // tie at the k-th place (which ggml_top_k's heap resolves) is seen.
        float sel_v[5];
        int sel_n[5];
#pragma unroll
        for (int r = 0; r < 5; ++r) {
            sel_v[r] = 0.0f;
            sel_n[r] = -1;
        }
        if (needg[g]) {
            if (Tsel == 1) {
                // The best evaluated candidate: each lane's own, then the
                // better of the partner rows'
                // (r^1, then r^2).  ranks_before is a total order on finite
                // values over the lanes' disjoint codes; a frame with a
                // non-finite candidate is left to the exact scan.
                bool nonfin = false;
#pragma unroll
                for (int j = 0; j < TOPL; ++j) {
                    const int cn = cand_n[g][j];
                    if (!__any(cn >= 0)) continue;
                    const float cv = cand_val[j];
                    nonfin = nonfin || (cn >= 0 && !(cv - cv == 0.0f));
                    const bool take = cn >= 0 && (sel_n[0] < 0 || ranks_before<RECIPE>(cv, cn, sel_v[0], sel_n[0]));
                    sel_v[0] = take ? cv : sel_v[0];
                    sel_n[0] = take ? cn : sel_n[0];
                }
                best_rows<RECIPE, 1>(sel_v[0], sel_n[0], kq);
                best_rows<RECIPE, 2>(sel_v[0], sel_n[0], kq);
                if (rows_max(nonfin ? 1.0f : 0.0f) != 0.0f) ok = false;
            } else {
                // Top-k: each lane ranks its own candidates into a list of 5
                // (k <= 4 places and the next one), then the lists of the
                // frame's 4 lanes are merged across rows (partner row r^1,
                // then r^2; merge_rows5).  The order is total for finite
                // values and the lanes' codes are disjoint, so the list is
                // the frame's exact top 5; a frame with a non-finite
                // candidate is left to the exact scan.
                bool nonfin = false;
#pragma unroll
                for (int j = 0; j < TOPL; ++j) {
                    int cn = cand_n[g][j];
                    if (!__any(cn >= 0)) continue;
                    float cv = cand_val[j];
                    nonfin = nonfin || (cn >= 0 && !(cv - cv == 0.0f));
#pragma unroll
                    for (int r = 0; r < 5; ++r) {
                        const bool take = cn >= 0 && (sel_n[r] < 0 || topk_before<RECIPE>(cv, cn, sel_v[r], sel_n[r]));
                        const float tv = sel_v[r];
                        const int tn = sel_n[r];
                        sel_v[r] = take ? cv : tv;
                        sel_n[r] = take ? cn : tn;
                        cv = take ? tv : cv;
                        cn = take ? tn : cn;
                    }
                }
                merge_rows5<RECIPE, 1>(sel_v, sel_n, kq);
                merge_rows5<RECIPE, 2>(sel_v, sel_n, kq);
                if (rows_max(nonfin ? 1.0f : 0.0f) != 0.0f) ok = false;
            }
            // S' of the T-th exact value in v units, against the bound of unkept codes.
            if (sel_n[Tk - 1] < 0) {
                ok = false;
            } else {
                const float sv = sel_v[Tk - 1];
                float sprime;
                if (RECIPE == OMNI) sprime = 0.5f * sv;
                else if (RECIPE == HIGGS) sprime = 0.5f * sv + 0.5f * x2;
                else sprime = -0.5f * sv + 0.5f * nxx2[g];
                // DIRECT's offset |x|^2/2 comes from fp32 partial sums
                // (relative error <= (K + 8) u); widen E by it.
                const float off_err = RECIPE == DIRECT ? 0.5f * (K + 8) * u * nxx2[g] * 1.01f : 0.0f;
                ok = ok && (sv - sv == 0.0f) && (sprime - off_err > tau + E);
                // Every evaluated candidate must be finite for the order to be exact.
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (r < Tk && sel_n[r] >= 0 && !(sel_v[r] - sel_v[r] == 0.0f)) ok = false;
                // With Tk ties at the maximum, a further tie outside the list
                // could hold the larger index argmax keeps: scan exactly.
                if (RECIPE != DIRECT && Tk > 1 && sv == sel_v[0]) ok = false;
                // A tie at the k-th place: ggml_top_k keeps whichever of the
                // tied codes its heap keeps; the exact scan replays it.
                if (RECIPE != DIRECT && a.topk > 0 && sel_n[Tk] >= 0 && sel_v[Tk] == sv) ok = false;
            }
            // argmax among exact ties keeps ggml's last index
            int w = sel_n[0];
            if (RECIPE != DIRECT)
#pragma unroll
                for (int r = 1; r < 4; ++r)
                    if (r < Tk && sel_n[r] >= 0 && sel_v[r] == sel_v[0] && sel_n[r] > w) w = sel_n[r];
            win_code[g] = w;
        } else {
            // One candidate clears the threshold: it wins if it also clears
            // every dropped code by 2E (no exact value is needed).
            ok = ok && (best0g[g] - E > tau + E);
            const float kb = best0g[g];
            // owner lane of the best key
            const bool mine = top[g][0] == kb;
            const unsigned local = __float_as_uint(kb) & kmask;
            int n = mine ? static_cast<int>((local >> 2) * 16 + kq * 4 + (local & 3)) : 0x7fffffff;
            {
                int nq[4];
                rows4(n, nq);
                n = min(min(nq[0], nq[1]), min(nq[2], nq[3]));
            }
            win_code[g] = n;
            ok = ok && n < N;
        }
        if (speculate) {
            // an uncertified frame continues with the best evaluated code
            const int w = win_code[g];
            win_code[g] = w >= 0 && w < N ? w : 0;
            if (a.misspeculate) {
                // test hooks: the verification sees every frame, continued
                // with a code that is not its best (1: the fix-up recomputes
                // it) or with its best code and distances one bit off (2:
                // the verification corrects them in place)
                ok = false;
                if (a.misspeculate == 1) win_code[g] = win_code[g] + 1 < N ? win_code[g] + 1 : 0;
            }
        }
        win_ok[g] = ok || (speculate && live);

        if (kq == 0 && live) {
            if (!ok && !speculate) {
                const int slot = atomicAdd(a.fail_count, 1);
                a.fail_list[slot] = static_cast<int32_t>(m);
            } else {
                if (!ok) {
                    atomicAdd(a.fail_count, 1);
                    const int slot = atomicAdd(a.spec_count, 1);
                    a.spec_list[2 * slot] = static_cast<int32_t>(m);
                    a.spec_list[2 * slot + 1] = a.s;
                }
                a.idx[m * a.Q + a.s] = win_code[g];
                const unsigned flip = speculate && a.misspeculate == 2 ? 1u : 0u;   // test hook 2
                if (a.dist) {
                    const float v = sel_v[0];   // the argmax's value (ties share it)
                    a.dist[m * a.Q + a.s] = __uint_as_float(__float_as_uint(RECIPE == DIRECT ? v : -v) ^ flip);
                }
                for (int r = 0; r < a.topk; ++r) {
                    a.topk_idx[(m * a.Q + a.s) * a.topk + r] = sel_n[r] < 0 ? 0 : sel_n[r];
                    a.topk_dist[(m * a.Q + a.s) * a.topk + r] =
                        __uint_as_float(__float_as_uint(RECIPE == DIRECT ? sel_v[r] : -sel_v[r]) ^ flip);
                }
            }
        }
    }

    if (!update) return win_ok[0] && m_base + col < a.M ? win_code[0] : -1;

    // ---- phase 3: residual update r -= c[code] for certified frames ----
    // Rows across the lanes (coalesced), and the loads of kP3 frames issued
    // before the first wait so one memory round trip covers all of them.
    constexpr int kP3 = 16;
    constexpr int KV = (K + 4 * kWave - 1) / (4 * kWave);   // float4 per lane per row
#pragma unroll
    for (int g = 0; g < FG; ++g) {
#pragma unroll
        for (int f0 = 0; f0 < 16; f0 += kP3) {
            bool okf[kP3];
            int64_t mrow[kP3];
            int use[kP3];
#pragma unroll
            for (int t = 0; t < kP3; ++t) {
                const int f = f0 + t;
                const int64_t m = m_base + g * 16 + f;
                okf[t] = m < a.M && __builtin_amdgcn_readlane(win_ok[g] ? 1 : 0, f) != 0;
                mrow[t] = okf[t] ? m : 0;
                // rows of frames that are skipped are clamped to row 0, so the
                // loads below need no branches (only the stores are predicated)
                use[t] = okf[t] ? __builtin_amdgcn_readlane(win_code[g], f) : 0;
            }
            if (a.force_idx) {
#pragma unroll
                for (int t = 0; t < kP3; ++t) {
                    if (!okf[t]) continue;
                    int u2 = a.force_idx[mrow[t] * a.Q + a.s];
                    if (u2 < 0 || u2 >= N) {
                        if (lane == 0) a.flags[AQ_FLAG_BAD_INDEX] = 1;
                        u2 = 0;
                    }
                    use[t] = u2;
                }
            }
            if (!a.xout) continue;   // last stage, no residual asked for
#pragma unroll
            for (int kv = 0; kv < KV; ++kv) {
                const int k = (kv * kWave + lane) * 4;
                const bool inb = k < K;
                const int kc = inb ? k : 0;
                f32x4 xv[kP3], cv[kP3];
#pragma unroll
                for (int t = 0; t < kP3; ++t) {
                    xv[t] = *reinterpret_cast<const f32x4 *>(a.xin + mrow[t] * K + kc);
                    cv[t] = *reinterpret_cast<const f32x4 *>(a.cbf + static_cast<int64_t>(use[t]) * K + kc);
                }
#pragma unroll
                for (int t = 0; t < kP3; ++t) {
                    if (okf[t] && inb) {
                        f32x4 o;
#pragma unroll
                        for (int q = 0; q < 4; ++q) o[q] = __fsub_rn(xv[t][q], cv[t][q]);
                        *reinterpret_cast<f32x4 *>(a.xout + mrow[t] * K + k) = o;
                    }
                }
            }
        }
    }
    return win_ok[0] && m_base + col < a.M ? win_code[0] : -1;
}


// Certificate, exact re-ranking and residual update of one stage.  A wave
// takes 16 frames (4 lanes per frame, the sweep's lane layout), merges each
// lane's key lists of all code splits and applies the certificate; the
// frames it cannot settle go to the refine pass.
template <int RECIPE, bool Q8, int KS, int TOPL>
__global__ __launch_bounds__(kThreads) void euclid_select_kernel(StageArgs a) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int col = lane & 15;
    const int64_t m_base = (static_cast<int64_t>(blockIdx.x) * kWaves + wave) * 16;
    // Waves past the last frame group leave at once (no block barrier
    // follows; the exact-evaluation queues are per wave).
    if (m_base >= a.M) return;
    // Merge the lane's key lists of every split.  tau_l bounds every key the
    // lane dropped, in the sweep (each split's TOPL-th key) or here.
    const int64_t ngroups = (a.M + 15) / 16;
    const int64_t gi = m_base / 16;
    float top[TOPL], taul = -INFINITY;
#pragma unroll
    for (int j = 0; j < TOPL; ++j) top[j] = -INFINITY;
    // the sweep's split count for this group's tile
    const int nsp = m_base >= a.tile2 * (kWaves * groups_for(KS) * 16) ? a.nsplit2 : a.nsplit;
    for (int sp = 0; sp < nsp; ++sp) {
#pragma unroll
        for (int j = 0; j < TOPL; ++j) {
            const float key = a.keys[((static_cast<int64_t>(sp) * ngroups + gi) * TOPL + j) * kWave + lane];
            if (j == TOPL - 1) taul = fmaxf(taul, key);
#pragma unroll
            for (int i = TOPL - 1; i > 0; --i) top[i] = __builtin_amdgcn_fmed3f(top[i - 1], top[i], key);
            top[0] = __builtin_amdgcn_fmed3f(top[0], key, 3.40282347e38f);
        }
    }
    taul = fmaxf(taul, top[TOPL - 1]);
    const int64_t m = m_base + col;
    const int64_t mc = m < a.M ? m : a.M - 1;
    __shared__ SelLds<Q8, KS * 32, TOPL> sl[kWaves];
    select_group<RECIPE, Q8, KS, TOPL>(a, m_base, top, taul, a.norms[mc], a.norms[a.M + mc], a.norms[2 * a.M + mc],
                                       sl[wave], false, a.xin + m_base * (KS * 32), KS * 32, true);
}

// ------------------------------------------------------------- exact scan

// Frames that neither certificate settles get an exact scan.  The recipe
// value of every code (one code per thread) is computed over the whole grid
// when a stage has at most kScanSplitFrames such frames (the block that
// completes a frame's values then selects for it), else by the frame's own
// block.  The selection, per frame: in parallel (winner and best topk + 1 codes per
// thread, merged over the block), which is the reference's result unless a
// value is NaN or the k-th and (k+1)-th values tie; in those cases wave 0
// walks the values (kScanChunk at a time in LDS) in code order with the
// reference's selection rules, so the result is the reference's by
// construction, ties and NaN included:
//  * ggml recipes: ggml_vec_argmax_f32 (running MAX(max, v), index of the
//    last element equal to the running max, a NaN restarts it) and
//    ggml_top_k's std::partial_sort heap;
//  * DIRECT: the first index of the minimum distance (strict <, NaN never
//    wins) and the k smallest distances (ties by index).
// The walk takes 64 codes per step: a chunk without NaN is reduced with a
// wave max / min and a ballot, and the heap only visits codes that beat its
// root.

// One step of libstdc++'s binary heap (GCC 11.4 std::__adjust_heap followed
// by std::__push_heap) with comp(a, b) = value(a) > value(b): the root holds
// the worst kept element.  std::partial_sort builds the heap over the first k
// codes and lets each later code that is strictly better than the root
// replace it, which decides which of several equal values ggml_top_k keeps.
__device__ void heap_adjust(int *hn, float *hv, int hole, int len, int vn, float vv) {
    const int top = hole;
    int child = hole;
    while (child < (len - 1) / 2) {
        child = 2 * (child + 1);
        if (hv[child] > hv[child - 1]) child--;
        hn[hole] = hn[child];
        hv[hole] = hv[child];
        hole = child;
    }
    if ((len & 1) == 0 && child == (len - 2) / 2) {
        child = 2 * (child + 1);
        hn[hole] = hn[child - 1];
        hv[hole] = hv[child - 1];
        hole = child - 1;
    }
    int parent = (hole - 1) / 2;
    while (hole > top && hv[parent] > vv) {
        hn[hole] = hn[parent];
        hv[hole] = hv[parent];
        hole = parent;
        parent = (hole - 1) / 2;
    }
    hn[hole] = vn;
    hv[hole] = vv;
}

constexpr int kScanThreads = 256;
constexpr int kScanChunk = 2048;
// Frames per stage whose exact values the scan spreads over its grid; with
// more, each frame's block computes its own.
constexpr int kScanSplitFrames = 64;
constexpr int kScanQuadCodes = kScanThreads / 4;   // codes per spread item, four lanes each
// Order-preserving key of a non-NaN value: a > b (as floats) exactly when
// ukey(a) > ukey(b); -0 and +0, which compare equal, share a key.  Every key
// is at least ukey(-inf) = 0x007FFFFF.
__device__ inline uint32_t ukey(float v) {
    const unsigned b = __float_as_uint(__fadd_rn(v, 0.0f));
    return b ^ ((b >> 31) ? 0xFFFFFFFFu : 0x80000000u);
}

// Total-order key of a recipe value for the parallel selection of the exact
// scan: a larger key ranks first (ggml recipes: larger value, then smaller
// index; DIRECT: smaller value, then smaller index, the order of its top-k).
// NaN has none: 0, which no value reaches, stands for "no code".
template <int RECIPE>
__device__ inline uint64_t rank_key(float v, int n) {
    if (v != v) return 0;
    const uint32_t o = RECIPE == DIRECT ? ~ukey(v) : ukey(v);
    return (static_cast<uint64_t>(o) << 32) | static_cast<uint32_t>(~n);
}

__device__ inline int key_index(uint64_t k) { return static_cast<int>(~static_cast<uint32_t>(k)); }

// k or its DPP-permuted copy (CTRL: a permutation inside rows of 16 lanes),
// whichever is larger.
template <int CTRL>
__device__ inline uint64_t dpp_max_u64(uint64_t k) {
    const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(k)), CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(k >> 32)), CTRL, 0xF, 0xF, false);
    const uint64_t o = (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo);
    return o > k ? o : k;
}

// Largest key over a wave (every lane active), the same in every lane: lane
// xor 1 and xor 2 (quad_perm), half-row and row mirrors leave each row's
// maximum in all its lanes; lanes 0, 16, 32, 48 are compared in scalar
// registers.
__device__ inline uint64_t wave_max_u64(uint64_t k) {
    k = dpp_max_u64<0xB1>(k);
    k = dpp_max_u64<0x4E>(k);
    k = dpp_max_u64<0x141>(k);
    k = dpp_max_u64<0x140>(k);
    uint64_t m = 0;
#pragma unroll
    for (int row = 0; row < kWave / 16; ++row) {
        const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(k)), 16 * row);
        const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(k >> 32)), 16 * row);
        const uint64_t q = (static_cast<uint64_t>(hi) << 32) | lo;
        m = q > m ? q : m;
    }
    return m;
}

// heap_adjust(hn, hv, 0, LEN, nv, v) for a heap of LEN <= 4 entries, with
// the values as ukey keys (kv = ukey(v)): the root replaced by (kv, nv) and
// sifted down, then the new entry pushed up, std::__adjust_heap's cases
// written out so that a wave-uniform heap stays in scalar registers.
template <int LEN>
__device__ inline void heap_replace_root(uint32_t (&k)[4], int (&n)[4], uint32_t kv, int nv) {
    if (LEN == 1) {
        k[0] = kv;
        n[0] = nv;
    } else if (LEN == 2) {
        if (k[1] > kv) {
            k[0] = kv;
            n[0] = nv;
        } else {
            k[0] = k[1];
            n[0] = n[1];
            k[1] = kv;
            n[1] = nv;
        }
    } else if (LEN == 3) {
        // the hole moves to the child with the smaller value (child 2 on equality)
        const bool one = k[2] > k[1];
        const uint32_t ks = one ? k[1] : k[2];
        const int ns = one ? n[1] : n[2];
        if (ks > kv) {
            k[0] = kv;
            n[0] = nv;
        } else {
            k[0] = ks;
            n[0] = ns;
            if (one) {
                k[1] = kv;
                n[1] = nv;
            } else {
                k[2] = kv;
                n[2] = nv;
            }
        }
    } else if (k[2] > k[1]) {
        // hole to child 1, then to its only child 3; push up from 3
        if (!(k[3] > kv)) {
            k[0] = k[1];
            n[0] = n[1];
            k[1] = k[3];
            n[1] = n[3];
            k[3] = kv;
            n[3] = nv;
        } else if (!(k[1] > kv)) {
            k[0] = k[1];
            n[0] = n[1];
            k[1] = kv;
            n[1] = nv;
        } else {
            k[0] = kv;
            n[0] = nv;
        }
    } else if (!(k[2] > kv)) {
        // hole to child 2 (a leaf); push up from 2
        k[0] = k[2];
        n[0] = n[2];
        k[2] = kv;
        n[2] = nv;
    } else {
        k[0] = kv;
        n[0] = nv;
    }
}

// ggml_top_k's std::partial_sort heap over src[0, N) (no NaN), by one wave
// with the heap in scalar registers: std::make_heap of the first LEN codes,
// then each later code strictly above the root replaces it
// (std::__heap_select).  The next 64 values load while a chunk is walked.
// Lane 0 leaves the heap in hn / hv.
template <int LEN>
__device__ void heap_walk(const float *src, int N, int *hn, float *hv) {
    const int lane = threadIdx.x & (kWave - 1);
    uint32_t k[4] = {0, 0, 0, 0};
    int n[4] = {0, 0, 0, 0};
#pragma unroll
    for (int q = 0; q < LEN; ++q) {
        k[q] = __builtin_amdgcn_readfirstlane(ukey(src[q]));
        n[q] = q;
    }
    // std::make_heap: __adjust_heap at 1 (LEN 4: its only child 3), then at 0
    if (LEN == 4 && !(k[3] > k[1])) {
        const uint32_t t = k[1];
        k[1] = k[3];
        k[3] = t;
        n[1] = 3;
        n[3] = 1;
    }
    if (LEN >= 2) heap_replace_root<LEN>(k, n, k[0], n[0]);
    uint32_t root = k[0];
    float v = LEN + lane < N ? src[LEN + lane] : -INFINITY;
    for (int c0 = LEN; c0 < N; c0 += kWave) {
        const int nx = c0 + kWave + lane;
        const float vn = nx < N ? src[nx] : -INFINITY;
        const uint32_t uk = ukey(v);
        unsigned long long take = __ballot(uk > root);
        while (take != 0) {
            const int f = __ffsll(static_cast<long long>(take)) - 1;
            heap_replace_root<LEN>(k, n, __builtin_amdgcn_readlane(uk, f), c0 + f);
            root = k[0];
            take = __ballot(lane > f && uk > root);
        }
        v = vn;
    }
    if (lane == 0)
#pragma unroll
        for (int q = 0; q < LEN; ++q) {
            hn[q] = n[q];
            hv[q] = src[n[q]];
        }
}

// ---------------------------------------------------- spread exact values
// The exact values of every code of up to scap open frames, spread over the
// grid: item (slot, chunk) writes svals[slot][chunk codes].  F32 codebooks
// in tinyBLAS order take four lanes per code (lane q of a quad accumulates
// k = 16 l + 4 q + t, t < 4: tinyBLAS lanes 4q .. 4q+3) and kScanQuadCodes
// codes per item, every row and frame read issued at once, then reduce16's
// tree across the quad (lanes q, q ^ 2 hold accumulators j, j + 8; lanes 0,
// 1 then hold t3[j], t3[j + 4]).  Otherwise a code per thread, kScanThreads
// codes per item, from the frame staged in xs (its Q8_0 blocks in xq, xd)
// while the block stays on one slot (cur).  x2s: the frame's
// sum_rows(x*x) (Higgs).  Called by every thread of a kScanThreads block.
template <int RECIPE, bool Q8>
__device__ inline bool spread_quad(const StageArgs &a) { return !Q8 && RECIPE != DIRECT && a.order == 0; }
// Whether the open frames of a stage skip the split pass: at most scap of
// them, and their exact values read at most kDirectElems codebook elements
// (count * N * K; 64 MiB of fp32 rows), above which the split pass, which
// reads the fp16 codebook once per 64 open frames, costs less.
constexpr int64_t kDirectElems = int64_t{1} << 24;
__device__ inline bool direct_scan(const StageArgs &a, int count, int K) {
    return count <= a.scap && static_cast<int64_t>(count) * a.N * K <= kDirectElems;
}
template <int RECIPE, bool Q8>
__device__ inline int spread_chunks(const StageArgs &a) {
    const int cpi = spread_quad<RECIPE, Q8>(a) ? kScanQuadCodes : kScanThreads;
    return (a.N + cpi - 1) / cpi;
}
// The quad path's values of one chunk of codes for the frame xr (global
// memory or LDS) into out[n]; x2s (Higgs) is read after a block barrier.
template <int RECIPE, int K>
__device__ void quad_values(const StageArgs &a, float *out, int chunk, const float *xr, float &x2s) {
    const int tid = threadIdx.x;
    {
        const int n = chunk * kScanQuadCodes + tid / 4;
        const int q = tid & 3;
        const int nc = n < a.N ? n : a.N - 1;
        const float *cr = a.cbf + static_cast<int64_t>(nc) * K;
        const float sa = RECIPE == OMNI ? 2.0f : 1.0f;
        // up to 256 elements' reads in flight at once (32 float4 registers)
        constexpr int KC = K < 256 ? K : 256;
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k0 = 0; k0 < K; k0 += KC) {
            f32x4 vc[KC / 16], vx[KC / 16];
#pragma unroll
            for (int l = 0; l < KC / 16; ++l) {
                vc[l] = *reinterpret_cast<const f32x4 *>(cr + k0 + 16 * l + 4 * q);
                vx[l] = *reinterpret_cast<const f32x4 *>(xr + k0 + 16 * l + 4 * q);
            }
#pragma unroll
            for (int l = 0; l < KC / 16; ++l)
#pragma unroll
                for (int t = 0; t < 4; ++t) acc[t] = __fmaf_rn(vc[l][t] * sa, vx[l][t], acc[t]);
        }
        float t3[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) t3[t] = __fadd_rn(__shfl_xor(acc[t], 2), acc[t]);
        float t6[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) t6[t] = __fadd_rn(__shfl_xor(t3[t], 1), t3[t]);
        const float dot = __fadd_rn(__fadd_rn(t6[0], t6[2]), __fadd_rn(t6[1], t6[3]));
        if (RECIPE == HIGGS) __syncthreads();   // x2s
        if (q == 0 && n < a.N) {
            const float v = RECIPE == OMNI ? __fadd_rn(dot, a.bias[n])
                                           : __fsub_rn(__fsub_rn(__fmul_rn(dot, 2.0f), x2s), a.e2[n]);
            out[n] = v;
        }
    }
}
// The values of codes [n0, n1) of the frame xs (LDS) into rv[n] by one
// kScanThreads block in the quad layout of quad_values, two kScanQuadCodes
// chunks per pass with all their row reads issued together.  x2: the
// frame's sum_rows(x*x) (Higgs).
template <int RECIPE, int K>
__device__ void block_values_quad(const StageArgs &a, const float *xs, float x2, float *rv, int n0, int n1) {
    const int tid = threadIdx.x;
    const int q = tid & 3, cl = tid >> 2;
    const float sa = RECIPE == OMNI ? 2.0f : 1.0f;
    constexpr int U = 2;
    f32x4 vx[K / 16];
#pragma unroll
    for (int l = 0; l < K / 16; ++l) vx[l] = *reinterpret_cast<const f32x4 *>(xs + 16 * l + 4 * q);
    for (int c0 = n0; c0 < n1; c0 += U * kScanQuadCodes) {
        f32x4 vc[U][K / 16];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int n = c0 + u * kScanQuadCodes + cl;
            const float *cr = a.cbf + static_cast<int64_t>(n < n1 ? n : n1 - 1) * K;
#pragma unroll
            for (int l = 0; l < K / 16; ++l) vc[u][l] = *reinterpret_cast<const f32x4 *>(cr + 16 * l + 4 * q);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int l = 0; l < K / 16; ++l)
#pragma unroll
                for (int t = 0; t < 4; ++t) acc[t] = __fmaf_rn(vc[u][l][t] * sa, vx[l][t], acc[t]);
            float t3[4], t6[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) t3[t] = __fadd_rn(__shfl_xor(acc[t], 2), acc[t]);
#pragma unroll
            for (int t = 0; t < 4; ++t) t6[t] = __fadd_rn(__shfl_xor(t3[t], 1), t3[t]);
            const float dot = __fadd_rn(__fadd_rn(t6[0], t6[2]), __fadd_rn(t6[1], t6[3]));
            const int n = c0 + u * kScanQuadCodes + cl;
            if (q == 0 && n < n1)
                rv[n] = RECIPE == OMNI ? __fadd_rn(dot, a.bias[n])
                                       : __fsub_rn(__fsub_rn(__fmul_rn(dot, 2.0f), x2), a.e2[n]);
        }
    }
}
// The Higgs values of codes [n0, n1) against a Q8_0 codebook into rv[n] by
// one kScanThreads block: ggml_vec_dot_q8_0_q8_0's eight accumulators (one
// per 4-byte group of a block) on the 8 lanes of a code, hsum_float_8 by DPP
// (hsum8_dpp; dot_q8_k's arithmetic), so that a code row's
// quants are read by 8 neighbouring lanes, two codes per group and pass.
// xq / xd: the frame's quantised blocks (LDS), x2 its sum_rows(x*x).
template <int K>
__device__ void block_values_q8(const StageArgs &a, const int8_t *xq, const float *xd, float x2, float *rv, int n0,
                                int n1) {
    constexpr int NB = K / 32;
    constexpr int G = kScanThreads / 8;   // codes per pass and code slot
    constexpr int P = 2;
    const int j = threadIdx.x & 7, grp = threadIdx.x >> 3;
    const int jw = q8_lane_word(j);
    int xw[NB];
    float xs[NB];
#pragma unroll
    for (int ib = 0; ib < NB; ++ib) {
        xw[ib] = reinterpret_cast<const int *>(xq)[8 * ib + jw];
        xs[ib] = xd[ib];
    }
    for (int c0 = n0; c0 < n1; c0 += P * G) {
        int cq[P][NB];
        float cd[P][NB];
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int n = c0 + p * G + grp;
            const int nn = n < n1 ? n : n1 - 1;
            const int *cqp = reinterpret_cast<const int *>(a.q8 + static_cast<int64_t>(nn) * K) + jw;
            const float *cdp = a.q8d + static_cast<int64_t>(nn) * NB;
#pragma unroll
            for (int ib = 0; ib < NB; ++ib) {
                cq[p][ib] = cqp[8 * ib];
                cd[p][ib] = cdp[ib];
            }
        }
#pragma unroll
        for (int p = 0; p < P; ++p) {
            float acc = 0.0f;
#pragma unroll
            for (int ib = 0; ib < NB; ++ib)
                acc = __fmaf_rn(__fmul_rn(cd[p][ib], xs[ib]),
                                static_cast<float>(__builtin_amdgcn_sdot4(cq[p][ib], xw[ib], 0, false)), acc);
            acc = hsum8_dpp(acc);
            const int n = c0 + p * G + grp;
            if (j == 0 && n < n1) rv[n] = __fsub_rn(__fsub_rn(__fmul_rn(acc, 2.0f), x2), a.e2[n]);
        }
    }
}
template <int RECIPE, bool Q8, int K>
__device__ void spread_item(const StageArgs &a, int slot, int chunk, int &cur, float *xs, int8_t *xq, float *xd,
                            float &x2s) {
    const int tid = threadIdx.x;
    constexpr bool kQuadOk = !Q8 && RECIPE != DIRECT;
    if (kQuadOk && spread_quad<RECIPE, Q8>(a)) {
        const int64_t m = a.fail_list[slot];
        const float *xr = a.xin + m * K;
        __syncthreads();   // the previous item's readers of x2s
        if (RECIPE == HIGGS && tid == 0) x2s = sum_squares_k<K>(xr);
        if constexpr (kQuadOk) quad_values<RECIPE, K>(a, a.svals + static_cast<int64_t>(slot) * a.N, chunk, xr, x2s);
        return;
    }
    if (slot != cur) {
        const int64_t m = a.fail_list[slot];
        __syncthreads();
        for (int k = tid; k < K; k += kScanThreads) xs[k] = a.xin[m * K + k];
        __syncthreads();
        if (tid == 0) x2s = RECIPE == HIGGS ? sum_squares_k<K>(xs) : 0.0f;
        if (Q8 && tid < K / 32) quantize_block_q8(xs + 32 * tid, xq + 32 * tid, xd + tid);
        __syncthreads();
        cur = slot;
    }
    const int n = chunk * kScanThreads + tid;
    if (n < a.N) a.svals[static_cast<int64_t>(slot) * a.N + n] = exact_value_kq<RECIPE, Q8, K>(a, xs, n, x2s, xq, xd);
}

// The exact scan's per-frame arithmetic at the compile-time width K = 32 KS,
// or at the run-time width K (KS = 0: any width).
template <int RECIPE, bool Q8, int KS>
__device__ inline float scan_value(const StageArgs &a, int K, const float *__restrict__ x, int n, float x2,
                                   const int8_t *__restrict__ xq, const float *__restrict__ xd) {
    if constexpr (KS != 0) return exact_value_kq<RECIPE, Q8, KS * 32>(a, x, n, x2, xq, xd);
    else return exact_value<RECIPE, Q8>(a, K, x, n, x2, xq, xd);
}
template <int KS>
__device__ inline float scan_sum_squares(const float *__restrict__ x, int K) {
    if constexpr (KS != 0) {
        return sum_squares_k<KS * 32>(x);
    } else {
        double s = 0.0;
        for (int k = 0; k < K; ++k) s += static_cast<double>(__fmul_rn(x[k], x[k]));
        return static_cast<float>(s);
    }
}

// Shared state of the exact scan's selection for one frame.
struct ScanSh {
    float rv[kScanChunk];
    int heap_n[4];
    float heap_v[4];
    int o_code, o_sel_n[4];
    float o_code_v, o_sel_v[4], o_x2;
    uint64_t w_top[kScanThreads / kWave][5], w_win[kScanThreads / kWave], o_key[5], o_win;
    int w_nan[kScanThreads / kWave];
};

// The exact scan's selection for one frame, by a whole kScanThreads block:
// every code's recipe value (from sv when pre, else computed from the frame
// xs in LDS, with x2 its sum_rows(x*x) and xq / xd its Q8_0 blocks) and the
// reference's selection rules; the winner and the top-k land in
// sh.o_code / o_code_v / o_sel_n / o_sel_v.
template <int RECIPE, bool Q8, int KS>
__device__ void scan_select(const StageArgs &a, int K, bool pre, const float *sv, const float *xs, const int8_t *xq,
                            const float *xd, float x2, ScanSh &sh) {
    constexpr int ST = kScanThreads;
    constexpr int PT = kScanChunk / ST;   // values per thread of a one-chunk frame
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int ktop = a.topk;
    float *rv = sh.rv;
    int *heap_n = sh.heap_n;
    float *heap_v = sh.heap_v;
    int &o_code = sh.o_code;
    int *o_sel_n = sh.o_sel_n;
    float &o_code_v = sh.o_code_v;
    float *o_sel_v = sh.o_sel_v;
    uint64_t(*w_top)[5] = sh.w_top;
    uint64_t *w_win = sh.w_win;
    uint64_t *o_key = sh.o_key;
    uint64_t &o_win = sh.o_win;
    int *w_nan = sh.w_nan;
    auto value = [&](int n) -> float { return pre ? sv[n] : scan_value<RECIPE, Q8, KS>(a, K, xs, n, x2, xq, xd); };
    // The frame's values.  Codes that fit one chunk (N <= kScanChunk):
    // PT per thread in registers (code tid + j * ST), and all in rv in
    // code order; more codes: read from the grid's values (pre), or
    // computed chunk by chunk by the walk below.
    const bool have_all = pre || a.N <= kScanChunk;
    const bool in_regs = a.N <= kScanChunk;
    float vr[PT];
    if (in_regs && pre) {
#pragma unroll
        for (int j = 0; j < PT; ++j) {
            const int i = tid + j * ST;
            vr[j] = i < a.N ? sv[i] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < PT; ++j)
            if (tid + j * ST < a.N) rv[tid + j * ST] = vr[j];
    } else if (in_regs) {
#pragma unroll 4
        for (int i = tid; i < a.N; i += ST) rv[i] = scan_value<RECIPE, Q8, KS>(a, K, xs, i, x2, xq, xd);
    }
    __syncthreads();
    if (in_regs && !pre) {
#pragma unroll
        for (int j = 0; j < PT; ++j) {
            const int i = tid + j * ST;
            vr[j] = i < a.N ? rv[i] : 0.0f;
        }
    }
    // Parallel selection, unless a ggml recipe meets a NaN (its argmax
    // restarts there) or the values are not all at hand: the winner and
    // the best L codes in rank_key order.  Each wave takes L rounds of a
    // wave-wide max over its keys below the previous round's, then wave
    // 0 does the same over the waves' lists.
    bool slow = !have_all;
    bool tie = false;
    if (have_all) {
        const int L = RECIPE == DIRECT ? (ktop > 1 ? ktop : 1) : ktop + 1;
        const int wv = tid / kWave;
        bool nan = false;
        uint64_t kr[PT];
#pragma unroll
        for (int j = 0; j < PT; ++j) {
            const bool ok = in_regs && tid + j * ST < a.N;
            nan |= ok && vr[j] != vr[j];
            kr[j] = ok ? rank_key<RECIPE>(vr[j], tid + j * ST) : 0;
        }
        uint64_t prev = ~0ull;
        for (int r = 0; r < L; ++r) {
            const bool want_w = RECIPE != DIRECT && r == 0;   // ggml argmax: the largest value, its last index
            uint64_t best = 0, wb = 0;
            auto consider = [&](uint64_t k, int i) {
                best = k < prev && k > best ? k : best;
                const uint64_t w = (k & 0xFFFFFFFF00000000ull) | static_cast<uint32_t>(i);
                if (want_w && k != 0 && w > wb) wb = w;
            };
            if (in_regs) {
#pragma unroll
                for (int j = 0; j < PT; ++j) consider(kr[j], tid + j * ST);
            } else {
                for (int i = tid; i < a.N; i += ST) {
                    const float v = sv[i];
                    nan |= v != v;
                    consider(rank_key<RECIPE>(v, i), i);
                }
            }
            best = wave_max_u64(best);
            if (lane == 0) w_top[wv][r] = best;
            if (want_w) {
                wb = wave_max_u64(wb);
                if (lane == 0) w_win[wv] = wb;
            }
            prev = best;
        }
        if (RECIPE != DIRECT) {
            const bool wnan = __any(nan);
            if (lane == 0) w_nan[wv] = wnan ? 1 : 0;
        }
        __syncthreads();
        if (RECIPE != DIRECT)
            for (int w = 0; w < ST / kWave; ++w) slow |= w_nan[w] != 0;
        if (!slow) {
            if (wv == 0) {
                const uint64_t c = lane < (ST / kWave) * L ? w_top[lane / L][lane % L] : 0;
                uint64_t pv = ~0ull;
                for (int r = 0; r < L; ++r) {
                    const uint64_t b = wave_max_u64(c < pv ? c : 0);
                    if (lane == 0) o_key[r] = b;
                    pv = b;
                }
                if (RECIPE != DIRECT && lane == 0) {
                    uint64_t w = w_win[0];
                    for (int q = 1; q < ST / kWave; ++q) w = w_win[q] > w ? w_win[q] : w;
                    o_win = w;
                }
            }
            __syncthreads();
            // ggml_top_k keeps, of codes tied at the k-th place, what its
            // heap leaves: replayed below
            tie = RECIPE != DIRECT && ktop > 0 && o_key[ktop] != 0 && (o_key[ktop - 1] >> 32) == (o_key[ktop] >> 32);
            if (tid == 0) {
                // an index below 0 stands for no code (key 0: DIRECT with
                // every value NaN, or fewer codes than places).  Tested on
                // the index, not as key == 0: ROCm 7.2's compiler lowered
                // (key == 0 ? 0 : key_index(key)) here to a scalar select
                // on the flag of the preceding s_not_b32, i.e. always 0.
                const int n = RECIPE == DIRECT ? key_index(o_key[0]) : static_cast<int>(static_cast<uint32_t>(o_win));
                o_code = n < 0 ? 0 : n;
                o_code_v = n < 0 ? INFINITY : (in_regs ? rv[n] : sv[n]);
                if (!tie)
                    for (int r = 0; r < ktop; ++r) {
                        const int q = key_index(o_key[r]);
                        o_sel_n[r] = q < 0 ? 0 : q;
                        o_sel_v[r] = q < 0 ? INFINITY : (in_regs ? rv[q] : sv[q]);
                    }
            }
            if (tie && wv == 0) {
                // rv (LDS) and sv (global) in separate instances, so that
                // each reads through its own address space
                switch (ktop) {
                    case 1: in_regs ? heap_walk<1>(rv, a.N, heap_n, heap_v) : heap_walk<1>(sv, a.N, heap_n, heap_v); break;
                    case 2: in_regs ? heap_walk<2>(rv, a.N, heap_n, heap_v) : heap_walk<2>(sv, a.N, heap_n, heap_v); break;
                    case 3: in_regs ? heap_walk<3>(rv, a.N, heap_n, heap_v) : heap_walk<3>(sv, a.N, heap_n, heap_v); break;
                    default: in_regs ? heap_walk<4>(rv, a.N, heap_n, heap_v) : heap_walk<4>(sv, a.N, heap_n, heap_v); break;
                }
            }
        }
    }
    // The walk (a ggml recipe with a NaN, or values computed chunk by
    // chunk): wave 0 replays the reference's sequential selection.
    // wave 0's running selection state (uniform across its lanes)
    float mx = RECIPE == DIRECT ? INFINITY : -INFINITY;
    int id = 0;
    float root = 0.0f;   // heap root (ggml recipes) / k-th kept distance (DIRECT)
    int kept = 0;        // DIRECT: entries in the kept list
    for (int base = 0; base < (slow ? a.N : 0); base += kScanChunk) {
        const int len = min(kScanChunk, a.N - base);
        // unrolled so that the row loads of several codes are in flight at
        // once; a single chunk is in rv since pass 1
        if (a.N > kScanChunk) {
#pragma unroll 4
            for (int i = tid; i < len; i += ST) rv[i] = value(base + i);
        }
        __syncthreads();
        if (tid < kWave) {
            for (int c0 = 0; c0 < len; c0 += kWave) {
                const int i = c0 + lane;
                const bool in = i < len;
                const float v = in ? rv[i] : 0.0f;
                if (RECIPE == DIRECT) {
                    // first index of the minimum: strict <, NaN never wins
                    // (a chunk with no code below the running minimum is
                    // skipped after one ballot)
                    float cm = INFINITY;
                    if (__any(in && v < mx)) {
                        cm = in ? v : INFINITY;
#pragma unroll
                        for (int off = 1; off < kWave; off <<= 1) cm = fminf(cm, __shfl_xor(cm, off));
                    }
                    if (cm < mx) {
                        const unsigned long long eq = __ballot(in && v == cm);
                        const int first = __ffsll(static_cast<long long>(eq)) - 1;
                        mx = cm;
                        id = base + c0 + first;
                    }
                    if (ktop > 0) {
                        // the k smallest (value, index): insert, in code
                        // order, every code that ranks before the k-th
                        int from = 0;
                        while (true) {
                            const bool cand = in && lane >= from && v == v &&
                                              (kept < ktop || v < root);
                            const unsigned long long take = __ballot(cand);
                            if (take == 0) break;
                            const int f = __ffsll(static_cast<long long>(take)) - 1;
                            const float vf = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), f));
                            if (lane == 0) {
                                int p = kept < ktop ? kept : ktop - 1;
                                while (p > 0 && vf < heap_v[p - 1]) {
                                    heap_v[p] = heap_v[p - 1];
                                    heap_n[p] = heap_n[p - 1];
                                    --p;
                                }
                                heap_v[p] = vf;
                                heap_n[p] = base + c0 + f;
                            }
                            __builtin_amdgcn_wave_barrier();
                            kept = min(kept + 1, ktop);
                            root = heap_v[ktop - 1];
                            from = f + 1;
                        }
                    }
                    continue;
                }
                // ggml_vec_argmax_f32
                const bool nan_chunk = __any(in && v != v) || mx != mx;
                if (nan_chunk) {
                    const int cl = min(kWave, len - c0);
                    for (int t = 0; t < cl; ++t) {
                        const float vt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), t));
                        mx = mx > vt ? mx : vt;
                        if (mx == vt) id = base + c0 + t;
                    }
                } else if (__any(in && v >= mx)) {
                    // only a chunk with a code >= the running max can
                    // move the argmax (MAX keeps a later equal element)
                    float cm = in ? v : -INFINITY;
#pragma unroll
                    for (int off = 1; off < kWave; off <<= 1) cm = fmaxf(cm, __shfl_xor(cm, off));
                    const unsigned long long eq = __ballot(in && v == cm);
                    if (eq != 0 && !(mx > cm)) {
                        const int last = 63 - __clzll(static_cast<long long>(eq));
                        mx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), last));
                        id = base + c0 + last;
                    }
                }
                if (ktop > 0) {
                    // ggml_top_k: the first ktop codes build the heap,
                    // a later code replaces the root if strictly better
                    for (int t = 0; t < kWave && base + c0 + t < ktop; ++t) {
                        const int n_t = base + c0 + t;
                        const float vt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), t));
                        if (lane == 0) {
                            heap_n[n_t] = n_t;
                            heap_v[n_t] = vt;
                            if (n_t == ktop - 1 && ktop >= 2)
                                for (int par = (ktop - 2) / 2;; --par) {
                                    heap_adjust(heap_n, heap_v, par, ktop, heap_n[par], heap_v[par]);
                                    if (par == 0) break;
                                }
                        }
                        __builtin_amdgcn_wave_barrier();
                        if (n_t == ktop - 1) root = heap_v[0];
                    }
                    int from = 0;   // lanes before `from` are done
                    while (true) {
                        const unsigned long long take =
                            __ballot(in && lane >= from && base + i >= ktop && v > root);
                        if (take == 0) break;
                        const int f = __ffsll(static_cast<long long>(take)) - 1;
                        const float vf = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), f));
                        if (lane == 0) heap_adjust(heap_n, heap_v, 0, ktop, base + c0 + f, vf);
                        __builtin_amdgcn_wave_barrier();
                        root = heap_v[0];
                        from = f + 1;
                    }
                }
            }
        }
        __syncthreads();
    }
    if (tid == 0 && (slow || tie)) {
        if (slow) {
            o_code = id;
            o_code_v = mx;
        }
        // the kept set, best first, ties by index
        int used[4] = {-1, -1, -1, -1};
        const int nk = RECIPE == DIRECT ? kept : ktop;
        for (int r = 0; r < ktop; ++r) {
            int b = -1;
            for (int q = 0; q < nk; ++q) {
                bool u = false;
                for (int t = 0; t < r; ++t) u |= used[t] == q;
                if (!u && (b < 0 || topk_before<RECIPE>(heap_v[q], heap_n[q], heap_v[b], heap_n[b]))) b = q;
            }
            used[r] = b;
            o_sel_n[r] = b < 0 ? 0 : heap_n[b];
            o_sel_v[r] = b < 0 ? INFINITY : heap_v[b];
        }
    }
    __syncthreads();
}

template <int RECIPE, bool Q8, int KS>
__global__ __launch_bounds__(kScanThreads) void euclid_exact_scan_kernel(StageArgs a) {
    // KS = 0: the width is a run-time argument and every frame of the batch
    // is scanned (no frame list, no spread values)
    const int K = KS != 0 ? KS * 32 : a.K;
    constexpr int ST = kScanThreads;
    extern __shared__ __align__(16) unsigned char lds[];
    float *xs = reinterpret_cast<float *>(lds);                         // [K]
    int8_t *xq = reinterpret_cast<int8_t *>(xs + K);                    // [K]
    float *xd = reinterpret_cast<float *>(xq + K);                      // [K/32]
    __shared__ ScanSh sh;
    int &o_code = sh.o_code;
    int *o_sel_n = sh.o_sel_n;
    float &o_code_v = sh.o_code_v, *o_sel_v = sh.o_sel_v, &o_x2 = sh.o_x2;
    const int tid = threadIdx.x;
    const int count = KS != 0 ? *a.fail_count : static_cast<int>(a.M);
    // pre: up to a.scap frames, whose code values the grid computes first
    // (one (frame, kScanThreads-code chunk) item per block and pass); the
    // block that completes a frame's last chunk selects for it
    const bool pre = KS != 0 && count <= a.scap;
    __shared__ int o_last;
    auto scan_slot = [&](int slot) {
        const int64_t m = KS != 0 ? a.fail_list[slot] : slot;
        __syncthreads();
        if (!pre) {
            for (int k = tid; k < K; k += ST) xs[k] = a.xin[m * K + k];
            __syncthreads();
            if (tid == 0) o_x2 = RECIPE == HIGGS ? scan_sum_squares<KS>(xs, K) : 0.0f;   // unrolled: LDS reads in flight
            if (Q8 && tid < K / 32) quantize_block_q8(xs + 32 * tid, xq + 32 * tid, xd + tid);
            __syncthreads();
        }
        const float x2 = pre ? 0.0f : o_x2;
        const float *sv = pre ? a.svals + static_cast<int64_t>(slot) * a.N : nullptr;
        scan_select<RECIPE, Q8, KS>(a, K, pre, sv, xs, xq, xd, x2, sh);
        __syncthreads();
        const int code = o_code;
        if (tid == 0) {
            a.idx[m * a.Q + a.s] = code;
            if (a.dist) a.dist[m * a.Q + a.s] = RECIPE == DIRECT ? o_code_v : -o_code_v;
            for (int r = 0; r < a.topk; ++r) {
                a.topk_idx[(m * a.Q + a.s) * a.topk + r] = o_sel_n[r];
                a.topk_dist[(m * a.Q + a.s) * a.topk + r] = RECIPE == DIRECT ? o_sel_v[r] : -o_sel_v[r];
            }
        }
        int use = code;
        if (a.force_idx) {
            use = a.force_idx[m * a.Q + a.s];
            if (use < 0 || use >= a.N) {
                if (tid == 0) a.flags[AQ_FLAG_BAD_INDEX] = 1;
                use = 0;
            }
        }
        if (a.xout)
            for (int k = tid; k < K; k += ST)
                a.xout[m * K + k] = __fsub_rn(a.xin[m * K + k], a.cbf[static_cast<int64_t>(use) * K + k]);
    };
    // Values already spread by the refine_values launch: the select left
    // few open frames (direct_scan), and refine_select handed them all on
    // (the kernel boundary orders their values before these reads).
    const bool ready = pre && a.open_count != nullptr && direct_scan(a, *a.open_count, K);
    if (!pre || ready) {
        for (int slot = blockIdx.x; slot < count; slot += gridDim.x) scan_slot(slot);
        return;
    }
    if constexpr (KS != 0) {
    const int nch = spread_chunks<RECIPE, Q8>(a);
    int cur = -1;
    for (int item = blockIdx.x; item < count * nch; item += gridDim.x) {
        const int slot = item / nch;   // block-uniform
        spread_item<RECIPE, Q8, KS * 32>(a, slot, item % nch, cur, xs, xq, xd, o_x2);
        // release: this block's values before the frame's counter; the block
        // that brings it to nch sees every chunk's values after its acquire
        __threadfence();
        __syncthreads();
        if (tid == 0) o_last = atomicAdd(&a.slot_done[slot], 1) == nch - 1;
        __syncthreads();
        if (o_last) {
            __threadfence();
            scan_slot(slot);
            if (tid == 0) a.slot_done[slot] = 0;   // ready for the next stage
            cur = -1;                              // scan_slot used xs
        }
    }
    }
}

// ------------------------------------------------------------- refine pass

// Frames the fp16 certificate leaves open are scored again with split fp16
// operands before any exact scan.  With x = x_h + x_l + x_r and
// c = c_h + c_l + c_r (x_h = fp16(x), x_l = fp16(x - x_h), x_r the exact
// remainder; likewise c), the refined score is
//   s(n) = x_h.c_h + (x_h.c_l + x_l.c_h) - |c_n|^2/2
// from three MFMAs per K slice.  The dropped terms x_h.c_r + x_l.c_l +
// x_l.c_r + x_r.c are bounded by Cauchy-Schwarz with the frame's |x_h|,
// |x_l|, |x_r| and the codebook's largest |c_l|, |c_r|, |c|: about 2^-22 of
// |x||c|, against 2^-11 for plain fp16 (less where x_l or c_l fall into
// fp16's subnormal range; the bounds use the measured remainders).  The
// same certificate as in the stage kernel then settles nearly every open
// frame; the rest go to the exact scan.  When no more open frames than the
// exact scan spreads over the grid are left, the pass is skipped:
// refine_values computes their exact values over the grid instead,
// refine_select hands the list on, and the exact scan selects.
//  * refine_values: a wave takes 16 open frames x one slice of rs codes and
//    keeps, per lane, its kTopR best keys (score with the slice-local code
//    index in the low 6 mantissa bits) in a key buffer.
//  * refine_select: a wave per frame merges the key lists of all slices,
//    evaluates every key within 2E of the T-th key exactly, applies the
//    certificate and writes codes, distances, top-k and the residual.


// LDS image of one 16-code block for the refine pass: fp16 high and low
// rows (XOR-swizzled 16-byte pieces, as in the sweep) and -|c|^2/2.
template <int KS>
struct RefTile {
    static constexpr int K = KS * 32;
    static constexpr int ROWB = K * 2;
    static constexpr int CH16 = K / 8;
    static constexpr int SWZ = CH16 >= 16 ? 15 : CH16 - 1;
    static constexpr int ROWS16 = 16 * CH16;                    // 16-byte pieces per 16-row array
    static constexpr int PIECES = 2 * ROWS16;                   // high + low
    static constexpr int STG = (PIECES + kThreads - 1) / kThreads;
    static constexpr int BUFB = 2 * 16 * ROWB + 16 * 4;
};

template <int RECIPE, bool Q8, int KS>
__global__ __launch_bounds__(kWave * kRWaves, KS <= 8 ? 2 : 1) void euclid_refine_values_kernel(StageArgs a, RefArgs rf) {
    using T = RefTile<KS>;
    constexpr int K = KS * 32;
    static_assert(kWave * kRWaves == kThreads && kThreads == kScanThreads,
                  "refine blocks have the sweep's and the spread items' shape");
    __shared__ __align__(16) unsigned char lds[2 * T::BUFB];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int col = lane & 15, kq = lane >> 4;
    const int open = *a.fail_count;
    if (direct_scan(a, open, K)) {
        // Few open frames: no split pass.  Their exact values, spread over
        // the grid, for the exact scan, which then only selects.
        float *xs = reinterpret_cast<float *>(lds);
        int8_t *xq = reinterpret_cast<int8_t *>(xs + K);
        float *xd = reinterpret_cast<float *>(xq + K);
        float *x2s = xd + K / 32;
        const int nch = spread_chunks<RECIPE, Q8>(a);
        int cur = -1;
        for (int item = blockIdx.x; item < open * nch; item += gridDim.x)
            spread_item<RECIPE, Q8, K>(a, item / nch, item % nch, cur, xs, xq, xd, *x2s);
        return;
    }
    const RefShape rsh = ref_shape(rf, a.N, open);
    const int count = rsh.cap;
    const int ntiles = (count + 16 * kRWaves - 1) / (16 * kRWaves);
    const int64_t nwork = static_cast<int64_t>(ntiles) * rsh.nslices;
    unsigned vkeep;
    asm volatile("v_mov_b32 %0, %1" : "=v"(vkeep) : "s"(~63u));

    auto piece_off = [&](int buf, int p) -> int {   // byte offset of staged piece p
        const int arr = p / T::ROWS16, q = p % T::ROWS16;
        const int r = q / T::CH16, j = q % T::CH16;
        return buf * T::BUFB + arr * (16 * T::ROWB) + r * T::ROWB + ((j ^ (r & T::SWZ)) * 16);
    };
    using MX = Mx;
    auto lds_a = [&](int buf, int arr, int ks) -> typename MX::V8 {
        const int j = ks * 4 + kq;
        return *reinterpret_cast<const typename MX::V8 *>(lds + buf * T::BUFB + arr * (16 * T::ROWB) + col * T::ROWB +
                                                 ((j ^ (col & T::SWZ)) * 16));
    };
    // global source of piece p of block n16 (16 codes from n16)
    auto piece_src = [&](int n16, int p) -> const u32x4 * {
        const int arr = p / T::ROWS16, q = p % T::ROWS16;
        const uint16_t *base = arr == 0 ? a.cbh : rf.cbl;
        return reinterpret_cast<const u32x4 *>(base + static_cast<int64_t>(n16) * K) + q;
    };

    for (int64_t w = blockIdx.x; w < nwork; w += gridDim.x) {
        const int tile = static_cast<int>(w / rsh.nslices), sl = static_cast<int>(w % rsh.nslices);
        const int fs = (tile * kRWaves + wave) * 16 + col;
        const int64_t m = a.fail_list[fs < count ? fs : count - 1];
        const float *xr = a.xin + m * K;
        u32x4 xh[KS], xl[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const f32x4 lo = *reinterpret_cast<const f32x4 *>(xr + ks * 32 + kq * 8);
            const f32x4 hi = *reinterpret_cast<const f32x4 *>(xr + ks * 32 + kq * 8 + 4);
            float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            if (Q8) q8_image_block(v);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                using E = typename MX::E;
                const typename MX::V2 ph = {static_cast<E>(v[2 * t]), static_cast<E>(v[2 * t + 1])};
                const unsigned wh = __builtin_bit_cast(unsigned, ph);
                const float d0 = v[2 * t] - MX::lo(wh);
                const float d1 = v[2 * t + 1] - MX::hi(wh);
                const typename MX::V2 pl = {static_cast<E>(d0), static_cast<E>(d1)};
                xh[ks][t] = wh;
                xl[ks][t] = __builtin_bit_cast(unsigned, pl);
            }
        }
        float top[kTopR];
#pragma unroll
        for (int j = 0; j < kTopR; ++j) top[j] = -INFINITY;
        const int n0 = sl * rsh.rs;
        const int nb = min(rsh.rs, a.N - n0) / 16;

        // stage block 0 of the slice
        __syncthreads();   // the previous work item's last reads of buffer 0/1
#pragma unroll
        for (int i = 0; i < T::STG; ++i) {
            const int p = threadIdx.x + i * kThreads;
            if (p < T::PIECES) *reinterpret_cast<u32x4 *>(lds + piece_off(0, p)) = *piece_src(n0, p);
        }
        if (threadIdx.x < 16) reinterpret_cast<float *>(lds + 2 * 16 * T::ROWB)[threadIdx.x] = a.nhh[n0 + threadIdx.x];
        __syncthreads();
        for (int b = 0; b < nb; ++b) {
            const int buf = b & 1;
            const bool more = b + 1 < nb;
            // the next block's pieces are fetched while this one computes
            u32x4 stg[T::STG];
            float hst = 0.0f;
            if (more) {
#pragma unroll
                for (int i = 0; i < T::STG; ++i) {
                    const int p = threadIdx.x + i * kThreads;
                    if (p < T::PIECES) stg[i] = *piece_src(n0 + (b + 1) * 16, p);
                }
                if (threadIdx.x < 16) hst = a.nhh[n0 + (b + 1) * 16 + threadIdx.x];
            }
            f32x4 acc = *reinterpret_cast<const f32x4 *>(lds + buf * T::BUFB + 2 * 16 * T::ROWB + kq * 16);
            f32x4 acx = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const typename MX::V8 ah = lds_a(buf, 0, ks);
                const typename MX::V8 al = lds_a(buf, 1, ks);
                const typename MX::V8 bh = __builtin_bit_cast(typename MX::V8, xh[ks]);
                acc = MX::mfma(ah, bh, acc);
                acx = MX::mfma(al, bh, acx);
                acx = MX::mfma(ah, __builtin_bit_cast(typename MX::V8, xl[ks]), acx);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float key = key_of(acc[i] + acx[i], static_cast<unsigned>(b * 4 + i), vkeep);
#pragma unroll
                for (int j = kTopR - 1; j > 0; --j) top[j] = __builtin_amdgcn_fmed3f(top[j - 1], top[j], key);
                top[0] = __builtin_amdgcn_fmed3f(top[0], key, 3.40282347e38f);
            }
            if (more) {
#pragma unroll
                for (int i = 0; i < T::STG; ++i) {
                    const int p = threadIdx.x + i * kThreads;
                    if (p < T::PIECES) *reinterpret_cast<u32x4 *>(lds + piece_off(buf ^ 1, p)) = stg[i];
                }
                if (threadIdx.x < 16) reinterpret_cast<float *>(lds + (buf ^ 1) * T::BUFB + 2 * 16 * T::ROWB)[threadIdx.x] = hst;
            }
            __syncthreads();
        }
        if (fs < count) {
            f32x4 *dst = reinterpret_cast<f32x4 *>(rf.keys + ((static_cast<int64_t>(fs) * rsh.nslices + sl) * 4 + kq) * kTopR);
            *dst = f32x4{top[0], top[1], top[2], top[3]};
        }
    }
}

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) v += __shfl_xor(v, off);
    return v;
}

// Exact values of one frame's candidates cn[0 .. ncand), in exact_value_kq's
// arithmetic, with several candidates per pass and coalesced row reads:
//  * tinyBLAS order: 16 lanes per candidate, lane j accumulating the
//    elements k = 16 l + j, then _mm512_reduce_add_ps's pairing tree as DPP
//    row rotations 8, 4, 2, 1; two candidates per 16-lane row and pass, so
//    that their row reads are in flight together;
//  * Q8_0 (ggml_vec_dot_q8_0_q8_0): 8 lanes per candidate, lane j taking the
//    j-th 4-element group of every block, then hsum_float_8 as lane
//    exchanges 4, 2, 1;
//  * otherwise one candidate per lane.
// x, xq, xd may live in LDS; every lane of the wave calls this.
template <int RECIPE, bool Q8, int K>
__device__ void exact_values_frame(const StageArgs &a, const float *__restrict__ x, float x2, const int8_t *xq,
                                   const float *xd, const int *cn, float *cv, int ncand, int lane) {
    if (!Q8 && RECIPE != DIRECT && a.order == 0) {
        constexpr int P = 2;
        const int j = lane & 15, grp = lane >> 4;
        const float sa = RECIPE == OMNI ? 2.0f : 1.0f;
        for (int c0 = grp; c0 < ncand; c0 += 4 * P) {
            int n[P];
            float acc[P];
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const int c = c0 + 4 * p;
                n[p] = cn[c < ncand ? c : c0];
                acc[p] = 0.0f;
            }
#pragma unroll
            for (int l = 0; l < K / 16; ++l)
#pragma unroll
                for (int p = 0; p < P; ++p)
                    acc[p] = __fmaf_rn(a.cbf[static_cast<int64_t>(n[p]) * K + 16 * l + j] * sa, x[16 * l + j], acc[p]);
#pragma unroll
            for (int p = 0; p < P; ++p) {
                float v = row_ror_add<8>(acc[p]);
                v = row_ror_add<4>(v);
                v = row_ror_add<2>(v);
                v = row_ror_add<1>(v);
                const int c = c0 + 4 * p;
                if (j == 0 && c < ncand)
                    cv[c] = RECIPE == OMNI ? __fadd_rn(v, a.bias[n[p]])
                                           : __fsub_rn(__fsub_rn(__fmul_rn(v, 2.0f), x2), a.e2[n[p]]);
            }
        }
    } else if (Q8) {
        const int j = lane & 7, grp = lane >> 3;
        const int *xqi = reinterpret_cast<const int *>(xq) + j;
        for (int c = grp; c < ncand; c += 8) {
            const int n = cn[c];
            const int *cq = reinterpret_cast<const int *>(a.q8 + static_cast<int64_t>(n) * K) + j;
            const float *cd = a.q8d + static_cast<int64_t>(n) * (K / 32);
            float acc = 0.0f;
#pragma unroll
            for (int ib = 0; ib < K / 32; ++ib) {
                const float dd = __fmul_rn(cd[ib], xd[ib]);
                acc = __fmaf_rn(dd, static_cast<float>(__builtin_amdgcn_sdot4(cq[8 * ib], xqi[8 * ib], 0, false)), acc);
            }
            acc = __fadd_rn(acc, __shfl_xor(acc, 4));
            acc = __fadd_rn(acc, __shfl_xor(acc, 2));
            acc = __fadd_rn(acc, __shfl_xor(acc, 1));
            if (j == 0) cv[c] = __fsub_rn(__fsub_rn(__fmul_rn(acc, 2.0f), x2), a.e2[n]);
        }
    } else {
        for (int c = lane; c < ncand; c += kWave) cv[c] = exact_value_kq<RECIPE, Q8, K>(a, x, cn[c], x2, xq, xd);
    }
}

template <int RECIPE, bool Q8, int KS>
__global__ __launch_bounds__(kWave) void euclid_refine_select_kernel(StageArgs a, RefArgs rf) {
    constexpr int K = KS * 32;
    constexpr int KPL = K / kWave;   // frame elements per lane
    __shared__ int cand_n[kRCand];
    __shared__ float cand_v[kRCand];
    __shared__ float keys_s[kRKeyLds];     // the frame's keys of every slice
    __shared__ float xs[K];                // the frame (exact evaluation reads it here)
    __shared__ int8_t xq[Q8 ? K : 4];      // its Q8_0 blocks
    __shared__ float xd[Q8 ? K / 32 : 1];
    __shared__ float x2s;
    const int lane = threadIdx.x;
    const float u = 5.9604645e-8f;   // 2^-24
    const int Tk = a.topk > 0 ? a.topk : 1;
    const int Tsel = a.topk > 0 ? a.topk + 1 : 1;
    const int count = *a.fail_count;
    if (direct_scan(a, count, K)) {
        // few open frames: no split pass, the exact scan takes the list
        if (blockIdx.x == 0) {
            for (int i = lane; i < count; i += kWave) rf.list2[i] = a.fail_list[i];
            if (lane == 0) *rf.count2 = count;
        }
        return;
    }
    const RefShape rsh = ref_shape(rf, a.N, count);
    const int nk = rsh.nslices * 4 * kTopR;
    for (int slot = blockIdx.x; slot < count; slot += gridDim.x) {
        const int64_t m = a.fail_list[slot];
        const float *xr = a.xin + m * K;
        bool ok = slot < rsh.cap && !a.exact_only;

        // Norms of the split of x (of its Q8_0 image for a Q8_0 codebook).
        // Element k = lane + 64 j; a 32-wide Q8_0 block is 32 adjacent lanes.
        float sh = 0.0f, sl = 0.0f, sr = 0.0f, sxx = 0.0f;
#pragma unroll
        for (int j = 0; j < KPL; ++j) {
            float v = xr[lane + kWave * j];
            xs[lane + kWave * j] = v;
            if (Q8) {
                float am = fabsf(v);
#pragma unroll
                for (int off = 1; off < 32; off <<= 1) am = fmaxf(am, __shfl_xor(am, off));
                const float dq = static_cast<float>(static_cast<_Float16>(__fdiv_rn(am, 127.0f)));
                const float id = am != 0.0f ? __fdiv_rn(127.0f, am) : 0.0f;
                v = __fmul_rn(__builtin_rintf(__fmul_rn(v, id)), dq);
            }
            const float h = static_cast<float>(static_cast<Mx::E>(v));
            const float d = v - h;
            const float l = static_cast<float>(static_cast<Mx::E>(d));
            const float r = d - l;
            sh = __fmaf_rn(h, h, sh);
            sl = __fmaf_rn(l, l, sl);
            sr = __fmaf_rn(r, r, sr);
            sxx = __fmaf_rn(v, v, sxx);
        }
        const float nxh = sqrtf(wave_sum(sh)) * 1.0001f, nxl = sqrtf(wave_sum(sl)) * 1.0001f;
        const float nxr = sqrtf(wave_sum(sr)) * 1.0001f, nxx2 = wave_sum(sxx);
        const float nxe = nxh + nxl + nxr;   // >= |x|
        // Bound E (v units) on |s(n) - S'(n)| for every code n: dropped split
        // terms, fp32 accumulation of 3K products from -|c|^2/2, the recipe's
        // own fp32 rounding, and the 6 index bits of the keys.
        const float e_split = nxh * rf.crmax + nxl * rf.clmax + nxl * rf.crmax + nxr * a.cmax;
        const float mag = nxh * a.chmax + nxh * rf.clmax + nxl * a.chmax + 0.5f * a.cmax * a.cmax;
        const float e_acc = (3 * K + 8) * u * mag;
        const float e_rec = (K + 16) * u * (nxe * a.cmax + nxe * nxe + a.cmax * a.cmax);
        const float vmax = mag + e_acc;
        const float E = 1.02f * (e_split + e_acc + e_rec + 4.0f * u * vmax) + ldexpf(vmax, 6 - 23) + 1e-30f;
        ok = ok && (E < INFINITY);

        // Keys of every slice: tau bounds every code a lane dropped; vT is
        // the T-th largest key (ties by position).
        // Keys exist only for slots below the capacity (refine_values wrote
        // them); a frame past it, or with E = inf, reads none and goes to the
        // exact scan.  `ok` is uniform over the block (one wave; E comes from
        // butterfly sums), so the barriers below are reached by every lane.
        const float *kp = rf.keys + static_cast<int64_t>(slot) * nk;
        // The frame's keys are read three times below: from LDS when they fit.
        if (ok && nk <= kRKeyLds) {
            __syncthreads();   // the previous frame's reads of keys_s
            for (int e0 = 0; e0 < nk; e0 += 16 * kWave) {   // 16 loads in flight per lane
                float t[16];
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int e = e0 + j * kWave + lane;
                    t[j] = e < nk ? kp[e] : 0.0f;
                }
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int e = e0 + j * kWave + lane;
                    if (e < nk) keys_s[e] = t[j];
                }
            }
            __syncthreads();
            kp = keys_s;
        }
        float tau = -INFINITY;
        float vT = -INFINITY;
        int ncand = 0;
        if (ok) {
            for (int e = lane * kTopR + kTopR - 1; e < nk; e += kWave * kTopR) tau = fmaxf(tau, kp[e]);
#pragma unroll
            for (int off = 1; off < kWave; off <<= 1) tau = fmaxf(tau, __shfl_xor(tau, off));
            float pv = INFINITY;
            int pp = -1;
            for (int t = 0; t < Tk; ++t) {
                float bv = -INFINITY;
                int bp = 0x7fffffff;
                for (int e = lane; e < nk; e += kWave) {
                    const float kv = kp[e];
                    const bool after = kv < pv || (kv == pv && e > pp);
                    if (after && (kv > bv || (kv == bv && e < bp))) {
                        bv = kv;
                        bp = e;
                    }
                }
#pragma unroll
                for (int off = 1; off < kWave; off <<= 1) {
                    const float ov = __shfl_xor(bv, off);
                    const int op = __shfl_xor(bp, off);
                    if (ov > bv || (ov == bv && op < bp)) {
                        bv = ov;
                        bp = op;
                    }
                }
                pv = bv;
                pp = bp;
            }
            vT = pv;
            ok = (vT - vT == 0.0f);
        }
        if (ok) {
            const float thr = vT - 2.0f * E;
            for (int e0 = 0; e0 < nk; e0 += kWave) {
                const int e = e0 + lane;
                const float kv = e < nk ? kp[e] : -INFINITY;
                const bool c = e < nk && kv >= thr && kv > -INFINITY;
                const unsigned long long bal = __ballot(c);
                const int pos = ncand + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                                            static_cast<unsigned>(bal >> 32),
                                            __builtin_amdgcn_mbcnt_lo(static_cast<unsigned>(bal), 0u)));
                if (c && pos < kRCand) {
                    const int slc = e / (4 * kTopR), q = (e / kTopR) % 4;
                    const unsigned local = __float_as_uint(kv) & 63u;
                    cand_n[pos] = slc * rsh.rs + static_cast<int>(local >> 2) * 16 + q * 4 + static_cast<int>(local & 3);
                }
                ncand += __popcll(bal);
            }
            if (ncand > kRCand) ok = false;
        }
        __syncthreads();
        if (ok) {
            if (Q8 && lane < K / 32) quantize_block_q8(xs + 32 * lane, xq + 32 * lane, xd + lane);
            if (RECIPE == HIGGS && lane == 0) x2s = sum_squares_k<K>(xs);
        }
        __syncthreads();
        const float x2c = RECIPE == HIGGS ? x2s : 0.0f;
        if (ok) exact_values_frame<RECIPE, Q8, K>(a, xs, x2c, xq, xd, cand_n, cand_v, ncand, lane);
        __syncthreads();

        // Ranked selection of the evaluated candidates (every lane computes
        // the same list), then the certificate.
        float sel_v[5];
        int sel_n[5];
#pragma unroll
        for (int r = 0; r < 5; ++r) {
            sel_v[r] = 0.0f;
            sel_n[r] = -1;
        }
        int win = 0;
        if (ok) {
            for (int c = 0; c < ncand; ++c) {
                float cv = cand_v[c];
                int cn = cand_n[c];
#pragma unroll
                for (int r = 0; r < 5; ++r) {
                    const bool before = a.topk == 0 ? ranks_before<RECIPE>(cv, cn, sel_v[r], sel_n[r])
                                                    : topk_before<RECIPE>(cv, cn, sel_v[r], sel_n[r]);
                    const bool take = r < Tsel && (sel_n[r] < 0 || before);
                    const float tv = sel_v[r];
                    const int tn = sel_n[r];
                    sel_v[r] = take ? cv : tv;
                    sel_n[r] = take ? cn : tn;
                    cv = take ? tv : cv;
                    cn = take ? tn : cn;
                }
            }
            float sv = 0.0f;
#pragma unroll
            for (int r = 0; r < 5; ++r)
                if (r == Tk - 1) sv = sel_v[r];
            bool have = false;
#pragma unroll
            for (int r = 0; r < 5; ++r)
                if (r == Tk - 1) have = sel_n[r] >= 0;
            if (!have) {
                ok = false;
            } else {
                float sprime;
                if (RECIPE == OMNI) sprime = 0.5f * sv;
                else if (RECIPE == HIGGS) sprime = 0.5f * sv + 0.5f * x2c;
                else sprime = -0.5f * sv + 0.5f * nxx2;
                const float off_err = RECIPE == DIRECT ? 0.5f * (K + 8) * u * nxx2 * 1.01f : 0.0f;
                ok = (sv - sv == 0.0f) && (sprime - off_err > tau + E);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (r < Tk && sel_n[r] >= 0 && !(sel_v[r] - sel_v[r] == 0.0f)) ok = false;
                if (RECIPE != DIRECT && Tk > 1 && sv == sel_v[0]) ok = false;
#pragma unroll
                for (int r = 1; r < 5; ++r)
                    if (RECIPE != DIRECT && a.topk > 0 && r == Tk && sel_n[r] >= 0 && sel_v[r] == sv) ok = false;
            }
            win = sel_n[0];
            if (RECIPE != DIRECT)
#pragma unroll
                for (int r = 1; r < 4; ++r)
                    if (r < Tk && sel_n[r] >= 0 && sel_v[r] == sel_v[0] && sel_n[r] > win) win = sel_n[r];
        }
        if (!ok) {
            if (lane == 0) {
                const int s2 = atomicAdd(rf.count2, 1);
                rf.list2[s2] = static_cast<int32_t>(m);
            }
            continue;
        }
        if (lane == 0) {
            a.idx[m * a.Q + a.s] = win;
            if (a.dist) a.dist[m * a.Q + a.s] = RECIPE == DIRECT ? sel_v[0] : -sel_v[0];
            for (int r = 0; r < a.topk; ++r) {
                float v = 0.0f;
                int n = 0;
#pragma unroll
                for (int q = 0; q < 5; ++q)
                    if (q == r) {
                        v = sel_v[q];
                        n = sel_n[q];
                    }
                a.topk_idx[(m * a.Q + a.s) * a.topk + r] = n;
                a.topk_dist[(m * a.Q + a.s) * a.topk + r] = RECIPE == DIRECT ? v : -v;
            }
        }
        int use = win;
        if (a.force_idx) {
            use = a.force_idx[m * a.Q + a.s];
            if (use < 0 || use >= a.N) {
                if (lane == 0) a.flags[AQ_FLAG_BAD_INDEX] = 1;
                use = 0;
            }
        }
        if (a.xout) {
#pragma unroll
            for (int j = 0; j < KPL; ++j) {
                const int k = lane + kWave * j;
                a.xout[m * K + k] = __fsub_rn(xs[k], a.cbf[static_cast<int64_t>(use) * K + k]);
            }
        }
    }
}


// ------------------------------------------------------------- cascade
// The residual cascade of every stage in one launch.  A block of kCWaves
// waves owns kCRows x FG x 16 frames through all stages; per stage it
//  1. converts its frames' residual to fp16 fragments in registers (wave w
//     takes row w % kCRows; waves w and w + kCRows hold the same frames);
//  2. sweeps the stage's codebook through double-buffered LDS chunks, waves
//     0 .. kCRows-1 taking the even 16-code blocks of each chunk and the
//     others the odd ones (two waves per SIMD share every staged chunk);
//  3. merges the two halves' keys and runs the select of the block's
//     kCRows x FG groups over its waves: certificate, exact re-ranking,
//     outputs and the residual update, in place.  A frame the certificate
//     cannot settle continues with its best exactly evaluated code and is
//     listed for the exact verification that follows the cascade
//     (euclid_verify_kernel); a frame whose guess was wrong is recomputed
//     from that stage on by euclid_fixup_kernel.
// No block depends on another: the launch needs no grid synchronisation,
// and the stages of a block follow each other with block barriers only.
constexpr int kCWaves = 8;
constexpr int kCThreads = kCWaves * kWave;
constexpr int kCRows = kCWaves / 2;

template <int KS>
struct CTile {
    using T = Tile<KS>;
    static constexpr int BUFB = T::CHUNKB + kCThreads * 4;    // chunk + one |c|^2/2 slot per thread
    static constexpr int STAGE16 = T::CHUNKB / 16 / kCThreads;
    static constexpr int SWEEP = 2 * BUFB;
};

constexpr int cmax3(int a, int b, int c) { return a > b ? (a > c ? a : c) : (b > c ? b : c); }

// Dynamic LDS of the cascade kernel: a phase region (the chunk buffers while
// sweeping; then the second half's keys; then the waves' select queues) and
// the merged keys (TOPL keys and the dropped-key bound per lane) and frame
// norms of every group, which the select phase reads.
template <int KS, int FG, int TOPL, bool Q8>
struct CLayout {
    static constexpr int K = KS * 32;
    static constexpr int G = kCRows * FG;
    static constexpr int SEL = kCWaves * static_cast<int>(sizeof(SelLds<Q8, K, TOPL>));
    static constexpr int MERGE = G * TOPL * kWave * 4;
    static constexpr int PHASE = (cmax3(CTile<KS>::SWEEP, SEL, MERGE) + 15) / 16 * 16;
    static constexpr int SELK = G * (TOPL + 1) * kWave * 4;
    static constexpr int NRM = G * 3 * 16 * 4;
    static constexpr int BYTES = PHASE + SELK + NRM;
};

// StageArgs of stage s of a cascade.
__device__ inline StageArgs cascade_stage(const CascadeArgs &c, int s, int K) {
    StageArgs a = c.a;
    const int64_t NK = static_cast<int64_t>(a.N) * K;
    a.s = s;
    a.cbh += s * NK;
    a.nhh += static_cast<int64_t>(s) * a.N;
    a.cbf += s * NK;
    a.bias += static_cast<int64_t>(s) * a.N;
    a.e2 += static_cast<int64_t>(s) * a.N;
    if (a.q8) {
        a.q8 += s * NK;
        a.q8d += s * (NK / 32);
    }
    a.cmax = c.bounds[3 * s];
    a.dcmax = c.bounds[3 * s + 1];
    a.chmax = c.bounds[3 * s + 2];
    a.xin = s == 0 ? c.x0 : c.work;
    a.xout = (s + 1 < a.Q || c.write_last) ? c.work : nullptr;
    a.fail_count = c.counts + (s % 64);
    return a;
}

template <int RECIPE, bool Q8, int KS, int FG, int TOPL>
__global__ __launch_bounds__(kCThreads, 1) void euclid_cascade_kernel(CascadeArgs c) {
    using T = Tile<KS>;
    using CT = CTile<KS>;
    using LY = CLayout<KS, FG, TOPL, Q8>;
    using MX = Mx;
    constexpr int K = T::K;
    constexpr int BPC = T::CC / 16;
    constexpr int NB = BPC / 2;   // blocks of a chunk per half
    static_assert(BPC % 2 == 0, "the halves take alternate 16-code blocks");
    static_assert(T::CHUNKB % (16 * kCThreads) == 0, "a chunk splits evenly over the block");
    extern __shared__ __align__(16) unsigned char lds[];
    float *selk = reinterpret_cast<float *>(lds + LY::PHASE);             // [G][TOPL + 1][64]
    float *nrm = reinterpret_cast<float *>(lds + LY::PHASE + LY::SELK);   // [G][3][16]

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);   // uniform: addresses stay scalar
    const int row = wave % kCRows, half = wave / kCRows;
    const int col = lane & 15, kq = lane >> 4;
    const int64_t M = c.a.M;
    const int N = c.a.N;
    const int64_t m_tile = static_cast<int64_t>(blockIdx.x) * (LY::G * 16);
    if (m_tile >= M) return;   // block-uniform
    const int64_t m_row = m_tile + row * (FG * 16);
    for (int i = threadIdx.x; i < LY::G * 16; i += kCThreads)
        if (m_tile + i < M) c.bad_stage[m_tile + i] = c.a.Q;

    int lbits = 0;   // bits of the lane-local code index (N/4 codes per lane)
    while ((1 << lbits) < N / 4) ++lbits;
    const unsigned kmask = (1u << lbits) - 1u;
    unsigned vkeep;
    asm volatile("v_mov_b32 %0, %1" : "=v"(vkeep) : "s"(~kmask));
    const int nch = N / T::CC;
    constexpr int R = KS % 4 == 0 ? 4 : 2;
    constexpr int L = R - 1;
    constexpr int PPB = (CT::STAGE16 + NB - 1) / NB;   // staged pieces per block
    constexpr int kWaitLoads = 0x0070;                 // s_waitcnt vmcnt(0) lgkmcnt(0)
    const int hsrc = threadIdx.x < T::CC ? threadIdx.x : 0;
    const StageOffsets<T, kCThreads> so;

    for (int s = 0; s < c.a.Q; ++s) {
        const StageArgs a = cascade_stage(c, s, K);
        // ---- the frames' residual -> fp16 fragments, rounding norms ----
        u32x4 xb[FG][KS];
        float nx2[FG], nd2[FG], nxx2[FG];
#pragma unroll
        for (int g = 0; g < FG; ++g) {
            const int64_t m = m_row + g * 16 + col;
            const int64_t mc = m < M ? m : M - 1;
            const float *xr = a.xin + mc * K;
            float sx = 0.0f, sd = 0.0f, sxx = 0.0f;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const f32x4 lo = *reinterpret_cast<const f32x4 *>(xr + ks * 32 + kq * 8);
                const f32x4 hi = *reinterpret_cast<const f32x4 *>(xr + ks * 32 + kq * 8 + 4);
                float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                if (Q8) q8_image_block(v);
                u32x4 packed;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const typename MX::V2 pr = {static_cast<typename MX::E>(v[2 * t]),
                                                static_cast<typename MX::E>(v[2 * t + 1])};
                    const unsigned w = __builtin_bit_cast(unsigned, pr);
                    packed[t] = w;
                    const float r0 = MX::lo(w), r1 = MX::hi(w);
                    sx = __fmaf_rn(r0, r0, sx);
                    sx = __fmaf_rn(r1, r1, sx);
                    const float d0 = v[2 * t] - r0, d1 = v[2 * t + 1] - r1;
                    sd = __fmaf_rn(d0, d0, sd);
                    sd = __fmaf_rn(d1, d1, sd);
                    sxx = __fmaf_rn(v[2 * t], v[2 * t], sxx);
                    sxx = __fmaf_rn(v[2 * t + 1], v[2 * t + 1], sxx);
                }
                xb[g][ks] = packed;
            }
            sx = rows_sum(sx);
            sd = rows_sum(sd);
            sxx = rows_sum(sxx);
            nx2[g] = sx;
            nd2[g] = sd;
            nxx2[g] = sxx;
        }

        // ---- sweep of the stage's codebook ----
        float top[FG][TOPL];
#pragma unroll
        for (int g = 0; g < FG; ++g)
#pragma unroll
            for (int j = 0; j < TOPL; ++j) top[g][j] = -INFINITY;
        auto lds_a = [&](int buf, int blk, int ks) -> typename MX::V8 {
            const int r = blk * 16 + col;
            const int j = ks * 4 + kq;
            return *reinterpret_cast<const typename MX::V8 *>(lds + buf * CT::BUFB + r * T::ROWB + ((j ^ (r & T::SWZ)) * 16));
        };
        auto lds_h = [&](int buf, int blk) -> f32x4 {
            return *reinterpret_cast<const f32x4 *>(lds + buf * CT::BUFB + T::CHUNKB + (blk * 16 + kq * 4) * 4);
        };
        // direct global-to-LDS staging, as in the sweep kernel (lane l of
        // wave w lands at piece k * kCThreads + 64 w + l)
        const unsigned char *cbb = reinterpret_cast<const unsigned char *>(a.cbh);
        auto stage_piece = [&](int buf, int chunk, int k) {
            const unsigned char *gp = cbb + (static_cast<int64_t>(chunk) * T::CHUNKB + so.uni(k)) + so.lane(k);
            unsigned char *d = lds + buf * CT::BUFB + (k * kCThreads + wave * kWave) * 16;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)gp,
                                             (__attribute__((address_space(3))) void *)d, 16, 0, 0);
        };
        auto stage_h = [&](int buf, int chunk) {
            const float *gp = a.nhh + static_cast<int64_t>(chunk) * T::CC + hsrc;
            unsigned char *d = lds + buf * CT::BUFB + T::CHUNKB + wave * kWave * 4;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)gp,
                                             (__attribute__((address_space(3))) void *)d, 4, 0, 0);
        };
        __syncthreads();   // the previous stage's select is done with the phase region
#pragma unroll
        for (int k = 0; k < CT::STAGE16; ++k) stage_piece(0, 0, k);
        stage_h(0, 0);
        __builtin_amdgcn_s_waitcnt(kWaitLoads);
        __syncthreads();

        typename MX::V8 ring[R];
#pragma unroll
        for (int l = 0; l < L; ++l) ring[l] = lds_a(0, half, l);
        f32x4 hcur = lds_h(0, half);
        f32x4 accp[FG];
#pragma unroll
        for (int g = 0; g < FG; ++g) accp[g] = f32x4{-3.40282347e38f, -3.40282347e38f, -3.40282347e38f, -3.40282347e38f};
        unsigned lprev = 0;
        auto epilogue = [&](const f32x4 (&acc)[FG], unsigned local0) {
#pragma unroll
            for (int g = 0; g < FG; ++g)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float key = key_of(acc[g][i], local0 + i, vkeep);
#pragma unroll
                    for (int j = TOPL - 1; j > 0; --j) top[g][j] = __builtin_amdgcn_fmed3f(top[g][j - 1], top[g][j], key);
                    top[g][0] = __builtin_amdgcn_fmed3f(top[g][0], key, 3.40282347e38f);
                }
        };
        for (int ch = 0; ch < nch; ++ch) {
            const int buf = ch & 1;
            const int cs = ch + 1 < nch ? ch + 1 : ch;   // the last chunk re-stages itself (no branch)
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const int b = 2 * i + half;
#pragma unroll
                for (int j = 0; j < PPB; ++j) {
                    const int k = i + j * NB;
                    if (k < CT::STAGE16) stage_piece(buf ^ 1, cs, k);
                }
                if (i == 0) stage_h(buf ^ 1, cs);
                f32x4 acc[FG];
#pragma unroll
                for (int g = 0; g < FG; ++g) acc[g] = hcur;
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const int pk = ks + L;
                    if (pk < KS) ring[pk % R] = lds_a(buf, b, pk);
                    else if (i + 1 < NB) ring[pk % R] = lds_a(buf, b + 2, pk - KS);
#pragma unroll
                    for (int g = 0; g < FG; ++g)
                        acc[g] = MX::mfma(ring[ks % R], __builtin_bit_cast(typename MX::V8, xb[g][ks]), acc[g]);
                }
                epilogue(accp, lprev);
                if (i + 1 < NB) hcur = lds_h(buf, b + 2);
#pragma unroll
                for (int q = 0; q < KS * FG; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, (4 * 4 * FG + 4 * FG) / (KS * FG) + 1, 0);   // VALU
                }
#pragma unroll
                for (int g = 0; g < FG; ++g) accp[g] = acc[g];
                lprev = static_cast<unsigned>((ch * BPC + b) * 4);
            }
            __builtin_amdgcn_s_waitcnt(kWaitLoads);
            __syncthreads();
#pragma unroll
            for (int l = 0; l < L; ++l) ring[l] = lds_a(buf ^ 1, half, l);
            hcur = lds_h(buf ^ 1, half);
        }
        epilogue(accp, lprev);

        // ---- merge the halves' keys; groups' keys and norms to LDS ----
        __syncthreads();   // every wave is done with the chunk buffers
        float *mk = reinterpret_cast<float *>(lds);   // [G][TOPL][64], the second half's keys
        if (half == 1) {
#pragma unroll
            for (int g = 0; g < FG; ++g)
#pragma unroll
                for (int j = 0; j < TOPL; ++j) mk[((row * FG + g) * TOPL + j) * kWave + lane] = top[g][j];
        }
        __syncthreads();
        if (half == 0) {
#pragma unroll
            for (int g = 0; g < FG; ++g) {
                const int gi = row * FG + g;
                // tau bounds every key either half dropped
                float taul = top[g][TOPL - 1];
#pragma unroll
                for (int j = 0; j < TOPL; ++j) {
                    const float key = mk[(gi * TOPL + j) * kWave + lane];
                    if (j == TOPL - 1) taul = fmaxf(taul, key);
#pragma unroll
                    for (int i = TOPL - 1; i > 0; --i) top[g][i] = __builtin_amdgcn_fmed3f(top[g][i - 1], top[g][i], key);
                    top[g][0] = __builtin_amdgcn_fmed3f(top[g][0], key, 3.40282347e38f);
                }
                taul = fmaxf(taul, top[g][TOPL - 1]);
#pragma unroll
                for (int j = 0; j < TOPL; ++j) selk[(gi * (TOPL + 1) + j) * kWave + lane] = top[g][j];
                selk[(gi * (TOPL + 1) + TOPL) * kWave + lane] = taul;
                if (kq == 0) {
                    nrm[(gi * 3 + 0) * 16 + col] = nx2[g];
                    nrm[(gi * 3 + 1) * 16 + col] = nd2[g];
                    nrm[(gi * 3 + 2) * 16 + col] = nxx2[g];
                }
            }
        }
        __syncthreads();

        // ---- select of the block's groups over its waves ----
        SelLds<Q8, K, TOPL> *sl = reinterpret_cast<SelLds<Q8, K, TOPL> *>(lds);
        for (int gi = wave; gi < LY::G; gi += kCWaves) {
            const int64_t mb = m_tile + gi * 16;
            if (mb >= M) break;   // wave-uniform; later groups are further on
            float tp[TOPL];
#pragma unroll
            for (int j = 0; j < TOPL; ++j) tp[j] = selk[(gi * (TOPL + 1) + j) * kWave + lane];
            const float taul = selk[(gi * (TOPL + 1) + TOPL) * kWave + lane];
            select_group<RECIPE, Q8, KS, TOPL>(a, mb, tp, taul, nrm[(gi * 3 + 0) * 16 + col], nrm[(gi * 3 + 1) * 16 + col],
                                               nrm[(gi * 3 + 2) * 16 + col], sl[wave], true, a.xin + mb * K, K, true);
        }
        __syncthreads();   // the stage's residuals are written before the next stage reads them
    }
}

// ------------------------------------------------------------- resident cascade
// The residual cascade with the residual held in registers.  A block of
// kRsWaves waves (one per SIMD, up to 512 registers each) owns kRsWaves x FG
// x 16 frames through all stages.  Wave w keeps the fp32 residual of its FG
// frame groups in the MFMA fragment layout (lane (col, kq) of group g holds
// x[16 g + col][32 ks + 8 kq + t], t < 8) and per stage
//  1. builds the fp16 fragments and rounding norms from it;
//  2. sweeps the stage's whole codebook through double-buffered LDS chunks
//     that the block's waves stage together (no code split between waves,
//     so no merge of key lists);
//  3. per group: copies the residual rows into its LDS scratch (read by the
//     exact re-ranking), runs the select (certificate, exact re-ranking and
//     outputs; a frame the certificate cannot settle continues with its
//     best evaluated code and is listed for euclid_verify_kernel) and
//     subtracts the chosen (or forced) code's row in registers.
// Only the last stage's residual is written to memory.
constexpr int kRsWaves = 4;
constexpr int kRsThreads = kRsWaves * kWave;

// The resident residual lives in accumulation registers (AGPRs): the sweep
// keeps the architectural registers for its fragments, accumulators and
// key lists, and the residual is read and written only between sweeps.
__device__ inline float agpr_put(float x) {
    float a;
    asm("v_accvgpr_write_b32 %0, %1" : "=a"(a) : "v"(x));
    return a;
}
__device__ inline float agpr_get(float a) {
    float x;
    asm("v_accvgpr_read_b32 %0, %1" : "=v"(x) : "a"(a));
    return x;
}

template <int KS, int FG, int TOPL, bool Q8>
struct RsLayout {
    static constexpr int K = KS * 32;
    static constexpr int BUFB = Tile<KS>::CHUNKB + kRsThreads * 4;   // chunk + one |c|^2/2 slot per thread
    static constexpr int STAGE16 = Tile<KS>::CHUNKB / 16 / kRsThreads;
    static constexpr int SWEEP = 2 * BUFB;
    static constexpr int XSTR = K + 4;   // row stride of the scratch rows (floats; padded against bank conflicts)
    static constexpr int SELB = (static_cast<int>(sizeof(SelLds<Q8, K, TOPL>)) + 15) / 16 * 16;
    static constexpr int WSCR = SELB + 16 * XSTR * 4;                 // per wave: select queues + 16 rows
    static constexpr int BYTES = SWEEP > kRsWaves * WSCR ? SWEEP : kRsWaves * WSCR;
    static constexpr int FRAMES = kRsWaves * FG * 16;
};

template <int RECIPE, bool Q8, int KS, int FG, int TOPL>
__global__ __launch_bounds__(kRsThreads, 1) void euclid_resident_kernel(CascadeArgs c) {
    using T = Tile<KS>;
    using LY = RsLayout<KS, FG, TOPL, Q8>;
    using MX = Mx;
    constexpr int K = T::K;
    constexpr int BPC = T::CC / 16;                       // 16-code blocks per chunk
    static_assert(T::CHUNKB % (16 * kRsThreads) == 0, "a chunk splits evenly over the block");
    constexpr int PPB = (LY::STAGE16 + BPC - 1) / BPC;    // staged pieces per block
    extern __shared__ __align__(16) unsigned char lds[];

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);   // uniform: addresses stay scalar
    const int col = lane & 15, kq = lane >> 4;
    const int64_t M = c.a.M;
    const int N = c.a.N;
    const int64_t m_tile = static_cast<int64_t>(blockIdx.x) * LY::FRAMES;
    if (m_tile >= M) return;   // block-uniform
    const int64_t m_wave = m_tile + wave * (FG * 16);
    for (int i = threadIdx.x; i < LY::FRAMES; i += kRsThreads)
        if (m_tile + i < M) c.bad_stage[m_tile + i] = c.a.Q;

    int lbits = 0;   // bits of the lane-local code index (N/4 codes per lane)
    while ((1 << lbits) < N / 4) ++lbits;
    const unsigned kmask = (1u << lbits) - 1u;
    unsigned vkeep;
    asm volatile("v_mov_b32 %0, %1" : "=v"(vkeep) : "s"(~kmask));
    const int nch = N / T::CC;
    constexpr int R = KS % 4 == 0 ? 4 : 2;
    constexpr int L = R - 1;
    constexpr int kWaitLoads = 0x0070;   // s_waitcnt vmcnt(0) lgkmcnt(0)
    const int hsrc = threadIdx.x < T::CC ? threadIdx.x : 0;
    const StageOffsets<T, kRsThreads> so;

    // the stage-0 input, in the fragment layout (rows past M read row M - 1),
    // held in AGPRs
    float xr[FG][KS][8];
#pragma unroll
    for (int g = 0; g < FG; ++g) {
        const int64_t m = m_wave + g * 16 + col;
        const float *row = c.x0 + (m < M ? m : M - 1) * K;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const f32x4 lo = *reinterpret_cast<const f32x4 *>(row + ks * 32 + kq * 8);
            const f32x4 hi = *reinterpret_cast<const f32x4 *>(row + ks * 32 + kq * 8 + 4);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                xr[g][ks][t] = agpr_put(lo[t]);
                xr[g][ks][4 + t] = agpr_put(hi[t]);
            }
        }
    }

    for (int s = 0; s < c.a.Q; ++s) {
        const StageArgs a = cascade_stage(c, s, K);
        // ---- fp16 fragments and rounding norms of the residual ----
        u32x4 xb[FG][KS];
        float nx2[FG], nd2[FG], nxx2[FG];
#pragma unroll
        for (int g = 0; g < FG; ++g) {
            float sx = 0.0f, sd = 0.0f, sxx = 0.0f;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                float v[8];
#pragma unroll
                for (int t = 0; t < 8; ++t) v[t] = agpr_get(xr[g][ks][t]);
                // a Q8_0 codebook scores the query's Q8_0 image (as the sweep)
                if (Q8) q8_image_block(v);
                u32x4 packed;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const float v0 = v[2 * t], v1 = v[2 * t + 1];
                    const typename MX::V2 pr = {static_cast<typename MX::E>(v0), static_cast<typename MX::E>(v1)};
                    const unsigned w = __builtin_bit_cast(unsigned, pr);
                    packed[t] = w;
                    const float r0 = MX::lo(w), r1 = MX::hi(w);
                    sx = __fmaf_rn(r0, r0, sx);
                    sx = __fmaf_rn(r1, r1, sx);
                    const float d0 = v0 - r0, d1 = v1 - r1;
                    sd = __fmaf_rn(d0, d0, sd);
                    sd = __fmaf_rn(d1, d1, sd);
                    sxx = __fmaf_rn(v0, v0, sxx);
                    sxx = __fmaf_rn(v1, v1, sxx);
                }
                xb[g][ks] = packed;
            }
            sx = rows_sum(sx);
            sd = rows_sum(sd);
            sxx = rows_sum(sxx);
            nx2[g] = sx;
            nd2[g] = sd;
            nxx2[g] = sxx;
        }

        // ---- sweep of the stage's codebook ----
        float top[FG][TOPL];
#pragma unroll
        for (int g = 0; g < FG; ++g)
#pragma unroll
            for (int j = 0; j < TOPL; ++j) top[g][j] = -INFINITY;
        auto lds_a = [&](int buf, int blk, int ks) -> typename MX::V8 {
            const int r = blk * 16 + col;
            const int j = ks * 4 + kq;
            return *reinterpret_cast<const typename MX::V8 *>(lds + buf * LY::BUFB + r * T::ROWB + ((j ^ (r & T::SWZ)) * 16));
        };
        auto lds_h = [&](int buf, int blk) -> f32x4 {
            return *reinterpret_cast<const f32x4 *>(lds + buf * LY::BUFB + T::CHUNKB + (blk * 16 + kq * 4) * 4);
        };
        // direct global-to-LDS staging, as in the sweep kernel (lane l of
        // wave w lands at piece k * kRsThreads + 64 w + l)
        const unsigned char *cbb = reinterpret_cast<const unsigned char *>(a.cbh);
        auto stage_piece = [&](int buf, int chunk, int k) {
            const unsigned char *gp = cbb + (static_cast<int64_t>(chunk) * T::CHUNKB + so.uni(k)) + so.lane(k);
            unsigned char *d = lds + buf * LY::BUFB + (k * kRsThreads + wave * kWave) * 16;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)gp,
                                             (__attribute__((address_space(3))) void *)d, 16, 0, 0);
        };
        auto stage_h = [&](int buf, int chunk) {
            const float *gp = a.nhh + static_cast<int64_t>(chunk) * T::CC + hsrc;
            unsigned char *d = lds + buf * LY::BUFB + T::CHUNKB + wave * kWave * 4;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)gp,
                                             (__attribute__((address_space(3))) void *)d, 4, 0, 0);
        };
        __syncthreads();   // the previous stage's select is done with the scratch
#pragma unroll
        for (int k = 0; k < LY::STAGE16; ++k) stage_piece(0, 0, k);
        stage_h(0, 0);
        __builtin_amdgcn_s_waitcnt(kWaitLoads);
        __syncthreads();

        typename MX::V8 ring[R];
#pragma unroll
        for (int l = 0; l < L; ++l) ring[l] = lds_a(0, 0, l);
        f32x4 hcur = lds_h(0, 0);
        f32x4 accp[FG];
#pragma unroll
        for (int g = 0; g < FG; ++g) accp[g] = f32x4{-3.40282347e38f, -3.40282347e38f, -3.40282347e38f, -3.40282347e38f};
        unsigned lprev = 0;
        // key e (< 4 FG) of the previous block's sums into its group's list
        auto insert_key = [&](const f32x4 (&acc)[FG], unsigned local0, int e) {
            const int g = e / 4, i = e % 4;
            const float key = key_of(acc[g][i], local0 + i, vkeep);
#pragma unroll
            for (int j = TOPL - 1; j > 0; --j) top[g][j] = __builtin_amdgcn_fmed3f(top[g][j - 1], top[g][j], key);
            top[g][0] = __builtin_amdgcn_fmed3f(top[g][0], key, 3.40282347e38f);
        };
        constexpr int E = 4 * FG;   // keys per block and lane
        for (int ch = 0; ch < nch; ++ch) {
            const int buf = ch & 1;
            const int cs = ch + 1 < nch ? ch + 1 : ch;   // the last chunk re-stages itself (no branch)
#pragma unroll
            for (int b = 0; b < BPC; ++b) {
#pragma unroll
                for (int j = 0; j < PPB; ++j) {
                    const int k = b + j * BPC;
                    if (k < LY::STAGE16) stage_piece(buf ^ 1, cs, k);
                }
                if (b == 0) stage_h(buf ^ 1, cs);
                const f32x4 hnext = b + 1 < BPC ? lds_h(buf, b + 1) : hcur;
                f32x4 acc[FG];
#pragma unroll
                for (int g = 0; g < FG; ++g) acc[g] = hcur;
                // One wave per SIMD hides no latency behind another wave:
                // scheduling barriers keep each step's fragment load L steps
                // ahead of its MFMAs (the compiler would sink it next to
                // them), and each step takes its share of the previous
                // block's keys.
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const int pk = ks + L;
                    if (pk < KS) ring[pk % R] = lds_a(buf, b, pk);
                    else if (b + 1 < BPC) ring[pk % R] = lds_a(buf, b + 1, pk - KS);
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int g = 0; g < FG; ++g)
                        acc[g] = MX::mfma(ring[ks % R], __builtin_bit_cast(typename MX::V8, xb[g][ks]), acc[g]);
#pragma unroll
                    for (int e = ks * E / KS; e < (ks + 1) * E / KS; ++e) insert_key(accp, lprev, e);
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int g = 0; g < FG; ++g) accp[g] = acc[g];
                hcur = hnext;
                lprev = static_cast<unsigned>((ch * BPC + b) * 4);
            }
            __builtin_amdgcn_s_waitcnt(kWaitLoads);
            __syncthreads();
#pragma unroll
            for (int l = 0; l < L; ++l) ring[l] = lds_a(buf ^ 1, 0, l);
            hcur = lds_h(buf ^ 1, 0);
        }
#pragma unroll
        for (int e = 0; e < E; ++e) insert_key(accp, lprev, e);
        __syncthreads();   // every wave is done with the chunk buffers

        // ---- select and residual update of the wave's groups ----
        unsigned char *ws = lds + wave * LY::WSCR;
        SelLds<Q8, K, TOPL> &sl = *reinterpret_cast<SelLds<Q8, K, TOPL> *>(ws);
        float *xs = reinterpret_cast<float *>(ws + LY::SELB);
#pragma unroll
        for (int g = 0; g < FG; ++g) {
            const int64_t mb = m_wave + g * 16;
            if (mb >= M) break;   // wave-uniform; later groups are further on
            // the group's rows, for the exact re-ranking
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                float *d = xs + col * LY::XSTR + ks * 32 + kq * 8;
                *reinterpret_cast<f32x4 *>(d) = f32x4{agpr_get(xr[g][ks][0]), agpr_get(xr[g][ks][1]),
                                                      agpr_get(xr[g][ks][2]), agpr_get(xr[g][ks][3])};
                *reinterpret_cast<f32x4 *>(d + 4) = f32x4{agpr_get(xr[g][ks][4]), agpr_get(xr[g][ks][5]),
                                                          agpr_get(xr[g][ks][6]), agpr_get(xr[g][ks][7])};
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const int code = select_group<RECIPE, Q8, KS, TOPL>(a, mb, top[g], top[g][TOPL - 1], nx2[g], nd2[g],
                                                                   nxx2[g], sl, true, xs, LY::XSTR, false);
            // r -= c[code] (the forced code where given) in registers
            const int64_t m = mb + col;
            int use = code >= 0 ? code : 0;
            if (a.force_idx && m < M) {
                use = a.force_idx[m * a.Q + s];
                if (use < 0 || use >= N) {
                    a.flags[AQ_FLAG_BAD_INDEX] = 1;
                    use = 0;
                }
            }
            if (s + 1 < a.Q || c.write_last) {
                const float *crow = a.cbf + static_cast<int64_t>(use) * K;
                f32x4 cv[KS][2];
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    cv[ks][0] = *reinterpret_cast<const f32x4 *>(crow + ks * 32 + kq * 8);
                    cv[ks][1] = *reinterpret_cast<const f32x4 *>(crow + ks * 32 + kq * 8 + 4);
                }
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                    for (int t = 0; t < 8; ++t)
                        xr[g][ks][t] = agpr_put(__fsub_rn(agpr_get(xr[g][ks][t]), cv[ks][t / 4][t % 4]));
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    }

    // the residual after the last stage
    if (c.write_last) {
#pragma unroll
        for (int g = 0; g < FG; ++g) {
            const int64_t m = m_wave + g * 16 + col;
            if (m >= M) continue;
            float *row = c.work + m * K;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                *reinterpret_cast<f32x4 *>(row + ks * 32 + kq * 8) =
                    f32x4{agpr_get(xr[g][ks][0]), agpr_get(xr[g][ks][1]), agpr_get(xr[g][ks][2]), agpr_get(xr[g][ks][3])};
                *reinterpret_cast<f32x4 *>(row + ks * 32 + kq * 8 + 4) =
                    f32x4{agpr_get(xr[g][ks][4]), agpr_get(xr[g][ks][5]), agpr_get(xr[g][ks][6]), agpr_get(xr[g][ks][7])};
            }
        }
    }
}

// The residual of frame m entering stage s of a cascade, replayed from the
// input in the cascade's arithmetic (r -= c_t[code_t], t < s, the forced
// codes where given), into xs (every thread of the block).
__device__ inline void replay_residual(const CascadeArgs &c, int64_t m, int s, float *xs, int K) {
    const StageArgs &a = c.a;
    const int32_t *codes = (a.force_idx ? a.force_idx : a.idx) + m * a.Q;
    constexpr int B = 8;   // stages whose codes and rows are read together
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
        float v = c.x0[m * K + k];
        for (int t0 = 0; t0 < s; t0 += B) {
            int u[B];
#pragma unroll
            for (int j = 0; j < B; ++j) {
                u[j] = t0 + j < s ? codes[t0 + j] : 0;
                if (u[j] < 0 || u[j] >= a.N) u[j] = 0;
            }
            float cv[B];
#pragma unroll
            for (int j = 0; j < B; ++j)
                cv[j] = t0 + j < s ? a.cbf[(static_cast<int64_t>(t0 + j) * a.N + u[j]) * K + k] : 0.0f;
#pragma unroll
            for (int j = 0; j < B; ++j)
                if (t0 + j < s) v = __fsub_rn(v, cv[j]);
        }
        xs[k] = v;
    }
}

// The recipe's per-frame terms of the frame in xs: sum_rows(x*x) (Higgs)
// into sh.o_x2, and the Q8_0 query blocks into xq / xd.
template <int RECIPE, bool Q8, int KS>
__device__ inline void scan_prepare(const float *xs, int8_t *xq, float *xd, ScanSh &sh) {
    constexpr int K = KS * 32;
    __syncthreads();
    if (threadIdx.x == 0) sh.o_x2 = RECIPE == HIGGS ? sum_squares_k<K>(xs) : 0.0f;
    if (Q8 && threadIdx.x < K / 32) quantize_block_q8(xs + 32 * threadIdx.x, xq + 32 * threadIdx.x, xd + threadIdx.x);
    __syncthreads();
}

__device__ inline bool same_bits(float x, float y) { return __float_as_uint(x) == __float_as_uint(y); }

// Exact verification of the cascade's speculative (frame, stage) pairs, a
// block per pair: the stage's input residual is replayed, every code's
// recipe value computed and the reference's selection made (the exact
// scan's); where the code differs from the cascade's, the frame's earliest
// wrong stage is recorded for the fix-up, and where only the distance or
// top-k list differ they are corrected in place.  F32 codebooks in tinyBLAS
// order and Q8_0 codebooks take the values that euclid_verify_values_kernel
// spread over the grid (up to a.scap pairs), or compute them in the block
// (coalesced code-row reads: the quad layout, or 8 lanes per Q8_0 code).
template <int RECIPE, bool Q8, int KS>
__device__ inline void scan_frame(const StageArgs &a, const float *xs, const int8_t *xq, const float *xd, ScanSh &sh) {
    constexpr int K = KS * 32;
    constexpr bool kQuadOk = !Q8 && RECIPE != DIRECT;
    if constexpr (kQuadOk) {
        if (spread_quad<RECIPE, Q8>(a) && a.N <= kScanChunk) {
            block_values_quad<RECIPE, K>(a, xs, sh.o_x2, sh.rv, 0, a.N);
            __syncthreads();
            scan_select<RECIPE, Q8, KS>(a, K, true, sh.rv, xs, xq, xd, sh.o_x2, sh);
            return;
        }
    }
    if constexpr (Q8 && RECIPE == HIGGS) {
        if (a.N <= kScanChunk) {
            block_values_q8<K>(a, xq, xd, sh.o_x2, sh.rv, 0, a.N);
            __syncthreads();
            scan_select<RECIPE, Q8, KS>(a, K, true, sh.rv, xs, xq, xd, sh.o_x2, sh);
            return;
        }
    }
    scan_select<RECIPE, Q8, KS>(a, K, false, nullptr, xs, xq, xd, sh.o_x2, sh);
}

// Whether the verification takes its pairs' values from
// euclid_verify_values_kernel (into a.svals, up to a.scap pairs).
template <int RECIPE, bool Q8>
__device__ inline bool verify_spread(const StageArgs &a, int count) {
    const bool form = Q8 ? RECIPE == HIGGS : RECIPE != DIRECT && spread_quad<RECIPE, Q8>(a);
    return form && count <= a.scap;
}
constexpr int kVerifyPart = 128;   // codes per item of euclid_verify_values_kernel

// The exact values of the speculative pairs' codes, spread over the grid in
// (pair, kVerifyPart codes) items, for euclid_verify_kernel (the kernel
// boundary orders them before their reader): a.svals[p][n].
template <int RECIPE, bool Q8, int KS>
__global__ __launch_bounds__(kScanThreads) void euclid_verify_values_kernel(CascadeArgs c) {
    constexpr int K = KS * 32;
    constexpr bool kQuadOk = !Q8 && RECIPE != DIRECT;
    if constexpr (kQuadOk || (Q8 && RECIPE == HIGGS)) {
        extern __shared__ __align__(16) unsigned char lds[];
        float *xs = reinterpret_cast<float *>(lds);
        int8_t *xq = reinterpret_cast<int8_t *>(xs + K);
        float *xd = reinterpret_cast<float *>(xq + K);
        __shared__ ScanSh sh;
        const int count = *c.a.spec_count;
        if (!verify_spread<RECIPE, Q8>(c.a, count)) return;   // grid-uniform
        const int parts = (c.a.N + kVerifyPart - 1) / kVerifyPart;
        for (int item = blockIdx.x; item < count * parts; item += gridDim.x) {
            const int p = item / parts, part = item - p * parts;
            const int64_t m = c.a.spec_list[2 * p];
            const int s = c.a.spec_list[2 * p + 1];
            const StageArgs a = cascade_stage(c, s, K);
            __syncthreads();   // the previous item's readers of xs
            replay_residual(c, m, s, xs, K);
            scan_prepare<RECIPE, Q8, KS>(xs, xq, xd, sh);
            const int n0 = part * kVerifyPart, n1 = min(a.N, n0 + kVerifyPart);
            float *rv = a.svals + static_cast<int64_t>(p) * a.N;
            if constexpr (Q8) block_values_q8<K>(a, xq, xd, sh.o_x2, rv, n0, n1);
            else block_values_quad<RECIPE, K>(a, xs, sh.o_x2, rv, n0, n1);
        }
    }
}

template <int RECIPE, bool Q8, int KS>
__global__ __launch_bounds__(kScanThreads) void euclid_verify_kernel(CascadeArgs c) {
    constexpr int K = KS * 32;
    extern __shared__ __align__(16) unsigned char lds[];
    float *xs = reinterpret_cast<float *>(lds);
    int8_t *xq = reinterpret_cast<int8_t *>(xs + K);
    float *xd = reinterpret_cast<float *>(xq + K);
    __shared__ ScanSh sh;
    const int count = *c.a.spec_count;
    const bool spread = verify_spread<RECIPE, Q8>(c.a, count);
    for (int p = blockIdx.x; p < count; p += gridDim.x) {
        const int64_t m = c.a.spec_list[2 * p];
        const int s = c.a.spec_list[2 * p + 1];
        const StageArgs a = cascade_stage(c, s, K);
        __syncthreads();
        if (spread) {
            // values from euclid_verify_values_kernel; the selection reads
            // neither the frame nor its norms
            scan_select<RECIPE, Q8, KS>(a, K, true, a.svals + static_cast<int64_t>(p) * a.N, xs, xq, xd, 0.0f, sh);
        } else {
            replay_residual(c, m, s, xs, K);
            scan_prepare<RECIPE, Q8, KS>(xs, xq, xd, sh);
            scan_frame<RECIPE, Q8, KS>(a, xs, xq, xd, sh);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            // A wrong code sends the frame to the fix-up from this stage on;
            // with the right code (the later stages' input is then right)
            // a wrong distance or top-k list is corrected here.
            const int64_t o = m * a.Q + s;
            const bool bad = a.idx[o] != sh.o_code;
            if (bad) {
                if (atomicMin(&c.bad_stage[m], s) == a.Q) c.bad_list[atomicAdd(c.bad_count, 1)] = static_cast<int32_t>(m);
            } else {
                if (a.dist) a.dist[o] = RECIPE == DIRECT ? sh.o_code_v : -sh.o_code_v;
                for (int r = 0; r < a.topk; ++r) {
                    a.topk_idx[o * a.topk + r] = sh.o_sel_n[r];
                    a.topk_dist[o * a.topk + r] = RECIPE == DIRECT ? sh.o_sel_v[r] : -sh.o_sel_v[r];
                }
            }
        }
    }
}

// Recomputes the frames whose speculation was wrong from their earliest
// wrong stage on, a block per frame, with the exact scan of every stage.
template <int RECIPE, bool Q8, int KS>
__global__ __launch_bounds__(kScanThreads) void euclid_fixup_kernel(CascadeArgs c) {
    constexpr int K = KS * 32;
    extern __shared__ __align__(16) unsigned char lds[];
    float *xs = reinterpret_cast<float *>(lds);
    int8_t *xq = reinterpret_cast<int8_t *>(xs + K);
    float *xd = reinterpret_cast<float *>(xq + K);
    __shared__ ScanSh sh;
    const int nb = *c.bad_count;
    for (int b = blockIdx.x; b < nb; b += gridDim.x) {
        const int64_t m = c.bad_list[b];
        const int t0 = c.bad_stage[m];
        __syncthreads();
        replay_residual(c, m, t0, xs, K);
        for (int s = t0; s < c.a.Q; ++s) {
            const StageArgs a = cascade_stage(c, s, K);
            scan_prepare<RECIPE, Q8, KS>(xs, xq, xd, sh);
            scan_frame<RECIPE, Q8, KS>(a, xs, xq, xd, sh);
            __syncthreads();
            const int64_t o = m * a.Q + s;
            if (threadIdx.x == 0) {
                a.idx[o] = sh.o_code;
                if (a.dist) a.dist[o] = RECIPE == DIRECT ? sh.o_code_v : -sh.o_code_v;
                for (int r = 0; r < a.topk; ++r) {
                    a.topk_idx[o * a.topk + r] = sh.o_sel_n[r];
                    a.topk_dist[o * a.topk + r] = RECIPE == DIRECT ? sh.o_sel_v[r] : -sh.o_sel_v[r];
                }
                atomicAdd(&c.counts[64 + (s % 64)], 1);
            }
            int use = sh.o_code;
            if (a.force_idx) {
                use = a.force_idx[o];
                if (use < 0 || use >= a.N) {
                    if (threadIdx.x == 0) a.flags[AQ_FLAG_BAD_INDEX] = 1;
                    use = 0;
                }
            }
            for (int k = threadIdx.x; k < K; k += blockDim.x)
                xs[k] = __fsub_rn(xs[k], a.cbf[static_cast<int64_t>(use) * K + k]);
        }
        __syncthreads();
        if (c.write_last)
            for (int k = threadIdx.x; k < K; k += blockDim.x) c.work[m * K + k] = xs[k];
    }
}

// Cascade kernels of a width (null where the frame tiles would not keep
// two waves per SIMD busy: the widest codebooks take the stage pipeline).
template <int RECIPE, bool Q8, int KS, int TOPL>
constexpr CascadeFn cascade_fn() {
    if constexpr (KS == 2 || KS == 8) return euclid_cascade_kernel<RECIPE, Q8, KS, groups_for(KS), TOPL>;
    else return nullptr;
}
template <int RECIPE, bool Q8, int KS>
constexpr CascadeFn verify_fn() {
    if constexpr (KS == 2 || KS == 8) return euclid_verify_kernel<RECIPE, Q8, KS>;
    else return nullptr;
}
template <int RECIPE, bool Q8, int KS>
constexpr CascadeFn verify_values_fn() {
    if constexpr (KS == 2 || KS == 8) return euclid_verify_values_kernel<RECIPE, Q8, KS>;
    else return nullptr;
}
template <int RECIPE, bool Q8, int KS>
constexpr CascadeFn fixup_fn() {
    if constexpr (KS == 2 || KS == 8) return euclid_fixup_kernel<RECIPE, Q8, KS>;
    else return nullptr;
}
template <int KS>
constexpr int cascade_lds_bytes() {
    if constexpr (KS == 2 || KS == 8) return CLayout<KS, groups_for(KS), 4, true>::BYTES;
    else return 0;
}
// Register-resident cascade: K = 256 (3 groups of fp32 residual and fp16
// fragments per wave fit its 512 registers).  The Q8_0 variant for top-k
// keeps six keys per lane in place of four: its fp16 images of q * d leave
// about 2.7 % of the frames of each stage uncertified with four (their
// verification then costs more than the cascade saves), a few with six.
constexpr int kRsGroups = 3;
template <bool Q8, int TOPL>
constexpr int resident_keys() { return Q8 && TOPL == 4 ? 6 : TOPL; }
template <int RECIPE, bool Q8, int KS, int TOPL>
constexpr CascadeFn resident_fn() {
    if constexpr (KS == 8) return euclid_resident_kernel<RECIPE, Q8, KS, kRsGroups, resident_keys<Q8, TOPL>()>;
    else return nullptr;
}
template <int KS>
constexpr int resident_lds_bytes() {   // the largest variant's (Q8_0, six keys)
    if constexpr (KS == 8) return RsLayout<KS, kRsGroups, resident_keys<true, 4>(), true>::BYTES;
    else return 0;
}

}  // namespace

// Defines aq_euclid::kernels_ks<KS>(): the kernel table of one width.
#define AQ_EUCLID_KS_TABLE(KS)                                                                                  \
    namespace aq_euclid {                                                                                       \
    const KsKernels *kernels_ks##KS() {                                                                         \
        constexpr int FG = groups_for(KS);                                                                      \
        static const KsKernels t = {                                                                            \
            {{euclid_sweep_kernel<false, KS, FG, 3>, euclid_sweep_kernel<false, KS, FG, 4>},                  \
             {euclid_sweep_kernel<true, KS, FG, 3>, euclid_sweep_kernel<true, KS, FG, 4>}},                    \
            {{euclid_select_kernel<OMNI, false, KS, 3>, euclid_select_kernel<OMNI, false, KS, 4>},            \
             {euclid_select_kernel<HIGGS, false, KS, 3>, euclid_select_kernel<HIGGS, false, KS, 4>},          \
             {euclid_select_kernel<DIRECT, false, KS, 3>, euclid_select_kernel<DIRECT, false, KS, 4>},        \
             {euclid_select_kernel<HIGGS, true, KS, 3>, euclid_select_kernel<HIGGS, true, KS, 4>}},           \
            {euclid_refine_values_kernel<OMNI, false, KS>, euclid_refine_values_kernel<HIGGS, false, KS>,       \
             euclid_refine_values_kernel<DIRECT, false, KS>, euclid_refine_values_kernel<HIGGS, true, KS>},     \
            {euclid_refine_select_kernel<OMNI, false, KS>, euclid_refine_select_kernel<HIGGS, false, KS>,       \
             euclid_refine_select_kernel<DIRECT, false, KS>, euclid_refine_select_kernel<HIGGS, true, KS>},     \
            {euclid_exact_scan_kernel<OMNI, false, KS>, euclid_exact_scan_kernel<HIGGS, false, KS>,             \
             euclid_exact_scan_kernel<DIRECT, false, KS>, euclid_exact_scan_kernel<HIGGS, true, KS>},           \
            sweep_lds_bytes<KS>(),                                                                              \
            Tile<KS>::CC,                                                                                       \
            {{cascade_fn<OMNI, false, KS, 3>(), cascade_fn<OMNI, false, KS, 4>()},                              \
             {cascade_fn<HIGGS, false, KS, 3>(), cascade_fn<HIGGS, false, KS, 4>()},                            \
             {cascade_fn<DIRECT, false, KS, 3>(), cascade_fn<DIRECT, false, KS, 4>()},                          \
             {cascade_fn<HIGGS, true, KS, 3>(), cascade_fn<HIGGS, true, KS, 4>()}},                             \
            {verify_fn<OMNI, false, KS>(), verify_fn<HIGGS, false, KS>(), verify_fn<DIRECT, false, KS>(),       \
             verify_fn<HIGGS, true, KS>()},                                                                     \
            {verify_values_fn<OMNI, false, KS>(), verify_values_fn<HIGGS, false, KS>(),                         \
             verify_values_fn<DIRECT, false, KS>(), verify_values_fn<HIGGS, true, KS>()},                       \
            {fixup_fn<OMNI, false, KS>(), fixup_fn<HIGGS, false, KS>(), fixup_fn<DIRECT, false, KS>(),          \
             fixup_fn<HIGGS, true, KS>()},                                                                      \
            cascade_lds_bytes<KS>(),                                                                            \
            kCRows * groups_for(KS) * 16,                                                                       \
            {{resident_fn<OMNI, false, KS, 3>(), resident_fn<OMNI, false, KS, 4>()},                            \
             {resident_fn<HIGGS, false, KS, 3>(), resident_fn<HIGGS, false, KS, 4>()},                          \
             {resident_fn<DIRECT, false, KS, 3>(), resident_fn<DIRECT, false, KS, 4>()},                        \
             {resident_fn<HIGGS, true, KS, 3>(), resident_fn<HIGGS, true, KS, 4>()}},                           \
            resident_lds_bytes<KS>(),                                                                           \
            kRsWaves * kRsGroups * 16};                                                                         \
        return &t;                                                                                              \
    }                                                                                                           \
    }
