// aq_mi355x.hpp -- C++ host interface over the C ABI (aq_mi355x.h), shaped
// like the reference's quantizer call sites so they can switch to the MI355X
// library without changing their code around the call.
//
//  * aq::engine::runtime::VectorQuantizer mirrors engine::runtime::
//    VectorQuantizer (include/engine/framework/runtime/host_ops.h:87-96,
//    src/framework/runtime/host_ops.cpp:236-273): same argument meaning,
//    same result (the nearest codewords, shape {batch, steps, dim}), same
//    error ("VectorQuantizer input size mismatch" as std::runtime_error).
//  * aq::DacRvq is the Fish Audio encode / decode quantizer
//    (src/models/fish_audio/codec.cpp:552-611) for callers holding host
//    latents or device pointers.
//  * aq::EuclideanRvq is the OmniVoice / Higgs / Qwen3 residual quantizer
//    (omnivoice/audio_tokenizer.cpp:1886-1927, higgs_audio_tts/codec.cpp:
//    958-1016, qwen3_tts/tokenizer_speech_encoder.cpp:287-349).
//
// Every failure of the library is rethrown as std::runtime_error carrying
// the library's message.  Host-vector overloads copy through device buffers
// owned by the call; device-pointer overloads enqueue on the context's
// stream and do not synchronise.
#ifndef AQ_MI355X_HPP
#define AQ_MI355X_HPP

#include "aq_mi355x.h"

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace aq {

struct FloatHostTensor {
    std::vector<float> values;
    std::vector<int64_t> shape;
};

struct IntHostTensor {
    std::vector<int32_t> values;
    std::vector<int64_t> shape;
};

namespace detail {

inline void hip_check(hipError_t e, const char *what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// Device buffer owned by one call.
template <typename T>
class DeviceBuffer {
public:
    explicit DeviceBuffer(size_t n) : n_(n) {
        if (n_ > 0) hip_check(hipMalloc(reinterpret_cast<void **>(&p_), n_ * sizeof(T)), "hipMalloc");
    }
    DeviceBuffer(const DeviceBuffer &) = delete;
    DeviceBuffer &operator=(const DeviceBuffer &) = delete;
    ~DeviceBuffer() {
        if (p_) (void)hipFree(p_);
    }
    T *get() const { return p_; }
    void upload(const T *src, hipStream_t s) {
        if (n_) hip_check(hipMemcpyAsync(p_, src, n_ * sizeof(T), hipMemcpyHostToDevice, s), "hipMemcpyAsync");
    }
    void download(T *dst, hipStream_t s) const {
        if (n_) hip_check(hipMemcpyAsync(dst, p_, n_ * sizeof(T), hipMemcpyDeviceToHost, s), "hipMemcpyAsync");
    }

private:
    T *p_ = nullptr;
    size_t n_ = 0;
};

}  // namespace detail

// One device + stream; not shared between threads (as a reference session).
class Context {
public:
    explicit Context(int device = 0, hipStream_t stream = nullptr) : stream_(stream) {
        const aq_status st = aq_ctx_create(device, stream, &ctx_);
        if (st != AQ_OK)
            throw std::runtime_error("aq_ctx_create failed (status " + std::to_string(static_cast<int>(st)) +
                                     "): no usable MI355X device " + std::to_string(device));
    }
    Context(const Context &) = delete;
    Context &operator=(const Context &) = delete;
    ~Context() {
        if (ctx_) aq_ctx_destroy(ctx_);
    }
    aq_ctx *get() const { return ctx_; }
    hipStream_t stream() const { return stream_; }
    void check(aq_status st) const {
        if (st != AQ_OK) throw std::runtime_error(aq_last_error(ctx_));
    }
    void synchronize() const { check(aq_ctx_synchronize(ctx_)); }

private:
    aq_ctx *ctx_ = nullptr;
    hipStream_t stream_ = nullptr;
};

// Euclidean VQ / RVQ with the reference recipe's arithmetic.
class EuclideanRvq {
public:
    // codebooks: Q x N x K floats (AQ_CB_F32) or Q x N x (K/32) GGUF
    // block_q8_0 records (AQ_CB_Q8_0), uploaded once.
    EuclideanRvq(Context &ctx, int64_t Q, int64_t N, int64_t K, const void *codebooks, aq_euclid_recipe recipe,
                 aq_codebook_type type = AQ_CB_F32)
        : ctx_(&ctx), Q_(Q), N_(N), K_(K) {
        ctx.check(aq_euclid_upload(ctx.get(), Q, N, K, type, codebooks, recipe, &cb_));
    }
    EuclideanRvq(const EuclideanRvq &) = delete;
    EuclideanRvq &operator=(const EuclideanRvq &) = delete;
    ~EuclideanRvq() {
        if (cb_) aq_euclid_release(cb_);
    }
    int64_t stages() const { return Q_; }
    int64_t codebook_size() const { return N_; }
    int64_t dim() const { return K_; }
    const aq_codebooks *handle() const { return cb_; }

    // Device pointers: x [M, K]; codes [M, Q]; residual [M, K] or null.
    void encode(const float *x, int64_t M, int32_t *codes, float *residual = nullptr, float *dist = nullptr,
                int topk = 0, int32_t *topk_idx = nullptr, float *topk_dist = nullptr,
                const int32_t *force_idx = nullptr) const {
        ctx_->check(aq_euclid_encode(ctx_->get(), cb_, x, M, codes, residual, dist, topk, topk_idx, topk_dist,
                                     force_idx));
    }

    // Host latent [frames, K] (frame-major) -> codes {frames, Q}.
    IntHostTensor encode(const std::vector<float> &latent, int64_t frames) const {
        if (static_cast<int64_t>(latent.size()) != frames * K_)
            throw std::runtime_error("EuclideanRvq latent size mismatch");
        detail::DeviceBuffer<float> x(latent.size());
        detail::DeviceBuffer<int32_t> c(static_cast<size_t>(frames * Q_));
        x.upload(latent.data(), ctx_->stream());
        encode(x.get(), frames, c.get());
        IntHostTensor out;
        out.shape = {frames, Q_};
        out.values.resize(static_cast<size_t>(frames * Q_));
        c.download(out.values.data(), ctx_->stream());
        ctx_->synchronize();
        return out;
    }

    // Device pointers: out[m] = sum over stages of codebook[s][codes[m, s]].
    void decode(const int32_t *codes, int64_t M, float *out) const {
        ctx_->check(aq_euclid_decode(ctx_->get(), cb_, codes, M, out));
    }

    // Device pointers: out[m] = codebook[stage][idx[m]] (get_rows).
    void gather(int64_t stage, const int32_t *idx, int64_t M, float *out) const {
        ctx_->check(aq_codebook_gather(ctx_->get(), cb_, stage, idx, M, out));
    }

private:
    Context *ctx_;
    int64_t Q_, N_, K_;
    aq_codebooks *cb_ = nullptr;
};

// DAC cosine RVQ: Fish Audio (codec.cpp:552-611) and, by recipe, IndexTTS2,
// Vevo2 and the OuteTTS host loop (dac.cpp:376-456).
class DacRvq {
public:
    // Host weights: w_in [Q,8,D], b_in [Q,8] or null, codebook [Q,N,8],
    // w_out [Q,D,8] (null: codes-only single stage), b_out [Q,D] or null
    // (weight norm already folded).
    DacRvq(Context &ctx, int64_t Q, int64_t D, int64_t N, const float *w_in, const float *b_in, const float *codebook,
           const float *w_out, const float *b_out, aq_dac_recipe recipe = AQ_DAC_FISH)
        : ctx_(&ctx), Q_(Q), D_(D), N_(N) {
        ctx.check(aq_dac_upload_ex(ctx.get(), Q, D, N, w_in, b_in, codebook, w_out, b_out, recipe, &st_));
    }
    DacRvq(const DacRvq &) = delete;
    DacRvq &operator=(const DacRvq &) = delete;
    ~DacRvq() {
        if (st_) aq_dac_release(st_);
    }

    // Device pointers: x [M, D] (M = clips * clip_len), codes [M, Q].
    void encode(const float *x, int64_t M, int64_t clip_len, int32_t *codes, float *residual = nullptr,
                float *recon = nullptr, const int32_t *force_idx = nullptr) const {
        ctx_->check(aq_dac_encode(ctx_->get(), st_, x, M, clip_len, codes, residual, recon, force_idx));
    }

    // Host latent [frames, D] -> codes {frames, Q}.
    IntHostTensor encode(const std::vector<float> &latent, int64_t frames, int64_t clip_len) const {
        if (static_cast<int64_t>(latent.size()) != frames * D_)
            throw std::runtime_error("DacRvq latent size mismatch");
        detail::DeviceBuffer<float> x(latent.size());
        detail::DeviceBuffer<int32_t> c(static_cast<size_t>(frames * Q_));
        x.upload(latent.data(), ctx_->stream());
        encode(x.get(), frames, clip_len, c.get());
        IntHostTensor out;
        out.shape = {frames, Q_};
        out.values.resize(static_cast<size_t>(frames * Q_));
        c.download(out.values.data(), ctx_->stream());
        ctx_->synchronize();
        return out;
    }

    // Device pointers: recon [M, D] = sum_s (W_out[s] c[s][codes[m,s]] + b_out[s]).
    void decode(const int32_t *codes, int64_t M, float *recon) const {
        ctx_->check(aq_dac_decode(ctx_->get(), st_, codes, M, recon));
    }

    const aq_dac_stages *handle() const { return st_; }

private:
    Context *ctx_;
    int64_t Q_, D_, N_;
    aq_dac_stages *st_ = nullptr;
};

// MOSS RLFQ quantizer (MossAudioTokenizerQuantizer,
// models/moss/shared/audio_tokenizer_quantizer.cpp): fp64 encode, fp32 decode.
class MossQuantizer {
public:
    // Host weights, weight norm folded: input_w [R,C], input_b [R], in_w
    // [Q,8,R], in_b [Q,8], codebook [Q,N,8], out_w [Q,R,8], out_b [Q,R],
    // output_w [C,R] and output_b [C] (both null: encode only).
    MossQuantizer(Context &ctx, int64_t Q, int64_t N, int64_t code_dim, int64_t rvq_dim, const float *input_w,
                  const float *input_b, const float *in_w, const float *in_b, const float *codebook,
                  const float *out_w, const float *out_b, const float *output_w, const float *output_b)
        : ctx_(&ctx), Q_(Q), C_(code_dim) {
        ctx.check(aq_moss_upload(ctx.get(), Q, N, code_dim, rvq_dim, input_w, input_b, in_w, in_b, codebook, out_w,
                                 out_b, output_w, output_b, &q_));
    }
    MossQuantizer(const MossQuantizer &) = delete;
    MossQuantizer &operator=(const MossQuantizer &) = delete;
    ~MossQuantizer() {
        if (q_) aq_moss_release(q_);
    }

    // Device pointers: hidden [M, C] -> codes [M, Q]; residual [M, R] doubles or null.
    void encode(const float *hidden, int64_t M, int32_t *codes, double *residual = nullptr,
                const int32_t *force_idx = nullptr) const {
        ctx_->check(aq_moss_encode(ctx_->get(), q_, hidden, M, codes, residual, force_idx));
    }

    // The reference's signature: hidden [frames, C] host, codes [Q][frames].
    std::vector<std::vector<int32_t>> encode(const std::vector<float> &hidden, int64_t frames) const {
        if (frames <= 0) throw std::runtime_error("MOSS codec quantizer requires a non-empty encoder latent");
        if (static_cast<int64_t>(hidden.size()) != frames * C_)
            throw std::runtime_error("MOSS codec quantizer got a mis-shaped encoder latent");
        detail::DeviceBuffer<float> h(hidden.size());
        detail::DeviceBuffer<int32_t> c(static_cast<size_t>(frames * Q_));
        h.upload(hidden.data(), ctx_->stream());
        encode(h.get(), frames, c.get());
        std::vector<int32_t> flat(static_cast<size_t>(frames * Q_));
        c.download(flat.data(), ctx_->stream());
        ctx_->synchronize();
        std::vector<std::vector<int32_t>> codes(static_cast<size_t>(Q_), std::vector<int32_t>(static_cast<size_t>(frames)));
        for (int64_t m = 0; m < frames; ++m)
            for (int64_t s = 0; s < Q_; ++s) codes[static_cast<size_t>(s)][static_cast<size_t>(m)] = flat[static_cast<size_t>(m * Q_ + s)];
        return codes;
    }

    // Device pointers: codes [M, Q] -> latent [M, C] (frame-major).
    void decode(const int32_t *codes, int64_t M, float *latent) const {
        ctx_->check(aq_moss_decode(ctx_->get(), q_, codes, M, latent));
    }

private:
    Context *ctx_;
    int64_t Q_, C_;
    aq_moss_quantizer *q_ = nullptr;
};

namespace engine::runtime {

// engine::runtime::VectorQuantizer on the MI355X: the nearest codeword of
// every input vector by squared Euclidean distance (rounded products added
// in order, first index of the minimum), returned as codewords.
class VectorQuantizer {
public:
    explicit VectorQuantizer(Context &ctx) : ctx_(&ctx) {}

    // Any dim and codebook_size, as the reference: shapes outside the fast
    // kernels' tiles take the library's exact any-width scan.  The size check
    // is the reference's (a plain product of the arguments); frames exist
    // only for batch > 0 and steps > 0, as its loops run.  An empty codebook
    // with frames to encode is an error here (the reference reads past the
    // end of its codebook vector).
    FloatHostTensor compute(const std::vector<float> &input, const std::vector<float> &codebook, int64_t batch,
                            int64_t steps, int64_t dim, int64_t codebook_size) const {
        if (static_cast<int64_t>(input.size()) != batch * steps * dim ||
            static_cast<int64_t>(codebook.size()) != codebook_size * dim) {
            throw std::runtime_error("VectorQuantizer input size mismatch");
        }
        FloatHostTensor result;
        result.shape = {batch, steps, dim};
        result.values.resize(input.size());
        const int64_t M = batch > 0 && steps > 0 ? batch * steps : 0;
        if (M == 0 || dim <= 0) return result;
        if (codebook_size <= 0) throw std::runtime_error("VectorQuantizer: empty codebook");
        EuclideanRvq rvq(*ctx_, 1, codebook_size, dim, codebook.data(), AQ_EUCLID_DIRECT);
        detail::DeviceBuffer<float> x(input.size()), out(input.size());
        detail::DeviceBuffer<int32_t> idx(static_cast<size_t>(M));
        x.upload(input.data(), ctx_->stream());
        rvq.encode(x.get(), M, idx.get());
        rvq.gather(0, idx.get(), M, out.get());
        out.download(result.values.data(), ctx_->stream());
        ctx_->synchronize();
        return result;
    }

private:
    Context *ctx_;
};

}  // namespace engine::runtime

}  // namespace aq

#endif  // AQ_MI355X_HPP
