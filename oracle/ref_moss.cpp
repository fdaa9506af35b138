// Reference harness: the MOSS RLFQ quantizer (MossAudioTokenizerQuantizer,
// src/models/moss/shared/audio_tokenizer_quantizer.cpp), compiled from the
// reference's sources (oracle/Makefile) and driven through its public
// constructor / encode / decode.  Test infrastructure only.
//
// The constructor reads its weights from an engine::assets::TensorSource by
// name; MapSource below implements that interface over in-memory vectors
// (the weight-norm parameters g and v, the biases and the codebooks).
#include "engine/framework/assets/tensor_source.h"
#include "engine/models/moss/shared/audio_tokenizer_quantizer.h"

#include <chrono>
#include <cstdint>
#include <map>
#include <omp.h>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

class MapSource final : public engine::assets::TensorSource {
public:
    std::map<std::string, std::vector<float>, std::less<>> tensors_;
    std::filesystem::path path_;

    const std::filesystem::path &source_path() const noexcept override { return path_; }
    bool has_tensor(std::string_view name) const noexcept override { return tensors_.find(name) != tensors_.end(); }
    engine::assets::TensorMetadata require_metadata(std::string_view name) const override {
        throw std::runtime_error("MapSource: no metadata for " + std::string(name));
    }
    std::vector<engine::assets::TensorMetadata> tensors() const override { return {}; }
    engine::assets::RawTensorData require_tensor_data(std::string_view name) const override {
        throw std::runtime_error("MapSource: no raw data for " + std::string(name));
    }
    std::vector<float> require_f32(std::string_view name,
                                   const std::optional<std::vector<int64_t>> &) const override {
        const auto it = tensors_.find(name);
        if (it == tensors_.end()) throw std::runtime_error("MapSource: missing " + std::string(name));
        return it->second;
    }
    std::optional<std::vector<float>> optional_f32(std::string_view name,
                                                   const std::optional<std::vector<int64_t>> &) const override {
        const auto it = tensors_.find(name);
        if (it == tensors_.end()) return std::nullopt;
        return it->second;
    }
    int64_t require_i64_scalar(std::string_view name) const override {
        throw std::runtime_error("MapSource: no scalar " + std::string(name));
    }

    void put(const std::string &name, const float *p, int64_t n) { tensors_[name].assign(p, p + n); }
    void put_wn(const std::string &prefix, const float *g, const float *v, int64_t out_ch, int64_t in_ch) {
        put(prefix + ".parametrizations.weight.original0", g, out_ch);
        put(prefix + ".parametrizations.weight.original1", v, out_ch * in_ch);
    }
};

struct MossWeights {
    int64_t C, R, Q, N;
    const float *ip_g, *ip_v, *ip_b;      // input_proj  [R], [R,C], [R]
    const float *in_g, *in_v, *in_b;      // per stage   [Q,8], [Q,8,R], [Q,8]
    const float *cb;                      //             [Q,N,8]
    const float *out_g, *out_v, *out_b;   // per stage   [Q,R], [Q,R,8], [Q,R]
    const float *op_g, *op_v, *op_b;      // output_proj [C], [C,R], [C]
};

engine::models::moss::MossAudioTokenizerQuantizer make(const MossWeights &w, MapSource &src) {
    src.put_wn("quantizer.input_proj", w.ip_g, w.ip_v, w.R, w.C);
    src.put("quantizer.input_proj.bias", w.ip_b, w.R);
    src.put_wn("quantizer.output_proj", w.op_g, w.op_v, w.C, w.R);
    src.put("quantizer.output_proj.bias", w.op_b, w.C);
    for (int64_t s = 0; s < w.Q; ++s) {
        const std::string p = "quantizer.quantizers." + std::to_string(s);
        src.put(p + ".codebook.weight", w.cb + s * w.N * 8, w.N * 8);
        src.put_wn(p + ".in_proj", w.in_g + s * 8, w.in_v + s * 8 * w.R, 8, w.R);
        src.put(p + ".in_proj.bias", w.in_b + s * 8, 8);
        src.put_wn(p + ".out_proj", w.out_g + s * w.R, w.out_v + s * w.R * 8, w.R, 8);
        src.put(p + ".out_proj.bias", w.out_b + s * w.R, w.R);
    }
    engine::models::moss::AudioTokenizerQuantizerConfig cfg;
    cfg.codebook_size = w.N;
    cfg.codebook_dim = 8;
    cfg.rvq_dim = w.R;
    cfg.code_dim = w.C;
    cfg.num_quantizers = w.Q;
    return engine::models::moss::MossAudioTokenizerQuantizer(src, w.Q, cfg);
}

}  // namespace

// hidden [frames, C] -> idx [frames, Q] (the reference returns [Q][frames]).
// Returns 0, or -1 when the reference throws.
extern "C" __attribute__((visibility("default"))) int aqref_moss_encode(const MossWeights *w, const float *hidden,
                                                                         int64_t frames, int32_t *idx) {
    try {
        MapSource src;
        const auto q = make(*w, src);
        std::vector<float> h(hidden, hidden + frames * w->C);
        const auto codes = q.encode(h, frames);
        for (int64_t s = 0; s < w->Q; ++s)
            for (int64_t m = 0; m < frames; ++m) idx[m * w->Q + s] = codes[static_cast<size_t>(s)][static_cast<size_t>(m)];
    } catch (...) {
        return -1;
    }
    return 0;
}

// The same encode with the constructor outside the clock: returns the
// milliseconds encode() took (threads > 0 sets the OpenMP team), or -1.
extern "C" __attribute__((visibility("default"))) double aqref_moss_encode_timed(const MossWeights *w,
                                                                                  const float *hidden, int64_t frames,
                                                                                  int32_t *idx, int threads) {
    if (threads > 0) omp_set_num_threads(threads);
    try {
        MapSource src;
        const auto q = make(*w, src);
        std::vector<float> h(hidden, hidden + frames * w->C);
        const auto t0 = std::chrono::steady_clock::now();
        const auto codes = q.encode(h, frames);
        const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        for (int64_t s = 0; s < w->Q; ++s)
            for (int64_t m = 0; m < frames; ++m) idx[m * w->Q + s] = codes[static_cast<size_t>(s)][static_cast<size_t>(m)];
        return ms;
    } catch (...) {
        return -1.0;
    }
}

// idx [frames, Q] -> latent [C, frames] (channel-major, as the reference returns it).
extern "C" __attribute__((visibility("default"))) int aqref_moss_decode(const MossWeights *w, const int32_t *idx,
                                                                         int64_t frames, float *latent) {
    try {
        MapSource src;
        const auto q = make(*w, src);
        std::vector<std::vector<int32_t>> codes(static_cast<size_t>(w->Q), std::vector<int32_t>(static_cast<size_t>(frames)));
        for (int64_t s = 0; s < w->Q; ++s)
            for (int64_t m = 0; m < frames; ++m) codes[static_cast<size_t>(s)][static_cast<size_t>(m)] = idx[m * w->Q + s];
        const auto out = q.decode(codes);
        std::copy(out.begin(), out.end(), latent);
    } catch (...) {
        return -1;
    }
    return 0;
}
