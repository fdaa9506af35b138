// Reference harness: the OuteTTS DAC host quantizer, compiled from the
// reference's own source (src/community_models/outetts/dac.cpp, included
// below as is; test infrastructure only, never part of the product).
//
// quantize_reference (dac.cpp:376-456) lives in an anonymous namespace of that
// file, so this translation unit includes the file and calls it.  It is built
// with hidden visibility and section GC (oracle/Makefile), which drops the
// file's graph code and its references to the rest of the reference engine.
#include "community_models/outetts/dac.cpp"

#include <chrono>
#include <cstdint>
#include <cstring>
#include <omp.h>

// x [frames, 1024] frame-major; per stage s in {0, 1}: w_in [8,1024],
// b_in [8], codebook [1024,8], w_out [1024,8], b_out [1024] (weight norm
// already folded, as HostQuantizerWeights holds them); idx [frames, 2].
// threads > 0 sets the OpenMP team the reference's loops use.  Returns the
// milliseconds quantize_reference took, or -1 when the reference throws.
extern "C" __attribute__((visibility("default"))) double aqref_outetts_rvq(
    const float *x, int64_t frames, const float *w_in, const float *b_in, const float *codebook,
    const float *w_out, const float *b_out, int32_t *idx, int threads) {
    namespace ot = engine::models::outetts;
    constexpr int64_t D = 1024, N = 1024;
    std::vector<ot::HostQuantizerWeights> q(2);
    for (int s = 0; s < 2; ++s) {
        q[s].in_weight.assign(w_in + s * 8 * D, w_in + (s + 1) * 8 * D);
        q[s].in_bias.assign(b_in + s * 8, b_in + (s + 1) * 8);
        q[s].codebook.assign(codebook + s * N * 8, codebook + (s + 1) * N * 8);
        q[s].out_weight.assign(w_out + s * D * 8, w_out + (s + 1) * D * 8);
        q[s].out_bias.assign(b_out + s * D, b_out + (s + 1) * D);
    }
    if (threads > 0) omp_set_num_threads(threads);
    double ms = 0.0;
    try {
        std::vector<float> fm(x, x + frames * D);
        const auto t0 = std::chrono::steady_clock::now();
        const auto codes = ot::quantize_reference(fm, q);
        ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        for (int64_t m = 0; m < frames; ++m) {
            idx[m * 2 + 0] = codes.first[static_cast<size_t>(m)];
            idx[m * 2 + 1] = codes.second[static_cast<size_t>(m)];
        }
    } catch (...) {
        return -1.0;
    }
    return ms;
}

// fold_weight_norm (dac.cpp:91-110) as the loader calls it: v [dim0, dim1,
// kernel], g [dim0] -> out [dim0, dim1, kernel].
extern "C" __attribute__((visibility("default"))) void aqref_outetts_fold(const float *v, const float *g, int64_t dim0,
                                                                         int64_t dim1, int64_t kernel, float *out) {
    namespace ot = engine::models::outetts;
    const std::vector<float> vv(v, v + dim0 * dim1 * kernel), gg(g, g + dim0);
    const std::vector<float> w = ot::fold_weight_norm(vv, gg, dim0, dim1, kernel);
    std::memcpy(out, w.data(), w.size() * sizeof(float));
}
