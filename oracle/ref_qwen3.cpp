// Reference harness: the Qwen3-TTS speech-tokenizer quantizer
// (quantize_projected, src/models/qwen3_tts/tokenizer_speech_encoder.cpp:
// 305-349, with codebook_embedding :271-285 and nearest_code :287-303),
// compiled from the reference's own source, which is included below as is
// (test infrastructure only, never part of the product).  Built with hidden
// visibility and section GC (oracle/Makefile), which drops the file's graph
// code and its references to the rest of the reference engine.
#include "models/qwen3_tts/tokenizer_speech_encoder.cpp"

#include <chrono>
#include <cstdint>
#include <cstring>

// semantic, acoustic: channel-major [256, frames] as the encoder graph leaves
// them; embedding_sum [16, 2048, 256] and cluster_usage [16, 2048] (stage 0
// the semantic codebook, stages 1..15 the acoustic ones); codes [frames, 16]
// as the reference returns them.  Returns milliseconds, or -1 when the
// reference throws.
extern "C" __attribute__((visibility("default"))) double aqref_qwen3_quantize(
    const float *semantic, const float *acoustic, int64_t frames, const float *embedding_sum,
    const float *cluster_usage, int32_t *codes) {
    namespace q3 = engine::models::qwen3_tts;
    constexpr int64_t S = 16, N = 2048, K = 256;
    q3::Qwen3SpeechTokenizerEncoderWeights w;
    for (int64_t s = 0; s < S; ++s) {
        q3::CodebookWeights cb;
        cb.embedding_sum.assign(embedding_sum + s * N * K, embedding_sum + (s + 1) * N * K);
        cb.cluster_usage.assign(cluster_usage + s * N, cluster_usage + (s + 1) * N);
        (s == 0 ? w.semantic_codebooks : w.acoustic_codebooks).push_back(std::move(cb));
    }
    try {
        std::vector<float> sem(semantic, semantic + K * frames), ac(acoustic, acoustic + K * frames);
        const auto t0 = std::chrono::steady_clock::now();
        const auto out = q3::quantize_projected(sem, ac, frames, w);
        const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        std::memcpy(codes, out.data(), out.size() * sizeof(int32_t));
        return ms;
    } catch (...) {
        return -1.0;
    }
}
