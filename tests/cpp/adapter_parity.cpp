// C++ host-interface parity test (test infrastructure): drives the library
// through include/aq_mi355x.hpp the way audio.cpp's call sites would, and
// checks every result bit for bit against the plain-C oracle
// (oracle/aq_oracle.c, pinned to the reference's ggml build).
//
// Exit status: 0 all checks passed, 1 a check failed, 77 no GPU (the
// context could not be created; the error path itself is still checked).
#include "aq_mi355x.hpp"

extern "C" {
#include "aq_oracle.h"
}

#include <cmath>
#include <memory>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

int failures = 0;

void expect(bool ok, const char *what) {
    std::printf("%s %s\n", ok ? "PASS" : "FAIL", what);
    std::fflush(stdout);
    if (!ok) ++failures;
}

// Deterministic normal variates (splitmix64 + Box-Muller), test data only.
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed) {}
    uint64_t next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    double uniform() { return ((next() >> 11) + 1) * (1.0 / 9007199254740992.0); }
    std::vector<float> normal(size_t n, double std) {
        std::vector<float> v(n);
        for (auto &x : v) x = static_cast<float>(std * std::sqrt(-2.0 * std::log(uniform())) * std::cos(6.283185307179586 * uniform()));
        return v;
    }
};

bool same_bits(const float *a, const float *b, size_t n) { return std::memcmp(a, b, n * sizeof(float)) == 0; }

}  // namespace

int main() {
    // The reference's size check and message, with or without a GPU.
    std::unique_ptr<aq::Context> ctx;
    try {
        ctx = std::make_unique<aq::Context>(0);
    } catch (const std::runtime_error &e) {
        std::printf("SKIP no GPU: %s\n", e.what());
        return 77;
    }
    aq::engine::runtime::VectorQuantizer vq(*ctx);
    try {
        vq.compute(std::vector<float>(10), std::vector<float>(2048 * 256), 1, 2, 256, 2048);
        expect(false, "VectorQuantizer size check throws");
    } catch (const std::runtime_error &e) {
        expect(std::string(e.what()) == "VectorQuantizer input size mismatch", "VectorQuantizer size check message");
    }

    Rng rng(7);
    {   // VectorQuantizer: batch 2 x steps 300 x dim 256 against 2048 codewords
        const int64_t B = 2, T = 300, K = 256, N = 2048;
        const auto x = rng.normal(B * T * K, 1.0);
        const auto cb = rng.normal(N * K, 1.0 / 16);
        const auto got = vq.compute(x, cb, B, T, K, N);
        std::vector<int32_t> idx(B * T);
        std::vector<float> res(B * T * K), dist(B * T), want(B * T * K);
        aqo_direct_rvq(x.data(), B * T, K, 1, N, cb.data(), nullptr, idx.data(), res.data(), dist.data());
        aqo_gather_f32(cb.data(), N, K, idx.data(), B * T, want.data());
        expect(got.shape == std::vector<int64_t>({B, T, K}), "VectorQuantizer result shape");
        expect(same_bits(got.values.data(), want.data(), want.size()), "VectorQuantizer codewords == oracle");
    }
    {   // EuclideanRvq, OmniVoice recipe, 3 stages
        const int64_t M = 1000, K = 256, Q = 3, N = 2048;
        const auto x = rng.normal(M * K, 1.0);
        const auto cb = rng.normal(Q * N * K, 1.0 / 16);
        aq::EuclideanRvq rvq(*ctx, Q, N, K, cb.data(), AQ_EUCLID_OMNIVOICE);
        const auto codes = rvq.encode(x, M);
        std::vector<int32_t> idx(M * Q);
        std::vector<float> res(M * K), lb(M * Q);
        aqo_euclid_rvq(x.data(), M, K, Q, N, cb.data(), nullptr, idx.data(), res.data(), lb.data());
        expect(codes.values == idx, "EuclideanRvq (OmniVoice) codes == oracle");
    }
    {   // DacRvq, Fish recipe, 4 stages, 2 clips of 750 frames
        const int64_t B = 2, T = 750, D = 1024, Q = 4, N = 1024;
        const auto x = rng.normal(B * T * D, 1.0);
        const auto w_in = rng.normal(Q * 8 * D, 1.0 / 32);
        const auto cb = rng.normal(Q * N * 8, 1.0);
        const auto w_out = rng.normal(Q * D * 8, 0.35);
        const auto b_in = rng.normal(Q * 8, 0.1);
        const auto b_out = rng.normal(Q * D, 0.1);
        aq::DacRvq dac(*ctx, Q, D, N, w_in.data(), b_in.data(), cb.data(), w_out.data(), b_out.data());
        const auto codes = dac.encode(x, B * T, T);
        std::vector<int32_t> idx(B * T * Q);
        std::vector<float> res(B * T * D), rec(B * T * D);
        aqo_dac_rvq(x.data(), B, T, D, Q, N, w_in.data(), b_in.data(), cb.data(), w_out.data(), b_out.data(), nullptr,
                    idx.data(), res.data(), rec.data());
        expect(codes.values == idx, "DacRvq (Fish) codes == oracle");
    }
    {   // DacRvq, OuteTTS host-loop recipe, its shapes (2 stages, D = N = 1024)
        const int64_t M = 500, D = 1024, Q = 2, N = 1024;
        const auto x = rng.normal(M * D, 1.0);
        const auto w_in = rng.normal(Q * 8 * D, 1.0 / 32);
        const auto cb = rng.normal(Q * N * 8, 1.0);
        const auto w_out = rng.normal(Q * D * 8, 0.35);
        const auto b_in = rng.normal(Q * 8, 0.1);
        const auto b_out = rng.normal(Q * D, 0.1);
        aq::DacRvq dac(*ctx, Q, D, N, w_in.data(), b_in.data(), cb.data(), w_out.data(), b_out.data(),
                       AQ_DAC_OUTETTS);
        const auto codes = dac.encode(x, M, M);
        std::vector<int32_t> idx(M * Q);
        std::vector<float> res(M * D);
        aqo_outetts_rvq(x.data(), M, D, Q, N, w_in.data(), b_in.data(), cb.data(), w_out.data(), b_out.data(), nullptr,
                        idx.data(), res.data());
        expect(codes.values == idx, "DacRvq (OuteTTS) codes == oracle");
    }
    {   // MossQuantizer with the reference's encode signature ([Q][frames] codes)
        const int64_t M = 64, C = 768, R = 512, Q = 12, N = 1024;
        const auto h = rng.normal(M * C, 1.0);
        auto fold = [&](int64_t lead, int64_t out_ch, int64_t in_ch) {
            const auto v = rng.normal(lead * out_ch * in_ch, 1.0);
            std::vector<float> g(static_cast<size_t>(lead * out_ch), 1.25f), w(v.size());
            for (int64_t i = 0; i < lead; ++i)
                aqo_moss_weight_norm(g.data() + i * out_ch, v.data() + i * out_ch * in_ch, out_ch, in_ch,
                                     w.data() + i * out_ch * in_ch);
            return w;
        };
        const auto w_ip = fold(1, R, C), w_in = fold(Q, 8, R), w_out = fold(Q, R, 8), w_op = fold(1, C, R);
        const auto b_ip = rng.normal(R, 0.1), b_in = rng.normal(Q * 8, 0.1), b_out = rng.normal(Q * R, 0.1);
        const auto b_op = rng.normal(C, 0.1);
        const auto cb = rng.normal(Q * N * 8, 1.0);
        aq::MossQuantizer moss(*ctx, Q, N, C, R, w_ip.data(), b_ip.data(), w_in.data(), b_in.data(), cb.data(),
                               w_out.data(), b_out.data(), w_op.data(), b_op.data());
        const auto codes = moss.encode(h, M);
        std::vector<int32_t> idx(M * Q);
        aqo_moss_rvq(h.data(), M, C, R, Q, N, w_ip.data(), b_ip.data(), w_in.data(), b_in.data(), cb.data(),
                     w_out.data(), b_out.data(), nullptr, idx.data(), nullptr);
        bool same = codes.size() == static_cast<size_t>(Q);
        for (int64_t s = 0; same && s < Q; ++s)
            for (int64_t m = 0; m < M; ++m) same = same && codes[s][m] == idx[m * Q + s];
        expect(same, "MossQuantizer codes [Q][frames] == oracle");
        try {
            (void)moss.encode(std::vector<float>(10), 2);
            expect(false, "MossQuantizer shape check throws");
        } catch (const std::runtime_error &e) {
            expect(std::string(e.what()) == "MOSS codec quantizer got a mis-shaped encoder latent",
                   "MossQuantizer shape message");
        }
    }
    {   // VectorQuantizer at a dim and codebook size outside the fast tiles
        const int64_t B = 2, T = 50, K = 100, N = 1000;
        const auto x = rng.normal(B * T * K, 1.0);
        const auto cb = rng.normal(N * K, 0.25);
        const auto got = vq.compute(x, cb, B, T, K, N);
        std::vector<int32_t> idx(B * T);
        std::vector<float> res(B * T * K), dist(B * T), want(B * T * K);
        aqo_direct_rvq(x.data(), B * T, K, 1, N, cb.data(), nullptr, idx.data(), res.data(), dist.data());
        aqo_gather_f32(cb.data(), N, K, idx.data(), B * T, want.data());
        expect(same_bits(got.values.data(), want.data(), want.size()), "VectorQuantizer dim 100 x 1000 == oracle");
    }
    {   // errors surface as std::runtime_error with the library's message
        try {
            const auto cb = rng.normal(100 * 40, 1.0);
            aq::EuclideanRvq bad(*ctx, 1, 100, 40, cb.data(), AQ_EUCLID_HIGGS, AQ_CB_F32_AS_Q8_0);
            expect(false, "Q8_0 rows of partial blocks throw");
        } catch (const std::runtime_error &e) {
            expect(std::string(e.what()).find("aq_euclid_upload") != std::string::npos, "Q8_0 partial block message");
        }
    }
    std::printf("%s (%d failed)\n", failures ? "FAILED" : "OK", failures);
    return failures ? 1 : 0;
}
