// Parity program for the reference-header binding (test infrastructure):
// calls engine::runtime::VectorQuantizer -- the reference's own class, as
// declared by its header -- whose compute() is the MI355X binding of
// ref_host_ops_adapter.cpp, at codebook dims inside and outside the fast
// kernels' tiles, and checks the codewords bit for bit against the oracle's
// restatement of the reference loop (oracle/aq_oracle.c aqo_direct_rvq,
// pinned to the reference's compiled host_ops.cpp in tests/test_oracle.py).
//
// Exit status: 0 all checks passed, 1 a check failed, 77 no GPU.
#include "engine/framework/runtime/host_ops.h"

#include <hip/hip_runtime_api.h>

extern "C" {
#include "aq_oracle.h"
}

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

int failures = 0;

void expect(bool ok, const std::string &what) {
    std::printf("%s %s\n", ok ? "PASS" : "FAIL", what.c_str());
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
        for (auto &x : v)
            x = static_cast<float>(std * std::sqrt(-2.0 * std::log(uniform())) * std::cos(6.283185307179586 * uniform()));
        return v;
    }
};

}  // namespace

int main() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        std::printf("SKIP no GPU\n");
        return 77;
    }
    const engine::runtime::VectorQuantizer vq;   // the reference's type
    try {
        (void)vq.compute(std::vector<float>(10), std::vector<float>(1000 * 8), 1, 2, 8, 1000);
        expect(false, "size check throws");
    } catch (const std::runtime_error &e) {
        expect(std::string(e.what()) == "VectorQuantizer input size mismatch", "size check message");
    }
    Rng rng(11);
    for (const int64_t dim : {8, 100, 128, 256, 1024}) {
        const int64_t B = 3, T = 70, N = dim == 256 ? 2048 : 1000;
        const auto x = rng.normal(static_cast<size_t>(B * T * dim), 1.0);
        const auto cb = rng.normal(static_cast<size_t>(N * dim), 0.25);
        const engine::runtime::FloatHostTensor got = vq.compute(x, cb, B, T, dim, N);
        std::vector<int32_t> idx(static_cast<size_t>(B * T));
        std::vector<float> res(x.size()), dist(static_cast<size_t>(B * T)), want(x.size());
        aqo_direct_rvq(x.data(), B * T, dim, 1, N, cb.data(), nullptr, idx.data(), res.data(), dist.data());
        aqo_gather_f32(cb.data(), N, dim, idx.data(), B * T, want.data());
        const std::string tag = "dim " + std::to_string(dim) + " x " + std::to_string(N) + " codewords";
        expect(got.shape == std::vector<int64_t>({B, T, dim}), tag + ": shape");
        expect(got.values.size() == want.size() &&
                   std::memcmp(got.values.data(), want.data(), want.size() * sizeof(float)) == 0,
               tag + ": codewords == oracle");
    }
    {   // no frames: the reference's loops do not run
        const auto got = vq.compute({}, std::vector<float>(5 * 16), 0, 4, 16, 5);
        expect(got.values.empty() && got.shape == std::vector<int64_t>({0, 4, 16}), "empty batch");
    }
    std::printf("%s (%d failed)\n", failures ? "FAILED" : "OK", failures);
    return failures ? 1 : 0;
}
