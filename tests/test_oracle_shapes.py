"""CPU pins of the oracle at every shape the reference accepts.

The reference's quantizers take any codebook width, codebook size and latent
width (VectorQuantizer::compute, src/framework/runtime/host_ops.cpp:236-273;
ggml's mul_mat and conv graphs).  Outside the fast widths the arithmetic
that matters is ggml_vec_dot_f32's scalar leftover loop (n % 64 elements,
ggml-cpu/vec.cpp:125-128), whose code GCC lays out per target ISA.  These
tests pin the oracle's rule for it against oracle/_ref's own ggml builds and
then the whole recipes at odd shapes.
"""

import numpy as np
import pytest

from aqmi import synth
from oracle import REF_DIR, Oracle, Ref


def _beq(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.fixture(scope="module")
def o():
    return Oracle()


def _ref(isa):
    if not (REF_DIR / f"libaqref-{isa}.so").exists():
        pytest.skip("oracle/_ref not built here (needs /root/reference)")
    return Ref(isa)


@pytest.fixture(scope="module")
def ref():
    return _ref("native")


@pytest.mark.parametrize("isa,tail", [("native", 4), ("v4", 8)])
def test_vec_dot_leftover_rule_matches_ggml(o, isa, tail):
    """ggml_vec_dot_f32 on every length 1..200 (leftovers 0..63 after the
    64-wide blocks): the native build fuses the last rem % 4 leftovers, the
    x86-64-v4 build the last rem % 8.  A rule that fuses none of them, or
    all of them, fails on both builds."""
    r = _ref(isa)
    f = o.lib.aqo_vec_dot_f32_tail
    wrong = {0: 0, 1: 0}
    for n in range(1, 201):
        x = synth.normal(41, n, (n,))
        y = synth.normal(42, n, (n,), 0.3)
        want = np.float32(r.lib.aqref_vec_dot_f32(n, x, y))
        got = np.float32(f(n, x, y, tail))
        assert got.view(np.uint32) == want.view(np.uint32), (isa, n)
        # planted mistakes: no fused leftover (mod 1), every leftover fused (mod 64)
        wrong[0] += np.float32(f(n, x, y, 1)).view(np.uint32) != want.view(np.uint32)
        wrong[1] += np.float32(f(n, x, y, 64)).view(np.uint32) != want.view(np.uint32)
    assert wrong[0] > 10 and wrong[1] > 10
    if isa == "native":
        assert np.float32(o.lib.aqo_vec_dot_f32(7, x[:7], y[:7])) == np.float32(f(7, x, y, 4))


@pytest.mark.parametrize("K", [1, 7, 8, 13, 39, 100, 128, 1024])
@pytest.mark.parametrize("M", [1, 2, 40])
def test_oracle_euclid_any_width_vs_ggml(o, ref, K, M):
    """OmniVoice and Higgs logits at widths outside the fast set, N = 1000
    (not a multiple of any tile), one query (vec_dot order) and batches
    (tinyBLAS when K % 16 == 0)."""
    N = 1000
    x = synth.normal(5, 1, (M, K))
    cb = synth.normal(5, 2, (2, N, K), 0.25)
    cfg = dict(x=x, M=M, K=K, Q=2, N=N, codebook=cb)
    a, b = o.euclid_rvq(cfg), ref.euclid_rvq(cfg)
    assert np.array_equal(a["idx"], b["idx"])
    assert _beq(a["residual"], b["residual"]) and _beq(a["logit"], b["logit"])
    a, b = o.higgs_rvq(cfg), ref.higgs_rvq(cfg)
    assert np.array_equal(a["idx"], b["idx"])
    assert _beq(a["residual"], b["residual"]) and _beq(a["dist"], b["dist"])


@pytest.mark.parametrize("K", [8, 100, 128, 1024])
def test_oracle_direct_any_width_vs_vector_quantizer(o, ref, K):
    """engine::runtime::VectorQuantizer (compiled from the reference) at
    dims 8, 100, 128, 1024 with 1000 codewords."""
    N, M = 1000, 60
    x = synth.normal(6, 1, (M, K))
    cb = synth.normal(6, 2, (N, K), 0.25)
    want = ref.vector_quantizer(x, cb, batch=3)
    got = o.direct_rvq(dict(x=x, M=M, K=K, Q=1, N=N, codebook=cb[None]))
    assert _beq(cb[got["idx"][:, 0]], want)


@pytest.mark.parametrize("K,M", [(128, 1), (128, 33), (1024, 5), (32, 17)])
def test_oracle_higgs_q8_any_width_vs_ggml(o, ref, K, M):
    """Q8_0 codebooks (GGUF blocks) at widths outside the fast set, top-4."""
    N = 1000
    cfg = dict(x=synth.normal(7, 1, (M, K)), M=M, K=K, Q=2, N=N,
               codebook_q8=synth.q8_0_random_codebook(7, 2, 2 * N, K).reshape(2, N, K // 32))
    a, b = o.higgs_rvq(cfg, topk=4), ref.higgs_rvq(cfg, topk=4)
    assert np.array_equal(a["idx"], b["idx"])
    assert _beq(a["residual"], b["residual"]) and _beq(a["dist"], b["dist"])
    assert np.array_equal(a["topk_idx"], b["topk_idx"])


@pytest.mark.parametrize("D,N,T", [(96, 1000, 8), (96, 1000, 5), (99, 1000, 8), (1536, 1000, 8), (1536, 1000, 6),
                                   (70, 7, 3), (1000, 64, 4), (2048, 300, 4)])
@pytest.mark.parametrize("recipe", [0, 1, 2])
def test_oracle_dac_any_shape_vs_ggml(o, ref, D, N, T, recipe):
    """The cosine cascade at latent widths and codebook sizes outside the
    fast kernel's: D % 64 != 0 (vec_dot leftovers, tinyBLAS when D % 16 ==
    0 and T % 4 == 0), D > 1024, N not a multiple of 64."""
    B, Q = 2, 3
    cfg = dict(kind="dac", B=B, T=T, D=D, Q=Q, N=N, x=synth.normal(21, 1, (B * T, D)),
               **synth.dac_weights(21, Q, D, N, bias=True))
    a, b = o.dac_rvq(cfg, recipe=recipe), ref.dac_rvq(cfg, recipe=recipe)
    assert np.array_equal(a["idx"], b["idx"])
    assert _beq(a["residual"], b["residual"]) and _beq(a["recon"], b["recon"])
