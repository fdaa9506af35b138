"""CPU checks that pin the oracle (oracle/aq_oracle.c) before it is trusted.

Three kinds of pins:
  1. golden fixtures written by the reference's own ggml CPU build
     (tests/golden/make_golden.py) -- run everywhere, including the GPU box;
  2. bit-exact agreement with oracle/_ref (ggml compiled from the reference
     sources) on seeded inputs of every recipe -- run where _ref is built;
  3. closed forms and special cases that a plausible restatement mistake (a
     dropped term, wrong tie rule, wrong rounding mode, transposed operand)
     would fail.
"""

import hashlib

import numpy as np
import pytest

from conftest import GOLDEN

from aqmi import synth
from oracle import REF_DIR, Oracle, Ref


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _beq(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.fixture(scope="module")
def o():
    return Oracle()


@pytest.fixture(scope="module")
def ref():
    if not (REF_DIR / "libaqref-native.so").exists():
        pytest.skip("oracle/_ref not built here (needs /root/reference)")
    return Ref("native")


# ---------------------------------------------------------------- fixtures --

@pytest.mark.parametrize("name,cfg_id,bias", [("dac_cfg0.npz", 0, False), ("dac_cfg0_bias.npz", 0, True),
                                              ("dac_cfg1.npz", 1, False)])
def test_oracle_dac_matches_golden(o, name, cfg_id, bias):
    g = np.load(GOLDEN / name)
    cfg = synth.make_config(cfg_id)
    if bias:
        cfg.update(synth.dac_weights(cfg["seed"], cfg["Q"], cfg["D"], cfg["N"], bias=True))
    out = o.dac_rvq(cfg)
    assert np.array_equal(out["idx"], g["idx"].astype(np.int32))
    assert _sha(out["residual"]) == str(g["residual_sha"])
    assert _sha(out["recon"]) == str(g["recon_sha"])


def _sorted_topk(idx, val):
    order = np.lexsort((idx, -val.astype(np.float64)), axis=-1)
    return np.take_along_axis(idx, order, -1), np.take_along_axis(val, order, -1)


def test_oracle_mimi_matches_golden_prefix(o):
    """configs[2] (OmniVoice recipe): frames are independent through the
    cascade, so the oracle on the first rows must reproduce the fixture's
    first rows (codes, best logits and final residual, bit for bit)."""
    g = np.load(GOLDEN / "mimi_cfg2.npz")
    rows = 64
    cfg = synth.make_config(2, rows=rows)
    out = o.euclid_rvq(cfg)
    assert np.array_equal(out["idx"], g["idx"][:rows].astype(np.int32))
    assert _beq(out["logit"], g["logit_head"])
    assert _beq(out["residual"], g["residual_head"])


def test_oracle_kmeans_matches_golden_prefix(o):
    """configs[3] (Higgs recipe, one stage of 16384 centroids, K = 768)."""
    g = np.load(GOLDEN / "kmeans_cfg3.npz")
    rows = 48
    cfg = synth.make_config(3, rows=rows)
    out = o.higgs_rvq(cfg)
    assert np.array_equal(out["idx"][:, 0], g["idx"][:rows].astype(np.int32))
    assert _beq(out["dist"][:, 0], g["dist_head"][:rows])


def test_oracle_q8_topk_matches_golden_prefix(o):
    """configs[4] (Q8_0 codebooks, Higgs recipe, top-4 sets with logits)."""
    g = np.load(GOLDEN / "q8_cfg4.npz")
    rows = 64
    cfg = synth.make_config(4, rows=rows)
    out = o.higgs_rvq(cfg, topk=4)
    assert np.array_equal(out["idx"], g["idx"][:rows].astype(np.int32))
    assert _beq(out["residual"], g["residual_head"])
    ti, tl = _sorted_topk(out["topk_idx"], out["topk_logit"])
    assert np.array_equal(ti, g["topk_idx_head"])
    assert _beq(tl, g["topk_logit_head"])


def test_generator_is_stable():
    """The fixtures assume the seeded generator never changes."""
    x = synth.normal(1, 1, (4,))
    assert x.view(np.uint32).tolist() == np.array(x, np.float32).view(np.uint32).tolist()
    assert _sha(synth.normal(1, 1, (1000,))) == _sha(synth.normal(1, 1, (1000,)))
    z = synth.normal(123, 7, (200000,))
    assert abs(float(z.mean())) < 0.01 and abs(float(z.std()) - 1.0) < 0.01


# ------------------------------------------------------ bit-exact vs ggml --

@pytest.mark.parametrize("T", [750, 752, 5])
def test_oracle_dac_bit_exact_vs_ggml(o, ref, T):
    cfg = dict(kind="dac", B=2, T=T, D=1024, Q=3, N=1024, x=synth.normal(21, 1, (2 * T, 1024)),
               **synth.dac_weights(21, 3, 1024, 1024, bias=True))
    a, b = o.dac_rvq(cfg), ref.dac_rvq(cfg)
    assert np.array_equal(a["idx"], b["idx"])
    assert _beq(a["residual"], b["residual"]) and _beq(a["recon"], b["recon"])


@pytest.mark.parametrize("recipe", [1, 2])
@pytest.mark.parametrize("T", [75, 5])
def test_oracle_dac_recipes_bit_exact_vs_ggml(o, ref, recipe, T):
    """IndexTTS2 (ggml_sqr, no bias; 1.0F / (float)sqrt codebook rows) and
    Vevo2 (+1e-20; (float)(1 / norm) rows) normalisation, N = 8192 as in
    IndexTTS2's semantic codec, against the ggml op sequences."""
    cfg = dict(kind="dac", B=2, T=T, D=1024, Q=2, N=8192, x=synth.normal(22, 1, (2 * T, 1024)),
               **synth.dac_weights(22, 2, 1024, 8192, bias=True))
    a, b = o.dac_rvq(cfg, recipe=recipe), ref.dac_rvq(cfg, recipe=recipe)
    assert np.array_equal(a["idx"], b["idx"])
    assert _beq(a["residual"], b["residual"]) and _beq(a["recon"], b["recon"])


def test_oracle_dac_recipe_edge_cases(o, ref):
    """A zero projection: Fish and Vevo2 divide by sqrt(eps) (codes defined),
    IndexTTS2 divides by 0 (NaN scores; ggml_argmax's NaN rule picks the
    code).  A zero codebook row: Fish maps it to 0, IndexTTS2 to NaN, Vevo2
    rejects the codebook."""
    T = 6
    w = synth.dac_weights(23, 1, 64, 128, bias=False)
    x = synth.normal(23, 1, (T, 64))
    x[2] = 0.0
    cfg = dict(kind="dac", B=1, T=T, D=64, Q=1, N=128, x=x, **w)
    for recipe in (0, 1, 2):
        a, b = o.dac_rvq(cfg, recipe=recipe), ref.dac_rvq(cfg, recipe=recipe)
        assert np.array_equal(a["idx"], b["idx"])
    w2 = dict(w)
    w2["codebook"] = w["codebook"].copy()
    w2["codebook"][0, 5] = 0.0
    cfg2 = dict(cfg, **w2)
    for recipe in (0, 1):
        a, b = o.dac_rvq(cfg2, recipe=recipe), ref.dac_rvq(cfg2, recipe=recipe)
        assert np.array_equal(a["idx"], b["idx"])
    with pytest.raises(ValueError):
        o.dac_rvq(cfg2, recipe=2)
    with pytest.raises(ValueError):
        ref.dac_rvq(cfg2, recipe=2)


@pytest.mark.parametrize("M", [1, 2, 5, 64])
def test_oracle_euclid_bit_exact_vs_ggml(o, ref, M):
    cfg = synth.make_config(2, rows=M)
    cfg["Q"] = 3
    cfg["codebook"] = cfg["codebook"][:3]
    a, b = o.euclid_rvq(cfg), ref.euclid_rvq(cfg)
    assert np.array_equal(a["idx"], b["idx"])
    assert _beq(a["residual"], b["residual"]) and _beq(a["logit"], b["logit"])


@pytest.mark.parametrize("M", [1, 3, 32])
def test_oracle_higgs_f32_bit_exact_vs_ggml(o, ref, M):
    cfg = synth.make_config(3, rows=M)
    cfg["codebook"] = cfg["codebook"][:, :1024]
    cfg["N"] = 1024
    a, b = o.higgs_rvq(cfg), ref.higgs_rvq(cfg)
    assert np.array_equal(a["idx"], b["idx"])
    assert _beq(a["residual"], b["residual"]) and _beq(a["dist"], b["dist"])


@pytest.mark.parametrize("M", [1, 3, 48])
def test_oracle_higgs_q8_bit_exact_vs_ggml(o, ref, M):
    cfg = synth.make_config(4, rows=M)
    cfg["Q"] = 3
    cfg["codebook_q8"] = cfg["codebook_q8"][:3]
    a, b = o.higgs_rvq(cfg, topk=4), ref.higgs_rvq(cfg, topk=4)
    assert np.array_equal(a["idx"], b["idx"])
    assert _beq(a["residual"], b["residual"]) and _beq(a["dist"], b["dist"])
    # the oracle restates ggml_top_k's own order (heap, then dst[0] <-> dst[1])
    assert np.array_equal(a["topk_idx"], b["topk_idx"])
    assert _beq(a["topk_logit"], b["topk_logit"])


@pytest.mark.parametrize("n,k", [(1, 1), (2, 2), (5, 4), (6, 3), (17, 4), (64, 2), (2048, 4), (2048, 1)])
def test_top_k_heap_selection_matches_ggml(o, ref, n, k):
    """Rows drawn from a handful of values (many exact ties, also at the k-th
    place) and rows with NaN / inf: which tied codes ggml_top_k keeps is
    decided by std::partial_sort's heap; the restatement must keep the same
    ones, in the same order.  A plain stable sort would fail these."""
    rng = np.random.default_rng(n * 10 + k)
    rows = [rng.integers(0, 4, size=n).astype(np.float32) for _ in range(200)]
    rows += [rng.normal(size=n).astype(np.float32) for _ in range(20)]
    for _ in range(20):
        r = rng.integers(0, 3, size=n).astype(np.float32)
        r[rng.integers(0, n, size=max(1, n // 5))] = np.nan
        r[rng.integers(0, n)] = np.inf
        rows.append(r)
    v = np.stack(rows)
    a, b = o.top_k(v, k), ref.top_k(v, k)
    assert np.array_equal(a, b)
    if n in (5, 6, 17):
        # on these rows the set is not "the smallest indices among ties"
        stable = np.argsort(-v[:200].astype(np.float64), axis=1, kind="stable")[:, :k]
        assert not np.array_equal(np.sort(stable, 1), np.sort(b[:200], 1))


def test_oracle_q8_quantize_matches_ggml(o, ref):
    x = synth.normal(8, 1, (64 * 32,))
    x[:32] = 0.0                                 # amax = 0 block
    x[32:64] = np.linspace(-3, 3, 32)
    ya = np.zeros(64, dtype=synth.Q8_DTYPE)
    yb = np.zeros(64, dtype=synth.Q8_DTYPE)
    o.lib.aqo_quantize_row_q8_0_x86(x, ya.ctypes.data, x.size)
    ref.lib.aqref_quantize_row_q8_0(x, yb.ctypes.data, x.size)
    assert ya.tobytes() == yb.tobytes()
    o.lib.aqo_quantize_row_q8_0_ref(x, ya.ctypes.data, x.size)
    ref.lib.aqref_quantize_chunk_q8_0(x, yb.ctypes.data, 1, x.size)
    assert ya.tobytes() == yb.tobytes()


def test_reference_cpu_view_bug_is_real(ref):
    """Fish l2_normalize_last on the CPU backend divides a permuted view;
    ggml's CPU binary op reads it as contiguous rows.  The as-is graph gives
    codes unrelated to the exact cosine argmax; the materialised graph (what
    the oracle follows) agrees with float64 math."""
    cfg = synth.make_config(0)
    x = cfg["x"].astype(np.float64)
    p = x @ cfg["w_in"][0].astype(np.float64).T
    cb = cfg["codebook"][0].astype(np.float64)
    exact = ((p / np.linalg.norm(p, axis=1, keepdims=True)) @ (cb / np.linalg.norm(cb, axis=1, keepdims=True)).T).argmax(1)
    asis = ref.dac_rvq(cfg, materialize=False)["idx"][:, 0]
    fixed = ref.dac_rvq(cfg, materialize=True)["idx"][:, 0]
    assert (fixed == exact).mean() > 0.99
    assert (asis == exact).mean() < 0.05


# ------------------------------------------------ closed forms / special --

def test_argmax_last_index_and_nan(o):
    assert o.lib.aqo_argmax_f32(5, np.array([1, 3, 3, 2, 3], np.float32)) == 4
    assert o.lib.aqo_argmax_f32(3, np.full(3, -np.inf, np.float32)) == 2
    assert o.lib.aqo_argmax_f32(4, np.array([0, 0, 0, 0], np.float32)) == 3
    # NaN restarts ggml's running max: [5, NaN, 1] -> index 2 (not 0).
    assert o.lib.aqo_argmax_f32(3, np.array([5, np.nan, 1], np.float32)) == 2
    assert o.lib.aqo_argmax_f32(3, np.array([5, 1, np.nan], np.float32)) == 0


def test_fp16_round_to_nearest_even(o):
    vals = np.concatenate([synth.normal(3, 9, (5000,)) * 1e-3, synth.normal(3, 10, (5000,)) * 100,
                           np.array([65504, 65520, 65519.99, 1e-8, 5.96e-8, 2.98e-8, 2.99e-8, -0.0, np.inf, -np.inf],
                                    np.float32)]).astype(np.float32)
    got = np.array([o.lib.aqo_fp32_to_fp16(float(v)) for v in vals], np.uint16)
    want = vals.astype(np.float16).view(np.uint16)               # numpy converts with RNE
    assert np.array_equal(got, want)
    back = np.array([o.lib.aqo_fp16_to_fp32(int(h)) for h in want[:200]], np.float32)
    assert _beq(back, want[:200].view(np.float16).astype(np.float32))


def test_q8_quantize_known_answers(o):
    """x86 query quantisation: d = fp16(amax/127), q = RNE(x * 127/amax)."""
    x = np.zeros(32, np.float32)
    x[0] = 127.0                                  # amax = 127 -> id = 1
    x[1], x[2], x[3], x[4] = 0.5, 1.5, 2.5, -0.5  # half-way cases round to even
    x[5] = -127.0
    y = np.zeros(1, dtype=synth.Q8_DTYPE)
    o.lib.aqo_quantize_row_q8_0_x86(x, y.ctypes.data, 32)
    assert float(y["d"][0]) == 1.0
    assert y["qs"][0][:6].tolist() == [127, 0, 2, 2, 0, -127]
    # reference (weight-side) rounding is half away from zero
    o.lib.aqo_quantize_row_q8_0_ref(x, y.ctypes.data, 32)
    assert y["qs"][0][:6].tolist() == [127, 1, 2, 3, -1, -127]


def test_q8_dot_is_exact_int_dot_times_scales(o):
    """Integer block dots are exact (|sum| <= 32*127^2 < 2^24); with scales of
    1 the product equals the exact integer dot product."""
    a = synth.q8_0_random_codebook(4, 1, 1, 256)[0]
    b = synth.q8_0_random_codebook(4, 3, 1, 256)[0]
    a["d"] = 1.0
    b["d"] = 1.0
    exact = int((a["qs"].astype(np.int64) * b["qs"].astype(np.int64)).sum())
    assert o.lib.aqo_dot_q8_0(8, a.ctypes.data, b.ctypes.data) == float(exact)


def test_dot_orders_close_to_exact(o):
    """Both fp32 summation orders stay within the classical error bound of the
    exact dot product, and differ from each other (so the order matters)."""
    x = synth.normal(5, 1, (1024,))
    y = synth.normal(5, 2, (1024,))
    exact = float(np.dot(x.astype(np.float64), y.astype(np.float64)))
    bound = 1024 * 2 ** -24 * float(np.abs(x.astype(np.float64) * y).sum())
    v = o.lib.aqo_vec_dot_f32(1024, x, y)
    t = o.lib.aqo_tinyblas_dot_f32(1024, x, y)
    assert abs(v - exact) <= bound and abs(t - exact) <= bound
    diffs = sum(o.lib.aqo_vec_dot_f32(1024, synth.normal(s, 1, (1024,)), y) !=
                o.lib.aqo_tinyblas_dot_f32(1024, synth.normal(s, 1, (1024,)), y) for s in range(40))
    assert diffs > 0


def test_euclid_query_equal_codeword(o):
    """x = c_n is its own nearest codeword (distance 0 in exact math)."""
    cfg = synth.make_config(2, rows=8)
    cfg["Q"] = 1
    cb = cfg["codebook"][:1]
    picks = np.array([3, 100, 2047, 0, 512, 9, 77, 1500])
    cfg["x"] = cb[0][picks].copy()
    cfg["codebook"] = cb
    out = o.euclid_rvq(cfg)
    assert out["idx"][:, 0].tolist() == picks.tolist()
    assert np.abs(out["residual"]).max() == 0.0
    out2 = o.higgs_rvq(cfg)
    assert out2["idx"][:, 0].tolist() == picks.tolist()


def test_euclid_matches_f64_argmin_away_from_ties(o):
    cfg = synth.make_config(2, rows=64)
    cfg["Q"] = 1
    cfg["codebook"] = cfg["codebook"][:1]
    out = o.euclid_rvq(cfg)
    x = cfg["x"].astype(np.float64)
    c = cfg["codebook"][0].astype(np.float64)
    d = (x * x).sum(1)[:, None] + (c * c).sum(1)[None, :] - 2 * x @ c.T
    srt = np.sort(d, 1)
    gap = (srt[:, 1] - srt[:, 0]) / np.maximum(srt[:, 0], 1e-30)
    ok = gap > 1e-5
    assert (out["idx"][ok, 0] == d.argmin(1)[ok]).all()


def test_dac_one_hot_codebook(o):
    """Codebook rows +-e_i: the cosine argmax is the signed coordinate of the
    projection with the largest |value| (distinct values, no ties)."""
    D, N, T = 128, 16, 9
    w = synth.dac_weights(6, 1, D, N)
    cb = np.zeros((1, N, 8), np.float32)
    for n in range(N):
        cb[0, n, n % 8] = 1.0 if n < 8 else -1.0
    w["codebook"] = cb
    x = synth.normal(6, 1, (T, D))
    cfg = dict(kind="dac", B=1, T=T, D=D, Q=1, N=N, x=x, **w)
    out = o.dac_rvq(cfg)
    p = x.astype(np.float64) @ w["w_in"][0].astype(np.float64).T
    j = np.abs(p).argmax(1)
    want = np.where(p[np.arange(T), j] > 0, j, j + 8)
    assert out["idx"][:, 0].tolist() == want.tolist()


def test_gather_identity_and_range(o):
    cb = synth.normal(7, 1, (64, 256))
    idx = np.arange(64, dtype=np.int32)
    out = np.zeros((64, 256), np.float32)
    assert o.lib.aqo_gather_f32(cb, 64, 256, idx, 64, out) == 0
    assert _beq(out, cb)
    assert o.lib.aqo_gather_f32(cb, 64, 256, np.array([64], np.int32), 1, out) == -1


# ------------------------------------------------ direct-distance recipe --

def test_oracle_direct_matches_reference_vector_quantizer(o, ref):
    """engine::runtime::VectorQuantizer::compute, compiled from the reference
    sources, returns the nearest codewords; the restatement's codes gather
    the same rows bit for bit."""
    cfg = synth.make_config(2, rows=40)
    cb = cfg["codebook"][0]
    want = ref.vector_quantizer(cfg["x"], cb, batch=4)
    c = dict(x=cfg["x"], M=40, K=256, Q=1, N=cb.shape[0], codebook=cb[None])
    got = o.direct_rvq(c)
    assert _beq(cb[got["idx"][:, 0]], want)


def test_oracle_direct_first_index_on_ties(o, ref):
    cb = synth.normal(9, 2, (64, 32), 0.5)
    cb[1::2] = cb[0::2]
    x = cb[[4, 5, 10]].copy() + np.float32(0.0)
    c = dict(x=x, M=3, K=32, Q=1, N=64, codebook=cb[None])
    got = o.direct_rvq(c)
    assert got["idx"][:, 0].tolist() == [4, 4, 10]          # first of the equal minima
    assert _beq(ref.vector_quantizer(x, cb), cb[got["idx"][:, 0]])


def test_reference_vector_quantizer_size_check(ref):
    with pytest.raises(RuntimeError):
        ref.vector_quantizer(np.zeros((4, 8), np.float32), np.zeros((3, 7), np.float32))


def test_ema_codebook_closed_form(o):
    """codebook_embedding (qwen3_tts/tokenizer_speech_encoder.cpp:271-285):
    sum / std::max(usage, 1e-5).  Pinned by the format's special cases:
    usage 1 is the identity, usage below eps (0, negative, subnormal) divides
    by eps, a NaN usage stays NaN (std::max keeps its first argument when the
    comparison is false), and otherwise out * usage recovers sum to within
    one rounding of each operation."""
    rng = np.random.default_rng(5)
    Q, N, K = 2, 16, 8
    es = rng.standard_normal((Q, N, K)).astype(np.float32)
    cu = rng.uniform(0.5, 100.0, (Q, N)).astype(np.float32)
    cu[0, 0] = 1.0
    cu[0, 1] = 0.0
    cu[0, 2] = -3.0
    cu[0, 3] = 1e-40
    cu[0, 4] = np.nan
    cu[0, 5] = 1e-5
    cu[0, 6] = np.inf
    out = o.ema_codebook(es, cu, 1e-5)
    assert np.array_equal(out[0, 0], es[0, 0])
    eps = np.float32(1e-5)
    for n in (1, 2, 3, 5):
        assert np.array_equal(out[0, n], es[0, n] / eps)
    assert np.isnan(out[0, 4]).all()
    assert np.array_equal(out[0, 6], es[0, 6] / np.float32(np.inf))
    rest = np.ones((Q, N), bool)
    rest[0, :7] = False
    back = (out * cu[:, :, None]).astype(np.float64)
    err = np.abs(back - es) / np.maximum(np.abs(es), 1e-30)
    assert (err[rest] <= 2.5 * 2.0 ** -24).all()


# ------------------------------------------------- host-loop DAC quantizers --

@pytest.mark.parametrize("M,near_dup", [(1, False), (300, False), (2000, True)])
def test_oracle_outetts_bit_exact_vs_reference(o, ref, M, near_dup):
    cfg = synth.outetts_config(M)
    if near_dup:
        cfg["codebook"] = synth.near_duplicate_pairs(cfg["codebook"], 7)
    assert np.array_equal(o.outetts_rvq(cfg)["idx"], ref.outetts_rvq(cfg))


def test_outetts_pin_detects_fused_multiply_add(ref, tmp_path):
    """The near-duplicate comparison is not vacuous: the same restatement
    built with contraction (FMA) disagrees with the reference."""
    import shutil
    import subprocess
    from oracle import HERE
    if not shutil.which("gcc") or " fma " not in open("/proc/cpuinfo").read():
        pytest.skip("needs gcc and an FMA-capable host")
    so = tmp_path / "liboracle_fma.so"
    subprocess.run(["gcc", "-O2", "-fPIC", "-ffp-contract=fast", "-mfma", "-std=c11", "-shared", "-o", str(so),
                    str(HERE / "aq_oracle.c"), "-lm"], check=True)
    cfg = synth.outetts_config(2000)
    cfg["codebook"] = synth.near_duplicate_pairs(cfg["codebook"], 7)
    wrong = Oracle(so).outetts_rvq(cfg)["idx"]
    assert (wrong != ref.outetts_rvq(cfg)).sum() > 10


@pytest.mark.parametrize("M", [1, 37])
def test_oracle_moss_bit_exact_vs_reference(o, ref, M):
    cfg = synth.moss_config(M, Q=4, N=256)
    out = o.moss_rvq(cfg)
    assert np.array_equal(out["idx"], ref.moss_encode(cfg))
    assert _beq(o.moss_decode(cfg, out["idx"]), ref.moss_decode(cfg, out["idx"]))


def test_oracle_moss_full_shape_vs_reference(o, ref):
    """The MOSS-Audio-Tokenizer-v2 shape: 768 -> 512, 12 x 1024 x 8."""
    cfg = synth.moss_config(24)
    out = o.moss_rvq(cfg)
    assert np.array_equal(out["idx"], ref.moss_encode(cfg))
    assert _beq(o.moss_decode(cfg, out["idx"]), ref.moss_decode(cfg, out["idx"]))


def test_oracle_moss_zero_projection_takes_first_code(o, ref):
    """A stage whose in-projection is zero (g = 0, zero bias): the encoding is
    0 / max(0, 1e-12) = 0, every dot is 0 and the first code wins."""
    cfg = synth.moss_config(9, Q=3, N=128)
    cfg["in_g"][1] = 0.0
    cfg["in_b"][1] = 0.0
    out = o.moss_rvq(cfg)
    assert (out["idx"][:, 1] == 0).all()
    assert np.array_equal(out["idx"], ref.moss_encode(cfg))


def test_oracle_moss_weight_norm_closed_form(o):
    """w = g v / |v| row-wise: rows of w have norm g (to fp32 rounding)."""
    g = synth.uniform(3, 1, (16,), 0.5, 2.0)
    v = synth.normal(3, 2, (16, 40))
    w = o.moss_weight_norm(g, v)
    np.testing.assert_allclose(np.linalg.norm(w.astype(np.float64), axis=1), g, rtol=1e-6)
    assert (np.sign(w) == np.sign(v)).all()


@pytest.mark.parametrize("shape", [(8, 1024, 1), (1024, 8, 1), (64, 32, 7), (3, 5, 3)])
def test_oracle_outetts_weight_norm_matches_reference(o, ref, shape):
    """fold_weight_norm (outetts/dac.cpp:91-110) from the reference's own
    source, bit for bit, on conv shapes [out, in, kernel] (the quantizer's
    1x1 in / out projections and wider kernels), including a zero-magnitude
    row and a row whose v is tiny."""
    v = synth.normal(17, shape[0], shape, 1.0)
    v[min(1, shape[0] - 1)] *= 1e-30
    g = synth.uniform(17, 99, (shape[0],), 0.1, 3.0)
    g[0] = 0.0
    assert np.array_equal(o.outetts_weight_norm(v, g).view(np.uint32), ref.outetts_fold(v, g).view(np.uint32))


def test_oracle_outetts_weight_norm_closed_form(o):
    """w = g v / |v| row-wise: rows of w have norm g (to fp32 rounding), and
    the result does not depend on v's scale (up to rounding)."""
    g = synth.uniform(18, 1, (16,), 0.5, 2.0)
    v = synth.normal(18, 2, (16, 40))
    w = o.outetts_weight_norm(v, g)
    np.testing.assert_allclose(np.linalg.norm(w.astype(np.float64), axis=1), g, rtol=1e-6)
    np.testing.assert_allclose(o.outetts_weight_norm(v * 8.0, g), w, rtol=1e-6)


@pytest.mark.parametrize("n_out,k,M,q8,bias", [(64, 1024, 1, False, True), (64, 1024, 2, False, True),
                                                (128, 512, 37, False, False), (1024, 64, 5, False, True),
                                                (64, 1024, 1, True, True), (256, 512, 33, True, False)])
def test_oracle_linear_matches_reference(o, ref, n_out, k, M, q8, bias):
    """LinearModule (mul_mat + add) against the reference's ggml graph, bit
    for bit: F32 weights with one frame (ggml_vec_dot_f32) and batches
    (tinyBLAS), and Q8_0 weights (x quantised, int8 block dots)."""
    from aqmi import synth as sy

    w = sy.normal(19, n_out + k, (n_out, k), 0.05)
    if q8:
        w = sy.q8_0_quantize_ref(w)
    x = sy.normal(19, M, (M, k), 1.0)
    b = sy.normal(19, 3, (n_out,), 0.1) if bias else None
    assert np.array_equal(o.linear(w, b, x).view(np.uint32), ref.linear(w, b, x).view(np.uint32))


def test_oracle_moss_decode_range(o, ref):
    cfg = synth.moss_config(2, Q=2, N=64)
    bad = np.array([[0, 64], [1, 2]], np.int32)
    with pytest.raises(IndexError):
        o.moss_decode(cfg, bad)
    with pytest.raises(IndexError):
        ref.moss_decode(cfg, bad)


def test_oracle_outetts_matches_golden(o):
    g = np.load(GOLDEN / "outetts_neardup.npz")
    cfg = synth.outetts_config(3001)
    cfg["codebook"] = synth.near_duplicate_pairs(cfg["codebook"], 7)
    assert np.array_equal(o.outetts_rvq(cfg)["idx"], g["idx"].astype(np.int32))


def test_oracle_moss_matches_golden(o):
    g = np.load(GOLDEN / "moss_v2.npz")
    cfg = synth.moss_config(256)
    out = o.moss_rvq(cfg)
    assert np.array_equal(out["idx"], g["idx"].astype(np.int32))
    assert _sha(o.moss_decode(cfg, out["idx"])) == str(g["latent_sha"])


def test_synth_moss_fold_is_the_reference_fold(o):
    """bench.py folds the MOSS weights with numpy (aqmi.synth.moss_fold); the
    bits must be the reference's reconstruct_weight_norm (via the oracle)."""
    cfg = synth.moss_config(1, Q=3, N=64)
    a, b = synth.moss_fold(cfg), o.moss_fold(cfg)
    for k in a:
        assert _beq(a[k], b[k]), k


# ------------------------------------------- projected cascades (OmniVoice / Higgs) --

@pytest.mark.parametrize("recipe,cb_q8,proj_q8,M,topk", [
    (0, False, False, 37, 0), (0, False, True, 21, 0), (1, False, False, 30, 0), (1, True, True, 25, 4),
    (1, False, True, 9, 0), (1, True, False, 12, 2), (0, False, False, 1, 0), (1, True, True, 1, 0),
    (1, False, False, 1, 3)])
def test_oracle_projected_bit_exact_vs_ggml(o, ref, recipe, cb_q8, proj_q8, M, topk):
    """project_in -> score -> argmax (top_k) -> lookup -> project_out -> sub
    per stage, against the reference's op graph on ggml (M = 1 takes
    ggml_vec_dot_f32 for the F32 products, M >= 2 tinyBLAS)."""
    cfg = synth.projected_config(M, recipe=recipe, cb_q8=cb_q8, proj_q8=proj_q8, Q=3)
    a = o.projected_rvq(cfg, topk=topk)
    b = ref.projected_rvq(cfg, topk=topk)
    assert np.array_equal(a["idx"], b["idx"])
    assert _beq(a["residual"], b["residual"])
    assert _beq(a["dist"], b["dist"])
    if topk:
        assert np.array_equal(a["topk_idx"], b["topk_idx"])
        assert _beq(a["topk_logit"], b["topk_logit"])


@pytest.mark.parametrize("cb_q8,proj_q8,M", [(False, False, 40), (True, True, 33), (False, True, 1)])
def test_oracle_projected_decode_vs_ggml(o, ref, cb_q8, proj_q8, M):
    cfg = synth.projected_config(M, recipe=1, cb_q8=cb_q8, proj_q8=proj_q8, Q=4)
    idx = o.projected_rvq(cfg)["idx"]
    assert _beq(o.projected_decode(cfg, idx), ref.projected_decode(cfg, idx))
    bad = idx.copy()
    bad[0, 2] = cfg["N"]
    with pytest.raises(IndexError):
        o.projected_decode(cfg, bad)


@pytest.mark.parametrize("recipe", [0, 1])
def test_projected_with_selector_weights_is_the_plain_cascade(o, recipe):
    """project_in = [I_K 0] and project_out = its transpose, no biases: the
    projection picks the first K hidden channels exactly, so the projected
    cascade must give the plain cascade's codes on those channels, their
    residual, and leave the other channels untouched.  A transposed weight,
    a sub in codebook space or a dropped stage fails this."""
    H, K, N, Q, M = 256, 64, 256, 3, 50
    cfg = synth.projected_config(M, recipe=recipe, H=H, K=K, N=N, Q=Q)
    sel = np.zeros((Q, K, H), np.float32)
    sel[:, np.arange(K), np.arange(K)] = 1.0
    cfg.update(w_in=sel, w_out=np.ascontiguousarray(sel.transpose(0, 2, 1)), b_in=None, b_out=None)
    out = o.projected_rvq(cfg)
    plain = dict(x=np.ascontiguousarray(cfg["x"][:, :K]), M=M, K=K, Q=Q, N=N, codebook=cfg["codebook"])
    want = o.euclid_rvq(plain) if recipe == 0 else o.higgs_rvq(plain)
    assert np.array_equal(out["idx"], want["idx"])
    assert np.array_equal(out["residual"][:, :K], want["residual"])
    assert _beq(out["residual"][:, K:], cfg["x"][:, K:])


def test_synth_q8_weight_rounding_matches_ggml(ref):
    """synth.q8_0_quantize_ref is the reference weight store's rounding
    (ggml_quantize_chunk -> quantize_row_q8_0_ref)."""
    w = synth.normal(5, 9, (16, 256), 0.3)
    w[0, :32] = np.arange(32) - 15.5          # half-way values after scaling
    w[1, :32] = 0.0                           # amax = 0 block
    got = synth.q8_0_quantize_ref(w)
    want = np.zeros((16, 8), dtype=synth.Q8_DTYPE)
    ref.lib.aqref_quantize_chunk_q8_0(np.ascontiguousarray(w, np.float32), want.ctypes.data_as(__import__("ctypes").c_void_p), 16, 256)
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8))


@pytest.mark.parametrize("tag,kw,topk", [
    ("higgs_f32", dict(recipe=1), 0), ("higgs_q8", dict(recipe=1, cb_q8=True, proj_q8=True), 4),
    ("omnivoice_f32", dict(recipe=0), 0), ("omnivoice_q8proj", dict(recipe=0, proj_q8=True), 0)])
def test_oracle_projected_matches_golden(o, tag, kw, topk):
    """The projected cascades at the reference's shapes (1024 -> 64, 8 x 1024
    codes, 400 frames) against fixtures the reference's graphs wrote."""
    g = np.load(GOLDEN / f"projected_{tag}.npz")
    cfg = synth.projected_config(400, **kw)
    out = o.projected_rvq(cfg, topk=topk)
    assert np.array_equal(out["idx"], g["idx"].astype(np.int32))
    assert _sha(out["residual"]) == str(g["residual_sha"])
    assert _sha(out["dist"]) == str(g["dist_sha"])
    if topk:
        ti, tl = _sorted_topk(out["topk_idx"], out["topk_logit"])
        assert _sha(ti.astype(np.int32)) == str(g["topk_idx_sha"])
        assert _sha(tl) == str(g["topk_logit_sha"])
    assert _sha(o.projected_decode(cfg, out["idx"])) == str(g["decode_sha"])


def test_oracle_qwen3_cascade_matches_golden(o):
    """Qwen3's 1 + 15 stage DIRECT cascade over EMA codebooks, read
    channel-major, against the reference's own quantize_projected."""
    g = np.load(GOLDEN / "qwen3_cascade.npz")
    cfg = synth.qwen3_config(g["idx"].shape[0])
    assert np.array_equal(o.qwen3_quantize(cfg), g["idx"].astype(np.int32))


def test_oracle_qwen3_vs_reference_function(o, ref):
    cfg = synth.qwen3_config(25, seed=21)
    assert np.array_equal(o.qwen3_quantize(cfg), ref.qwen3_quantize(cfg))


def test_oracle_fish_mixed_cascade_vs_ggml_and_golden(o, ref):
    """Fish's semantic 4096-code stage before 1024-code residual stages."""
    cfg = synth.fish_config(2, 100, Qr=3)
    a, b = o.dac_rvq_mixed(cfg), ref.dac_rvq_mixed(cfg)
    assert np.array_equal(a["idx"], b["idx"])
    assert _beq(a["residual"], b["residual"]) and _beq(a["recon"], b["recon"])


def test_oracle_fish_mixed_matches_golden(o):
    g = np.load(GOLDEN / "fish_mixed.npz")
    out = o.dac_rvq_mixed(synth.fish_config(4, 250))
    assert np.array_equal(out["idx"], g["idx"].astype(np.int32))
    assert _sha(out["residual"]) == str(g["residual_sha"])
    assert _sha(out["recon"]) == str(g["recon_sha"])
