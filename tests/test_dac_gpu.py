"""GPU parity of the DAC cosine RVQ path (aq_dac_* through the C ABI).

The bar is bit-exactness: the codes, the final residual and the
reconstruction must equal the oracle's (the reference's ggml CPU arithmetic)
bit for bit.  Full BASELINE sizes are checked against golden fixtures written
by the reference's own ggml build (tests/golden/make_golden.py); other shapes
against the plain-C oracle on the same seeded inputs.
"""

import hashlib

import numpy as np
import pytest

from conftest import GOLDEN

pytestmark = pytest.mark.gpu


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def torch():
    import torch as t

    if not t.cuda.is_available():
        pytest.skip("no GPU")
    return t


@pytest.fixture(scope="module")
def ctx(torch):
    import aqmi

    return aqmi.Context(0)


@pytest.fixture(scope="module")
def oracle():
    from oracle import Oracle

    return Oracle()


def run_gpu(torch, ctx, cfg, force_idx=None, clip_len=None):
    import aqmi

    st = aqmi.DacStages(ctx, cfg["w_in"], cfg.get("b_in"), cfg["codebook"], cfg["w_out"], cfg.get("b_out"))
    x = torch.from_numpy(np.ascontiguousarray(cfg["x"])).cuda()
    M = x.shape[0]
    idx = torch.full((M, cfg["Q"]), -1, dtype=torch.int32, device="cuda")
    res = torch.empty((M, cfg["D"]), dtype=torch.float32, device="cuda")
    rec = torch.empty((M, cfg["D"]), dtype=torch.float32, device="cuda")
    fi = None if force_idx is None else torch.from_numpy(np.ascontiguousarray(force_idx, np.int32)).cuda()
    st.encode(x, clip_len or cfg["T"], idx, res, rec, fi)
    torch.cuda.synchronize()
    out = dict(idx=idx.cpu().numpy(), residual=res.cpu().numpy(), recon=rec.cpu().numpy(), stages=st)
    return out


@pytest.mark.parametrize("name,cfg_id,bias", [("dac_cfg0.npz", 0, False), ("dac_cfg0_bias.npz", 0, True),
                                              ("dac_cfg1.npz", 1, False)])
def test_dac_matches_reference_fixture(torch, ctx, name, cfg_id, bias):
    from aqmi import synth

    print(f"[gpu] dac fixture {name}", flush=True)
    g = np.load(GOLDEN / name)
    cfg = synth.make_config(cfg_id)
    if bias:
        cfg.update(synth.dac_weights(cfg["seed"], cfg["Q"], cfg["D"], cfg["N"], bias=True))
    out = run_gpu(torch, ctx, cfg)
    assert np.array_equal(out["idx"], g["idx"].astype(np.int32)), "codes differ from the ggml reference"
    assert _sha(out["residual"]) == str(g["residual_sha"]), "residual not bit-identical"
    assert _sha(out["recon"]) == str(g["recon_sha"]), "reconstruction not bit-identical"


@pytest.mark.parametrize("D,N,Q,B,T", [(512, 1024, 4, 3, 250), (1024, 2048, 2, 2, 375), (256, 512, 3, 5, 33),
                                       (64, 64, 2, 1, 7)])
def test_dac_matches_oracle_shapes(torch, ctx, oracle, D, N, Q, B, T):
    from aqmi import synth

    print(f"[gpu] dac shape D={D} N={N} Q={Q} B={B} T={T}", flush=True)
    cfg = dict(kind="dac", B=B, T=T, D=D, Q=Q, N=N, x=synth.normal(11, 1, (B * T, D)),
               **synth.dac_weights(11, Q, D, N, bias=True))
    out = run_gpu(torch, ctx, cfg)
    ref = oracle.dac_rvq(cfg)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(out["residual"].view(np.uint32), ref["residual"].view(np.uint32))
    assert np.array_equal(out["recon"].view(np.uint32), ref["recon"].view(np.uint32))


def test_dac_teacher_forced(torch, ctx, oracle):
    """Stage-wise parity: force random codes into the residual update."""
    from aqmi import synth

    cfg = synth.make_config(1, rows=750)
    rng = np.random.default_rng(5)
    force = rng.integers(0, cfg["N"], size=(750, cfg["Q"]), dtype=np.int32)
    out = run_gpu(torch, ctx, cfg, force_idx=force)
    ref = oracle.dac_rvq(cfg, force_idx=force)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(out["residual"].view(np.uint32), ref["residual"].view(np.uint32))


def test_dac_decode_matches_encode_recon(torch, ctx, oracle):
    """Decode of the encode's codes equals its recon, and decode of arbitrary
    codes (teacher-forced, so independent of the encode) equals the oracle's
    out-projection sum for them."""
    from aqmi import synth

    cfg = synth.make_config(1, rows=1500)
    out = run_gpu(torch, ctx, cfg)
    st = out["stages"]
    idx = torch.from_numpy(out["idx"]).cuda()
    dec = torch.empty((1500, cfg["D"]), dtype=torch.float32, device="cuda")
    st.decode(idx, dec)
    torch.cuda.synchronize()
    assert np.array_equal(dec.cpu().numpy().view(np.uint32), out["recon"].view(np.uint32))
    rng = np.random.default_rng(17)
    cfg0 = synth.make_config(1, rows=750)
    force = rng.integers(0, cfg0["N"], size=(750, cfg0["Q"]), dtype=np.int32)
    want = oracle.dac_rvq(cfg0, force_idx=force)["recon"]
    dec2 = torch.empty((750, cfg0["D"]), dtype=torch.float32, device="cuda")
    st.decode(torch.from_numpy(force).cuda(), dec2)
    torch.cuda.synchronize()
    assert np.array_equal(dec2.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_dac_errors(torch, ctx):
    import aqmi
    from aqmi import synth

    cfg = synth.make_config(0)
    st = aqmi.DacStages(ctx, cfg["w_in"], cfg["b_in"], cfg["codebook"], cfg["w_out"], cfg["b_out"])
    x = torch.zeros((750, 1024), dtype=torch.float32, device="cuda")
    idx = torch.empty((750, 1), dtype=torch.int32, device="cuda")
    with pytest.raises(aqmi.AqError) as e:
        st.encode(x, 700, idx)                        # 750 is not a multiple of 700
    assert e.value.status == 2
    bad = torch.full((750, 1), 5000, dtype=torch.int32, device="cuda")
    with pytest.raises(aqmi.AqError) as e:
        st.encode(x, 750, idx, force_idx=bad)
    assert e.value.status == 3
    out = torch.empty((750, 1024), dtype=torch.float32, device="cuda")
    with pytest.raises(aqmi.AqError) as e:
        st.decode(bad, out)
    assert e.value.status == 3
    with pytest.raises(aqmi.AqError) as e:   # an empty codebook
        aqmi.DacStages(ctx, np.zeros((1, 8, 100), np.float32), None, np.zeros((1, 0, 8), np.float32),
                       np.zeros((1, 100, 8), np.float32), None)
    assert e.value.status == 2


def test_dac_zero_input_and_special_codebook(torch, ctx, oracle):
    """Zero frames (p = 0 -> pn = 0, all scores 0 -> last index wins) and a
    codebook of signed one-hots, where the code is fixed by the sign and
    position of the largest projected coordinate."""
    from aqmi import synth

    D, N, Q, T = 128, 64, 2, 5
    w = synth.dac_weights(3, Q, D, N)
    cb = np.zeros((Q, N, 8), np.float32)
    for n in range(16):
        cb[:, n, n % 8] = 1.0 if n < 8 else -1.0
    cb[:, 16:, :] = synth.normal(3, 77, (Q, N - 16, 8))
    w["codebook"] = cb
    x = synth.normal(3, 1, (2 * T, D))
    x[:T] = 0.0
    cfg = dict(kind="dac", B=2, T=T, D=D, Q=Q, N=N, x=x, **w)
    out = run_gpu(torch, ctx, cfg)
    ref = oracle.dac_rvq(cfg)
    assert np.array_equal(out["idx"], ref["idx"])
    assert (out["idx"][:T, 0] == N - 1).all()          # all-zero scores: ggml keeps the last index
    assert np.array_equal(out["residual"].view(np.uint32), ref["residual"].view(np.uint32))


def test_dac_near_duplicate_codes(torch, ctx, oracle):
    """Codebook rows in near-identical pairs (relative perturbations of 1e-7
    and exact duplicates): scores of a pair differ by a few ulps, so the
    approximate-score certificate fails and the exact ggml rescoring decides,
    including the last-index rule on exact ties."""
    from aqmi import synth

    D, N, Q, T = 256, 512, 3, 7
    w = synth.dac_weights(12, Q, D, N)
    cb = synth.normal(12, 90, (Q, N, 8))
    cb[:, 1::2] = cb[:, 0::2] * np.float32(1.0 + 1e-7)
    cb[:, 2:8:2] = cb[:, 3:9:2]                       # a few exact duplicates
    w["codebook"] = cb.astype(np.float32)
    x = synth.normal(12, 1, (6 * T, D))
    # frames equal to a projected codeword direction make the pair the winner
    cfg = dict(kind="dac", B=6, T=T, D=D, Q=Q, N=N, x=x, **w)
    out = run_gpu(torch, ctx, cfg)
    ref = oracle.dac_rvq(cfg)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(out["residual"].view(np.uint32), ref["residual"].view(np.uint32))


def test_dac_nonfinite_frames(torch, ctx, oracle):
    """NaN / Inf latents follow ggml's argmax on NaN scores (the running max
    restarts), replayed exactly; finite frames are unaffected."""
    from aqmi import synth

    D, N, Q, T = 128, 256, 2, 9
    w = synth.dac_weights(13, Q, D, N)
    x = synth.normal(13, 1, (T, D))
    x[1, 5] = np.nan
    x[4, :] = np.inf
    x[6, 0] = -np.inf
    cfg = dict(kind="dac", B=1, T=T, D=D, Q=Q, N=N, x=x, **w)
    out = run_gpu(torch, ctx, cfg)
    ref = oracle.dac_rvq(cfg)
    assert np.array_equal(out["idx"], ref["idx"])
    a, b = out["residual"], ref["residual"]
    assert np.array_equal(np.isnan(a), np.isnan(b))
    ok = ~np.isnan(a)
    assert np.array_equal(a[ok].view(np.uint32), b[ok].view(np.uint32))


@pytest.mark.parametrize("M", [1, 63, 750, 2000, 6000])
def test_dac_launch_shapes(torch, ctx, oracle, M):
    """Frame counts that select different frames-per-wave / block shapes,
    including partially filled waves."""
    from aqmi import synth

    print(f"[gpu] dac launch M={M}", flush=True)
    D, N, Q = 1024, 1024, 2
    x = synth.normal(14, 1, (M, D))
    cfg = dict(kind="dac", B=1, T=M, D=D, Q=Q, N=N, x=x, **synth.dac_weights(14, Q, D, N, bias=True))
    if M % 4 == 0:                       # one clip of M frames would select the tinyBLAS order
        cfg["T"] = M // 8 if (M // 8) % 4 else 1
        cfg["B"] = M // cfg["T"]
    out = run_gpu(torch, ctx, cfg)
    ref = oracle.dac_rvq(cfg)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(out["residual"].view(np.uint32), ref["residual"].view(np.uint32))
    assert np.array_equal(out["recon"].view(np.uint32), ref["recon"].view(np.uint32))


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("recipe", [1, 2])
def test_dac_recipes_match_oracle(torch, ctx, oracle, recipe):
    """IndexTTS2 (no eps; 1.0F / (float)|c| rows) and Vevo2 (1e-20; zero rows
    rejected) normalisation through the full residual cascade, bit for bit."""
    import aqmi
    from aqmi import synth

    print(f"[gpu] dac recipe {recipe}", flush=True)
    T, B, D, N, Q = 75, 2, 1024, 1024, 3
    cfg = dict(kind="dac", B=B, T=T, D=D, Q=Q, N=N, x=synth.normal(41, 1, (B * T, D)),
               **synth.dac_weights(41, Q, D, N, bias=True))
    st = aqmi.DacStages(ctx, cfg["w_in"], cfg["b_in"], cfg["codebook"], cfg["w_out"], cfg["b_out"], recipe)
    x = torch.from_numpy(cfg["x"]).cuda()
    idx = torch.full((B * T, Q), -1, dtype=torch.int32, device="cuda")
    res = torch.empty((B * T, D), dtype=torch.float32, device="cuda")
    rec = torch.empty((B * T, D), dtype=torch.float32, device="cuda")
    st.encode(x, T, idx, res, rec)
    torch.cuda.synchronize()
    ref = oracle.dac_rvq(cfg, recipe=recipe)
    assert np.array_equal(idx.cpu().numpy(), ref["idx"])
    assert np.array_equal(_bits(res.cpu().numpy()), _bits(ref["residual"]))
    assert np.array_equal(_bits(rec.cpu().numpy()), _bits(ref["recon"]))


@pytest.mark.parametrize("recipe", [0, 1, 2])
def test_dac_large_codebook_codes_only(torch, ctx, oracle, recipe):
    """IndexTTS2's semantic codec shape: one stage, D = 1024, N = 8192 (too
    large for LDS next to W_in: read from device memory), codes only (no
    out-projection), with a zero frame (IndexTTS2 divides by 0: NaN scores,
    ggml_argmax's NaN rule)."""
    import aqmi
    from aqmi import synth

    print(f"[gpu] dac large codebook recipe {recipe}", flush=True)
    T, B, D, N = 75, 2, 1024, 8192
    w = synth.dac_weights(42, 1, D, N, bias=True)
    x = synth.normal(42, 1, (B * T, D))
    x[3] = 0.0
    w["b_in"][:] = 0.0
    cfg = dict(kind="dac", B=B, T=T, D=D, Q=1, N=N, x=x, w_in=w["w_in"], b_in=w["b_in"], codebook=w["codebook"],
               w_out=None, b_out=None)
    st = aqmi.DacStages(ctx, w["w_in"], w["b_in"], w["codebook"], None, None, recipe)
    xd = torch.from_numpy(x).cuda()
    idx = torch.full((B * T, 1), -1, dtype=torch.int32, device="cuda")
    st.encode(xd, T, idx)
    torch.cuda.synchronize()
    ref = oracle.dac_rvq(cfg, recon=False, recipe=recipe)
    assert np.array_equal(idx.cpu().numpy(), ref["idx"])
    with pytest.raises(aqmi.AqError):
        st.encode(xd, T, idx, torch.empty((B * T, D), dtype=torch.float32, device="cuda"))


def test_dac_large_codebook_cascade(torch, ctx, oracle):
    """N = 4096 with two stages and the out-projection: codebook in device
    memory, residual and reconstruction bit for bit."""
    from aqmi import synth

    print("[gpu] dac large codebook cascade", flush=True)
    T, B, D, N, Q = 75, 2, 1024, 4096, 2
    cfg = dict(kind="dac", B=B, T=T, D=D, Q=Q, N=N, x=synth.normal(43, 1, (B * T, D)),
               **synth.dac_weights(43, Q, D, N, bias=True))
    out = run_gpu(torch, ctx, cfg)
    ref = oracle.dac_rvq(cfg)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(_bits(out["residual"]), _bits(ref["residual"]))
    assert np.array_equal(_bits(out["recon"]), _bits(ref["recon"]))


def test_dac_vevo2_rejects_zero_codebook_row(torch, ctx):
    import aqmi
    from aqmi import synth

    w = synth.dac_weights(44, 1, 64, 128, bias=False)
    w["codebook"][0, 7] = 0.0
    with pytest.raises(aqmi.AqError):
        aqmi.DacStages(ctx, w["w_in"], None, w["codebook"], None, None, aqmi.DAC_VEVO2)


@pytest.mark.parametrize("T,B,D", [(752, 2, 1024), (4, 3, 1024), (100, 2, 768), (8, 5, 64), (12, 4, 512)])
def test_dac_tinyblas_inprojection(torch, ctx, oracle, T, B, D):
    """Clip lengths that are a multiple of 4 make ggml compute the
    in-projection with tinyBLAS (16 FMA accumulators over k = 16 u + t, then
    _mm512_reduce_add_ps), the other summation order; codes, residual and
    reconstruction bit for bit, including widths whose swizzle is off
    (D = 768)."""
    from aqmi import synth

    print(f"[gpu] dac tinyblas T={T} B={B} D={D}", flush=True)
    N, Q = 1024, 3
    cfg = dict(kind="dac", B=B, T=T, D=D, Q=Q, N=N, x=synth.normal(45, 1, (B * T, D)),
               **synth.dac_weights(45, Q, D, N, bias=True))
    out = run_gpu(torch, ctx, cfg)
    ref = oracle.dac_rvq(cfg)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(_bits(out["residual"]), _bits(ref["residual"]))
    assert np.array_equal(_bits(out["recon"]), _bits(ref["recon"]))


def test_fish_mixed_cascade_chained_matches_golden(torch, ctx):
    """Fish's semantic quantizer (4096 codes) and its 8 residual quantizers
    (1024 codes) as two uploaded stage sets chained through aq_dac_encode_ex
    (codes written into one [M, 9] array, the residual handed on, the recon
    continued): codes, residual and recon equal the single cascade of the
    reference's graph recipe, and the chained decode equals the recon."""
    import aqmi
    from aqmi import synth

    print("[gpu] fish mixed-N cascade", flush=True)
    g = np.load(GOLDEN / "fish_mixed.npz")
    cfg = synth.fish_config(4, 250)
    M, D, T, Q = 1000, cfg["D"], cfg["T"], cfg["Q"]
    sem = aqmi.DacStages(ctx, cfg["w_in"][:1], cfg["b_in"][:1], cfg["codebook0"][None], cfg["w_out"][:1],
                         cfg["b_out"][:1])
    rest = aqmi.DacStages(ctx, cfg["w_in"][1:], cfg["b_in"][1:], cfg["codebook"], cfg["w_out"][1:], cfg["b_out"][1:])
    x = torch.from_numpy(cfg["x"]).cuda()
    idx = torch.full((M, Q), -1, dtype=torch.int32, device="cuda")
    r1 = torch.empty((M, D), dtype=torch.float32, device="cuda")
    res = torch.empty((M, D), dtype=torch.float32, device="cuda")
    rec = torch.empty((M, D), dtype=torch.float32, device="cuda")
    rows = (T * D, D, 1)
    sem.encode_ex(x, M, T, rows, idx.data_ptr(), Q, r1, rec, False)
    rest.encode_ex(r1, M, T, rows, idx.data_ptr() + 4, Q, res, rec, True)
    torch.cuda.synchronize()
    assert np.array_equal(idx.cpu().numpy(), g["idx"].astype(np.int32))
    assert _sha(res.cpu().numpy()) == str(g["residual_sha"])
    assert _sha(rec.cpu().numpy()) == str(g["recon_sha"])
    dec = torch.empty((M, D), dtype=torch.float32, device="cuda")
    sem.decode_ex(idx.data_ptr(), Q, M, dec, False)
    rest.decode_ex(idx.data_ptr() + 4, Q, M, dec, True)
    torch.cuda.synchronize()
    assert _sha(dec.cpu().numpy()) == str(g["recon_sha"])


@pytest.mark.parametrize("T", [75, 76])
def test_dac_channel_major_input(torch, ctx, oracle, T):
    """The encoder's [B, D, T] latent read in place: the same codes, residual
    and recon as the frame-major call (T = 76 takes tinyBLAS order)."""
    import aqmi
    from aqmi import synth

    print(f"[gpu] dac channel-major T={T}", flush=True)
    B, D, Q, N = 3, 1024, 3, 1024
    cfg = dict(B=B, T=T, D=D, Q=Q, N=N, x=synth.normal(71, 1, (B * T, D)), **synth.dac_weights(71, Q, D, N, bias=True))
    st = aqmi.DacStages(ctx, cfg["w_in"], cfg["b_in"], cfg["codebook"], cfg["w_out"], cfg["b_out"])
    bdt = np.ascontiguousarray(cfg["x"].reshape(B, T, D).transpose(0, 2, 1))
    M = B * T
    idx = torch.full((M, Q), -1, dtype=torch.int32, device="cuda")
    res = torch.empty((M, D), dtype=torch.float32, device="cuda")
    rec = torch.empty((M, D), dtype=torch.float32, device="cuda")
    st.encode_ex(torch.from_numpy(bdt).cuda(), M, T, (D * T, 1, T), idx.data_ptr(), Q, res, rec)
    torch.cuda.synchronize()
    ref = oracle.dac_rvq(cfg)
    assert np.array_equal(idx.cpu().numpy(), ref["idx"])
    assert np.array_equal(res.cpu().numpy().view(np.uint32), ref["residual"].view(np.uint32))
    assert np.array_equal(rec.cpu().numpy().view(np.uint32), ref["recon"].view(np.uint32))


def _ms_case(case, D, N, Q, B, T, bias):
    from aqmi import synth

    w = synth.dac_weights(61, Q, D, N, bias=bias)
    x = synth.normal(61, 1, (B * T, D))
    if case == "near_dup":                 # scores of a pair a few ulps apart: exact rescoring decides
        cb = synth.normal(62, 90, (Q, N, 8))
        cb[:, 1::2] = cb[:, 0::2] * np.float32(1.0 + 1e-7)
        cb[:, 2:8:2] = cb[:, 3:9:2]
        w["codebook"] = cb.astype(np.float32)
    elif case == "special":                # zero frames (all scores 0), one-hot codes, NaN / Inf frames
        cb = w["codebook"]
        for n in range(16):
            cb[:, n, :] = 0.0
            cb[:, n, n % 8] = 1.0 if n < 8 else -1.0
        x[:T] = 0.0
        x[T + 1, 5] = np.nan
        x[T + 4, :] = np.inf
    return dict(kind="dac", B=B, T=T, D=D, Q=Q, N=N, x=x, **w)


@pytest.mark.parametrize("case,D,N,Q,B,T,bias", [
    ("random", 1024, 1024, 3, 3, 75, True),       # vec_dot order, a partial last block
    ("random", 1024, 1024, 2, 2, 76, True),       # tinyBLAS order (T % 4 == 0)
    ("random", 512, 512, 3, 4, 33, False),
    ("random", 64, 128, 2, 2, 12, True),
    ("random", 768, 256, 2, 3, 50, True),
    ("random", 768, 384, 2, 3, 52, True),        # tinyBLAS order without the bank swizzle (D / 64 = 12)
    ("near_dup", 256, 512, 3, 6, 7, False),
    ("special", 128, 128, 2, 3, 9, True),
])
def test_dac_matrix_scores_match_oracle(torch, ctx, oracle, monkeypatch, capfd, case, D, N, Q, B, T, bias):
    """The matrix-core score kernel (split fp16 scores over a block's 24
    frames; AQ_DAC_MS=1 takes it whatever the launch shape) bit for bit
    against the oracle and against the per-wave score kernel (AQ_DAC_MS=0):
    codes, residual and reconstruction, in both in-projection orders,
    including near-tied codes, zero, NaN and Inf frames."""
    print(f"[gpu] dac matrix scores {case} D={D} N={N} Q={Q} B={B} T={T}", flush=True)
    cfg = _ms_case(case, D, N, Q, B, T, bias)
    monkeypatch.setenv("AQ_DEBUG", "1")
    monkeypatch.setenv("AQ_DAC_MS", "1")
    ms = run_gpu(torch, ctx, cfg)
    assert "aq_dac matrix scores" in capfd.readouterr().err
    monkeypatch.setenv("AQ_DAC_MS", "0")
    vw = run_gpu(torch, ctx, cfg)
    assert "aq_dac matrix scores" not in capfd.readouterr().err
    ref = oracle.dac_rvq(cfg)
    for out in (ms, vw):
        assert np.array_equal(out["idx"], ref["idx"])
        for k in ("residual", "recon"):
            a, b = out[k], ref[k]
            assert np.array_equal(np.isnan(a), np.isnan(b))
            ok = ~np.isnan(a)
            assert np.array_equal(_bits(a[ok]), _bits(b[ok])), k


def test_dac_matrix_scores_teacher_forced(torch, ctx, oracle, monkeypatch):
    """Teacher forcing on the matrix-core score kernel: forced codes drive the
    residual, the chosen codes are still reported, and a forced code out of
    range is an error."""
    import aqmi
    from aqmi import synth

    D, N, Q, B, T = 1024, 1024, 3, 2, 75
    cfg = dict(kind="dac", B=B, T=T, D=D, Q=Q, N=N, x=synth.normal(63, 1, (B * T, D)),
               **synth.dac_weights(63, Q, D, N, bias=True))
    forced = np.random.default_rng(63).integers(0, N, (B * T, Q)).astype(np.int32)
    monkeypatch.setenv("AQ_DAC_MS", "1")
    out = run_gpu(torch, ctx, cfg, force_idx=forced)
    ref = oracle.dac_rvq(cfg, force_idx=forced)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(_bits(out["residual"]), _bits(ref["residual"]))
    assert np.array_equal(_bits(out["recon"]), _bits(ref["recon"]))
    bad = forced.copy()
    bad[5, 1] = N
    with pytest.raises(aqmi.AqError):
        run_gpu(torch, ctx, cfg, force_idx=bad)


@pytest.mark.parametrize("recipe", [1, 2])
def test_dac_matrix_scores_recipes(torch, ctx, oracle, monkeypatch, recipe):
    """IndexTTS2 and Vevo2 normalisation on the matrix-core score kernel,
    through the cascade and as one codes-only stage (no out-projection, a
    zero frame: IndexTTS2's NaN query takes the exact rescoring)."""
    import aqmi
    from aqmi import synth

    print(f"[gpu] dac matrix scores recipe {recipe}", flush=True)
    monkeypatch.setenv("AQ_DAC_MS", "1")
    T, B, D, N, Q = 75, 2, 1024, 1024, 3
    cfg = dict(kind="dac", B=B, T=T, D=D, Q=Q, N=N, x=synth.normal(64, 1, (B * T, D)),
               **synth.dac_weights(64, Q, D, N, bias=True))
    st = aqmi.DacStages(ctx, cfg["w_in"], cfg["b_in"], cfg["codebook"], cfg["w_out"], cfg["b_out"], recipe)
    x = torch.from_numpy(cfg["x"]).cuda()
    idx = torch.full((B * T, Q), -1, dtype=torch.int32, device="cuda")
    res = torch.empty((B * T, D), dtype=torch.float32, device="cuda")
    rec = torch.empty((B * T, D), dtype=torch.float32, device="cuda")
    st.encode(x, T, idx, res, rec)
    torch.cuda.synchronize()
    ref = oracle.dac_rvq(cfg, recipe=recipe)
    assert np.array_equal(idx.cpu().numpy(), ref["idx"])
    assert np.array_equal(_bits(res.cpu().numpy()), _bits(ref["residual"]))
    assert np.array_equal(_bits(rec.cpu().numpy()), _bits(ref["recon"]))

    xz = cfg["x"].copy()
    xz[3] = 0.0
    b0 = np.zeros_like(cfg["b_in"][:1])
    one = dict(kind="dac", B=B, T=T, D=D, Q=1, N=N, x=xz, w_in=cfg["w_in"][:1], b_in=b0,
               codebook=cfg["codebook"][:1], w_out=None, b_out=None)
    st1 = aqmi.DacStages(ctx, one["w_in"], b0, one["codebook"], None, None, recipe)
    idx1 = torch.full((B * T, 1), -1, dtype=torch.int32, device="cuda")
    st1.encode(torch.from_numpy(xz).cuda(), T, idx1)
    torch.cuda.synchronize()
    ref1 = oracle.dac_rvq(one, recon=False, recipe=recipe)
    assert np.array_equal(idx1.cpu().numpy(), ref1["idx"])
