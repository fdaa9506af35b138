"""GPU parity of the host-loop DAC quantizers (OuteTTS fp32, MOSS fp64)
through the C ABI.

The bar is bit-exactness against the oracle's restatement (itself pinned to
the reference's own sources in tests/test_oracle.py): codes, the final
residual (fp32 for OuteTTS, fp64 for MOSS) and the MOSS decode latent.  The
near-duplicate codebooks make every code depend on the last rounding of the
distance, so a fused multiply-add or a reordered sum shows up as a code
change, not only as a residual bit.
"""

import numpy as np
import pytest

from conftest import GOLDEN

pytestmark = pytest.mark.gpu


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


def _beq(a, b):
    a, b = np.asarray(a), np.asarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))


# ------------------------------------------------------------------ OuteTTS

def run_outetts(torch, ctx, cfg, force_idx=None):
    import aqmi

    st = aqmi.DacStages(ctx, cfg["w_in"], cfg.get("b_in"), cfg["codebook"], cfg["w_out"], cfg.get("b_out"),
                        recipe=aqmi.DAC_OUTETTS)
    x = torch.from_numpy(np.ascontiguousarray(cfg["x"])).cuda()
    M = x.shape[0]
    idx = torch.full((M, cfg["Q"]), -1, dtype=torch.int32, device="cuda")
    res = torch.empty((M, cfg["D"]), dtype=torch.float32, device="cuda")
    fi = None if force_idx is None else torch.from_numpy(np.ascontiguousarray(force_idx, np.int32)).cuda()
    st.encode(x, M, idx, res, None, fi)
    torch.cuda.synchronize()
    return dict(idx=idx.cpu().numpy(), residual=res.cpu().numpy(), stages=st)


@pytest.mark.parametrize("M,Q,near_dup", [(1, 2, False), (37, 2, False), (3001, 2, True), (200, 5, True)])
def test_outetts_matches_oracle(torch, ctx, oracle, M, Q, near_dup):
    from aqmi import synth

    cfg = synth.outetts_config(M, Q=Q)
    if near_dup:
        cfg["codebook"] = synth.near_duplicate_pairs(cfg["codebook"], 7)
    print(f"outetts M={M} Q={Q} near_dup={near_dup}", flush=True)
    got = run_outetts(torch, ctx, cfg)
    want = oracle.outetts_rvq(cfg)
    assert np.array_equal(got["idx"], want["idx"])
    assert _beq(got["residual"], want["residual"])


@pytest.mark.parametrize("D,N", [(64, 8), (512, 256), (2048, 64)])
def test_outetts_other_shapes(torch, ctx, oracle, D, N):
    from aqmi import synth

    cfg = synth.outetts_config(45, D=D, N=N, Q=3)
    got = run_outetts(torch, ctx, cfg)
    want = oracle.outetts_rvq(cfg)
    assert np.array_equal(got["idx"], want["idx"])
    assert _beq(got["residual"], want["residual"])


def test_outetts_teacher_forcing_and_edge_rows(torch, ctx, oracle):
    """Zero frames (|p| = 0: p / 1e-12), a NaN frame (every distance NaN: code
    0, as the strict < never fires) and an infinite one; forced codes."""
    from aqmi import synth

    cfg = synth.outetts_config(40)
    cfg["x"][3] = 0.0
    cfg["x"][4, 7] = np.nan
    cfg["x"][5, 9] = np.inf
    cfg["b_in"][:] = 0.0
    rng = np.random.default_rng(3)
    force = rng.integers(0, cfg["N"], (40, cfg["Q"])).astype(np.int32)
    for fi in (None, force):
        got = run_outetts(torch, ctx, cfg, fi)
        want = oracle.outetts_rvq(cfg, force_idx=fi)
        assert np.array_equal(got["idx"], want["idx"])
        assert _beq(got["residual"], want["residual"])
    assert (got["idx"][4] == 0).all()


def test_outetts_decode_is_the_conv_sum(torch, ctx, oracle):
    """aq_dac_decode on OuteTTS stages: sum over stages of the 1x1-conv
    out-projection of the codes, the Fish decode arithmetic (the same ggml
    graph ops), checked against the oracle's forced reconstruction."""
    from aqmi import synth

    cfg = synth.outetts_config(64)
    got = run_outetts(torch, ctx, cfg)
    out = torch.empty((64, cfg["D"]), dtype=torch.float32, device="cuda")
    got["stages"].decode(torch.from_numpy(got["idx"]).cuda(), out)
    torch.cuda.synchronize()
    fish = dict(cfg, B=1, T=64)
    want = oracle.dac_rvq(fish, force_idx=got["idx"])["recon"]
    assert _beq(out.cpu().numpy(), want)


def test_outetts_errors(torch, ctx):
    import aqmi
    from aqmi import synth

    cfg = synth.outetts_config(8, D=1024)
    st = aqmi.DacStages(ctx, cfg["w_in"], cfg["b_in"], cfg["codebook"], cfg["w_out"], cfg["b_out"],
                        recipe=aqmi.DAC_OUTETTS)
    x = torch.from_numpy(cfg["x"]).cuda()
    idx = torch.empty((8, 2), dtype=torch.int32, device="cuda")
    rec = torch.empty((8, 1024), dtype=torch.float32, device="cuda")
    with pytest.raises(aqmi.AqError, match="recon"):
        st.encode(x, 8, idx, None, rec)
    bad = np.full((8, 2), 1024, np.int32)
    with pytest.raises(aqmi.AqError, match="force_idx"):
        st.encode(x, 8, idx, None, None, torch.from_numpy(bad).cuda())
    with pytest.raises(aqmi.AqError, match="OuteTTS shape"):
        aqmi.DacStages(ctx, cfg["w_in"][:, :, :1000], cfg["b_in"], cfg["codebook"], cfg["w_out"][:, :1000],
                       cfg["b_out"][:, :1000], recipe=aqmi.DAC_OUTETTS)


# --------------------------------------------------------------------- MOSS

def moss_upload(ctx, oracle, cfg, decode=True):
    import aqmi

    f = oracle.moss_fold(cfg)
    return aqmi.MossQuantizer(ctx, f["w_ip"], cfg["ip_b"], f["w_in"], cfg["in_b"], cfg["codebook"], f["w_out"],
                              cfg["out_b"], f["w_op"] if decode else None, cfg["op_b"] if decode else None), f


def run_moss(torch, ctx, oracle, cfg, force_idx=None):
    q, f = moss_upload(ctx, oracle, cfg)
    h = torch.from_numpy(np.ascontiguousarray(cfg["hidden"])).cuda()
    M = h.shape[0]
    idx = torch.full((M, cfg["Q"]), -1, dtype=torch.int32, device="cuda")
    res = torch.empty((M, cfg["R"]), dtype=torch.float64, device="cuda")
    fi = None if force_idx is None else torch.from_numpy(np.ascontiguousarray(force_idx, np.int32)).cuda()
    q.encode(h, idx, res, fi)
    lat = torch.empty((M, cfg["C"]), dtype=torch.float32, device="cuda")
    q.decode(idx, lat)
    torch.cuda.synchronize()
    return dict(idx=idx.cpu().numpy(), residual=res.cpu().numpy(), latent=lat.cpu().numpy(), q=q, folded=f)


@pytest.mark.parametrize("M", [1, 19, 600])
def test_moss_matches_oracle(torch, ctx, oracle, M):
    from aqmi import synth

    cfg = synth.moss_config(M)
    print(f"moss M={M}", flush=True)
    got = run_moss(torch, ctx, oracle, cfg)
    want = oracle.moss_rvq(cfg, folded=got["folded"])
    assert np.array_equal(got["idx"], want["idx"])
    assert _beq(got["residual"], want["residual"])
    assert _beq(got["latent"], oracle.moss_decode(cfg, got["idx"], folded=got["folded"]))


def test_moss_other_shapes_and_forcing(torch, ctx, oracle):
    from aqmi import synth

    cfg = synth.moss_config(70, C=100, R=128, Q=3, N=72)
    force = np.random.default_rng(5).integers(0, 72, (70, 3)).astype(np.int32)
    for fi in (None, force):
        got = run_moss(torch, ctx, oracle, cfg, fi)
        want = oracle.moss_rvq(cfg, force_idx=fi, folded=got["folded"])
        assert np.array_equal(got["idx"], want["idx"])
        assert _beq(got["residual"], want["residual"])


def test_moss_zero_projection_and_nan(torch, ctx, oracle):
    """A zero in-projection stage (all dots 0: first code) and a NaN frame
    (every dot NaN: the strict > never fires, code 0)."""
    from aqmi import synth

    cfg = synth.moss_config(16, Q=3, N=128)
    cfg["in_g"][1] = 0.0
    cfg["in_b"][1] = 0.0
    cfg["hidden"][2, 5] = np.nan
    got = run_moss(torch, ctx, oracle, cfg)
    want = oracle.moss_rvq(cfg, folded=got["folded"])
    assert np.array_equal(got["idx"], want["idx"])
    assert _beq(got["residual"], want["residual"])
    assert (got["idx"][:, 1] == 0).all() and (got["idx"][2] == 0).all()


def test_moss_errors(torch, ctx, oracle):
    import aqmi
    from aqmi import synth

    cfg = synth.moss_config(4, Q=2, N=64, C=32, R=64)
    q, _ = moss_upload(ctx, oracle, cfg)
    h = torch.from_numpy(cfg["hidden"]).cuda()
    idx = torch.empty((4, 2), dtype=torch.int32, device="cuda")
    with pytest.raises(aqmi.AqError, match="non-empty encoder latent"):
        q.encode(h[:0], idx)
    with pytest.raises(aqmi.AqError, match="code index out of range"):
        q.decode(torch.full((4, 2), 64, dtype=torch.int32, device="cuda"), torch.empty((4, 32), device="cuda"))
    enc_only, _ = moss_upload(ctx, oracle, cfg, decode=False)
    with pytest.raises(aqmi.AqError, match="encode only"):
        enc_only.decode(idx, torch.empty((4, 32), device="cuda"))
    f = oracle.moss_fold(cfg)
    with pytest.raises(aqmi.AqError, match="unsupported shape"):
        aqmi.MossQuantizer(ctx, f["w_ip"][:48], cfg["ip_b"][:48], f["w_in"][:, :, :48], cfg["in_b"], cfg["codebook"],
                           f["w_out"][:, :48], cfg["out_b"][:, :48])


def test_outetts_golden(torch, ctx):
    """Codes the reference's quantize_reference wrote (tests/golden)."""
    from aqmi import synth

    g = np.load(GOLDEN / "outetts_neardup.npz")
    cfg = synth.outetts_config(3001)
    cfg["codebook"] = synth.near_duplicate_pairs(cfg["codebook"], 7)
    assert np.array_equal(run_outetts(torch, ctx, cfg)["idx"], g["idx"].astype(np.int32))


def test_moss_golden(torch, ctx, oracle):
    """Codes and decoded latent the reference's MossAudioTokenizerQuantizer
    wrote (tests/golden)."""
    import hashlib
    from aqmi import synth

    g = np.load(GOLDEN / "moss_v2.npz")
    got = run_moss(torch, ctx, oracle, synth.moss_config(256))
    assert np.array_equal(got["idx"], g["idx"].astype(np.int32))
    assert hashlib.sha256(np.ascontiguousarray(got["latent"]).tobytes()).hexdigest() == str(g["latent_sha"])
