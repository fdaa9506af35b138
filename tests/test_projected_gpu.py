"""GPU parity of the projected cascades (OmniVoice / Higgs with per-stage
project_in / project_out, aq_euclid_upload_projected) and of strided
(channel-major) input, through the C ABI.

Codes, the hidden-space residual, the reported logits, top-k sets and the
decode are compared bit for bit with the oracle (pinned to the reference's
own op graphs on ggml in test_oracle.py) and with fixtures those graphs
wrote; the Qwen3 cascade with the fixture written by the reference's own
quantize_projected.
"""

import hashlib

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


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def upload(ctx, cfg):
    import aqmi

    cbt = aqmi.CB_Q8_0 if "codebook_q8" in cfg else aqmi.CB_F32
    pt = aqmi.CB_Q8_0 if "w_in_q8" in cfg else aqmi.CB_F32
    cb = cfg["codebook_q8"] if cbt else cfg["codebook"]
    wi = cfg["w_in_q8"] if pt else cfg["w_in"]
    wo = cfg["w_out_q8"] if pt else cfg["w_out"]
    return aqmi.Codebooks.projected(ctx, cb, wi, cfg.get("b_in"), wo, cfg.get("b_out"), cfg["recipe"], cbt, pt)


def run(torch, ctx, cfg, topk=0, force=None, x=None, strided=None):
    cbs = upload(ctx, cfg)
    M, Q, H = cfg["M"], cfg["Q"], cfg["H"]
    xd = torch.from_numpy(np.ascontiguousarray(cfg["x"] if x is None else x, np.float32)).cuda()
    idx = torch.full((M, Q), -1, dtype=torch.int32, device="cuda")
    res = torch.empty((M, H), dtype=torch.float32, device="cuda")
    dist = torch.empty((M, Q), dtype=torch.float32, device="cuda")
    tki = torch.empty((M, Q, max(topk, 1)), dtype=torch.int32, device="cuda")
    tkd = torch.empty((M, Q, max(topk, 1)), dtype=torch.float32, device="cuda")
    fi = None if force is None else torch.from_numpy(np.ascontiguousarray(force, np.int32)).cuda()
    if strided is None:
        cbs.encode(xd, idx, res, dist, topk, tki if topk else None, tkd if topk else None, fi)
    else:
        cbs.encode_strided(xd, M, *strided, idx, res, dist, topk, tki if topk else None, tkd if topk else None, fi)
    torch.cuda.synchronize()
    out = dict(idx=idx.cpu().numpy(), residual=res.cpu().numpy(), dist=dist.cpu().numpy(), cbs=cbs)
    if topk:
        out["topk_idx"] = tki.cpu().numpy()
        out["topk_dist"] = tkd.cpu().numpy()
    return out


def sorted_topk(idx, logit):
    order = np.lexsort((idx, -logit.astype(np.float64)), axis=-1)
    return np.take_along_axis(idx, order, -1), np.take_along_axis(logit, order, -1)


def check(out, ref, topk=0):
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))
    assert np.array_equal(bits(out["dist"]), bits(ref["dist"]))
    if topk:
        gi, gl = sorted_topk(out["topk_idx"], -out["topk_dist"])
        ri, rl = sorted_topk(ref["topk_idx"], ref["topk_logit"])
        assert np.array_equal(gi, ri)
        assert np.array_equal(bits(gl), bits(rl))


CASES = [
    ("higgs_f32", dict(recipe=1), 0),
    ("higgs_q8", dict(recipe=1, cb_q8=True, proj_q8=True), 4),
    ("omnivoice_f32", dict(recipe=0), 0),
    ("omnivoice_q8proj", dict(recipe=0, proj_q8=True), 0),
]


@pytest.mark.parametrize("tag,kw,topk", CASES)
def test_projected_matches_golden(torch, ctx, tag, kw, topk):
    """8 stages, hidden 1024 -> 64, 1024 codes, 400 frames: codes, residual,
    logits, top-4 and decode against the reference graphs' fixtures."""
    from aqmi import synth

    print(f"[gpu] projected golden {tag}", flush=True)
    g = np.load(GOLDEN / f"projected_{tag}.npz")
    cfg = synth.projected_config(400, **kw)
    out = run(torch, ctx, cfg, topk=topk)
    assert np.array_equal(out["idx"], g["idx"].astype(np.int32))
    assert sha(out["residual"]) == str(g["residual_sha"])
    assert sha(out["dist"]) == str(g["dist_sha"])
    if topk:
        ti, tl = sorted_topk(out["topk_idx"], -out["topk_dist"])
        assert sha(ti.astype(np.int32)) == str(g["topk_idx_sha"])
        assert sha(tl) == str(g["topk_logit_sha"])
    dec = torch.empty((400, cfg["H"]), dtype=torch.float32, device="cuda")
    out["cbs"].decode(torch.from_numpy(out["idx"]).cuda(), dec)
    torch.cuda.synchronize()
    assert sha(dec.cpu().numpy()) == str(g["decode_sha"])


@pytest.mark.parametrize("kw,M,topk", [
    (dict(recipe=1), 1, 0), (dict(recipe=0), 1, 0), (dict(recipe=1, cb_q8=True, proj_q8=True), 1, 2),
    (dict(recipe=1, proj_q8=True), 37, 0), (dict(recipe=1, cb_q8=True), 50, 3),
    (dict(recipe=0, H=512, K=256, N=512, Q=3), 77, 0), (dict(recipe=1, H=768, K=64, N=256, Q=2), 2, 1)])
def test_projected_matches_oracle(torch, ctx, oracle, kw, M, topk):
    """Other weight types, one frame (ggml_vec_dot_f32 order), other widths
    and ragged M against the oracle."""
    from aqmi import synth

    print(f"[gpu] projected oracle {kw} M={M} topk={topk}", flush=True)
    kw = dict(kw)
    kw.setdefault("Q", 3)
    cfg = synth.projected_config(M, **kw)
    out = run(torch, ctx, cfg, topk=topk)
    check(out, oracle.projected_rvq(cfg, topk=topk), topk)
    dec = torch.empty((M, cfg["H"]), dtype=torch.float32, device="cuda")
    out["cbs"].decode(torch.from_numpy(out["idx"]).cuda(), dec)
    torch.cuda.synchronize()
    assert np.array_equal(bits(dec.cpu().numpy()), bits(oracle.projected_decode(cfg, out["idx"])))


@pytest.mark.parametrize("proj_q8", [False, True])
def test_projected_teacher_forced(torch, ctx, oracle, proj_q8):
    from aqmi import synth

    print(f"[gpu] projected teacher forcing proj_q8={proj_q8}", flush=True)
    cfg = synth.projected_config(90, recipe=1, proj_q8=proj_q8, Q=4)
    force = np.random.default_rng(5).integers(0, cfg["N"], size=(90, 4), dtype=np.int32)
    out = run(torch, ctx, cfg, force=force)
    check(out, oracle.projected_rvq(cfg, force_idx=force))


def test_projected_channel_major_input(torch, ctx, oracle):
    """The encoder's [B, C, T] latent read in place (3 clips of 70 frames)."""
    from aqmi import synth

    print("[gpu] projected channel-major", flush=True)
    B, T = 3, 70
    cfg = synth.projected_config(B * T, recipe=0, Q=3)
    H = cfg["H"]
    bct = np.ascontiguousarray(cfg["x"].reshape(B, T, H).transpose(0, 2, 1))
    out = run(torch, ctx, cfg, x=bct, strided=(T, H * T, 1, T))
    check(out, oracle.projected_rvq(cfg))


def test_projected_errors(torch, ctx):
    import aqmi
    from aqmi import synth

    cfg = synth.projected_config(4, recipe=1, Q=2)
    with pytest.raises(aqmi.AqError) as e:
        aqmi.Codebooks.projected(ctx, cfg["codebook"], cfg["w_in"], cfg["b_in"], cfg["w_out"], cfg["b_out"],
                                 aqmi.DIRECT)
    assert e.value.status == 5
    bad = synth.projected_config(4, recipe=1, Q=1, H=96)
    with pytest.raises(aqmi.AqError) as e:
        aqmi.Codebooks.projected(ctx, bad["codebook"], bad["w_in"], bad["b_in"], bad["w_out"], bad["b_out"], aqmi.HIGGS)
    assert e.value.status == 2
    force = np.array([[0, 0], [0, cfg["N"]], [0, 0], [0, 0]], np.int32)
    with pytest.raises(aqmi.AqError) as e:
        run(torch, ctx, cfg, force=force)
    assert e.value.status == 3


# ------------------------------------------------------------ strided input --

def test_qwen3_cascade_matches_reference_golden(torch, ctx):
    """Qwen3-TTS's speech tokenizer: EMA codebooks materialised on device, the
    semantic stage and the 15-stage acoustic cascade (DIRECT recipe, 2048 x
    256) read from the encoder's channel-major latents in place, against the
    codes of the reference's own quantize_projected."""
    import aqmi
    from aqmi import synth

    print("[gpu] qwen3 cascade", flush=True)
    g = np.load(GOLDEN / "qwen3_cascade.npz")
    F = g["idx"].shape[0]
    cfg = synth.qwen3_config(F)
    es, cu = cfg["embedding_sum"], cfg["cluster_usage"]
    sem = aqmi.Codebooks.from_ema(ctx, es[:1], cu[:1], aqmi.DIRECT)
    ac = aqmi.Codebooks.from_ema(ctx, es[1:], cu[1:], aqmi.DIRECT)
    K = cfg["K"]
    codes = torch.full((F, 16), -1, dtype=torch.int32, device="cuda")
    s_idx = torch.empty((F, 1), dtype=torch.int32, device="cuda")
    a_idx = torch.empty((F, 15), dtype=torch.int32, device="cuda")
    xs = torch.from_numpy(cfg["semantic"]).cuda()
    xa = torch.from_numpy(cfg["acoustic"]).cuda()
    sem.encode_strided(xs, F, F, K * F, 1, F, s_idx)
    ac.encode_strided(xa, F, F, K * F, 1, F, a_idx)
    codes[:, :1] = s_idx
    codes[:, 1:] = a_idx
    torch.cuda.synchronize()
    assert np.array_equal(codes.cpu().numpy(), g["idx"].astype(np.int32))


@pytest.mark.parametrize("recipe", [0, 1, 2])
def test_euclid_channel_major_matches_frame_major(torch, ctx, oracle, recipe):
    """[B, C, T] input (2 clips of 150 frames) gives the frame-major result."""
    import aqmi
    from aqmi import synth

    print(f"[gpu] euclid channel-major recipe={recipe}", flush=True)
    cfg = synth.make_config(2, rows=300)
    cfg["Q"] = 2
    cfg["codebook"] = np.ascontiguousarray(cfg["codebook"][:2])
    B, T, K = 2, 150, cfg["K"]
    bct = np.ascontiguousarray(cfg["x"].reshape(B, T, K).transpose(0, 2, 1))
    cbs = aqmi.Codebooks(ctx, cfg["codebook"], recipe)
    idx = torch.empty((300, 2), dtype=torch.int32, device="cuda")
    res = torch.empty((300, K), dtype=torch.float32, device="cuda")
    cbs.encode_strided(torch.from_numpy(bct).cuda(), 300, T, K * T, 1, T, idx, res)
    torch.cuda.synchronize()
    ref = {0: oracle.euclid_rvq, 1: oracle.higgs_rvq, 2: oracle.direct_rvq}[recipe](cfg)
    assert np.array_equal(idx.cpu().numpy(), ref["idx"])
    assert np.array_equal(bits(res.cpu().numpy()), bits(ref["residual"]))
