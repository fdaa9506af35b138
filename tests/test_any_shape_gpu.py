"""GPU parity at every shape the reference accepts (aq_euclid_* and aq_dac_*).

The reference's quantizers take any codebook width K, codebook size N and
latent width D (VectorQuantizer::compute, src/framework/runtime/
host_ops.cpp:236-273; ggml's mul_mat / conv graphs).  Shapes outside the
fast kernels' tiles go to the any-shape kernels: a run-time-width exact scan
for the Euclidean recipes and a run-time-D cascade for the DAC recipes.
Codes, residuals, distances, top-k sets and reconstructions are compared
bit for bit with the oracle, which tests/test_oracle_shapes.py pins against
the reference's ggml build at these shapes.
"""

import numpy as np
import pytest

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


def _dev(torch, a, dtype=None):
    return torch.from_numpy(np.ascontiguousarray(a if dtype is None else a.astype(dtype))).cuda()


def run_euclid(torch, ctx, cb_host, recipe, x, cb_type=0, topk=0, force=None):
    import aqmi

    cbs = aqmi.Codebooks(ctx, cb_host, recipe, cb_type)
    M = x.shape[0]
    xd = _dev(torch, x, np.float32)
    idx = torch.full((M, cbs.Q), -1, dtype=torch.int32, device="cuda")
    res = torch.empty((M, cbs.K), dtype=torch.float32, device="cuda")
    dist = torch.empty((M, cbs.Q), dtype=torch.float32, device="cuda")
    tki = torch.empty((M, cbs.Q, max(topk, 1)), dtype=torch.int32, device="cuda")
    tkd = torch.empty((M, cbs.Q, max(topk, 1)), dtype=torch.float32, device="cuda")
    fi = None if force is None else _dev(torch, force, np.int32)
    cbs.encode(xd, idx, res, dist, topk, tki if topk else None, tkd if topk else None, fi)
    torch.cuda.synchronize()
    out = dict(idx=idx.cpu().numpy(), residual=res.cpu().numpy(), dist=dist.cpu().numpy(), cbs=cbs,
               scans=cbs.exact_scans())
    if topk:
        out["topk_idx"] = tki.cpu().numpy()
        out["topk_dist"] = tkd.cpu().numpy()
    return out


def _sorted_topk(idx, val):
    o = np.lexsort((idx, -val), axis=-1)
    return np.take_along_axis(idx, o, -1), np.take_along_axis(val, o, -1)


def check_topk(out, ref):
    gi, gl = _sorted_topk(out["topk_idx"], -out["topk_dist"])
    ri, rl = _sorted_topk(ref["topk_idx"], ref["topk_logit"])
    assert np.array_equal(gi, ri)
    assert np.array_equal(bits(gl), bits(rl))


@pytest.mark.parametrize("K", [8, 100, 128, 1024])
@pytest.mark.parametrize("M", [1, 2, 300])
@pytest.mark.parametrize("recipe", [0, 1, 2])
def test_euclid_any_width_matches_oracle(torch, ctx, oracle, K, M, recipe):
    from aqmi import synth

    print(f"[gpu] any-width euclid K={K} M={M} recipe={recipe}", flush=True)
    N, Q = 1000, 2
    x = synth.normal(51, 1, (M, K))
    cb = synth.normal(51, 2, (Q, N, K), 0.25)
    cfg = dict(x=x, M=M, K=K, Q=Q, N=N, codebook=cb)
    out = run_euclid(torch, ctx, cb, recipe, x)
    if recipe == 0:
        ref = oracle.euclid_rvq(cfg)
        want_dist = -ref["logit"]
    elif recipe == 1:
        ref = oracle.higgs_rvq(cfg)
        want_dist = ref["dist"]
    else:
        ref = oracle.direct_rvq(cfg)
        want_dist = ref["dist"]
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))
    assert np.array_equal(bits(out["dist"]), bits(want_dist))
    assert out["scans"].tolist() == [M] * Q   # every frame decided by the exact scan


@pytest.mark.parametrize("K,N", [(256, 1000), (64, 100), (33, 5)])
def test_euclid_fast_width_odd_size_and_tiny(torch, ctx, oracle, K, N):
    """A fast width with a codebook size off the chunk grid, and tiny codebooks."""
    import aqmi
    from aqmi import synth

    print(f"[gpu] any-size euclid K={K} N={N}", flush=True)
    M, Q = 257, 3
    x = synth.normal(52, 1, (M, K))
    cb = synth.normal(52, 2, (Q, N, K), 0.25)
    cfg = dict(x=x, M=M, K=K, Q=Q, N=N, codebook=cb)
    out = run_euclid(torch, ctx, cb, aqmi.OMNIVOICE, x)
    ref = oracle.euclid_rvq(cfg)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))


@pytest.mark.parametrize("K", [100, 1024])
def test_euclid_any_width_topk(torch, ctx, oracle, K):
    import aqmi
    from aqmi import synth

    print(f"[gpu] any-width higgs top-4 K={K}", flush=True)
    M, N, Q = 200, 1000, 2
    x = synth.normal(53, 1, (M, K))
    cb = synth.normal(53, 2, (Q, N, K), 0.25)
    # exact duplicate codes, so ties meet the top-4 heap
    cb[:, 1::7] = cb[:, 0::7][:, : cb[:, 1::7].shape[1]]
    cfg = dict(x=x, M=M, K=K, Q=Q, N=N, codebook=cb)
    out = run_euclid(torch, ctx, cb, aqmi.HIGGS, x, topk=4)
    ref = oracle.higgs_rvq(cfg, topk=4)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))
    check_topk(out, ref)


@pytest.mark.parametrize("K", [128, 1024])
def test_euclid_any_width_q8_topk(torch, ctx, oracle, K):
    import aqmi
    from aqmi import synth

    print(f"[gpu] any-width higgs q8 top-4 K={K}", flush=True)
    M, N, Q = 150, 1000, 2
    cbq = synth.q8_0_random_codebook(54, 2, Q * N, K).reshape(Q, N, K // 32)
    x = synth.normal(54, 1, (M, K))
    cfg = dict(x=x, M=M, K=K, Q=Q, N=N, codebook_q8=cbq)
    out = run_euclid(torch, ctx, cbq, aqmi.HIGGS, x, cb_type=aqmi.CB_Q8_0, topk=4)
    ref = oracle.higgs_rvq(cfg, topk=4)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))
    assert np.array_equal(bits(out["dist"]), bits(ref["dist"]))
    check_topk(out, ref)


def test_euclid_any_width_teacher_forcing_and_strided(torch, ctx, oracle):
    import aqmi
    from aqmi import synth

    print("[gpu] any-width forced + channel-major", flush=True)
    K, N, Q, B, T = 100, 1000, 3, 3, 70
    M = B * T
    x = synth.normal(55, 1, (M, K))
    cb = synth.normal(55, 2, (Q, N, K), 0.25)
    force = (np.arange(M * Q).reshape(M, Q) * 37) % N
    cfg = dict(x=x, M=M, K=K, Q=Q, N=N, codebook=cb)
    out = run_euclid(torch, ctx, cb, aqmi.DIRECT, x, force=force)
    ref = oracle.direct_rvq(cfg, force_idx=force)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))
    # channel-major [B, K, T], read in place
    cm = np.ascontiguousarray(x.reshape(B, T, K).transpose(0, 2, 1))
    cbs = out["cbs"]
    idx = torch.full((M, Q), -1, dtype=torch.int32, device="cuda")
    res = torch.empty((M, K), dtype=torch.float32, device="cuda")
    cbs.encode_strided(_dev(torch, cm), M, T, K * T, 1, T, idx, res)
    torch.cuda.synchronize()
    ref2 = oracle.direct_rvq(cfg)
    assert np.array_equal(idx.cpu().numpy(), ref2["idx"])
    assert np.array_equal(bits(res.cpu().numpy()), bits(ref2["residual"]))


def test_euclid_any_width_rejects_partial_q8_blocks(torch, ctx):
    import aqmi

    cb = np.zeros((1, 16, 40), np.float32)
    with pytest.raises(aqmi.AqError) as e:
        aqmi.Codebooks(ctx, cb, aqmi.HIGGS, aqmi.CB_F32_AS_Q8_0)
    assert e.value.status == 2


# ------------------------------------------------------------------ DAC --

def run_dac(torch, ctx, cfg, recipe=0, force=None, clip_len=None):
    import aqmi

    st = aqmi.DacStages(ctx, cfg["w_in"], cfg.get("b_in"), cfg["codebook"], cfg["w_out"], cfg.get("b_out"), recipe)
    M = cfg["x"].shape[0]
    idx = torch.full((M, cfg["Q"]), -1, dtype=torch.int32, device="cuda")
    res = torch.empty((M, cfg["D"]), dtype=torch.float32, device="cuda")
    rec = torch.empty((M, cfg["D"]), dtype=torch.float32, device="cuda")
    fi = None if force is None else _dev(torch, force, np.int32)
    st.encode(_dev(torch, cfg["x"]), clip_len or cfg["T"], idx, res, rec, fi)
    torch.cuda.synchronize()
    return dict(idx=idx.cpu().numpy(), residual=res.cpu().numpy(), recon=rec.cpu().numpy(), stages=st)


@pytest.mark.parametrize("D,N,T", [(96, 1000, 8), (96, 1000, 5), (99, 1000, 8), (1536, 1000, 8), (1536, 1000, 6),
                                   (70, 7, 3), (1000, 64, 4), (2048, 300, 4), (1024, 1000, 75)])
@pytest.mark.parametrize("recipe", [0, 1, 2])
def test_dac_any_shape_matches_oracle(torch, ctx, oracle, D, N, T, recipe):
    from aqmi import synth

    print(f"[gpu] any-shape dac D={D} N={N} T={T} recipe={recipe}", flush=True)
    B, Q = 3, 3
    cfg = dict(kind="dac", B=B, T=T, D=D, Q=Q, N=N, x=synth.normal(56, 1, (B * T, D)),
               **synth.dac_weights(56, Q, D, N, bias=True))
    out = run_dac(torch, ctx, cfg, recipe)
    ref = oracle.dac_rvq(cfg, recipe=recipe)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))
    assert np.array_equal(bits(out["recon"]), bits(ref["recon"]))


def test_dac_any_shape_forced_decode_and_strided(torch, ctx, oracle):
    from aqmi import synth

    print("[gpu] any-shape dac forced + decode + channel-major", flush=True)
    B, T, D, N, Q = 2, 40, 1536, 1000, 4
    cfg = dict(kind="dac", B=B, T=T, D=D, Q=Q, N=N, x=synth.normal(57, 1, (B * T, D)),
               **synth.dac_weights(57, Q, D, N, bias=True))
    M = B * T
    force = (np.arange(M * Q).reshape(M, Q) * 13) % N
    out = run_dac(torch, ctx, cfg, force=force)
    ref = oracle.dac_rvq(cfg, force_idx=force)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))
    assert np.array_equal(bits(out["recon"]), bits(ref["recon"]))
    # decode of the forced codes is the teacher-forced recon
    st = out["stages"]
    rec = torch.empty((M, D), dtype=torch.float32, device="cuda")
    st.decode(_dev(torch, force, np.int32), rec)
    torch.cuda.synchronize()
    assert np.array_equal(bits(rec.cpu().numpy()), bits(ref["recon"]))
    # channel-major [B, D, T] in place
    cm = np.ascontiguousarray(cfg["x"].reshape(B, T, D).transpose(0, 2, 1))
    idx = torch.full((M, Q), -1, dtype=torch.int32, device="cuda")
    res = torch.empty((M, D), dtype=torch.float32, device="cuda")
    rc = torch.empty((M, D), dtype=torch.float32, device="cuda")
    st.encode_ex(_dev(torch, cm), M, T, (D * T, 1, T), idx.data_ptr(), Q, res, rc)
    torch.cuda.synchronize()
    ref2 = oracle.dac_rvq(cfg)
    assert np.array_equal(idx.cpu().numpy(), ref2["idx"])
    assert np.array_equal(bits(res.cpu().numpy()), bits(ref2["residual"]))
    assert np.array_equal(bits(rc.cpu().numpy()), bits(ref2["recon"]))
