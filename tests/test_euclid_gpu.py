"""GPU parity of the Euclidean VQ / RVQ path (aq_euclid_* through the C ABI).

Every recipe is compared with the oracle on the same seeded inputs: codes
equal, the final residual and the reported distances bit-identical, top-k
sets and values identical.  The fp16 matrix-core scores only choose
candidates; the certificate plus the exact re-rank make the outputs the
reference arithmetic's, which these tests check at shapes the oracle
finishes in seconds (full BASELINE sizes are checked against golden
fixtures in test_golden_gpu.py).
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


@pytest.fixture(autouse=True, params=["resident", "cascade", "stages"])
def pipeline(request, monkeypatch):
    """Every test runs on each encode pipeline: the default (the one-launch
    cascade with the residual in registers for f32 codebooks at K = 256, the
    per-stage kernels otherwise), the one-launch cascade with the residual in
    memory (AQ_EUCLID_PIPELINE=cascade) and the per-stage kernels
    (AQ_EUCLID_PIPELINE=stages)."""
    if request.param == "resident":
        monkeypatch.delenv("AQ_EUCLID_PIPELINE", raising=False)
    else:
        monkeypatch.setenv("AQ_EUCLID_PIPELINE", request.param)
    return request.param


def effective(pipeline, K, cb_type=0):
    """The pipeline an encode takes under the `pipeline` fixture's setting."""
    return "stages" if pipeline == "resident" and K != 256 else pipeline


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


def run(torch, ctx, cb_host, recipe, x, cb_type=0, topk=0, force=None, want_dist=True):
    import aqmi

    cbs = aqmi.Codebooks(ctx, cb_host, recipe, cb_type)
    M = x.shape[0]
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    idx = torch.full((M, cbs.Q), -1, dtype=torch.int32, device="cuda")
    res = torch.empty((M, cbs.K), dtype=torch.float32, device="cuda")
    dist = torch.empty((M, cbs.Q), dtype=torch.float32, device="cuda") if want_dist else None
    tki = torch.empty((M, cbs.Q, max(topk, 1)), dtype=torch.int32, device="cuda")
    tkd = torch.empty((M, cbs.Q, max(topk, 1)), dtype=torch.float32, device="cuda")
    fi = None if force is None else torch.from_numpy(np.ascontiguousarray(force, np.int32)).cuda()
    cbs.encode(xd, idx, res, dist, topk, tki if topk else None, tkd if topk else None, fi)
    torch.cuda.synchronize()
    out = dict(idx=idx.cpu().numpy(), residual=res.cpu().numpy(), cbs=cbs, fails=cbs.failures())
    if want_dist:
        out["dist"] = dist.cpu().numpy()
    if topk:
        out["topk_idx"] = tki.cpu().numpy()
        out["topk_dist"] = tkd.cpu().numpy()
    return out


def mimi(rows, Q=3):
    from aqmi import synth

    cfg = synth.make_config(2, rows=rows)
    cfg["Q"] = Q
    cfg["codebook"] = np.ascontiguousarray(cfg["codebook"][:Q])
    return cfg


@pytest.mark.parametrize("M", [1, 17, 191, 193, 1000])
def test_omnivoice_matches_oracle(torch, ctx, oracle, M):
    import aqmi

    print(f"[gpu] omnivoice M={M}", flush=True)
    cfg = mimi(M)
    out = run(torch, ctx, cfg["codebook"], aqmi.OMNIVOICE, cfg["x"])
    ref = oracle.euclid_rvq(cfg)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))
    assert np.array_equal(bits(out["dist"]), bits(-ref["logit"]))


@pytest.mark.parametrize("K,N,M,Q", [(768, 1024, 300, 1), (64, 1024, 500, 2), (256, 2048, 400, 2)])
def test_higgs_f32_matches_oracle(torch, ctx, oracle, K, N, M, Q):
    import aqmi
    from aqmi import synth

    print(f"[gpu] higgs f32 K={K} N={N} M={M}", flush=True)
    cfg = synth.make_config(3, rows=M)
    cb = synth.normal(21, 3, (Q, N, K), 1.0)
    x = cfg["x"][:, :K].copy()
    c = dict(x=x, M=M, K=K, Q=Q, N=N, codebook=cb)
    out = run(torch, ctx, cb, aqmi.HIGGS, x)
    ref = oracle.higgs_rvq(c)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))
    assert np.array_equal(bits(out["dist"]), bits(ref["dist"]))


def test_higgs_q8_topk_matches_oracle(torch, ctx, oracle):
    import aqmi
    from aqmi import synth

    print("[gpu] higgs q8 topk", flush=True)
    cfg = synth.make_config(4, rows=300)
    cfg["Q"] = 2
    cfg["codebook_q8"] = np.ascontiguousarray(cfg["codebook_q8"][:2])
    out = run(torch, ctx, cfg["codebook_q8"], aqmi.HIGGS, cfg["x"], cb_type=aqmi.CB_Q8_0, topk=4)
    ref = oracle.higgs_rvq(cfg, topk=4)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))
    assert np.array_equal(bits(out["dist"]), bits(ref["dist"]))
    check_topk(out, ref)


def test_higgs_q8_query_blocks_with_special_values(torch, ctx, oracle):
    """The query's Q8_0 blocks: an all-zero block (amax 0), a block of values
    near 1e-38 (127 / amax overflows to inf: every quant -128, scale 0), a
    block holding +-inf and one holding a NaN, in frames otherwise near the
    codes, so that the certificate and the exact values meet each kind of
    block; codes, residuals, distances and top-4 against the oracle."""
    import aqmi
    from aqmi import synth

    print("[gpu] higgs q8 special query blocks", flush=True)
    Q, N, K, M = 2, 2048, 256, 320
    cb = np.stack([synth.q8_0_random_codebook(91, 10 + s, N, K) for s in range(Q)])
    x = (synth.q8_0_dequantize(cb[0])[np.arange(M) % N] + synth.normal(91, 2, (M, K), 0.05)).astype(np.float32)
    x[0::5, 32:64] = 0.0
    x[1::5, 64:96] = synth.normal(91, 3, (len(range(1, M, 5)), 32), 1.0e-38)
    x[2::5, 96:128] = x[2::5, 96:128] * np.float32(1.0e-39)   # subnormal block
    x[3, 130] = np.inf
    x[4, 200] = -np.inf
    x[7, 10] = np.nan
    cfg = dict(x=x, M=M, K=K, Q=Q, N=N, codebook_q8=cb)
    out = run(torch, ctx, cb, aqmi.HIGGS, x, cb_type=aqmi.CB_Q8_0, topk=4)
    ref = oracle.higgs_rvq(cfg, topk=4)
    assert np.array_equal(out["idx"], ref["idx"])
    for key in ("residual", "dist"):
        a, b = out[key], ref[key]
        assert np.array_equal(np.isnan(a), np.isnan(b))
        assert np.array_equal(bits(a[~np.isnan(a)]), bits(b[~np.isnan(b)]))
    fin = np.isfinite(x).all(1)   # top-k of the non-finite frames: codes above
    check_topk({k: out[k][fin] for k in ("topk_idx", "topk_dist")},
               {k: ref[k][fin] for k in ("topk_idx", "topk_logit")})


def test_direct_matches_oracle(torch, ctx, oracle):
    import aqmi

    print("[gpu] direct", flush=True)
    cfg = mimi(300, Q=2)
    out = run(torch, ctx, cfg["codebook"], aqmi.DIRECT, cfg["x"])
    ref = oracle.direct_rvq(cfg)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))
    assert np.array_equal(bits(out["dist"]), bits(ref["dist"]))


@pytest.mark.parametrize("recipe", [0, 1, 2])
def test_exact_ties_and_zero_distance(torch, ctx, oracle, recipe):
    """Duplicated codewords (exact ties) and queries equal to codewords
    (distance 0): the certificate cannot settle these, the exact scan must
    apply the reference's tie rule (ggml argmax: last index; DIRECT: first)."""
    from aqmi import synth

    print(f"[gpu] ties recipe={recipe}", flush=True)
    Q, N, K, M = 2, 2048, 256, 200
    cb = synth.normal(31, 2, (Q, N, K), 1.0 / 16)
    cb[:, 1::2] = cb[:, 0::2]
    x = synth.normal(31, 1, (M, K))
    x[:50] = cb[0, 10:60]
    cfg = dict(x=x, M=M, K=K, Q=Q, N=N, codebook=cb)
    out = run(torch, ctx, cb, recipe, x)
    ref = {0: oracle.euclid_rvq, 1: oracle.higgs_rvq, 2: oracle.direct_rvq}[recipe](cfg)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))
    assert out["fails"].sum() > 0


def test_teacher_forced(torch, ctx, oracle):
    import aqmi

    cfg = mimi(400)
    rng = np.random.default_rng(3)
    force = rng.integers(0, cfg["N"], size=(400, cfg["Q"]), dtype=np.int32)
    out = run(torch, ctx, cfg["codebook"], aqmi.OMNIVOICE, cfg["x"], force=force)
    ref = oracle.euclid_rvq(cfg, force_idx=force)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))


def test_nonfinite_queries(torch, ctx, oracle):
    import aqmi

    cfg = mimi(64, Q=2)
    x = cfg["x"].copy()
    x[3, 7] = np.nan
    x[9, :] = np.inf
    cfg["x"] = x
    out = run(torch, ctx, cfg["codebook"], aqmi.OMNIVOICE, x)
    ref = oracle.euclid_rvq(cfg)
    assert np.array_equal(out["idx"], ref["idx"])
    a, b = out["residual"], ref["residual"]
    assert np.array_equal(np.isnan(a), np.isnan(b))
    assert np.array_equal(bits(a[~np.isnan(a)]), bits(b[~np.isnan(b)]))


def test_gather_and_decode(torch, ctx):
    import aqmi
    from aqmi import synth

    cfg = mimi(10)
    cbs = aqmi.Codebooks(ctx, cfg["codebook"], aqmi.OMNIVOICE)
    N, K = cbs.N, cbs.K
    idx = torch.arange(N, dtype=torch.int32, device="cuda")
    out = torch.empty((N, K), dtype=torch.float32, device="cuda")
    cbs.gather(1, idx, out)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out.cpu().numpy()), bits(cfg["codebook"][1]))
    codes = np.stack([np.arange(50) * 7 % N, np.arange(50) * 13 % N, np.arange(50) * 3 % N], 1).astype(np.int32)
    dec = torch.empty((50, K), dtype=torch.float32, device="cuda")
    cbs.decode(torch.from_numpy(codes).cuda(), dec)
    torch.cuda.synchronize()
    want = np.full((50, K), -0.0, np.float32)
    for s in range(3):
        want = (want + cfg["codebook"][s][codes[:, s]]).astype(np.float32)
    assert np.array_equal(bits(dec.cpu().numpy()), bits(want))
    bad = torch.tensor([0, N], dtype=torch.int32, device="cuda")
    with pytest.raises(aqmi.AqError) as e:
        cbs.gather(0, bad, out[:2])
    assert e.value.status == 3
    with pytest.raises(aqmi.AqError) as e:   # an empty codebook
        aqmi.Codebooks(ctx, synth.normal(1, 1, (1, 0, 256)), aqmi.OMNIVOICE)
    assert e.value.status == 2
    q8 = synth.q8_0_random_codebook(1, 1, 64, 256)[None]
    with pytest.raises(aqmi.AqError) as e:
        aqmi.Codebooks(ctx, q8, aqmi.OMNIVOICE, aqmi.CB_Q8_0)
    assert e.value.status == 5


def test_certificate_settles_almost_every_frame(torch, ctx):
    """On the Mimi workload the exact scan is the rare path."""
    import aqmi

    cfg = mimi(4000, Q=2)
    out = run(torch, ctx, cfg["codebook"], aqmi.OMNIVOICE, cfg["x"], want_dist=False)
    print(f"[gpu] fallback frames per stage: {out['fails'].tolist()}", flush=True)
    assert (out["fails"] <= 40).all()


@pytest.mark.parametrize("cb_type", [0, 1])
def test_topk_with_more_ties_than_k(torch, ctx, oracle, cb_type):
    """Six copies of one codeword and queries on it: top-4 lists the four
    smallest tied indices (ggml top_k order) while the code is the last tied
    index (ggml argmax), which lies outside the top-4 list."""
    import aqmi
    from aqmi import synth

    print(f"[gpu] topk ties cb_type={cb_type}", flush=True)
    Q, N, K, M = 1, 1024, 256, 64
    if cb_type == 1:
        cb = synth.q8_0_random_codebook(41, 1, N, K)[None]
        dq = synth.q8_0_dequantize(cb[0])
        for j in (100, 300, 500, 700, 900):
            cb[0, j] = cb[0, 7]
        x = np.repeat(dq[7][None], M, 0) + synth.normal(41, 2, (M, K), 1e-4)
    else:
        cb = synth.normal(41, 1, (Q, N, K), 1.0)
        for j in (100, 300, 500, 700, 900):
            cb[0, j] = cb[0, 7]
        x = np.repeat(cb[0, 7][None], M, 0) + synth.normal(41, 2, (M, K), 1e-4)
    x = x.astype(np.float32)
    cfg = dict(x=x, M=M, K=K, Q=Q, N=N, codebook=cb) if cb_type == 0 else dict(x=x, M=M, K=K, Q=Q, N=N, codebook_q8=cb)
    out = run(torch, ctx, cb, aqmi.HIGGS, x, cb_type=cb_type, topk=4)
    ref = oracle.higgs_rvq(cfg, topk=4)
    assert (ref["idx"] == 900).all()
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))
    check_topk(out, ref)


def sorted_topk(idx, logit):
    order = np.lexsort((idx, -logit.astype(np.float64)), axis=-1)
    return np.take_along_axis(idx, order, -1), np.take_along_axis(logit, order, -1)


def check_topk(out, ref):
    """Top-k lists as sets (ggml_top_k leaves them in heap order), with the
    logits of each member bit for bit."""
    gi, gl = sorted_topk(out["topk_idx"], -out["topk_dist"])
    ri, rl = sorted_topk(ref["topk_idx"], ref["topk_logit"])
    assert np.array_equal(gi, ri)
    assert np.array_equal(bits(gl), bits(rl))


def quantize_q8_rows(rows):
    """Any valid block_q8_0 image of float rows (test data only)."""
    from aqmi import synth

    n, k = rows.shape
    b = rows.reshape(n, k // 32, 32)
    amax = np.abs(b).max(-1)
    d = (amax / 127.0).astype(np.float16)
    df = d.astype(np.float32)
    q = np.where(df[..., None] > 0, np.rint(b / np.where(df > 0, df, 1)[..., None]), 0).clip(-127, 127)
    out = np.zeros((n, k // 32), dtype=synth.Q8_DTYPE)
    out["d"] = d
    out["qs"] = q.astype(np.int8)
    return out


@pytest.mark.parametrize("cb_type", [0, 1])
def test_topk_tie_at_kth_place_follows_ggml_heap(torch, ctx, oracle, cb_type):
    """Codes 200 and 1000 are identical and rank 4th/5th behind codes 1500,
    1600 and 1700: which of the two ggml_top_k keeps is decided by
    std::partial_sort's heap (the oracle restates it, pinned against ggml),
    not by index order.  The certificate must hand these frames to the
    exact scan, which replays the heap."""
    import aqmi
    from aqmi import synth

    print(f"[gpu] topk kth-place tie cb_type={cb_type}", flush=True)
    N, K, M = 2048, 256, 64
    base = synth.normal(51, 1, (K,))
    cbf = synth.normal(51, 2, (N, K), 1.0)
    cbf[1500] = base + synth.normal(51, 3, (K,), 0.05)
    cbf[1600] = base + synth.normal(51, 4, (K,), 0.06)
    cbf[1700] = base + synth.normal(51, 5, (K,), 0.07)
    cbf[200] = base + synth.normal(51, 6, (K,), 0.2)
    cbf[1000] = cbf[200]
    x = (base[None] + synth.normal(51, 7, (M, K), 1e-3)).astype(np.float32)
    if cb_type == 1:
        cb = quantize_q8_rows(cbf)[None]
        cfg = dict(x=x, M=M, K=K, Q=1, N=N, codebook_q8=cb)
    else:
        cb = cbf[None].astype(np.float32)
        cfg = dict(x=x, M=M, K=K, Q=1, N=N, codebook=cb)
    out = run(torch, ctx, cb, aqmi.HIGGS, x, cb_type=cb_type, topk=4)
    ref = oracle.higgs_rvq(cfg, topk=4)
    ri, _ = sorted_topk(ref["topk_idx"], ref["topk_logit"])
    assert set(ri[:, 0, :3].ravel().tolist()) <= {1500, 1600, 1700}
    assert np.isin(ri[:, 0, 3], [200, 1000]).all()
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))
    check_topk(out, ref)
    assert out["fails"][0] == M


@pytest.mark.parametrize("recipe,cb_type,topk,dup,inf", [
    (1, 0, 4, 3, False), (1, 1, 4, 3, False), (1, 0, 3, 2, False), (1, 0, 2, 3, False), (1, 0, 1, 3, False),
    (1, 0, 3, 3, True), (2, 0, 0, 3, True), (0, 0, 0, 3, True)])
@pytest.mark.parametrize("N,M", [(2048, 40), (2048, 150), (4096, 40), (4096, 150)])
def test_exact_scan_with_repeated_codes(torch, ctx, oracle, recipe, cb_type, topk, dup, inf, N, M, pipeline):
    """Every codeword appears dup times, so each frame's best value ties
    exactly with dup - 1 others.  When the k-th and (k+1)-th places tie too
    (k not a multiple of dup), no certificate settles the frame: every frame
    of both stages goes to the exact scan, and ggml_top_k's heap (of k = 1
    to 4 entries) decides which copy stays.  Otherwise (inf) a -inf codebook
    entry (no NaN: the queries' first element is positive) makes the
    codebook non-finite, which sends every frame to the scan too.  Up to 64
    frames per stage take values computed over the whole grid, more are
    evaluated by their own block; 2048 codes fit the scan's LDS chunk, 4096
    do not.  The ggml argmax takes the last tied index, DIRECT the first."""
    from aqmi import synth

    print(f"[gpu] repeated codes recipe={recipe} cb_type={cb_type} topk={topk} dup={dup} inf={inf} N={N} M={M}",
          flush=True)
    Q, K = 2, 256
    rep = np.arange(N) // dup * dup
    if cb_type == 1:
        cb = np.stack([synth.q8_0_random_codebook(71, 10 + s, N, K) for s in range(Q)])[:, rep]
        x = (synth.q8_0_dequantize(cb[0])[(7 * np.arange(M)) % N] + synth.normal(71, 2, (M, K), 0.05)).astype(np.float32)
        cfg = dict(x=x, M=M, K=K, Q=Q, N=N, codebook_q8=cb)
    else:
        cb = np.ascontiguousarray(synth.normal(71, 3, (Q, N, K), 1.0 / 16)[:, rep])
        x = synth.normal(71, 1, (M, K), 1.0)
        if inf:
            cb[0, 5, 0] = -np.inf
            x[:, 0] = np.abs(x[:, 0]) + 0.25
        cfg = dict(x=x, M=M, K=K, Q=Q, N=N, codebook=cb)
    out = run(torch, ctx, cb, recipe, x, cb_type=cb_type, topk=topk)
    ref = {0: oracle.euclid_rvq, 1: oracle.higgs_rvq, 2: oracle.direct_rvq}[recipe]
    ref = ref(cfg, topk=topk) if recipe == 1 else ref(cfg)
    scans = out["cbs"].exact_scans()
    print(f"[gpu] open frames {out['fails'].tolist()}, exact scans per stage {scans.tolist()}", flush=True)
    # on the cascade every open frame is verified by the exact scan
    assert ((scans if effective(pipeline, K, cb_type) == "stages" else out["fails"]) >= 0.9 * M).all()
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))
    if recipe == 0:
        assert np.array_equal(bits(out["dist"]), bits(-ref["logit"]))
    else:
        assert np.array_equal(bits(out["dist"]), bits(ref["dist"]))
    if topk:
        check_topk(out, ref)


def test_ema_codebook_and_upload(torch, ctx, oracle):
    """aq_ema_codebook bit for bit against the oracle (usage below eps, zero,
    NaN), and aq_euclid_upload_ema encoding exactly like an upload of the
    oracle's materialised codebook (Qwen3's nearest_code: DIRECT recipe)."""
    import aqmi

    print("[gpu] ema codebook", flush=True)
    rng = np.random.default_rng(11)
    Q, N, K, M = 3, 2048, 256, 257
    es = (rng.standard_normal((Q, N, K)) * 4.0).astype(np.float32)
    cu = rng.uniform(1.0, 30.0, (Q, N)).astype(np.float32)
    cu[0, :4] = [0.0, 1e-7, -1.0, 1e-5]
    want = oracle.ema_codebook(es, cu, 1e-5)
    d_es = torch.from_numpy(es).cuda()
    d_cu = torch.from_numpy(cu).cuda()
    d_out = torch.empty_like(d_es)
    aqmi.ema_codebook(ctx, d_es, d_cu, 1e-5, d_out)
    torch.cuda.synchronize()
    assert np.array_equal(bits(d_out.cpu().numpy()), bits(want))
    cu_nan = cu.copy()
    cu_nan[1, 7] = np.nan
    aqmi.ema_codebook(ctx, d_es, torch.from_numpy(cu_nan).cuda(), 1e-5, d_out)
    torch.cuda.synchronize()
    got = d_out.cpu().numpy()
    assert np.isnan(got[1, 7]).all() and np.array_equal(bits(np.delete(got[1], 7, 0)), bits(np.delete(want[1], 7, 0)))

    x = (rng.standard_normal((M, K)) * 4.0).astype(np.float32)
    cbs = aqmi.Codebooks.from_ema(ctx, es, cu, aqmi.DIRECT)
    xd = torch.from_numpy(x).cuda()
    idx = torch.full((M, Q), -1, dtype=torch.int32, device="cuda")
    res = torch.empty((M, K), dtype=torch.float32, device="cuda")
    cbs.encode(xd, idx, res)
    torch.cuda.synchronize()
    ref = oracle.direct_rvq(dict(x=x, M=M, K=K, Q=Q, N=N, codebook=want))
    assert np.array_equal(idx.cpu().numpy(), ref["idx"])
    assert np.array_equal(bits(res.cpu().numpy()), bits(ref["residual"]))


@pytest.mark.parametrize("recipe,cb_type,K,N,M,Q,topk", [
    (0, 0, 512, 1024, 333, 2, 0), (1, 0, 512, 1024, 250, 2, 0), (1, 1, 512, 1024, 250, 2, 4),
    (2, 0, 512, 512, 300, 3, 0), (1, 1, 64, 1024, 400, 3, 4), (1, 1, 768, 256, 200, 2, 2),
    (1, 1, 64, 256, 1, 2, 0)])
def test_other_widths_and_q8_widths(torch, ctx, oracle, recipe, cb_type, K, N, M, Q, topk):
    """K = 512 (its own translation unit) for every recipe, and Q8_0
    codebooks at K = 64 and 768, against the oracle."""
    from aqmi import synth

    print(f"[gpu] width K={K} recipe={recipe} cb_type={cb_type} topk={topk}", flush=True)
    x = synth.normal(61, 1, (M, K), 1.0)
    if cb_type == 1:
        cb = np.stack([synth.q8_0_random_codebook(61, 10 + s, N, K) for s in range(Q)])
        # queries near the dequantised codes keep the distances in the codebook's range
        x = (synth.q8_0_dequantize(cb[0])[np.arange(M) % N] + synth.normal(61, 2, (M, K), 0.05)).astype(np.float32)
        cfg = dict(x=x, M=M, K=K, Q=Q, N=N, codebook_q8=cb)
    else:
        cb = synth.normal(61, 3, (Q, N, K), 1.0 / 16)
        cfg = dict(x=x, M=M, K=K, Q=Q, N=N, codebook=cb)
    out = run(torch, ctx, cb, recipe, x, cb_type=cb_type, topk=topk)
    ref = {0: oracle.euclid_rvq, 1: oracle.higgs_rvq, 2: oracle.direct_rvq}[recipe]
    ref = ref(cfg, topk=topk) if recipe == 1 else ref(cfg)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))
    if recipe == 0:
        assert np.array_equal(bits(out["dist"]), bits(-ref["logit"]))
    else:
        assert np.array_equal(bits(out["dist"]), bits(ref["dist"]))
    if topk:
        check_topk(out, ref)


def near_duplicate_groups(rows, Q=2):
    """Mimi-shaped data whose codewords come in groups of 8 that differ by
    multiples of 2^-13 (relative) and fall in the same sweep lane (codes
    16 apart): more near-ties than a lane keeps, closer than the fp16
    certificate can separate and far apart for the split-fp16 refine pass,
    so every frame is left open and the refine pass settles it."""
    from aqmi import synth

    cfg = mimi(rows, Q=Q)
    cb = cfg["codebook"]
    Qn, N, K = cb.shape
    g = cb.reshape(Qn, N // 128, 8, 16, K)
    scale = (1.0 + np.arange(8, dtype=np.float32) * np.float32(2.0 ** -13))[None, None, :, None, None]
    g[:] = (g[:, :, :1] * scale + synth.normal(72, 1, g.shape, 2.0 ** -20)).astype(np.float32)
    cfg["codebook"] = np.ascontiguousarray(g.reshape(Qn, N, K))
    half = rows // 2
    cfg["x"][:half] = (cfg["codebook"][0, (37 * np.arange(half)) % N]
                       + synth.normal(72, 2, (half, K), 0.05)).astype(np.float32)
    return cfg


@pytest.mark.parametrize("recipe", [0, 1, 2])
def test_refine_pass_settles_near_duplicates(torch, ctx, oracle, recipe, pipeline):
    """More open frames than the exact scan spreads (64) go through the
    split-fp16 refine pass, which settles nearly all of them; results are
    the reference's.  (Up to 512 open frames the pass works in 32-code
    slices, whose lane lists keep two members of each group.)  On the
    cascade, every open frame continues with its best exact candidate and is
    verified; where the group's true best was dropped from the lane's keys
    the fix-up recomputes the frame."""
    print(f"[gpu] refine near duplicates recipe={recipe} {pipeline}", flush=True)
    cfg = near_duplicate_groups(400)
    out = run(torch, ctx, cfg["codebook"], recipe, cfg["x"])
    ref = {0: oracle.euclid_rvq, 1: oracle.higgs_rvq, 2: oracle.direct_rvq}[recipe](cfg)
    scans = out["cbs"].exact_scans()
    print(f"[gpu] open frames {out['fails'].tolist()}, exact scans {scans.tolist()}", flush=True)
    if pipeline == "stages":
        assert (out["fails"] > 64).all() and (scans < out["fails"] // 4).all()
    else:
        assert (out["fails"] > 64).all()
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))
    if recipe == 0:
        assert np.array_equal(bits(out["dist"]), bits(-ref["logit"]))
    else:
        assert np.array_equal(bits(out["dist"]), bits(ref["dist"]))


def test_refine_capacity_overflow_goes_to_exact_scan(torch, ctx, oracle, monkeypatch, pipeline):
    """With the refine pass's key buffer capped at 2048 floats (test hook
    AQ_EUCLID_REFINE_KEY_FLOATS: too few for short or middle slices of the
    open frames, and 16 frames of long-slice keys), every further frame the
    first certificate leaves open must reach the exact scan without reading
    keys past the buffer, and the results stay the reference's."""
    import aqmi

    if pipeline != "stages":
        pytest.skip("the refine pass belongs to the per-stage pipeline")
    print("[gpu] refine capacity overflow", flush=True)
    cfg = near_duplicate_groups(400)
    monkeypatch.setenv("AQ_EUCLID_REFINE_KEY_FLOATS", "2048")
    out = run(torch, ctx, cfg["codebook"], aqmi.OMNIVOICE, cfg["x"])
    scans = out["cbs"].exact_scans()
    ref = oracle.euclid_rvq(cfg)
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))
    assert np.array_equal(bits(out["dist"]), bits(-ref["logit"]))
    print(f"[gpu] open frames {out['fails'].tolist()}, exact scans {scans.tolist()}", flush=True)
    assert (out["fails"] > 64).all() and (scans >= out["fails"] - 16).all() and (scans <= out["fails"]).all()


@pytest.mark.parametrize("recipe,cb_type,topk,K", [(0, 0, 0, 256), (1, 0, 4, 256), (2, 0, 0, 256), (1, 1, 4, 256),
                                                   (1, 0, 3, 64), (0, 0, 0, 64)])
@pytest.mark.parametrize("M,Q", [(37, 3), (700, 8)])
def test_cascade_fixup_recomputes_wrong_continuations(torch, ctx, oracle, monkeypatch, pipeline, recipe, cb_type,
                                                      topk, K, M, Q):
    """Test hook AQ_EUCLID_TEST_MISSPECULATE=1: in the cascade every frame of
    every stage continues with a code that is not its best.  The exact
    verification must find each frame's earliest wrong stage and the fix-up
    recompute the frame from there: every output (codes, distances, top-k,
    residual) ends as the reference's."""
    from aqmi import synth

    if effective(pipeline, K, cb_type) == "stages":
        pytest.skip("speculation belongs to the one-launch cascades")
    print(f"[gpu] cascade fix-up recipe={recipe} cb_type={cb_type} topk={topk} K={K} M={M} Q={Q}", flush=True)
    N = 1024
    x = synth.normal(81, 1, (M, K), 1.0)
    if cb_type == 1:
        cb = np.stack([synth.q8_0_random_codebook(81, 10 + s, N, K) for s in range(Q)])
        cfg = dict(x=x, M=M, K=K, Q=Q, N=N, codebook_q8=cb)
    else:
        cb = synth.normal(81, 2, (Q, N, K), 1.0 / 16)
        cfg = dict(x=x, M=M, K=K, Q=Q, N=N, codebook=cb)
    monkeypatch.setenv("AQ_EUCLID_TEST_MISSPECULATE", "1")
    out = run(torch, ctx, cb, recipe, x, cb_type=cb_type, topk=topk)
    ref = {0: oracle.euclid_rvq, 1: oracle.higgs_rvq, 2: oracle.direct_rvq}[recipe]
    ref = ref(cfg, topk=topk) if recipe == 1 else ref(cfg)
    scans = out["cbs"].exact_scans()
    print(f"[gpu] speculated {out['fails'].tolist()}, recomputed {scans.tolist()}", flush=True)
    assert out["fails"].tolist() == [M] * Q
    assert scans.tolist() == [M] * Q   # every frame is wrong from stage 0 on: all stages recomputed
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))
    if recipe == 0:
        assert np.array_equal(bits(out["dist"]), bits(-ref["logit"]))
    else:
        assert np.array_equal(bits(out["dist"]), bits(ref["dist"]))
    if topk:
        check_topk(out, ref)


@pytest.mark.parametrize("recipe,cb_type,topk,K", [(0, 0, 0, 256), (1, 0, 4, 256), (1, 1, 4, 256), (2, 0, 0, 64)])
def test_cascade_verification_corrects_outputs_in_place(torch, ctx, oracle, monkeypatch, pipeline, recipe, cb_type,
                                                        topk, K):
    """Test hook AQ_EUCLID_TEST_MISSPECULATE=2: every frame of every stage
    continues with its best code but writes its distances (and top-k
    distances) one bit off, uncertified.  The verification must find the
    codes right and correct the outputs in place, without sending the
    frames to the fix-up: every output ends as the reference's."""
    from aqmi import synth

    if effective(pipeline, K, cb_type) == "stages":
        pytest.skip("speculation belongs to the one-launch cascades")
    M, Q, N = 300, 4, 1024
    print(f"[gpu] cascade in-place correction recipe={recipe} cb_type={cb_type} topk={topk} K={K}", flush=True)
    x = synth.normal(83, 1, (M, K), 1.0)
    if cb_type == 1:
        cb = np.stack([synth.q8_0_random_codebook(83, 10 + s, N, K) for s in range(Q)])
        cfg = dict(x=x, M=M, K=K, Q=Q, N=N, codebook_q8=cb)
    else:
        cb = synth.normal(83, 2, (Q, N, K), 1.0 / 16)
        cfg = dict(x=x, M=M, K=K, Q=Q, N=N, codebook=cb)
    monkeypatch.setenv("AQ_EUCLID_TEST_MISSPECULATE", "2")
    out = run(torch, ctx, cb, recipe, x, cb_type=cb_type, topk=topk)
    ref = {0: oracle.euclid_rvq, 1: oracle.higgs_rvq, 2: oracle.direct_rvq}[recipe]
    ref = ref(cfg, topk=topk) if recipe == 1 else ref(cfg)
    scans = out["cbs"].exact_scans()
    print(f"[gpu] verified {out['fails'].tolist()}, recomputed {scans.tolist()}", flush=True)
    assert out["fails"].tolist() == [M] * Q
    # only a frame whose best evaluated code was not the reference's (a
    # genuine misspeculation, rare) goes to the fix-up
    assert (scans < M // 10).all()
    assert np.array_equal(out["idx"], ref["idx"])
    assert np.array_equal(bits(out["residual"]), bits(ref["residual"]))
    if recipe == 0:
        assert np.array_equal(bits(out["dist"]), bits(-ref["logit"]))
    else:
        assert np.array_equal(bits(out["dist"]), bits(ref["dist"]))
    if topk:
        check_topk(out, ref)


def test_sweep_split_parts_agree(torch, ctx, oracle, monkeypatch):
    """A grid of several rounds of sweep blocks takes one code-split count
    for the tiles of its whole rounds and a finer one for the last, partial
    round.  The results are the bits of one split count for every tile
    (test hook AQ_EUCLID_TEST_SPLIT=uniform) and, on frames of both parts,
    the reference's."""
    import aqmi
    from aqmi import synth

    M, K, N, Q = 70000, 512, 1024, 2   # 547 tiles of 128 frames: 512 in whole rounds, then 35
    print(f"[gpu] sweep split parts M={M} K={K} N={N} Q={Q}", flush=True)
    x = synth.normal(91, 1, (M, K), 1.0)
    cb = synth.normal(91, 2, (Q, N, K), 1.0 / 16)
    monkeypatch.setenv("AQ_EUCLID_PIPELINE", "stages")
    two = run(torch, ctx, cb, aqmi.HIGGS, x)
    monkeypatch.setenv("AQ_EUCLID_TEST_SPLIT", "uniform")
    one = run(torch, ctx, cb, aqmi.HIGGS, x)
    assert np.array_equal(two["idx"], one["idx"])
    assert np.array_equal(bits(two["dist"]), bits(one["dist"]))
    assert np.array_equal(bits(two["residual"]), bits(one["residual"]))
    for lo in (0, 68000):   # a tile of the whole rounds, one of the last round
        sub = dict(x=x[lo:lo + 1000], M=1000, K=K, Q=Q, N=N, codebook=cb)
        ref = oracle.higgs_rvq(sub)
        assert np.array_equal(two["idx"][lo:lo + 1000], ref["idx"])
        assert np.array_equal(bits(two["dist"][lo:lo + 1000]), bits(ref["dist"]))
