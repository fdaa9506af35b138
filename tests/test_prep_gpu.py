"""GPU parity of the codebook ingest and preparation done on the device:
weight-norm folding (aq_weight_norm_fold) against the oracle's restatement
of both loaders' folds (the OuteTTS one pinned to the reference's own
fold_weight_norm in test_oracle.py), and codebooks uploaded from device
memory (aq_euclid_upload_device) encoding exactly like host uploads.  The
device-side preparation inside aq_euclid_upload / aq_dac_upload /
aq_moss_upload is covered by every parity test of those paths.
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


@pytest.mark.parametrize("shape", [(8, 1024, 1), (1024, 8, 1), (64, 32, 7), (512, 1024, 1)])
@pytest.mark.parametrize("rule", [0, 1])
def test_weight_norm_fold_matches_oracle(torch, ctx, oracle, rule, shape):
    """Both folds bit for bit (a zero magnitude, a tiny row), out of place
    and in place."""
    import aqmi
    from aqmi import synth

    print(f"[gpu] weight norm fold rule={rule} shape={shape}", flush=True)
    v = synth.normal(23, shape[0], shape, 1.0)
    v[min(1, shape[0] - 1)] *= 1e-30
    g = synth.uniform(23, 77, (shape[0],), 0.1, 3.0)
    g[0] = 0.0
    if rule == aqmi.WN_OUTETTS:
        want = oracle.outetts_weight_norm(v, g)
    else:
        want = oracle.moss_weight_norm(g, v.reshape(shape[0], -1)).reshape(shape)
    dv = torch.from_numpy(v).cuda()
    dg = torch.from_numpy(g).cuda()
    out = torch.empty_like(dv)
    aqmi.weight_norm_fold(ctx, dv, dg, rule, out)
    aqmi.weight_norm_fold(ctx, dv, dg, rule, dv)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out.cpu().numpy()), bits(want))
    assert np.array_equal(bits(dv.cpu().numpy()), bits(want))


def test_weight_norm_fold_errors(torch, ctx):
    import aqmi

    dv = torch.zeros((4, 8), device="cuda")
    dg = torch.ones(4, device="cuda")
    with pytest.raises(aqmi.AqError):
        aqmi.weight_norm_fold(ctx, dv, dg, 7, dv)


@pytest.mark.parametrize("cb_type,recipe", [(0, 0), (0, 2), (1, 1)])
def test_upload_from_device_memory(torch, ctx, cb_type, recipe):
    """A codebook handed over in device memory encodes exactly like the same
    codebook uploaded from the host (codes, residual, distances, top-k)."""
    import aqmi
    from aqmi import synth

    print(f"[gpu] device upload cb_type={cb_type} recipe={recipe}", flush=True)
    Q, N, K, M = 2, 1024, 256, 300
    topk = 4 if recipe == 1 else 0
    if cb_type == 1:
        cb = np.stack([synth.q8_0_random_codebook(29, 10 + s, N, K) for s in range(Q)])
        x = (synth.q8_0_dequantize(cb[0])[np.arange(M) % N] + synth.normal(29, 2, (M, K), 0.05)).astype(np.float32)
        dcb = torch.from_numpy(np.frombuffer(cb.tobytes(), np.uint8).copy()).cuda()
    else:
        cb = synth.normal(29, 3, (Q, N, K), 1.0 / 16)
        x = synth.normal(29, 1, (M, K), 1.0)
        dcb = torch.from_numpy(cb).cuda()
    outs = []
    for cbs in (aqmi.Codebooks(ctx, cb, recipe, cb_type),
                aqmi.Codebooks.from_device(ctx, dcb, recipe, cb_type, shape=(Q, N, K))):
        xd = torch.from_numpy(x).cuda()
        idx = torch.full((M, Q), -1, dtype=torch.int32, device="cuda")
        res = torch.empty((M, K), dtype=torch.float32, device="cuda")
        dist = torch.empty((M, Q), dtype=torch.float32, device="cuda")
        tki = torch.zeros((M, Q, 4), dtype=torch.int32, device="cuda")
        tkd = torch.zeros((M, Q, 4), dtype=torch.float32, device="cuda")
        cbs.encode(xd, idx, res, dist, topk, tki if topk else None, tkd if topk else None, None)
        torch.cuda.synchronize()
        outs.append([t.cpu().numpy() for t in (idx, res, dist, tki, tkd)])
    for a, b in zip(*outs):
        assert np.array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                              b.view(np.uint32) if b.dtype == np.float32 else b)


def test_upload_quantises_f32_like_the_weight_store(torch, ctx, oracle):
    """CB_F32_AS_Q8_0: F32 codebooks quantised to Q8_0 on the device give the
    blocks of the reference weight store's ggml_quantize_chunk
    (synth.q8_0_quantize_ref, pinned to the reference in test_oracle.py):
    the gathered rows equal the dequantised reference blocks bit for bit, and
    encodes (codes, residual, distances, top-4) equal an upload of those
    blocks and the oracle.  Rows include zeros, ties at amax and halves."""
    import aqmi
    from aqmi import synth

    print("[gpu] f32 -> q8_0 upload", flush=True)
    Q, N, K, M = 2, 1024, 256, 200
    f = synth.normal(31, 5, (Q, N, K), 0.3)
    f[0, 3] = 0.0
    f[0, 4, :32] = 1.0
    f[1, 9, :32] = np.linspace(-63.5, 63.5, 32, dtype=np.float32) / 127.0
    blocks = synth.q8_0_quantize_ref(f)
    x = (synth.q8_0_dequantize(blocks[0])[np.arange(M) % N] + synth.normal(31, 6, (M, K), 0.02)).astype(np.float32)
    got = aqmi.Codebooks(ctx, f, aqmi.HIGGS, aqmi.CB_F32_AS_Q8_0)
    ref = aqmi.Codebooks(ctx, blocks, aqmi.HIGGS, aqmi.CB_Q8_0)
    for s in range(Q):
        idx = torch.arange(N, dtype=torch.int32, device="cuda")
        rows = torch.empty((N, K), dtype=torch.float32, device="cuda")
        got.gather(s, idx, rows)
        torch.cuda.synchronize()
        assert np.array_equal(bits(rows.cpu().numpy()), bits(synth.q8_0_dequantize(blocks[s])))
    outs = []
    for cbs in (got, ref):
        xd = torch.from_numpy(x).cuda()
        idx = torch.full((M, Q), -1, dtype=torch.int32, device="cuda")
        res = torch.empty((M, K), dtype=torch.float32, device="cuda")
        dist = torch.empty((M, Q), dtype=torch.float32, device="cuda")
        tki = torch.zeros((M, Q, 4), dtype=torch.int32, device="cuda")
        tkd = torch.zeros((M, Q, 4), dtype=torch.float32, device="cuda")
        cbs.encode(xd, idx, res, dist, 4, tki, tkd, None)
        torch.cuda.synchronize()
        outs.append([t.cpu().numpy() for t in (idx, res, dist)])
    want = oracle.higgs_rvq(dict(x=x, M=M, K=K, Q=Q, N=N, codebook_q8=blocks), topk=4)
    assert np.array_equal(outs[0][0], want["idx"])
    assert np.array_equal(bits(outs[0][1]), bits(want["residual"]))
    for a, b in zip(*outs):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("n_out,k,M,q8,bias", [(64, 1024, 1, False, True), (64, 1024, 2, False, True),
                                                (128, 512, 301, False, False), (1024, 64, 77, False, True),
                                                (64, 1024, 1, True, True), (256, 512, 333, True, False),
                                                (512, 2496, 40, False, True), (128, 1984, 40, True, True),
                                                (40960, 256, 1, False, True), (128, 2496, 1, False, False)])
def test_linear_matches_oracle(torch, ctx, oracle, n_out, k, M, q8, bias):
    """aq_linear (encoder output projection) bit for bit against the
    oracle's LinearModule (pinned to the reference's ggml graph in
    test_oracle.py): one frame and batches, F32 and Q8_0 weights, the
    largest supported widths."""
    import aqmi
    from aqmi import synth

    print(f"[gpu] linear {n_out}x{k} M={M} q8={q8}", flush=True)
    w = synth.normal(37, n_out + k, (n_out, k), 0.05)
    if q8:
        w = synth.q8_0_quantize_ref(w)
    x = synth.normal(37, M, (M, k), 1.0)
    b = synth.normal(37, 3, (n_out,), 0.1) if bias else None
    lin = aqmi.Linear(ctx, w, b)
    out = torch.empty((M, n_out), dtype=torch.float32, device="cuda")
    lin.forward(torch.from_numpy(x).cuda(), out)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out.cpu().numpy()), bits(oracle.linear(w, b, x)))


@pytest.mark.parametrize("q8", [False, True])
def test_linear_channel_major_input(torch, ctx, oracle, q8):
    """The encoder's [B, C, T] output read in place (frames of two clips):
    the same bits as the frame-major rows."""
    import aqmi
    from aqmi import synth

    B, Cc, T, n_out = 2, 512, 150, 128
    w = synth.normal(38, 1, (n_out, Cc), 0.05)
    if q8:
        w = synth.q8_0_quantize_ref(w)
    lat = synth.normal(38, 2, (B, Cc, T), 1.0)
    x = np.ascontiguousarray(lat.transpose(0, 2, 1).reshape(B * T, Cc))
    lin = aqmi.Linear(ctx, w, synth.normal(38, 3, (n_out,), 0.1))
    out = torch.empty((B * T, n_out), dtype=torch.float32, device="cuda")
    lin.forward(torch.from_numpy(lat).cuda(), out, M=B * T, clip_len=T, strides=(Cc * T, 1, T))
    torch.cuda.synchronize()
    assert np.array_equal(bits(out.cpu().numpy()), bits(oracle.linear(w, synth.normal(38, 3, (n_out,), 0.1), x)))


def test_linear_errors(torch, ctx):
    import aqmi

    with pytest.raises(aqmi.AqError):
        aqmi.Linear(ctx, np.zeros((60, 64), np.float32))
    with pytest.raises(aqmi.AqError):
        aqmi.Linear(ctx, np.zeros((64, 2560), np.float32))


@pytest.mark.parametrize("q8,last_ok", [(False, 2496), (True, 1984)])
def test_lds_limits_include_static_lds(torch, ctx, q8, last_ok):
    """The projection kernels keep 16 frames' rows in LDS: the largest
    hidden size that fits next to the kernels' static LDS uploads, the next
    multiple of 64 returns AQ_E_SHAPE before anything is launched (linear and
    projected uploads alike)."""
    import aqmi
    from aqmi import synth

    print(f"[gpu] LDS limit q8={q8}", flush=True)

    def weights(rows, cols):
        w = synth.normal(39, rows + cols, (rows, cols), 0.05)
        return synth.q8_0_quantize_ref(w) if q8 else w

    aqmi.Linear(ctx, weights(64, last_ok)).close()
    with pytest.raises(aqmi.AqError) as e:
        aqmi.Linear(ctx, weights(64, last_ok + 64))
    assert e.value.status == 2
    Q, N, K = 1, 256, 64
    cb = synth.normal(39, 5, (Q, N, K), 0.3)
    for H, ok in ((last_ok, True), (last_ok + 64, False)):
        w_in = np.stack([weights(K, H)])
        w_out = np.stack([weights(H, K)])
        if ok:
            aqmi.Codebooks.projected(ctx, cb, w_in, None, w_out, None, aqmi.HIGGS,
                                     proj_type=aqmi.CB_Q8_0 if q8 else aqmi.CB_F32).close()
        else:
            with pytest.raises(aqmi.AqError) as e:
                aqmi.Codebooks.projected(ctx, cb, w_in, None, w_out, None, aqmi.HIGGS,
                                         proj_type=aqmi.CB_Q8_0 if q8 else aqmi.CB_F32)
            assert e.value.status == 2
