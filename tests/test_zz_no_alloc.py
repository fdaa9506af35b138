"""aq_euclid_encode_noalloc through the C ABI: its outputs equal
aq_euclid_encode's bit for bit on two calls in a row (the second smaller, so
the shared scratch region holds the first call's contents), with and without
a caller residual buffer, for plain, Q8_0 top-k, projected and any-width
codebooks; calls from two contexts on two streams, enqueued back to back,
are ordered rather than racing on the shared region; a warmed-up call
allocates no device memory; and a call that needs more than the region
fails cleanly."""

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


def outputs(torch, cbs, x, topk, with_residual, noalloc):
    M, Q, H = x.shape[0], cbs.Q, cbs.H
    idx = torch.full((M, Q), -1, dtype=torch.int32, device="cuda")
    res = torch.empty((M, H), dtype=torch.float32, device="cuda") if with_residual else None
    dist = torch.empty((M, Q), dtype=torch.float32, device="cuda")
    tki = torch.empty((M, Q, topk), dtype=torch.int32, device="cuda") if topk else None
    tkd = torch.empty((M, Q, topk), dtype=torch.float32, device="cuda") if topk else None
    enc = cbs.encode_noalloc if noalloc else cbs.encode
    enc(x, idx, res, dist, topk, tki, tkd)
    torch.cuda.synchronize()
    out = [idx.cpu().numpy(), dist.cpu().numpy().view(np.uint32)]
    if with_residual:
        out.append(res.cpu().numpy().view(np.uint32))
    if topk:
        out += [tki.cpu().numpy(), tkd.cpu().numpy().view(np.uint32)]
    return out


def compare(torch, cbs, xs, topk):
    for x, with_residual in zip(xs, (True, False)):
        print(f"[gpu] no-alloc M={x.shape[0]} residual={with_residual} topk={topk}", flush=True)
        got = outputs(torch, cbs, x, topk, with_residual, noalloc=True)
        want = outputs(torch, cbs, x, topk, with_residual, noalloc=False)
        for a, b in zip(got, want):
            assert np.array_equal(a, b)


def test_noalloc_plain_matches_encode(torch, ctx):
    import aqmi
    from aqmi import synth

    cfg = synth.make_config(2, rows=5000)
    cbs = aqmi.Codebooks(ctx, cfg["codebook"][:3], aqmi.OMNIVOICE)
    x = torch.from_numpy(cfg["x"]).cuda()
    compare(torch, cbs, [x, x[:1203].contiguous()], 0)


def test_noalloc_q8_topk_matches_encode(torch, ctx):
    import aqmi
    from aqmi import synth

    cfg = synth.make_config(4, rows=3000)
    cbs = aqmi.Codebooks(ctx, cfg["codebook_q8"][:2], aqmi.HIGGS, aqmi.CB_Q8_0)
    x = torch.from_numpy(cfg["x"]).cuda()
    compare(torch, cbs, [x, x[:517].contiguous()], 4)


def test_noalloc_projected_matches_encode(torch, ctx):
    import aqmi
    from aqmi import synth

    cfg = synth.projected_config(300, recipe=1, Q=4)
    cbs = aqmi.Codebooks.projected(ctx, cfg["codebook"], cfg["w_in"], cfg["b_in"], cfg["w_out"], cfg["b_out"],
                                   aqmi.HIGGS)
    x = torch.from_numpy(cfg["x"]).cuda()
    compare(torch, cbs, [x, x[:64].contiguous()], 0)


def test_noalloc_rejects_what_does_not_fit(torch, ctx):
    """A full Mimi batch without a residual buffer needs 49 MB of work space,
    more than the 32 MiB region; with the caller's residual buffer it fits."""
    import aqmi
    from aqmi import synth

    cfg = synth.make_config(2)
    cbs = aqmi.Codebooks(ctx, cfg["codebook"][:1], aqmi.OMNIVOICE)
    x = torch.from_numpy(cfg["x"]).cuda()
    idx = torch.empty((x.shape[0], 1), dtype=torch.int32, device="cuda")
    with pytest.raises(aqmi.AqError) as e:
        cbs.encode_noalloc(x, idx)
    assert e.value.status == 2
    res = torch.empty_like(x)
    cbs.encode_noalloc(x, idx, res)
    want = torch.empty_like(idx)
    cbs.encode(x, want)
    torch.cuda.synchronize()
    assert torch.equal(idx, want)


def test_noalloc_any_width_matches_encode(torch, ctx):
    import aqmi
    from aqmi import synth

    cb = synth.normal(61, 2, (2, 1000, 100), 0.25)
    cbs = aqmi.Codebooks(ctx, cb, aqmi.DIRECT)
    x = torch.from_numpy(synth.normal(61, 1, (700, 100))).cuda()
    compare(torch, cbs, [x, x[:99].contiguous()], 0)


def test_noalloc_two_contexts_two_streams_are_ordered(torch):
    """Two contexts, each on its own stream, call the no-allocation entry
    point back to back with no host synchronisation between them; both
    results equal aq_euclid_encode's."""
    import aqmi
    from aqmi import synth

    print("[gpu] no-alloc two contexts on two streams", flush=True)
    cfg = synth.make_config(2, rows=4000)
    c1, c2 = aqmi.Context(0), aqmi.Context(0)
    b1 = aqmi.Codebooks(c1, cfg["codebook"][:3], aqmi.OMNIVOICE)
    b2 = aqmi.Codebooks(c2, cfg["codebook"][3:6], aqmi.HIGGS)
    x1 = torch.from_numpy(cfg["x"]).cuda()
    x2 = torch.from_numpy(cfg["x"][::-1].copy()).cuda()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = []
    for rep in range(2):
        i1 = torch.full((4000, 3), -1, dtype=torch.int32, device="cuda")
        i2 = torch.full((4000, 3), -1, dtype=torch.int32, device="cuda")
        d1 = torch.empty((4000, 3), dtype=torch.float32, device="cuda")
        d2 = torch.empty((4000, 3), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        with torch.cuda.stream(s1):
            b1.encode_noalloc(x1, i1, None, d1)
        with torch.cuda.stream(s2):
            b2.encode_noalloc(x2, i2, None, d2)
        torch.cuda.synchronize()
        outs.append([t.cpu().numpy() for t in (i1, d1, i2, d2)])
    w1 = torch.empty((4000, 3), dtype=torch.int32, device="cuda")
    w2 = torch.empty((4000, 3), dtype=torch.int32, device="cuda")
    e1 = torch.empty((4000, 3), dtype=torch.float32, device="cuda")
    e2 = torch.empty((4000, 3), dtype=torch.float32, device="cuda")
    b1.encode(x1, w1, None, e1)
    b2.encode(x2, w2, None, e2)
    torch.cuda.synchronize()
    want = [t.cpu().numpy() for t in (w1, e1, w2, e2)]
    for got in outs:
        for a, b in zip(got, want):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    b1.close(), b2.close(), c1.close(), c2.close()


def test_noalloc_allocates_no_device_memory(torch):
    """A fresh context whose only encodes are no-allocation calls: after a
    first call (which looks up the region), further calls at the same or a
    larger shape leave the device's free memory unchanged."""
    import aqmi
    from aqmi import synth

    print("[gpu] no-alloc leaves free device memory unchanged", flush=True)
    cfg = synth.make_config(2, rows=6000)
    c = aqmi.Context(0)
    cbs = aqmi.Codebooks(c, cfg["codebook"][:2], aqmi.OMNIVOICE)
    x = torch.from_numpy(cfg["x"]).cuda()
    idx = torch.empty((6000, 2), dtype=torch.int32, device="cuda")
    dist = torch.empty((6000, 2), dtype=torch.float32, device="cuda")
    cbs.encode_noalloc(x[:100].contiguous(), idx[:100], None, dist[:100])
    torch.cuda.synchronize()
    xs = [x[:3000].contiguous(), x]
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    for xi in xs:
        cbs.encode_noalloc(xi, idx[: xi.shape[0]], None, dist[: xi.shape[0]])
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0
    cbs.close(), c.close()
