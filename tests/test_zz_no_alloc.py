"""aq_euclid_encode_noalloc through the C ABI: its outputs equal
aq_euclid_encode's bit for bit on two calls in a row (the second smaller, so
the shared scratch region holds the first call's contents), with and without
a caller residual buffer, for plain, Q8_0 top-k and projected codebooks; and
a call that needs more than the region fails cleanly."""

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
