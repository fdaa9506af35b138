"""The Euclidean encode captured in a HIP graph (torch.cuda.graph over the
context's stream) and replayed: every replay, with eager encodes of other
inputs and synchronisations between the replays, gives the eager result
bit for bit.  The encode enqueues kernels only (its counters are cleared by
a kernel, not a memset node), once the context's scratch has grown to the
shape in an eager call.  Covers the few-open-frames path (the exact scan
takes the frames directly), the split-fp16 refine pass and Q8_0 top-4."""

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


def buffers(torch, M, Q, K, topk):
    dev = dict(device="cuda")
    return dict(idx=torch.full((M, Q), -1, dtype=torch.int32, **dev),
                res=torch.empty((M, K), dtype=torch.float32, **dev),
                dist=torch.empty((M, Q), dtype=torch.float32, **dev),
                tki=torch.empty((M, Q, max(topk, 1)), dtype=torch.int32, **dev),
                tkd=torch.empty((M, Q, max(topk, 1)), dtype=torch.float32, **dev))


def encode(cbs, x, b, topk):
    cbs.encode(x, b["idx"], b["res"], b["dist"], topk, b["tki"] if topk else None, b["tkd"] if topk else None)


def snapshot(b, topk):
    keys = ["idx", "res", "dist"] + (["tki", "tkd"] if topk else [])
    return [b[k].cpu().numpy().view(np.uint32) if b[k].dtype != b["idx"].dtype else b[k].cpu().numpy() for k in keys]


def check_graph(torch, cbs, x, x_other, topk):
    M, K = x.shape
    b = buffers(torch, M, cbs.Q, K, topk)
    encode(cbs, x, b, topk)                  # eager: grows the scratch, the expected result
    torch.cuda.synchronize()
    want = snapshot(b, topk)
    other = buffers(torch, M, cbs.Q, K, topk)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            encode(cbs, x, b, topk)
    torch.cuda.synchronize()
    cbs.ctx.use_current_stream()
    for rep in range(3):
        for t in b.values():
            t.fill_(-7)
        encode(cbs, x_other, other, topk)    # eager work on the same scratch between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = snapshot(b, topk)
        for w, o in zip(want, got):
            assert np.array_equal(w, o), f"replay {rep}"
    cbs.ctx.use_current_stream()


def test_graph_replays_plain_cascade(torch, ctx):
    import aqmi
    from aqmi import synth

    print("[gpu] graph capture: plain cascade", flush=True)
    cfg = synth.make_config(2, rows=4000)
    cb = np.ascontiguousarray(cfg["codebook"][:3])
    cbs = aqmi.Codebooks(ctx, cb, aqmi.OMNIVOICE)
    x = torch.from_numpy(cfg["x"]).cuda()
    check_graph(torch, cbs, x, x.flip(0).contiguous(), 0)


def test_graph_replays_refine_pass(torch, ctx):
    """Near-duplicate code groups leave every frame open (the refine pass)."""
    import aqmi
    from aqmi import synth

    print("[gpu] graph capture: refine pass", flush=True)
    cfg = synth.make_config(2, rows=400)
    cb = np.ascontiguousarray(cfg["codebook"][:2])
    Qn, N, K = cb.shape
    g = cb.reshape(Qn, N // 128, 8, 16, K)
    scale = (1.0 + np.arange(8, dtype=np.float32) * np.float32(2.0 ** -13))[None, None, :, None, None]
    g[:] = (g[:, :, :1] * scale + synth.normal(72, 1, g.shape, 2.0 ** -20)).astype(np.float32)
    cb = np.ascontiguousarray(g.reshape(Qn, N, K))
    cbs = aqmi.Codebooks(ctx, cb, aqmi.HIGGS)
    x = torch.from_numpy(cfg["x"]).cuda()
    check_graph(torch, cbs, x, x.flip(0).contiguous(), 0)
    assert (cbs.failures() > 64).all()


def test_graph_replays_q8_topk(torch, ctx):
    import aqmi
    from aqmi import synth

    print("[gpu] graph capture: Q8_0 top-4", flush=True)
    Q, N, K, M = 3, 2048, 256, 2000
    cb = np.stack([synth.q8_0_random_codebook(81, 10 + s, N, K) for s in range(Q)])
    xh = (synth.q8_0_dequantize(cb[0])[np.arange(M) % N] + synth.normal(81, 2, (M, K), 0.05)).astype(np.float32)
    cbs = aqmi.Codebooks(ctx, cb, aqmi.HIGGS, aqmi.CB_Q8_0)
    x = torch.from_numpy(xh).cuda()
    check_graph(torch, cbs, x, x.flip(0).contiguous(), 4)
