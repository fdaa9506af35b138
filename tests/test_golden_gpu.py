"""Full BASELINE sizes on the GPU against the golden fixtures that the
reference's own ggml CPU build wrote (tests/golden/make_golden.py).

Codes are compared index for index, and the fp32 outputs (final residual,
winning logits / distances, top-4 lists) through SHA-256 digests of their
bytes, i.e. bit for bit.  The DAC configs are covered in test_dac_gpu.py.
"""

import hashlib

import numpy as np
import pytest

from conftest import GOLDEN

pytestmark = pytest.mark.gpu


def sha(a):
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


def encode(torch, ctx, cb_host, recipe, x, cb_type=0, topk=0):
    import aqmi

    cbs = aqmi.Codebooks(ctx, cb_host, recipe, cb_type)
    M = x.shape[0]
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    idx = torch.empty((M, cbs.Q), dtype=torch.int32, device="cuda")
    res = torch.empty((M, cbs.K), dtype=torch.float32, device="cuda")
    dist = torch.empty((M, cbs.Q), dtype=torch.float32, device="cuda")
    tki = torch.empty((M, cbs.Q, max(topk, 1)), dtype=torch.int32, device="cuda")
    tkd = torch.empty((M, cbs.Q, max(topk, 1)), dtype=torch.float32, device="cuda")
    cbs.encode(xd, idx, res, dist, topk, tki if topk else None, tkd if topk else None)
    torch.cuda.synchronize()
    out = dict(idx=idx.cpu().numpy(), residual=res.cpu().numpy(), dist=dist.cpu().numpy(),
               fails=cbs.failures())
    if topk:
        out["topk_idx"] = tki.cpu().numpy()
        out["topk_dist"] = tkd.cpu().numpy()
    cbs.close()
    return out


def test_mimi_cfg2_matches_reference(torch, ctx):
    import aqmi
    from aqmi import synth

    print("[gpu] golden mimi configs[2] 48000 x 8 x 2048 x 256", flush=True)
    g = np.load(GOLDEN / "mimi_cfg2.npz")
    cfg = synth.make_config(2)
    out = encode(torch, ctx, cfg["codebook"], aqmi.OMNIVOICE, cfg["x"])
    print(f"[gpu] exact-scan frames per stage {out['fails'].tolist()}", flush=True)
    assert np.array_equal(out["idx"], g["idx"].astype(np.int32))
    assert sha(out["residual"]) == str(g["residual_sha"])
    assert sha(-out["dist"]) == str(g["logit_sha"])


def test_kmeans_cfg3_matches_reference(torch, ctx):
    import aqmi
    from aqmi import synth

    print("[gpu] golden k-means configs[3] 200000 x 16384 x 768", flush=True)
    g = np.load(GOLDEN / "kmeans_cfg3.npz")
    cfg = synth.make_config(3)
    out = encode(torch, ctx, cfg["codebook"], aqmi.HIGGS, cfg["x"])
    print(f"[gpu] exact-scan frames {out['fails'].tolist()}", flush=True)
    assert np.array_equal(out["idx"][:, 0], g["idx"].astype(np.int32))
    assert sha(out["dist"]) == str(g["dist_sha"])


def test_q8_cfg4_matches_reference(torch, ctx):
    import aqmi
    from aqmi import synth

    print("[gpu] golden q8_0 configs[4] 48000 x 8 x 2048 x 256, top-4", flush=True)
    g = np.load(GOLDEN / "q8_cfg4.npz")
    cfg = synth.make_config(4)
    out = encode(torch, ctx, cfg["codebook_q8"], aqmi.HIGGS, cfg["x"], cb_type=aqmi.CB_Q8_0, topk=4)
    print(f"[gpu] exact-scan frames per stage {out['fails'].tolist()}", flush=True)
    assert np.array_equal(out["idx"], g["idx"].astype(np.int32))
    assert sha(out["residual"]) == str(g["residual_sha"])
    assert sha(out["dist"]) == str(g["dist_sha"])
    logit = -out["topk_dist"]
    order = np.lexsort((out["topk_idx"], -logit.astype(np.float64)), axis=-1)
    ti = np.take_along_axis(out["topk_idx"], order, -1)
    tl = np.take_along_axis(logit, order, -1)
    assert sha(ti.astype(np.int32)) == str(g["topk_idx_sha"])
    assert sha(tl) == str(g["topk_logit_sha"])
