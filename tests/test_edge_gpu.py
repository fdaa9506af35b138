"""Empty and ragged batches through the C ABI on the GPU.

An empty batch (M = 0) enqueues nothing and returns AQ_OK, whatever its data
pointers hold (torch hands out null pointers for empty tensors), as the
reference's VectorQuantizer::compute returns an empty result for batch = 0
(src/framework/runtime/host_ops.cpp:236-273).  MOSS is the exception: its
quantizer rejects an empty latent with the reference's message
(audio_tokenizer_quantizer.cpp).  A clip layout that does not tile M, and M
past the 32-bit frame range, are shape errors raised before any launch."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

AQ_E_SHAPE = 2


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


def empty(torch, *shape, dtype=None):
    return torch.empty(shape, dtype=dtype or torch.float32, device="cuda")


@pytest.mark.parametrize("cb_type", [0, 1])
def test_euclid_empty_batch(torch, ctx, cb_type):
    import aqmi
    from aqmi import synth

    print(f"[gpu] euclid empty batch, cb_type {cb_type}", flush=True)
    cfg = synth.make_config(2, rows=64)
    Q, N, K = 3, 2048, 256
    if cb_type:
        cb = np.stack([synth.q8_0_random_codebook(81, 10 + s, N, K) for s in range(Q)])
    else:
        cb = np.ascontiguousarray(cfg["codebook"][:Q])
    cbs = aqmi.Codebooks(ctx, cb, aqmi.HIGGS, cb_type)
    x = empty(torch, 0, K)
    idx = empty(torch, 0, Q, dtype=torch.int32)
    cbs.encode(x, idx, empty(torch, 0, K), empty(torch, 0, Q), 4, empty(torch, 0, Q, 4, dtype=torch.int32),
               empty(torch, 0, Q, 4))
    cbs.encode(x, idx)
    cbs.encode_noalloc(x, idx, topk=2)   # top-k outputs absent: nothing to write
    cbs.decode(idx, empty(torch, 0, K))
    cbs.gather(1, empty(torch, 0, dtype=torch.int32), empty(torch, 0, K))
    # a non-empty batch still runs on the same context afterwards
    xs = torch.from_numpy(np.ascontiguousarray(cfg["x"][:64])).cuda()
    got = torch.full((64, Q), -1, dtype=torch.int32, device="cuda")
    cbs.encode(xs, got)
    torch.cuda.synchronize()
    assert int(got.min()) >= 0 and int(got.max()) < N


def test_euclid_batch_past_frame_range(torch, ctx):
    import aqmi
    from aqmi import synth

    print("[gpu] euclid M past 2^31 - 1", flush=True)
    cfg = synth.make_config(2, rows=64)
    cbs = aqmi.Codebooks(ctx, np.ascontiguousarray(cfg["codebook"][:1]), aqmi.OMNIVOICE)
    x = torch.from_numpy(np.ascontiguousarray(cfg["x"][:64])).cuda()
    idx = torch.empty((64, 1), dtype=torch.int32, device="cuda")
    st = ctx.lib.aq_euclid_encode(ctx.h, cbs.h, x.data_ptr(), 1 << 31, idx.data_ptr(), None, None, 0, None, None,
                                  None)
    assert st == AQ_E_SHAPE


def test_dac_empty_and_ragged_batches(torch, ctx):
    import aqmi
    from aqmi import synth

    print("[gpu] dac empty and ragged batches", flush=True)
    cfg = synth.make_config(0)
    st = aqmi.DacStages(ctx, cfg["w_in"], cfg.get("b_in"), cfg["codebook"], cfg["w_out"], cfg.get("b_out"))
    D, Q = cfg["D"], cfg["Q"]
    st.encode(empty(torch, 0, D), 4, empty(torch, 0, Q, dtype=torch.int32), empty(torch, 0, D), empty(torch, 0, D))
    st.decode(empty(torch, 0, Q, dtype=torch.int32), empty(torch, 0, D))
    x = torch.zeros((6, D), dtype=torch.float32, device="cuda")
    idx = torch.empty((6, Q), dtype=torch.int32, device="cuda")
    with pytest.raises(aqmi.AqError) as e:
        st.encode(x, 4, idx)   # 6 frames are not whole clips of 4
    assert e.value.status == AQ_E_SHAPE
    st.encode(x, 3, idx)
    torch.cuda.synchronize()
    assert int(idx.min()) >= 0


def test_projected_and_linear_empty_batch(torch, ctx):
    import aqmi
    from aqmi import synth

    print("[gpu] projected cascade and encoder Linear, empty batch", flush=True)
    cfg = synth.projected_config(8, Q=2)
    cbs = aqmi.Codebooks.projected(ctx, cfg["codebook"], cfg["w_in"], cfg.get("b_in"), cfg["w_out"], cfg.get("b_out"),
                                   cfg["recipe"])
    H = cfg["w_in"].shape[-1]
    cbs.encode(empty(torch, 0, H), empty(torch, 0, 2, dtype=torch.int32))
    cbs.encode_strided(empty(torch, 0), 0, 1, H, H, 1, empty(torch, 0, 2, dtype=torch.int32))
    rng = np.random.default_rng(5)
    lin = aqmi.Linear(ctx, rng.standard_normal((64, 128)).astype(np.float32))
    lin.forward(empty(torch, 0, 128), empty(torch, 0, 64))
    torch.cuda.synchronize()


def test_moss_rejects_empty_latent(torch, ctx):
    import aqmi
    from aqmi import synth

    print("[gpu] moss empty latent", flush=True)
    cfg = synth.moss_config(4, Q=2, N=64, C=32, R=64)
    f = synth.moss_fold(cfg)
    q = aqmi.MossQuantizer(ctx, f["w_ip"], cfg["ip_b"], f["w_in"], cfg["in_b"], cfg["codebook"], f["w_out"],
                           cfg["out_b"], f["w_op"], cfg["op_b"])
    with pytest.raises(aqmi.AqError) as e:
        q.encode(empty(torch, 0, 32), empty(torch, 0, 2, dtype=torch.int32))
    assert e.value.status == AQ_E_SHAPE
    assert "MOSS codec quantizer requires a non-empty encoder latent" in str(e.value)
    with pytest.raises(aqmi.AqError) as e:
        q.decode(empty(torch, 0, 2, dtype=torch.int32), empty(torch, 0, 32))
    assert "requires a non-empty code sequence" in str(e.value)


def test_handles_outlive_their_context(torch):
    """Handles released after the context that created them (as Python's
    collector may order it): no handle reads its creator, so the releases
    leave no HIP error behind, and a new context uploads and encodes."""
    import aqmi
    from aqmi import synth

    print("[gpu] handles released after their context", flush=True)
    c = aqmi.Context(0)
    cfg = synth.make_config(2, rows=64)
    cbs = aqmi.Codebooks(c, np.ascontiguousarray(cfg["codebook"][:2]), aqmi.OMNIVOICE)
    d0 = synth.make_config(0)
    st = aqmi.DacStages(c, d0["w_in"], d0.get("b_in"), d0["codebook"], d0["w_out"], d0.get("b_out"))
    mc = synth.moss_config(4, Q=2, N=64, C=32, R=64)
    f = synth.moss_fold(mc)
    q = aqmi.MossQuantizer(c, f["w_ip"], mc["ip_b"], f["w_in"], mc["in_b"], mc["codebook"], f["w_out"], mc["out_b"])
    lin = aqmi.Linear(c, np.ones((64, 64), np.float32))
    torch.cuda.synchronize()
    c.close()
    for h in (cbs, st, q, lin):
        h.close()
    c2 = aqmi.Context(0)
    again = aqmi.Codebooks(c2, np.ascontiguousarray(cfg["codebook"][:2]), aqmi.OMNIVOICE)
    x = torch.from_numpy(np.ascontiguousarray(cfg["x"])).cuda()
    idx = torch.full((64, 2), -1, dtype=torch.int32, device="cuda")
    again.encode(x, idx)
    torch.cuda.synchronize()
    assert int(idx.min()) >= 0
    again.close()
    c2.close()


def test_foreign_sticky_error_is_not_ours(torch, ctx):
    """A HIP error that the caller's own code left in the thread's last-error
    slot (here hipSetDevice on a device that does not exist) does not make
    the next upload or encode fail: the library's launch checks see only
    its own calls."""
    import ctypes
    import aqmi
    from aqmi import synth

    print("[gpu] foreign sticky HIP error", flush=True)
    hip = ctypes.CDLL("libamdhip64.so")
    cur = ctypes.c_int(-1)
    assert hip.hipGetDevice(ctypes.byref(cur)) == 0
    torch.cuda.synchronize()
    assert hip.hipSetDevice(ctypes.c_int(4096)) != 0   # invalid device ordinal, left unread
    cfg = synth.make_config(2, rows=64)
    cbs = aqmi.Codebooks(ctx, np.ascontiguousarray(cfg["codebook"][:2]), aqmi.OMNIVOICE)
    x = torch.from_numpy(np.ascontiguousarray(cfg["x"])).cuda()   # (torch's own launch checks read the slot)
    idx = torch.full((64, 2), -1, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    assert hip.hipSetDevice(ctypes.c_int(4096)) != 0
    cbs.encode(x, idx)
    torch.cuda.synchronize()
    assert int(idx.min()) >= 0
    assert hip.hipGetDevice(ctypes.byref(cur)) == 0 and cur.value == 0
