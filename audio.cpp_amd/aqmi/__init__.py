"""Python binding of the MI355X quantizer C ABI (include/aq_mi355x.h).

Loads audio.cpp_amd/libaq_mi355x.so with ctypes.  Device buffers are torch
tensors on the context's device; their data pointers and the current torch
stream are passed straight through the ABI, so torch is only the allocator and
stream provider.  There is no fallback: if the library or a GPU is missing,
construction raises.
"""

from __future__ import annotations

import ctypes as C
import pathlib

import numpy as np

PKG = pathlib.Path(__file__).resolve().parent.parent
LIB_PATH = PKG / "libaq_mi355x.so"

AQ_OK = 0
STATUS_NAMES = {
    0: "AQ_OK", 1: "AQ_E_INVALID_ARG", 2: "AQ_E_SHAPE", 3: "AQ_E_INDEX_RANGE",
    4: "AQ_E_DEVICE", 5: "AQ_E_UNSUPPORTED", 6: "AQ_E_NOMEM",
}

# Every symbol include/aq_mi355x.h declares (checked by the CPU test suite).
EXPORTED = [
    "aq_abi_version", "aq_ctx_create", "aq_ctx_destroy", "aq_ctx_set_stream", "aq_ctx_synchronize",
    "aq_last_error", "aq_dac_upload", "aq_dac_upload_ex", "aq_dac_release", "aq_dac_encode", "aq_dac_decode",
    "aq_euclid_upload", "aq_euclid_release", "aq_euclid_encode", "aq_euclid_failures", "aq_euclid_exact_scans",
    "aq_codebook_gather", "aq_ema_codebook", "aq_euclid_upload_ema",
    "aq_euclid_decode", "aq_ctx_set_timing", "aq_ctx_read_timing",
    "aq_moss_upload", "aq_moss_release", "aq_moss_encode", "aq_moss_decode",
    "aq_euclid_encode_strided", "aq_euclid_upload_projected", "aq_euclid_encode_noalloc",
    "aq_dac_encode_ex", "aq_dac_decode_ex", "aq_euclid_upload_device", "aq_weight_norm_fold",
    "aq_linear_upload", "aq_linear_forward", "aq_linear_release",
]

# aq_euclid_recipe / aq_codebook_type
OMNIVOICE, HIGGS, DIRECT = 0, 1, 2
# aq_dac_recipe
DAC_FISH, DAC_INDEXTTS2, DAC_VEVO2, DAC_OUTETTS = 0, 1, 2, 3
CB_F32, CB_Q8_0, CB_F32_AS_Q8_0 = 0, 1, 2


class AqError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


def load_library(path: str | pathlib.Path | None = None) -> C.CDLL:
    path = pathlib.Path(path) if path else LIB_PATH
    if not path.exists():
        raise FileNotFoundError(f"{path} is not built; run python audio.cpp_amd/build.py")
    lib = C.CDLL(str(path))
    vp, i64 = C.c_void_p, C.c_int64
    lib.aq_abi_version.restype = C.c_int
    lib.aq_ctx_create.argtypes = [C.c_int, vp, C.POINTER(vp)]
    lib.aq_ctx_destroy.argtypes = [vp]
    lib.aq_ctx_set_stream.argtypes = [vp, vp]
    lib.aq_ctx_synchronize.argtypes = [vp]
    lib.aq_last_error.restype = C.c_char_p
    lib.aq_last_error.argtypes = [vp]
    lib.aq_dac_upload.argtypes = [vp, i64, i64, i64, vp, vp, vp, vp, vp, C.POINTER(vp)]
    lib.aq_dac_upload_ex.argtypes = [vp, i64, i64, i64, vp, vp, vp, vp, vp, C.c_int, C.POINTER(vp)]
    lib.aq_dac_release.argtypes = [vp]
    lib.aq_dac_encode.argtypes = [vp, vp, vp, i64, i64, vp, vp, vp, vp]
    lib.aq_dac_decode.argtypes = [vp, vp, vp, i64, vp]
    lib.aq_dac_encode_ex.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, vp, i64, vp, vp, C.c_int, vp]
    lib.aq_dac_decode_ex.argtypes = [vp, vp, vp, i64, i64, vp, C.c_int]
    lib.aq_ctx_set_timing.argtypes = [vp, C.c_int]
    lib.aq_ctx_read_timing.argtypes = [vp, vp, C.c_int, C.POINTER(C.c_int)]
    lib.aq_euclid_upload.argtypes = [vp, i64, i64, i64, C.c_int, vp, C.c_int, C.POINTER(vp)]
    lib.aq_euclid_release.argtypes = [vp]
    lib.aq_euclid_encode.argtypes = [vp, vp, vp, i64, vp, vp, vp, C.c_int, vp, vp, vp]
    lib.aq_euclid_failures.argtypes = [vp, vp, vp]
    lib.aq_euclid_exact_scans.argtypes = [vp, vp, vp]
    lib.aq_codebook_gather.argtypes = [vp, vp, i64, vp, i64, vp]
    lib.aq_ema_codebook.argtypes = [vp, vp, vp, i64, i64, i64, C.c_float, vp]
    lib.aq_euclid_upload_ema.argtypes = [vp, i64, i64, i64, vp, vp, C.c_float, C.c_int, C.POINTER(vp)]
    lib.aq_euclid_upload_device.argtypes = [vp, i64, i64, i64, C.c_int, vp, C.c_int, C.POINTER(vp)]
    lib.aq_weight_norm_fold.argtypes = [vp, vp, vp, i64, i64, C.c_int, vp]
    lib.aq_linear_upload.argtypes = [vp, i64, i64, C.c_int, vp, vp, C.POINTER(vp)]
    lib.aq_linear_forward.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, vp]
    lib.aq_linear_release.argtypes = [vp]
    lib.aq_euclid_decode.argtypes = [vp, vp, vp, i64, vp]
    lib.aq_euclid_encode_noalloc.argtypes = [vp, vp, vp, i64, vp, vp, vp, C.c_int, vp, vp, vp]
    lib.aq_euclid_encode_strided.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, vp, vp, vp, C.c_int, vp, vp, vp]
    lib.aq_euclid_upload_projected.argtypes = [vp, i64, i64, i64, i64, C.c_int, vp, C.c_int, vp, vp, vp, vp,
                                               C.c_int, C.POINTER(vp)]
    lib.aq_moss_upload.argtypes = [vp, i64, i64, i64, i64] + [vp] * 9 + [C.POINTER(vp)]
    lib.aq_moss_release.argtypes = [vp]
    lib.aq_moss_encode.argtypes = [vp, vp, vp, i64, vp, vp, vp]
    lib.aq_moss_decode.argtypes = [vp, vp, vp, i64, vp]
    for name in EXPORTED:
        fn = getattr(lib, name)
        if name not in ("aq_abi_version", "aq_last_error"):
            fn.restype = C.c_int
    return lib


def _host_ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"] and a.dtype == np.float32
    return a.ctypes.data_as(C.c_void_p)


def _dptr(t) -> int | None:
    if t is None:
        return None
    assert t.is_cuda and t.is_contiguous(), "device tensors must be contiguous CUDA/HIP tensors"
    return t.data_ptr()


class Context:
    """aq_ctx on one device, bound to torch's current stream of that device."""

    def __init__(self, device: int = 0, lib: C.CDLL | None = None):
        import torch

        if not torch.cuda.is_available():
            raise RuntimeError("no GPU visible: the MI355X quantizer has no CPU fallback")
        self.torch = torch
        self.lib = lib or load_library()
        self.device = device
        h = C.c_void_p()
        stream = torch.cuda.current_stream(device).cuda_stream
        st = self.lib.aq_ctx_create(device, C.c_void_p(stream), C.byref(h))
        if st != AQ_OK:
            raise AqError(st, "aq_ctx_create failed")
        self.h = h

    def check(self, st: int):
        if st != AQ_OK:
            raise AqError(st, self.lib.aq_last_error(self.h).decode())

    def use_current_stream(self):
        s = self.torch.cuda.current_stream(self.device).cuda_stream
        self.check(self.lib.aq_ctx_set_stream(self.h, C.c_void_p(s)))

    def synchronize(self):
        self.check(self.lib.aq_ctx_synchronize(self.h))

    def set_timing(self, enable: bool):
        self.check(self.lib.aq_ctx_set_timing(self.h, 1 if enable else 0))

    def read_timing(self, capacity: int = 1 << 16) -> np.ndarray:
        """Durations (ms) of the library's main kernels since timing started."""
        buf = np.zeros(capacity, np.float32)
        n = C.c_int()
        self.check(self.lib.aq_ctx_read_timing(self.h, buf.ctypes.data_as(C.c_void_p), capacity, C.byref(n)))
        return buf[: min(n.value, capacity)].copy()

    def close(self):
        if getattr(self, "h", None):
            self.lib.aq_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DacStages:
    """Uploaded DAC RVQ weights (aq_dac_upload_ex).  recipe: DAC_FISH,
    DAC_INDEXTTS2 or DAC_VEVO2 (query / codebook normalisation of the ggml
    graphs), or DAC_OUTETTS (the OuteTTS fp32 host loop); w_out None uploads
    a codes-only single stage."""

    def __init__(self, ctx: Context, w_in, b_in, codebook, w_out, b_out, recipe: int = 0):
        self.ctx = ctx
        w_in = np.ascontiguousarray(w_in, np.float32)
        cb = np.ascontiguousarray(codebook, np.float32)
        w_out = None if w_out is None else np.ascontiguousarray(w_out, np.float32)
        b_in = None if b_in is None else np.ascontiguousarray(b_in, np.float32)
        b_out = None if b_out is None else np.ascontiguousarray(b_out, np.float32)
        self.Q, _, self.D = w_in.shape
        self.N = cb.shape[1]
        self.recipe = recipe
        h = C.c_void_p()
        ctx.check(ctx.lib.aq_dac_upload_ex(ctx.h, self.Q, self.D, self.N, _host_ptr(w_in), _host_ptr(b_in),
                                           _host_ptr(cb), _host_ptr(w_out), _host_ptr(b_out), recipe, C.byref(h)))
        self.h = h

    def encode(self, x, clip_len: int, idx, residual=None, recon=None, force_idx=None):
        M = x.shape[0]
        self.ctx.use_current_stream()
        self.ctx.check(self.ctx.lib.aq_dac_encode(self.ctx.h, self.h, _dptr(x), M, clip_len, _dptr(idx), _dptr(residual),
                                                  _dptr(recon), _dptr(force_idx)))

    def decode(self, idx, out):
        self.ctx.use_current_stream()
        self.ctx.check(self.ctx.lib.aq_dac_decode(self.ctx.h, self.h, _dptr(idx), idx.shape[0], _dptr(out)))

    def encode_ex(self, x, M: int, clip_len: int, strides, idx_ptr: int, idx_ld: int, residual=None, recon=None,
                  recon_accumulate: bool = False, force_ptr: int | None = None):
        """aq_dac_encode_ex: strides = (clip_stride, frame_stride, chan_stride)
        in floats; idx_ptr / force_ptr are device addresses of the first code
        of this stage set (row stride idx_ld)."""
        self.ctx.use_current_stream()
        self.ctx.check(self.ctx.lib.aq_dac_encode_ex(self.ctx.h, self.h, x.data_ptr(), M, clip_len, *strides, idx_ptr,
                                                     idx_ld, _dptr(residual), _dptr(recon),
                                                     1 if recon_accumulate else 0, force_ptr))

    def decode_ex(self, idx_ptr: int, idx_ld: int, M: int, out, accumulate: bool = False):
        self.ctx.use_current_stream()
        self.ctx.check(self.ctx.lib.aq_dac_decode_ex(self.ctx.h, self.h, idx_ptr, idx_ld, M, _dptr(out),
                                                     1 if accumulate else 0))

    def close(self):
        if getattr(self, "h", None):
            self.ctx.lib.aq_dac_release(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class MossQuantizer:
    """MOSS RLFQ quantizer (aq_moss_upload): folded conv weights as the
    reference's constructor builds them; output_w / output_b None = encode
    only.  Shapes: input_w [R, C], input_b [R], in_w [Q, 8, R], in_b [Q, 8],
    codebook [Q, N, 8], out_w [Q, R, 8], out_b [Q, R], output_w [C, R],
    output_b [C]."""

    def __init__(self, ctx: Context, input_w, input_b, in_w, in_b, codebook, out_w, out_b, output_w=None,
                 output_b=None):
        self.ctx = ctx
        f = lambda a: None if a is None else np.ascontiguousarray(a, np.float32)
        arrs = [f(a) for a in (input_w, input_b, in_w, in_b, codebook, out_w, out_b, output_w, output_b)]
        self.R, self.C = arrs[0].shape
        self.Q, self.N = arrs[4].shape[:2]
        h = C.c_void_p()
        ctx.check(ctx.lib.aq_moss_upload(ctx.h, self.Q, self.N, self.C, self.R, *[_host_ptr(a) for a in arrs],
                                         C.byref(h)))
        self.h = h

    def encode(self, hidden, idx, residual=None, force_idx=None):
        """hidden [M, C] f32, idx [M, Q] i32, residual [M, R] f64 (device)."""
        self.ctx.use_current_stream()
        self.ctx.check(self.ctx.lib.aq_moss_encode(self.ctx.h, self.h, _dptr(hidden), hidden.shape[0], _dptr(idx),
                                                   _dptr(residual), _dptr(force_idx)))

    def decode(self, idx, out):
        """idx [M, Q] i32 -> out [M, C] f32 (device)."""
        self.ctx.use_current_stream()
        self.ctx.check(self.ctx.lib.aq_moss_decode(self.ctx.h, self.h, _dptr(idx), idx.shape[0], _dptr(out)))

    def close(self):
        if getattr(self, "h", None):
            self.ctx.lib.aq_moss_release(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Codebooks:
    """Uploaded Euclidean codebooks (aq_euclid_upload).

    codebook: float32 [Q, N, K] (CB_F32, or CB_F32_AS_Q8_0: quantised to
    Q8_0 on the device as the reference's weight store does at load) or a
    structured block_q8_0 array [Q, N, K/32] (CB_Q8_0, dtype
    aqmi.synth.Q8_DTYPE).  recipe: OMNIVOICE, HIGGS or DIRECT."""

    def __init__(self, ctx: Context, codebook, recipe: int, cb_type: int = CB_F32):
        self.ctx = ctx
        if cb_type in (CB_F32, CB_F32_AS_Q8_0):
            cb = np.ascontiguousarray(codebook, np.float32)
            self.Q, self.N, self.K = cb.shape
        else:
            cb = np.ascontiguousarray(codebook)
            assert cb.dtype.itemsize == 34, "Q8_0 blocks are 34 bytes"
            self.Q, self.N, nb = cb.shape
            self.K = nb * 32
        self.recipe = recipe
        self.H = self.K
        h = C.c_void_p()
        ctx.check(ctx.lib.aq_euclid_upload(ctx.h, self.Q, self.N, self.K, cb_type, cb.ctypes.data_as(C.c_void_p),
                                           recipe, C.byref(h)))
        self.h = h

    @classmethod
    def projected(cls, ctx: Context, codebook, w_in, b_in, w_out, b_out, recipe: int, cb_type: int = CB_F32,
                  proj_type: int = CB_F32):
        """aq_euclid_upload_projected: OmniVoice / Higgs stages with
        project_in w_in [Q, K, H] (+ b_in [Q, K]) and project_out w_out
        [Q, H, K] (+ b_out [Q, H]); F32 arrays or block_q8_0 arrays of the
        same rows (proj_type CB_Q8_0).  Encode takes x and residual [M, H]."""
        self = cls.__new__(cls)
        self.ctx = ctx
        if cb_type == CB_F32:
            cb = np.ascontiguousarray(codebook, np.float32)
            self.Q, self.N, self.K = cb.shape
        else:
            cb = np.ascontiguousarray(codebook)
            self.Q, self.N, nb = cb.shape
            self.K = nb * 32
        if proj_type == CB_F32:
            wi = np.ascontiguousarray(w_in, np.float32)
            wo = np.ascontiguousarray(w_out, np.float32)
            self.H = wi.shape[2]
        else:
            wi = np.ascontiguousarray(w_in)
            wo = np.ascontiguousarray(w_out)
            self.H = wi.shape[2] * 32
        bi = None if b_in is None else np.ascontiguousarray(b_in, np.float32)
        bo = None if b_out is None else np.ascontiguousarray(b_out, np.float32)
        self.recipe = recipe
        h = C.c_void_p()
        ctx.check(ctx.lib.aq_euclid_upload_projected(ctx.h, self.Q, self.N, self.K, self.H, cb_type,
                                                     cb.ctypes.data_as(C.c_void_p), proj_type,
                                                     wi.ctypes.data_as(C.c_void_p), _host_ptr(bi),
                                                     wo.ctypes.data_as(C.c_void_p), _host_ptr(bo), recipe,
                                                     C.byref(h)))
        self.h = h
        return self

    @classmethod
    def from_device(cls, ctx: Context, codebook, recipe: int, cb_type: int = CB_F32, shape=None):
        """aq_euclid_upload_device: codebook a device tensor, float32 [Q, N, K]
        (CB_F32) or the raw block_q8_0 bytes (uint8, CB_Q8_0; shape = (Q, N, K))."""
        self = cls.__new__(cls)
        self.ctx = ctx
        if cb_type in (CB_F32, CB_F32_AS_Q8_0):
            self.Q, self.N, self.K = codebook.shape
        else:
            self.Q, self.N, self.K = shape
            assert codebook.numel() == self.Q * self.N * self.K // 32 * 34
        self.recipe = recipe
        self.H = self.K
        h = C.c_void_p()
        ctx.use_current_stream()
        ctx.check(ctx.lib.aq_euclid_upload_device(ctx.h, self.Q, self.N, self.K, cb_type, _dptr(codebook), recipe,
                                                  C.byref(h)))
        self.h = h
        return self

    @classmethod
    def from_ema(cls, ctx: Context, embedding_sum, cluster_usage, recipe: int, eps: float = 1.0e-5):
        """aq_euclid_upload_ema: codebooks materialised from EMA statistics
        (embedding_sum [Q, N, K], cluster_usage [Q, N], host float32)."""
        es = np.ascontiguousarray(embedding_sum, np.float32)
        cu = np.ascontiguousarray(cluster_usage, np.float32)
        self = cls.__new__(cls)
        self.ctx = ctx
        self.Q, self.N, self.K = es.shape
        assert cu.shape == (self.Q, self.N)
        self.recipe = recipe
        self.H = self.K
        h = C.c_void_p()
        ctx.check(ctx.lib.aq_euclid_upload_ema(ctx.h, self.Q, self.N, self.K, es.ctypes.data_as(C.c_void_p),
                                               cu.ctypes.data_as(C.c_void_p), eps, recipe, C.byref(h)))
        self.h = h
        return self


    def encode(self, x, idx, residual=None, dist=None, topk: int = 0, topk_idx=None, topk_dist=None,
               force_idx=None):
        self.ctx.use_current_stream()
        self.ctx.check(self.ctx.lib.aq_euclid_encode(self.ctx.h, self.h, _dptr(x), x.shape[0], _dptr(idx),
                                                     _dptr(residual), _dptr(dist), topk, _dptr(topk_idx),
                                                     _dptr(topk_dist), _dptr(force_idx)))

    def encode_noalloc(self, x, idx, residual=None, dist=None, topk: int = 0, topk_idx=None, topk_dist=None,
                       force_idx=None):
        """aq_euclid_encode_noalloc: the same encode without device allocation."""
        self.ctx.use_current_stream()
        self.ctx.check(self.ctx.lib.aq_euclid_encode_noalloc(self.ctx.h, self.h, _dptr(x), x.shape[0], _dptr(idx),
                                                             _dptr(residual), _dptr(dist), topk, _dptr(topk_idx),
                                                             _dptr(topk_dist), _dptr(force_idx)))

    def encode_strided(self, x, M: int, clip_len: int, clip_stride: int, frame_stride: int, chan_stride: int, idx,
                       residual=None, dist=None, topk: int = 0, topk_idx=None, topk_dist=None, force_idx=None):
        """aq_euclid_encode_strided: x is any device tensor holding frame m,
        channel c at (m // clip_len) * clip_stride + (m % clip_len) *
        frame_stride + c * chan_stride (in floats)."""
        assert x.is_cuda and x.dtype == self.ctx.torch.float32
        self.ctx.use_current_stream()
        self.ctx.check(self.ctx.lib.aq_euclid_encode_strided(
            self.ctx.h, self.h, x.data_ptr(), M, clip_len, clip_stride, frame_stride, chan_stride, _dptr(idx),
            _dptr(residual), _dptr(dist), topk, _dptr(topk_idx), _dptr(topk_dist), _dptr(force_idx)))

    def failures(self) -> np.ndarray:
        """Frames per stage the fp16 certificate left open (refine pass or exact scan)."""
        out = np.zeros(64, np.int32)
        self.ctx.check(self.ctx.lib.aq_euclid_failures(self.ctx.h, self.h, out.ctypes.data_as(C.c_void_p)))
        return out[: min(self.Q, 64)]

    def exact_scans(self) -> np.ndarray:
        """Frames per stage the refine pass left to the exact scan."""
        out = np.zeros(64, np.int32)
        self.ctx.check(self.ctx.lib.aq_euclid_exact_scans(self.ctx.h, self.h, out.ctypes.data_as(C.c_void_p)))
        return out[: min(self.Q, 64)]

    def gather(self, stage: int, idx, out):
        self.ctx.use_current_stream()
        self.ctx.check(self.ctx.lib.aq_codebook_gather(self.ctx.h, self.h, stage, _dptr(idx), idx.shape[0],
                                                       _dptr(out)))

    def decode(self, idx, out):
        self.ctx.use_current_stream()
        self.ctx.check(self.ctx.lib.aq_euclid_decode(self.ctx.h, self.h, _dptr(idx), idx.shape[0], _dptr(out)))

    def close(self):
        if getattr(self, "h", None):
            self.ctx.lib.aq_euclid_release(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Linear:
    """aq_linear: an encoder output Linear with ggml's CPU arithmetic.

    w: float32 [out, in] or block_q8_0 [out, in/32] (host); bias [out] or
    None."""

    def __init__(self, ctx: Context, w, bias=None):
        self.ctx = ctx
        wt = CB_F32 if w.dtype == np.float32 else CB_Q8_0
        w = np.ascontiguousarray(w)
        self.out_features = w.shape[0]
        self.in_features = w.shape[1] * (1 if wt == CB_F32 else 32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        h = C.c_void_p()
        ctx.check(ctx.lib.aq_linear_upload(ctx.h, self.out_features, self.in_features, wt,
                                           w.ctypes.data_as(C.c_void_p), _host_ptr(b), C.byref(h)))
        self.h = h

    def forward(self, x, out, M=None, clip_len=None, strides=None):
        """x device: frame-major [M, in] or any layout given by
        strides = (clip_stride, frame_stride, chan_stride) with clip_len
        frames per clip; out device [M, out]."""
        if strides is None:
            M = x.shape[0]
            clip_len, strides = max(M, 1), (max(M, 1) * self.in_features, self.in_features, 1)
        self.ctx.use_current_stream()
        self.ctx.check(self.ctx.lib.aq_linear_forward(self.ctx.h, self.h, _dptr(x), M, clip_len, *strides, _dptr(out)))

    def close(self):
        if getattr(self, "h", None):
            self.ctx.lib.aq_linear_release(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# aq_wn_rule
WN_OUTETTS, WN_MOSS = 0, 1


def weight_norm_fold(ctx: Context, v, g, rule: int, out):
    """aq_weight_norm_fold on device tensors: v [rows, ...] (the trailing axes
    are one row), g [rows]; out like v (may be v)."""
    rows = v.shape[0]
    ctx.use_current_stream()
    ctx.check(ctx.lib.aq_weight_norm_fold(ctx.h, _dptr(v), _dptr(g), rows, v.numel() // rows, rule, _dptr(out)))


def ema_codebook(ctx: Context, embedding_sum, cluster_usage, eps: float, out):
    """aq_ema_codebook on device tensors: out = embedding_sum / max(usage, eps)."""
    Q, N, K = embedding_sum.shape
    ctx.use_current_stream()
    ctx.check(ctx.lib.aq_ema_codebook(ctx.h, _dptr(embedding_sum), _dptr(cluster_usage), Q, N, K, eps, _dptr(out)))
