"""Oracle for the quantizer path -- TEST INFRASTRUCTURE ONLY.

`Oracle` wraps liboracle.so (the plain-C restatement in aq_oracle.c).
`Ref` wraps oracle/_ref/libaqref-<isa>.so (the reference's own ggml CPU
backend compiled from /root/reference by oracle/Makefile, plus
ref_harness.cpp).  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this package, and only as the checker or the
labelled CPU baseline -- the product path never does.
"""

from __future__ import annotations

import ctypes as C
import os
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
# AQ_REF_DIR selects another directory of builds (the sanitizer build of
# tests/test_sanitizers.py)
REF_DIR = pathlib.Path(os.environ.get("AQ_REF_DIR") or HERE / "_ref")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i64 = C.c_int64


def _opt(a, dtype):
    if a is None:
        return None
    a = np.ascontiguousarray(a, dtype=dtype)
    return a.ctypes.data_as(C.c_void_p)


def build_oracle() -> pathlib.Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return HERE / "liboracle.so"


def host_isa() -> str:
    """Best _ref variant this CPU can run: native (only where it was built),
    else v4 (AVX-512) or v3 (AVX2)."""
    flags = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("flags"):
                flags = line
                break
    except OSError:
        pass
    if " avx512f " in flags and " avx512bw " in flags and " avx512vl " in flags:
        return "v4"
    return "v3"


class Oracle:
    def __init__(self, path: str | os.PathLike | None = None):
        # AQ_ORACLE_LIB selects another build of the same source (the
        # sanitizer build of tests/test_sanitizers.py)
        path = pathlib.Path(path or os.environ.get("AQ_ORACLE_LIB") or HERE / "liboracle.so")
        if not path.exists():
            build_oracle()
        self.lib = C.CDLL(str(path))
        L = self.lib
        L.aqo_vec_dot_f32.restype = C.c_float
        L.aqo_vec_dot_f32.argtypes = [C.c_int, _f32p, _f32p]
        L.aqo_vec_dot_f32_tail.restype = C.c_float
        L.aqo_vec_dot_f32_tail.argtypes = [C.c_int, _f32p, _f32p, C.c_int]
        L.aqo_tinyblas_dot_f32.restype = C.c_float
        L.aqo_tinyblas_dot_f32.argtypes = [C.c_int, _f32p, _f32p]
        L.aqo_argmax_f32.restype = C.c_int
        L.aqo_argmax_f32.argtypes = [C.c_int, _f32p]
        L.aqo_sum_f32.restype = C.c_float
        L.aqo_sum_f32.argtypes = [C.c_int, _f32p]
        L.aqo_fp32_to_fp16.restype = C.c_uint16
        L.aqo_fp32_to_fp16.argtypes = [C.c_float]
        L.aqo_fp16_to_fp32.restype = C.c_float
        L.aqo_fp16_to_fp32.argtypes = [C.c_uint16]
        L.aqo_quantize_row_q8_0_x86.argtypes = [_f32p, C.c_void_p, C.c_int]
        L.aqo_quantize_row_q8_0_ref.argtypes = [_f32p, C.c_void_p, C.c_int]
        L.aqo_dequantize_row_q8_0.argtypes = [C.c_void_p, _f32p, C.c_int]
        L.aqo_dot_q8_0.restype = C.c_float
        L.aqo_dot_q8_0.argtypes = [C.c_int, C.c_void_p, C.c_void_p]
        L.aqo_dac_rvq.restype = C.c_int
        L.aqo_dac_rvq.argtypes = [_f32p, _i64, _i64, _i64, _i64, _i64, _f32p, C.c_void_p, _f32p, _f32p,
                                  C.c_void_p, C.c_void_p, _i32p, _f32p, C.c_void_p]
        L.aqo_dac_rvq_ex.restype = C.c_int
        L.aqo_dac_rvq_ex.argtypes = [_f32p, _i64, _i64, _i64, _i64, _i64, _f32p, C.c_void_p, _f32p, C.c_void_p,
                                     C.c_void_p, C.c_void_p, _i32p, _f32p, C.c_void_p, C.c_int]
        L.aqo_euclid_rvq.restype = C.c_int
        L.aqo_euclid_rvq.argtypes = [_f32p, _i64, _i64, _i64, _i64, _f32p, C.c_void_p, _i32p, _f32p, C.c_void_p]
        L.aqo_higgs_rvq.restype = C.c_int
        L.aqo_top_k_f32.restype = None
        L.aqo_top_k_f32.argtypes = [_f32p, _i64, C.c_int, _i32p]
        L.aqo_higgs_rvq.argtypes = [_f32p, _i64, _i64, _i64, _i64, C.c_void_p, C.c_int, C.c_int, C.c_void_p,
                                    _i32p, _f32p, C.c_void_p, C.c_void_p, C.c_void_p]
        L.aqo_direct_rvq.restype = C.c_int
        L.aqo_direct_rvq.argtypes = [_f32p, _i64, _i64, _i64, _i64, _f32p, C.c_void_p, _i32p, _f32p, C.c_void_p]
        L.aqo_gather_f32.restype = C.c_int
        L.aqo_gather_f32.argtypes = [_f32p, _i64, _i64, _i32p, _i64, _f32p]
        L.aqo_gather_q8_0.restype = C.c_int
        L.aqo_gather_q8_0.argtypes = [C.c_void_p, _i64, _i64, _i32p, _i64, _f32p]
        L.aqo_ema_codebook.restype = C.c_int
        L.aqo_ema_codebook.argtypes = [_f32p, _f32p, _i64, _i64, _i64, C.c_float, _f32p]
        L.aqo_outetts_rvq.argtypes = [_f32p, _i64, _i64, _i64, _i64, _f32p, C.c_void_p, _f32p, _f32p,
                                      C.c_void_p, C.c_void_p, _i32p, _f32p]
        L.aqo_linear.restype = C.c_int
        L.aqo_linear.argtypes = [C.c_void_p, C.c_int, C.c_void_p, _i64, _i64, _i64, _f32p, _f32p]
        L.aqo_outetts_weight_norm.restype = None
        L.aqo_outetts_weight_norm.argtypes = [_f32p, _f32p, _i64, _i64, _f32p]
        L.aqo_moss_weight_norm.restype = None
        L.aqo_moss_weight_norm.argtypes = [_f32p, _f32p, _i64, _i64, _f32p]
        L.aqo_moss_normalize_rows.restype = None
        L.aqo_moss_normalize_rows.argtypes = [_f32p, _i64, _i64, _f32p]
        L.aqo_moss_rvq.argtypes = [_f32p, _i64, _i64, _i64, _i64, _i64, _f32p, _f32p, _f32p, _f32p, _f32p,
                                   _f32p, _f32p, C.c_void_p, _i32p, C.c_void_p]
        L.aqo_dac_rvq_mixed.argtypes = [_f32p, _i64, _i64, _i64, _i64, _i64, _i64, _f32p, C.c_void_p, _f32p, _f32p,
                                        _f32p, C.c_void_p, C.c_void_p, _i32p, _f32p, _f32p]
        L.aqo_projected_rvq.argtypes = [_f32p, _i64, _i64, _i64, _i64, _i64, C.c_int, C.c_void_p, C.c_int,
                                        C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                                        C.c_void_p, _i32p, _f32p, C.c_void_p, C.c_void_p, C.c_void_p]
        L.aqo_projected_decode.argtypes = [_i32p, _i64, _i64, _i64, _i64, _i64, C.c_void_p, C.c_int, C.c_void_p,
                                           C.c_void_p, C.c_int, _f32p]
        L.aqo_moss_decode.argtypes = [_i32p, _i64, _i64, _i64, _i64, _i64, _f32p, _f32p, _f32p, _f32p, _f32p,
                                      _f32p]

    # -- whole path --------------------------------------------------------
    def dac_rvq(self, cfg: dict, force_idx=None, recon: bool = True, recipe: int = 0):
        """recipe 0 Fish, 1 IndexTTS2, 2 Vevo2; cfg["w_out"] None: codes only."""
        x = np.ascontiguousarray(cfg["x"], np.float32)
        B, T, D, Q, N = cfg["B"], cfg["T"], cfg["D"], cfg["Q"], cfg["N"]
        M = x.shape[0]
        assert M % T == 0
        B = M // T
        idx = np.zeros((M, Q), np.int32)
        res = np.zeros((M, D), np.float32)
        rec = np.zeros((M, D), np.float32) if recon else None
        fi = np.ascontiguousarray(force_idx, np.int32) if force_idx is not None else None
        rc = self.lib.aqo_dac_rvq_ex(x, B, T, D, Q, N, np.ascontiguousarray(cfg["w_in"], np.float32),
                                     _opt(cfg.get("b_in"), np.float32), np.ascontiguousarray(cfg["codebook"], np.float32),
                                     _opt(cfg.get("w_out"), np.float32), _opt(cfg.get("b_out"), np.float32),
                                     None if fi is None else fi.ctypes.data_as(C.c_void_p), idx, res,
                                     None if rec is None else rec.ctypes.data_as(C.c_void_p), recipe)
        if rc == -2:
            raise ValueError("the recipe rejects a zero codebook row")
        assert rc == 0
        return dict(idx=idx, residual=res, recon=rec)

    def dac_rvq_mixed(self, cfg: dict, force_idx=None):
        """The Fish cascade with a semantic stage of N0 codes (fish_config)."""
        x = np.ascontiguousarray(cfg["x"], np.float32)
        M, D = x.shape
        Q = cfg["Q"]
        idx = np.zeros((M, Q), np.int32)
        res = np.zeros((M, D), np.float32)
        rec = np.zeros((M, D), np.float32)
        fi = np.ascontiguousarray(force_idx, np.int32) if force_idx is not None else None
        rc = self.lib.aqo_dac_rvq_mixed(x, M // cfg["T"], cfg["T"], D, Q, cfg["N0"], cfg["N"],
                                        np.ascontiguousarray(cfg["w_in"], np.float32), _opt(cfg.get("b_in"), np.float32),
                                        np.ascontiguousarray(cfg["codebook0"], np.float32),
                                        np.ascontiguousarray(cfg["codebook"], np.float32),
                                        np.ascontiguousarray(cfg["w_out"], np.float32), _opt(cfg.get("b_out"), np.float32),
                                        None if fi is None else fi.ctypes.data_as(C.c_void_p), idx, res, rec)
        assert rc == 0
        return dict(idx=idx, residual=res, recon=rec)

    def euclid_rvq(self, cfg: dict, force_idx=None):
        x = np.ascontiguousarray(cfg["x"], np.float32)
        M, K = x.shape
        Q, N = cfg["Q"], cfg["N"]
        idx = np.zeros((M, Q), np.int32)
        res = np.zeros((M, K), np.float32)
        lb = np.zeros((M, Q), np.float32)
        fi = np.ascontiguousarray(force_idx, np.int32) if force_idx is not None else None
        rc = self.lib.aqo_euclid_rvq(x, M, K, Q, N, np.ascontiguousarray(cfg["codebook"], np.float32),
                                     None if fi is None else fi.ctypes.data_as(C.c_void_p), idx, res,
                                     lb.ctypes.data_as(C.c_void_p))
        assert rc == 0
        return dict(idx=idx, residual=res, logit=lb)

    def direct_rvq(self, cfg: dict, force_idx=None):
        x = np.ascontiguousarray(cfg["x"], np.float32)
        M, K = x.shape
        Q, N = cfg["Q"], cfg["N"]
        idx = np.zeros((M, Q), np.int32)
        res = np.zeros((M, K), np.float32)
        dist = np.zeros((M, Q), np.float32)
        fi = np.ascontiguousarray(force_idx, np.int32) if force_idx is not None else None
        rc = self.lib.aqo_direct_rvq(x, M, K, Q, N, np.ascontiguousarray(cfg["codebook"], np.float32),
                                     None if fi is None else fi.ctypes.data_as(C.c_void_p), idx, res,
                                     dist.ctypes.data_as(C.c_void_p))
        assert rc == 0
        return dict(idx=idx, residual=res, dist=dist)

    def outetts_rvq(self, cfg: dict, force_idx=None):
        """OuteTTS quantize_reference generalised to Q stages; codes and the
        residual after the last stage."""
        x = np.ascontiguousarray(cfg["x"], np.float32)
        M, D = x.shape
        Q, N = cfg["Q"], cfg["N"]
        idx = np.zeros((M, Q), np.int32)
        res = np.zeros((M, D), np.float32)
        fi = np.ascontiguousarray(force_idx, np.int32) if force_idx is not None else None
        rc = self.lib.aqo_outetts_rvq(x, M, D, Q, N, np.ascontiguousarray(cfg["w_in"], np.float32),
                                      _opt(cfg.get("b_in"), np.float32), np.ascontiguousarray(cfg["codebook"], np.float32),
                                      np.ascontiguousarray(cfg["w_out"], np.float32), _opt(cfg.get("b_out"), np.float32),
                                      None if fi is None else fi.ctypes.data_as(C.c_void_p), idx, res)
        assert rc == 0
        return dict(idx=idx, residual=res)

    def outetts_weight_norm(self, v, g):
        """fold_weight_norm: v [rows, ...] (trailing axes one row), g [rows]."""
        v = np.ascontiguousarray(v, np.float32)
        g = np.ascontiguousarray(g, np.float32).reshape(-1)
        w = np.zeros_like(v)
        self.lib.aqo_outetts_weight_norm(v, g, v.shape[0], v.size // v.shape[0], w)
        return w

    def moss_weight_norm(self, g, v):
        """reconstruct_weight_norm over the last two axes of v ([..., out, in])."""
        v = np.ascontiguousarray(v, np.float32)
        g = np.ascontiguousarray(g, np.float32)
        out_ch, in_ch = v.shape[-2:]
        lead = int(np.prod(v.shape[:-2], dtype=np.int64))
        w = np.zeros_like(v)
        vf, gf, wf = v.reshape(lead, out_ch, in_ch), g.reshape(lead, out_ch), w.reshape(lead, out_ch, in_ch)
        for i in range(lead):
            gi, vi, wi = np.ascontiguousarray(gf[i]), np.ascontiguousarray(vf[i]), np.zeros((out_ch, in_ch), np.float32)
            self.lib.aqo_moss_weight_norm(gi, vi, out_ch, in_ch, wi)
            wf[i] = wi
        return w

    def moss_fold(self, cfg: dict) -> dict:
        """The folded conv weights the MOSS constructor builds from (g, v)."""
        return dict(w_ip=self.moss_weight_norm(cfg["ip_g"], cfg["ip_v"]),
                    w_in=self.moss_weight_norm(cfg["in_g"], cfg["in_v"]),
                    w_out=self.moss_weight_norm(cfg["out_g"], cfg["out_v"]),
                    w_op=self.moss_weight_norm(cfg["op_g"], cfg["op_v"]))

    def moss_rvq(self, cfg: dict, force_idx=None, folded: dict | None = None):
        """MOSS encode: codes [M, Q] and the fp64 residual [M, R]."""
        f = folded or self.moss_fold(cfg)
        h = np.ascontiguousarray(cfg["hidden"], np.float32)
        M, Cd = h.shape
        R, Q, N = cfg["R"], cfg["Q"], cfg["N"]
        idx = np.zeros((M, Q), np.int32)
        res = np.zeros((M, R), np.float64)
        fi = np.ascontiguousarray(force_idx, np.int32) if force_idx is not None else None
        a = lambda k: np.ascontiguousarray(cfg[k], np.float32)
        rc = self.lib.aqo_moss_rvq(h, M, Cd, R, Q, N, f["w_ip"], a("ip_b"), f["w_in"], a("in_b"), a("codebook"),
                                   f["w_out"], a("out_b"), None if fi is None else fi.ctypes.data_as(C.c_void_p),
                                   idx, res.ctypes.data_as(C.c_void_p))
        assert rc == 0
        return dict(idx=idx, residual=res)

    def moss_decode(self, cfg: dict, idx, folded: dict | None = None):
        """MOSS dequantisation, frame-major latent [M, C]."""
        f = folded or self.moss_fold(cfg)
        idx = np.ascontiguousarray(idx, np.int32)
        M = idx.shape[0]
        Cd, R, Q, N = cfg["C"], cfg["R"], cfg["Q"], cfg["N"]
        out = np.zeros((M, Cd), np.float32)
        a = lambda k: np.ascontiguousarray(cfg[k], np.float32)
        rc = self.lib.aqo_moss_decode(idx, M, Cd, R, Q, N, a("codebook"), f["w_out"], a("out_b"), f["w_op"],
                                      a("op_b"), out)
        if rc == -1:
            raise IndexError("MOSS codec code index out of range")
        assert rc == 0
        return out

    def ema_codebook(self, embedding_sum, cluster_usage, eps: float = 1.0e-5):
        """codebook_embedding: sum / std::max(usage, eps), per stage [Q, N, K]."""
        es = np.ascontiguousarray(embedding_sum, np.float32)
        cu = np.ascontiguousarray(cluster_usage, np.float32)
        Q, N, K = es.shape
        assert cu.shape == (Q, N)
        out = np.zeros_like(es)
        assert self.lib.aqo_ema_codebook(es, cu, Q, N, K, eps, out) == 0
        return out

    def qwen3_quantize(self, cfg: dict):
        """The Qwen3 cascade from the oracle's parts: EMA codebooks, then the
        DIRECT recipe on the semantic latent (stage 0) and on the acoustic
        latent (stages 1..15), both read channel-major.  Codes [frames, 16]."""
        cb = self.ema_codebook(cfg["embedding_sum"], cfg["cluster_usage"], 1.0e-5)
        F, K, N = cfg["frames"], cfg["K"], cfg["N"]
        sem = self.direct_rvq(dict(x=np.ascontiguousarray(cfg["semantic"].T), M=F, K=K, Q=1, N=N, codebook=cb[:1]))
        ac = self.direct_rvq(dict(x=np.ascontiguousarray(cfg["acoustic"].T), M=F, K=K, Q=cfg["S"] - 1, N=N,
                                  codebook=cb[1:]))
        return np.concatenate([sem["idx"], ac["idx"]], axis=1)

    def top_k(self, v, k: int):
        """aqo_top_k_f32 over the rows of v."""
        v = np.ascontiguousarray(v, np.float32)
        out = np.zeros((v.shape[0], k), np.int32)
        for r in range(v.shape[0]):
            self.lib.aqo_top_k_f32(v[r], v.shape[1], k, out[r])
        return out

    def higgs_rvq(self, cfg: dict, force_idx=None, topk: int = 0):
        x = np.ascontiguousarray(cfg["x"], np.float32)
        M, K = x.shape
        Q, N = cfg["Q"], cfg["N"]
        if "codebook_q8" in cfg:
            cb = np.ascontiguousarray(cfg["codebook_q8"])
            cbt = 1
        else:
            cb = np.ascontiguousarray(cfg["codebook"], np.float32)
            cbt = 0
        idx = np.zeros((M, Q), np.int32)
        res = np.zeros((M, K), np.float32)
        dist = np.zeros((M, Q), np.float32)
        tki = np.zeros((M, Q, max(topk, 1)), np.int32)
        tkl = np.zeros((M, Q, max(topk, 1)), np.float32)
        fi = np.ascontiguousarray(force_idx, np.int32) if force_idx is not None else None
        rc = self.lib.aqo_higgs_rvq(x, M, K, Q, N, cb.ctypes.data_as(C.c_void_p), cbt, topk,
                                    None if fi is None else fi.ctypes.data_as(C.c_void_p), idx, res,
                                    dist.ctypes.data_as(C.c_void_p), tki.ctypes.data_as(C.c_void_p),
                                    tkl.ctypes.data_as(C.c_void_p))
        assert rc == 0
        out = dict(idx=idx, residual=res, dist=dist)
        if topk:
            out["topk_idx"] = tki
            out["topk_logit"] = tkl
        return out


    def projected_rvq(self, cfg: dict, force_idx=None, topk: int = 0):
        """OmniVoice / Higgs RVQ with per-stage projections (aqo_projected_rvq)."""
        x = np.ascontiguousarray(cfg["x"], np.float32)
        M, H = x.shape
        Q, N, K = cfg["Q"], cfg["N"], cfg["K"]
        cb, cbt = _cb_arg(cfg)
        wi, wo, pt = _proj_args(cfg)
        idx = np.zeros((M, Q), np.int32)
        res = np.zeros((M, H), np.float32)
        dist = np.zeros((M, Q), np.float32)
        tki = np.zeros((M, Q, max(topk, 1)), np.int32)
        tkl = np.zeros((M, Q, max(topk, 1)), np.float32)
        fi = np.ascontiguousarray(force_idx, np.int32) if force_idx is not None else None
        rc = self.lib.aqo_projected_rvq(
            x, M, H, K, Q, N, cfg["recipe"], cb.ctypes.data_as(C.c_void_p), cbt, wi.ctypes.data_as(C.c_void_p),
            _opt(cfg.get("b_in"), np.float32), wo.ctypes.data_as(C.c_void_p), _opt(cfg.get("b_out"), np.float32), pt,
            topk, None if fi is None else fi.ctypes.data_as(C.c_void_p), idx, res, dist.ctypes.data_as(C.c_void_p),
            tki.ctypes.data_as(C.c_void_p), tkl.ctypes.data_as(C.c_void_p))
        assert rc == 0
        out = dict(idx=idx, residual=res, dist=dist)
        if topk:
            out["topk_idx"] = tki
            out["topk_logit"] = tkl
        return out

    def linear(self, w, bias, x):
        """LinearModule over the rows of x [M, k]: w F32 [n_out, k] or
        block_q8_0 [n_out, k/32]; bias [n_out] or None (aqo_linear)."""
        x = np.ascontiguousarray(x, np.float32)
        M, k = x.shape
        wt = 0 if w.dtype == np.float32 else 1
        w = np.ascontiguousarray(w)
        n_out = w.shape[0]
        out = np.zeros((M, n_out), np.float32)
        assert self.lib.aqo_linear(w.ctypes.data_as(C.c_void_p), wt, _opt(bias, np.float32), n_out, k, M, x, out) == 0
        return out

    def projected_decode(self, cfg: dict, idx):
        """Sum over stages of project_out(c[idx]) (aqo_projected_decode)."""
        idx = np.ascontiguousarray(idx, np.int32)
        M = idx.shape[0]
        Q, N, K, H = cfg["Q"], cfg["N"], cfg["K"], cfg["H"]
        cb, cbt = _cb_arg(cfg)
        _, wo, pt = _proj_args(cfg)
        out = np.zeros((M, H), np.float32)
        rc = self.lib.aqo_projected_decode(idx, M, H, K, Q, N, cb.ctypes.data_as(C.c_void_p), cbt,
                                           wo.ctypes.data_as(C.c_void_p), _opt(cfg.get("b_out"), np.float32), pt, out)
        if rc != 0:
            raise IndexError("code outside [0, N)")
        return out


def _cb_arg(cfg: dict):
    if "codebook_q8" in cfg:
        return np.ascontiguousarray(cfg["codebook_q8"]), 1
    return np.ascontiguousarray(cfg["codebook"], np.float32), 0


def _proj_args(cfg: dict):
    if "w_in_q8" in cfg:
        return np.ascontiguousarray(cfg["w_in_q8"]), np.ascontiguousarray(cfg["w_out_q8"]), 1
    return np.ascontiguousarray(cfg["w_in"], np.float32), np.ascontiguousarray(cfg["w_out"], np.float32), 0

class _MossWeights(C.Structure):
    """MossWeights in ref_moss.cpp."""
    _fields_ = [("C", C.c_int64), ("R", C.c_int64), ("Q", C.c_int64), ("N", C.c_int64)] + [
        (n, C.POINTER(C.c_float)) for n in ("ip_g", "ip_v", "ip_b", "in_g", "in_v", "in_b", "cb", "out_g", "out_v",
                                              "out_b", "op_g", "op_v", "op_b")]


class Ref:
    """The reference's own ggml CPU backend (oracle/_ref)."""

    def __init__(self, isa: str | None = None):
        # `native` is tuned for the machine that built it; elsewhere use the
        # portable x86-64-v4 / v3 builds.
        isa = isa or host_isa()
        path = REF_DIR / f"libaqref-{isa}.so"
        if not path.exists():
            raise FileNotFoundError(f"{path} not built (make -C oracle ref needs /root/reference)")
        self.isa = isa
        self.lib = C.CDLL(str(path))
        L = self.lib
        L.aqref_dac_rvq.restype = C.c_double
        L.aqref_dac_rvq.argtypes = [_f32p, _i64, _i64, _i64, _i64, _i64, _f32p, C.c_void_p, _f32p, _f32p,
                                    C.c_void_p, _i32p, _f32p, C.c_void_p, C.c_void_p, C.c_int, C.c_int]
        L.aqref_dac_rvq_ex.restype = C.c_double
        L.aqref_dac_rvq_ex.argtypes = [_f32p, _i64, _i64, _i64, _i64, _i64, _f32p, C.c_void_p, _f32p, _f32p,
                                       C.c_void_p, _i32p, _f32p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]
        L.aqref_euclid_rvq.restype = C.c_double
        L.aqref_euclid_rvq.argtypes = [_f32p, _i64, _i64, _i64, _i64, _f32p, _i32p, _f32p, C.c_void_p, C.c_int]
        L.aqref_higgs_rvq.restype = C.c_double
        L.aqref_higgs_rvq.argtypes = [_f32p, _i64, _i64, _i64, _i64, C.c_void_p, C.c_int, C.c_int,
                                      _i32p, _f32p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int]
        L.aqref_dac_rvq_mixed.restype = C.c_double
        L.aqref_dac_rvq_mixed.argtypes = [_f32p, _i64, _i64, _i64, _i64, _i64, _i64, _f32p, C.c_void_p, _f32p, _f32p,
                                          _f32p, C.c_void_p, _i32p, _f32p, _f32p, C.c_int]
        L.aqref_projected_rvq.restype = C.c_double
        L.aqref_projected_rvq.argtypes = [_f32p, _i64, _i64, _i64, _i64, _i64, C.c_int, C.c_void_p, C.c_int,
                                          C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                                          _i32p, _f32p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int]
        L.aqref_projected_decode.restype = C.c_double
        L.aqref_projected_decode.argtypes = [_i32p, _i64, _i64, _i64, _i64, _i64, C.c_void_p, C.c_int, C.c_void_p,
                                             C.c_void_p, C.c_int, _f32p, C.c_int]
        L.aqref_qwen3_quantize.restype = C.c_double
        L.aqref_qwen3_quantize.argtypes = [_f32p, _f32p, _i64, _f32p, _f32p, _i32p]
        L.aqref_quantize_row_q8_0.argtypes = [_f32p, C.c_void_p, _i64]
        L.aqref_vector_quantizer.restype = C.c_int
        L.aqref_vector_quantizer.argtypes = [_f32p, _i64, _i64, _i64, _i64, _f32p, _i64, _i64, _f32p]
        L.aqref_quantize_chunk_q8_0.argtypes = [_f32p, C.c_void_p, _i64, _i64]
        L.aqref_vec_dot_f32.restype = C.c_float
        L.aqref_vec_dot_f32.argtypes = [C.c_int, _f32p, _f32p]
        L.aqref_top_k.restype = None
        L.aqref_top_k.argtypes = [_f32p, _i64, _i64, C.c_int, _i32p, C.c_int]
        L.aqref_linear.restype = C.c_double
        L.aqref_linear.argtypes = [C.c_void_p, C.c_int, C.c_void_p, _i64, _i64, _i64, _f32p, _f32p, C.c_int]
        L.aqref_outetts_fold.restype = None
        L.aqref_outetts_fold.argtypes = [_f32p, _f32p, _i64, _i64, _i64, _f32p]
        L.aqref_outetts_rvq.restype = C.c_double
        L.aqref_outetts_rvq.argtypes = [_f32p, _i64, _f32p, _f32p, _f32p, _f32p, _f32p, _i32p, C.c_int]
        L.aqref_moss_encode_timed.restype = C.c_double
        L.aqref_moss_encode_timed.argtypes = [C.POINTER(_MossWeights), _f32p, _i64, _i32p, C.c_int]
        L.aqref_moss_encode.restype = C.c_int
        L.aqref_moss_encode.argtypes = [C.POINTER(_MossWeights), _f32p, _i64, _i32p]
        L.aqref_moss_decode.restype = C.c_int
        L.aqref_moss_decode.argtypes = [C.POINTER(_MossWeights), _i32p, _i64, _f32p]

    def linear(self, w, bias, x, threads: int = 8):
        """The reference's LinearModule graph (mul_mat + add) on x [M, k]."""
        x = np.ascontiguousarray(x, np.float32)
        M, k = x.shape
        wt = 0 if w.dtype == np.float32 else 1
        w = np.ascontiguousarray(w)
        n_out = w.shape[0]
        out = np.zeros((M, n_out), np.float32)
        self.lib.aqref_linear(w.ctypes.data_as(C.c_void_p), wt, _opt(bias, np.float32), n_out, k, M, x, out, threads)
        return out

    def outetts_fold(self, v, g):
        """The reference's fold_weight_norm: v [dim0, dim1, kernel], g [dim0]."""
        v = np.ascontiguousarray(v, np.float32)
        g = np.ascontiguousarray(g, np.float32).reshape(-1)
        w = np.zeros_like(v)
        self.lib.aqref_outetts_fold(v, g, v.shape[0], v.shape[1], v.shape[2], w)
        return w

    def outetts_rvq(self, cfg: dict, threads: int = 0, timed: bool = False):
        """The reference's quantize_reference (2 stages, D = N = 1024): codes
        [M, 2] (and its milliseconds when timed)."""
        x = np.ascontiguousarray(cfg["x"], np.float32)
        M = x.shape[0]
        assert cfg["Q"] == 2 and cfg["D"] == 1024 and cfg["N"] == 1024
        a = lambda k: np.ascontiguousarray(cfg[k], np.float32)
        idx = np.zeros((M, 2), np.int32)
        ms = self.lib.aqref_outetts_rvq(x, M, a("w_in"), a("b_in"), a("codebook"), a("w_out"), a("b_out"), idx,
                                        threads)
        if ms < 0:
            raise RuntimeError("OuteTTS DAC encoder produced invalid acoustic latents")
        return (idx, ms) if timed else idx

    def _moss_weights(self, cfg: dict):
        keep = {k: np.ascontiguousarray(cfg[k], np.float32) for k in
                ("ip_g", "ip_v", "ip_b", "in_g", "in_v", "in_b", "codebook", "out_g", "out_v", "out_b",
                 "op_g", "op_v", "op_b")}
        p = lambda k: keep[k].ctypes.data_as(C.POINTER(C.c_float))
        w = _MossWeights(cfg["C"], cfg["R"], cfg["Q"], cfg["N"], p("ip_g"), p("ip_v"), p("ip_b"), p("in_g"),
                         p("in_v"), p("in_b"), p("codebook"), p("out_g"), p("out_v"), p("out_b"), p("op_g"),
                         p("op_v"), p("op_b"))
        return w, keep

    def moss_encode(self, cfg: dict):
        """MossAudioTokenizerQuantizer::encode: codes [M, Q]."""
        w, keep = self._moss_weights(cfg)
        h = np.ascontiguousarray(cfg["hidden"], np.float32)
        idx = np.zeros((h.shape[0], cfg["Q"]), np.int32)
        if self.lib.aqref_moss_encode(C.byref(w), h, h.shape[0], idx) != 0:
            raise RuntimeError("MOSS codec quantizer rejected its input")
        return idx

    def moss_encode_timed(self, cfg: dict, threads: int = 0):
        """encode() alone on the clock: (codes [M, Q], milliseconds)."""
        w, keep = self._moss_weights(cfg)
        h = np.ascontiguousarray(cfg["hidden"], np.float32)
        idx = np.zeros((h.shape[0], cfg["Q"]), np.int32)
        ms = self.lib.aqref_moss_encode_timed(C.byref(w), h, h.shape[0], idx, threads)
        if ms < 0:
            raise RuntimeError("MOSS codec quantizer rejected its input")
        return idx, ms

    def moss_decode(self, cfg: dict, idx):
        """MossAudioTokenizerQuantizer::decode, returned frame-major [M, C]."""
        w, keep = self._moss_weights(cfg)
        idx = np.ascontiguousarray(idx, np.int32)
        M = idx.shape[0]
        out = np.zeros((cfg["C"], M), np.float32)
        if self.lib.aqref_moss_decode(C.byref(w), idx, M, out) != 0:
            raise IndexError("MOSS codec code index out of range")
        return np.ascontiguousarray(out.T)

    def top_k(self, v, k: int, threads: int = 8):
        """ggml_top_k over the rows of v, in ggml's order."""
        v = np.ascontiguousarray(v, np.float32)
        rows, n = v.shape
        out = np.zeros((rows, k), np.int32)
        self.lib.aqref_top_k(v, rows, n, k, out, threads)
        return out

    def dac_rvq(self, cfg: dict, threads: int = 8, recon: bool = True, materialize: bool = True, recipe: int = 0):
        x = np.ascontiguousarray(cfg["x"], np.float32)
        T, D, Q, N = cfg["T"], cfg["D"], cfg["Q"], cfg["N"]
        M = x.shape[0]
        B = M // T
        idx = np.zeros((M, Q), np.int32)
        res = np.zeros((M, D), np.float32)
        rec = np.zeros((M, D), np.float32) if recon else None
        ms = self.lib.aqref_dac_rvq_ex(x, B, T, D, Q, N, np.ascontiguousarray(cfg["w_in"], np.float32),
                                       _opt(cfg.get("b_in"), np.float32), np.ascontiguousarray(cfg["codebook"], np.float32),
                                       np.ascontiguousarray(cfg["w_out"], np.float32), _opt(cfg.get("b_out"), np.float32),
                                       idx, res, None if rec is None else rec.ctypes.data_as(C.c_void_p), None, threads,
                                       1 if materialize else 0, recipe)
        if ms < 0:
            raise ValueError("the recipe rejects a zero codebook row")
        return dict(idx=idx, residual=res, recon=rec, ms=ms)

    def dac_rvq_mixed(self, cfg: dict, threads: int = 8):
        x = np.ascontiguousarray(cfg["x"], np.float32)
        M, D = x.shape
        Q = cfg["Q"]
        idx = np.zeros((M, Q), np.int32)
        res = np.zeros((M, D), np.float32)
        rec = np.zeros((M, D), np.float32)
        ms = self.lib.aqref_dac_rvq_mixed(x, M // cfg["T"], cfg["T"], D, Q, cfg["N0"], cfg["N"],
                                          np.ascontiguousarray(cfg["w_in"], np.float32),
                                          _opt(cfg.get("b_in"), np.float32),
                                          np.ascontiguousarray(cfg["codebook0"], np.float32),
                                          np.ascontiguousarray(cfg["codebook"], np.float32),
                                          np.ascontiguousarray(cfg["w_out"], np.float32),
                                          _opt(cfg.get("b_out"), np.float32), idx, res, rec, threads)
        return dict(idx=idx, residual=res, recon=rec, ms=ms)

    def euclid_rvq(self, cfg: dict, threads: int = 8):
        x = np.ascontiguousarray(cfg["x"], np.float32)
        M, K = x.shape
        Q, N = cfg["Q"], cfg["N"]
        idx = np.zeros((M, Q), np.int32)
        res = np.zeros((M, K), np.float32)
        lb = np.zeros((M, Q), np.float32)
        ms = self.lib.aqref_euclid_rvq(x, M, K, Q, N, np.ascontiguousarray(cfg["codebook"], np.float32), idx, res,
                                       lb.ctypes.data_as(C.c_void_p), threads)
        return dict(idx=idx, residual=res, logit=lb, ms=ms)

    def higgs_rvq(self, cfg: dict, topk: int = 0, threads: int = 8):
        x = np.ascontiguousarray(cfg["x"], np.float32)
        M, K = x.shape
        Q, N = cfg["Q"], cfg["N"]
        if "codebook_q8" in cfg:
            cb = np.ascontiguousarray(cfg["codebook_q8"])
            cbt = 1
        else:
            cb = np.ascontiguousarray(cfg["codebook"], np.float32)
            cbt = 0
        idx = np.zeros((M, Q), np.int32)
        res = np.zeros((M, K), np.float32)
        dist = np.zeros((M, Q), np.float32)
        tki = np.zeros((M, Q, max(topk, 1)), np.int32)
        tkl = np.zeros((M, Q, max(topk, 1)), np.float32)
        ms = self.lib.aqref_higgs_rvq(x, M, K, Q, N, cb.ctypes.data_as(C.c_void_p), cbt, topk, idx, res,
                                      dist.ctypes.data_as(C.c_void_p),
                                      tki.ctypes.data_as(C.c_void_p) if topk else None,
                                      tkl.ctypes.data_as(C.c_void_p) if topk else None, threads)
        out = dict(idx=idx, residual=res, dist=dist, ms=ms)
        if topk:
            out["topk_idx"] = tki
            out["topk_logit"] = tkl
        return out

    def projected_rvq(self, cfg: dict, topk: int = 0, threads: int = 8):
        """The OmniVoice / Higgs graphs with projections (aqref_projected_rvq)."""
        x = np.ascontiguousarray(cfg["x"], np.float32)
        M, H = x.shape
        Q, N, K = cfg["Q"], cfg["N"], cfg["K"]
        cb, cbt = _cb_arg(cfg)
        wi, wo, pt = _proj_args(cfg)
        idx = np.zeros((M, Q), np.int32)
        res = np.zeros((M, H), np.float32)
        dist = np.zeros((M, Q), np.float32)
        tki = np.zeros((M, Q, max(topk, 1)), np.int32)
        tkl = np.zeros((M, Q, max(topk, 1)), np.float32)
        ms = self.lib.aqref_projected_rvq(
            x, M, H, K, Q, N, cfg["recipe"], cb.ctypes.data_as(C.c_void_p), cbt, wi.ctypes.data_as(C.c_void_p),
            _opt(cfg.get("b_in"), np.float32), wo.ctypes.data_as(C.c_void_p), _opt(cfg.get("b_out"), np.float32), pt,
            topk, idx, res, dist.ctypes.data_as(C.c_void_p), tki.ctypes.data_as(C.c_void_p) if topk else None,
            tkl.ctypes.data_as(C.c_void_p) if topk else None, threads)
        out = dict(idx=idx, residual=res, dist=dist, ms=ms)
        if topk:
            out["topk_idx"] = tki
            out["topk_logit"] = tkl
        return out

    def projected_decode(self, cfg: dict, idx, threads: int = 8):
        idx = np.ascontiguousarray(idx, np.int32)
        M = idx.shape[0]
        cb, cbt = _cb_arg(cfg)
        _, wo, pt = _proj_args(cfg)
        out = np.zeros((M, cfg["H"]), np.float32)
        self.lib.aqref_projected_decode(idx, M, cfg["H"], cfg["K"], cfg["Q"], cfg["N"], cb.ctypes.data_as(C.c_void_p),
                                        cbt, wo.ctypes.data_as(C.c_void_p), _opt(cfg.get("b_out"), np.float32), pt, out,
                                        threads)
        return out

    def qwen3_quantize(self, cfg: dict):
        """quantize_projected of the Qwen3 speech tokenizer (the reference's own
        function): codes [frames, 16]."""
        F = cfg["frames"]
        codes = np.zeros((F, cfg["S"]), np.int32)
        ms = self.lib.aqref_qwen3_quantize(np.ascontiguousarray(cfg["semantic"], np.float32),
                                           np.ascontiguousarray(cfg["acoustic"], np.float32), F,
                                           np.ascontiguousarray(cfg["embedding_sum"], np.float32),
                                           np.ascontiguousarray(cfg["cluster_usage"], np.float32), codes)
        if ms < 0:
            raise RuntimeError("the reference quantizer threw")
        return codes

    def vector_quantizer(self, x, codebook, batch: int = 1):
        """engine::runtime::VectorQuantizer::compute: nearest codewords."""
        x = np.ascontiguousarray(x, np.float32)
        cb = np.ascontiguousarray(codebook, np.float32)
        M, K = x.shape
        out = np.zeros_like(x)
        rc = self.lib.aqref_vector_quantizer(x, x.size, batch, M // batch, K, cb, cb.size, cb.shape[0], out)
        if rc != 0:
            raise RuntimeError("VectorQuantizer input size mismatch")
        return out
