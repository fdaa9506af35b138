"""Near-tie accounting of the BASELINE fixtures (writes near_ties.json).

For every frame and stage of the golden configs, on the residual the
reference's own codes leave (teacher forcing), the two smallest distances
d1 <= d2 are computed in fp64 from the exact fp32 inputs and
gap_rel = (d2 - d1) / max(d1, 1e-30); a frame-stage is a near-tie when
gap_rel <= 1e-5.  Distances: Euclidean |r - c|^2 (for Q8_0 codebooks on the
query's Q8_0 image, x86 quantize_row_q8_0, against the dequantised codes);
cosine d = 1 - cos between the in-projected residual and the normalised
codebook rows (DAC).  Also counted: frame-stages whose fp64 argmin differs
from the reference's code outside the near-ties (expected 0).

    python tests/golden/near_ties.py
"""

from __future__ import annotations

import json
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "audio.cpp_amd"))

from aqmi import synth  # noqa: E402
from oracle import Oracle  # noqa: E402

TIE = 1e-5


def two_smallest(d: np.ndarray):
    part = np.partition(d, 1, axis=1)[:, :2]
    return part[:, 0], part[:, 1], np.argmin(d, axis=1)


def account(d1, d2, amin, ref_code):
    gap = (d2 - d1) / np.maximum(d1, 1e-30)
    tie = gap <= TIE
    return int(tie.sum()), int(((amin != ref_code) & ~tie).sum()), float(gap.min())


def euclid_stage(r: np.ndarray, c: np.ndarray, chunk: int = 8192):
    """fp64 two smallest |r - c|^2 per row, in row chunks."""
    c64 = c.astype(np.float64)
    cn = (c64 * c64).sum(1)
    d1s, d2s, ams = [], [], []
    for i in range(0, r.shape[0], chunk):
        r64 = r[i:i + chunk].astype(np.float64)
        d = (r64 * r64).sum(1)[:, None] - 2.0 * (r64 @ c64.T) + cn[None, :]
        d1, d2, am = two_smallest(d)
        d1s.append(d1)
        d2s.append(d2)
        ams.append(am)
    return np.concatenate(d1s), np.concatenate(d2s), np.concatenate(ams)


def q8_image(x: np.ndarray) -> np.ndarray:
    """x86 quantize_row_q8_0 of each 32-block, as q * d in fp32."""
    b = x.reshape(x.shape[0], -1, 32).astype(np.float32)
    amax = np.abs(b).max(-1)
    d = (amax / np.float32(127.0)).astype(np.float16).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(amax != 0, np.float32(127.0) / np.where(amax != 0, amax, 1), 0).astype(np.float32)
    q = np.clip(np.rint((b * idv[..., None]).astype(np.float32)), -128, 127)
    return (q * d[..., None]).astype(np.float32).reshape(x.shape)


def euclid_cfg(cfg_id: int, fixture: str) -> dict:
    cfg = synth.make_config(cfg_id)
    idx = np.load(HERE / fixture)["idx"].astype(np.int64).reshape(cfg["M"], cfg["Q"])
    q8 = "codebook_q8" in cfg
    cbs = synth.q8_0_dequantize(cfg["codebook_q8"]) if q8 else cfg["codebook"]
    r = np.array(cfg["x"], np.float32)
    ties, wrong, gmin = [], [], []
    for s in range(cfg["Q"]):
        c = np.asarray(cbs[s], np.float32)
        d1, d2, am = euclid_stage(q8_image(r) if q8 else r, c)
        t, w, g = account(d1, d2, am, idx[:, s])
        ties.append(t)
        wrong.append(w)
        gmin.append(g)
        r = (r - c[idx[:, s]]).astype(np.float32)
        print(f"  {fixture} stage {s}: near-ties {t}, argmin differs outside ties {w}", flush=True)
    return dict(near_ties_per_stage=ties, argmin_differs_outside_ties=wrong, min_gap_rel=min(gmin),
                frame_stages=int(cfg["M"] * cfg["Q"]))


def dac_cfg(cfg_id: int, fixture: str) -> dict:
    o = Oracle()
    cfg = synth.make_config(cfg_id)
    M, Q, D, N = cfg["x"].shape[0], cfg["Q"], cfg["D"], cfg["N"]
    idx = np.load(HERE / fixture)["idx"].astype(np.int32).reshape(M, Q)
    r = np.array(cfg["x"], np.float32)
    ties, wrong, gmin = [], [], []
    for s in range(Q):
        w_in = cfg["w_in"][s].astype(np.float64)
        p = r.astype(np.float64) @ w_in.T + cfg["b_in"][s].astype(np.float64)[None, :]
        pn = p / np.linalg.norm(p, axis=1, keepdims=True)
        c = cfg["codebook"][s].astype(np.float64)
        cn = c / np.maximum(np.linalg.norm(c, axis=1, keepdims=True), 1e-300)
        d = 1.0 - pn @ cn.T
        d1, d2, am = two_smallest(d)
        t, w, g = account(d1, d2, am, idx[:, s])
        ties.append(t)
        wrong.append(w)
        gmin.append(g)
        # the fp32 residual after stages 0..s, teacher-forced on the reference's codes
        sub = dict(cfg, x=cfg["x"], Q=s + 1, w_in=cfg["w_in"][:s + 1], b_in=cfg["b_in"][:s + 1],
                   codebook=cfg["codebook"][:s + 1], w_out=cfg["w_out"][:s + 1], b_out=cfg["b_out"][:s + 1])
        r = o.dac_rvq(sub, force_idx=idx[:, :s + 1], recon=False)["residual"]
        print(f"  {fixture} stage {s}: near-ties {t}, argmin differs outside ties {w}", flush=True)
    return dict(near_ties_per_stage=ties, argmin_differs_outside_ties=wrong, min_gap_rel=min(gmin),
                frame_stages=int(M * Q))


def main():
    out = {"definition": "gap_rel = (d2 - d1) / max(d1, 1e-30) in fp64 on the reference's residual path; "
                         "near-tie when gap_rel <= 1e-5", "tie": TIE}
    out["dac_cfg0.npz"] = dac_cfg(0, "dac_cfg0.npz")
    out["dac_cfg1.npz"] = dac_cfg(1, "dac_cfg1.npz")
    out["mimi_cfg2.npz"] = euclid_cfg(2, "mimi_cfg2.npz")
    out["q8_cfg4.npz"] = euclid_cfg(4, "q8_cfg4.npz")
    out["kmeans_cfg3.npz"] = euclid_cfg(3, "kmeans_cfg3.npz")
    (HERE / "near_ties.json").write_text(json.dumps(out, indent=1) + "\n")
    print("wrote near_ties.json")


if __name__ == "__main__":
    main()
