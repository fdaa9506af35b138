"""Writes the golden fixtures from the reference's own ggml CPU backend.

Runs in the build container only: it loads oracle/_ref/libaqref-native.so,
which oracle/Makefile compiles from /root/reference/external/ggml (plus
oracle/ref_harness.cpp, which builds the reference recipes' op graphs).
Inputs come from audio.cpp_amd/aqmi/synth.py (deterministic, seeded), so a
fixture stores only outputs: codes, and SHA-256 digests of the fp32 residual
and reconstruction bytes (bit-exact checks), plus small value samples.

    python tests/golden/make_golden.py [dac] [mimi] [kmeans] [q8] [outetts] [moss] [qwen3] [projected] [fish]
"""

from __future__ import annotations

import hashlib
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "audio.cpp_amd"))

from aqmi import synth  # noqa: E402
from oracle import Ref  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def save(name: str, **arrays):
    path = HERE / name
    np.savez_compressed(path, **arrays)
    print(f"wrote {path.name} ({path.stat().st_size} bytes)")


def dac(ref: Ref, cfg_id: int, name: str, bias: bool = False, **over):
    cfg = synth.make_config(cfg_id)
    if bias:
        cfg.update(synth.dac_weights(cfg["seed"], cfg["Q"], cfg["D"], cfg["N"], bias=True))
    cfg.update(over)
    out = ref.dac_rvq(cfg)
    save(name, idx=out["idx"].astype(np.uint16), residual_sha=np.array(sha(out["residual"])),
         recon_sha=np.array(sha(out["recon"])), residual_head=out["residual"][:4, :16].copy(),
         recon_head=out["recon"][:4, :16].copy(), bias=np.array(bias), ggml_isa=np.array(ref.isa))


def sorted_topk(idx: np.ndarray, val: np.ndarray):
    """ggml_top_k leaves the k best in no particular order: sort each list by
    (value desc, index asc) so fixtures compare as sets."""
    order = np.lexsort((idx, -val.astype(np.float64)), axis=-1)
    return np.take_along_axis(idx, order, -1), np.take_along_axis(val, order, -1)


def mimi(ref: Ref, name: str):
    """BASELINE configs[2] with the OmniVoice score recipe (logit = 2c.r - |c|^2)."""
    cfg = synth.make_config(2)
    out = ref.euclid_rvq(cfg)
    save(name, idx=out["idx"].astype(np.uint16), residual_sha=np.array(sha(out["residual"])),
         logit_sha=np.array(sha(out["logit"])), residual_head=out["residual"][:64].copy(),
         logit_head=out["logit"][:64].copy(), recipe=np.array("omnivoice"), ggml_isa=np.array(ref.isa))


def kmeans(ref: Ref, name: str, chunk: int = 20000):
    """BASELINE configs[3] with the Higgs recipe (dist = |r|^2 + |c|^2 - 2c.r).
    Rows are independent, so the 200k x 16384 score matrix is evaluated in row
    chunks (multiples of 16 rows keep ggml on the same tinyBLAS path)."""
    cfg = synth.make_config(3)
    M = cfg["M"]
    idx = np.zeros((M, 1), np.int32)
    dist = np.zeros((M, 1), np.float32)
    for r0 in range(0, M, chunk):
        part = dict(cfg, x=cfg["x"][r0:r0 + chunk], M=min(chunk, M - r0))
        out = ref.higgs_rvq(part)
        idx[r0:r0 + chunk] = out["idx"]
        dist[r0:r0 + chunk] = out["dist"]
        print(f"  k-means rows {r0}..{r0 + part['M']}", flush=True)
    save(name, idx=idx[:, 0].astype(np.uint16), dist_sha=np.array(sha(dist)), dist_head=dist[:256, 0].copy(),
         recipe=np.array("higgs"), ggml_isa=np.array(ref.isa))


def q8(ref: Ref, name: str):
    """Q8_0 codebooks, Higgs recipe, top-4 per stage."""
    cfg = synth.make_config(4)
    out = ref.higgs_rvq(cfg, topk=4)
    ti, tl = sorted_topk(out["topk_idx"], out["topk_logit"])
    save(name, idx=out["idx"].astype(np.uint16), residual_sha=np.array(sha(out["residual"])),
         dist_sha=np.array(sha(out["dist"])), topk_idx_sha=np.array(sha(ti.astype(np.int32))),
         topk_logit_sha=np.array(sha(tl)), residual_head=out["residual"][:64].copy(),
         topk_idx_head=ti[:64].copy(), topk_logit_head=tl[:64].copy(), recipe=np.array("higgs-q8_0"),
         ggml_isa=np.array(ref.isa))


def outetts(ref: Ref, name: str):
    """OuteTTS host loop (quantize_reference), 3001 frames, near-duplicate
    codebooks (synth.near_duplicate_pairs seed 7): codes only -- the
    reference function returns nothing else."""
    cfg = synth.outetts_config(3001)
    cfg["codebook"] = synth.near_duplicate_pairs(cfg["codebook"], 7)
    save(name, idx=ref.outetts_rvq(cfg).astype(np.int16))


def moss(ref: Ref, name: str):
    """MOSS-Audio-Tokenizer-v2 quantizer (768 -> 512, 12 x 1024 x 8), 256
    frames: the reference's codes, and its decode of them (frame-major)."""
    cfg = synth.moss_config(256)
    idx = ref.moss_encode(cfg)
    lat = ref.moss_decode(cfg, idx)
    save(name, idx=idx.astype(np.int16), latent_sha=sha(lat), latent_head=lat[:2, :16])


def host_loop_bench(ref: Ref):
    """Codes of bench.py's outetts_rvq and moss_rvq workloads (6 000 frames
    each), from the reference's own functions."""
    save("outetts_bench.npz", idx=ref.outetts_rvq(synth.outetts_config(6000)).astype(np.int16))
    save("moss_bench.npz", idx=ref.moss_encode(synth.moss_config(6000)).astype(np.int16))


def qwen3(ref: Ref, name: str, frames: int = 600):
    """Qwen3-TTS speech-tokenizer cascade (quantize_projected, the reference's
    own function): 1 semantic + 15 acoustic EMA codebooks of 2048 x 256 on
    channel-major latents, codes [frames, 16]."""
    save(name, idx=ref.qwen3_quantize(synth.qwen3_config(frames)).astype(np.int16))


def projected(ref: Ref):
    """OmniVoice / Higgs cascades with projections (hidden 1024, dim 64, 1024
    codes, 8 stages) from the reference's op graphs on ggml."""
    cases = [("higgs_f32", dict(recipe=1), 0), ("higgs_q8", dict(recipe=1, cb_q8=True, proj_q8=True), 4),
             ("omnivoice_f32", dict(recipe=0), 0), ("omnivoice_q8proj", dict(recipe=0, proj_q8=True), 0)]
    for tag, kw, topk in cases:
        cfg = synth.projected_config(400, **kw)
        out = ref.projected_rvq(cfg, topk=topk)
        arrays = dict(idx=out["idx"].astype(np.int16), residual_sha=np.array(sha(out["residual"])),
                      dist_sha=np.array(sha(out["dist"])), residual_head=out["residual"][:4, :16].copy())
        if topk:
            ti, tl = sorted_topk(out["topk_idx"], out["topk_logit"])
            arrays.update(topk_idx_sha=np.array(sha(ti.astype(np.int32))), topk_logit_sha=np.array(sha(tl)))
        dec = ref.projected_decode(cfg, out["idx"])
        arrays.update(decode_sha=np.array(sha(dec)))
        save(f"projected_{tag}.npz", **arrays)


def fish_mixed(ref: Ref, name: str):
    """The Fish cascade: a 4096-code semantic stage then 8 residual stages of
    1024 codes, 4 clips x 250 frames, latent 1024 (the reference's graph
    recipe on ggml): codes, and digests of the residual and the recon."""
    out = ref.dac_rvq_mixed(synth.fish_config(4, 250))
    save(name, idx=out["idx"].astype(np.int16), residual_sha=np.array(sha(out["residual"])),
         recon_sha=np.array(sha(out["recon"])))


def main():
    which = set(sys.argv[1:]) or {"dac", "mimi", "kmeans", "q8", "outetts", "moss", "qwen3", "projected", "fish"}
    ref = Ref("native")
    if "dac" in which:
        dac(ref, 0, "dac_cfg0.npz")
        dac(ref, 1, "dac_cfg1.npz")
        dac(ref, 0, "dac_cfg0_bias.npz", bias=True)
    if "mimi" in which:
        mimi(ref, "mimi_cfg2.npz")
    if "kmeans" in which:
        kmeans(ref, "kmeans_cfg3.npz")
    if "q8" in which:
        q8(ref, "q8_cfg4.npz")
    if "outetts" in which:
        outetts(ref, "outetts_neardup.npz")
    if "moss" in which:
        moss(ref, "moss_v2.npz")
        host_loop_bench(ref)
    if "qwen3" in which:
        qwen3(ref, "qwen3_cascade.npz")
    if "projected" in which:
        projected(ref)
    if "fish" in which:
        fish_mixed(ref, "fish_mixed.npz")


if __name__ == "__main__":
    main()
