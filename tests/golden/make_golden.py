"""Writes the golden fixtures from the reference's own ggml CPU backend.

Runs in the build container only: it loads oracle/_ref/libaqref-native.so,
which oracle/Makefile compiles from /root/reference/external/ggml (plus
oracle/ref_harness.cpp, which builds the reference recipes' op graphs).
Inputs come from audio.cpp_amd/aqmi/synth.py (deterministic, seeded), so a
fixture stores only outputs: codes, and SHA-256 digests of the fp32 residual
and reconstruction bytes (bit-exact checks), plus small value samples.

    python tests/golden/make_golden.py
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


def main():
    ref = Ref("native")
    dac(ref, 0, "dac_cfg0.npz")
    dac(ref, 1, "dac_cfg1.npz")
    dac(ref, 0, "dac_cfg0_bias.npz", bias=True)


if __name__ == "__main__":
    main()
