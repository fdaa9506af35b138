"""Builds the MI355X quantizer library: audio.cpp_amd/libaq_mi355x.so.

hipcc compiles every HIP / C++ source in csrc/ for gfx950 only.  Flags:
  -ffp-contract=off      no implicit FMA: every fused multiply-add in the
                         kernels is written out (__fmaf_rn) where the
                         reference arithmetic has one, so results stay
                         bit-identical to the ggml CPU backend.
  -fno-gpu-flush-denormals-to-zero   IEEE fp32 subnormals, as on the CPU.
  -target-feature -packed-fp32-ops   no v_pk_{add,mul,fma}_f32 generation.
Usage: python audio.cpp_amd/build.py [--jobs N] [--changed]
(--changed recompiles only sources newer than their objects.)
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT = PKG / "libaq_mi355x.so"
BUILD = PKG / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
    "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]


def sources() -> list[pathlib.Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


# Per-source flags.  aq_euclid_ks8.hip holds the register-resident cascade
# (one wave per SIMD, residual in AGPRs): MFMA results in VGPRs keep its key
# epilogue free of AGPR-to-VGPR copies, and a higher full-unroll limit lets
# its per-group select loop (the Q8_0 variant's body is the largest) unroll,
# so that the residual array is indexed by constants and stays in registers
# (unrolled short, it would live in scratch memory).
SOURCE_FLAGS = {"aq_euclid_ks8.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-mllvm", "-pragma-unroll-threshold=200000"]}


def compile_one(src: pathlib.Path) -> pathlib.Path:
    obj = BUILD / (src.name + ".o")
    cmd = [HIPCC, *FLAGS, *SOURCE_FLAGS.get(src.name, []), "-x", "hip", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed on {src.name}")
    return obj


def _stale(src: pathlib.Path) -> bool:
    """Object missing or older than its source or any shared header."""
    obj = BUILD / (src.name + ".o")
    if not obj.exists():
        return True
    deps = [src, *CSRC.glob("*.hpp"), *(ROOT / "include").glob("*.h")]
    return max(d.stat().st_mtime for d in deps) > obj.stat().st_mtime


def build(jobs: int | None = None, changed_only: bool = False) -> pathlib.Path:
    """Compile every source (or, with changed_only, the stale ones) and link."""
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    if changed_only:
        srcs = [s for s in srcs if _stale(s)]
    if srcs:
        with cf.ThreadPoolExecutor(max_workers=jobs or min(8, len(srcs))) as ex:
            list(ex.map(compile_one, srcs))
    objs = [BUILD / (s.name + ".o") for s in sources()]
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    subprocess.run(cmd, check=True)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    jobs = None
    if "--jobs" in sys.argv:
        jobs = int(sys.argv[sys.argv.index("--jobs") + 1])
    print(build(jobs, changed_only="--changed" in sys.argv))
