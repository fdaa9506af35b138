"""Seeded synthetic workloads for the quantizer path.

The generator is counter-based and uses only IEEE basic operations
(+, -, *, /, sqrt) on float64, so every machine produces the same float32
inputs bit for bit (no libm log/cos whose last ulp differs across builds):

  base(seed, stream) = splitmix64(splitmix64(seed) ^ (stream * 0xD1B54A32D192ED03))
  a_i = splitmix64(base + 2 i),  b_i = splitmix64(base + 2 i + 1)      (mod 2**64)
  u1  = ((a_i >> 11) + 1) * 2**-53  in (0, 1]
  u2  =  (b_i >> 11)      * 2**-53  in [0, 1)
  normal_i  = sqrt(-2 ln u1) * cos(2 pi u2)          (Box-Muller, first output)
  uniform_i = lo + (hi - lo) * ((a_i >> 11) * 2**-53)

`ln` and `cos` are evaluated with fixed series in float64 (see _det_log and
_det_cos), accurate to a few 1e-16.  `N(0, s)` means standard deviation s.

The BASELINE workloads (configs 0-4) are built by `make_config`.
"""

from __future__ import annotations

import os

import numpy as np

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)
_GOLD = np.uint64(0x9E3779B97F4A7C15)
_C1 = np.uint64(0xBF58476D1CE4E5B9)
_C2 = np.uint64(0x94D049BB133111EB)
_STREAM = np.uint64(0xD1B54A32D192ED03)
_TWO_M53 = float(2.0 ** -53)
_LN2 = 0.6931471805599453094172321
_TWO_PI = 6.283185307179586476925287


def _splitmix64(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = z + _GOLD
        z = (z ^ (z >> np.uint64(30))) * _C1
        z = (z ^ (z >> np.uint64(27))) * _C2
        return z ^ (z >> np.uint64(31))


def _base(seed: int, stream: int) -> np.uint64:
    s = _splitmix64(np.array([seed], dtype=np.uint64))[0]
    with np.errstate(over="ignore"):
        k = np.uint64(stream) * _STREAM
    return _splitmix64(np.array([s ^ k], dtype=np.uint64))[0]


def _det_log(x: np.ndarray) -> np.ndarray:
    """ln(x) for x in (0, 1] using frexp and the atanh series."""
    m, e = np.frexp(x)                      # x = m * 2**e, m in [0.5, 1)
    small = m < 0.7071067811865476
    m = np.where(small, m * 2.0, m)         # m in [sqrt(1/2), sqrt(2))
    e = np.where(small, e - 1, e).astype(np.float64)
    s = (m - 1.0) / (m + 1.0)
    s2 = s * s
    acc = np.full_like(s, 1.0 / 23.0)
    for k in range(21, 0, -2):
        acc = acc * s2 + 1.0 / k
    return e * _LN2 + 2.0 * s * acc


def _det_cos_2pi(t: np.ndarray) -> np.ndarray:
    """cos(2 pi t) for t in [0, 1) with range reduction to [0, pi/2]."""
    r = t - np.floor(t + 0.5)               # [-0.5, 0.5)
    a = np.abs(r)                           # [0, 0.5]
    flip = a > 0.25
    a = np.where(flip, 0.5 - a, a)          # [0, 0.25]
    x = a * _TWO_PI
    x2 = x * x
    acc = np.zeros_like(x)
    fact = [1.0]
    for k in range(1, 26):
        fact.append(fact[-1] * k)
    for k in range(12, -1, -1):
        acc = acc * x2 + ((-1.0) ** k) / fact[2 * k]
    return np.where(flip, -acc, acc)


def _uniform53(z: np.ndarray) -> np.ndarray:
    return (z >> np.uint64(11)).astype(np.float64) * _TWO_M53


_CHUNK = 1 << 20   # elements per pass: keeps the float64 temporaries in cache


def _normal_chunk(base: np.uint64, i0: int, n: int) -> np.ndarray:
    i = np.arange(i0, i0 + n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        a = _splitmix64(base + np.uint64(2) * i)
        b = _splitmix64(base + np.uint64(2) * i + np.uint64(1))
    u1 = ((a >> np.uint64(11)).astype(np.float64) + 1.0) * _TWO_M53
    u2 = _uniform53(b)
    return np.sqrt(-2.0 * _det_log(u1)) * _det_cos_2pi(u2)


def normal(seed: int, stream: int, shape, std: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    base = _base(seed, stream)
    out = np.empty(n, np.float32)

    def fill(i0):
        m = min(_CHUNK, n - i0)
        out[i0:i0 + m] = (_normal_chunk(base, i0, m) * float(std)).astype(np.float32)

    starts = range(0, n, _CHUNK)
    if len(starts) > 2:
        # numpy releases the GIL inside these element-wise loops
        from concurrent.futures import ThreadPoolExecutor

        with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as pool:
            list(pool.map(fill, starts))
    else:
        for i0 in starts:
            fill(i0)
    return out.reshape(shape)


def uniform(seed: int, stream: int, shape, lo: float, hi: float) -> np.ndarray:
    n = int(np.prod(shape))
    base = _base(seed, stream)
    i = np.arange(n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        a = _splitmix64(base + np.uint64(2) * i)
    return (lo + (hi - lo) * _uniform53(a)).astype(np.float32).reshape(shape)


def uniform_f64(seed: int, stream: int, shape) -> np.ndarray:
    n = int(np.prod(shape))
    base = _base(seed, stream)
    i = np.arange(n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        a = _splitmix64(base + np.uint64(2) * i)
    return _uniform53(a).reshape(shape)


# --------------------------------------------------------------------------
# Q8_0 block helpers (GGUF block_q8_0 = { fp16 d; int8 qs[32] }, 34 bytes)

Q8_BLOCK = 32
Q8_BYTES = 34
Q8_DTYPE = np.dtype([("d", "<f2"), ("qs", "i1", (32,))])


def q8_0_random_codebook(seed: int, stream: int, rows: int, dim: int) -> np.ndarray:
    """Blocks with qs ~ U{-127..127} and d ~ U(1e-3, 1e-2) rounded to fp16."""
    nb = dim // Q8_BLOCK
    u = uniform_f64(seed, stream, (rows, nb, Q8_BLOCK))
    qs = (np.floor(u * 255.0) - 127.0).astype(np.int8)
    d = uniform(seed, stream + 1, (rows, nb), 1e-3, 1e-2).astype(np.float16)
    out = np.zeros((rows, nb), dtype=Q8_DTYPE)
    out["d"] = d
    out["qs"] = qs
    return out


def q8_0_dequantize(blocks: np.ndarray) -> np.ndarray:
    """Reference dequantisation y = q * d (ggml-quants.c:491-505)."""
    d = blocks["d"].astype(np.float32)[..., None]
    return (blocks["qs"].astype(np.float32) * d).reshape(blocks.shape[:-1] + (-1,))


# --------------------------------------------------------------------------
# BASELINE.json configs

DAC_DIM = 8


def dac_weights(seed: int, Q: int, D: int, N: int, bias: bool = False):
    """Per-stage DAC weights: W_in [Q,8,D] ~N(0,1/sqrt(D)), codebook [Q,N,8]
    ~N(0,1), W_out [Q,D,8] ~N(0,1/sqrt(8)); biases zero unless `bias`."""
    w_in = np.stack([normal(seed, 100 * s + 2, (DAC_DIM, D), 1.0 / np.sqrt(D)) for s in range(Q)])
    cb = np.stack([normal(seed, 100 * s + 3, (N, DAC_DIM), 1.0) for s in range(Q)])
    w_out = np.stack([normal(seed, 100 * s + 4, (D, DAC_DIM), 1.0 / np.sqrt(DAC_DIM)) for s in range(Q)])
    if bias:
        b_in = np.stack([normal(seed, 100 * s + 5, (DAC_DIM,), 0.1) for s in range(Q)])
        b_out = np.stack([normal(seed, 100 * s + 6, (D,), 0.1) for s in range(Q)])
    else:
        b_in = np.zeros((Q, DAC_DIM), np.float32)
        b_out = np.zeros((Q, D), np.float32)
    return dict(w_in=w_in, b_in=b_in, codebook=cb, w_out=w_out, b_out=b_out)


def make_config(i: int, rows: int | None = None) -> dict:
    """Inputs of BASELINE config i.  `rows` truncates the frame axis (the
    generator is counter-based, so a truncated config is an exact prefix)."""
    if i == 0:
        B, T, D, Q, N = 1, 750, 1024, 1, 1024
        M = B * T if rows is None else rows
        x = normal(1, 1, (B * T, D))[:M]
        return dict(kind="dac", seed=1, B=B, T=T, D=D, Q=Q, N=N, x=x, **dac_weights(1, Q, D, N))
    if i == 1:
        B, T, D, Q, N = 8, 750, 1024, 12, 1024
        x = normal(2, 1, (B * T, D))
        if rows is not None:
            x = x[:rows]
        return dict(kind="dac", seed=2, B=B, T=T, D=D, Q=Q, N=N, x=x, **dac_weights(2, Q, D, N))
    if i == 2:
        M, K, Q, N = 48000, 256, 8, 2048
        M = M if rows is None else rows
        x = normal(3, 1, (M, K))
        cb = np.stack([normal(3, 100 * s + 2, (N, K), 1.0 / 16.0) for s in range(Q)])
        return dict(kind="euclid", seed=3, M=M, K=K, Q=Q, N=N, x=x, codebook=cb)
    if i == 3:
        M, K, N = 200000, 768, 16384
        M = M if rows is None else rows
        z = normal(4, 1, (M, K))
        s = uniform(4, 2, (K,), 0.5, 2.0)
        x = (z * s[None, :]).astype(np.float32)
        cb = normal(4, 3, (N, K), 1.0)[None]
        return dict(kind="kmeans", seed=4, M=M, K=K, Q=1, N=N, x=x, codebook=cb)
    if i == 4:
        M, K, Q, N = 48000, 256, 8, 2048
        M = M if rows is None else rows
        x = normal(5, 1, (M, K))
        cb = np.stack([q8_0_random_codebook(5, 100 * s + 2, N, K) for s in range(Q)])
        return dict(kind="q8_0", seed=5, M=M, K=K, Q=Q, N=N, x=x, codebook_q8=cb, topk=4)
    raise ValueError(f"unknown config {i}")


def q8_0_quantize_ref(rows: np.ndarray) -> np.ndarray:
    """block_q8_0 image of float rows [..., K] with the weight-side rounding
    (quantize_row_q8_0_ref, ggml-quants.c:236-256: d = amax / 127 in fp32,
    id = 1 / d, q = roundf(x * id), d stored as fp16)."""
    x = np.ascontiguousarray(rows, np.float32)
    b = x.reshape(x.shape[:-1] + (x.shape[-1] // Q8_BLOCK, Q8_BLOCK))
    amax = np.abs(b).max(-1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, np.float32(1.0)), np.float32(0.0)).astype(np.float32)
    v = (b * idv[..., None]).astype(np.float32).astype(np.float64)
    q = np.sign(v) * np.floor(np.abs(v) + 0.5)          # roundf: half away from zero
    out = np.zeros(b.shape[:-1], dtype=Q8_DTYPE)
    out["d"] = d.astype(np.float16)
    out["qs"] = q.astype(np.int8)
    return out


# --------------------------------------------------------------------------
# Projected Euclidean RVQ (OmniVoice / Higgs acoustic quantizers; test shapes)

def projected_config(M: int, recipe: int = 1, seed: int = 13, H: int = 1024, K: int = 64, N: int = 1024, Q: int = 8,
                     cb_q8: bool = False, proj_q8: bool = False) -> dict:
    """Inputs of the OmniVoice (recipe 0) / Higgs (recipe 1) quantizer with
    projections, at the reference's shapes (hidden 1024, codebook dim 64,
    1024 codes, 8 stages; higgs_audio_tts/codec.cpp:34-37): x [M, H] ~N(0,1),
    project_in W [Q, K, H] ~N(0, 1/sqrt(H)) with bias ~N(0, 0.1), codebooks
    [Q, N, K] ~N(0, 1), project_out W [Q, H, K] ~N(0, 1/sqrt(K)) with bias
    ~N(0, 0.1).  cb_q8 / proj_q8 store the codebook / the projection weights
    as GGUF Q8_0 (weight-side rounding), as a Q8_0 codec weight type does."""
    x = normal(seed, 1, (M, H))
    w_in = np.stack([normal(seed, 100 * s + 2, (K, H), 1.0 / np.sqrt(H)) for s in range(Q)])
    b_in = np.stack([normal(seed, 100 * s + 3, (K,), 0.1) for s in range(Q)])
    cb = np.stack([normal(seed, 100 * s + 4, (N, K), 1.0) for s in range(Q)])
    w_out = np.stack([normal(seed, 100 * s + 5, (H, K), 1.0 / np.sqrt(K)) for s in range(Q)])
    b_out = np.stack([normal(seed, 100 * s + 6, (H,), 0.1) for s in range(Q)])
    cfg = dict(kind="projected", seed=seed, recipe=recipe, M=M, H=H, K=K, Q=Q, N=N, x=x, b_in=b_in, b_out=b_out)
    if cb_q8:
        cfg["codebook_q8"] = q8_0_quantize_ref(cb)
    else:
        cfg["codebook"] = cb
    if proj_q8:
        cfg["w_in_q8"] = q8_0_quantize_ref(w_in)
        cfg["w_out_q8"] = q8_0_quantize_ref(w_out)
    else:
        cfg["w_in"] = w_in
        cfg["w_out"] = w_out
    return cfg


def fish_config(B: int, T: int, seed: int = 15, D: int = 1024, N0: int = 4096, N: int = 1024, Qr: int = 8,
                bias: bool = True) -> dict:
    """The Fish Audio quantizer cascade (fish_audio/codec.cpp:570-611): a
    semantic stage of N0 = 4096 codes, then Qr residual stages of N = 1024
    codes, all dim 8, latent dim D; DAC-style weights (dac_weights) with the
    semantic codebook [N0, 8] ~N(0,1) drawn separately."""
    Q = 1 + Qr
    w = dac_weights(seed, Q, D, N, bias=bias)
    cb0 = normal(seed, 7, (N0, DAC_DIM), 1.0)
    return dict(kind="fish", seed=seed, B=B, T=T, D=D, Q=Q, N0=N0, N=N, x=normal(seed, 1, (B * T, D)),
                w_in=w["w_in"], b_in=w["b_in"], codebook0=cb0, codebook=np.ascontiguousarray(w["codebook"][1:]),
                w_out=w["w_out"], b_out=w["b_out"])


def qwen3_config(frames: int, seed: int = 14, S: int = 16, N: int = 2048, K: int = 256) -> dict:
    """Qwen3-TTS speech-tokenizer quantizer inputs (tokenizer_speech_encoder.cpp
    shapes: 1 semantic + 15 acoustic EMA codebooks of 2048 x 256): the
    encoder's projected semantic and acoustic latents channel-major [K, frames]
    ~N(0,1) as the graph leaves them, cluster_usage [S, N] ~U(1, 30) and
    embedding_sum = usage * N(0, 1/4) per row, so the codebooks
    (embedding_sum / usage) are close to N(0, 1/4)."""
    usage = uniform(seed, 1, (S, N), 1.0, 30.0)
    es = (normal(seed, 2, (S, N, K), 0.25) * usage[..., None]).astype(np.float32)
    return dict(kind="qwen3", seed=seed, frames=frames, S=S, N=N, K=K, embedding_sum=es, cluster_usage=usage,
                semantic=normal(seed, 3, (K, frames)), acoustic=normal(seed, 4, (K, frames)))


# --------------------------------------------------------------------------
# Host-loop DAC quantizers (test shapes; not BASELINE configs)

def outetts_config(M: int, seed: int = 11, D: int = 1024, Q: int = 2, N: int = 1024, bias: bool = True) -> dict:
    """OuteTTS DAC quantizer inputs (dac.cpp:376-456 shapes: D = N = 1024,
    Q = 2): x [M, D] ~N(0,1) and DAC-style weights with biases."""
    x = normal(seed, 1, (M, D))
    return dict(kind="outetts", seed=seed, M=M, D=D, Q=Q, N=N, x=x, **dac_weights(seed, Q, D, N, bias=bias))


def moss_config(M: int, seed: int = 12, C: int = 768, R: int = 512, Q: int = 12, N: int = 1024) -> dict:
    """MOSS RLFQ quantizer inputs (audio_tokenizer_quantizer.cpp, config
    code_dim 768, rvq_dim 512, 12 x 1024 x 8): hidden [M, C] ~N(0,1); every
    weight-normalised conv as (g ~U(0.5, 2), v ~N(0,1)); biases ~N(0, 0.1);
    codebooks ~N(0,1)."""
    def wn(stream, out_ch, in_ch, lead=()):
        g = uniform(seed, stream, lead + (out_ch,), 0.5, 2.0)
        v = normal(seed, stream + 1, lead + (out_ch, in_ch), 1.0)
        return g, v
    ip_g, ip_v = wn(10, R, C)
    op_g, op_v = wn(20, C, R)
    in_g, in_v = wn(30, 8, R, (Q,))
    out_g, out_v = wn(40, R, 8, (Q,))
    return dict(kind="moss", seed=seed, M=M, C=C, R=R, Q=Q, N=N,
                hidden=normal(seed, 1, (M, C)),
                ip_g=ip_g, ip_v=ip_v, ip_b=normal(seed, 12, (R,), 0.1),
                op_g=op_g, op_v=op_v, op_b=normal(seed, 22, (C,), 0.1),
                in_g=in_g, in_v=in_v, in_b=normal(seed, 32, (Q, 8), 0.1),
                out_g=out_g, out_v=out_v, out_b=normal(seed, 42, (Q, R), 0.1),
                codebook=normal(seed, 50, (Q, N, 8), 1.0))


def near_duplicate_pairs(cb: np.ndarray, seed: int) -> np.ndarray:
    """Codebooks [Q, N, dim] whose odd codes repeat the even code before them
    with one component moved up by one ulp: the winner of each pair depends
    on the last rounding of its score, so a test on them sees arithmetic
    slips (a fused multiply-add, another summation order) as code changes."""
    cb = np.array(cb, np.float32, copy=True)
    rng = np.random.default_rng(seed)
    for s in range(cb.shape[0]):
        half = cb.shape[1] // 2
        cb[s, 1::2] = cb[s, 0::2]
        k = rng.integers(0, cb.shape[2], half)
        rows = cb[s, 1::2]
        rows[np.arange(half), k] = np.nextafter(rows[np.arange(half), k], np.float32(np.inf))
        cb[s, 1::2] = rows
    return cb


def moss_fold(cfg: dict) -> dict:
    """The folded conv weights of a moss_config, w = v * (float)(g / |v|) per
    output row with |v|^2 summed in order in double, as the MOSS loader's
    weight-norm reconstruction builds them from (g, v)."""
    def fold(g, v):
        v = np.asarray(v, np.float32)
        v64 = v.astype(np.float64)
        norm = np.cumsum(v64 * v64, axis=-1)[..., -1]
        scale = (np.asarray(g, np.float32).astype(np.float64) / np.sqrt(norm)).astype(np.float32)
        return (v * scale[..., None]).astype(np.float32)
    return dict(w_ip=fold(cfg["ip_g"], cfg["ip_v"]), w_in=fold(cfg["in_g"], cfg["in_v"]),
                w_out=fold(cfg["out_g"], cfg["out_v"]), w_op=fold(cfg["op_g"], cfg["op_v"]))
