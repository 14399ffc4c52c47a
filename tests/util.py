"""Shared helpers for the parity tests: seeded inputs and the error metric.

Tolerance (stated once, used by every floating-point parity test):
  rel_err(y, ref) = max_i |y_i - ref_i| / max_i |ref_i|  <= TOL = 1e-3,
where ref is the fp32 (or fp64) accumulation over identically rounded
operands.  fp16/bf16 outputs must in addition be the round-to-nearest of a
value within ACC_DELTA * max|ref| of ref (rounded_ok): the output rounding is
exact and only the accumulation order may differ from the reference.
Dequantised weights and embedding rows are compared bit for bit.
"""
from __future__ import annotations

import numpy as np

TOL = 1e-3
ACC_DELTA = 1e-4


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def gaussian(seed: int, shape, sigma: float = 1.0) -> np.ndarray:
    return (rng(seed).standard_normal(shape) * sigma).astype(np.float32)


def weights(seed: int, rows: int, K: int, sigma: float = 0.02) -> np.ndarray:
    """Q4_K bytes [rows, K/256*144] of N(0, sigma) weights (CPU quantiser)."""
    from oracle import oracle as orc
    return orc.quantize(gaussian(seed, (rows, K), sigma))


def x_f16(seed: int, shape) -> np.ndarray:
    """fp16 activations N(0,1) as uint16 bits."""
    return gaussian(seed, shape).astype(np.float16).view(np.uint16)


def rel_err(y, ref) -> float:
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = np.max(np.abs(ref))
    if denom == 0:
        return float(np.max(np.abs(y)))
    return float(np.max(np.abs(y - ref)) / denom)


def bits_value(bits, kind: str) -> np.ndarray:
    b = np.asarray(bits, dtype=np.uint16)
    if kind == "f16":
        return b.view(np.float16).astype(np.float64)
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def spacing(bits, kind: str) -> np.ndarray:
    """Distance from |value| to the next larger representable magnitude."""
    mag = np.asarray(bits, dtype=np.uint16) & 0x7FFF
    nxt = np.minimum(mag + 1, 0x7BFF if kind == "f16" else 0x7F7F).astype(np.uint16)
    return np.abs(bits_value(nxt, kind) - bits_value(mag, kind))


def rounded_ok(y_bits, ref, kind: str = "f16", delta: float = ACC_DELTA,
               extra=None) -> np.ndarray:
    """True where the 16-bit output y is RNE of some z with |z - ref| <=
    delta * max|ref|, i.e. |y - ref| <= spacing(y)/2 + delta * max|ref|
    (+ `extra`, an additional per-element allowance such as a first rounding)."""
    y = bits_value(y_bits, kind).reshape(np.shape(ref))
    ref = np.asarray(ref, dtype=np.float64)
    sp = np.maximum(spacing(y_bits, kind).reshape(ref.shape), 0)
    allow = sp / 2 + delta * np.max(np.abs(ref))
    if extra is not None:
        allow = allow + extra
    return np.abs(y - ref) <= allow * (1 + 1e-12)


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """RNE fp32 -> bf16 bits via torch (an implementation independent of the oracle)."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def zipf_ids(seed: int, n: int, vocab: int, s: float = 1.1) -> np.ndarray:
    """Bounded Zipf(s) over ranks 1..vocab by inverse CDF, ranks mapped to ids
    through a seeded permutation (repeats allowed)."""
    r = rng(seed)
    ranks = np.arange(1, vocab + 1, dtype=np.float64)
    cdf = np.cumsum(ranks ** -s)
    cdf /= cdf[-1]
    u = r.random(n)
    rank_idx = np.minimum(np.searchsorted(cdf, u, side="left"), vocab - 1)
    perm = r.permutation(vocab)
    return perm[rank_idx].astype(np.int32)


def gemv_path(N: int, M: int, K: int) -> bool:
    """Whether rxq4_gemm_f16 runs Q4_K with N fp16 tokens on the decode GEMV
    kernels (exact weights) rather than the MFMA kernels (fp16-rounded
    weights): one token always; 2 tokens, and 3 on at least 4 MiB of
    weights, on the multi-token GEMV while its x fits (registers up to 16
    blocks a row, else N * K/256 * 576 bytes of LDS)."""
    if N == 1:
        return True
    if not (N == 2 or (N == 3 and M * (K // 256) * 144 >= 4 << 20)):
        return False
    slots = 4 * (K // 256)
    return (slots <= 64 and 64 % slots == 0) or N * (K // 256) * 576 <= 160 * 1024
