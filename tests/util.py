"""Shared helpers for the parity tests: seeded inputs and the error metric.

Tolerance (stated once, used by every floating-point parity test):
  rel_err(y, ref) = max_i |y_i - ref_i| / max_i |ref_i|  <= TOL = 1e-3,
where ref is the fp32 (or fp64) accumulation over identically rounded
operands.  fp16/bf16 outputs are additionally required to lie within
ULPS_OUT units in the last place of RNE(ref).  Dequantised weights and
embedding rows are compared bit for bit.
"""
from __future__ import annotations

import numpy as np

TOL = 1e-3
ULPS_OUT = 1


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


def f16_ulp_dist(a_bits, b_bits) -> np.ndarray:
    """Distance in fp16 ulps between two fp16 bit arrays (finite values)."""
    def key(b):
        b = np.asarray(b, dtype=np.int32)
        return np.where(b & 0x8000, 0x8000 - (b & 0x7FFF), 0x8000 + (b & 0x7FFF))
    return np.abs(key(a_bits) - key(b_bits))


def bf16_ulp_dist(a_bits, b_bits) -> np.ndarray:
    return f16_ulp_dist(a_bits, b_bits)  # same sign-magnitude ordering trick on 16 bits


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
