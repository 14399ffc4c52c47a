"""Q5_K / Q6_K test blocks, packed from the GGML block description.

Written from the format description, not from the oracle: each weight's
quantised value, scale, min and high bits are placed by index, so a test can
compare the oracle's (and the GPU's) dequantisation with the closed form.

Q6_K (210 B per 256 weights): ql[128] @0, qh[64] @128, int8 scales[16] @192,
fp16 d @208.  Weight i = 128*h + 32*j + l (h < 2, j < 4, l < 32) has its low
4 bits in nibble (j >> 1) of ql[64*h + 32*(j & 1) + l], its high 2 bits at
bit 2*j of qh[32*h + l], scale scales[i // 16]; w = d * scale * (q - 32).

Q5_K (176 B): fp16 d @0, fp16 dmin @2, scales[12] @4 (the Q4_K 6-bit
scale/min packing), qh[32] @16, qs[128] @48.  Weight i = 64*il + 32*hi + l
has its low 4 bits in nibble hi of qs[32*il + l] and its fifth bit at bit
2*il + hi of qh[l]; sub-block 2*il + hi; w = d*sc*q - dmin*m.
"""
from __future__ import annotations

import numpy as np

Q5_BYTES, Q6_BYTES = 176, 210

_i = np.arange(256)


def pack_scale_min(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """6-bit scales/mins [..., 8] -> the 12-byte K-quant packing."""
    sc = sc.astype(np.uint8)
    mn = mn.astype(np.uint8)
    out = np.zeros(sc.shape[:-1] + (12,), np.uint8)
    for j in range(4):
        out[..., j] = (sc[..., j] & 63) | ((sc[..., j + 4] >> 4) << 6)
        out[..., j + 4] = (mn[..., j] & 63) | ((mn[..., j + 4] >> 4) << 6)
        out[..., j + 8] = (sc[..., j + 4] & 15) | ((mn[..., j + 4] & 15) << 4)
    return out


def pack_q6k(q: np.ndarray, sc: np.ndarray, d16: np.ndarray) -> np.ndarray:
    """q [R, nb, 256] in 0..63, sc [R, nb, 16] int8, d16 [R, nb] fp16 bits
    -> uint8 [R, nb * 210]."""
    R, nb = q.shape[:2]
    q = q.astype(np.uint8)
    out = np.zeros((R, nb, Q6_BYTES), np.uint8)
    h, j, l = _i // 128, (_i % 128) // 32, _i % 32
    for i in range(256):
        out[:, :, 64 * h[i] + 32 * (j[i] & 1) + l[i]] |= ((q[:, :, i] & 15) << int(4 * (j[i] >> 1))).astype(np.uint8)
        out[:, :, 128 + 32 * h[i] + l[i]] |= ((q[:, :, i] >> 4) << int(2 * j[i])).astype(np.uint8)
    out[:, :, 192:208] = sc.astype(np.int8).view(np.uint8)
    d16 = np.asarray(d16, np.uint16)
    out[:, :, 208] = d16 & 0xFF
    out[:, :, 209] = d16 >> 8
    return out.reshape(R, nb * Q6_BYTES)


def pack_q5k(q, sc, mn, d16, dmin16) -> np.ndarray:
    """q [R, nb, 256] in 0..31, sc/mn [R, nb, 8] in 0..63, d16/dmin16 [R, nb]
    fp16 bits -> uint8 [R, nb * 176]."""
    R, nb = q.shape[:2]
    q = q.astype(np.uint8)
    out = np.zeros((R, nb, Q5_BYTES), np.uint8)
    d16 = np.asarray(d16, np.uint16)
    dmin16 = np.asarray(dmin16, np.uint16)
    out[:, :, 0], out[:, :, 1] = d16 & 0xFF, d16 >> 8
    out[:, :, 2], out[:, :, 3] = dmin16 & 0xFF, dmin16 >> 8
    out[:, :, 4:16] = pack_scale_min(sc, mn)
    il, hi, l = _i // 64, (_i % 64) // 32, _i % 32
    for i in range(256):
        out[:, :, 48 + 32 * il[i] + l[i]] |= ((q[:, :, i] & 15) << int(4 * hi[i])).astype(np.uint8)
        out[:, :, 16 + l[i]] |= (((q[:, :, i] >> 4) & 1) << int(2 * il[i] + hi[i])).astype(np.uint8)
    return out.reshape(R, nb * Q5_BYTES)


def expected_q6k(q, sc, d16) -> np.ndarray:
    """Closed form d * sc[i // 16] * (q - 32) (exact in fp32) -> [R, nb*256]."""
    d = np.asarray(d16, np.uint16).view(np.float16).astype(np.float64)
    s = np.repeat(sc.astype(np.float64), 16, axis=-1)
    w = d[..., None] * s * (q.astype(np.float64) - 32)
    return w.astype(np.float32).reshape(q.shape[0], -1)


def expected_q5k(q, sc, mn, d16, dmin16) -> np.ndarray:
    """(d*sc)*q - dmin*m: both products exact in fp32, one fp32 rounding."""
    d = np.asarray(d16, np.uint16).view(np.float16).astype(np.float32)
    dm = np.asarray(dmin16, np.uint16).view(np.float16).astype(np.float32)
    s = np.repeat(sc.astype(np.float32), 32, axis=-1)
    m = np.repeat(mn.astype(np.float32), 32, axis=-1)
    w = (d[..., None] * s) * q.astype(np.float32) - dm[..., None] * m
    return w.astype(np.float32).reshape(q.shape[0], -1)


def _d16(rng, shape, lo_exp=-17, hi_exp=-11):
    """fp16 bits of positive values 2^lo_exp .. 2^hi_exp (subnormals below
    2^-14 included)."""
    v = np.exp2(rng.uniform(lo_exp, hi_exp, shape)).astype(np.float16)
    return v.view(np.uint16)


def random_q6k(rng, rows: int, K: int):
    """Random Q6_K rows: every q and every int8 scale value can occur."""
    nb = K // 256
    q = rng.integers(0, 64, (rows, nb, 256))
    sc = rng.integers(-128, 128, (rows, nb, 16))
    d16 = _d16(rng, (rows, nb))
    return pack_q6k(q, sc, d16), (q, sc, d16)


def random_q5k(rng, rows: int, K: int):
    nb = K // 256
    q = rng.integers(0, 32, (rows, nb, 256))
    sc = rng.integers(0, 64, (rows, nb, 8))
    mn = rng.integers(0, 64, (rows, nb, 8))
    d16 = _d16(rng, (rows, nb), -14, -9)
    dmin16 = _d16(rng, (rows, nb), -15, -10)
    return pack_q5k(q, sc, mn, d16, dmin16), (q, sc, mn, d16, dmin16)


def random_blocks(t: int, rng, rows: int, K: int) -> np.ndarray:
    """Raw rows of ggml type t (13 or 14) with weights of order 0.01..0.1."""
    return (random_q5k if t == 13 else random_q6k)(rng, rows, K)[0]
