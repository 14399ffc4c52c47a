"""Pins the CPU oracle (oracle/q4k_oracle.c) with checks that do not restate it.

Each test names the oracle function it pins and the independent fact used:
numpy's / torch's own IEEE conversions, a separately written numpy decoder of
the GGML Q4_K layout (reference q4_gemm.cu:147-154, 192-202, 545-572),
closed forms, exact integer arithmetic, an fp64 error bound, and a
pure-Python float32 transcription of the reference loop
(q4_gemm.cu:1750-1784) on tiny shapes.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc
from tests import util

QK = 256
BB = 144


# --------------------------------------------------------------- conversions
def test_fp16_decode_all_patterns():
    """orc_fp16_to_f32 == numpy float16->float32 for all 65536 patterns."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = orc.fp16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def _fp16_tie_inputs():
    h = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16)  # finite, positive
    lo = h[:-1].view(np.float16).astype(np.float64)
    hi = h[1:].view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)  # exact: fp16 neighbours' midpoint fits fp32
    u = mid.view(np.uint32)
    cand = np.concatenate([u, u - 1, u + 1]).view(np.float32)
    return np.concatenate([cand, -cand])


def test_f32_to_fp16_ties_and_random():
    """orc_f32_to_fp16 == numpy's RNE float32->float16 on every fp16 midpoint
    (+-1 ulp), overflow / underflow boundaries and random bit patterns."""
    r = util.rng(1)
    rand = r.integers(0, 2**32, size=150_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    special = np.array([65504, 65519.996, 65520, 65536, 1e30, np.inf, -np.inf, 2**-24, 2**-25,
                        2**-25 * 1.0000001, 3 * 2**-26, 6.1e-5, 0.0, -0.0, 1e-40],
                       dtype=np.float32)
    vals = np.concatenate([_fp16_tie_inputs(), rand, special])
    vals = vals[~np.isnan(vals)]
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    ours = orc.f32_to_fp16(vals)
    bad = np.nonzero(ours != ref)[0]
    assert bad.size == 0, (vals[bad[:5]], ours[bad[:5]], ref[bad[:5]])
    nan_out = orc.f32_to_fp16(np.array([np.nan], np.float32))[0]
    assert (nan_out & 0x7C00) == 0x7C00 and (nan_out & 0x3FF) != 0


def test_f32_to_bf16_matches_torch():
    """orc_f32_to_bf16 == torch's RNE cast, including exact ties."""
    r = util.rng(2)
    rand = r.integers(0, 2**32, size=100_000, dtype=np.uint64).astype(np.uint32)
    ties = (r.integers(0, 2**16, size=20_000, dtype=np.uint64).astype(np.uint32) << 16) | 0x8000
    u = np.concatenate([rand, ties, ties ^ 1, ties - 1]).view(np.float32)
    u = u[np.isfinite(u)]
    ref = util.f32_to_bf16_bits(u)
    ours = orc.f32_to_bf16(u)
    assert np.array_equal(ours, ref)


# ------------------------------------------------------- scale / min packing
def np_pack_scales(sc, mn) -> np.ndarray:
    """Independent numpy statement of the GGML 12-byte layout: bytes 0-3 hold
    sc[0..3] in bits 0-5 and bits 4-5 of sc[4..7] in bits 6-7; bytes 4-7 the
    same for m; bytes 8-11 hold sc[4..7] bits 0-3 (low nibble) and m[4..7]
    bits 0-3 (high nibble)."""
    sc = np.asarray(sc, dtype=np.uint32)
    mn = np.asarray(mn, dtype=np.uint32)
    out = np.zeros(12, dtype=np.uint32)
    out[0:4] = (sc[0:4] & 0x3F) | ((sc[4:8] & 0x30) << 2)
    out[4:8] = (mn[0:4] & 0x3F) | ((mn[4:8] & 0x30) << 2)
    out[8:12] = (sc[4:8] & 0x0F) | ((mn[4:8] & 0x0F) << 4)
    return out.astype(np.uint8)


def test_scale_pack_known_vector():
    """A hand-checked vector: sc = 0,1,2,3,60,61,62,63; m = 63,62,61,60,16,17,48,33."""
    sc = [0, 1, 2, 3, 60, 61, 62, 63]
    mn = [63, 62, 61, 60, 16, 17, 48, 33]
    expect = np.array([0xC0, 0xC1, 0xC2, 0xC3, 0x7F, 0x7E, 0xFD, 0xBC,
                       0x0C, 0x1D, 0x0E, 0x1F], dtype=np.uint8)
    assert np.array_equal(np_pack_scales(sc, mn), expect)
    assert np.array_equal(orc.pack_scale_min_k4(sc, mn), expect)
    for j in range(8):
        assert orc.get_scale_min_k4(j, expect) == (sc[j], mn[j])


def test_scale_unpack_exhaustive():
    """orc_get_scale_min_k4 inverts the independent packer for every (sc, m)
    in 64x64 at every sub-block index, with random neighbours."""
    r = util.rng(3)
    for j in range(8):
        for s in range(64):
            for m in range(0, 64, 1):
                sc = r.integers(0, 64, 8)
                mn = r.integers(0, 64, 8)
                sc[j], mn[j] = s, m
                packed = np_pack_scales(sc, mn)
                got = orc.get_scale_min_k4(j, packed)
                assert got == (s, m)
            # full vector once per (j, s): every other index still decodes
            for jj in range(8):
                assert orc.get_scale_min_k4(jj, packed) == (sc[jj], mn[jj])


def test_oracle_packer_matches_independent_packer():
    r = util.rng(4)
    for _ in range(2000):
        sc = r.integers(0, 64, 8)
        mn = r.integers(0, 64, 8)
        assert np.array_equal(orc.pack_scale_min_k4(sc, mn), np_pack_scales(sc, mn))


# ------------------------------------------------------------------ dequant
def np_dequant(W: np.ndarray, K: int) -> np.ndarray:
    """Vectorised numpy dequantiser written from the format description:
    element e of a block has quant byte qs[32*(e//64) + e%32], low nibble if
    e%64 < 32 else high nibble, sub-block e//32; w = (d*sc)*q - dmin*m (fp32)."""
    nb = K // QK
    blk = np.asarray(W, dtype=np.uint8).reshape(-1, BB)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    dmin = blk[:, 2:4].copy().view(np.float16).astype(np.float32).ravel()
    s = blk[:, 4:16].astype(np.uint32)
    sc = np.empty((blk.shape[0], 8), np.uint32)
    mn = np.empty((blk.shape[0], 8), np.uint32)
    sc[:, 0:4] = s[:, 0:4] & 0x3F
    mn[:, 0:4] = s[:, 4:8] & 0x3F
    sc[:, 4:8] = (s[:, 8:12] & 0x0F) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:8] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    qs = blk[:, 16:].astype(np.uint32)
    e = np.arange(QK)
    byte = qs[:, 32 * (e // 64) + e % 32]
    q = np.where((e % 64) < 32, byte & 0xF, byte >> 4).astype(np.float32)
    sub = e // 32
    ds = d[:, None] * sc[:, sub].astype(np.float32)
    dm = dmin[:, None] * mn[:, sub].astype(np.float32)
    w = ds * q - dm
    return w.reshape(-1, nb * QK)


def random_blocks(seed: int, rows: int, K: int, dscale=None) -> np.ndarray:
    """Random Q4_K bytes with finite d/dmin (random fp16 incl. subnormals and
    negatives) and random scales / quants."""
    r = util.rng(seed)
    nb = K // QK
    W = r.integers(0, 256, size=(rows * nb, BB), dtype=np.uint64).astype(np.uint8)
    hdr = W[:, 0:4].copy().view(np.uint16)
    if dscale is None:
        bad = (hdr & 0x7C00) == 0x7C00  # inf / nan -> clear exponent MSB
        hdr[bad] &= 0xBFFF
    else:
        hdr[:] = np.asarray(dscale, dtype=np.float16).view(np.uint16)
    W[:, 0:4] = hdr.view(np.uint8).reshape(-1, 4)
    return W.reshape(rows, nb * BB)


@pytest.mark.parametrize("K", [256, 2048, 11008])
def test_dequant_matches_independent_decoder(K):
    W = random_blocks(10 + K, 6, K)
    ours = orc.dequant_f32(W, K)
    ref = np_dequant(W, K)
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


def test_dequant_f16_bf16_are_rne_of_f32():
    K = 2048
    W = random_blocks(11, 8, K)
    f32 = orc.dequant_f32(W, K)
    with np.errstate(over="ignore"):
        assert np.array_equal(orc.dequant_f16(W, K), f32.astype(np.float16).view(np.uint16))
    assert np.array_equal(orc.dequant_bf16(W, K), util.f32_to_bf16_bits(f32))


def _block(d, dmin, sc, mn, qbyte):
    b = np.zeros(BB, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:4] = np.array([dmin], np.float16).view(np.uint8)
    b[4:16] = np_pack_scales(sc, mn)
    b[16:] = qbyte
    return b


def test_dequant_closed_forms():
    """q = 0 gives -dmin*m; q = 15 gives 15*d*sc - dmin*m; d = 0 gives -dmin*m;
    dmin = 0 gives d*sc*q; a subnormal d scales exactly."""
    sc = np.arange(8) * 9 % 64
    mn = (np.arange(8) * 7 + 3) % 64
    sub = np.repeat(np.arange(8), 32)
    cases = [
        (0.5, 0.25, 0x00, lambda: -np.float32(0.25) * mn[sub]),
        (0.5, 0.25, 0xFF, lambda: np.float32(0.5) * sc[sub] * 15 - np.float32(0.25) * mn[sub]),
        (0.0, 0.125, 0x5A, lambda: -np.float32(0.125) * mn[sub]),
        (-2.0, 0.0, 0x11, lambda: np.float32(-2.0) * sc[sub] * 1.0),
        (2.0**-24, 0.0, 0xFF, lambda: np.float32(2.0**-24) * sc[sub] * 15),
    ]
    for d, dmin, qb, expect in cases:
        got = orc.dequant_f32(_block(d, dmin, sc, mn, qb), QK)[0]
        assert np.array_equal(got, np.asarray(expect(), np.float32)), (d, dmin, qb)


def test_embed_rows_gather_and_oob():
    K = 512
    W = random_blocks(12, 10, K)
    ids = np.array([3, 3, 0, 9, -1, 10, 5], np.int32)
    out = orc.embed_rows_f16(W, K, ids)
    full = orc.dequant_f16(W, K)
    for i, t in enumerate(ids):
        if 0 <= t < 10:
            assert np.array_equal(out[i], full[t])
        else:
            assert not out[i].any()


# --------------------------------------------------------------------- GEMV
def test_gemv_one_hot_selects_a_column():
    """x = e_k: y[row] is exactly the dequantised weight w[row, k]."""
    K = 2048
    W = util.weights(20, 40, K)
    w = orc.dequant_f32(W, K)
    for k in (0, 31, 32, 63, 64, 255, 256, 1000, 2047):
        x = np.zeros(K, np.float16)
        x[k] = 1.0
        y = orc.gemv_f32(W, K, x.view(np.uint16))
        assert np.array_equal(y, w[:, k]), k


def test_gemv_integer_operands_exact():
    """d = dmin = 1 and small integer x: every product and partial sum is an
    integer below 2^24, so the fp32 result equals the int64 dot product."""
    K, M = 2048, 24
    r = util.rng(21)
    nb = K // QK
    blocks = []
    for _ in range(M * nb):
        blocks.append(_block(1.0, 1.0, r.integers(0, 64, 8), r.integers(0, 64, 8),
                             r.integers(0, 256, 128)))
    W = np.stack(blocks).reshape(M, nb * BB)
    wint = np_dequant(W, K).astype(np.int64)
    x = r.integers(-4, 5, K)
    y = orc.gemv_f32(W, K, x.astype(np.float16).view(np.uint16))
    assert np.array_equal(y.astype(np.int64), wint @ x)


def test_gemv_fp64_error_bound():
    """|y32 - y64| <= 2*K*2^-24 * sum|w*x| (recursive-summation bound)."""
    K, M = 11008, 64
    W = util.weights(22, M, K)
    x16 = util.x_f16(23, K)
    x32 = x16.view(np.float16).astype(np.float32)
    y = orc.gemv_f32(W, K, x16).astype(np.float64)
    y64 = orc.gemv_f64(W, K, x32)
    w = orc.dequant_f32(W, K).astype(np.float64)
    bound = 2 * K * 2.0**-24 * (np.abs(w) @ np.abs(x32.astype(np.float64)))
    assert np.all(np.abs(y - y64) <= bound)
    assert np.allclose(y64, w @ x32.astype(np.float64), rtol=1e-12, atol=1e-12)


def py_gemv_row(W, K, x16, row):
    """Pure-Python float32 transcription of gemv_quant_cpu's Q4_K loop
    (q4_gemm.cu:1753-1784): blocks in order; per 64 elements, 32 low nibbles
    then 32 high nibbles; acc += (d1*q - dm1) * x, all in float32."""
    f32 = np.float32
    nb = K // QK
    blk = np.asarray(W, np.uint8).reshape(-1, nb, BB)[row]
    x = np.asarray(x16, np.uint16).view(np.float16).astype(np.float32)
    acc = f32(0)
    for b in range(nb):
        raw = blk[b]
        dall = f32(raw[0:2].view(np.float16)[0])
        dmin = f32(raw[2:4].view(np.float16)[0])
        s = raw[4:16]
        for il in range(4):
            pair = []
            for j in (2 * il, 2 * il + 1):
                if j < 4:
                    sc, m = int(s[j]) & 63, int(s[j + 4]) & 63
                else:
                    sc = (int(s[j + 4]) & 0xF) | ((int(s[j - 4]) >> 6) << 4)
                    m = (int(s[j + 4]) >> 4) | ((int(s[j]) >> 6) << 4)
                pair.append((f32(dall * f32(sc)), f32(dmin * f32(m))))
            q = raw[16 + 32 * il: 16 + 32 * il + 32]
            k = b * QK + 64 * il
            for l in range(32):
                acc = f32(acc + f32(f32(f32(pair[0][0] * f32(int(q[l]) & 0xF)) - pair[0][1]) * x[k + l]))
            for l in range(32):
                acc = f32(acc + f32(f32(f32(pair[1][0] * f32(int(q[l]) >> 4)) - pair[1][1]) * x[k + 32 + l]))
    return acc


def test_gemv_bit_exact_vs_python_transcription():
    """Bit-exact on tiny shapes, including an input built so that summation
    order changes the result (the order itself is what is pinned)."""
    K = 512
    W = util.weights(24, 3, K)
    x = util.gaussian(25, K)
    x[:32] *= 3000.0   # large early terms: later small terms round differently
    x16 = x.astype(np.float16).view(np.uint16)
    y = orc.gemv_f32(W, K, x16)
    for row in range(3):
        assert y[row].view(np.uint32) == py_gemv_row(W, K, x16, row).view(np.uint32)
    # the same terms summed in reverse order differ: the check is order-sensitive
    w = orc.dequant_f32(W, K)
    xf = x16.view(np.float16).astype(np.float32)
    diffs = 0
    for row in range(3):
        rv = np.float32(0)
        for k in reversed(range(K)):
            rv = np.float32(rv + np.float32(w[row, k] * xf[k]))
        diffs += int(rv != y[row])
    assert diffs >= 1


def test_gemv_f16_and_add_rounding():
    """fp16 output is RNE(fp32); the add variant rounds twice
    (q4_gemm.cu:1941-1945), checked with numpy float16 arithmetic."""
    K = 2048
    W = util.weights(26, 300, K)
    x16 = util.x_f16(27, K)
    res16 = util.x_f16(28, 300)
    y32 = orc.gemv_f32(W, K, x16)
    assert np.array_equal(orc.gemv_f16(W, K, x16), y32.astype(np.float16).view(np.uint16))
    proj = y32.astype(np.float16).astype(np.float32)
    expect = (proj + res16.view(np.float16).astype(np.float32)).astype(np.float16)
    assert np.array_equal(orc.gemv_add_f16(W, K, x16, res16), expect.view(np.uint16))


def test_gemm_tokens_is_per_token_gemv_and_mt_is_bit_identical():
    K, M, N = 1024, 50, 5
    W = util.weights(29, M, K)
    x16 = util.x_f16(30, (N, K))
    y = orc.gemm_tokens_f32(W, K, x16)
    for t in range(N):
        assert np.array_equal(y[t], orc.gemv_f32(W, K, x16[t]))
        assert np.array_equal(orc.gemv_f32(W, K, x16[t], threads=4), y[t])


def test_gemm_f64_matches_numpy():
    K, M, N = 512, 33, 7
    W = util.weights(31, M, K)
    x = util.gaussian(32, (N, K))
    for kind in ("f16", "bf16"):
        y = orc.gemm_f64(W, K, x, kind)
        w = orc.dequant_f32(W, K)
        if kind == "f16":
            wr = w.astype(np.float16).astype(np.float64)
        else:
            wr = orc.bits_bf16_to_f32(util.f32_to_bf16_bits(w)).astype(np.float64)
        assert np.allclose(y, x.astype(np.float64) @ wr.T, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- quantiser
def test_quantizer_round_trip_bound():
    """Each value is reproduced within half a quant step plus the scale
    rounding; the RMS error is a few percent of the signal."""
    K, M = 2048, 64
    src = util.gaussian(33, (M, K), 0.02)
    W = orc.quantize(src)
    deq = orc.dequant_f32(W, K)
    blk = W.reshape(-1, BB)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    dmin = blk[:, 2:4].copy().view(np.float16).astype(np.float32).ravel()
    err = np.abs(deq - src).reshape(-1, QK)
    # step <= d*63; scale rounding costs <= d/2 per unit of q (q <= 15) and dmin/2
    bound = (d * 63) / 2 + 8 * d + dmin / 2
    assert np.all(err.max(axis=1) <= bound * 1.0001)
    rms = np.sqrt(np.mean((deq - src) ** 2)) / np.sqrt(np.mean(src ** 2))
    assert rms < 0.12


def test_quantizer_headers_follow_definition():
    """d and dmin are fp16(max span / 63) and fp16(max offset / 63)."""
    src = util.gaussian(34, (4, 512), 0.02)
    W = orc.quantize(src).reshape(-1, BB)
    v = src.reshape(-1, 8, 32)
    mo = np.maximum(-v.min(axis=2), 0)
    span = (np.maximum(v.max(axis=2), 0) + mo) / np.float32(15)
    d = (span.max(axis=1) / np.float32(63)).astype(np.float16)
    dmin = (mo.max(axis=1) / np.float32(63)).astype(np.float16)
    assert np.array_equal(W[:, 0:2].copy().view(np.float16).ravel(), d)
    assert np.array_equal(W[:, 2:4].copy().view(np.float16).ravel(), dmin)
