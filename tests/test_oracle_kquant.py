"""Oracle pins for the Q5_K (13) and Q6_K (14) formats (CPU only).

Every check compares the oracle with something it was not derived from:
the closed-form value of blocks packed by index (tests/kquant_blocks.py),
exact integer arithmetic, one-hot extraction, or an fp64 bound.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc
from tests import kquant_blocks as kb
from tests import util


def test_q6k_dequant_closed_form_random():
    W, (q, sc, d16) = kb.random_q6k(util.rng(600), 5, 1024)
    got = orc.kq_dequant_f32(W, 1024, 14)
    assert np.array_equal(got, kb.expected_q6k(q, sc, d16))


def test_q6k_dequant_exhaustive_values():
    """Every 6-bit q at every position class, every int8 scale, negative and
    subnormal d."""
    R, nb = 4, 4
    q = (np.arange(R * nb * 256).reshape(R, nb, 256) * 37 + 11) % 64
    sc = (np.arange(R * nb * 16).reshape(R, nb, 16) % 256) - 128
    d16 = np.array([[0x3C00, 0xBC00, 0x0001, 0x83FF]] * R, np.uint16)  # 1, -1, min subnormal, -max subnormal
    W = kb.pack_q6k(q, sc, d16)
    assert np.array_equal(orc.kq_dequant_f32(W, nb * 256, 14), kb.expected_q6k(q, sc, d16))


def test_q6k_one_position_moves_one_weight():
    """Changing one q changes exactly the weight the description names."""
    q = np.full((1, 1, 256), 32)
    sc = np.ones((1, 1, 16), np.int64)
    d16 = np.array([[0x3C00]], np.uint16)
    base = orc.kq_dequant_f32(kb.pack_q6k(q, sc, d16), 256, 14)[0]
    assert not base.any()
    for i in (0, 15, 16, 31, 32, 63, 64, 95, 96, 127, 128, 160, 200, 255):
        q2 = q.copy()
        q2[0, 0, i] = 63
        w = orc.kq_dequant_f32(kb.pack_q6k(q2, sc, d16), 256, 14)[0]
        assert np.flatnonzero(w).tolist() == [i] and w[i] == 31.0


def test_q5k_dequant_closed_form():
    W, (q, sc, mn, d16, dm16) = kb.random_q5k(util.rng(601), 6, 768)
    got = orc.kq_dequant_f32(W, 768, 13)
    assert np.array_equal(got, kb.expected_q5k(q, sc, mn, d16, dm16))


def test_q5k_exhaustive_q_and_fifth_bit():
    R, nb = 2, 2
    q = (np.arange(R * nb * 256).reshape(R, nb, 256) * 13 + 5) % 32
    sc = (np.arange(R * nb * 8).reshape(R, nb, 8) * 7) % 64
    mn = (np.arange(R * nb * 8).reshape(R, nb, 8) * 11 + 3) % 64
    d16 = np.array([[0x3C00, 0x2E66]] * R, np.uint16)
    dm16 = np.array([[0x3800, 0x0200]] * R, np.uint16)
    W = kb.pack_q5k(q, sc, mn, d16, dm16)
    assert np.array_equal(orc.kq_dequant_f32(W, nb * 256, 13), kb.expected_q5k(q, sc, mn, d16, dm16))


@pytest.mark.parametrize("t", [13, 14])
def test_kq_gemv_one_hot_selects_a_column(t):
    """The CPU loop (reference gemv_quant_cpu order) and the element-wise
    dequant (embedding kernel order) must agree on every position."""
    K = 512
    W = kb.random_blocks(t, util.rng(610 + t), 7, K)
    dq = orc.kq_dequant_f32(W, K, t)
    for k in range(0, K, 3):
        x = np.zeros(K, np.float16)
        x[k] = 1.0
        y = orc.kq_gemv_f32(W, K, t, x.view(np.uint16))
        assert np.array_equal(y, dq[:, k]), k


def test_kq_gemv_integer_operands_exact():
    rng = util.rng(620)
    K, R = 1024, 9
    # Q6_K with d = 1: integer weights sc*(q-32), |w| <= 4*32
    q = rng.integers(0, 64, (R, K // 256, 256))
    sc = rng.integers(-4, 5, (R, K // 256, 16))
    W6 = kb.pack_q6k(q, sc, np.full((R, K // 256), 0x3C00, np.uint16))
    # Q5_K with d = dmin = 1: w = sc*q - m
    q5 = rng.integers(0, 32, (R, K // 256, 256))
    s5 = rng.integers(0, 4, (R, K // 256, 8))
    m5 = rng.integers(0, 4, (R, K // 256, 8))
    one = np.full((R, K // 256), 0x3C00, np.uint16)
    W5 = kb.pack_q5k(q5, s5, m5, one, one)
    x = rng.integers(-2, 3, K).astype(np.float16)
    for t, W, wint in ((14, W6, kb.expected_q6k(q, sc, one)),
                       (13, W5, kb.expected_q5k(q5, s5, m5, one, one))):
        exact = wint.astype(np.int64) @ x.astype(np.int64)
        assert np.array_equal(orc.kq_gemv_f32(W, K, t, x.view(np.uint16)), exact.astype(np.float32))


@pytest.mark.parametrize("t", [13, 14])
def test_kq_gemv_fp64_bound(t):
    K = 2048
    W = kb.random_blocks(t, util.rng(630 + t), 16, K)
    x16 = util.x_f16(631, K)
    xv = x16.view(np.float16).astype(np.float32)
    y = orc.kq_gemv_f32(W, K, t, x16).astype(np.float64)
    dq = orc.kq_dequant_f32(W, K, t).astype(np.float64)
    y64 = dq @ xv.astype(np.float64)
    assert np.allclose(orc.kq_gemm_f64(W, K, t, xv, None)[0], y64, rtol=1e-12, atol=0)
    bound = (K + 2) * 2.0 ** -24 * (np.abs(dq) @ np.abs(xv.astype(np.float64)))
    assert np.all(np.abs(y - y64) <= bound)


def test_kq_type12_forwards_to_q4k():
    K = 512
    W = util.weights(640, 5, K)
    x16 = util.x_f16(641, K)
    assert np.array_equal(orc.kq_gemv_f32(W, K, 12, x16), orc.gemv_f32(W, K, x16))
    assert np.array_equal(orc.kq_dequant_f32(W, K, 12), orc.dequant_f32(W, K))


def test_kq_embed_is_rne_of_dequant_and_zero_out_of_range():
    K = 512
    W = kb.random_blocks(14, util.rng(650), 11, K)
    ids = np.array([3, 0, 10, -1, 11, 3], np.int32)
    got = orc.kq_embed_rows_f16(W, K, 14, ids)
    dq = orc.kq_dequant_f32(W, K, 14)
    for i, r in enumerate(ids):
        want = dq[r].astype(np.float16).view(np.uint16) if 0 <= r < 11 else np.zeros(K, np.uint16)
        assert np.array_equal(got[i], want)
