"""The host GEMV (rxq4_host_gemv), the path the C++ API takes for weights the
GPU cannot read and under JLLM_FAST_GEMV=0 (reference q4_gemm.cu:1886-1899,
1916-1947, 1994-2016), checked on the CPU against the oracle's restatement of
gemv_quant_cpu (q4_gemm.cu:1742-1854): every output bit for bit, fp32 and
fp16 outputs and the residual's double rounding, Q4_K / Q5_K / Q6_K, on the
single-thread and the row-parallel schedule.  No GPU call is made.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc
from tests import util

rxq4 = pytest.importorskip("rxq4")
from rxq4 import capi  # noqa: E402


def _weights(seed, rows, K, t):
    src = util.gaussian(seed, (rows, K), 0.02)
    return orc.quantize(src) if t == 12 else orc.quantize_ggml(src, t)


def _oracle_f32(W, K, t, x16):
    return orc.gemv_f32(W, K, x16) if t == 12 else orc.kq_gemv_f32(W, K, t, x16)


@pytest.mark.parametrize("t", [12, 13, 14])
@pytest.mark.parametrize("rows,K", [(1, 256), (7, 512), (33, 2048), (5, 11008)])
def test_host_gemv_f32_bit_exact(t, rows, K):
    W = _weights(100 + rows + t, rows, K, t)
    x = util.x_f16(200 + K, K)
    y = capi.host_gemv(W, x, rows, K, t, "f32")
    ref = _oracle_f32(W, K, t, x)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("t", [12, 13, 14])
def test_host_gemv_row_parallel_bit_exact(t):
    # 2048 x 2048 takes the multi-threaded schedule; rows are independent
    W = _weights(300 + t, 2048, 2048, t)
    x = util.x_f16(301, 2048)
    y = capi.host_gemv(W, x, 2048, 2048, t, "f32")
    assert np.array_equal(y.view(np.uint32), _oracle_f32(W, 2048, t, x).view(np.uint32))


def test_host_gemv_f16_and_add_bit_exact():
    W = _weights(400, 64, 2048, 12)
    x = util.x_f16(401, 2048)
    res = util.x_f16(402, 64)
    assert np.array_equal(capi.host_gemv(W, x, 64, 2048, 12, "f16"), orc.gemv_f16(W, 2048, x))
    assert np.array_equal(capi.host_gemv(W, x, 64, 2048, 12, "f16", residual=res),
                          orc.gemv_add_f16(W, 2048, x, res))


def test_host_gemv_fp16_rounding_over_the_whole_range():
    # y values from fp16 subnormals to overflow (x scaled by powers of two,
    # and a matrix whose d is 2^10 larger): the fp32 -> fp16 rounding must
    # be numpy's round-to-nearest-even everywhere, infinity above 65504
    K, rows = 256, 64
    W = _weights(500, rows, K, 12)
    big = W.reshape(rows, 144).copy()
    d = big[:, 0:2].copy().view(np.float16)[:, 0].astype(np.float32) * np.float32(1024.0)
    big[:, 0:2] = d.astype(np.float16).reshape(rows, 1).view(np.uint8)
    x0 = util.gaussian(501, K)
    seen_sub = seen_inf = False
    for M in (W, big):
        for k in range(-24, 12, 2):
            x = (x0 * np.float32(2.0 ** k)).astype(np.float16).view(np.uint16)
            y16 = capi.host_gemv(M, x, rows, K, 12, "f16")
            y32 = capi.host_gemv(M, x, rows, K, 12, "f32")
            with np.errstate(over="ignore"):
                assert np.array_equal(y16, y32.astype(np.float16).view(np.uint16)), k
            h = y16.view(np.float16)
            seen_inf |= bool(np.isinf(h).any())
            seen_sub |= bool(((h != 0) & (np.abs(h) < np.float16(6.104e-5))).any())
    assert seen_sub and seen_inf


def test_host_gemv_statuses():
    W = _weights(600, 4, 256, 12)
    x = util.x_f16(601, 256)
    with pytest.raises(rxq4.RxQ4Error) as e:
        capi.host_gemv(W, x, 4, 256, 15, "f32")
    assert e.value.status == rxq4.UNSUPPORTED_QUANT_FORMAT
    with pytest.raises(rxq4.RxQ4Error) as e:
        capi.host_gemv(W, x, 4, 255, 12, "f32")
    assert e.value.status == rxq4.INVALID_ARGUMENT
    n = capi.host_gemv_calls()
    assert capi.host_gemv(W, x, 0, 256, 12, "f32").shape == (0,)
    capi.host_gemv(W, x, 4, 256, 12, "f32")
    assert capi.host_gemv_calls() == n + 1
