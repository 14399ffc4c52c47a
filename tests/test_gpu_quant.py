"""GPU ggml-compatible quantiser (rxq4_quantize) against its CPU restatement
(oracle/ggml_quant_oracle.c, pinned in tests/test_oracle_quant.py): the
bytes must be identical for Q4_K, Q5_K and Q6_K, on Gaussian rows, partial
workgroups and degenerate blocks (zeros, constants, spikes, positive-only,
subnormal and large magnitudes)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import rxq4
from oracle import oracle as orc
from rxq4 import capi
from tests import util

pytestmark = pytest.mark.gpu


def edge_rows(K: int) -> np.ndarray:
    r = util.rng(1100)
    rows = [np.zeros(K), np.full(K, 0.75), np.linspace(0.01, 0.5, K), -np.linspace(0.01, 0.5, K),
            np.where(np.arange(K) % 97 == 5, -3.0, 0.0), r.standard_normal(K) * 1e-39,
            r.standard_normal(K) * 1e-20, r.standard_normal(K) * 3e4,
            np.round(r.standard_normal(K) * 4) / 8, r.standard_normal(K) ** 3]
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("t", [12, 13, 14])
@pytest.mark.parametrize("rows,K", [(1, 256), (3, 2816), (40, 2048), (7, 11008)])
def test_quantize_bytes_match_oracle(t, rows, K):
    print(f"quantize type {t} rows={rows} K={K}", flush=True)
    x = (util.rng(1110 + rows + t).standard_normal((rows, K)) * 0.02).astype(np.float32)
    got = capi.quantize_ggml(torch.from_numpy(x).cuda(), t).cpu().numpy()
    want = orc.quantize_ggml(x, t)
    assert got.shape == want.shape
    bad = np.nonzero((got != want).any(axis=1))[0]
    assert bad.size == 0, f"rows {bad[:5]} differ"


@pytest.mark.parametrize("t", [12, 13, 14])
def test_quantize_edge_blocks(t):
    x = edge_rows(512)
    got = capi.quantize_ggml(torch.from_numpy(x).cuda(), t).cpu().numpy()
    want = orc.quantize_ggml(x, t)
    for i in range(x.shape[0]):
        assert np.array_equal(got[i], want[i]), f"edge row {i}"


def test_quantize_feeds_the_gemv():
    M, K = 300, 2048
    w = (util.rng(1120).standard_normal((M, K)) * 0.02).astype(np.float32)
    x16 = util.x_f16(1121, K)
    xd = torch.from_numpy(x16.view(np.int16)).cuda()
    for t in (12, 13, 14):
        q = capi.quantize_ggml(torch.from_numpy(w).cuda(), t)
        y = torch.empty(M, dtype=torch.float16, device="cuda")
        capi.gemv_f16(y, q, xd, M, K, ggml_type=t)
        ref = orc.kq_gemv_f32(q.cpu().numpy(), K, t, x16)
        assert util.rounded_ok(y.view(torch.int16).cpu().numpy().view(np.uint16), ref).all()


def test_quantize_argument_checks():
    L = capi.lib()
    src = torch.zeros((2, 256), dtype=torch.float32, device="cuda")
    dst = torch.empty(1024, dtype=torch.uint8, device="cuda")
    assert L.rxq4_quantize(dst.data_ptr(), 15, src.data_ptr(), 2, 256, None) == \
        rxq4.UNSUPPORTED_QUANT_FORMAT
    assert L.rxq4_quantize(dst.data_ptr(), 12, src.data_ptr(), 2, 100, None) == \
        rxq4.INVALID_ARGUMENT
    assert L.rxq4_quantize(dst.data_ptr() + 2, 12, src.data_ptr(), 2, 256, None) == \
        rxq4.INVALID_ARGUMENT
    assert L.rxq4_quantize(dst.data_ptr() + 2, 14, src.data_ptr(), 2, 256, None) == rxq4.SUCCESS
    assert L.rxq4_quantize(dst.data_ptr(), 12, src.data_ptr(), 0, 256, None) == rxq4.SUCCESS
    torch.cuda.synchronize()
