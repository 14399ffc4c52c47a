"""The CPU oracle reproduces the committed golden fixtures bit for bit
(tests/golden/make_golden.py wrote them from the same oracle; this freezes
its behaviour against accidental change)."""
from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "q4k_golden.npz")


def golden():
    return np.load(GOLDEN, allow_pickle=False)


@pytest.mark.parametrize("case", ["c0", "c1", "c2"])
def test_oracle_reproduces_golden(case):
    g = golden()
    rows, K = (int(v) for v in g[f"{case}_shape"])
    W, x16, res16 = g[f"{case}_W"], g[f"{case}_x16"], g[f"{case}_res16"]
    assert W.shape == (rows, K // 256 * 144)
    assert np.array_equal(orc.dequant_f32(W, K).view(np.uint32), g[f"{case}_deq_f32"])
    assert np.array_equal(orc.dequant_f16(W, K), g[f"{case}_deq_f16"])
    assert np.array_equal(orc.dequant_bf16(W, K), g[f"{case}_deq_bf16"])
    assert np.array_equal(orc.gemv_f32(W, K, x16).view(np.uint32), g[f"{case}_y_f32"])
    assert np.array_equal(orc.gemv_f16(W, K, x16), g[f"{case}_y_f16"])
    assert np.array_equal(orc.gemv_add_f16(W, K, x16, res16), g[f"{case}_y_add_f16"])


def test_oracle_reproduces_golden_embedding():
    g = golden()
    assert np.array_equal(orc.embed_rows_f16(g["emb_W"], 2048, g["emb_ids"]), g["emb_rows_f16"])
