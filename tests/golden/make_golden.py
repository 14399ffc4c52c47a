"""Writes tests/golden/q4k_golden.npz: small seeded Q4_K fixtures with the
oracle's expected outputs.

The reference ships no fixtures for this path (its tests cover only its
Triton library), so these vectors come from this build's CPU oracle
(oracle/q4k_oracle.c, a restatement of the reference's CPU path, pinned by
tests/test_oracle.py).  They freeze the oracle's results: tests/test_golden.py
re-derives them on the CPU and the GPU tests compare the HIP kernels with them.

Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle as orc  # noqa: E402

CASES = [(16, 512), (3, 2048), (2, 11008)]  # (rows, K)


def make() -> dict:
    out = {}
    for i, (rows, K) in enumerate(CASES):
        r = np.random.default_rng(1000 + i)
        src = (r.standard_normal((rows, K)) * 0.02).astype(np.float32)
        W = orc.quantize(src)
        x16 = (r.standard_normal(K)).astype(np.float16).view(np.uint16)
        res16 = (r.standard_normal(rows)).astype(np.float16).view(np.uint16)
        tag = f"c{i}"
        out[f"{tag}_shape"] = np.array([rows, K], np.int64)
        out[f"{tag}_W"] = W
        out[f"{tag}_x16"] = x16
        out[f"{tag}_res16"] = res16
        out[f"{tag}_deq_f32"] = orc.dequant_f32(W, K).view(np.uint32)
        out[f"{tag}_deq_f16"] = orc.dequant_f16(W, K)
        out[f"{tag}_deq_bf16"] = orc.dequant_bf16(W, K)
        out[f"{tag}_y_f32"] = orc.gemv_f32(W, K, x16).view(np.uint32)
        out[f"{tag}_y_f16"] = orc.gemv_f16(W, K, x16)
        out[f"{tag}_y_add_f16"] = orc.gemv_add_f16(W, K, x16, res16)
    # embedding table [64 x 2048] and a gather with repeats and out-of-range ids
    r = np.random.default_rng(2000)
    table = orc.quantize((r.standard_normal((64, 2048)) * 0.02).astype(np.float32))
    ids = np.array([5, 63, 0, 5, 17, -1, 64, 42], np.int32)
    out["emb_W"] = table
    out["emb_ids"] = ids
    out["emb_rows_f16"] = orc.embed_rows_f16(table, 2048, ids)
    return out


if __name__ == "__main__":
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "q4k_golden.npz")
    np.savez_compressed(path, **make())
    print(path, os.path.getsize(path), "bytes")
