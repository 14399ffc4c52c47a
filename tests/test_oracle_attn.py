"""Oracle pins for decode / prefill attention (CPU only).

Each check compares the oracle with something it was not derived from:
closed forms (one position, equal keys, q = 0), the fp64 softmax, the GQA
head-to-KV mapping, int8 KV against fp16 on exactly representable values,
and causality of prefill.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc
from tests import util


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def case(seed, seq, n_heads=8, n_kv=2, hd=64):
    r = util.rng(seed)
    q = f16(r.standard_normal(n_heads * hd))
    k = f16(r.standard_normal((seq, n_kv, hd)))
    v = f16(r.standard_normal((seq, n_kv, hd)))
    return q, k, v


def test_single_position_returns_v():
    q, k, v = case(800, 1)
    out = orc.attn_decode_f32(q, k, v, 8, 2, 64, 1, 0.125)
    vv = v.view(np.float16).astype(np.float32)
    want = np.concatenate([vv[0, h // 4] for h in range(8)])
    assert np.array_equal(out, want)


def test_equal_keys_and_zero_q_give_the_mean():
    seq = 37
    q, k, v = case(801, seq)
    k[:] = k[0]
    vv = v.view(np.float16).astype(np.float64)
    mean = np.concatenate([vv[:, h // 4].mean(axis=0) for h in range(8)])
    out = orc.attn_decode_f32(q, k, v, 8, 2, 64, seq, 0.125)
    assert np.allclose(out, mean, rtol=0, atol=1e-5)
    q0 = np.zeros_like(q)
    _, k2, _ = case(802, seq)
    out0 = orc.attn_decode_f32(q0, k2, v, 8, 2, 64, seq, 0.125)
    assert np.allclose(out0, mean, rtol=0, atol=1e-5)


@pytest.mark.parametrize("seq", [5, 300, 2048])
def test_fp64_bound(seq):
    q, k, v = case(803 + seq, seq, 16, 4, 128)
    out = orc.attn_decode_f32(q, k, v, 16, 4, 128, seq, 1 / np.sqrt(128))
    ref = orc.attn_decode_f64(q, k, v, 16, 4, 128, seq, 1 / np.sqrt(128))
    assert np.max(np.abs(out - ref)) <= 1e-5 * max(1.0, np.max(np.abs(ref)))


def test_gqa_mapping():
    seq = 50
    q, k, v = case(810, seq)
    qq = q.reshape(8, 64).copy()
    qq[1] = qq[0]   # same group (heads 0-3 -> kv head 0)
    qq[4] = qq[0]   # other group (kv head 1)
    out = orc.attn_decode_f32(qq.ravel(), k, v, 8, 2, 64, seq, 0.125).reshape(8, 64)
    assert np.array_equal(out[0], out[1])
    ref4 = orc.attn_decode_f32(qq[4], k[:, 1:2].copy(), v[:, 1:2].copy(), 1, 1, 64, seq, 0.125)
    assert np.array_equal(out[4], ref4)


def test_int8_kv_equals_fp16_on_representable_values():
    seq, n_kv, hd = 64, 2, 64
    r = util.rng(820)
    ki = r.integers(-127, 128, (seq, n_kv, hd)).astype(np.int8)
    vi = r.integers(-127, 128, (seq, n_kv, hd)).astype(np.int8)
    ks = np.exp2(r.integers(-8, -3, (seq, n_kv))).astype(np.float32)
    vs = np.exp2(r.integers(-8, -3, (seq, n_kv))).astype(np.float32)
    k16 = f16(ki.astype(np.float32) * ks[:, :, None])
    v16 = f16(vi.astype(np.float32) * vs[:, :, None])
    q = f16(r.standard_normal(8 * hd))
    a = orc.attn_decode_f32(q, ki, vi, 8, n_kv, hd, seq, 0.125, True, ks, vs)
    b = orc.attn_decode_f32(q, k16, v16, 8, n_kv, hd, seq, 0.125)
    assert np.array_equal(a, b)
    # NULL scales mean 1
    c = orc.attn_decode_f32(q, ki, vi, 8, n_kv, hd, seq, 0.125, True, None, None)
    d = orc.attn_decode_f32(q, f16(ki.astype(np.float32)), f16(vi.astype(np.float32)), 8, n_kv,
                            hd, seq, 0.125)
    assert np.array_equal(c, d)


def test_prefill_is_causal_decode():
    n_tok, start = 6, 10
    seq = start + n_tok
    r = util.rng(830)
    q = f16(r.standard_normal((n_tok, 8 * 64)))
    _, k, v = case(831, seq)
    out = orc.attn_prefill_f32(q, k, v, 8, 2, 64, n_tok, start, 0.125).reshape(n_tok, -1)
    for t in range(n_tok):
        assert np.array_equal(out[t], orc.attn_decode_f32(q[t], k, v, 8, 2, 64, start + t + 1, 0.125))
    k2, v2 = k.copy(), v.copy()
    k2[start + 3:] = f16(r.standard_normal(k2[start + 3:].shape))
    v2[start + 3:] = f16(r.standard_normal(v2[start + 3:].shape))
    out2 = orc.attn_prefill_f32(q, k2, v2, 8, 2, 64, n_tok, start, 0.125).reshape(n_tok, -1)
    assert np.array_equal(out2[:3], out[:3]) and not np.array_equal(out2[3:], out[3:])


def test_empty_sequence_gives_zeros():
    q, k, v = case(840, 1)
    assert not orc.attn_decode_f32(q, k, v, 8, 2, 64, 0, 0.125).any()
