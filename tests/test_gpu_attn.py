"""GPU parity of decode / prefill attention against the CPU oracle.

Bar: the fp16 output is within rel_err <= 1e-3 of the fp64 attention over
the same fp16 (or int8 x scale) operands, and correctly rounded up to
accumulation order (tests/util.py rounded_ok).  The reference CPU path
(oracle attn_*_f32) is held to the same bar.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import rxq4
from oracle import oracle as orc
from rxq4 import api, capi
from tests import util

pytestmark = pytest.mark.gpu


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def dev16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(torch.float16)


def host16(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def check(got_bits, ref64, ref32):
    got = got_bits.view(np.float16).astype(np.float64)
    assert util.rel_err(got, ref64) <= util.TOL
    assert util.rel_err(ref32, ref64) <= util.TOL
    assert util.rounded_ok(got_bits, ref64).all()


# (n_heads, n_kv, head_dim, seq_len): GQA 4 (Qwen3-4B-like), MHA, one KV head
# for 16 query heads (the matrix-core kernel's largest group: one workgroup
# per KV head, all 16 heads in its MFMA columns), groups of 6 and 7 (12/2 and
# 28/4 heads: zero-padded MFMA columns), a group of 32 (32/1 heads: past the
# matrix-core kernel's 16, the VALU kernel with four 8-head groups per KV
# head), head_dim 64/80/256, empty / one / tile-boundary / multi-chunk
# sequences; 7000, 8192 and 16384 positions split into 55 and 64 chunks of
# several tiles each (the combine's maximum of 64).
DECODE = [(32, 8, 128, 0), (32, 8, 128, 1), (32, 8, 128, 256), (32, 8, 128, 257),
          (32, 8, 128, 1500), (32, 8, 128, 4097), (8, 8, 64, 700), (16, 1, 128, 3000),
          (4, 2, 80, 333), (4, 1, 256, 2100), (16, 1, 128, 7000), (32, 8, 128, 8192),
          (32, 8, 128, 16384), (12, 2, 128, 1000), (28, 4, 128, 2500), (32, 1, 128, 1800),
          (32, 1, 64, 600)]


@pytest.mark.parametrize("H,KV,D,S", DECODE)
def test_decode_fp16(H, KV, D, S):
    print(f"attention decode H={H} KV={KV} D={D} S={S}", flush=True)
    r = util.rng(900 + S + D)
    q = f16(r.standard_normal(H * D))
    k = f16(r.standard_normal((max(S, 1), KV, D)))
    v = f16(r.standard_normal((max(S, 1), KV, D)))
    scale = 1.0 / np.sqrt(D)
    out = torch.empty(H * D, dtype=torch.float16, device="cuda")
    capi.attention_decode_f16(out, dev16(q), dev16(k), dev16(v), H, KV, D, S, scale)
    ref64 = orc.attn_decode_f64(q, k, v, H, KV, D, S, scale)
    ref32 = orc.attn_decode_f32(q, k, v, H, KV, D, S, scale)
    if S == 0:
        assert not host16(out).any()
        return
    check(host16(out), ref64, ref32)


# (n_heads, n_kv, head_dim): the matrix-core decode kernel at head_dim 128
# (GQA 4, 6 and 7) and 64 (GQA 8), and the VALU kernel at head_dim 80 (GQA 2)
# and at head_dim 128 with a group of 32
@pytest.mark.parametrize("H,KV,D", [(32, 8, 128), (16, 2, 64), (8, 4, 80), (12, 2, 128),
                                    (28, 4, 128), (32, 1, 128)])
@pytest.mark.parametrize("scales", [True, False])
@pytest.mark.parametrize("S", [2000, 9000])
def test_decode_int8(H, KV, D, scales, S):
    print(f"attention decode int8 H={H} KV={KV} D={D} S={S} scales={scales}", flush=True)
    r = util.rng(910 + D)
    q = f16(r.standard_normal(H * D))
    ki = r.integers(-127, 128, (S, KV, D)).astype(np.int8)
    vi = r.integers(-127, 128, (S, KV, D)).astype(np.int8)
    ks = (r.random((S, KV)) * 0.02 + 0.001).astype(np.float32) if scales else None
    vs = (r.random((S, KV)) * 0.02 + 0.001).astype(np.float32) if scales else None
    scale = 1.0 / np.sqrt(D) if scales else 0.002
    out = torch.empty(H * D, dtype=torch.float16, device="cuda")
    t = lambda a: None if a is None else torch.from_numpy(a).cuda()  # noqa: E731
    capi.attention_decode_f16(out, dev16(q), t(ki), t(vi), H, KV, D, S, scale, True, t(ks), t(vs))
    ref64 = orc.attn_decode_f64(q, ki, vi, H, KV, D, S, scale, True, ks, vs)
    ref32 = orc.attn_decode_f32(q, ki, vi, H, KV, D, S, scale, True, ks, vs)
    check(host16(out), ref64, ref32)


@pytest.mark.parametrize("N,start", [(7, 100), (300, 0), (5, 1200)])
def test_prefill_api(N, start):
    H, KV, D = 16, 4, 128
    S = start + N
    r = util.rng(920 + N)
    q = f16(r.standard_normal((N, H * D)))
    k = f16(r.standard_normal((S, KV, D)))
    v = f16(r.standard_normal((S, KV, D)))
    scale = 1.0 / np.sqrt(D)
    out = torch.empty((N, H * D), dtype=torch.float16, device="cuda")
    qd, kd, vd = dev16(q), dev16(k), dev16(v)
    a = api.AttentionPrefillBatchedArgs(output=out.data_ptr(), q=qd.data_ptr(), k_cache=kd.data_ptr(),
                                        v_cache=vd.data_ptr(), n_heads=H, n_kv_heads=KV, head_dim=D,
                                        N=N, start_pos=start, scale=scale)
    assert api.call("flash_attention_prefill_batched", a) == rxq4.SUCCESS
    got = host16(out).reshape(N, -1)
    ref32 = orc.attn_prefill_f32(q, k, v, H, KV, D, N, start, scale).reshape(N, -1)
    for t in range(N):
        ref64 = orc.attn_decode_f64(q[t], k, v, H, KV, D, start + t + 1, scale)
        check(got[t], ref64, ref32[t])


def test_decode_api_matches_c_abi():
    H, KV, D, S = 32, 8, 128, 900
    r = util.rng(930)
    q = f16(r.standard_normal(H * D))
    k = f16(r.standard_normal((S, KV, D)))
    v = f16(r.standard_normal((S, KV, D)))
    qd, kd, vd = dev16(q), dev16(k), dev16(v)
    o1 = torch.empty(H * D, dtype=torch.float16, device="cuda")
    o2 = torch.empty_like(o1)
    capi.attention_decode_f16(o1, qd, kd, vd, H, KV, D, S, 0.088)
    a = api.AttentionDecodeArgs(output=o2.data_ptr(), q=qd.data_ptr(), k_cache=kd.data_ptr(),
                                v_cache=vd.data_ptr(), n_heads=H, n_kv_heads=KV, head_dim=D,
                                seq_len=S, scale=0.088)
    assert api.call("flash_attention_decode", a) == rxq4.SUCCESS
    assert torch.equal(o1, o2)


# (n_heads, n_kv, head_dim, N, start_pos, int8): GQA groups 1, 2 (6 heads per
# KV head: two head blocks), 4, 8 and 32 (two blocks of 16), head_dim 64 and
# 128 (matrix-core prefill) and 80 (VALU kernel), N not a multiple of the
# token block, int8 with and without scales.  A workgroup pairs an early
# token half block with the mirror late one: odd half-block counts (100,
# 520, 530 tokens at 8 tokens a half block) leave the middle one paired with
# itself.  The last two have more workgroups (8 KV heads x 33-34 pairs of
# 8-token half blocks) than the 256 CUs and take the one-group kernel; the
# others the two-group kernel (both stage V row-major and read it back with
# transposing LDS reads).
PREFILL = [(32, 8, 128, 100, 0, False), (16, 4, 128, 300, 37, False), (8, 8, 64, 70, 5, False),
           (16, 2, 64, 33, 200, False), (32, 1, 128, 20, 10, False), (12, 2, 128, 17, 3, False),
           (16, 4, 128, 50, 64, "scales"), (8, 2, 64, 40, 0, "plain"), (4, 2, 80, 9, 4, False),
           (32, 8, 128, 520, 0, False), (32, 8, 128, 530, 3, "scales")]


@pytest.mark.parametrize("H,KV,D,N,start,i8", PREFILL)
def test_prefill_shapes(H, KV, D, N, start, i8):
    print(f"attention prefill H={H} KV={KV} D={D} N={N} start={start} int8={i8}", flush=True)
    S = start + N
    r = util.rng(940 + N + D)
    q = f16(r.standard_normal((N, H * D)))
    if i8:
        k = r.integers(-127, 128, (S, KV, D)).astype(np.int8)
        v = r.integers(-127, 128, (S, KV, D)).astype(np.int8)
        ks = (r.random((S, KV)) * 0.02 + 0.001).astype(np.float32) if i8 == "scales" else None
        vs = (r.random((S, KV)) * 0.02 + 0.001).astype(np.float32) if i8 == "scales" else None
        scale = 1.0 / np.sqrt(D) if i8 == "scales" else 0.002
        kd, vd = torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda()
    else:
        k = f16(r.standard_normal((S, KV, D)))
        v = f16(r.standard_normal((S, KV, D)))
        ks = vs = None
        scale = 1.0 / np.sqrt(D)
        kd, vd = dev16(k), dev16(v)
    t = lambda a: None if a is None else torch.from_numpy(a).cuda()  # noqa: E731
    out = torch.empty((N, H * D), dtype=torch.float16, device="cuda")
    capi.attention_prefill_f16(out, dev16(q), kd, vd, H, KV, D, N, start, scale, bool(i8), t(ks), t(vs))
    got = host16(out).reshape(N, -1)
    ref32 = orc.attn_prefill_f32(q, k, v, H, KV, D, N, start, scale, bool(i8), ks, vs).reshape(N, -1)
    for tk in range(N):
        ref64 = orc.attn_decode_f64(q[tk], k, v, H, KV, D, start + tk + 1, scale, bool(i8), ks, vs)
        check(got[tk], ref64, ref32[tk])
