"""GPU parity of the HIP kernels against the CPU oracle and the golden fixtures.

Bars (tests/util.py): dequantised weights and embedding rows bit-exact;
GEMV/GEMM outputs within rel_err <= 1e-3 of the fp32/fp64 oracle over the
same rounded operands, 16-bit outputs correctly rounded up to accumulation
order (tests/util.py rounded_ok).  Calls go
through the C ABI (rxq4.capi) and the reflex::infer C++ API (rxq4.api).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

import rxq4
from oracle import oracle as orc
from rxq4 import api, capi
from tests import kquant_blocks as kb
from tests import util

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "q4k_golden.npz")


def dev(a: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda()
    return torch.from_numpy(a).cuda()


def host16(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy().view(np.uint16)


def f16(bits: np.ndarray) -> np.ndarray:
    return bits.view(np.float16).astype(np.float32)


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


# ------------------------------------------------------------ dequantisation
def test_embedding_row_golden_bit_exact(golden):
    table = dev(golden["emb_W"])
    ids, expect = golden["emb_ids"], golden["emb_rows_f16"]
    out = torch.empty(2048, dtype=torch.float16, device="cuda")
    for i, t in enumerate(ids):
        if not 0 <= t < 64:
            continue
        out.zero_()
        a = api.DequantEmbeddingRowArgs(dst=out.data_ptr(), weights=table.data_ptr(),
                                        ggml_type=12, token_id=int(t), hidden_dim=2048)
        assert api.call("dequant_embedding_row", a) == rxq4.SUCCESS
        assert np.array_equal(host16(out), expect[i]), t
        out.zero_()
        capi.embed_row_f16(out, table, int(t), 2048)
        assert np.array_equal(host16(out), expect[i]), t


def test_embedding_rows_batched_golden_and_oob(golden):
    table = dev(golden["emb_W"])
    ids = dev(golden["emb_ids"])
    out = torch.full((ids.numel(), 2048), 7.0, dtype=torch.float16, device="cuda")
    capi.embed_rows_f16(out, table, 64, ids, 2048)
    assert np.array_equal(host16(out), golden["emb_rows_f16"])


@pytest.mark.parametrize("K", [256, 1024, 2048, 6144, 11008])
def test_embedding_rows_zipf(K):
    vocab = 3000
    Wn = util.weights(40 + K, vocab, K)
    ids = util.zipf_ids(41, 4096, vocab)
    W, idt = dev(Wn), dev(ids)
    out = torch.empty((ids.size, K), dtype=torch.float16, device="cuda")
    capi.embed_rows_f16(out, W, vocab, idt, K)
    assert np.array_equal(host16(out), orc.embed_rows_f16(Wn, K, ids))


def test_embedding_rows_full_table_zipf():
    """BASELINE configs[4] at full size: the [151936 x 2048] Q4_K table of
    ggml-quantised N(0, 0.02) weights, 4096 Zipf(1.1) ids over the whole
    vocabulary (repeats allowed, the last row included), bit-exact against
    the oracle's dequantisation of the addressed rows."""
    vocab, K = 151936, 2048
    g = torch.Generator(device="cuda").manual_seed(46)
    src = torch.randn((vocab, K), generator=g, device="cuda") * 0.02
    table = capi.quantize_ggml(src, 12)
    del src
    ids = util.zipf_ids(47, 4096, vocab)
    ids[-1] = vocab - 1
    out = torch.empty((ids.size, K), dtype=torch.float16, device="cuda")
    capi.embed_rows_f16(out, table, vocab, dev(ids), K)
    got = host16(out)
    ref = orc.embed_rows_f16(table.cpu().numpy(), K, ids)
    assert np.array_equal(got, ref)
    assert np.unique(ids).size > 1000  # the Zipf draw spreads over the table


def test_embedding_special_values():
    """Subnormal, negative and zero scales dequantise bit-exactly too."""
    from tests.test_oracle import random_blocks
    K = 2048
    Wn = random_blocks(42, 50, K)
    out = torch.empty((50, K), dtype=torch.float16, device="cuda")
    ids = np.arange(50, dtype=np.int32)
    capi.embed_rows_f16(out, dev(Wn), 50, dev(ids), K)
    got, ref = host16(out), orc.embed_rows_f16(Wn, K, ids)
    with np.errstate(invalid="ignore"):
        same = (got == ref) | (np.isnan(got.view(np.float16)) & np.isnan(ref.view(np.float16)))
    assert same.all()


@pytest.mark.parametrize("rows,K", [(64, 2048), (3, 11008), (1, 256), (500, 512)])
def test_gpu_quantizer_matches_oracle(rows, K):
    src = util.gaussian(43 + rows, (rows, K), 0.02)
    src[0, :7] = [0, -0.0, 1e-8, -1e-8, 0.5, -0.7, 3e-3]
    got = capi.quantize(dev(src)).cpu().numpy()
    assert np.array_equal(got, orc.quantize(src))


# ---------------------------------------------------------------------- GEMV
# register kernel (slots | 64), LDS kernel (other K: 2816, 1536, 5632, 11008,
# 16384, 65536)
SHAPES = [(2048, 2048), (7, 256), (33, 512), (2560, 2048), (301, 4096), (64, 11008),
          (50, 2816), (3, 65536), (129, 1024), (70, 1536), (45, 5632), (20, 16384),
          (2051, 11008)]


@pytest.mark.parametrize("M,K", SHAPES)
def test_gemv_f32_and_f16(M, K):
    Wn = util.weights(50 + M + K, M, K)
    x16 = util.x_f16(51 + K, K)
    ref = orc.gemv_f32(Wn, K, x16)
    W, x = dev(Wn), dev(x16)
    y32 = torch.empty(M, dtype=torch.float32, device="cuda")
    capi.gemv_f32(y32, W, x, M, K)
    assert util.rel_err(y32.cpu().numpy(), ref) <= util.TOL
    y16 = torch.empty(M, dtype=torch.float16, device="cuda")
    capi.gemv_f16(y16, W, x, M, K)
    assert util.rel_err(f16(host16(y16)), ref) <= util.TOL
    assert util.rounded_ok(host16(y16), ref).all()


def test_gemv_golden(golden):
    for case in ("c0", "c1", "c2"):
        rows, K = (int(v) for v in golden[f"{case}_shape"])
        W, x = dev(golden[f"{case}_W"]), dev(golden[f"{case}_x16"])
        ref = golden[f"{case}_y_f32"].view(np.float32)
        y32 = torch.empty(rows, dtype=torch.float32, device="cuda")
        capi.gemv_f32(y32, W, x, rows, K)
        assert util.rel_err(y32.cpu().numpy(), ref) <= util.TOL
        y16 = torch.empty(rows, dtype=torch.float16, device="cuda")
        capi.gemv_f16(y16, W, x, rows, K)
        assert util.rounded_ok(host16(y16), ref).all()
        assert util.rel_err(f16(host16(y16)), f16(golden[f"{case}_y_f16"])) <= util.TOL


@pytest.mark.parametrize("M,K", [(2048, 2048), (2048, 11008), (37, 512)])
def test_gemv_add_and_in_place(M, K):
    Wn = util.weights(60 + K, M, K)
    x16, res16 = util.x_f16(61, K), util.x_f16(62, M)
    ref16 = orc.gemv_add_f16(Wn, K, x16, res16)
    y32 = orc.gemv_f32(Wn, K, x16)
    W, x, res = dev(Wn), dev(x16), dev(res16)
    y = torch.empty(M, dtype=torch.float16, device="cuda")
    capi.gemv_add_f16(y, W, x, res, M, K)
    # double rounding: the projection is rounded to fp16 before the add
    # (q4_gemm.cu:774-777), which may move it by half an ulp of the projection
    proj_sp = util.spacing(orc.f32_to_fp16(y32), "f16")
    exact = y32.astype(np.float64) + f16(res16)
    assert util.rounded_ok(host16(y), exact, delta=util.ACC_DELTA, extra=proj_sp / 2).all()
    assert util.rel_err(f16(host16(y)), f16(ref16)) <= util.TOL
    # y aliases residual (reference q4_gemm.cu:774-777 reads then writes per row)
    a = api.GemvQuantAddArgs(y=res.data_ptr(), weights=W.data_ptr(), ggml_type=12,
                             x=x.data_ptr(), residual=res.data_ptr(), M=M, K=K)
    assert api.call("gemv_quant_add", a) == rxq4.SUCCESS
    assert np.array_equal(host16(res), host16(y))


def test_api_pair_and_triple_match_single_gemvs():
    K = 2048
    x16 = util.x_f16(70, K)
    x = dev(x16)
    # gate+up pair (11008 + 11008) and an odd split that straddles a wave step
    for M0, M1 in [(11008, 11008), (3, 5)]:
        W0n, W1n = util.weights(71, M0, K), util.weights(72, M1, K)
        W0, W1 = dev(W0n), dev(W1n)
        y0 = torch.empty(M0, dtype=torch.float16, device="cuda")
        y1 = torch.empty(M1, dtype=torch.float16, device="cuda")
        a = api.GemvQuantPairArgs(y0=y0.data_ptr(), weights0=W0.data_ptr(), ggml_type0=12, M0=M0,
                                  y1=y1.data_ptr(), weights1=W1.data_ptr(), ggml_type1=12, M1=M1,
                                  x=x.data_ptr(), K=K)
        assert api.call("gemv_quant_pair", a) == rxq4.SUCCESS
        for yv, Wn in ((y0, W0n), (y1, W1n)):
            ref = orc.gemv_f32(Wn, K, x16)
            assert util.rounded_ok(host16(yv), ref).all()
    # fused QKV triple: 2048 / 256 / 256
    Ms = (2048, 256, 256)
    Wn = [util.weights(73 + i, m, K) for i, m in enumerate(Ms)]
    Wd = [dev(w) for w in Wn]
    ys = [torch.empty(m, dtype=torch.float16, device="cuda") for m in Ms]
    a = api.GemvQuantTripleArgs(
        y0=ys[0].data_ptr(), weights0=Wd[0].data_ptr(), ggml_type0=12, M0=Ms[0],
        y1=ys[1].data_ptr(), weights1=Wd[1].data_ptr(), ggml_type1=12, M1=Ms[1],
        y2=ys[2].data_ptr(), weights2=Wd[2].data_ptr(), ggml_type2=12, M2=Ms[2],
        x=x.data_ptr(), K=K)
    assert api.call("gemv_quant_triple", a) == rxq4.SUCCESS
    for yv, w in zip(ys, Wn):
        ref = orc.gemv_f32(w, K, x16)
        assert util.rounded_ok(host16(yv), ref).all()


def test_pair_on_long_rows():
    """A pair whose rows take the LDS kernel (long rows)."""
    K = 11008
    x16 = util.x_f16(75, K)
    x = dev(x16)
    Ws = [util.weights(76, 13, K), util.weights(77, 30, K)]
    ys = [torch.empty(w.shape[0], dtype=torch.float16, device="cuda") for w in Ws]
    Wd = [dev(w) for w in Ws]
    capi.gemv_multi_f16([(ys[0], Wd[0], 13), (ys[1], Wd[1], 30)], x, K)
    for yv, Wn in zip(ys, Ws):
        assert util.rounded_ok(host16(yv), orc.gemv_f32(Wn, K, x16)).all()


@pytest.mark.host_path
def test_api_gemv_pointer_resolution():
    """weights_device alias wins over a host `weights` pointer; a device
    `weights` pointer resolves by itself; host memory alone takes the
    reference's host path (q4_gemm.cu:1886-1899), bit for bit its CPU loop."""
    M, K = 256, 2048
    Wn = util.weights(80, M, K)
    x16 = util.x_f16(81, K)
    ref = orc.gemv_f32(Wn, K, x16)
    W, x = dev(Wn), dev(x16)
    y = torch.empty(M, dtype=torch.float16, device="cuda")
    host_ptr = Wn.ctypes.data
    a = api.GemvQuantArgs(y=y.data_ptr(), weights=host_ptr, weights_device=W.data_ptr(),
                          ggml_type=12, x=x.data_ptr(), M=M, K=K)
    assert api.call("gemv_quant", a) == rxq4.SUCCESS
    assert util.rounded_ok(host16(y), ref).all()
    y.zero_()
    a = api.GemvQuantArgs(y=y.data_ptr(), weights=W.data_ptr(), ggml_type=12, x=x.data_ptr(),
                          M=M, K=K)
    assert api.call("gemv_quant", a) == rxq4.SUCCESS
    assert util.rounded_ok(host16(y), ref).all()
    n0 = capi.host_gemv_calls()
    a = api.GemvQuantArgs(y=y.data_ptr(), weights=host_ptr, ggml_type=12, x=x.data_ptr(),
                          M=M, K=K)
    assert api.call("gemv_quant", a) == rxq4.SUCCESS
    assert np.array_equal(host16(y), orc.gemv_f16(Wn, K, x16))
    assert capi.host_gemv_calls() == n0 + 1
    a = api.GemvQuantArgs(y=y.data_ptr(), weights=W.data_ptr(), ggml_type=15, x=x.data_ptr(),
                          M=M, K=K)
    assert api.call("gemv_quant", a) == rxq4.UNSUPPORTED_QUANT_FORMAT
    f = api.GemvQuantF32Args(y=torch.empty(M, device="cuda").data_ptr(), weights=W.data_ptr(),
                             ggml_type=12, x=x.data_ptr(), M=M, K=K)
    assert api.call("gemv_quant_f32", f) == rxq4.SUCCESS


def test_lm_head_full_size_properties():
    """[151936 x 2048] fp32 logits: sampled rows vs the oracle; y(2x) == 2 y(x)
    bit for bit (power-of-two scaling is exact); rows are independent (a row
    permutation of W permutes y bit for bit)."""
    M, K = 151936, 2048
    g = torch.Generator(device="cuda").manual_seed(90)
    src = torch.randn((M, K), generator=g, device="cuda") * 0.02
    W = capi.quantize(src)
    del src
    x16 = util.x_f16(91, K)
    x = dev(x16)
    y = torch.empty(M, dtype=torch.float32, device="cuda")
    capi.gemv_f32(y, W, x, M, K)
    rows = np.sort(util.rng(92).choice(M, 1024, replace=False))
    Wn = W[torch.from_numpy(rows).cuda()].cpu().numpy()
    ref = orc.gemv_f32(Wn, K, x16)
    assert util.rel_err(y.cpu().numpy()[rows], ref) <= util.TOL
    x2 = (x.view(torch.float16) * 2).view(torch.int16)
    y2 = torch.empty_like(y)
    capi.gemv_f32(y2, W, x2, M, K)
    assert torch.equal(y2, y * 2)
    perm = torch.randperm(M, generator=torch.Generator().manual_seed(93)).cuda()
    Wp = W[perm].contiguous()
    yp = torch.empty_like(y)
    capi.gemv_f32(yp, Wp, x, M, K)
    assert torch.equal(yp, y[perm])


# ---------------------------------------------------------------------- GEMM
# (8200, N <= 16): the small-batch kernel's two-row-tile shape, with a
# partial last tile (8200 = 256 * 32 + 8).
# (1000, 200) and (264, 130): 16-bit outputs staged through LDS with a
# partial last row tile and token tile.
# (2048, 8 / 16, 11008) and (600, 6, 4096): small batches of long rows, K split
# over workgroups with fp32 partials.  (16400, 7, 512) and (16384, 16, 256):
# small batches on 64-row workgroups with x staged in LDS (at least one per
# CU), the first with a partial last tile.  (520, 129, 256): one super-block
# per row and a last token tile of one token.  (300, 20, 65536): the largest
# K, 128 K-splits.
GEMM_CASES = [(300, 2, 2048), (2048, 5, 2048), (1000, 16, 2048), (2048, 17, 2048),
              (300, 100, 11008), (2048, 512, 2048), (129, 33, 512), (8200, 3, 512),
              (8200, 16, 256), (1000, 200, 2048), (264, 130, 512), (2048, 8, 11008),
              (2048, 16, 11008), (600, 6, 4096), (16400, 7, 512), (16384, 16, 256),
              (520, 129, 256), (300, 20, 65536)]


@pytest.mark.parametrize("M,N,K", GEMM_CASES)
def test_gemm_bf16(M, N, K):
    Wn = util.weights(100 + M + N, M, K)
    xb = util.f32_to_bf16_bits(util.gaussian(101 + N, (N, K)))
    xv = orc.bits_bf16_to_f32(xb)
    ref = orc.gemm_f64(Wn, K, xv, "bf16")
    W = dev(Wn)
    x = torch.from_numpy(xb.view(np.int16)).cuda().view(torch.bfloat16)
    y32 = torch.empty((N, M), dtype=torch.float32, device="cuda")
    capi.gemm(y32, W, x, M, N, K)
    assert util.rel_err(y32.cpu().numpy(), ref) <= util.TOL
    yb = torch.empty((N, M), dtype=torch.bfloat16, device="cuda")
    capi.gemm(yb, W, x, M, N, K)
    got = yb.view(torch.int16).cpu().numpy().view(np.uint16)
    assert util.rounded_ok(got, ref, "bf16").all()


@pytest.mark.parametrize("M,N,K", [(300, 3, 2048), (2048, 16, 2048), (1000, 40, 2048),
                                   (256, 512, 2048), (200, 20, 11008), (16400, 9, 256)])
def test_api_gemm_quant_batched_f16(M, N, K):
    Wn = util.weights(110 + N, M, K)
    x16 = util.x_f16(111 + N, (N, K))
    ref32 = orc.gemm_tokens_f32(Wn, K, x16)   # reference CPU semantics (per-token GEMV)
    # the same operands as the kernel: the decode GEMV on the exact weights
    # (util.gemv_path), else the MFMA tiles on fp16-rounded weights
    ref64 = (orc.kq_gemm_f64(Wn, K, 12, f16(x16), None) if util.gemv_path(N, M, K)
             else orc.gemm_f64(Wn, K, f16(x16), "f16"))
    W, x = dev(Wn), dev(x16)
    y = torch.empty((N, M), dtype=torch.float16, device="cuda")
    a = api.GemmQuantBatchedArgs(y=y.data_ptr(), weights=W.data_ptr(), ggml_type=12,
                                 x=x.data_ptr(), M=M, N=N, K=K)
    assert api.call("gemm_quant_batched", a) == rxq4.SUCCESS
    got = f16(host16(y))
    assert util.rel_err(got, ref32) <= util.TOL
    assert util.rounded_ok(host16(y), ref64).all()


# 2..4 fp16 tokens on the multi-token decode GEMV (every token's activations
# in registers: register kernel for K 256..4096, LDS kernel for 1536 / 11008).
# The launcher picks it for 2 tokens (3 on wide matrices); the cases it sends
# to the MFMA kernel run in a child process with RXQ4_MULTI_TOKEN_GEMV=1.
MT_CASES = [(300, 2, 2048), (2048, 4, 2048), (129, 3, 11008), (70, 4, 1536), (33, 2, 256),
            (17, 4, 4096), (5000, 2, 512)]


@pytest.mark.parametrize("M,N,K", MT_CASES)
def test_multi_token_gemv_equals_per_token_gemv(M, N, K):
    if not util.gemv_path(N, M, K):
        env = dict(os.environ, RXQ4_MULTI_TOKEN_GEMV="1")
        code = ("import sys; sys.path[:0] = [%r, %r]\n"
                "from tests import test_gpu_parity as t\n"
                "t.check_multi_token_gemv(%d, %d, %d)\nprint('multi-token ok')\n"
                % (ROOT, os.path.join(ROOT, "reflex-infer_amd"), M, N, K))
        r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True,
                           text=True, timeout=300)
        assert r.returncode == 0, r.stderr[-2000:]
        assert "multi-token ok" in r.stdout
        return
    check_multi_token_gemv(M, N, K)


def check_multi_token_gemv(M, N, K):
    print(f"multi-token GEMV M={M} N={N} K={K}", flush=True)
    Wn = util.weights(140 + N + K, M, K)
    x16 = util.x_f16(141 + N, (N, K))
    ref32 = orc.gemm_tokens_f32(Wn, K, x16)
    W, x = dev(Wn), dev(x16)
    y16 = torch.empty((N, M), dtype=torch.float16, device="cuda")
    capi.gemm_f16(y16, W, x, M, N, K)
    y32 = torch.empty((N, M), dtype=torch.float32, device="cuda")
    capi.gemm(y32, W, x.view(torch.float16), M, N, K)
    assert util.rel_err(y32.cpu().numpy(), ref32) <= util.TOL
    assert util.rounded_ok(host16(y16), ref32).all()
    # the same arithmetic, in the same order, as one GEMV per token
    for t in range(N):
        g16 = torch.empty(M, dtype=torch.float16, device="cuda")
        g32 = torch.empty(M, dtype=torch.float32, device="cuda")
        capi.gemv_f16(g16, W, x[t], M, K)
        capi.gemv_f32(g32, W, x[t], M, K)
        assert torch.equal(y16[t], g16) and torch.equal(y32[t], g32)


@pytest.mark.parametrize("t", [12, 14])
@pytest.mark.parametrize("K", [512, 2048])  # one K split / four (the reduction kernel stores)
def test_gemm_output_at_any_element_alignment(t, K):
    """y one element past a 16-byte boundary: the kernels fall back to
    element stores and write the same values as into an aligned y."""
    M, N = 512, 40
    Wn = (util.weights(160, M, K) if t == 12 else kb.random_blocks(t, util.rng(161), M, K))
    W = dev(Wn)
    xb = util.f32_to_bf16_bits(util.gaussian(162, (N, K)))
    x = torch.from_numpy(xb.view(np.int16)).cuda().view(torch.bfloat16)
    for dtype in (torch.bfloat16, torch.float32):
        ya = torch.empty((N, M), dtype=dtype, device="cuda")
        capi.gemm(ya, W, x, M, N, K, ggml_type=t)
        buf = torch.full((N * M + 8,), -7.0, dtype=dtype, device="cuda")
        yo = buf[1:1 + N * M].view(N, M)
        assert yo.data_ptr() % 16 != 0
        capi.gemm(yo, W, x, M, N, K, ggml_type=t)
        assert torch.equal(yo, ya)
        assert buf[0].item() == -7.0 and bool((buf[1 + N * M:] == -7.0).all())


def test_gemm_n1_is_the_gemv():
    M, K = 512, 2048
    Wn = util.weights(120, M, K)
    x16 = util.x_f16(121, (1, K))
    W, x = dev(Wn), dev(x16)
    y = torch.empty((1, M), dtype=torch.float16, device="cuda")
    capi.gemm_f16(y, W, x, M, 1, K)
    y2 = torch.empty(M, dtype=torch.float16, device="cuda")
    capi.gemv_f16(y2, W, x, M, K)
    assert torch.equal(y[0], y2)


def test_gemm_full_size_sampled_rows():
    """m = 512 tokens on [11008 x 2048]: 256 sampled rows vs the fp64 oracle."""
    M, N, K = 11008, 512, 2048
    g = torch.Generator(device="cuda").manual_seed(130)
    W = capi.quantize(torch.randn((M, K), generator=g, device="cuda") * 0.02)
    x = torch.randn((N, K), generator=g, device="cuda").to(torch.bfloat16)
    y = torch.empty((N, M), dtype=torch.float32, device="cuda")
    capi.gemm(y, W, x, M, N, K)
    rows = np.sort(util.rng(131).choice(M, 256, replace=False))
    Wn = W[torch.from_numpy(rows).cuda()].cpu().numpy()
    xv = x.float().cpu().numpy()
    ref = orc.gemm_f64(Wn, K, xv, "bf16")
    assert util.rel_err(y.cpu().numpy()[:, rows], ref) <= util.TOL


def test_split_k_paths_replay_in_a_graph():
    """The split-K GEMM (workspace + reduction launch) and the split
    small-batch kernel captured in a HIP graph: every replay, with eager
    work and synchronisation in between, equals the eager result."""
    cases = [(2048, 512, 11008, torch.bfloat16), (2048, 16, 11008, torch.float16)]
    for M, N, K, dt in cases:
        print(f"graph replay M={M} N={N} K={K}", flush=True)
        g = torch.Generator(device="cuda").manual_seed(180 + N)
        W = capi.quantize(torch.randn((M, K), generator=g, device="cuda") * 0.02)
        x = torch.randn((N, K), generator=g, device="cuda").to(dt)
        y_eager = torch.empty((N, M), dtype=dt, device="cuda")
        capi.gemm(y_eager, W, x, M, N, K)  # also sizes the workspace before capture
        torch.cuda.synchronize()
        y = torch.empty_like(y_eager)
        s = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            capi.gemm(y, W, x, M, N, K, stream=s)
        for rep in range(3):
            y.fill_(0)
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, y_eager), f"replay {rep}"
            # eager work on the same workspace between replays
            capi.gemm(y_eager, W, x, M, N, K)
            torch.cuda.synchronize()
