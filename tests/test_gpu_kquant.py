"""GPU parity of the Q5_K (13) and Q6_K (14) kernels against the CPU oracle.

Same bars as the Q4_K path (tests/util.py): embedding rows bit-exact;
GEMV/GEMM within rel_err <= 1e-3 of the oracle over identically rounded
operands, 16-bit outputs correctly rounded up to accumulation order.
Weights are random blocks packed by index (tests/kquant_blocks.py): every
quant value, scale and high-bit pattern occurs.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import rxq4
from oracle import oracle as orc
from rxq4 import api, capi
from tests import kquant_blocks as kb
from tests import util

pytestmark = pytest.mark.gpu


def dev(a: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda()
    return torch.from_numpy(a).cuda()


def host16(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy().view(np.uint16)


def f16(bits: np.ndarray) -> np.ndarray:
    return bits.view(np.float16).astype(np.float32)


# (rows, K): packed rows per wave step (K 2048 -> 2 rows, 256 -> 16 rows,
# 4096 -> 1 row), long rows (11008: 172 slots, 1536: 24 slots), a partial last
# step (37 rows), and a K whose x staging needs more than 64 KiB of LDS.
# 70001 x 2048 gives each of the 3072 waves (three four-wave workgroups per
# CU) 11-12 packed steps (the pipelined steady state, an odd last step and a
# reload past the end).
GEMV_SHAPES = [(256, 2048), (300, 256), (37, 4096), (100, 11008), (64, 1536), (3, 32768),
               (70001, 2048)]


@pytest.mark.parametrize("t", [13, 14])
@pytest.mark.parametrize("M,K", GEMV_SHAPES)
def test_kq_gemv_f32_f16(t, M, K):
    print(f"kq gemv type {t} M={M} K={K}", flush=True)
    Wn = kb.random_blocks(t, util.rng(700 + t + M), M, K)
    x16 = util.x_f16(701 + K, K)
    ref = orc.kq_gemv_f32(Wn, K, t, x16)
    W, x = dev(Wn), dev(x16)
    y32 = torch.empty(M, dtype=torch.float32, device="cuda")
    capi.gemv_f32(y32, W, x, M, K, ggml_type=t)
    assert util.rel_err(y32.cpu().numpy(), ref) <= util.TOL
    y16 = torch.empty(M, dtype=torch.float16, device="cuda")
    capi.gemv_f16(y16, W, x, M, K, ggml_type=t)
    assert util.rel_err(f16(host16(y16)), ref) <= util.TOL
    assert util.rounded_ok(host16(y16), ref).all()


@pytest.mark.parametrize("t", [13, 14])
@pytest.mark.parametrize("M,K", [(512, 2048), (70001, 2048), (300, 11008)])
def test_kq_gemv_add_in_place(t, M, K):
    print(f"kq gemv add in place type {t} M={M} K={K}", flush=True)
    Wn = kb.random_blocks(t, util.rng(710 + t), M, K)
    x16, res16 = util.x_f16(711, K), util.x_f16(712, M)
    y32 = orc.kq_gemv_f32(Wn, K, t, x16)
    W, x, res = dev(Wn), dev(x16), dev(res16)
    a = api.GemvQuantAddArgs(y=res.data_ptr(), weights=W.data_ptr(), ggml_type=t,
                             x=x.data_ptr(), residual=res.data_ptr(), M=M, K=K)
    assert api.call("gemv_quant_add", a) == rxq4.SUCCESS
    proj_sp = util.spacing(orc.f32_to_fp16(y32), "f16")
    exact = y32.astype(np.float64) + f16(res16)
    assert util.rounded_ok(host16(res), exact, extra=proj_sp / 2).all()


def test_api_mixed_q4_q4_q6_triple():
    """The Qwen3-4B fused QKV: Wq, Wk Q4_K, Wv Q6_K (reference
    q4_gemm.cu:892-939)."""
    K = 2048
    Ms = (2048, 256, 256)
    types = (12, 12, 14)
    x16 = util.x_f16(720, K)
    Wn = [util.weights(721, Ms[0], K), util.weights(722, Ms[1], K),
          kb.random_blocks(14, util.rng(723), Ms[2], K)]
    Wd = [dev(w) for w in Wn]
    ys = [torch.empty(m, dtype=torch.float16, device="cuda") for m in Ms]
    x = dev(x16)
    a = api.GemvQuantTripleArgs(
        y0=ys[0].data_ptr(), weights0=Wd[0].data_ptr(), ggml_type0=types[0], M0=Ms[0],
        y1=ys[1].data_ptr(), weights1=Wd[1].data_ptr(), ggml_type1=types[1], M1=Ms[1],
        y2=ys[2].data_ptr(), weights2=Wd[2].data_ptr(), ggml_type2=types[2], M2=Ms[2],
        x=x.data_ptr(), K=K)
    assert api.call("gemv_quant_triple", a) == rxq4.SUCCESS
    for yv, w, t in zip(ys, Wn, types):
        ref = orc.kq_gemv_f32(w, K, t, x16)
        assert util.rounded_ok(host16(yv), ref).all()
    # pair of two Q5_K matrices through the C ABI
    W5 = [kb.random_blocks(13, util.rng(724 + i), 300, K) for i in range(2)]
    y5 = [torch.empty(300, dtype=torch.float16, device="cuda") for _ in range(2)]
    W5d = [dev(w) for w in W5]
    capi.gemv_multi_f16([(y5[0], W5d[0], 300, 13), (y5[1], W5d[1], 300, 13)], x, K)
    for yv, w in zip(y5, W5):
        assert util.rounded_ok(host16(yv), orc.kq_gemv_f32(w, K, 13, x16)).all()


@pytest.mark.parametrize("K,Ms,types", [
    (256, (37, 0, 129), (14, 12, 13)),          # 16 rows per wave step, an empty range
    (11008, (5, 70, 3), (13, 14, 12)),          # long rows
    (1536, (64, 33, 100), (12, 13, 14)),        # 24 slots per row
])
def test_mixed_multi_one_launch(K, Ms, types):
    """Any mix of Q4_K / Q5_K / Q6_K ranges through gemv_multi (one launch)."""
    print(f"kq mixed multi K={K} M={Ms} types={types}", flush=True)
    x16 = util.x_f16(760 + K, K)
    Wn = [np.zeros(0, np.uint8) if m == 0 else
          util.weights(761 + i, m, K) if t == 12 else kb.random_blocks(t, util.rng(765 + i), m, K)
          for i, (m, t) in enumerate(zip(Ms, types))]
    Wd = [dev(w) if w.size else torch.empty(16, dtype=torch.uint8, device="cuda") for w in Wn]
    ys = [torch.zeros(max(m, 1), dtype=torch.float16, device="cuda") for m in Ms]
    x = dev(x16)
    capi.gemv_multi_f16([(y, w, m, t) for y, w, m, t in zip(ys, Wd, Ms, types)], x, K)
    for yv, w, m, t in zip(ys, Wn, Ms, types):
        if m == 0:
            assert not yv.any()
            continue
        ref = orc.kq_gemv_f32(w, K, t, x16)
        assert util.rounded_ok(host16(yv), ref).all()


@pytest.mark.parametrize("K", [256, 1024, 2048, 3072, 11008])
def test_q6k_embedding_bit_exact(K):
    V = 40
    Wn = kb.random_blocks(14, util.rng(730 + K), V, K)
    W = dev(Wn)
    dst = torch.empty(K, dtype=torch.float16, device="cuda")
    for tok in (0, 17, V - 1):
        a = api.DequantEmbeddingRowArgs(dst=dst.data_ptr(), weights=W.data_ptr(), ggml_type=14,
                                        token_id=tok, hidden_dim=K)
        assert api.call("dequant_embedding_row", a) == rxq4.SUCCESS
        want = orc.kq_embed_rows_f16(Wn, K, 14, np.array([tok], np.int32))[0]
        assert np.array_equal(host16(dst), want)
    ids = np.array([3, -1, V, 0, 39, 3, 12], np.int32)
    out = torch.empty((ids.size, K), dtype=torch.float16, device="cuda")
    capi.embed_rows_f16(out, W, V, dev(ids), K, ggml_type=14)
    assert np.array_equal(host16(out), orc.kq_embed_rows_f16(Wn, K, 14, ids))


def test_q6k_embedding_full_table_zipf():
    """The Q6_K gather at BASELINE configs[4]'s size: a [151936 x 2048] table
    of ggml-quantised N(0, 0.02) weights (rows of 1680 bytes), 4096 Zipf(1.1)
    ids over the whole vocabulary plus the last row and two out-of-range ids,
    bit-exact against the oracle's dequantisation of the addressed rows (the
    kernel's wave-uniform-row form: the K / 16 threads of a row are whole
    waves)."""
    vocab, K = 151936, 2048
    g = torch.Generator(device="cuda").manual_seed(48)
    src = torch.randn((vocab, K), generator=g, device="cuda") * 0.02
    table = capi.quantize_ggml(src, 14)
    del src
    ids = util.zipf_ids(49, 4096, vocab)
    ids[-1] = vocab - 1
    ids[5], ids[77] = -1, vocab
    out = torch.empty((ids.size, K), dtype=torch.float16, device="cuda")
    capi.embed_rows_f16(out, table, vocab, dev(ids), K, ggml_type=14)
    got = host16(out)
    ref = orc.kq_embed_rows_f16(table.cpu().numpy(), K, 14, ids)
    assert np.array_equal(got, ref)
    assert not got[5].any() and not got[77].any()
    assert np.unique(ids).size > 1000


@pytest.mark.parametrize("t", [13, 14])
# up to 16 tokens: the small-batch kernel (row tiles of 16 and 32); more:
# the MFMA GEMM (partial row and token tiles; the 64- and 40-row shapes split
# K 8 ways or more and take the four-wave workgroups; K = 11008 and 2304
# give Q6_K rows that start on odd 2-byte boundaries)
@pytest.mark.parametrize("M,N,K", [(300, 2, 2048), (129, 17, 512), (64, 40, 11008), (33, 5, 256),
                                   (600, 130, 1024), (2100, 70, 512), (1000, 300, 2304),
                                   (96, 40, 256), (40, 24, 65536)])
def test_kq_gemm(t, M, N, K):
    print(f"kq gemm type {t} M={M} N={N} K={K}", flush=True)
    Wn = kb.random_blocks(t, util.rng(740 + t + N), M, K)
    W = dev(Wn)
    # bf16 activations, fp32 and bf16 outputs
    xb = util.f32_to_bf16_bits(util.gaussian(741 + N, (N, K)))
    xv = orc.bits_bf16_to_f32(xb)
    ref = orc.kq_gemm_f64(Wn, K, t, xv, "bf16")
    x = torch.from_numpy(xb.view(np.int16)).cuda().view(torch.bfloat16)
    y32 = torch.empty((N, M), dtype=torch.float32, device="cuda")
    capi.gemm(y32, W, x, M, N, K, ggml_type=t)
    assert util.rel_err(y32.cpu().numpy(), ref) <= util.TOL
    yb = torch.empty((N, M), dtype=torch.bfloat16, device="cuda")
    capi.gemm(yb, W, x, M, N, K, ggml_type=t)
    assert util.rounded_ok(yb.view(torch.int16).cpu().numpy().view(np.uint16), ref, "bf16").all()
    # the reference API: fp16 in and out
    x16 = util.x_f16(742 + N, (N, K))
    ref16 = orc.kq_gemm_f64(Wn, K, t, f16(x16), "f16")
    y = torch.empty((N, M), dtype=torch.float16, device="cuda")
    xd = dev(x16)
    a = api.GemmQuantBatchedArgs(y=y.data_ptr(), weights=W.data_ptr(), ggml_type=t,
                                 x=xd.data_ptr(), M=M, N=N, K=K)
    assert api.call("gemm_quant_batched", a) == rxq4.SUCCESS
    assert util.rounded_ok(host16(y), ref16).all()


def test_kq_gemm_n1_is_the_gemv():
    M, K = 200, 2048
    Wn = kb.random_blocks(14, util.rng(750), M, K)
    x16 = util.x_f16(751, (1, K))
    W, x = dev(Wn), dev(x16)
    y = torch.empty((1, M), dtype=torch.float16, device="cuda")
    capi.gemm_f16(y, W, x, M, 1, K, ggml_type=14)
    y2 = torch.empty(M, dtype=torch.float16, device="cuda")
    capi.gemv_f16(y2, W, x, M, K, ggml_type=14)
    assert torch.equal(y[0], y2)


@pytest.mark.parametrize("t", [13, 14])
def test_kq_gemm_full_size_sampled_rows(t):
    """m = 512 on [11008 x 2048] and [2048 x 11008] (split K) with ggml-quantised
    weights: 192 sampled rows against the fp64 oracle on the bf16-rounded
    weights, fp32 out."""
    for M, K in ((11008, 2048), (2048, 11008)):
        print(f"kq gemm full size type {t} M={M} K={K}", flush=True)
        N = 512
        g = torch.Generator(device="cuda").manual_seed(770 + t + K)
        W = capi.quantize_ggml(torch.randn((M, K), generator=g, device="cuda") * 0.02, t)
        x = torch.randn((N, K), generator=g, device="cuda").to(torch.bfloat16)
        y = torch.empty((N, M), dtype=torch.float32, device="cuda")
        capi.gemm(y, W, x, M, N, K, ggml_type=t)
        rows = np.sort(util.rng(771 + t).choice(M, 192, replace=False))
        Wn = W[torch.from_numpy(rows).cuda()].cpu().numpy()
        ref = orc.kq_gemm_f64(Wn, K, t, x.float().cpu().numpy(), "bf16")
        assert util.rel_err(y.cpu().numpy()[:, rows], ref) <= util.TOL


def test_gemm_random_shapes_all_paths():
    """Seeded random shapes over every product path (multi-token GEMV,
    small-batch MFMA with and without the K split or LDS staging, the GEMM
    with and without split K), all three formats and both x types, against
    the fp64 oracle on the operand-rounded weights."""
    r = util.rng(790)
    for case in range(24):
        t = int(r.choice([12, 13, 14]))
        K = 256 * int(r.choice([1, 2, 3, 5, 8, 16, 17, 43]))
        M = int(r.integers(1, 700))
        N = int(r.choice([2, 3, 4, 5, 9, 16, 17, 40, 129, 300]))
        xt = r.choice(["f16", "bf16"])
        print(f"random gemm case {case}: type {t} M={M} N={N} K={K} x={xt}", flush=True)
        Wn = util.weights(800 + case, M, K) if t == 12 else kb.random_blocks(t, util.rng(800 + case), M, K)
        W = dev(Wn)
        xf = util.gaussian(900 + case, (N, K))
        y = torch.empty((N, M), dtype=torch.float32, device="cuda")
        if xt == "bf16":
            xb = util.f32_to_bf16_bits(xf)
            x = torch.from_numpy(xb.view(np.int16)).cuda().view(torch.bfloat16)
            xv = orc.bits_bf16_to_f32(xb)
        else:
            x16 = util.x_f16(900 + case, (N, K))
            x = dev(x16).view(torch.float16)
            xv = f16(x16)
        capi.gemm(y, W, x, M, N, K, ggml_type=t)
        # Q4_K with 1-3 fp16 tokens may run the GEMV (weights unrounded),
        # everything else the MFMA kernels on weights rounded to the x type
        wkind = None if (t == 12 and xt == "f16" and util.gemv_path(N, M, K)) else xt
        ref = orc.kq_gemm_f64(Wn, K, t, xv, wkind)
        assert util.rel_err(y.cpu().numpy(), ref) <= util.TOL, f"case {case}"


def test_q6k_row_slice_at_its_natural_2_byte_alignment():
    """A Q6_K [N x 11008] tensor has 9030-byte rows, so a slice that starts at
    an odd row sits 2 bytes past a dword (6 past a 16-byte boundary).  The C
    ABI takes it wherever the slice starts, as the reference does
    (q4_gemm.cu:2023-2076 check no alignment): GEMV, small batch, GEMM, the
    mixed triple and the gather on the slice match the oracle on the same rows."""
    K, N_rows, r0, M = 11008, 129, 1, 100
    rb = (K // 256) * 210
    Wn = kb.random_blocks(14, util.rng(790), N_rows, K).reshape(N_rows, rb)
    W = dev(Wn)
    Ws = W[r0:r0 + M]
    assert Ws.data_ptr() % 4 == 2 and Ws.data_ptr() % 16 != 0
    Wsn = np.ascontiguousarray(Wn[r0:r0 + M])
    x16 = util.x_f16(791, K)
    x = dev(x16)
    ref = orc.kq_gemv_f32(Wsn, K, 14, x16)
    y32 = torch.empty(M, dtype=torch.float32, device="cuda")
    capi.gemv_f32(y32, Ws, x, M, K, ggml_type=14)
    assert util.rel_err(y32.cpu().numpy(), ref) <= util.TOL
    y16 = torch.empty(M, dtype=torch.float16, device="cuda")
    capi.gemv_f16(y16, Ws, x, M, K, ggml_type=14)
    assert util.rounded_ok(host16(y16), ref).all()
    # the mixed triple with the Q6_K range as the slice
    Wq = util.weights(792, 64, K)
    ys = [torch.empty(64, dtype=torch.float16, device="cuda"),
          torch.empty(M, dtype=torch.float16, device="cuda")]
    capi.gemv_multi_f16([(ys[0], dev(Wq), 64, 12), (ys[1], Ws, M, 14)], x, K)
    assert util.rounded_ok(host16(ys[0]), orc.kq_gemv_f32(Wq, K, 12, x16)).all()
    assert util.rounded_ok(host16(ys[1]), ref).all()
    # small batch (4 tokens) and the GEMM (40 tokens), fp16 in and out
    for n in (4, 40):
        xn16 = util.x_f16(793 + n, (n, K))
        refn = orc.kq_gemm_f64(Wsn, K, 14, f16(xn16), "f16")
        yn = torch.empty((n, M), dtype=torch.float16, device="cuda")
        capi.gemm_f16(yn, Ws, dev(xn16), M, n, K, ggml_type=14)
        assert util.rounded_ok(host16(yn), refn).all(), n
    # gather from the sliced table
    ids = np.array([0, 5, M - 1, 5, M, -2], np.int32)
    out = torch.empty((ids.size, K), dtype=torch.float16, device="cuda")
    capi.embed_rows_f16(out, Ws, M, dev(ids), K, ggml_type=14)
    assert np.array_equal(host16(out), orc.kq_embed_rows_f16(Wsn, K, 14, ids))
    # a Q4_K slice still needs 16 bytes: refused, nothing launched
    Wq4 = dev(util.weights(794, 8, K))
    with pytest.raises(rxq4.RxQ4Error):
        capi.gemv_f16(torch.empty(4, dtype=torch.float16, device="cuda"), Wq4.view(-1)[2:], x, 4, K)
