"""GGUF ingest on the GPU: the device copy of a file's data section is
byte-identical to the file, and the reflex::infer API fed the mapped host
address as `weights` and the device copy as `weights_device` (the caller's
aliasing contract, reference include/reflex/infer.h:94-95, q4_gemm.cu:111-135)
computes the same GEMV / embedding rows as the oracle on the file's bytes.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import rxq4
from oracle import oracle as orc
from rxq4 import api, gguf
from tests import gguf_writer as gw
from tests import kquant_blocks as kb
from tests import util

pytestmark = pytest.mark.gpu


@pytest.mark.host_path
def test_upload_bytes_and_gemv_through_alias(tmp_path):
    K = 2048
    q4 = util.weights(850, 256, K)
    q6 = kb.random_blocks(14, util.rng(851), 40, K)
    tens = [("blk.0.attn_q.weight", 12, (K, 256), q4.tobytes()),
            ("token_embd.weight", 14, (K, 40), q6.tobytes()),
            ("output_norm.weight", 0, (K,), gw.f32_tensor(np.ones(K)))]
    path = tmp_path / "m.gguf"
    gw.write(path, [("general.architecture", gw.STRING, "qwen3")], tens)
    with gguf.GGUFFile(path) as f:
        dev = f.upload()
        torch.cuda.synchronize()
        host = np.fromfile(path, np.uint8)[-f.data_bytes:]
        assert np.array_equal(dev.data.cpu().numpy(), host)
        # GEMV: weights = mapped host address, weights_device = device alias.
        t = f.tensors["blk.0.attn_q.weight"]
        x16 = util.x_f16(852, K)
        x = torch.from_numpy(x16.view(np.int16)).cuda()
        y = torch.empty(t.rows, dtype=torch.float16, device="cuda")
        a = api.GemvQuantArgs(y=y.data_ptr(), weights=t.host, weights_device=dev.ptr(t.name),
                              ggml_type=t.ggml_type, x=x.data_ptr(), M=t.rows, K=t.row_length)
        assert api.call("gemv_quant", a) == rxq4.SUCCESS
        ref = orc.gemv_f32(f.host_array(t.name), K, x16)
        got = y.view(torch.int16).cpu().numpy().view(np.uint16)
        assert util.rounded_ok(got, ref).all()
        # The mapped host address alone (no alias) takes the reference's host
        # path (q4_gemm.cu:1886-1899): bit for bit its CPU loop.
        a.weights_device = None
        assert api.call("gemv_quant", a) == rxq4.SUCCESS
        got = y.view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(got, orc.gemv_f16(f.host_array(t.name), K, x16))
        # Q6_K embedding row through the alias, bit-exact.
        e = f.tensors["token_embd.weight"]
        dst = torch.empty(K, dtype=torch.float16, device="cuda")
        d = api.DequantEmbeddingRowArgs(dst=dst.data_ptr(), weights=e.host,
                                        weights_device=dev.ptr(e.name), ggml_type=14,
                                        token_id=17, hidden_dim=K)
        assert api.call("dequant_embedding_row", d) == rxq4.SUCCESS
        want = orc.kq_embed_rows_f16(f.host_array(e.name), K, 14, np.array([17], np.int32))[0]
        assert np.array_equal(dst.view(torch.int16).cpu().numpy().view(np.uint16), want)


def test_upload_spans_several_staging_chunks(tmp_path):
    """A 75 MB data section (the staging buffers hold 32 MB each), with an
    odd-sized tensor so the last chunk is partial."""
    r = np.random.default_rng(860)
    a = r.integers(0, 256, 40_000_011, dtype=np.uint8)
    b = r.integers(0, 256, 35_000_000, dtype=np.uint8)
    path = tmp_path / "big.gguf"
    gw.write(path, [], [("a", 24, (a.size,), a.tobytes()), ("b", 24, (b.size,), b.tobytes())])
    with gguf.GGUFFile(path) as f:
        dev = f.upload()
        torch.cuda.synchronize()
        assert torch.equal(dev.tensor("a").cpu(), torch.from_numpy(a))
        assert torch.equal(dev.tensor("b").cpu(), torch.from_numpy(b))
        assert dev.ptr("b") % 32 == 0


def test_upload_rejects_small_or_host_destination(tmp_path):
    path = tmp_path / "s.gguf"
    gw.write(path, [], [("w", 12, (256, 4), bytes(576))])
    with gguf.GGUFFile(path) as f:
        L = gguf.lib()
        small = torch.empty(1024, dtype=torch.uint8, device="cuda")
        assert L.rxq4_gguf_upload(f._h, small.data_ptr(), 100, None) == rxq4.INVALID_ARGUMENT
        host = torch.empty(4096, dtype=torch.uint8).pin_memory()
        base = host.data_ptr() + (-host.data_ptr()) % 256
        assert L.rxq4_gguf_upload(f._h, base, 1024, None) == rxq4.INVALID_ARGUMENT
