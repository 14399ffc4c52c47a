"""Dispatcher and argument checks of the C++ API and the C ABI that need no
GPU: the plug-in registry (reference src/dispatch.cpp:29-98), the attention
stubs, and validation that fails before any HIP call."""
from __future__ import annotations

import ctypes

import pytest

import rxq4
from rxq4 import api, capi


@pytest.fixture(autouse=True)
def _restore_registry():
    yield
    api.register_q4_backend(api.Q4Kernels())


def test_registry_starts_empty():
    k = api.registered_q4_backend()
    for name, _ in api.Q4Kernels._fields_:
        assert not ctypes.cast(getattr(k, name), ctypes.c_void_p).value, name


def test_registered_backend_receives_every_call():
    seen = {}

    def make(name, status):
        fnty = dict(api.Q4Kernels._fields_)[name]

        def cb(p):
            seen[name] = p.contents
            return status
        return fnty(cb)

    statuses = dict(zip([n for n, _ in api.Q4Kernels._fields_], [0, 1, 2, 3, 4, 5, 0]))
    cbs = {n: make(n, s) for n, s in statuses.items()}
    api.register_q4_backend(api.Q4Kernels(**cbs))

    k = api.registered_q4_backend()
    for n in statuses:
        assert ctypes.cast(getattr(k, n), ctypes.c_void_p).value == \
            ctypes.cast(cbs[n], ctypes.c_void_p).value

    a = api.GemvQuantArgs(y=0x1000, weights=0x2000, weights_device=0x3000, ggml_type=12,
                          x=0x4000, M=7, K=512, stream=0x5000)
    assert api.call("gemv_quant", a) == statuses["gemv_quant"]
    got = seen["gemv_quant"]
    assert (got.y, got.weights, got.weights_device, got.ggml_type, got.x, got.M, got.K,
            got.stream) == (0x1000, 0x2000, 0x3000, 12, 0x4000, 7, 512, 0x5000)
    assert api.call("gemv_quant_add", api.GemvQuantAddArgs(residual=0x77, M=3)) == 1
    assert seen["gemv_quant_add"].residual == 0x77
    assert api.call("gemv_quant_pair", api.GemvQuantPairArgs(M0=1, M1=2)) == 2
    assert (seen["gemv_quant_pair"].M0, seen["gemv_quant_pair"].M1) == (1, 2)
    assert api.call("gemv_quant_triple", api.GemvQuantTripleArgs(M2=9)) == 3
    assert seen["gemv_quant_triple"].M2 == 9
    assert api.call("gemm_quant_batched", api.GemmQuantBatchedArgs(N=5)) == 4
    assert seen["gemm_quant_batched"].N == 5
    assert api.call("gemv_quant_f32", api.GemvQuantF32Args(K=256)) == 5
    assert api.call("dequant_embedding_row", api.DequantEmbeddingRowArgs(token_id=11)) == 0
    assert seen["dequant_embedding_row"].token_id == 11


def test_null_member_restores_builtin_slot():
    fn = api.DequantEmbeddingRowFn(lambda p: 3)
    api.register_q4_backend(api.Q4Kernels(dequant_embedding_row=fn))
    assert api.call("dequant_embedding_row", api.DequantEmbeddingRowArgs(hidden_dim=100)) == 3
    api.register_q4_backend(api.Q4Kernels())
    # built-in path: hidden_dim % 256 != 0 is rejected before any HIP call
    assert api.call("dequant_embedding_row",
                    api.DequantEmbeddingRowArgs(hidden_dim=100)) == rxq4.INVALID_ARGUMENT
    assert api.call("dequant_embedding_row",
                    api.DequantEmbeddingRowArgs(hidden_dim=0)) == rxq4.INVALID_ARGUMENT


def test_attention_validates_before_launch():
    # no heads: nothing to do (the reference returns Success for every call)
    assert api.call("flash_attention_decode", api.AttentionDecodeArgs()) == rxq4.SUCCESS
    assert api.call("flash_attention_prefill_batched",
                    api.AttentionPrefillBatchedArgs()) == rxq4.SUCCESS
    # shape errors are reported before any HIP call
    bad_gqa = api.AttentionDecodeArgs(n_heads=6, n_kv_heads=4, head_dim=64, seq_len=8)
    assert api.call("flash_attention_decode", bad_gqa) == rxq4.INVALID_ARGUMENT
    bad_dim = api.AttentionPrefillBatchedArgs(n_heads=8, n_kv_heads=2, head_dim=72, N=2,
                                             kv_int8=True)
    assert api.call("flash_attention_prefill_batched", bad_dim) == rxq4.INVALID_ARGUMENT
    too_big = api.AttentionDecodeArgs(n_heads=8, n_kv_heads=8, head_dim=512, seq_len=8)
    assert api.call("flash_attention_decode", too_big) == rxq4.INVALID_ARGUMENT


def test_empty_gemm_is_a_no_op():
    assert api.call("gemm_quant_batched", api.GemmQuantBatchedArgs(M=0, N=4, K=256)) == 0
    assert api.call("gemm_quant_batched", api.GemmQuantBatchedArgs(M=4, N=0, K=256)) == 0


def test_c_abi_rejects_bad_arguments_before_launch():
    L = capi.lib()
    w = 0x10000  # never dereferenced: every call below fails validation first
    assert L.rxq4_gemv_f16(w, w, 15, w, 4, 256, None) == rxq4.UNSUPPORTED_QUANT_FORMAT
    assert L.rxq4_gemv_f16(w, w, 13, w, 4, 100, None) == rxq4.INVALID_ARGUMENT
    assert L.rxq4_gemm_f16(w, w, 14, w, 4, 4, 100, None) == rxq4.INVALID_ARGUMENT
    assert L.rxq4_gemv_f16(w, w, 12, w, 4, 100, None) == rxq4.INVALID_ARGUMENT
    assert "K=100" in capi.last_error()
    assert L.rxq4_gemv_f32(w, w + 4, 12, w, 4, 256, None) == rxq4.INVALID_ARGUMENT
    assert L.rxq4_gemv_f16(w, w, 12, w, 4, 65536 + 256, None) == rxq4.INVALID_ARGUMENT
    assert L.rxq4_gemv_multi_f16(None, 0, w, 256, None) == rxq4.INVALID_ARGUMENT
    assert L.rxq4_embed_row_f16(w, w, 12, 0, 300, None) == rxq4.INVALID_ARGUMENT
    assert L.rxq4_embed_row_f16(w, w, 13, 0, 256, None) == rxq4.UNSUPPORTED_QUANT_FORMAT
    assert L.rxq4_embed_rows_f16(w, w, 13, 8, w, 1, 256, None) == rxq4.UNSUPPORTED_QUANT_FORMAT
    assert L.rxq4_quantize_q4k(w, w, 4, 255, None) == rxq4.INVALID_ARGUMENT
    assert L.rxq4_gemm(w, 2, w, 12, w, 1, 4, 4, 256, None) == rxq4.INVALID_ARGUMENT  # bf16 y, f16 x
    assert L.rxq4_gemm(w, 1, w, 12, w + 8, 1, 4, 4, 256, None) == rxq4.INVALID_ARGUMENT
