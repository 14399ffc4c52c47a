"""ctypes binding of the C ABI in include/rxq4.h, plus torch-tensor helpers.

Every helper takes device tensors, passes raw pointers, launches on the given
stream (default: torch's current stream) and raises :class:`rxq4.RxQ4Error`
on a non-success status.
"""
from __future__ import annotations

import ctypes

import torch

from . import DTYPE_BF16, DTYPE_F16, DTYPE_F32, GGML_TYPE_Q4_K, SUCCESS, RxQ4Error, load

c_void_p, c_int, c_int64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64


class Rows(ctypes.Structure):
    """rxq4_rows: one output range of a multi-matrix GEMV."""
    _fields_ = [("y", c_void_p), ("w", c_void_p), ("ggml_type", c_int), ("M", c_int)]


# name -> (restype, argtypes); every name is declared in include/rxq4.h.
SIGNATURES = {
    "rxq4_gemv_f16": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_int, c_int, c_void_p]),
    "rxq4_gemv_add_f16": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int, c_int,
                                  c_void_p]),
    "rxq4_gemv_multi_f16": (c_int, [ctypes.POINTER(Rows), c_int, c_void_p, c_int, c_void_p]),
    "rxq4_gemv_f32": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_int, c_int, c_void_p]),
    "rxq4_gemm_f16": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_int, c_int, c_int,
                              c_void_p]),
    "rxq4_embed_row_f16": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "rxq4_gemm": (c_int, [c_void_p, c_int, c_void_p, c_int, c_void_p, c_int, c_int, c_int,
                          c_int, c_void_p]),
    "rxq4_embed_rows_f16": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_int, c_int,
                                    c_void_p]),
    "rxq4_gemm_noalloc": (c_int, [c_void_p, c_int, c_void_p, c_int, c_void_p, c_int, c_int, c_int,
                                  c_int, c_void_p]),
    "rxq4_quantize_q4k": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_void_p]),
    "rxq4_quantize": (c_int, [c_void_p, c_int, c_void_p, c_int64, c_int, c_void_p]),
    "rxq4_attention_decode_f16": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                          c_int, c_int, ctypes.c_float, c_int, c_void_p,
                                          c_void_p, c_void_p]),
    "rxq4_attention_prefill_f16": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                           c_int, c_int, c_int, ctypes.c_float, c_int, c_void_p,
                                           c_void_p, c_void_p]),
    "rxq4_host_gemv": (c_int, [c_void_p, c_int, c_void_p, c_int, c_void_p, c_void_p, c_int,
                               c_int]),
    "rxq4_host_gemv_calls": (ctypes.c_longlong, []),
    "rxq4_reserve_workspace": (c_int, [c_void_p]),
    "rxq4_release_workspace": (c_int, [c_void_p]),
    "rxq4_resolve_weights": (c_void_p, [c_void_p, c_void_p]),
    "rxq4_version": (ctypes.c_char_p, []),
    "rxq4_last_error": (ctypes.c_char_p, []),
}

_L = None


def _bind(lib: ctypes.CDLL) -> None:
    global _L
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _L = lib


def lib() -> ctypes.CDLL:
    if _L is None:
        load()
    return _L


def last_error() -> str:
    return lib().rxq4_last_error().decode()


def _check(status: int, what: str) -> int:
    if status != SUCCESS:
        raise RxQ4Error(status, f"{what} ({last_error()})")
    return status


def _stream(stream) -> int:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, torch.cuda.Stream):
        return stream.cuda_stream
    return int(stream)


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _dtype_code(t: torch.Tensor) -> int:
    return {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}[t.dtype]


def gemv_f16(y, w, x, M, K, stream=None, ggml_type=GGML_TYPE_Q4_K):
    return _check(lib().rxq4_gemv_f16(_ptr(y), _ptr(w), ggml_type, _ptr(x), M, K,
                                      _stream(stream)), "rxq4_gemv_f16")


def gemv_f32(y, w, x, M, K, stream=None, ggml_type=GGML_TYPE_Q4_K):
    return _check(lib().rxq4_gemv_f32(_ptr(y), _ptr(w), ggml_type, _ptr(x), M, K,
                                      _stream(stream)), "rxq4_gemv_f32")


def gemv_add_f16(y, w, x, residual, M, K, stream=None, ggml_type=GGML_TYPE_Q4_K):
    return _check(lib().rxq4_gemv_add_f16(_ptr(y), _ptr(w), ggml_type, _ptr(x), _ptr(residual),
                                          M, K, _stream(stream)), "rxq4_gemv_add_f16")


def gemv_multi_f16(ranges, x, K, stream=None):
    """ranges: list of (y, w, M) or (y, w, M, ggml_type)."""
    arr = (Rows * len(ranges))()
    for i, r in enumerate(ranges):
        y, w, M = r[0], r[1], r[2]
        t = r[3] if len(r) > 3 else GGML_TYPE_Q4_K
        arr[i] = Rows(_ptr(y), _ptr(w), t, M)
    return _check(lib().rxq4_gemv_multi_f16(arr, len(ranges), _ptr(x), K, _stream(stream)),
                  "rxq4_gemv_multi_f16")


def gemm_f16(y, w, x, M, N, K, stream=None, ggml_type=GGML_TYPE_Q4_K):
    return _check(lib().rxq4_gemm_f16(_ptr(y), _ptr(w), ggml_type, _ptr(x), M, N, K,
                                      _stream(stream)), "rxq4_gemm_f16")


def gemm(y, w, x, M, N, K, stream=None, ggml_type=GGML_TYPE_Q4_K):
    """Typed GEMM: dtypes taken from the tensors (x fp16|bf16, y fp32|fp16|bf16)."""
    return _check(lib().rxq4_gemm(_ptr(y), _dtype_code(y), _ptr(w), ggml_type, _ptr(x),
                                  _dtype_code(x), M, N, K, _stream(stream)), "rxq4_gemm")


def gemm_noalloc(y, w, x, M, N, K, stream=None, ggml_type=GGML_TYPE_Q4_K):
    """rxq4_gemm with its split partials in the library's fixed device array
    (allocates nothing)."""
    return _check(lib().rxq4_gemm_noalloc(_ptr(y), _dtype_code(y), _ptr(w), ggml_type, _ptr(x),
                                          _dtype_code(x), M, N, K, _stream(stream)),
                  "rxq4_gemm_noalloc")


def embed_row_f16(dst, w, token_id, hidden, stream=None, ggml_type=GGML_TYPE_Q4_K):
    return _check(lib().rxq4_embed_row_f16(_ptr(dst), _ptr(w), ggml_type, token_id, hidden,
                                           _stream(stream)), "rxq4_embed_row_f16")


def embed_rows_f16(dst, w, n_vocab, ids, hidden, stream=None, ggml_type=GGML_TYPE_Q4_K):
    return _check(lib().rxq4_embed_rows_f16(_ptr(dst), _ptr(w), ggml_type, n_vocab, _ptr(ids),
                                            ids.numel(), hidden, _stream(stream)),
                  "rxq4_embed_rows_f16")


def quantize_q4k(dst, src, n_rows, K, stream=None):
    return _check(lib().rxq4_quantize_q4k(_ptr(dst), _ptr(src), n_rows, K, _stream(stream)),
                  "rxq4_quantize_q4k")


def quantize(src: torch.Tensor, stream=None) -> torch.Tensor:
    """Quantise a device fp32 [rows, K] tensor to a uint8 [rows, K/256*144] tensor."""
    rows, K = src.shape
    dst = torch.empty((rows, (K // 256) * 144), dtype=torch.uint8, device=src.device)
    quantize_q4k(dst, src.contiguous(), rows, K, stream)
    return dst


_TYPE_BYTES = {12: 144, 13: 176, 14: 210}


def quantize_ggml(src: torch.Tensor, ggml_type: int = GGML_TYPE_Q4_K, stream=None) -> torch.Tensor:
    """ggml's reference quantiser on the GPU: device fp32 [rows, K] -> uint8
    [rows, K/256 * block bytes] of ggml_type 12, 13 or 14."""
    rows, K = src.shape
    dst = torch.empty((rows, (K // 256) * _TYPE_BYTES.get(ggml_type, 144)), dtype=torch.uint8,
                      device=src.device)
    _check(lib().rxq4_quantize(_ptr(dst), ggml_type, _ptr(src.contiguous()), rows, K,
                               _stream(stream)), "rxq4_quantize")
    return dst


def attention_decode_f16(out, q, k, v, n_heads, n_kv_heads, head_dim, seq_len, scale,
                         kv_int8=False, k_scales=None, v_scales=None, stream=None):
    return _check(lib().rxq4_attention_decode_f16(
        _ptr(out), _ptr(q), _ptr(k), _ptr(v), n_heads, n_kv_heads, head_dim, seq_len, scale,
        int(kv_int8), _ptr(k_scales), _ptr(v_scales), _stream(stream)), "rxq4_attention_decode_f16")


def attention_prefill_f16(out, q, k, v, n_heads, n_kv_heads, head_dim, N, start_pos, scale,
                          kv_int8=False, k_scales=None, v_scales=None, stream=None):
    return _check(lib().rxq4_attention_prefill_f16(
        _ptr(out), _ptr(q), _ptr(k), _ptr(v), n_heads, n_kv_heads, head_dim, N, start_pos, scale,
        int(kv_int8), _ptr(k_scales), _ptr(v_scales), _stream(stream)),
        "rxq4_attention_prefill_f16")


def host_gemv(w, x, M: int, K: int, ggml_type: int = GGML_TYPE_Q4_K, out: str = "f32",
              residual=None):
    """The host GEMV (rxq4_host_gemv) on numpy arrays: w uint8 blocks, x fp16
    bits (uint16); out "f32" -> float32 [M], "f16" -> uint16 fp16 bits [M];
    residual (uint16 fp16 bits [M]) gives the add variant."""
    import numpy as np
    w = np.ascontiguousarray(w)
    x = np.ascontiguousarray(x, dtype=np.uint16)
    y = np.empty(M, dtype=np.float32 if out == "f32" else np.uint16)
    res = None if residual is None else np.ascontiguousarray(residual, dtype=np.uint16)
    _check(lib().rxq4_host_gemv(y.ctypes.data, DTYPE_F32 if out == "f32" else DTYPE_F16,
                                w.ctypes.data, ggml_type, x.ctypes.data,
                                None if res is None else res.ctypes.data, M, K),
           "rxq4_host_gemv")
    return y


def host_gemv_calls() -> int:
    """Computations made by the host GEMV in this process so far."""
    return int(lib().rxq4_host_gemv_calls())


def reserve_workspace(stream=None):
    return _check(lib().rxq4_reserve_workspace(_stream(stream)), "rxq4_reserve_workspace")


def release_workspace(stream=None):
    return _check(lib().rxq4_release_workspace(_stream(stream)), "rxq4_release_workspace")
