"""numpy front end of the CPU oracle (oracle/q4k_oracle.c).

TEST INFRASTRUCTURE, NOT PRODUCT CODE: only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg may import this module, and only to check or
to time the CPU baseline.  Weights are uint8 arrays of raw Q4_K blocks
([rows, K/256*144]); fp16/bf16 values travel as uint16 bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")
QK_K = 256
BLOCK_BYTES = 144

_lib = None


def build() -> None:
    """Compile the oracle library (gcc; seconds)."""
    subprocess.run(["make", "-s", "-C", HERE, "-B", "_build/liboracle.so"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P, I, I64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
        sig = {
            "orc_fp16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_f32_to_fp16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_get_scale_min_k4": (None, [I, P, P, P]),
            "orc_pack_scale_min_k4": (None, [P, P, P]),
            "orc_dequant_rows_f32": (None, [P, I64, I64, I, P]),
            "orc_dequant_rows_f16": (None, [P, I64, I64, I, P]),
            "orc_dequant_rows_bf16": (None, [P, I64, I64, I, P]),
            "orc_embed_rows_f16": (None, [P, I64, I, P, I64, P]),
            "orc_gemv_f32": (None, [P, P, I64, I64, I, P]),
            "orc_gemv_f32_mt": (None, [P, P, I64, I, P, I]),
            "orc_gemv_f16": (None, [P, P, I64, I, P]),
            "orc_gemv_add_f16": (None, [P, P, P, I64, I, P]),
            "orc_gemm_tokens_f32": (None, [P, P, I64, I64, I, P]),
            "orc_gemv_f64": (None, [P, P, I64, I, P]),
            "orc_gemm_f64": (None, [P, P, I64, I64, I, I, P]),
            "orc_quantize_rows": (None, [P, I64, I, P]),
            "orc_quantize_ggml": (I, [I, P, I64, I, P]),
            "orc_block_bytes": (I, [I]),
            "orc_kq_dequant_rows_f32": (None, [P, I, I64, I64, I, P]),
            "orc_kq_embed_rows_f16": (None, [P, I, I64, I, P, I64, P]),
            "orc_kq_gemv_f32": (None, [P, I, P, I64, I64, I, P]),
            "orc_kq_gemm_f64": (None, [P, I, P, I64, I64, I, I, P]),
            "orc_attn_decode_f32": (None, [P, P, P, I, I, I, I, ctypes.c_float, I, P, P, P]),
            "orc_attn_prefill_f32": (None, [P, P, P, I, I, I, I, I, ctypes.c_float, I, P, P, P]),
            "orc_attn_decode_f64": (None, [P, P, P, I, I, I, I, ctypes.c_double, I, P, P, P]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def _w(W: np.ndarray, K: int) -> np.ndarray:
    W = np.ascontiguousarray(W, dtype=np.uint8)
    assert W.size % ((K // QK_K) * BLOCK_BYTES) == 0
    return W


def rows_of(W: np.ndarray, K: int) -> int:
    return W.size // ((K // QK_K) * BLOCK_BYTES)


def fp16_to_f32(bits: np.ndarray) -> np.ndarray:
    f = lib().orc_fp16_to_f32
    return np.array([f(int(b)) for b in np.asarray(bits).ravel()], dtype=np.float32)


def f32_to_fp16(vals: np.ndarray) -> np.ndarray:
    f = lib().orc_f32_to_fp16
    return np.array([f(float(v)) for v in np.asarray(vals, np.float32).ravel()], dtype=np.uint16)


def f32_to_bf16(vals: np.ndarray) -> np.ndarray:
    f = lib().orc_f32_to_bf16
    return np.array([f(float(v)) for v in np.asarray(vals, np.float32).ravel()], dtype=np.uint16)


def get_scale_min_k4(j: int, scales: np.ndarray):
    s = np.ascontiguousarray(scales, dtype=np.uint8)
    sc, mn = ctypes.c_uint8(), ctypes.c_uint8()
    lib().orc_get_scale_min_k4(j, _p(s), ctypes.byref(sc), ctypes.byref(mn))
    return sc.value, mn.value


def pack_scale_min_k4(sc, mn) -> np.ndarray:
    a = np.ascontiguousarray(sc, dtype=np.uint8)
    b = np.ascontiguousarray(mn, dtype=np.uint8)
    out = np.zeros(12, dtype=np.uint8)
    lib().orc_pack_scale_min_k4(_p(a), _p(b), _p(out))
    return out


def dequant_f32(W, K, row0=0, n_rows=None) -> np.ndarray:
    W = _w(W, K)
    n_rows = rows_of(W, K) - row0 if n_rows is None else n_rows
    out = np.empty((n_rows, K), dtype=np.float32)
    lib().orc_dequant_rows_f32(_p(W), row0, n_rows, K, _p(out))
    return out


def dequant_f16(W, K, row0=0, n_rows=None) -> np.ndarray:
    W = _w(W, K)
    n_rows = rows_of(W, K) - row0 if n_rows is None else n_rows
    out = np.empty((n_rows, K), dtype=np.uint16)
    lib().orc_dequant_rows_f16(_p(W), row0, n_rows, K, _p(out))
    return out


def dequant_bf16(W, K, row0=0, n_rows=None) -> np.ndarray:
    W = _w(W, K)
    n_rows = rows_of(W, K) - row0 if n_rows is None else n_rows
    out = np.empty((n_rows, K), dtype=np.uint16)
    lib().orc_dequant_rows_bf16(_p(W), row0, n_rows, K, _p(out))
    return out


def embed_rows_f16(W, K, ids) -> np.ndarray:
    W = _w(W, K)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    out = np.empty((ids.size, K), dtype=np.uint16)
    lib().orc_embed_rows_f16(_p(W), rows_of(W, K), K, _p(ids), ids.size, _p(out))
    return out


def gemv_f32(W, K, x16, row0=0, n_rows=None, threads=1) -> np.ndarray:
    """Reference CPU GEMV (fp32 out).  x16: uint16 fp16 bits [K]."""
    W = _w(W, K)
    x16 = np.ascontiguousarray(x16, dtype=np.uint16)
    n_rows = rows_of(W, K) - row0 if n_rows is None else n_rows
    y = np.empty(n_rows, dtype=np.float32)
    if threads > 1 and row0 == 0:
        lib().orc_gemv_f32_mt(_p(W), _p(x16), n_rows, K, _p(y), threads)
    else:
        lib().orc_gemv_f32(_p(W), _p(x16), row0, n_rows, K, _p(y))
    return y


def gemv_f16(W, K, x16) -> np.ndarray:
    W = _w(W, K)
    x16 = np.ascontiguousarray(x16, dtype=np.uint16)
    M = rows_of(W, K)
    y = np.empty(M, dtype=np.uint16)
    lib().orc_gemv_f16(_p(W), _p(x16), M, K, _p(y))
    return y


def gemv_add_f16(W, K, x16, res16) -> np.ndarray:
    W = _w(W, K)
    x16 = np.ascontiguousarray(x16, dtype=np.uint16)
    res16 = np.ascontiguousarray(res16, dtype=np.uint16)
    M = rows_of(W, K)
    y = np.empty(M, dtype=np.uint16)
    lib().orc_gemv_add_f16(_p(W), _p(x16), _p(res16), M, K, _p(y))
    return y


def gemm_tokens_f32(W, K, x16) -> np.ndarray:
    """Per-token reference GEMV: x16 [N, K] fp16 bits -> y [N, M] fp32."""
    W = _w(W, K)
    x16 = np.ascontiguousarray(x16, dtype=np.uint16)
    N = x16.shape[0]
    M = rows_of(W, K)
    y = np.empty((N, M), dtype=np.float32)
    lib().orc_gemm_tokens_f32(_p(W), _p(x16), M, N, K, _p(y))
    return y


def gemv_f64(W, K, x32) -> np.ndarray:
    W = _w(W, K)
    x32 = np.ascontiguousarray(x32, dtype=np.float32)
    M = rows_of(W, K)
    y = np.empty(M, dtype=np.float64)
    lib().orc_gemv_f64(_p(W), _p(x32), M, K, _p(y))
    return y


def gemm_f64(W, K, x32, wkind: str) -> np.ndarray:
    """fp64 GEMM with weights rounded to 'f16' or 'bf16'; x32 [N, K] fp32 values.
    (Unrounded weights: kq_gemm_f64(W, K, 12, x32, None).)"""
    assert wkind in ("f16", "bf16"), wkind
    W = _w(W, K)
    x32 = np.ascontiguousarray(x32, dtype=np.float32)
    N = x32.shape[0]
    M = rows_of(W, K)
    y = np.empty((N, M), dtype=np.float64)
    lib().orc_gemm_f64(_p(W), _p(x32), M, N, K, 1 if wkind == "bf16" else 0, _p(y))
    return y


def quantize(src: np.ndarray) -> np.ndarray:
    """fp32 [rows, K] -> uint8 [rows, K/256*144] (the build's own quantiser)."""
    src = np.ascontiguousarray(src, dtype=np.float32)
    rows, K = src.shape
    out = np.empty((rows, (K // QK_K) * BLOCK_BYTES), dtype=np.uint8)
    lib().orc_quantize_rows(_p(src), rows, K, _p(out))
    return out


# ---------------------------------------------------------------- Q5_K / Q6_K
TYPE_BYTES = {12: 144, 13: 176, 14: 210}


def quantize_ggml(src: np.ndarray, t: int) -> np.ndarray:
    """fp32 [rows, K] -> uint8 [rows, K/256 * bytes(t)] with ggml's reference
    quantiser for type t (12, 13, 14)."""
    src = np.ascontiguousarray(src, dtype=np.float32)
    rows, K = src.shape
    out = np.empty((rows, (K // QK_K) * TYPE_BYTES[t]), dtype=np.uint8)
    assert lib().orc_quantize_ggml(t, _p(src), rows, K, _p(out)) == 0
    return out


def _wt(W, K, t):
    W = np.ascontiguousarray(W, dtype=np.uint8)
    assert W.size % ((K // QK_K) * TYPE_BYTES[t]) == 0
    return W, W.size // ((K // QK_K) * TYPE_BYTES[t])


def kq_dequant_f32(W, K, t, row0=0, n_rows=None) -> np.ndarray:
    """Dequantise rows of ggml type t (12, 13, 14) to fp32."""
    W, rows = _wt(W, K, t)
    n_rows = rows - row0 if n_rows is None else n_rows
    out = np.empty((n_rows, K), dtype=np.float32)
    lib().orc_kq_dequant_rows_f32(_p(W), t, row0, n_rows, K, _p(out))
    return out


def kq_embed_rows_f16(W, K, t, ids) -> np.ndarray:
    W, rows = _wt(W, K, t)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    out = np.empty((ids.size, K), dtype=np.uint16)
    lib().orc_kq_embed_rows_f16(_p(W), t, rows, K, _p(ids), ids.size, _p(out))
    return out


def kq_gemv_f32(W, K, t, x16, row0=0, n_rows=None) -> np.ndarray:
    """Reference CPU GEMV (gemv_quant_cpu) for ggml type t; x16 fp16 bits [K]."""
    W, rows = _wt(W, K, t)
    x16 = np.ascontiguousarray(x16, dtype=np.uint16)
    n_rows = rows - row0 if n_rows is None else n_rows
    y = np.empty(n_rows, dtype=np.float32)
    lib().orc_kq_gemv_f32(_p(W), t, _p(x16), row0, n_rows, K, _p(y))
    return y


def kq_gemm_f64(W, K, t, x32, wkind: str | None) -> np.ndarray:
    """fp64 y[N, M] with weights rounded to 'f16' / 'bf16' / not at all (None)."""
    W, rows = _wt(W, K, t)
    x32 = np.ascontiguousarray(np.atleast_2d(x32), dtype=np.float32)
    N = x32.shape[0]
    y = np.empty((N, rows), dtype=np.float64)
    kind = {"f16": 0, "bf16": 1, None: -1}[wkind]
    lib().orc_kq_gemm_f64(_p(W), t, _p(x32), rows, N, K, kind, _p(y))
    return y


# ---------------------------------------------------------------- attention
def _kv(k, kv_int8):
    return np.ascontiguousarray(k, dtype=np.int8 if kv_int8 else np.uint16)


def attn_decode_f32(q16, k, v, n_heads, n_kv, head_dim, seq_len, scale, kv_int8=False,
                    ks=None, vs=None) -> np.ndarray:
    """Reference CPU decode attention; q16 fp16 bits [n_heads*head_dim]; k, v
    fp16 bits (uint16) or int8 [seq_len, n_kv, head_dim]."""
    q16 = np.ascontiguousarray(q16, dtype=np.uint16)
    k, v = _kv(k, kv_int8), _kv(v, kv_int8)
    ks = None if ks is None else np.ascontiguousarray(ks, dtype=np.float32)
    vs = None if vs is None else np.ascontiguousarray(vs, dtype=np.float32)
    out = np.empty(n_heads * head_dim, dtype=np.float32)
    lib().orc_attn_decode_f32(_p(q16), _p(k), _p(v), n_heads, n_kv, head_dim, seq_len, scale,
                              int(kv_int8), None if ks is None else _p(ks),
                              None if vs is None else _p(vs), _p(out))
    return out


def attn_prefill_f32(q16, k, v, n_heads, n_kv, head_dim, n_tok, start_pos, scale,
                     kv_int8=False, ks=None, vs=None) -> np.ndarray:
    q16 = np.ascontiguousarray(q16, dtype=np.uint16)
    k, v = _kv(k, kv_int8), _kv(v, kv_int8)
    ks = None if ks is None else np.ascontiguousarray(ks, dtype=np.float32)
    vs = None if vs is None else np.ascontiguousarray(vs, dtype=np.float32)
    out = np.empty(n_tok * n_heads * head_dim, dtype=np.float32)
    lib().orc_attn_prefill_f32(_p(q16), _p(k), _p(v), n_heads, n_kv, head_dim, n_tok, start_pos,
                               scale, int(kv_int8), None if ks is None else _p(ks),
                               None if vs is None else _p(vs), _p(out))
    return out


def attn_decode_f64(q16, k, v, n_heads, n_kv, head_dim, seq_len, scale, kv_int8=False,
                    ks=None, vs=None) -> np.ndarray:
    q16 = np.ascontiguousarray(q16, dtype=np.uint16)
    k, v = _kv(k, kv_int8), _kv(v, kv_int8)
    ks = None if ks is None else np.ascontiguousarray(ks, dtype=np.float32)
    vs = None if vs is None else np.ascontiguousarray(vs, dtype=np.float32)
    out = np.empty(n_heads * head_dim, dtype=np.float64)
    lib().orc_attn_decode_f64(_p(q16), _p(k), _p(v), n_heads, n_kv, head_dim, seq_len, scale,
                              int(kv_int8), None if ks is None else _p(ks),
                              None if vs is None else _p(vs), _p(out))
    return out


def f16_bits(a: np.ndarray) -> np.ndarray:
    return np.asarray(a, dtype=np.float16).view(np.uint16)


def bits_f16(b: np.ndarray) -> np.ndarray:
    return np.asarray(b, dtype=np.uint16).view(np.float16)


def bits_bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32)
