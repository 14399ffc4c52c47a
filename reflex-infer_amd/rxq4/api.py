"""The reflex::infer C++ API (include/reflex/infer.h) called from Python.

The structs below mirror the reference's argument blocks field for field
(reference include/reflex/infer.h:96-187 and 230-238); functions are the
library's exported C++ symbols (Itanium mangling of the reference
declarations), so a call here goes through exactly the code path a C++
caller compiled against the reference header takes: dispatcher, registered
backend or kernel seam, C ABI, HIP kernels.
"""
from __future__ import annotations

import ctypes

from . import load

c_void_p, c_int = ctypes.c_void_p, ctypes.c_int


class GemvQuantArgs(ctypes.Structure):
    _fields_ = [("y", c_void_p), ("weights", c_void_p), ("weights_device", c_void_p),
                ("ggml_type", c_int), ("x", c_void_p), ("M", c_int), ("K", c_int),
                ("stream", c_void_p)]


class GemvQuantAddArgs(ctypes.Structure):
    _fields_ = [("y", c_void_p), ("weights", c_void_p), ("weights_device", c_void_p),
                ("ggml_type", c_int), ("x", c_void_p), ("residual", c_void_p), ("M", c_int),
                ("K", c_int), ("stream", c_void_p)]


class GemvQuantPairArgs(ctypes.Structure):
    _fields_ = [("y0", c_void_p), ("weights0", c_void_p), ("weights0_device", c_void_p),
                ("ggml_type0", c_int), ("M0", c_int),
                ("y1", c_void_p), ("weights1", c_void_p), ("weights1_device", c_void_p),
                ("ggml_type1", c_int), ("M1", c_int),
                ("x", c_void_p), ("K", c_int), ("stream", c_void_p)]


class GemvQuantTripleArgs(ctypes.Structure):
    _fields_ = [("y0", c_void_p), ("weights0", c_void_p), ("weights0_device", c_void_p),
                ("ggml_type0", c_int), ("M0", c_int),
                ("y1", c_void_p), ("weights1", c_void_p), ("weights1_device", c_void_p),
                ("ggml_type1", c_int), ("M1", c_int),
                ("y2", c_void_p), ("weights2", c_void_p), ("weights2_device", c_void_p),
                ("ggml_type2", c_int), ("M2", c_int),
                ("x", c_void_p), ("K", c_int), ("stream", c_void_p)]


class GemmQuantBatchedArgs(ctypes.Structure):
    _fields_ = [("y", c_void_p), ("weights", c_void_p), ("weights_device", c_void_p),
                ("ggml_type", c_int), ("x", c_void_p), ("M", c_int), ("N", c_int),
                ("K", c_int), ("stream", c_void_p)]


class GemvQuantF32Args(ctypes.Structure):
    _fields_ = [("y", c_void_p), ("weights", c_void_p), ("weights_device", c_void_p),
                ("ggml_type", c_int), ("x", c_void_p), ("M", c_int), ("K", c_int),
                ("stream", c_void_p)]


class DequantEmbeddingRowArgs(ctypes.Structure):
    _fields_ = [("dst", c_void_p), ("weights", c_void_p), ("weights_device", c_void_p),
                ("ggml_type", c_int), ("token_id", c_int), ("hidden_dim", c_int),
                ("stream", c_void_p)]


class AttentionDecodeArgs(ctypes.Structure):
    _fields_ = [("output", c_void_p), ("q", c_void_p), ("k_cache", c_void_p),
                ("v_cache", c_void_p), ("n_heads", c_int), ("n_kv_heads", c_int),
                ("head_dim", c_int), ("seq_len", c_int), ("scale", ctypes.c_float),
                ("kv_int8", ctypes.c_bool), ("k_scales", c_void_p), ("v_scales", c_void_p),
                ("stream", c_void_p)]


class AttentionPrefillBatchedArgs(ctypes.Structure):
    _fields_ = [("output", c_void_p), ("q", c_void_p), ("k_cache", c_void_p),
                ("v_cache", c_void_p), ("n_heads", c_int), ("n_kv_heads", c_int),
                ("head_dim", c_int), ("N", c_int), ("start_pos", c_int),
                ("scale", ctypes.c_float), ("kv_int8", ctypes.c_bool), ("k_scales", c_void_p),
                ("v_scales", c_void_p), ("stream", c_void_p)]


Status = ctypes.c_uint8

# Function-pointer types of the plug-in table (reference infer.h:222-228).
GemvQuantFn = ctypes.CFUNCTYPE(Status, ctypes.POINTER(GemvQuantArgs))
GemvQuantAddFn = ctypes.CFUNCTYPE(Status, ctypes.POINTER(GemvQuantAddArgs))
GemvQuantPairFn = ctypes.CFUNCTYPE(Status, ctypes.POINTER(GemvQuantPairArgs))
GemvQuantTripleFn = ctypes.CFUNCTYPE(Status, ctypes.POINTER(GemvQuantTripleArgs))
GemmQuantBatchedFn = ctypes.CFUNCTYPE(Status, ctypes.POINTER(GemmQuantBatchedArgs))
GemvQuantF32Fn = ctypes.CFUNCTYPE(Status, ctypes.POINTER(GemvQuantF32Args))
DequantEmbeddingRowFn = ctypes.CFUNCTYPE(Status, ctypes.POINTER(DequantEmbeddingRowArgs))


class Q4Kernels(ctypes.Structure):
    _fields_ = [("gemv_quant", GemvQuantFn), ("gemv_quant_add", GemvQuantAddFn),
                ("gemv_quant_pair", GemvQuantPairFn), ("gemv_quant_triple", GemvQuantTripleFn),
                ("gemm_quant_batched", GemmQuantBatchedFn), ("gemv_quant_f32", GemvQuantF32Fn),
                ("dequant_embedding_row", DequantEmbeddingRowFn)]


# Exported symbol of each public function (Itanium mangling of the
# declarations in reference include/reflex/infer.h:270-282).
SYMBOLS = {
    "gemv_quant": ("_ZN6reflex5infer10gemv_quantERKNS0_13GemvQuantArgsE", GemvQuantArgs),
    "gemv_quant_add": ("_ZN6reflex5infer14gemv_quant_addERKNS0_16GemvQuantAddArgsE",
                       GemvQuantAddArgs),
    "gemv_quant_pair": ("_ZN6reflex5infer15gemv_quant_pairERKNS0_17GemvQuantPairArgsE",
                        GemvQuantPairArgs),
    "gemv_quant_triple": ("_ZN6reflex5infer17gemv_quant_tripleERKNS0_19GemvQuantTripleArgsE",
                          GemvQuantTripleArgs),
    "gemm_quant_batched": ("_ZN6reflex5infer18gemm_quant_batchedERKNS0_20GemmQuantBatchedArgsE",
                           GemmQuantBatchedArgs),
    "gemv_quant_f32": ("_ZN6reflex5infer14gemv_quant_f32ERKNS0_16GemvQuantF32ArgsE",
                       GemvQuantF32Args),
    "dequant_embedding_row": (
        "_ZN6reflex5infer21dequant_embedding_rowERKNS0_23DequantEmbeddingRowArgsE",
        DequantEmbeddingRowArgs),
    "flash_attention_decode": ("_ZN6reflex5infer22flash_attention_decodeERKNS0_19AttentionDecodeArgsE",
                               AttentionDecodeArgs),
    "flash_attention_prefill_batched": (
        "_ZN6reflex5infer31flash_attention_prefill_batchedERKNS0_27AttentionPrefillBatchedArgsE",
        AttentionPrefillBatchedArgs),
}
REGISTER_SYMBOL = "_ZN6reflex5infer19register_q4_backendERKNS0_9Q4KernelsE"
REGISTERED_SYMBOL = "_ZN6reflex5infer21registered_q4_backendEv"


def _fn(name):
    sym, argt = SYMBOLS[name]
    f = getattr(load(), sym)
    f.restype = Status
    f.argtypes = [ctypes.POINTER(argt)]
    return f


def call(name: str, args) -> int:
    """Call reflex::infer::<name>(args) and return the Status value."""
    return int(_fn(name)(ctypes.byref(args)))


def register_q4_backend(kernels: Q4Kernels) -> None:
    f = getattr(load(), REGISTER_SYMBOL)
    f.restype = None
    f.argtypes = [ctypes.POINTER(Q4Kernels)]
    f(ctypes.byref(kernels))


def registered_q4_backend() -> Q4Kernels:
    f = getattr(load(), REGISTERED_SYMBOL)
    f.restype = Q4Kernels
    f.argtypes = []
    return f()
