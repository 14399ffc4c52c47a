"""ctypes binding of include/rxq4_gguf.h: caller-side GGUF ingest.

``GGUFFile(path)`` maps a GGUF file read-only and exposes its metadata and
tensors; ``upload()`` copies the data section to the GPU once and returns the
device alias of every tensor, i.e. what a reflex-infer caller passes as
``weights`` (the mapped host address) and ``weights_device`` (the device
copy) in GemvQuantArgs and friends (reference include/reflex/infer.h:94-95).
The reference parses no GGUF itself (docs/library-architecture.md:60); this
is the caller side of that contract.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np
import torch

from . import NOT_IMPLEMENTED, PKG_DIR, SUCCESS, RxQ4Error, load

c_void_p, c_int, c_int64, c_uint64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64
c_char_p = ctypes.c_char_p

# GGUF metadata value types (include/rxq4_gguf.h RXQ4_GGUF_*).
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = \
    range(13)
_NP = {UINT8: np.uint8, INT8: np.int8, UINT16: np.uint16, INT16: np.int16, UINT32: np.uint32,
       INT32: np.int32, FLOAT32: np.float32, BOOL: np.bool_, UINT64: np.uint64, INT64: np.int64,
       FLOAT64: np.float64}
_INTS = {UINT8, INT8, UINT16, INT16, UINT32, INT32, UINT64, INT64}


class _TensorInfo(ctypes.Structure):
    _fields_ = [("name", c_char_p), ("ggml_type", c_int), ("n_dims", c_int),
                ("ne", c_int64 * 4), ("offset", c_uint64), ("nbytes", c_uint64),
                ("host", c_void_p)]


SIGNATURES = {
    "rxq4_gguf_open": (c_int, [c_char_p, ctypes.POINTER(c_void_p)]),
    "rxq4_gguf_close": (None, [c_void_p]),
    "rxq4_gguf_version": (ctypes.c_uint32, [c_void_p]),
    "rxq4_gguf_alignment": (ctypes.c_uint32, [c_void_p]),
    "rxq4_gguf_n_tensors": (c_int64, [c_void_p]),
    "rxq4_gguf_n_kv": (c_int64, [c_void_p]),
    "rxq4_gguf_data": (c_void_p, [c_void_p]),
    "rxq4_gguf_data_bytes": (c_uint64, [c_void_p]),
    "rxq4_gguf_tensor_info": (c_int, [c_void_p, c_int64, ctypes.POINTER(_TensorInfo)]),
    "rxq4_gguf_find_tensor": (c_int64, [c_void_p, c_char_p]),
    "rxq4_gguf_find_kv": (c_int64, [c_void_p, c_char_p]),
    "rxq4_gguf_kv_key": (c_int, [c_void_p, c_int64, ctypes.POINTER(c_char_p),
                                 ctypes.POINTER(c_int)]),
    "rxq4_gguf_kv_int": (c_int, [c_void_p, c_int64, ctypes.POINTER(c_int64)]),
    "rxq4_gguf_kv_float": (c_int, [c_void_p, c_int64, ctypes.POINTER(ctypes.c_double)]),
    "rxq4_gguf_kv_str": (c_int, [c_void_p, c_int64, ctypes.POINTER(c_void_p),
                                 ctypes.POINTER(c_uint64)]),
    "rxq4_gguf_kv_array": (c_int, [c_void_p, c_int64, ctypes.POINTER(c_int),
                                   ctypes.POINTER(c_uint64), ctypes.POINTER(c_void_p)]),
    "rxq4_gguf_kv_array_strs": (c_int, [c_void_p, c_int64, c_uint64, c_uint64,
                                        ctypes.POINTER(c_void_p), ctypes.POINTER(c_uint64)]),
    "rxq4_gguf_upload": (c_int, [c_void_p, c_void_p, c_uint64, c_void_p]),
    "rxq4_ggml_block_elems": (c_int, [c_int]),
    "rxq4_ggml_block_bytes": (c_int, [c_int]),
}

_bound = None


GGUF_LIB_PATH = os.path.join(PKG_DIR, "lib", "librxq4_gguf.so")


def lib() -> ctypes.CDLL:
    """librxq4_gguf.so (caller-side ingest, a library of its own: the
    drop-in kernel library parses no GGUF), bound once."""
    global _bound
    if _bound is None:
        load()  # the kernel library first: ingest reports errors through it
        if not os.path.exists(GGUF_LIB_PATH):
            raise RxQ4Error(NOT_IMPLEMENTED, f"{GGUF_LIB_PATH} is missing; build it with "
                            "__graft_entry__.build()")
        L = ctypes.CDLL(GGUF_LIB_PATH)
        L.rxq4_last_error.restype = c_char_p
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _bound = L
    return _bound


def _check(status: int, what: str) -> None:
    if status != SUCCESS:
        err = lib().rxq4_last_error()
        raise RxQ4Error(status, f"{what}: {err.decode() if err else ''}")


def block_geometry(ggml_type: int) -> tuple[int, int]:
    """(elements, bytes) per block of a GGML type; (0, 0) if unknown."""
    return lib().rxq4_ggml_block_elems(ggml_type), lib().rxq4_ggml_block_bytes(ggml_type)


@dataclass(frozen=True)
class Tensor:
    name: str
    ggml_type: int
    shape: tuple  # GGUF order: (ne0 = row length, ne1 = rows, ...)
    offset: int   # from the start of the data section
    nbytes: int
    host: int     # mapped address

    @property
    def rows(self) -> int:
        n = 1
        for d in self.shape[1:]:
            n *= d
        return n

    @property
    def row_length(self) -> int:
        return self.shape[0]


class GGUFFile:
    """A read-only mapped GGUF file (versions 2 and 3)."""

    def __init__(self, path: str):
        h = c_void_p()
        _check(lib().rxq4_gguf_open(str(path).encode(), ctypes.byref(h)), f"open {path}")
        self._h = h
        L = lib()
        self.version = int(L.rxq4_gguf_version(h))
        self.alignment = int(L.rxq4_gguf_alignment(h))
        self.data_bytes = int(L.rxq4_gguf_data_bytes(h))
        self.tensors: dict[str, Tensor] = {}
        info = _TensorInfo()
        for i in range(L.rxq4_gguf_n_tensors(h)):
            _check(L.rxq4_gguf_tensor_info(h, i, ctypes.byref(info)), "tensor_info")
            t = Tensor(info.name.decode("utf-8", "replace"), info.ggml_type, tuple(info.ne[:info.n_dims]),
                       int(info.offset), int(info.nbytes), int(info.host or 0))
            self.tensors[t.name] = t
        self.metadata = {self._key(i): self._value(i) for i in range(L.rxq4_gguf_n_kv(h))}

    # -- metadata -------------------------------------------------------------
    def _key(self, i: int) -> str:
        k, t = c_char_p(), c_int()
        _check(lib().rxq4_gguf_kv_key(self._h, i, ctypes.byref(k), ctypes.byref(t)), "kv_key")
        return k.value.decode("utf-8", "replace")

    def _value(self, i: int):
        L, h = lib(), self._h
        k, t = c_char_p(), c_int()
        _check(L.rxq4_gguf_kv_key(h, i, ctypes.byref(k), ctypes.byref(t)), "kv_key")
        t = t.value
        if t in _INTS or t == BOOL:
            v = c_int64()
            _check(L.rxq4_gguf_kv_int(h, i, ctypes.byref(v)), "kv_int")
            return bool(v.value) if t == BOOL else int(v.value)
        if t in (FLOAT32, FLOAT64):
            v = ctypes.c_double()
            _check(L.rxq4_gguf_kv_float(h, i, ctypes.byref(v)), "kv_float")
            return float(v.value)
        if t == STRING:
            p, n = c_void_p(), c_uint64()
            _check(L.rxq4_gguf_kv_str(h, i, ctypes.byref(p), ctypes.byref(n)), "kv_str")
            return ctypes.string_at(p.value, n.value).decode("utf-8", "replace") if n.value else ""
        et, n, p = c_int(), c_uint64(), c_void_p()
        _check(L.rxq4_gguf_kv_array(h, i, ctypes.byref(et), ctypes.byref(n), ctypes.byref(p)),
               "kv_array")
        if et.value == STRING:
            cnt = n.value
            ptrs, lens = (c_void_p * max(cnt, 1))(), (c_uint64 * max(cnt, 1))()
            _check(L.rxq4_gguf_kv_array_strs(h, i, 0, cnt, ptrs, lens), "kv_array_strs")
            return [ctypes.string_at(ptrs[j], lens[j]).decode("utf-8", "replace") if lens[j] else ""
                    for j in range(cnt)]
        dt = np.dtype(_NP[et.value])
        if n.value == 0:
            return np.zeros(0, dt)
        buf = (ctypes.c_uint8 * (n.value * dt.itemsize)).from_address(p.value)
        return np.frombuffer(buf, dtype=dt).copy()

    # -- tensors --------------------------------------------------------------
    def host_array(self, name: str) -> np.ndarray:
        """The tensor's bytes as a read-only uint8 view of the mapping."""
        t = self.tensors[name]
        if t.nbytes == 0:
            return np.zeros(0, np.uint8)
        buf = (ctypes.c_uint8 * t.nbytes).from_address(t.host)
        a = np.frombuffer(buf, dtype=np.uint8)
        a.flags.writeable = False
        return a

    def upload(self, device="cuda", stream=None) -> "DeviceCopy":
        """Copy the data section to the GPU (one allocation) and return it."""
        n = self.data_bytes
        buf = torch.empty(max(n, 256) + 256, dtype=torch.uint8, device=device)
        off = (-buf.data_ptr()) % 256
        view = buf[off:off + n]
        st = stream.cuda_stream if stream is not None else torch.cuda.current_stream(device).cuda_stream
        _check(lib().rxq4_gguf_upload(self._h, buf.data_ptr() + off, n, st), "upload")
        return DeviceCopy(self, buf, view)

    def close(self) -> None:
        if self._h:
            lib().rxq4_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceCopy:
    """The device copy of a file's data section: tensor i at base + offset_i."""

    def __init__(self, f: GGUFFile, storage: torch.Tensor, view: torch.Tensor):
        self.file = f
        self._storage = storage
        self.data = view

    def ptr(self, name: str) -> int:
        """`weights_device` alias of the tensor (device address)."""
        return self.data.data_ptr() + self.file.tensors[name].offset

    def tensor(self, name: str) -> torch.Tensor:
        t = self.file.tensors[name]
        return self.data[t.offset:t.offset + t.nbytes]
