"""Python bindings of the MI355X Q4_K weight-path library.

Two layers over ``lib/libreflex_infer_hip.so`` (built by ``make`` in the
package directory):

* ``rxq4.capi``: the C ABI of ``include/rxq4.h`` (plain pointers and sizes);
* ``rxq4.api``: the reflex::infer C++ API of ``include/reflex/infer.h`` called
  through its exported symbols with ctypes mirrors of the argument structs
  (reference include/reflex/infer.h:96-238), exactly as a C++ caller would.

Torch is used for device memory and streams only.  Nothing here has a CPU
fallback: if the library is missing, :func:`load` raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "lib", "libreflex_infer_hip.so")

# reflex::infer::Status values (reference include/reflex/infer.h:16-23).
SUCCESS = 0
UNSUPPORTED_DEVICE = 1
UNSUPPORTED_MODEL = 2
UNSUPPORTED_QUANT_FORMAT = 3
INVALID_ARGUMENT = 4
NOT_IMPLEMENTED = 5
STATUS_NAMES = {
    0: "Success",
    1: "UnsupportedDevice",
    2: "UnsupportedModel",
    3: "UnsupportedQuantFormat",
    4: "InvalidArgument",
    5: "NotImplemented",
}

GGML_TYPE_Q4_K = 12
QK_K = 256
BLOCK_BYTES = 144
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2

_lib = None


class RxQ4Error(RuntimeError):
    def __init__(self, status: int, what: str):
        super().__init__(f"{what}: {STATUS_NAMES.get(status, status)}")
        self.status = status


def load() -> ctypes.CDLL:
    """Load the HIP library (once).  Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RxQ4Error(NOT_IMPLEMENTED,
                            f"{LIB_PATH} is missing; build it with __graft_entry__.build()")
        _lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        from . import capi as _capi
        _capi._bind(_lib)
    return _lib


def row_bytes(K: int) -> int:
    return (K // QK_K) * BLOCK_BYTES
