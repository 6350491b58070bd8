"""ctypes binding of libtq.so, the C ABI declared in include/tq.h.

There is no fallback: if the library is missing or cannot be loaded, every
entry point raises.  The library is built in-tree by
``python -c "import __graft_entry__; __graft_entry__.build()"`` (or
``make -C tq-local_amd/csrc``).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("TQ_LIBTQ_PATH", Path(__file__).resolve().parent.parent / "libtq.so"))

TQ_OK = 0
ABI_VERSION = 1

#: every symbol include/tq.h declares, with (restype, argtypes)
_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_SZ = ctypes.c_size_t
SIGNATURES: dict[str, tuple] = {
    "tq_abi_version": (_I, []),
    "tq_status_string": (ctypes.c_char_p, [_I]),
    "tq_quantize_mse": (_I, [_P, _I, _I, _I64, _I, _I64, _I64, _I64, _I, _P, _P, _P, _P, _I64, _I64, _P]),
    "tq_quantize_prod": (_I, [_P, _I, _I, _I64, _I, _I64, _I64, _I64, _I, _P, _P, _P, _P, _P, _P, _P, _P,
                              _I64, _I64, _P]),
    "tq_decode_attention_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I64]),
    "tq_decode_attention": (_I, [_P, _I, _I, _I, _I, _P, _P, _I64, _I64, _P, _P, _P, _P, _P, _P, _I, _I, _I,
                                 _P, _P, _P, _P, _P, _F, _P, _P, _P, _P, _SZ, _P]),
    "tq_decode_attention_noalloc": (_I, [_P, _I, _I, _I, _I, _P, _P, _I64, _I64, _P, _P, _P, _P, _P, _P, _I, _I,
                                         _I, _P, _P, _P, _P, _P, _F, _P, _P, _P, _P]),
    "tq_dequantize_mse": (_I, [_P, _P, _I64, _I64, _I64, _I, _I, _P, _P, _P, _P]),
    "tq_dequantize_prod": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _P, _P, _P, _P, _P]),
    "tq_value_codebook_f16": (_I, [_P, _I, _I, _P]),
    "tq_group_matrix": (_I, [_P, _I, _P, _I, _P]),
    "tq_decode_attention_groups": (_I, [_P, _I, _I, _I, _I, _P, _P, _I64, _I64, _I, _P, _P, _P, _I, _P, _P, _P, _P,
                                        _P, _P, _P, _P, _P, _P, _P, _F, _P, _P, _P, _P, _SZ, _P]),
    "tq_quantize_group": (_I, [_P, _I, _I, _I64, _I, _I64, _I64, _I64, _P, _I, _I, _P, _P, _P, _P, _P, _P, _P,
                               _P, _I64, _I64, _P]),
    "tq_dequantize_group": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I, _P, _I, _I, _P, _P, _P, _I, _P, _P]),
}

_lib: ctypes.CDLL | None = None


class TQError(RuntimeError):
    """A libtq entry point returned a non-zero tq_status."""

    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn} failed with status {status}: {message}")
        self.status = status


def load() -> ctypes.CDLL:
    """Load libtq.so once; raise ImportError with the path if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"libtq.so not found at {LIB_PATH}: the TurboQuant HIP extension is not built "
            "(run __graft_entry__.build() or `make -C tq-local_amd/csrc`)"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    version = lib.tq_abi_version()
    if version != ABI_VERSION:
        raise ImportError(f"libtq ABI version {version} != expected {ABI_VERSION}")
    _lib = lib
    return lib


def check(fn: str, status: int) -> None:
    if status != TQ_OK:
        msg = load().tq_status_string(status).decode()
        raise TQError(fn, status, msg)


def call(fn: str, *args) -> None:
    """Call ``fn`` and raise TQError on a non-zero status."""
    check(fn, getattr(load(), fn)(*args))
