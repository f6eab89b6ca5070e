"""ctypes binding of libquantlib_amd.so (the C ABI declared in include/quantlib_amd.h).

Arguments are plain integers: device addresses (e.g. ``tensor.data_ptr()``),
sizes, and a HIP stream handle (``torch.cuda.current_stream().cuda_stream``
or 0).  Every wrapper raises :class:`QLError` when the entry point returns a
HIP error.  Importing this module never falls back to anything: if the shared
library was not built, :func:`lib` raises.
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import re

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "libquantlib_amd.so"
HEADER = HERE.parent / "include" / "quantlib_amd.h"

ROPE_INTERLEAVED = 0
ROPE_HALF = 1
PAGE_SIZE = 16

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float

# name -> argtypes (restype is hipError_t = int unless listed in _RESTYPES)
SIGNATURES = {
    "ql_version": [],
    "ql_rmsnorm_f32": [_p, _p, _p, _i, _i, _f, _p],
    "ql_rmsnorm_f16": [_p, _p, _p, _i, _i, _f, _p],
    "ql_add_rmsnorm_f32": [_p, _p, _p, _p, _i, _i, _f, _p],
    "ql_add_rmsnorm_f16": [_p, _p, _p, _p, _i, _i, _f, _p],
    "ql_add_f32": [_p, _p, _i64, _p],
    "ql_add_f16": [_p, _p, _i64, _p],
    "ql_rope_f32": [_p, _p, _i, _i, _i, _i, _i64, _i64, _p, _i, _f, _i, _p],
    "ql_rope_f16": [_p, _p, _i, _i, _i, _i, _i64, _i64, _p, _i, _f, _i, _p],
    "ql_swiglu_f32": [_p, _p, _p, _i, _i, _p],
    "ql_swiglu_f16": [_p, _p, _p, _i, _i, _p],
    "ql_softmax_f32": [_p, _p, _i, _i, _p],
    "ql_softmax_f16": [_p, _p, _i, _i, _p],
    "ql_embed_f32": [_p, _p, _i, _i, _i, _p, _p],
    "ql_embed_f16": [_p, _p, _i, _i, _i, _p, _p],
    "ql_embed_token_f32": [_p, _i, _i, _p, _p],
    "ql_embed_token_f16": [_p, _i, _i, _p, _p],
    "ql_kv_append_f32": [_p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _p],
    "ql_kv_append_f16": [_p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _p],
    "ql_paged_kv_append_f16": [_p, _p, _i, _p, _p, _p, _i, _i, _i, _i, _i, _p],
    "ql_paged_slot_mapping": [_p, _i, _i, _i, _p],
    "ql_f16_to_f32": [_p, _p, _i64, _p],
}

HIP_SUCCESS = 0
HIP_ERROR_INVALID_VALUE = 1


class QLError(RuntimeError):
    def __init__(self, name: str, code: int):
        super().__init__(f"{name} returned hipError_t {code} ({error_string(code)})")
        self.code = code


_lib = None
_hip = None


def lib() -> ctypes.CDLL:
    """Load the built library (once).  Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `make -C {HERE}` "
                "(or __graft_entry__.build()); there is no fallback path")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, args in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        _lib = handle
    return _lib


def error_string(code: int) -> str:
    global _hip
    try:
        if _hip is None:
            _hip = ctypes.CDLL("libamdhip64.so")
            _hip.hipGetErrorString.restype = ctypes.c_char_p
            _hip.hipGetErrorString.argtypes = [ctypes.c_int]
        return _hip.hipGetErrorString(code).decode()
    except OSError:
        return "unknown"


def call(name: str, *args) -> None:
    """Call entry point `name`; raise QLError on a non-zero hipError_t."""
    rc = getattr(lib(), name)(*args)
    if rc != HIP_SUCCESS:
        raise QLError(name, rc)


def raw(name: str, *args) -> int:
    """Call entry point `name` and return its hipError_t."""
    return getattr(lib(), name)(*args)


def declared_symbols(header: pathlib.Path = HEADER) -> list[str]:
    """Function names declared in a C header (the C ABI under test)."""
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(ql_[a-z0-9_]+)\s*\(", text)))


def version() -> int:
    return lib().ql_version()
