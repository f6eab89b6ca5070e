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
    "ql_rope_paged_kv_append_f16": [_p, _p, _p, _i, _i, _i, _i, _i64, _i64, _i64, _p, _i, _f, _i,
                                    _p, _p, _i, _p, _i, _i, _p],
    "ql_rope_q_paged_kv_append_f16": [_p, _p, _p, _i, _i, _i, _i, _i64, _i64, _i64, _p, _i, _f, _i,
                                      _p, _p, _i, _p, _i, _i, _p],
    "ql_rope_kv_append_f16": [_p, _p, _p, _i, _i, _i, _i, _i64, _i64, _i64, _p, _i, _f, _i, _p, _p,
                              _i, _i, _i, _i, _p],
    "ql_rope_kv_append_f32": [_p, _p, _p, _i, _i, _i, _i, _i64, _i64, _i64, _p, _i, _f, _i, _p, _p,
                              _i, _i, _i, _i, _p],
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
    "ql_f32_to_f16": [_p, _p, _i64, _p],
    "ql_flash_attention_f16": [_p, _p, _p, _p, _i, _i, _i, _i, _i, _p],
    "ql_attention_f16": [_p, _p, _p, _p, _i, _i, _i, _i, _i, _i64, _i64, _i64, _i, _p],
    "ql_decode_attention_workspace_size": [_i, _i, _i, _i, _p],
    "ql_decode_attention_f16": [_p, _p, _p, _p, _i, _i, _i, _i, _i64, _p, ctypes.c_size_t, _p],
    "ql_paged_attention_f16": [_p, _p, _i64, _i64, _i, _i, _p, _p, _i, _p, _i, _p, _p, _i, _i, _i,
                               _i, _i, _i, _i, _p],
    "ql_paged_decode_workspace_size": [_i, _i, _i, _i, _i, _p],
    "ql_batcher_create": [_i, _i, _i, _p],
    "ql_batcher_create_on_stack": [_p, _p, _i, _i, _i, _p],
    "ql_batcher_destroy": [_p],
    "ql_batcher_add_request": [_p, _i, _p, _i, _i],
    "ql_batcher_plan": [_p, _p],
    "ql_batcher_commit": [_p, _p, _i],
    "ql_batcher_stats": [_p, _p],
    "ql_batcher_pop_finished": [_p, _p, _p, _i, _p],
    "ql_argmax_f32": [_p, _i, _i, _i64, _p, _p],
    "ql_argmax_f16": [_p, _i, _i, _i64, _p, _p],
    "ql_gemm_f16": [_p, _p, _p, _i, _i, _i, _p],
    "ql_gemm_tune_f16": [_i, _i, _i, _p],
    "ql_engine_tune": [_p, _i, _p],
    "ql_fp8_num_scales": [_i, _i, _i, _i, _p],
    "ql_fp8_scales": [_p, _i, _i, _i, _i, _i, _i, _p, _p],
    "ql_fp8_quantize": [_p, _i, _i, _i, _i, _i, _i, _p, _p, _p],
    "ql_fp8_dequantize": [_p, _p, _i, _i, _i, _i, _i, _i, _p, _p],
    "ql_fp8_gemm_workspace_size": [_i, _i, _i, _i, _i, _p],
    "ql_fp8_gemm_f16": [_p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _p, _p, ctypes.c_size_t, _p],
    "ql_fp8_count_ref_special": [_p, ctypes.c_size_t, _i, _p, _p],
    "ql_engine_create": [_p, _i, _i, _i, _p],
    "ql_engine_destroy": [_p],
    "ql_engine_layer_f16": [_p, _p, _i, _p, _p, _p, _p, _p],
    "ql_engine_create_fp8": [_p, _i, _i, _i, _i, _i, _p],
    "ql_graph_begin": [_p],
    "ql_graph_end": [_p, _p],
    "ql_graph_launch": [_p, _p],
    "ql_graph_destroy": [_p],
    "ql_engine_layer_fp8": [_p, _p, _i, _p, _p, _p, _p, _p],
    "ql_engine_logits_f16": [_p, _p, _p, _p, _p, _i, _p, _i, _i, _p, _p, _p],
    "ql_paged_decode_attention_f16": [_p, _p, _i64, _i64, _i, _p, _i, _p, _i, _p, _p, _i, _i, _i,
                                      _i, _i, _i, _p, ctypes.c_size_t, _p],
    "ql_paged_decode_attention_f16_noalloc": [_p, _p, _i64, _i64, _i, _p, _i, _p, _i, _p, _p, _i,
                                              _i, _i, _i, _i, _i, _p],
}

DECODE_SCRATCH_BYTES = 8 << 20   # QL_DECODE_SCRATCH_BYTES

HIP_SUCCESS = 0
HIP_ERROR_INVALID_VALUE = 1
FP8_E4M3, FP8_E5M2 = 0, 1
FP8_MODE_REFERENCE, FP8_MODE_OCP, FP8_MODE_REFERENCE_CLEAN = 0, 1, 2
QUANT_PER_TENSOR, QUANT_PER_CHANNEL, QUANT_PER_GROUP = 0, 1, 2


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


# ---- HIP runtime plumbing -------------------------------------------------------------
# Device memory, a stream and events come from the same libamdhip64 the library
# links against (/opt/rocm).  A second HIP runtime in the process (e.g. the one
# bundled with a framework wheel, loaded under another file name) must not be
# mixed in: two runtimes on one device do not share allocations or streams.
_hiprt = None
_stream = None

H2D, D2H, D2D = 1, 2, 3


def hip() -> ctypes.CDLL:
    """libamdhip64 as loaded by libquantlib_amd.so (same runtime instance)."""
    global _hiprt
    if _hiprt is None:
        lib()
        h = ctypes.CDLL("libamdhip64.so.7")
        sig = {
            "hipMalloc": [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t],
            "hipFree": [_p],
            "hipMemcpy": [_p, _p, ctypes.c_size_t, ctypes.c_int],
            "hipMemset": [_p, ctypes.c_int, ctypes.c_size_t],
            "hipStreamCreate": [ctypes.POINTER(ctypes.c_void_p)],
            "hipStreamSynchronize": [_p],
            "hipDeviceSynchronize": [],
            "hipEventCreate": [ctypes.POINTER(ctypes.c_void_p)],
            "hipEventDestroy": [_p],
            "hipEventRecord": [_p, _p],
            "hipEventSynchronize": [_p],
            "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), _p, _p],
            "hipGetDeviceCount": [ctypes.POINTER(ctypes.c_int)],
            "hipSetDevice": [ctypes.c_int],
        }
        for name, args in sig.items():
            f = getattr(h, name)
            f.argtypes = args
            f.restype = ctypes.c_int
        _hiprt = h
    return _hiprt


def hip_check(rc: int, what: str) -> None:
    if rc != HIP_SUCCESS:
        raise QLError(what, rc)


def device_count() -> int:
    n = ctypes.c_int(0)
    rc = hip().hipGetDeviceCount(ctypes.byref(n))
    return n.value if rc == HIP_SUCCESS else 0


def stream() -> int:
    """The library-wide work stream (created once, default priority)."""
    global _stream
    if _stream is None:
        hip_check(hip().hipSetDevice(0), "hipSetDevice")
        s = ctypes.c_void_p()
        hip_check(hip().hipStreamCreate(ctypes.byref(s)), "hipStreamCreate")
        _stream = s.value
    return _stream


def synchronize() -> None:
    hip_check(hip().hipStreamSynchronize(stream()), "hipStreamSynchronize")


class DeviceArray:
    """A device allocation (or a window of one) with a numpy dtype and shape."""

    def __init__(self, shape, dtype, _owner=None, _ptr=None):
        import numpy as np
        self.dtype = np.dtype(dtype)
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.size = int(np.prod(self.shape)) if self.shape else 1
        self.nbytes = self.size * self.dtype.itemsize
        self._owner = _owner
        if _ptr is None:
            p = ctypes.c_void_p()
            hip_check(hip().hipMalloc(ctypes.byref(p), max(self.nbytes, 1)), "hipMalloc")
            self.ptr = p.value
            self._owns = True
        else:
            self.ptr = _ptr
            self._owns = False

    def data_ptr(self) -> int:
        return self.ptr

    def window(self, start: int, count: int, shape=None) -> "DeviceArray":
        """Elements [start, start+count) as a new array sharing this memory."""
        assert 0 <= start and start + count <= self.size
        owner = self if self._owns else self._owner
        return DeviceArray(shape or (count,), self.dtype, _owner=owner,
                           _ptr=self.ptr + start * self.dtype.itemsize)

    def fill_bytes(self, byte: int) -> "DeviceArray":
        hip_check(hip().hipMemset(self.ptr, byte, self.nbytes), "hipMemset")
        return self

    def upload(self, a) -> "DeviceArray":
        import numpy as np
        a = np.ascontiguousarray(a)
        assert a.nbytes == self.nbytes, (a.nbytes, self.nbytes)
        synchronize()
        hip_check(hip().hipMemcpy(self.ptr, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")
        return self

    def numpy(self):
        import numpy as np
        out = np.empty(self.shape, self.dtype)
        synchronize()
        hip_check(hip().hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, D2H), "hipMemcpy D2H")
        return out

    @classmethod
    def from_numpy(cls, a) -> "DeviceArray":
        import numpy as np
        a = np.ascontiguousarray(a)
        return cls(a.shape, a.dtype).upload(a)

    def __del__(self):
        if getattr(self, "_owns", False) and _hiprt is not None:
            try:
                _hiprt.hipFree(self.ptr)
            except Exception:  # interpreter shutdown
                pass


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        hip_check(hip().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.ev = e.value

    def record(self, s: int | None = None) -> None:
        hip_check(hip().hipEventRecord(self.ev, stream() if s is None else s), "hipEventRecord")

    def elapsed_ms(self, end: "Event") -> float:
        hip_check(hip().hipEventSynchronize(end.ev), "hipEventSynchronize")
        ms = ctypes.c_float()
        hip_check(hip().hipEventElapsedTime(ctypes.byref(ms), self.ev, end.ev), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        if _hiprt is not None:
            try:
                _hiprt.hipEventDestroy(self.ev)
            except Exception:
                pass


# ---- continuous batching (host only) ---------------------------------------------------
FINISH_LENGTH, FINISH_EOS, FINISH_EVICTED = 0, 1, 2
_i32p = ctypes.POINTER(ctypes.c_int32)


class StepPlan(ctypes.Structure):
    """ql_step_plan (include/quantlib_amd.h)."""
    _fields_ = [("n_seqs", _i), ("n_rows", _i), ("max_q_len", _i), ("max_ctx_len", _i),
                ("max_blocks", _i), ("req_ids", _i32p), ("is_prefill", _i32p),
                ("cu_q_lens", _i32p), ("ctx_lens", _i32p), ("block_tables", _i32p),
                ("token_ids", _i32p), ("positions", _i32p), ("slot_mapping", _i32p),
                ("sample_rows", _i32p)]


class BatcherCounts(ctypes.Structure):
    _fields_ = [("n_active", _i), ("n_pending", _i), ("free_blocks", _i), ("n_finished", _i)]


class Finished(ctypes.Structure):
    _fields_ = [("req_id", _i), ("reason", _i), ("prompt_len", _i), ("n_tokens", _i)]


class Batcher:
    """Thin wrapper of the ql_batcher_* C ABI; plan() returns numpy copies."""

    def __init__(self, n_blocks: int, max_active: int, eos_token: int = 2, stack=None,
                 free_count=None):
        import numpy as np
        self._np = np
        h = ctypes.c_void_p()
        if stack is None:
            call("ql_batcher_create", n_blocks, max_active, eos_token, ctypes.byref(h))
        else:   # borrow an external LIFO stack (numpy int32 array + 1-element count array)
            self._stack, self._count = stack, free_count
            call("ql_batcher_create_on_stack", stack.ctypes.data, free_count.ctypes.data, n_blocks,
                 max_active, eos_token, ctypes.byref(h))
        self.h = h.value

    def close(self):
        if self.h:
            call("ql_batcher_destroy", self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def add(self, req_id: int, prompt, max_gen: int):
        p = self._np.ascontiguousarray(prompt, self._np.int32)
        call("ql_batcher_add_request", self.h, req_id, p.ctypes.data, p.size, max_gen)

    def plan(self) -> dict:
        np = self._np
        pl = StepPlan()
        call("ql_batcher_plan", self.h, ctypes.byref(pl))
        n, r, mb = pl.n_seqs, pl.n_rows, pl.max_blocks

        def arr(ptr, count):
            return np.ctypeslib.as_array(ptr, shape=(count,)).copy() if count else np.zeros(0, np.int32)
        return {"n_seqs": n, "n_rows": r, "max_q_len": pl.max_q_len, "max_ctx_len": pl.max_ctx_len,
                "max_blocks": mb, "req_ids": arr(pl.req_ids, n), "is_prefill": arr(pl.is_prefill, n),
                "cu_q_lens": arr(pl.cu_q_lens, n + 1), "ctx_lens": arr(pl.ctx_lens, n),
                "block_tables": arr(pl.block_tables, n * mb).reshape(n, mb),
                "token_ids": arr(pl.token_ids, r), "positions": arr(pl.positions, r),
                "slot_mapping": arr(pl.slot_mapping, r), "sample_rows": arr(pl.sample_rows, n)}

    def commit(self, sampled):
        s = self._np.ascontiguousarray(sampled, self._np.int32)
        call("ql_batcher_commit", self.h, s.ctypes.data if s.size else None, s.size)

    def counts(self) -> dict:
        c = BatcherCounts()
        call("ql_batcher_stats", self.h, ctypes.byref(c))
        return {"n_active": c.n_active, "n_pending": c.n_pending, "free_blocks": c.free_blocks,
                "n_finished": c.n_finished}

    def pop_finished(self):
        """(req_id, reason, prompt_len, tokens) of the oldest finished request, or None."""
        np = self._np
        ev, got = Finished(), ctypes.c_int(0)
        buf = np.zeros(1 << 16, np.int32)
        call("ql_batcher_pop_finished", self.h, ctypes.byref(ev), buf.ctypes.data, buf.size,
             ctypes.byref(got))
        if not got.value:
            return None
        return ev.req_id, ev.reason, ev.prompt_len, buf[:min(ev.n_tokens, buf.size)].copy()


# ---- decoder-layer engine ----------------------------------------------------------------
class LayerDims(ctypes.Structure):
    """ql_layer_dims (include/quantlib_amd.h)."""
    _fields_ = [("hidden", _i), ("n_heads", _i), ("n_kv_heads", _i), ("head_dim", _i), ("ffn", _i),
                ("rope_theta", _f), ("rms_eps", _f), ("rope_pairing", _i)]


class LayerWeights(ctypes.Structure):
    """ql_layer_weights: device addresses of one layer's fp16 weights."""
    _fields_ = [("attn_norm", _p), ("wqkv", _p), ("wo", _p), ("ffn_norm", _p), ("w_gate", _p),
                ("w_up", _p), ("w_down", _p)]


class FP8Weight(ctypes.Structure):
    """ql_fp8_weight: device addresses of one matrix's FP8 codes and its scales."""
    _fields_ = [("codes", _p), ("scales", _p)]


class LayerWeightsFP8(ctypes.Structure):
    """ql_layer_weights_fp8: one layer's fp16 norms and FP8 matrices."""
    _fields_ = [("attn_norm", _p), ("wqkv", FP8Weight), ("wo", FP8Weight), ("ffn_norm", _p),
                ("w_gate", FP8Weight), ("w_up", FP8Weight), ("w_down", FP8Weight), ("format", _i),
                ("granularity", _i), ("group_size", _i), ("mode", _i)]


class StepDevice(ctypes.Structure):
    """ql_step_device: a step plan's arrays on the device plus the paged pool."""
    _fields_ = [("n_rows", _i), ("n_seqs", _i), ("max_q_len", _i), ("max_ctx_len", _i),
                ("max_blocks", _i), ("positions", _p), ("slot_mapping", _p), ("cu_q_lens", _p),
                ("ctx_lens", _p), ("block_tables", _p), ("k_blocks", _p), ("v_blocks", _p),
                ("n_blocks", _i), ("n_layers", _i)]
