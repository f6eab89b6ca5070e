"""ctypes binding of the CPU oracle (oracle.c).

TEST INFRASTRUCTURE ONLY: the parity checker for tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg.  Never imported by the product library.
All functions take and return numpy arrays (float32, or uint16 holding binary16
bit patterns) and work on copies unless named *_inplace.
"""
from __future__ import annotations

import ctypes
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float

_SIGS = {
    "or_f32_to_f16_n": ([_p, _p, _i64], None),
    "or_f16_to_f32_n": ([_p, _p, _i64], None),
    "or_rmsnorm_f32": ([_p, _p, _p, _i, _i, _f], None),
    "or_rmsnorm_f16": ([_p, _p, _p, _i, _i, _f], None),
    "or_add_rmsnorm_f32": ([_p, _p, _p, _p, _i, _i, _f], None),
    "or_add_rmsnorm_f16": ([_p, _p, _p, _p, _i, _i, _f], None),
    "or_add_f32": ([_p, _p, _i64], None),
    "or_add_f16": ([_p, _p, _i64], None),
    "or_rope_inv_freq": ([_i, _i, _f], ctypes.c_float),
    "or_rope_cos_sin": ([_i, _i, _i, _f, _p, _p], None),
    "or_rope_f32": ([_p, _i, _i, _i, _i64, _p, _i, _f, _i], None),
    "or_rope_f16": ([_p, _i, _i, _i, _i64, _p, _i, _f, _i], None),
    "or_swiglu_f32": ([_p, _p, _p, _i64], None),
    "or_swiglu_f16": ([_p, _p, _p, _i64], None),
    "or_softmax_f32": ([_p, _p, _i, _i], None),
    "or_softmax_f16": ([_p, _p, _i, _i], None),
    "or_softmax_reftest_cpu": ([_p, _p, _i, _i], None),
    "or_reftest_softmax_inputs": ([_p, _i64, ctypes.c_uint], None),
    "or_embed_f32": ([_p, _p, _i, _i, _i, _p], None),
    "or_embed_f16": ([_p, _p, _i, _i, _i, _p], None),
    "or_kv_append_f32": ([_p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i], None),
    "or_kv_append_f16": ([_p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i], None),
    "or_paged_kv_append_f16": ([_p, _p, _p, _i, _p, _p, _p, _i, _i, _i, _i, _i], None),
    "or_attention_f32": ([_p, _p, _p, _p, _i, _i, _i, _i, _i, _i64, _i64, _i64, _i], None),
    "or_attention_f16": ([_p, _p, _p, _p, _i, _i, _i, _i, _i, _i64, _i64, _i64, _i], None),
    "or_attention_reftest_cpu": ([_p, _p, _p, _p, _i, _i, _i], None),
    "or_reftest_attention_inputs": ([_p, _p, _p, _i64, ctypes.c_uint], None),
    "or_matmul_f16": ([_p, _p, _p, _i, _i, _i], None),
    "or_argmax_f32": ([_p, _i, _i, _p], None),
    "or_fp8_encode_ref": ([_f, _i], ctypes.c_uint8),
    "or_fp8_decode_ref": ([ctypes.c_uint8, _i], ctypes.c_float),
    "or_fp8_encode_ocp": ([_f, _i], ctypes.c_uint8),
    "or_fp8_decode_ocp": ([ctypes.c_uint8, _i], ctypes.c_float),
    "or_fp8_num_scales": ([_i, _i, _i, _i], ctypes.c_int),
    "or_fp8_scales": ([_p, _i, _i, _i, _i, _i, _i, _p], None),
    "or_fp8_quantize": ([_p, _i, _i, _i, _i, _i, _i, _p, _p], None),
    "or_fp8_dequantize": ([_p, _p, _i, _i, _i, _i, _i, _i, _p], None),
    "or_reftest_fp8_inputs": ([_p, _i64, ctypes.c_uint], None),
    "or_reftest_gemm_inputs": ([_p, _i64, _p, _i64, ctypes.c_uint], None),
    "or_gemm_reftest_cpu": ([_p, _p, _p, _i, _i, _i], None),
    "or_check_recip_division": ([], ctypes.c_longlong),
}

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C {HERE}`")
        h = ctypes.CDLL(str(LIB_PATH))
        for name, (args, res) in _SIGS.items():
            fn = getattr(h, name)
            fn.argtypes = args
            fn.restype = res
        _lib = h
    return _lib


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _u16(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint16)


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


# ---- binary16 codec -------------------------------------------------------------
def f32_to_f16(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_f16_n(_ptr(x), _ptr(out), x.size)
    return out


def f16_to_f32(h) -> np.ndarray:
    h = _u16(h)
    out = np.empty(h.shape, np.float32)
    lib().or_f16_to_f32_n(_ptr(h), _ptr(out), h.size)
    return out


# ---- ops --------------------------------------------------------------------------
def rmsnorm(x, w, eps: float, f16: bool = False) -> np.ndarray:
    conv = _u16 if f16 else _f32
    x, w = conv(x), conv(w)
    rows, dim = x.shape
    out = np.empty_like(x)
    fn = lib().or_rmsnorm_f16 if f16 else lib().or_rmsnorm_f32
    fn(_ptr(x), _ptr(w), _ptr(out), rows, dim, eps)
    return out


def add_rmsnorm(x, d, w, eps: float, f16: bool = False):
    """Returns (x_updated, out)."""
    conv = _u16 if f16 else _f32
    x, d, w = conv(x).copy(), conv(d), conv(w)
    rows, dim = x.shape
    out = np.empty_like(x)
    fn = lib().or_add_rmsnorm_f16 if f16 else lib().or_add_rmsnorm_f32
    fn(_ptr(x), _ptr(d), _ptr(w), _ptr(out), rows, dim, eps)
    return x, out


def add(x, d, f16: bool = False) -> np.ndarray:
    conv = _u16 if f16 else _f32
    x, d = conv(x).copy(), conv(d)
    fn = lib().or_add_f16 if f16 else lib().or_add_f32
    fn(_ptr(x), _ptr(d), x.size)
    return x


def rope_inv_freq(pair: int, head_dim: int, theta: float) -> float:
    return lib().or_rope_inv_freq(pair, head_dim, theta)


def rope_cos_sin(pos: int, pair: int, head_dim: int, theta: float):
    c, s = ctypes.c_float(), ctypes.c_float()
    lib().or_rope_cos_sin(pos, pair, head_dim, theta, ctypes.byref(c), ctypes.byref(s))
    return c.value, s.value


def rope(x, n_heads: int, head_dim: int, theta: float, pairing: int = 0, positions=None,
         pos_offset: int = 0, f16: bool = False) -> np.ndarray:
    """x: [n_tokens, row_stride] (row_stride >= n_heads*head_dim); returns a rotated copy."""
    conv = _u16 if f16 else _f32
    x = conv(x).copy()
    n_tokens, row_stride = x.shape
    pos = None if positions is None else _i32(positions)
    fn = lib().or_rope_f16 if f16 else lib().or_rope_f32
    fn(_ptr(x), n_tokens, n_heads, head_dim, row_stride, _ptr(pos), pos_offset, theta, pairing)
    return x


def swiglu(g, u, f16: bool = False) -> np.ndarray:
    conv = _u16 if f16 else _f32
    g, u = conv(g), conv(u)
    out = np.empty_like(g)
    fn = lib().or_swiglu_f16 if f16 else lib().or_swiglu_f32
    fn(_ptr(g), _ptr(u), _ptr(out), g.size)
    return out


def softmax(x, f16: bool = False) -> np.ndarray:
    conv = _u16 if f16 else _f32
    x = conv(x)
    rows, cols = x.shape
    out = np.empty_like(x)
    fn = lib().or_softmax_f16 if f16 else lib().or_softmax_f32
    fn(_ptr(x), _ptr(out), rows, cols)
    return out


def softmax_reftest_cpu(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().or_softmax_reftest_cpu(_ptr(x), _ptr(out), x.shape[0], x.shape[1])
    return out


def reftest_softmax_inputs(rows: int, cols: int, seed: int = 7) -> np.ndarray:
    out = np.empty((rows, cols), np.float32)
    lib().or_reftest_softmax_inputs(_ptr(out), out.size, seed)
    return out


def embed(table, ids, f16: bool = False) -> np.ndarray:
    conv = _u16 if f16 else _f32
    table, ids = conv(table), _i32(ids)
    vocab, dim = table.shape
    out = np.empty((ids.size, dim), table.dtype)
    fn = lib().or_embed_f16 if f16 else lib().or_embed_f32
    fn(_ptr(table), _ptr(ids), ids.size, vocab, dim, _ptr(out))
    return out


def kv_append_inplace(k_cache, v_cache, k_new, v_new, layer: int, pos: int, f16: bool = False):
    """k_cache/v_cache: [n_layers, max_seq, n_kv_heads, head_dim]; k_new/v_new: [T, n_kv_heads, head_dim]."""
    conv = _u16 if f16 else _f32
    k_new, v_new = conv(k_new), conv(v_new)
    n_layers, max_seq, hkv, hd = k_cache.shape
    fn = lib().or_kv_append_f16 if f16 else lib().or_kv_append_f32
    fn(_ptr(k_cache), _ptr(v_cache), _ptr(k_new), _ptr(v_new), layer, pos, k_new.shape[0], hkv, hd,
       max_seq, n_layers)


def paged_kv_append_inplace(k_pool, v_pool, block_offset, slots, k_new, v_new, layer: int,
                            n_layers: int, n_kv_heads: int, head_dim: int):
    """k_pool/v_pool: flat uint16 host pools; block_offset[b] = element offset of block b."""
    block_offset = np.ascontiguousarray(block_offset, np.int64)
    slots = _i32(slots)
    k_new, v_new = _u16(k_new), _u16(v_new)
    lib().or_paged_kv_append_f16(_ptr(k_pool), _ptr(v_pool), _ptr(block_offset), block_offset.size,
                                 _ptr(slots), _ptr(k_new), _ptr(v_new), slots.size, layer,
                                 n_layers, n_kv_heads, head_dim)


def attention(q, k, v, n_heads: int, n_kv_heads: int, causal: bool, f16: bool = False) -> np.ndarray:
    """q: [q_len, n_heads, d]; k, v: [kv_len, n_kv_heads, d] (contiguous).  The
    q_len queries are the last q_len positions of the kv_len keys."""
    conv = _u16 if f16 else _f32
    q, k, v = conv(q), conv(k), conv(v)
    q_len, kv_len, d = q.shape[0], k.shape[0], q.shape[-1]
    q2 = q.reshape(q_len, n_heads * d)
    out = np.zeros_like(q2)
    fn = lib().or_attention_f16 if f16 else lib().or_attention_f32
    fn(_ptr(q2), _ptr(k), _ptr(v), _ptr(out), q_len, kv_len, n_heads, n_kv_heads, d,
       n_heads * d, n_kv_heads * d, n_heads * d, int(causal))
    return out.reshape(q.shape)


def attention_reftest_cpu(q, k, v, n_heads: int) -> np.ndarray:
    """tests/test_attention.cu:22-56 (fp32 loop, MHA, no mask)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.zeros_like(q)
    lib().or_attention_reftest_cpu(_ptr(q), _ptr(k), _ptr(v), _ptr(out), q.shape[0], n_heads,
                                   q.shape[-1])
    return out


def reftest_attention_inputs(seq_len: int, n_heads: int, head_dim: int, seed: int = 99):
    n = seq_len * n_heads * head_dim
    q, k, v = (np.empty((seq_len, n_heads, head_dim), np.float32) for _ in range(3))
    lib().or_reftest_attention_inputs(_ptr(q), _ptr(k), _ptr(v), n, seed)
    return q, k, v


def matmul(x, w) -> np.ndarray:
    """y = x W^T for binary16 x [M, K], w [N, K] -> binary16 [M, N]."""
    x, w = _u16(x), _u16(w)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), np.uint16)
    lib().or_matmul_f16(_ptr(x), _ptr(w), _ptr(y), M, N, K)
    return y


def argmax(x) -> np.ndarray:
    x = _f32(x)
    x2 = x.reshape(-1, x.shape[-1])
    out = np.empty(x2.shape[0], np.int32)
    lib().or_argmax_f32(_ptr(x2), x2.shape[0], x2.shape[1], _ptr(out))
    return out.reshape(x.shape[:-1])


# ---- FP8 codec (fmt 0 = E4M3, 1 = E5M2; mode 0 = reference, 1 = OCP) -------------------
def fp8_encode(v: float, fmt: int, mode: int) -> int:
    return (lib().or_fp8_encode_ocp if mode else lib().or_fp8_encode_ref)(float(v), fmt)


def fp8_decode(q: int, fmt: int, mode: int) -> float:
    return (lib().or_fp8_decode_ocp if mode else lib().or_fp8_decode_ref)(int(q), fmt)


def fp8_num_scales(rows, cols, gran, group_size) -> int:
    return lib().or_fp8_num_scales(rows, cols, gran, group_size)


def fp8_quantize(x, fmt: int, gran: int, group_size: int, mode: int):
    """x: binary16 [rows, cols] -> (codes uint8 [rows, cols], scales float32)."""
    x = _u16(x)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.uint8)
    sc = np.empty(fp8_num_scales(rows, cols, gran, group_size), np.float32)
    lib().or_fp8_quantize(_ptr(x), rows, cols, fmt, gran, group_size, mode, _ptr(q), _ptr(sc))
    return q, sc


def fp8_dequantize(q, scales, fmt: int, gran: int, group_size: int, mode: int) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint8)
    scales = _f32(scales)
    rows, cols = q.shape
    out = np.empty((rows, cols), np.uint16)
    lib().or_fp8_dequantize(_ptr(q), _ptr(scales), rows, cols, fmt, gran, group_size, mode, _ptr(out))
    return out


def reftest_fp8_inputs(rows: int, cols: int, seed: int = 1) -> np.ndarray:
    out = np.empty((rows, cols), np.float32)
    lib().or_reftest_fp8_inputs(_ptr(out), out.size, seed)
    return out


def reftest_gemm_inputs(M: int, N: int, K: int, seed: int = 7):
    """quantlib_src/tests/test_gemm.cu:38-52: (A [M, K], W [N, K]) fp32, before rounding."""
    a = np.empty((M, K), np.float32)
    w = np.empty((N, K), np.float32)
    lib().or_reftest_gemm_inputs(_ptr(a), a.size, _ptr(w), w.size, seed)
    return a, w


def gemm_reftest_cpu(a, w) -> np.ndarray:
    """quantlib_src/tests/test_gemm.cu:17-27 on binary16 A [M, K], W [N, K]: fp32 C [M, N]."""
    a, w = _u16(a), _u16(w)
    M, K = a.shape
    N = w.shape[0]
    c = np.empty((M, N), np.float32)
    lib().or_gemm_reftest_cpu(_ptr(a), _ptr(w), _ptr(c), M, N, K)
    return c


def check_recip_division() -> int:
    """Mismatches of the reciprocal-and-correction division against fp32 division over
    one binade of divisors and every FP8 mantissa (0 expected)."""
    return int(lib().or_check_recip_division())
