"""Shared test helpers: seeded inputs, device transfer, tolerance checks.

Tolerances, |got - want| <= rtol*|want| + atol:
  fp32 RMSNorm / softmax / SwiGLU : rtol 1e-5, atol 2^-126 (fp32 subnormal results)
  fp32 RoPE                        : absolute 1e-6
  binary16 variants                : rtol 2e-3, atol 2^-24 (one binary16 subnormal step)
  gather / KV append               : bit-exact
"""
from __future__ import annotations

import numpy as np

RTOL_F32 = 1e-5
ATOL_F32 = 2.0 ** -126
ATOL_ROPE_F32 = 1e-6
RTOL_F16 = 2e-3
ATOL_F16 = 2.0 ** -24


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def normal(seed: int, shape, sigma: float = 1.0, clip: float | None = None) -> np.ndarray:
    x = rng(seed).standard_normal(size=shape, dtype=np.float32) * np.float32(sigma)
    if clip is not None:
        np.clip(x, -clip, clip, out=x)
    return x


def uniform(seed: int, shape, lo: float, hi: float) -> np.ndarray:
    return rng(seed).uniform(lo, hi, size=shape).astype(np.float32)


def causal_mask_inplace(x: np.ndarray) -> np.ndarray:
    """-inf strictly above the diagonal (column > row)."""
    rows, cols = x.shape
    x[np.triu_indices(rows, k=1, m=cols)] = -np.inf
    return x


def to_f16_bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x.astype(np.float16)).view(np.uint16)


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return h.view(np.float16).astype(np.float32)


def check_close(got: np.ndarray, want: np.ndarray, rtol: float, atol: float, what: str = ""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    nan_g, nan_w = np.isnan(got), np.isnan(want)
    assert np.array_equal(nan_g, nan_w), f"{what}: NaN pattern differs ({nan_g.sum()} vs {nan_w.sum()})"
    g, w = got[~nan_w], want[~nan_w]
    inf_w = np.isinf(w)
    assert np.array_equal(g[inf_w], w[inf_w]), f"{what}: inf mismatch"
    g, w = g[~inf_w], w[~inf_w]
    err = np.abs(g - w)
    bound = rtol * np.abs(w) + atol
    bad = err > bound
    if bad.any():
        i = int(np.argmax(err - bound))
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {g.size} elements outside rtol={rtol} atol={atol}; "
            f"worst got={g[i]!r} want={w[i]!r} err={err[i]:.3e}")
    return float((err / np.maximum(np.abs(w), atol)).max()) if err.size else 0.0


def check_f16(got_bits: np.ndarray, want_bits: np.ndarray, what: str = ""):
    return check_close(f16_bits_to_f32(got_bits), f16_bits_to_f32(want_bits), RTOL_F16, ATOL_F16,
                       what)


def check_abs(got: np.ndarray, want: np.ndarray, atol: float, what: str = ""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    m = float(err.max()) if err.size else 0.0
    assert m <= atol, f"{what}: max abs error {m:.3e} > {atol}"
    return m


# ---- device side: HIP runtime through the library's own binding (no framework) ------
def dev(a: np.ndarray, offset_elems: int = 0):
    """Copy a numpy array to the GPU.  offset_elems > 0 places it that many
    elements into a larger allocation (to exercise unaligned paths)."""
    import quantlib_amd as ql
    a = np.ascontiguousarray(a).reshape(-1)
    if offset_elems:
        buf = ql.DeviceArray((a.size + offset_elems,), a.dtype)
        d = buf.window(offset_elems, a.size)
        d.upload(a)
        return d
    return ql.DeviceArray.from_numpy(a)


def host(t, dtype=None, shape=None) -> np.ndarray:
    a = t.numpy().reshape(-1)
    if dtype is not None:
        a = a.view(dtype)
    if shape is not None:
        a = a.reshape(shape)
    return a


def empty(shape, dtype, fill_bits: int | None = None):
    """Device buffer; fill_bits sets every byte (guard pattern)."""
    import quantlib_amd as ql
    t = ql.DeviceArray((int(np.prod(shape)),), dtype)
    if fill_bits is not None:
        t.fill_bytes(fill_bits)
    return t


def stream() -> int:
    import quantlib_amd as ql
    return ql.stream()


def synchronize() -> None:
    import quantlib_amd as ql
    ql.synchronize()


def ptr(t) -> int:
    return t.ptr


GUARD = 64          # elements of guard band on each side of every output
GUARD_BYTE = 0xA5


class Out:
    """Device output buffer of n elements between two guard bands."""

    def __init__(self, n, dtype, offset=0):
        self.n, self.dtype, self.offset = n, dtype, offset
        self.buf = empty((n + 2 * GUARD + offset,), dtype, fill_bits=GUARD_BYTE)
        self.view = self.buf.window(GUARD + offset, n)

    @property
    def ptr(self):
        return self.view.data_ptr()

    def get(self, shape=None):
        a = host(self.buf)
        g0, g1 = a[:GUARD + self.offset], a[GUARD + self.offset + self.n:]
        for g in (g0, g1):
            assert np.all(g.view(np.uint8) == GUARD_BYTE), "write outside the output region"
        v = a[GUARD + self.offset:GUARD + self.offset + self.n]
        return v.reshape(shape) if shape is not None else v
