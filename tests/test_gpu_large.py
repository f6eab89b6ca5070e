"""GPU: problems of more than 2^31 elements (64-bit element indexing).

The reference's launchers size their grids with int products (rows * ffn_dim
in kernels/feedforward.cu:30); the C ABI takes int row and column counts but
indexes with 64-bit offsets, so a tensor may exceed 2^31 elements.  Each test
fills a >4 GiB device tensor by tiling a small seeded block (a 64-row tile
uploaded once, then doubled with device copies, so row r holds tile row
r % 64), runs the entry point once, and compares windows of the output --
the first rows, the rows around element 2^31 and the last rows -- with the
oracle's result for the same tile rows, at the op's tolerance."""
import numpy as np
import pytest

import oracle as orc
import quantlib_amd as ql
from helpers import (check_f16, dev, normal, stream, synchronize, to_f16_bits, uniform)

pytestmark = pytest.mark.gpu

TILE = 64
E31 = 2 ** 31


def _tiled(tile: np.ndarray, rows: int) -> "ql.DeviceArray":
    """Device [rows, tile.shape[1]] whose row r is tile row r % TILE."""
    cols = tile.shape[1]
    buf = ql.DeviceArray((rows * cols,), tile.dtype)
    buf.window(0, TILE * cols).upload(tile)
    filled = TILE
    item = tile.dtype.itemsize
    while filled < rows:
        n = min(filled, rows - filled)
        ql.hip_check(ql.hip().hipMemcpy(buf.ptr + filled * cols * item, buf.ptr, n * cols * item,
                                        ql.D2D), "hipMemcpy D2D")
        filled += n
    return buf


def _windows(rows: int, cols: int):
    b = E31 // cols
    return [(0, 8), (b - 5, b + 5), (rows - 8, rows)]


def _rows(buf, r0: int, r1: int, cols: int) -> np.ndarray:
    return buf.window(r0 * cols, (r1 - r0) * cols).numpy().reshape(r1 - r0, cols)


def test_swiglu_f16_beyond_2_31_elements():
    F = 14336
    rows = E31 // F + 200                       # 2,150,400,000 elements per tensor
    assert rows * F > E31
    g = to_f16_bits(normal(0x5A1, (TILE, F), clip=8.0))
    u = to_f16_bits(normal(0x5A2, (TILE, F), clip=8.0))
    dg, du = _tiled(g, rows), _tiled(u, rows)
    out = ql.DeviceArray((rows * F,), np.uint16)
    ql.call("ql_swiglu_f16", dg.ptr, du.ptr, out.ptr, rows, F, stream())
    synchronize()
    want = orc.swiglu(g, u, f16=True)
    for r0, r1 in _windows(rows, F):
        check_f16(_rows(out, r0, r1, F), want[np.arange(r0, r1) % TILE], f"swiglu rows {r0}..{r1}")


def test_add_rmsnorm_f16_beyond_2_31_elements():
    D = 4096
    rows = E31 // D + 130
    x = to_f16_bits(normal(0x5A3, (TILE, D)))
    d = to_f16_bits(normal(0x5A4, (TILE, D)))
    w = to_f16_bits(uniform(0x5A5, D, 0.5, 1.5))
    dx, dd, dw = _tiled(x, rows), _tiled(d, rows), dev(w)
    y = ql.DeviceArray((rows * D,), np.uint16)
    ql.call("ql_add_rmsnorm_f16", dx.ptr, dd.ptr, dw.ptr, y.ptr, rows, D, 1e-5, stream())
    synchronize()
    wx, wy = orc.add_rmsnorm(x, d, w, 1e-5, f16=True)
    for r0, r1 in _windows(rows, D):
        sel = np.arange(r0, r1) % TILE
        assert np.array_equal(_rows(dx, r0, r1, D), wx[sel]), f"x' rows {r0}..{r1}"
        check_f16(_rows(y, r0, r1, D), wy[sel], f"add_rmsnorm rows {r0}..{r1}")


def test_softmax_f16_beyond_2_31_elements():
    C = 4096
    rows = E31 // C + 130
    x = normal(0x5A6, (TILE, C), sigma=2.0)
    x[np.triu_indices(TILE, k=1 + C - TILE, m=C)] = -np.inf     # causal rows C-64 .. C-1
    xh = to_f16_bits(x)
    dx = _tiled(xh, rows)
    out = ql.DeviceArray((rows * C,), np.uint16)
    ql.call("ql_softmax_f16", dx.ptr, out.ptr, rows, C, stream())
    synchronize()
    want = orc.softmax(xh, f16=True)
    for r0, r1 in _windows(rows, C):
        check_f16(_rows(out, r0, r1, C), want[np.arange(r0, r1) % TILE], f"softmax rows {r0}..{r1}")


def test_embed_f16_beyond_2_31_elements():
    V, D = 32000, 4096
    T = E31 // D + 130
    r = np.random.default_rng(0x5A7)
    table = r.integers(0, 0x7C00, size=(V, D), dtype=np.uint16)     # finite binary16 values
    ids = r.integers(0, V, size=T).astype(np.int32)
    ids[-3] = -1                                                      # out of range: zero row
    dt, di = dev(table), dev(ids)
    out = ql.DeviceArray((T * D,), np.uint16)
    ql.call("ql_embed_f16", dt.ptr, di.ptr, T, V, D, out.ptr, stream())
    synchronize()
    for r0, r1 in _windows(T, D):
        want = orc.embed(table, ids[r0:r1], f16=True)
        assert np.array_equal(_rows(out, r0, r1, D), want), f"embed rows {r0}..{r1}"


def test_rope_f16_beyond_2_31_elements():
    H, HK, HD = 32, 8, 128
    T = E31 // (H * HD) + 130                                         # Q exceeds 2^31 elements
    q = to_f16_bits(normal(0x5A8, (TILE, H * HD)))
    k = to_f16_bits(normal(0x5A9, (TILE, HK * HD)))
    dq, dk = _tiled(q, T), _tiled(k, T)
    ql.call("ql_rope_f16", dq.ptr, dk.ptr, T, H, HK, HD, H * HD, HK * HD, None, 0, 5e5,
            ql.ROPE_HALF, stream())
    synchronize()
    for r0, r1 in _windows(T, H * HD):
        sel = np.arange(r0, r1) % TILE
        check_f16(_rows(dq, r0, r1, H * HD), orc.rope(q[sel], H, HD, 5e5, ql.ROPE_HALF,
                                                      pos_offset=r0, f16=True), f"rope q {r0}..{r1}")
        check_f16(_rows(dk, r0, r1, HK * HD), orc.rope(k[sel], HK, HD, 5e5, ql.ROPE_HALF,
                                                       pos_offset=r0, f16=True), f"rope k {r0}..{r1}")


def test_softmax_and_add_rmsnorm_f16_odd_width_beyond_2_31_elements():
    # rows of 4095 binary16 elements start at every offset mod 16: the covering-vector
    # paths, with row offsets past 2^31 elements
    C = 4095
    rows = E31 // C + 130
    x = normal(0x5AA, (TILE, C), sigma=2.0)
    xh = to_f16_bits(x)
    dx = _tiled(xh, rows)
    out = ql.DeviceArray((rows * C,), np.uint16)
    ql.call("ql_softmax_f16", dx.ptr, out.ptr, rows, C, stream())
    synchronize()
    want = orc.softmax(xh, f16=True)
    for r0, r1 in _windows(rows, C):
        check_f16(_rows(out, r0, r1, C), want[np.arange(r0, r1) % TILE], f"softmax rows {r0}..{r1}")
    del out
    d = to_f16_bits(normal(0x5AB, (TILE, C)))
    w = to_f16_bits(uniform(0x5AC, C, 0.5, 1.5))
    dd, dw = _tiled(d, rows), dev(w)
    y = ql.DeviceArray((rows * C,), np.uint16)
    ql.call("ql_add_rmsnorm_f16", dx.ptr, dd.ptr, dw.ptr, y.ptr, rows, C, 1e-5, stream())
    synchronize()
    wx, wy = orc.add_rmsnorm(xh, d, w, 1e-5, f16=True)
    for r0, r1 in _windows(rows, C):
        sel = np.arange(r0, r1) % TILE
        assert np.array_equal(_rows(dx, r0, r1, C), wx[sel]), f"x' rows {r0}..{r1}"
        check_f16(_rows(y, r0, r1, C), wy[sel], f"add_rmsnorm rows {r0}..{r1}")


@pytest.mark.parametrize("mode", [ql.FP8_MODE_REFERENCE, ql.FP8_MODE_OCP])
def test_fp8_per_tensor_quantize_and_dequantize_beyond_2_31_elements(mode):
    # one scale over more than 2^31 elements (workgroup maxima reduced in the code
    # buffer), then the codes and the dequantized rows in windows around element
    # 2^31: the tiled tensor has the tile's max (the reference mode's max sees the
    # same offsets mod 128, the rows being 4096 wide), so the tile quantized alone
    # gives the expected scale and codes
    C = 4096
    rows = E31 // C + 130
    x = to_f16_bits(uniform(0x5AD, (TILE, C), -3.0, 3.0))
    dx = _tiled(x, rows)
    q = ql.DeviceArray((rows * C,), np.uint8)
    sc = ql.DeviceArray((1,), np.float32)
    ql.call("ql_fp8_quantize", dx.ptr, rows, C, ql.FP8_E4M3, ql.QUANT_PER_TENSOR, 0, mode, q.ptr, sc.ptr, stream())
    synchronize()
    q_want, sc_want = orc.fp8_quantize(x, ql.FP8_E4M3, ql.QUANT_PER_TENSOR, 0, mode)
    assert np.array_equal(sc.numpy(), sc_want)
    for r0, r1 in _windows(rows, C):
        assert np.array_equal(_rows(q, r0, r1, C), q_want[np.arange(r0, r1) % TILE]), f"codes rows {r0}..{r1}"
    del dx
    y = ql.DeviceArray((rows * C,), np.uint16)
    ql.call("ql_fp8_dequantize", q.ptr, sc.ptr, rows, C, ql.FP8_E4M3, ql.QUANT_PER_TENSOR, 0, mode, y.ptr, stream())
    synchronize()
    y_want = orc.fp8_dequantize(q_want, sc_want, ql.FP8_E4M3, ql.QUANT_PER_TENSOR, 0, mode)
    for r0, r1 in _windows(rows, C):
        assert np.array_equal(_rows(y, r0, r1, C), y_want[np.arange(r0, r1) % TILE]), f"dequant rows {r0}..{r1}"


@pytest.mark.parametrize("mode", [ql.FP8_MODE_REFERENCE, ql.FP8_MODE_OCP])
def test_fp8_quantize_more_groups_than_a_grid_dimension(mode):
    # per channel with rows longer than one wavefront's group (16392 > 16384) and
    # more rows than grid y holds (65535): the block-strided maxima take grid z too
    C = 16392
    rows = 65535 + 101
    x = to_f16_bits(uniform(0x5AE, (TILE, C), -2.0, 2.0))
    dx = _tiled(x, rows)
    q = ql.DeviceArray((rows * C,), np.uint8)
    sc = ql.DeviceArray((rows,), np.float32)
    ql.call("ql_fp8_quantize", dx.ptr, rows, C, ql.FP8_E4M3, ql.QUANT_PER_CHANNEL, 0, mode, q.ptr, sc.ptr, stream())
    synchronize()
    q_want, sc_want = orc.fp8_quantize(x, ql.FP8_E4M3, ql.QUANT_PER_CHANNEL, 0, mode)
    assert np.array_equal(sc.numpy(), sc_want[np.arange(rows) % TILE])
    for r0, r1 in [(0, 4), (65533, 65539), (rows - 4, rows)]:
        assert np.array_equal(_rows(q, r0, r1, C), q_want[np.arange(r0, r1) % TILE]), f"codes rows {r0}..{r1}"
    # the scales entry alone (block-strided maxima with atomics, then finalized)
    sc2 = ql.DeviceArray((rows,), np.float32)
    ql.call("ql_fp8_scales", dx.ptr, rows, C, ql.FP8_E4M3, ql.QUANT_PER_CHANNEL, 0, mode, sc2.ptr, stream())
    synchronize()
    assert np.array_equal(sc2.numpy(), sc_want[np.arange(rows) % TILE])
