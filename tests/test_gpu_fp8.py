"""GPU parity of the FP8 weight codec (ql_fp8_scales / quantize / dequantize:
bit-exact against the oracle in both modes, both formats, all granularities,
including exhaustive encode and decode tables), of the FP8-weight GEMM
(ql_fp8_gemm_f16, both paths) and of the fp16 library GEMM (ql_gemm_f16).

GEMM tolerance, |got - want| <= 2^-10*|want| + 2^-10 * sum_k |a_k w_k|: the
oracle accumulates in double from the codec's dequantized weights; the kernels
accumulate in fp32, and the skinny path dequantizes with a multiply by 1/scale,
which can move a weight by one binary16 step (2^-11 relative)."""
import ctypes

import numpy as np
import pytest

import oracle as orc
import quantlib_amd as ql
from helpers import dev, empty, f16_bits_to_f32, host, normal, stream, to_f16_bits, uniform

pytestmark = pytest.mark.gpu

FMTS = [ql.FP8_E4M3, ql.FP8_E5M2]
MODES = [ql.FP8_MODE_REFERENCE, ql.FP8_MODE_OCP]


def n_scales(rows, cols, gran, gs):
    n = ctypes.c_int()
    ql.call("ql_fp8_num_scales", rows, cols, gran, gs, ctypes.byref(n))
    return n.value


def gpu_quantize(x, fmt, gran, gs, mode):
    rows, cols = x.shape
    q = empty((rows * cols,), np.uint8)
    sc = empty((max(n_scales(rows, cols, gran, gs), 1),), np.float32)
    dx = dev(x)
    ql.call("ql_fp8_quantize", dx.ptr, rows, cols, fmt, gran, gs, mode, q.ptr, sc.ptr, stream())
    return host(q, shape=(rows, cols)), host(sc)[:n_scales(rows, cols, gran, gs)]


def gpu_dequantize(q, sc, fmt, gran, gs, mode):
    rows, cols = q.shape
    out = empty((rows * cols,), np.uint16)
    dq, ds = dev(q), dev(sc)
    ql.call("ql_fp8_dequantize", dq.ptr, ds.ptr, rows, cols, fmt, gran, gs, mode, out.ptr, stream())
    return host(out, shape=(rows, cols))


def same_f16(a, b):
    fa, fb = f16_bits_to_f32(a), f16_bits_to_f32(b)
    nan = np.isnan(fb)
    return np.array_equal(np.isnan(fa), nan) and np.array_equal(a[~nan], b[~nan])


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("rows,cols,gran,gs", [
    (1024, 1024, ql.QUANT_PER_GROUP, 128),     # the reference test's shape and grouping
    (1024, 1024, ql.QUANT_PER_CHANNEL, 0), (1024, 1024, ql.QUANT_PER_TENSOR, 0),
    (64, 256, ql.QUANT_PER_GROUP, 100), (3, 1000, ql.QUANT_PER_GROUP, 7), (5, 33, ql.QUANT_PER_CHANNEL, 0),
    (4096, 4096, ql.QUANT_PER_TENSOR, 0)])      # one group larger than a wavefront pass
def test_fp8_codec_bit_exact(mode, fmt, rows, cols, gran, gs):
    x = to_f16_bits(uniform(rows + cols + gs, (rows, cols), -1.0, 1.0) *
                    np.float32(1.0 if fmt == ql.FP8_E4M3 else 300.0))
    q, sc = gpu_quantize(x, fmt, gran, gs, mode)
    q_want, sc_want = orc.fp8_quantize(x, fmt, gran, gs, mode)
    assert np.array_equal(sc, sc_want)
    assert np.array_equal(q, q_want), int((q != q_want).sum())
    assert same_f16(gpu_dequantize(q, sc, fmt, gran, gs, mode), orc.fp8_dequantize(q, sc, fmt, gran, gs, mode))


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("fmt", FMTS)
def test_fp8_encode_every_half_and_decode_every_code(mode, fmt):
    # groups of 32 whose first element is fmax: scale == 1, so codes = encode(x) for
    # every binary16 value up to fmax (both modes see all 32 offsets)
    fmax = 448.0 if fmt == ql.FP8_E4M3 else 57344.0
    h = np.arange(0, 0x10000, dtype=np.uint32).astype(np.uint16)
    h = h[np.abs(f16_bits_to_f32(h)) <= fmax]                      # finite, in range
    per = 31
    n_grp = -(-h.size // per)
    x = np.full((n_grp, 32), to_f16_bits(np.array([fmax], np.float32))[0], np.uint16)
    x[:, 1:].reshape(-1)[:h.size] = h
    q, sc = gpu_quantize(x, fmt, ql.QUANT_PER_GROUP, 32, mode)
    assert np.all(sc == 1.0)
    q_want, _ = orc.fp8_quantize(x, fmt, ql.QUANT_PER_GROUP, 32, mode)
    assert np.array_equal(q, q_want), int((q != q_want).sum())
    codes = np.arange(256, dtype=np.uint8).reshape(8, 32)
    ones = np.ones(8, np.float32)
    assert same_f16(gpu_dequantize(codes, ones, fmt, ql.QUANT_PER_GROUP, 32, mode),
                    orc.fp8_dequantize(codes, ones, fmt, ql.QUANT_PER_GROUP, 32, mode))


def gemm_bound(a, w_deq, want):
    af, wf = f16_bits_to_f32(a).astype(np.float64), f16_bits_to_f32(w_deq).astype(np.float64)
    return 2.0 ** -10 * np.abs(f16_bits_to_f32(want)) + 2.0 ** -10 * (np.abs(af) @ np.abs(wf).T)


def check_gemm(got, want, bound, what):
    err = np.abs(f16_bits_to_f32(got).astype(np.float64) - f16_bits_to_f32(want))
    bad = err > bound
    assert not bad.any(), f"{what}: {int(bad.sum())} elements out of bound, worst {float((err - bound).max()):.3e}"


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,N,K,gran,gs", [
    (1, 4096, 4096, ql.QUANT_PER_GROUP, 128), (7, 256, 14336, ql.QUANT_PER_CHANNEL, 0),
    (33, 1024, 1024, ql.QUANT_PER_TENSOR, 0), (64, 512, 512, ql.QUANT_PER_GROUP, 64),
    (65, 512, 512, ql.QUANT_PER_GROUP, 128), (200, 96, 320, ql.QUANT_PER_GROUP, 100),
    (16, 100, 256, ql.QUANT_PER_CHANNEL, 0)])
def test_fp8_gemm_matches_oracle(mode, fmt, M, N, K, gran, gs):
    a = to_f16_bits(normal(M + N + K, (M, K)))
    w = to_f16_bits(normal(M * N + K, (N, K), K ** -0.5))
    q, sc = orc.fp8_quantize(w, fmt, gran, gs, mode)
    w_deq = orc.fp8_dequantize(q, sc, fmt, gran, gs, mode)
    want = orc.matmul(a, w_deq)
    da, dq, ds = dev(a), dev(q), dev(sc)
    out = empty((M * N,), np.uint16)
    ws = empty((N * K,), np.uint16)
    ql.call("ql_fp8_gemm_f16", da.ptr, dq.ptr, ds.ptr, M, N, K, fmt, gran, gs, mode, out.ptr, ws.ptr,
            N * K * 2, stream())
    check_gemm(host(out, shape=(M, N)), want, gemm_bound(a, w_deq, want), f"fp8 gemm {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (64, 6144, 4096), (300, 512, 1000), (8192, 256, 512)])
def test_gemm_f16_matches_oracle(M, N, K):
    a = to_f16_bits(normal(M + K, (M, K)))
    w = to_f16_bits(normal(N + K, (N, K), K ** -0.5))
    da, dw = dev(a), dev(w)
    out = empty((M * N,), np.uint16)
    ql.call("ql_gemm_f16", da.ptr, dw.ptr, out.ptr, M, N, K, stream())
    want = orc.matmul(a, w)
    check_gemm(host(out, shape=(M, N)), want, gemm_bound(a, w, want), f"gemm {M}x{N}x{K}")
