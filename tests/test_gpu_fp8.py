"""GPU parity of the FP8 weight codec (ql_fp8_scales / quantize / dequantize:
bit-exact against the oracle in both modes, both formats, all granularities,
including exhaustive encode and decode tables), of the FP8-weight GEMM
(ql_fp8_gemm_f16, both paths) and of the fp16 library GEMM (ql_gemm_f16).

GEMM tolerance: with s = sum_k a_k w_k computed in double from the codec's
dequantized weights and b = 2^-10*|s| + 2^-10 * sum_k |a_k w_k|, the output must
lie in [rnd16(s - b), rnd16(s + b)] (rnd16 = round to nearest binary16, which
is monotone, so this is exactly "the kernel's unrounded fp32 result lies within
b of s", and an overflowing sum must give the same-signed infinity; a NaN is
only accepted where s is NaN).  The kernels accumulate in fp32.  The register
path either multiplies each decoded weight by 1/scale before rounding it to
binary16, which can move a weight by one binary16 step (2^-11 relative), or,
for per-tensor and per-row scales and for groups of a multiple of 64,
multiplies the fp32 sums of the exactly decoded codes by 1/scale, which skips
the weight rounding altogether (at most 2^-11 relative from the oracle's
rounded weights).  The same bound covers every launch shape (the split of K
over wavefronts and workgroups, hence the fp32 summation order, differs
between the whole-row, register and whole-line kernels)."""
import ctypes

import numpy as np
import pytest

import oracle as orc
import quantlib_amd as ql
from helpers import Out, dev, empty, f16_bits_to_f32, host, normal, stream, to_f16_bits, uniform

pytestmark = pytest.mark.gpu

FMTS = [ql.FP8_E4M3, ql.FP8_E5M2]
MODES = [ql.FP8_MODE_REFERENCE, ql.FP8_MODE_OCP]


def n_scales(rows, cols, gran, gs):
    n = ctypes.c_int()
    ql.call("ql_fp8_num_scales", rows, cols, gran, gs, ctypes.byref(n))
    return n.value


def gpu_quantize(x, fmt, gran, gs, mode):
    # codes and scales between guard bands: a write past either fails the test
    rows, cols = x.shape
    q = Out(rows * cols, np.uint8, offset=8)
    sc = Out(n_scales(rows, cols, gran, gs), np.float32)
    dx = dev(x)
    ql.call("ql_fp8_quantize", dx.ptr, rows, cols, fmt, gran, gs, mode, q.ptr, sc.ptr, stream())
    return q.get(shape=(rows, cols)), sc.get()


def gpu_dequantize(q, sc, fmt, gran, gs, mode):
    rows, cols = q.shape
    out = Out(rows * cols, np.uint16, offset=8)
    dq, ds = dev(q), dev(sc)
    ql.call("ql_fp8_dequantize", dq.ptr, ds.ptr, rows, cols, fmt, gran, gs, mode, out.ptr, stream())
    return out.get(shape=(rows, cols))


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
    (4096, 4096, ql.QUANT_PER_TENSOR, 0),       # one group larger than a wavefront pass
    # groups beyond one wavefront: workgroup maxima in the code buffer, reduced per group
    (3, 20000, ql.QUANT_PER_CHANNEL, 0), (5, 9000, ql.QUANT_PER_GROUP, 20000), (3, 6000, ql.QUANT_PER_TENSOR, 0),
    # power-of-two groups take the one-pass kernel (scales and codes from one read of x,
    # ql_fp8_scales' vector pass for the scales alone): every lane count
    (16, 512, ql.QUANT_PER_GROUP, 16), (5, 96, ql.QUANT_PER_GROUP, 32), (7, 64, ql.QUANT_PER_GROUP, 64),
    (8, 1024, ql.QUANT_PER_GROUP, 256), (16, 512, ql.QUANT_PER_GROUP, 512), (3, 200, ql.QUANT_PER_GROUP, 128),
    # ... and a partial last group (fewer lanes than the group spans)
    (3, 1000, ql.QUANT_PER_GROUP, 512), (5, 24, ql.QUANT_PER_GROUP, 16), (1, 8, ql.QUANT_PER_GROUP, 64),
    (16, 64, ql.QUANT_PER_GROUP, 8), (3, 40, ql.QUANT_PER_GROUP, 8),   # groups of 8: one lane each
    # other multiples of 8 below 256: 64 / V whole groups of V vectors per wavefront span
    (7, 96, ql.QUANT_PER_GROUP, 24), (5, 120, ql.QUANT_PER_GROUP, 40), (6, 744, ql.QUANT_PER_GROUP, 248),
    (3, 200, ql.QUANT_PER_GROUP, 56), (64, 960, ql.QUANT_PER_GROUP, 24), (33, 1000, ql.QUANT_PER_GROUP, 200),
    # other multiples of 8 from 256 to 16384 take the one-wavefront-per-group pass: up
    # to 8, 16 and 32 vectors per lane, per-channel rows, partial last groups
    (5, 1000, ql.QUANT_PER_GROUP, 200), (3, 1000, ql.QUANT_PER_GROUP, 1992), (7, 3000, ql.QUANT_PER_GROUP, 4104),
    (4, 8192, ql.QUANT_PER_CHANNEL, 0), (6, 14336, ql.QUANT_PER_CHANNEL, 0), (2, 16384, ql.QUANT_PER_GROUP, 16384),
    (9, 48, ql.QUANT_PER_GROUP, 48),
    # lengths that are not a multiple of 8 (groups start inside 16-byte vectors): one
    # thread per group up to 64 for the scales, then 8 elements per thread with each
    # element's own group scale, also below 8
    (16, 360, ql.QUANT_PER_GROUP, 36), (8, 1000, ql.QUANT_PER_GROUP, 3), (4, 1000, ql.QUANT_PER_GROUP, 1),
    (6, 64, ql.QUANT_PER_GROUP, 65), (2, 4096, ql.QUANT_PER_GROUP, 63), (7, 1000, ql.QUANT_PER_CHANNEL, 0)])
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
@pytest.mark.parametrize("rows,cols,gran,gs,offset", [
    (64, 256, ql.QUANT_PER_GROUP, 128, 0),       # power-of-two groups, 16-byte loads: every lane count
    (16, 512, ql.QUANT_PER_GROUP, 16, 0), (5, 96, ql.QUANT_PER_GROUP, 32, 0), (7, 64, ql.QUANT_PER_GROUP, 64, 0),
    (3, 40, ql.QUANT_PER_GROUP, 8, 0),
    (8, 1024, ql.QUANT_PER_GROUP, 256, 0), (16, 512, ql.QUANT_PER_GROUP, 512, 0), (3, 200, ql.QUANT_PER_GROUP, 128, 0),
    (7, 96, ql.QUANT_PER_GROUP, 24, 0), (3, 200, ql.QUANT_PER_GROUP, 56, 0),   # several short groups a wavefront
    (5, 1000, ql.QUANT_PER_GROUP, 200, 0), (64, 960, ql.QUANT_PER_GROUP, 24, 0),
    (3, 2000, ql.QUANT_PER_GROUP, 400, 0),       # one wavefront per group, scales only: 8, 16, 32 vectors a lane
    (3, 6000, ql.QUANT_PER_CHANNEL, 0, 0), (4, 14336, ql.QUANT_PER_CHANNEL, 0, 0), (3, 8200, ql.QUANT_PER_CHANNEL, 0, 0),
    (5, 1000, ql.QUANT_PER_GROUP, 200, 1),       # unaligned source: element loads
    (3, 1000, ql.QUANT_PER_GROUP, 7, 0), (8, 1000, ql.QUANT_PER_GROUP, 3, 0),   # one thread per group
    (16, 360, ql.QUANT_PER_GROUP, 36, 0), (4, 1000, ql.QUANT_PER_GROUP, 36, 1), (2, 4096, ql.QUANT_PER_GROUP, 63, 0),
    (1024, 1024, ql.QUANT_PER_TENSOR, 0, 0),     # groups over many workgroups, 16-byte loads
    (4096, 4096, ql.QUANT_PER_TENSOR, 0, 0), (2, 20000, ql.QUANT_PER_CHANNEL, 0, 0),
    (3, 9001, ql.QUANT_PER_CHANNEL, 0, 0),       # ... element loads (n % 8 != 0)
    (1024, 1024, ql.QUANT_PER_TENSOR, 0, 3)])
def test_fp8_scales_entry_bit_exact(mode, fmt, rows, cols, gran, gs, offset):
    # ql_fp8_scales alone, over each of its passes: the oracle's scales bit for bit
    x = to_f16_bits(uniform(7 * rows + cols + gs, (rows, cols), -1.0, 1.0) * np.float32(3.0))
    ns = n_scales(rows, cols, gran, gs)
    sc = empty((ns,), np.float32, fill_bits=0xFF)
    ql.call("ql_fp8_scales", dev(x, offset).ptr, rows, cols, fmt, gran, gs, mode, sc.ptr, stream())
    assert np.array_equal(host(sc), orc.fp8_quantize(x, fmt, gran, gs, mode)[1])


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


@pytest.mark.parametrize("gs", [32, 8])
@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("fmt", FMTS)
def test_fp8_dequantize_any_scale_bit_exact(mode, fmt, gs):
    # every code under log-uniform scales from 2^-100 to 2^100 (the dequantizer divides
    # by a corrected reciprocal for scales in [2^-90, 2^90] and by fp32 division
    # outside), plus scales at and just past those limits: bit for bit the oracle's
    # binary16(decode / scale), NaN for NaN.  Groups of 32 take the 16-codes-per-thread
    # kernel, groups of 8 the 8-codes one.
    rng = np.random.default_rng(40 + 2 * fmt + mode)
    n_grp = 2048
    edges = np.array([2.0 ** -90, 2.0 ** 90, np.nextafter(np.float32(2.0 ** -90), 0),
                      np.nextafter(np.float32(2.0 ** 90), np.float32(np.inf)), 1.0, 3.0, 448.0, 1e-8], np.float32)
    sc = np.concatenate([edges, np.exp2(rng.uniform(-100, 100, n_grp - edges.size))]).astype(np.float32)
    codes = np.resize(np.arange(256, dtype=np.uint8), (n_grp, 256))
    codes = np.ascontiguousarray(rng.permuted(codes, axis=1)).reshape(n_grp * 256 // gs, gs)
    scg = np.repeat(sc, 256 // gs)          # one row per group, each group's scale
    got = gpu_dequantize(codes, scg, fmt, ql.QUANT_PER_GROUP, gs, mode)
    want = orc.fp8_dequantize(codes, scg, fmt, ql.QUANT_PER_GROUP, gs, mode)
    assert same_f16(got, want), int((got != want).sum())


def gemm_exact(a, w_deq):
    """(s, b): the double-precision product of the binary16 operands and its bound."""
    af, wf = f16_bits_to_f32(a).astype(np.float64), f16_bits_to_f32(w_deq).astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        s = af @ wf.T
        b = 2.0 ** -10 * np.abs(s) + 2.0 ** -10 * (np.abs(af) @ np.abs(wf).T)
    return s, b


def check_gemm(got, exact, what):
    s, b = exact
    g = f16_bits_to_f32(got).astype(np.float64)
    nan_s = np.isnan(s)
    assert not np.isnan(g[~nan_s]).any(), f"{what}: {int(np.isnan(g[~nan_s]).sum())} NaN outputs"
    assert np.isnan(g[nan_s]).all(), f"{what}: NaN expected"
    s, b, g = s[~nan_s], b[~nan_s], g[~nan_s]
    with np.errstate(over="ignore", invalid="ignore"):
        lo = (s - b).astype(np.float16).astype(np.float64)
        hi = (s + b).astype(np.float16).astype(np.float64)
    bad = ~((lo <= g) & (g <= hi))
    if bad.any():
        i = int(np.flatnonzero(bad)[0])
        raise AssertionError(f"{what}: {int(bad.sum())} of {g.size} outputs outside "
                             f"[rnd16(s-b), rnd16(s+b)]; first got={g[i]!r} s={s[i]!r} b={b[i]!r}")
    return int(np.isinf(g).sum())


def gpu_fp8_gemm(a, q, sc, M, N, K, fmt, gran, gs, mode, workspace):
    """workspace: "query" (ql_fp8_gemm_workspace_size bytes), "none", or a byte count."""
    if workspace == "query":
        size = ctypes.c_size_t()
        ql.call("ql_fp8_gemm_workspace_size", M, N, K, gran, gs, ctypes.byref(size))
        nbytes = size.value
    else:
        nbytes = 0 if workspace == "none" else workspace
    da, dq, ds = dev(a), dev(q), dev(sc)
    out = empty((M * N,), np.uint16)
    ws = empty((max(nbytes, 16),), np.uint8)
    ql.call("ql_fp8_gemm_f16", da.ptr, dq.ptr, ds.ptr, M, N, K, fmt, gran, gs, mode, out.ptr,
            ws.ptr if nbytes else None, nbytes, stream())
    return host(out, shape=(M, N))


GEMM_CASES = [
    (1, 4096, 4096, ql.QUANT_PER_GROUP, 128), (7, 256, 14336, ql.QUANT_PER_CHANNEL, 0),
    (33, 1024, 1024, ql.QUANT_PER_TENSOR, 0), (64, 512, 512, ql.QUANT_PER_GROUP, 64),
    (65, 512, 512, ql.QUANT_PER_GROUP, 128), (200, 96, 320, ql.QUANT_PER_GROUP, 100),
    (16, 100, 256, ql.QUANT_PER_CHANNEL, 0),
    (64, 1024, 4096, ql.QUANT_PER_GROUP, 48),      # groups straddle rows: general scale index
    (24, 208, 1024, ql.QUANT_PER_GROUP, 16),       # 13 row tiles: one tile per workgroup
    (48, 480, 2048, ql.QUANT_PER_GROUP, 32),       # 30 row tiles: two per workgroup
    (16, 512, 3072, ql.QUANT_PER_GROUP, 48),       # K-splits start inside a group
    (8, 256, 4096, ql.QUANT_PER_GROUP, 16),        # unsplit: too many groups for the LDS table
    (64, 1024, 8192, ql.QUANT_PER_GROUP, 16),
    (20, 512, 1024, ql.QUANT_PER_CHANNEL, 0),      # two token tiles, four row tiles
    (3, 480, 448, ql.QUANT_PER_GROUP, 64),         # one token tile, two row tiles
    (5, 208, 320, ql.QUANT_PER_TENSOR, 0),         # one token tile, one row tile
    (30, 480, 512, ql.QUANT_PER_CHANNEL, 0),       # two token tiles, two row tiles
    (40, 208, 512, ql.QUANT_PER_GROUP, 64),        # four token tiles, one row tile
    # at most 8 tokens and K a multiple of 256: whole-row loads
    (4, 1024, 512, ql.QUANT_PER_GROUP, 128),       # 4 row tiles per workgroup, one wavefront each
    (8, 480, 512, ql.QUANT_PER_CHANNEL, 0),        # 30 row tiles: 2 per workgroup
    (5, 208, 256, ql.QUANT_PER_TENSOR, 0),         # 13 row tiles: 1 per workgroup, one chunk
    (1, 512, 768, ql.QUANT_PER_CHANNEL, 0),        # 3 chunks: a ring round and a remainder
    (8, 512, 1024, ql.QUANT_PER_GROUP, 256),       # 2 wavefronts per row tile
    (2, 256, 2048, ql.QUANT_PER_GROUP, 64),        # 4 wavefronts per row tile
    (3, 512, 4096, ql.QUANT_PER_GROUP, 512),       # 8 wavefronts per row tile
    (2, 256, 8192, ql.QUANT_PER_TENSOR, 0),        # 8 wavefronts per row tile and K-splits
    (1, 64, 32768, ql.QUANT_PER_GROUP, 64),        # without a workspace: group table too large
    (7, 1536, 1280, ql.QUANT_PER_GROUP, 128)]      # 5 chunks over 2 wavefronts


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,N,K,gran,gs", GEMM_CASES)
def test_fp8_gemm_matches_oracle(mode, fmt, M, N, K, gran, gs):
    a = to_f16_bits(normal(M + N + K, (M, K)))
    w = to_f16_bits(normal(M * N + K, (N, K), K ** -0.5))
    q, sc = orc.fp8_quantize(w, fmt, gran, gs, mode)
    w_deq = orc.fp8_dequantize(q, sc, fmt, gran, gs, mode)
    exact = gemm_exact(a, w_deq)
    # the oracle's product rounds to binary16 inside the interval
    want = orc.matmul(a, w_deq)
    check_gemm(want, exact, "oracle")
    # with the queried workspace (K split over workgroups when the register path
    # runs), then without one where the register path runs
    size = ctypes.c_size_t()
    ql.call("ql_fp8_gemm_workspace_size", M, N, K, gran, gs, ctypes.byref(size))
    register_path = size.value != N * K * 2
    assert register_path == (M <= 64 and N % 16 == 0 and K % 64 == 0)
    for workspace in ("query",) + (("none",) if register_path else ()):
        got = gpu_fp8_gemm(a, q, sc, M, N, K, fmt, gran, gs, mode, workspace)
        check_gemm(got, exact, f"fp8 gemm {M}x{N}x{K} workspace {workspace}")


# Shapes that select every launch variant of the FP8-weight GEMM's two register
# paths, run in all four format/mode pairs by the test below (ids name them):
# - register path, more than 8 tokens (or reference-mode E5M2): token tiles
#   MT = 1, 2, 4 (12, 24, 48 tokens) x row tiles per workgroup R = 4, 2, 1
#   (N = 128, 96, 80: 8, 6, 5 row tiles) x scale handling: per tensor, per row,
#   folded groups of 64 (MT <= 2; four token tiles take the LDS table), an LDS
#   table of groups of 32, groups of 48 that do not divide K (general index),
#   and groups of 16 over K = 8192, whose table only fits LDS once K is split
#   (the "none" workspace run keeps it whole);
#   (with four token tiles and four row tiles the whole-line kernel takes K a
#   multiple of 128, so the register kernel's cases there use K = 320);
# - whole-row path (at most 8 tokens, K a multiple of 256): row tiles x
#   wavefronts per tile (4,1) (2,1) (1,1) at K = 256, (2,2) (1,2) at K = 1024,
#   (1,4) at 2048 and (1,8) at 4096, each per tensor, per row and with folded
#   groups.
def _plan_cases():
    cases = []
    scales = [("tensor", ql.QUANT_PER_TENSOR, 0, 256), ("row", ql.QUANT_PER_CHANNEL, 0, 256),
              ("fold64", ql.QUANT_PER_GROUP, 64, 256), ("lds32", ql.QUANT_PER_GROUP, 32, 256),
              ("any48", ql.QUANT_PER_GROUP, 48, 256), ("table16", ql.QUANT_PER_GROUP, 16, 8192)]
    for mt, M in ((1, 12), (2, 24), (4, 48)):
        for r, N in ((4, 128), (2, 96), (1, 80)):
            for tag, gran, gs, K in scales:
                cases.append(pytest.param(M, N, K, gran, gs, id=f"regs-mt{mt}-r{r}-{tag}"))
    for (rw, kw), N, K in (((4, 1), 128, 256), ((2, 1), 96, 256), ((1, 1), 80, 256),
                           ((2, 2), 96, 1024), ((1, 2), 80, 1024), ((1, 4), 80, 2048),
                           ((1, 8), 80, 4096)):
        for tag, gran, gs in (("tensor", ql.QUANT_PER_TENSOR, 0), ("row", ql.QUANT_PER_CHANNEL, 0),
                              ("fold64", ql.QUANT_PER_GROUP, 64)):
            cases.append(pytest.param(3, N, K, gran, gs, id=f"rows-rw{rw}-kw{kw}-{tag}"))
    # four token tiles and four row tiles with K not a multiple of 128: the
    # whole-line kernel does not apply, so per-tensor and per-row scales stay on
    # the register kernel
    for tag, gran in (("tensor", ql.QUANT_PER_TENSOR), ("row", ql.QUANT_PER_CHANNEL)):
        cases.append(pytest.param(48, 128, 320, gran, 0, id=f"regs-mt4-r4-{tag}-k320"))
    return cases


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,N,K,gran,gs", _plan_cases())
def test_fp8_gemm_launch_variants(mode, fmt, M, N, K, gran, gs):
    a = to_f16_bits(normal(3 * M + N + K, (M, K)))
    w = to_f16_bits(normal(5 * N + K + gs, (N, K), K ** -0.5))
    q, sc = orc.fp8_quantize(w, fmt, gran, gs, mode)
    exact = gemm_exact(a, orc.fp8_dequantize(q, sc, fmt, gran, gs, mode))
    for workspace in ("query", "none"):
        got = gpu_fp8_gemm(a, q, sc, M, N, K, fmt, gran, gs, mode, workspace)
        check_gemm(got, exact, f"fp8 gemm {M}x{N}x{K} gran {gran} gs {gs} workspace {workspace}")


# One or two tokens with K a multiple of 16 take the contiguous-stream kernel: each
# wavefront walks its own run of rows, 1 KiB of a row per load instruction.  The
# shapes cover 1-3 rows per wavefront (N split evenly over at most 2048
# wavefronts, so runs of two lengths), N not a multiple of 16, rows of less
# than one instruction and a last instruction with 1, 4 or 40 live lanes, every
# scale kind (per tensor, per row, groups of 16, 48 and 128, which each lane's 16
# codes never straddle), and the largest token tile (two rows of 16384 codes:
# 64 KiB of LDS); K = 16400 at two tokens is past it and takes the other path.
STREAM_CASES = [
    (1, 100, 1040, ql.QUANT_PER_GROUP, 16), (2, 4100, 64, ql.QUANT_PER_CHANNEL, 0),
    (2, 300, 1536, ql.QUANT_PER_GROUP, 48), (1, 2049, 2048, ql.QUANT_PER_TENSOR, 0),
    (2, 64, 16384, ql.QUANT_PER_GROUP, 128), (1, 6000, 1664, ql.QUANT_PER_GROUP, 128),
    (2, 64, 16400, ql.QUANT_PER_GROUP, 16), (1, 512, 4096, ql.QUANT_PER_CHANNEL, 0)]


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,N,K,gran,gs", STREAM_CASES)
def test_fp8_gemm_stream_path(mode, fmt, M, N, K, gran, gs):
    a = to_f16_bits(normal(2 * M + N + K, (M, K)))
    w = to_f16_bits(normal(3 * N + K + gs, (N, K), K ** -0.5))
    q, sc = orc.fp8_quantize(w, fmt, gran, gs, mode)
    exact = gemm_exact(a, orc.fp8_dequantize(q, sc, fmt, gran, gs, mode))
    # the stream kernel needs no workspace; the path past its token tile does here
    stream_path = M * -(-K // 1024) * 2048 <= 65536
    for workspace in ("query",) + (("none",) if stream_path else ()):
        got = gpu_fp8_gemm(a, q, sc, M, N, K, fmt, gran, gs, mode, workspace)
        check_gemm(got, exact, f"fp8 gemm {M}x{N}x{K} gran {gran} gs {gs} workspace {workspace}")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,K", [(1, 1040), (2, 1040), (1, 64), (2, 4096)])
def test_fp8_gemm_stream_path_nonfinite_codes(fmt, M, K):
    """OCP inf and NaN codes in the first 16 codes of a row, the bytes that the
    stream kernel's lanes past K load (and must not use) when K is not a multiple
    of 1024: an infinite weight gives the same-signed infinite output, a NaN weight
    a NaN output, and the other rows are unaffected."""
    N = 256
    rng = np.random.default_rng(11 + M + K + fmt)
    codes = np.arange(256, dtype=np.uint8)
    bad = (codes & 0x7F) == 0x7F if fmt == ql.FP8_E4M3 else (codes & 0x7C) == 0x7C
    q = rng.choice(codes[~bad], size=(N, K)).astype(np.uint8)
    sc = rng.uniform(2.0, 8.0, N).astype(np.float32)
    nan_code = 0x7F if fmt == ql.FP8_E4M3 else 0x7E
    planted = {}
    for r in range(0, N, 7):
        kind = r // 7 % 3
        if fmt == ql.FP8_E4M3 and kind < 2:
            continue                                      # E4M3 (OCP) has no infinity
        col = int(rng.integers(0, min(K, 16)))
        q[r, col] = (0x7C, 0xFC, nan_code)[kind]
        planted[r] = (col, kind)
    a = to_f16_bits(normal(M + 3, (M, K)))
    af = f16_bits_to_f32(a)
    for r, (col, kind) in planted.items():
        a[:, col] = to_f16_bits(np.where(af[:, col] < 0, -1.0, 1.0).astype(np.float32))
    w_deq = orc.fp8_dequantize(q, sc, fmt, ql.QUANT_PER_CHANNEL, 0, ql.FP8_MODE_OCP)
    af, wf = f16_bits_to_f32(a).astype(np.float64), f16_bits_to_f32(w_deq).astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        s = af @ wf.T
    got = f16_bits_to_f32(gpu_fp8_gemm(a, q, sc, M, N, K, fmt, ql.QUANT_PER_CHANNEL, 0, ql.FP8_MODE_OCP,
                                       "query")).astype(np.float64)
    rows = np.array(sorted(planted))
    assert not np.isfinite(s[:, rows]).any()
    np.testing.assert_array_equal(np.isnan(got[:, rows]), np.isnan(s[:, rows]))
    fin = ~np.isnan(s[:, rows])
    np.testing.assert_array_equal(got[:, rows][fin], s[:, rows][fin])
    rest = np.setdiff1d(np.arange(N), rows)
    sub = gemm_exact(a, w_deq[rest])
    check_gemm(to_f16_bits(got[:, rest].astype(np.float32)), sub, f"fp8 gemm {M}x{N}x{K} unplanted rows")


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,N,K,gran,gs", [
    (64, 1024, 4096, ql.QUANT_PER_GROUP, 128),    # 16 row blocks, 8 K-splits, folded groups
    (48, 512, 2048, ql.QUANT_PER_CHANNEL, 0),     # 8 row blocks, 4 K-splits
    (40, 256, 8192, ql.QUANT_PER_GROUP, 32)])     # 16 K-splits, per-weight group scales
def test_fp8_gemm_reused_workspace(mode, fmt, M, N, K, gran, gs):
    """33-64 tokens with K-splits (the token copy and the fp32 partials share the
    workspace): calls that reuse one workspace, first filled with arbitrary bytes
    and then holding the call before's partials and copy, repeat the result bit for
    bit (the splits are summed in split order)."""
    a = to_f16_bits(normal(M + 3 * N + K, (M, K)))
    w = to_f16_bits(normal(N + K + gs, (N, K), K ** -0.5))
    q, sc = orc.fp8_quantize(w, fmt, gran, gs, mode)
    exact = gemm_exact(a, orc.fp8_dequantize(q, sc, fmt, gran, gs, mode))
    size = ctypes.c_size_t()
    ql.call("ql_fp8_gemm_workspace_size", M, N, K, gran, gs, ctypes.byref(size))
    da, dq, ds = dev(a), dev(q), dev(sc)
    ws = dev(np.full(size.value, 0xA5, np.uint8))
    outs = []
    for _ in range(3):
        out = empty((M * N,), np.uint16)
        ql.call("ql_fp8_gemm_f16", da.ptr, dq.ptr, ds.ptr, M, N, K, fmt, gran, gs, mode, out.ptr,
                ws.ptr, size.value, stream())
        outs.append(host(out, shape=(M, N)).copy())
    check_gemm(outs[0], exact, f"fp8 gemm {M}x{N}x{K} gran {gran} gs {gs}")
    for i, o in enumerate(outs[1:], 1):
        assert same_f16(o, outs[0]), f"call {i} differs"


@pytest.mark.parametrize("a_scale", [1.0, 2.0 ** -12])
@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,gran", [(1, ql.QUANT_PER_GROUP), (12, ql.QUANT_PER_GROUP), (64, ql.QUANT_PER_GROUP),
                                    (5, ql.QUANT_PER_CHANNEL)])
def test_fp8_gemm_every_code(mode, fmt, M, gran, a_scale):
    # raw codes, not encoder output: every byte appears in every 16-code run of some
    # rows, including the codes whose reference decode is not the OCP one (exponent 0
    # with a mantissa, 0x7F, E5M2 exponent 31); OCP mode leaves out its NaN / inf codes.
    # With a ~ N(0, 1) many E5M2 sums overflow binary16 (they must give the
    # same-signed infinity); with a scaled by 2^-12 every sum is finite and is
    # checked against the tolerance.
    N, K = 256, 512
    rng = np.random.default_rng(7 + M + 2 * fmt + 4 * mode)
    codes = np.arange(256, dtype=np.uint8)
    if mode == ql.FP8_MODE_OCP:
        bad = (codes & 0x7F) == 0x7F if fmt == ql.FP8_E4M3 else (codes & 0x7C) == 0x7C
        codes = codes[~bad]
    q = rng.choice(codes, size=(N, K)).astype(np.uint8)
    q[:128, :] = np.resize(codes, (128, K))               # every code in order
    gs = 128 if gran == ql.QUANT_PER_GROUP else 0
    sc = rng.uniform(2.0, 8.0, N * K // 128 if gs else N).astype(np.float32)
    a = to_f16_bits(normal(M + 11, (M, K)) * np.float32(a_scale))
    w_deq = orc.fp8_dequantize(q, sc, fmt, gran, gs, mode)
    exact = gemm_exact(a, w_deq)
    assert np.isfinite(exact[0]).all()
    check_gemm(orc.matmul(a, w_deq), exact, "oracle")
    got = gpu_fp8_gemm(a, q, sc, M, N, K, fmt, gran, gs, mode, "query")
    n_inf = check_gemm(got, exact, f"fp8 gemm codes fmt {fmt} mode {mode} M {M} gran {gran}")
    if a_scale < 1.0:
        assert n_inf == 0


def special_codes(fmt):
    """Codes whose reference decode differs from the OCP decode, from the oracle's two
    decoders (scale 4 keeps the reference's E5M2 exponent-31 values finite)."""
    q = np.arange(256, dtype=np.uint8).reshape(1, 256)
    sc = np.array([4.0], np.float32)
    ref = f16_bits_to_f32(orc.fp8_dequantize(q, sc, fmt, ql.QUANT_PER_TENSOR, 0, ql.FP8_MODE_REFERENCE))
    ocp = f16_bits_to_f32(orc.fp8_dequantize(q, sc, fmt, ql.QUANT_PER_TENSOR, 0, ql.FP8_MODE_OCP))
    same = (ref == ocp) | (np.isnan(ref) & np.isnan(ocp))
    return np.flatnonzero(~same.reshape(-1)).astype(np.uint8)


@pytest.mark.parametrize("fmt", FMTS)
def test_count_ref_special_matches_oracle_decoders(fmt):
    sp = special_codes(fmt)
    # E4M3: exponent 0 with a mantissa and 0x7F, both signs; E5M2: also exponent 31
    assert len(sp) == (16 if fmt == ql.FP8_E4M3 else 14)
    rng = np.random.default_rng(3 + fmt)
    count = empty((1,), np.uint64)
    for n, n_planted in ((0, 0), (7, 3), (4096, 0), (1_000_013, 57)):
        ok = np.setdiff1d(np.arange(256, dtype=np.uint8), sp)
        q = rng.choice(ok, size=n).astype(np.uint8)
        if n_planted:
            pos = rng.choice(n, n_planted, replace=False)
            q[pos] = rng.choice(sp, n_planted)
            q[-1] = sp[0]                                 # one in the last n % 16 codes
        want = int(np.isin(q, sp).sum())
        dq = dev(q) if n else empty((16,), np.uint8)
        ql.call("ql_fp8_count_ref_special", dq.ptr, n, fmt, count.ptr, stream())
        assert int(host(count)[0]) == want, (n, want)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,N,K,gran,gs", [
    (1, 4096, 4096, ql.QUANT_PER_GROUP, 128), (8, 1024, 2048, ql.QUANT_PER_CHANNEL, 0),
    (33, 512, 512, ql.QUANT_PER_GROUP, 64), (100, 256, 512, ql.QUANT_PER_TENSOR, 0)])
def test_fp8_gemm_clean_reference_codes(fmt, M, N, K, gran, gs):
    """Reference-encoded weights hold none of the codes whose decode differs; decoding
    them as QL_FP8_MODE_REFERENCE_CLEAN gives the reference-mode product (within the
    GEMM bound: the launch shape, hence the summation order, may differ) and the
    reference-mode dequantization bit for bit."""
    a = to_f16_bits(normal(M + 5, (M, K)))
    w = to_f16_bits(normal(N + 7, (N, K), K ** -0.5))
    q, sc = orc.fp8_quantize(w, fmt, gran, gs, ql.FP8_MODE_REFERENCE)
    count = empty((1,), np.uint64)
    dq = dev(q)
    ql.call("ql_fp8_count_ref_special", dq.ptr, q.size, fmt, count.ptr, stream())
    assert int(host(count)[0]) == int(np.isin(q, special_codes(fmt)).sum()) == 0
    w_deq = orc.fp8_dequantize(q, sc, fmt, gran, gs, ql.FP8_MODE_REFERENCE)
    exact = gemm_exact(a, w_deq)
    ref = gpu_fp8_gemm(a, q, sc, M, N, K, fmt, gran, gs, ql.FP8_MODE_REFERENCE, "query")
    clean = gpu_fp8_gemm(a, q, sc, M, N, K, fmt, gran, gs, ql.FP8_MODE_REFERENCE_CLEAN, "query")
    for got, what in ((ref, "reference"), (clean, "clean")):
        check_gemm(got, exact, f"{what} fp8 gemm {M}x{N}x{K}")
    # dequantize: identical codes decode identically
    outs = []
    for mode in (ql.FP8_MODE_REFERENCE, ql.FP8_MODE_REFERENCE_CLEAN):
        y = empty((N * K,), np.uint16)
        dsc = dev(sc)
        ql.call("ql_fp8_dequantize", dq.ptr, dsc.ptr, N, K, fmt, gran, gs, mode, y.ptr, stream())
        outs.append(host(y).copy())
    np.testing.assert_array_equal(outs[0], outs[1])


@pytest.mark.parametrize("M,N,K", [
    (1, 4096, 4096), (64, 6144, 4096), (300, 512, 1000), (8192, 256, 512),
    # few rows, odd widths
    (2, 4096, 4096), (16, 14336, 4096), (7, 1024, 14336), (9, 480, 512), (5, 100, 256), (3, 512, 1000)])
def test_gemm_f16_matches_oracle(M, N, K):
    a = to_f16_bits(normal(M + K, (M, K)))
    w = to_f16_bits(normal(N + K, (N, K), K ** -0.5))
    da, dw = dev(a), dev(w)
    out = empty((M * N,), np.uint16)
    ql.call("ql_gemm_f16", da.ptr, dw.ptr, out.ptr, M, N, K, stream())
    exact = gemm_exact(a, w)
    check_gemm(orc.matmul(a, w), exact, "oracle")
    check_gemm(host(out, shape=(M, N)), exact, f"gemm {M}x{N}x{K}")
