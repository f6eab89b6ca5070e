"""GPU parity: every C-ABI entry point against the CPU oracle on identical
seeded inputs, at the BASELINE configs (C1..C5) and at the edge shapes that
select each kernel variant (register-resident widths, multi-wavefront rows,
block-per-row fallback, unaligned pointers, ragged tails).  Outputs sit inside
guard bands that must survive untouched.

Tolerances are those of tests/helpers.py: fp32 rtol 1e-5 (RoPE: abs 1e-6),
binary16 rtol 2e-3 (+ one subnormal step), gather/KV append bit-exact."""
import numpy as np
import pytest

import oracle as orc
import quantlib_amd as ql
from helpers import (ATOL_F32, ATOL_ROPE_F32, GUARD, GUARD_BYTE, RTOL_F32, Out,
                     causal_mask_inplace, check_abs, check_close, check_f16, dev, empty,
                     f16_bits_to_f32, host, normal, ptr, stream, to_f16_bits, uniform)

pytestmark = pytest.mark.gpu

def _f16(x):
    return to_f16_bits(x)


# ---- RMSNorm --------------------------------------------------------------------------------
F32_DIMS = [(2048, 2048), (1, 4), (7, 256), (5, 260), (3, 1000), (4, 4096), (3, 5000), (2, 8192),
            (2, 16384), (2, 20000), (2, 32768), (2, 40000), (3, 1001), (1, 3)]
F16_DIMS = [(64, 4096), (1, 8), (7, 512), (5, 520), (3, 1000), (4, 8192), (3, 10000),
            (2, 16384), (2, 32768), (2, 65536), (2, 70000), (3, 1001), (1, 5)]


@pytest.mark.parametrize("rows,dim", F32_DIMS)
def test_rmsnorm_f32(rows, dim):
    x = normal(0x51A10001 + dim, (rows, dim))
    w = uniform(0x51A10002 + dim, dim, 0.5, 1.5)
    out = Out(rows * dim, np.float32)
    dx, dw = dev(x), dev(w)
    ql.call("ql_rmsnorm_f32", ptr(dx), ptr(dw), out.ptr, rows, dim, 1e-5, stream())
    check_close(out.get((rows, dim)), orc.rmsnorm(x, w, 1e-5), RTOL_F32, ATOL_F32,
                f"rmsnorm f32 {rows}x{dim}")


@pytest.mark.parametrize("rows,dim", F16_DIMS)
def test_rmsnorm_f16(rows, dim):
    x = _f16(normal(0x51A10011 + dim, (rows, dim)))
    w = _f16(uniform(0x51A10012 + dim, dim, 0.5, 1.5))
    out = Out(rows * dim, np.uint16)
    dx, dw = dev(x), dev(w)
    ql.call("ql_rmsnorm_f16", ptr(dx), ptr(dw), out.ptr, rows, dim, 1e-5, stream())
    check_f16(out.get((rows, dim)), orc.rmsnorm(x, w, 1e-5, f16=True), f"rmsnorm f16 {rows}x{dim}")


# At 4096 rows and more the vector path spreads each row over 1..16 wavefronts
# (the wavefronts-per-row count follows the width), so every instantiation of
# the many-rows kernel runs here, plain and fused, including the C5 final-norm
# shape (fp16 8192 x 4096), ragged widths and a row count that leaves a partial
# workgroup.
MANY_ROWS_F16 = [(8192, 4096), (4096, 512), (4096, 1024), (4096, 2048), (4097, 1000), (4096, 8192),
                 (4099, 64)]
MANY_ROWS_F32 = [(4096, 256), (4096, 512), (4096, 1024), (4096, 2048), (4099, 1000), (4096, 4096),
                 (4097, 36)]


@pytest.mark.parametrize("add", [False, True])
@pytest.mark.parametrize("rows,dim", MANY_ROWS_F16)
def test_rmsnorm_f16_many_rows(rows, dim, add):
    x = _f16(normal(0x51A10061 + dim, (rows, dim)))
    d = _f16(normal(0x51A10062 + dim, (rows, dim)))
    w = _f16(uniform(0x51A10063 + dim, dim, 0.5, 1.5))
    out = Out(rows * dim, np.uint16)
    dx, dd, dw = dev(x), dev(d), dev(w)
    if add:
        ql.call("ql_add_rmsnorm_f16", ptr(dx), ptr(dd), ptr(dw), out.ptr, rows, dim, 1e-5, stream())
        want_x, want = orc.add_rmsnorm(x, d, w, 1e-5, f16=True)
        assert np.array_equal(host(dx, shape=(rows, dim)), want_x)
    else:
        ql.call("ql_rmsnorm_f16", ptr(dx), ptr(dw), out.ptr, rows, dim, 1e-5, stream())
        want = orc.rmsnorm(x, w, 1e-5, f16=True)
        assert np.array_equal(host(dx, shape=(rows, dim)), x)     # input untouched
    check_f16(out.get((rows, dim)), want, f"{'add_' if add else ''}rmsnorm f16 {rows}x{dim}")


@pytest.mark.parametrize("add", [False, True])
@pytest.mark.parametrize("rows,dim", MANY_ROWS_F32)
def test_rmsnorm_f32_many_rows(rows, dim, add):
    x = normal(0x51A10071 + dim, (rows, dim))
    d = normal(0x51A10072 + dim, (rows, dim))
    w = uniform(0x51A10073 + dim, dim, 0.5, 1.5)
    out = Out(rows * dim, np.float32)
    dx, dd, dw = dev(x), dev(d), dev(w)
    if add:
        ql.call("ql_add_rmsnorm_f32", ptr(dx), ptr(dd), ptr(dw), out.ptr, rows, dim, 1e-5, stream())
        want_x, want = orc.add_rmsnorm(x, d, w, 1e-5)
        assert np.array_equal(host(dx, shape=(rows, dim)), want_x)
    else:
        ql.call("ql_rmsnorm_f32", ptr(dx), ptr(dw), out.ptr, rows, dim, 1e-5, stream())
        want = orc.rmsnorm(x, w, 1e-5)
        assert np.array_equal(host(dx, shape=(rows, dim)), x)
    check_close(out.get((rows, dim)), want, RTOL_F32, ATOL_F32,
                f"{'add_' if add else ''}rmsnorm f32 {rows}x{dim}")


# Widths that select the remaining vector-path variants (fewer than 4096 rows):
# one-wavefront rows of 4 vectors per lane (binary16 1032-2048 wide, fp32
# fused 516-1024) and 2 (fp32 fused 260-512); 16-wavefront rows of 2, 4 or 8
# vectors per lane for the fused add (binary16 8200-16384 and 32776-65536 wide,
# fp32 4100-8192, 8196-16384 and 16388-32768).
VARIANT_WIDTHS = [(True, False, 50, 2048), (True, True, 50, 2048), (True, True, 9, 1536),
                  (True, True, 3, 12288), (True, True, 2, 65536), (False, True, 7, 512),
                  (False, True, 5, 1000), (False, True, 3, 8192), (False, True, 2, 16384),
                  (False, True, 2, 32768)]


@pytest.mark.parametrize("f16,add,rows,dim", VARIANT_WIDTHS)
def test_rmsnorm_variant_widths(f16, add, rows, dim):
    x = normal(0x51A10081 + dim, (rows, dim))
    d = normal(0x51A10082 + dim, (rows, dim))
    w = uniform(0x51A10083 + dim, dim, 0.5, 1.5)
    if f16:
        x, d, w = _f16(x), _f16(d), _f16(w)
    dt = np.uint16 if f16 else np.float32
    out = Out(rows * dim, dt)
    dx, dd, dw = dev(x), dev(d), dev(w)
    sfx = "f16" if f16 else "f32"
    if add:
        ql.call(f"ql_add_rmsnorm_{sfx}", ptr(dx), ptr(dd), ptr(dw), out.ptr, rows, dim, 1e-5,
                stream())
        want_x, want = orc.add_rmsnorm(x, d, w, 1e-5, f16=f16)
        assert np.array_equal(host(dx, shape=(rows, dim)), want_x)
    else:
        ql.call(f"ql_rmsnorm_{sfx}", ptr(dx), ptr(dw), out.ptr, rows, dim, 1e-5, stream())
        want = orc.rmsnorm(x, w, 1e-5, f16=f16)
    tag = f"{'add_' if add else ''}rmsnorm {sfx} {rows}x{dim}"
    if f16:
        check_f16(out.get((rows, dim)), want, tag)
    else:
        check_close(out.get((rows, dim)), want, RTOL_F32, ATOL_F32, tag)


# Lengths that are not a multiple of a 16-byte vector, or rows at an offset: each row
# holds the aligned vectors that cover it (1 vector per lane over 1-16 wavefronts,
# then 2, 4, 8 per lane over 16), the vectors shared with a neighbouring row stored
# element by element.  One width per variant for each type, plain and fused; x, d
# and out at one offset mod 16 (and, last, at different offsets: the block-per-row
# loop).  Outputs between guard bands.
ANY_WIDTHS_F16 = [33, 1001, 2001, 4001, 4095, 10001, 30001, 65001]
ANY_WIDTHS_F32 = [33, 501, 1001, 2001, 4001, 8001, 16001, 32001]


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("add", [False, True])
@pytest.mark.parametrize("wi", range(8))
@pytest.mark.parametrize("off", [0, 3])
def test_rmsnorm_rows_at_any_offset(f16, add, wi, off):
    dim = (ANY_WIDTHS_F16 if f16 else ANY_WIDTHS_F32)[wi]
    rows = 5 if dim > 4096 else 37
    x = normal(0x51A10091 + dim + off, (rows, dim))
    d = normal(0x51A10092 + dim, (rows, dim))
    w = uniform(0x51A10093 + dim, dim, 0.5, 1.5)
    if f16:
        x, d, w = _f16(x), _f16(d), _f16(w)
    dt = np.uint16 if f16 else np.float32
    out = Out(rows * dim, dt, offset=off)
    dx, dd, dw = dev(x, off), dev(d, off), dev(w, 1)
    sfx = "f16" if f16 else "f32"
    tag = f"{'add_' if add else ''}rmsnorm {sfx} {rows}x{dim} +{off}"
    if add:
        ql.call(f"ql_add_rmsnorm_{sfx}", ptr(dx), ptr(dd), ptr(dw), out.ptr, rows, dim, 1e-5, stream())
        want_x, want = orc.add_rmsnorm(x, d, w, 1e-5, f16=f16)
        assert np.array_equal(host(dx, shape=(rows, dim)), want_x), tag
    else:
        ql.call(f"ql_rmsnorm_{sfx}", ptr(dx), ptr(dw), out.ptr, rows, dim, 1e-5, stream())
        want = orc.rmsnorm(x, w, 1e-5, f16=f16)
        assert np.array_equal(host(dx, shape=(rows, dim)), x), tag
    if f16:
        check_f16(out.get((rows, dim)), want, tag)
    else:
        check_close(out.get((rows, dim)), want, RTOL_F32, ATOL_F32, tag)


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("add,x_off,d_off,out_off,inplace", [
    (False, 1, 0, 1, True), (False, 6, 0, 6, True), (True, 2, 2, 0, False), (False, 1, 0, 0, False),
    (True, 0, 3, 0, False)])
def test_rmsnorm_any_in_place_and_mixed_offsets(f16, add, x_off, d_off, out_off, inplace):
    # plain RMSNorm in place (out = x, as the reference's two-pass kernel allows): a
    # row's covering loads read neighbouring rows' elements, which their own
    # workgroups may have overwritten already and which are never used; x, d and
    # out at different offsets mod 16 take the block-per-row loop
    rows, dim = 4097, 1001
    x = normal(0x51A100A1 + x_off, (rows, dim))
    d = normal(0x51A100A2, (rows, dim))
    w = uniform(0x51A100A3, dim, 0.5, 1.5)
    if f16:
        x, d, w = _f16(x), _f16(d), _f16(w)
    dt = np.uint16 if f16 else np.float32
    sfx = "f16" if f16 else "f32"
    dx, dd, dw = dev(x, x_off), dev(d, d_off), dev(w)
    out = None if inplace else Out(rows * dim, dt, offset=out_off)
    optr = ptr(dx) if inplace else out.ptr
    if add:
        ql.call(f"ql_add_rmsnorm_{sfx}", ptr(dx), ptr(dd), ptr(dw), optr, rows, dim, 1e-5, stream())
        want_x, want = orc.add_rmsnorm(x, d, w, 1e-5, f16=f16)
    else:
        ql.call(f"ql_rmsnorm_{sfx}", ptr(dx), ptr(dw), optr, rows, dim, 1e-5, stream())
        want_x, want = x, orc.rmsnorm(x, w, 1e-5, f16=f16)
    got = host(dx, shape=(rows, dim)) if inplace else out.get((rows, dim))
    if not inplace:
        assert np.array_equal(host(dx, shape=(rows, dim)), want_x)
    if f16:
        check_f16(got, want, f"rmsnorm f16 in place={inplace}")
    else:
        check_close(got, want, RTOL_F32, ATOL_F32, f"rmsnorm f32 in place={inplace}")


@pytest.mark.parametrize("f16", [False, True])
def test_rmsnorm_unaligned_pointers(f16):
    rows, dim = 9, 2048
    x = normal(31, (rows, dim))
    w = uniform(32, dim, 0.5, 1.5)
    if f16:
        x, w = _f16(x), _f16(w)
    dt = np.uint16 if f16 else np.float32
    out = Out(rows * dim, dt, offset=1)
    dx, dw = dev(x, offset_elems=1), dev(w, offset_elems=3)
    ql.call("ql_rmsnorm_f16" if f16 else "ql_rmsnorm_f32", ptr(dx), ptr(dw), out.ptr, rows, dim,
            1e-5, stream())
    want = orc.rmsnorm(x, w, 1e-5, f16=f16)
    if f16:
        check_f16(out.get((rows, dim)), want, "rmsnorm f16 unaligned")
    else:
        check_close(out.get((rows, dim)), want, RTOL_F32, ATOL_F32, "rmsnorm f32 unaligned")


@pytest.mark.parametrize("rows,dim", [(8192, 4096), (3, 4096), (5, 1000), (2, 20000), (3, 1001)])
def test_add_rmsnorm_f16(rows, dim):
    # C5: residual + RMSNorm at T=8192, hidden 4096 (and kernel-variant shapes)
    x = _f16(normal(0x51A10051, (rows, dim)))
    d = _f16(normal(0x51A10052, (rows, dim)))
    w = _f16(uniform(0x51A10053, dim, 0.5, 1.5))
    out = Out(rows * dim, np.uint16)
    dx, dd, dw = dev(x), dev(d), dev(w)
    ql.call("ql_add_rmsnorm_f16", ptr(dx), ptr(dd), ptr(dw), out.ptr, rows, dim, 1e-5, stream())
    want_x, want = orc.add_rmsnorm(x, d, w, 1e-5, f16=True)
    # the rounded residual sum is exact arithmetic: bit-exact
    assert np.array_equal(host(dx, shape=(rows, dim)), want_x)
    check_f16(out.get((rows, dim)), want, f"add_rmsnorm f16 {rows}x{dim}")


@pytest.mark.parametrize("rows,dim", [(2048, 2048), (3, 4096), (2, 50000), (3, 999)])
def test_add_rmsnorm_f32(rows, dim):
    x, d = normal(41, (rows, dim)), normal(42, (rows, dim))
    w = uniform(43, dim, 0.5, 1.5)
    out = Out(rows * dim, np.float32)
    dx, dd, dw = dev(x), dev(d), dev(w)
    ql.call("ql_add_rmsnorm_f32", ptr(dx), ptr(dd), ptr(dw), out.ptr, rows, dim, 1e-5, stream())
    want_x, want = orc.add_rmsnorm(x, d, w, 1e-5)
    assert np.array_equal(host(dx, shape=(rows, dim)), want_x)
    check_close(out.get((rows, dim)), want, RTOL_F32, ATOL_F32, f"add_rmsnorm f32 {rows}x{dim}")


# offsets: x and d not 16-byte aligned (at one offset: leading elements in block 0,
# then aligned vectors; fewer elements than that, or different offsets: the
# element-wise kernel)
@pytest.mark.parametrize("f16,n,offset,d_offset", [(False, 1 << 20, 0, 0), (True, 1 << 20, 0, 0), (False, 1001, 0, 0),
                                                   (True, 1003, 0, 0), (False, 4099, 1, 1), (True, 4101, 1, 1),
                                                   (True, 4101, 6, 6), (False, 2, 3, 3), (True, 4101, 1, 2),
                                                   (False, 4099, 0, 1)])
def test_residual_add(f16, n, offset, d_offset):
    x, d = normal(44, n), normal(45, n)
    if f16:
        x, d = _f16(x), _f16(d)
    dx, dd = dev(x, offset), dev(d, d_offset)
    ql.call("ql_add_f16" if f16 else "ql_add_f32", ptr(dx), ptr(dd), n, stream())
    assert np.array_equal(host(dx), orc.add(x, d, f16=f16))


# ---- RoPE -------------------------------------------------------------------------------------
def _rope_case(f16, T, H, HK, d, theta, pairing, seed, positions=None, pos_offset=0,
               q_extra=0, k_extra=0):
    qs, ks = H * d + q_extra, HK * d + k_extra
    q = normal(seed, (T, qs))
    k = normal(seed + 1, (T, ks))
    if f16:
        q, k = _f16(q), _f16(k)
    dq, dk = dev(q), dev(k)
    dpos = dev(np.asarray(positions, np.int32)) if positions is not None else None
    name = "ql_rope_f16" if f16 else "ql_rope_f32"
    ql.call(name, ptr(dq), ptr(dk), T, H, HK, d, qs, ks, ptr(dpos) if dpos is not None else None,
            pos_offset, theta, pairing, stream())
    wq = orc.rope(q, H, d, theta, pairing, positions, pos_offset, f16=f16)
    wk = orc.rope(k, HK, d, theta, pairing, positions, pos_offset, f16=f16)
    gq, gk = host(dq, shape=(T, qs)), host(dk, shape=(T, ks))
    tag = f"rope {'f16' if f16 else 'f32'} T={T} H={H}/{HK} d={d} pairing={pairing}"
    if f16:
        check_f16(gq, wq, tag + " Q")
        check_f16(gk, wk, tag + " K")
    else:
        check_abs(gq, wq, ATOL_ROPE_F32, tag + " Q")
        check_abs(gk, wk, ATOL_ROPE_F32, tag + " K")
    return gq, gk, q, k


@pytest.mark.parametrize("pairing", [ql.ROPE_INTERLEAVED, ql.ROPE_HALF])
def test_rope_f32_c2(pairing):
    # C2: Q[2048,32,64], K[2048,4,64], positions 0..2047, theta 1e4; norm preserved
    gq, _, q, _ = _rope_case(False, 2048, 32, 4, 64, 1e4, pairing, 0x51A10003)
    n0 = np.linalg.norm(q.reshape(2048, 32, 64).astype(np.float64), axis=2)
    n1 = np.linalg.norm(gq.reshape(2048, 32, 64).astype(np.float64), axis=2)
    assert np.max(np.abs(n0 - n1)) < 1e-5


@pytest.mark.parametrize("pairing", [ql.ROPE_HALF, ql.ROPE_INTERLEAVED])
def test_rope_f16_c5(pairing):
    # C5: Q 32x128, K 8x128, T=8192, theta 5e5
    _rope_case(True, 8192, 32, 8, 128, 5e5, pairing, 0x51A10005)


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("d", [2, 8, 16, 24, 32, 40, 48, 80, 96, 112, 120, 128, 136, 192, 256, 264, 2048])
def test_rope_head_dims(f16, d):
    for pairing in (ql.ROPE_INTERLEAVED, ql.ROPE_HALF):
        _rope_case(f16, 37, 3, 1, d, 1e4, pairing, 100 + d)


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("d", [24, 40, 48, 80, 96, 112, 192, 256])
def test_rope_head_dims_many_heads(f16, d):
    # head chunks that do not tile a wavefront: each pass takes the whole heads that
    # fit its 64 lanes (the rest idle), several passes per wavefront, several
    # wavefronts per token
    for pairing in (ql.ROPE_INTERLEAVED, ql.ROPE_HALF):
        _rope_case(f16, 29, 40, 8, d, 5e5, pairing, 300 + d)


@pytest.mark.parametrize("f16", [False, True])
def test_rope_positions_offset_and_fused_qkv_strides(f16):
    pos = np.random.default_rng(7).integers(0, 100_000, size=50).astype(np.int32)
    _rope_case(f16, 50, 8, 2, 64, 5e5, ql.ROPE_HALF, 200, positions=pos)
    _rope_case(f16, 50, 8, 2, 64, 5e5, ql.ROPE_INTERLEAVED, 210, pos_offset=4000)
    # Q rows padded to a fused [Q|K|V] stride: the padding must stay untouched
    gq, gk, q, k = _rope_case(f16, 40, 4, 2, 64, 1e4, ql.ROPE_HALF, 220, q_extra=256, k_extra=8)
    assert np.array_equal(gq[:, 4 * 64:], q[:, 4 * 64:])
    assert np.array_equal(gk[:, 2 * 64:], k[:, 2 * 64:])


@pytest.mark.parametrize("pairing", [ql.ROPE_HALF, ql.ROPE_INTERLEAVED])
@pytest.mark.parametrize("H,HK", [(5, 3), (1, 1), (7, 2), (64, 8)])
def test_rope_f16_d128_unit_shapes(pairing, H, HK):
    # binary16 head_dim 128 without a cache runs in 1 KiB units of four head
    # rows: units that straddle Q and K, idle lanes past the last head, padded
    # row strides (left untouched) and a positions array
    T = 37
    pos = np.random.default_rng(H * 10 + HK).integers(0, 1 << 17, size=T).astype(np.int32)
    gq, gk, q, k = _rope_case(True, T, H, HK, 128, 5e5, pairing, 240 + H, positions=pos,
                              q_extra=128, k_extra=8)
    assert np.array_equal(gq[:, H * 128:], q[:, H * 128:])
    assert np.array_equal(gk[:, HK * 128:], k[:, HK * 128:])
    # Q only and K only (the reference's launch_fp16_rope takes one tensor per call)
    for only_q in (True, False):
        x = _f16(normal(250 + H + only_q, (T, (H if only_q else HK) * 128)))
        dx = dev(x)
        n = H if only_q else HK
        ql.call("ql_rope_f16", ptr(dx) if only_q else None, None if only_q else ptr(dx), T,
                H if only_q else 9, HK if not only_q else 9, 128, n * 128, n * 128, None, 3, 5e5,
                pairing, stream())
        check_f16(host(dx, shape=(T, n * 128)), orc.rope(x, n, 128, 5e5, pairing, pos_offset=3, f16=True),
                  f"rope f16 d128 {'q' if only_q else 'k'} only")


def test_rope_q_only_and_k_only():
    T, H, d = 64, 4, 64
    q = normal(300, (T, H * d))
    dq = dev(q)
    ql.call("ql_rope_f32", ptr(dq), None, T, H, 7, d, H * d, 0, None, 0, 1e4, 0, stream())
    check_abs(host(dq, shape=(T, H * d)), orc.rope(q, H, d, 1e4, 0), ATOL_ROPE_F32, "q only")
    dk = dev(q)
    ql.call("ql_rope_f32", None, ptr(dk), T, 9, H, d, 0, H * d, None, 0, 1e4, 1, stream())
    check_abs(host(dk, shape=(T, H * d)), orc.rope(q, H, d, 1e4, 1), ATOL_ROPE_F32, "k only")


# ---- SwiGLU -------------------------------------------------------------------------------------
@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("rows,ffn", [(1, 5632), (32, 5632), (128, 5632), (512, 5632), (3, 1001),
                                      (1, 7)])
def test_swiglu_c3(f16, rows, ffn):
    g = normal(0x51A10004 + rows, (rows, ffn), clip=8.0)
    u = normal(0x51A10104 + rows, (rows, ffn), clip=8.0)
    if f16:
        g, u = _f16(g), _f16(u)
    out = Out(rows * ffn, np.uint16 if f16 else np.float32)
    dg, du = dev(g), dev(u)
    ql.call("ql_swiglu_f16" if f16 else "ql_swiglu_f32", ptr(dg), ptr(du), out.ptr, rows, ffn,
            stream())
    want = orc.swiglu(g, u, f16=f16)
    if f16:
        check_f16(out.get((rows, ffn)), want, f"swiglu f16 {rows}x{ffn}")
    else:
        check_close(out.get((rows, ffn)), want, RTOL_F32, ATOL_F32, f"swiglu f32 {rows}x{ffn}")


def test_swiglu_f16_c5():
    rows, ffn = 8192, 14336
    g = _f16(normal(0x51A10054, (rows, ffn), clip=8.0))
    u = _f16(normal(0x51A10055, (rows, ffn), clip=8.0))
    out = Out(rows * ffn, np.uint16)
    dg, du = dev(g), dev(u)
    ql.call("ql_swiglu_f16", ptr(dg), ptr(du), out.ptr, rows, ffn, stream())
    check_f16(out.get((rows, ffn)), orc.swiglu(g, u, f16=True), "swiglu f16 C5")


@pytest.mark.parametrize("f16", [False, True])
def test_swiglu_unaligned_and_extremes(f16):
    n = 4099
    g = normal(60, n, sigma=30.0)
    g[:6] = [0.0, 200.0, -200.0, np.inf, -np.inf, np.nan]
    u = normal(61, n)
    if f16:
        g, u = _f16(g), _f16(u)
    out = Out(n, np.uint16 if f16 else np.float32, offset=1)
    dg, du = dev(g, offset_elems=1), dev(u, offset_elems=2)
    ql.call("ql_swiglu_f16" if f16 else "ql_swiglu_f32", ptr(dg), ptr(du), out.ptr, 1, n, stream())
    want = orc.swiglu(g, u, f16=f16)
    got = out.get()
    if f16:
        check_f16(got, want, "swiglu f16 extremes")
    else:
        check_close(got, want, RTOL_F32, ATOL_F32, "swiglu f32 extremes")


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("n,off", [(4099, 1), (4099, 3), (24581, 7), (3, 1), (9, 5), (1 << 20, 2)])
def test_swiglu_at_a_shared_offset(f16, n, off):
    # gate, up and out at one offset mod 16: the elements up to the next 16-byte
    # boundary go to block 0, the rest streams as aligned vectors (n at most that
    # many elements: the element-wise kernel); guard bands around the output
    g = normal(62 + off, n, clip=8.0)
    u = normal(63 + off, n)
    if f16:
        g, u = _f16(g), _f16(u)
    out = Out(n, np.uint16 if f16 else np.float32, offset=off)
    dg, du = dev(g, offset_elems=off), dev(u, offset_elems=off)
    ql.call("ql_swiglu_f16" if f16 else "ql_swiglu_f32", ptr(dg), ptr(du), out.ptr, 1, n, stream())
    want = orc.swiglu(g, u, f16=f16)
    if f16:
        check_f16(out.get(), want, f"swiglu f16 n={n} +{off}")
    else:
        check_close(out.get(), want, RTOL_F32, ATOL_F32, f"swiglu f32 n={n} +{off}")


# ---- softmax -----------------------------------------------------------------------------------
@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("sigma", [2.0, 4.0])
def test_softmax_c4_causal(f16, sigma):
    # C4: logits[4096x4096] ~ N(0, sigma^2) with -inf above the diagonal
    n = 4096
    x = causal_mask_inplace(normal(0x51A10006, (n, n), sigma=sigma))
    if f16:
        x = _f16(x)
    out = Out(n * n, np.uint16 if f16 else np.float32)
    dx = dev(x)
    ql.call("ql_softmax_f16" if f16 else "ql_softmax_f32", ptr(dx), out.ptr, n, n, stream())
    want = orc.softmax(x, f16=f16)
    got = out.get((n, n))
    if f16:
        check_f16(got, want, f"softmax f16 C4 sigma={sigma}")
        assert np.all(got[np.triu_indices(n, 1)] == 0)
    else:
        check_close(got, want, RTOL_F32, ATOL_F32, f"softmax f32 C4 sigma={sigma}")
        assert np.all(got[np.triu_indices(n, 1)] == 0) and got[0, 0] == 1.0


def test_softmax_reference_test_thresholds():
    # tests/test_softmax.cu:38-47,88-106 on the GPU path: srand(7) U(-2,2) 2048x2048,
    # max abs error vs its cpu_softmax < 1e-5 and |row sum - 1| < 1e-5.
    x = orc.reftest_softmax_inputs(2048, 2048, 7)
    out = Out(2048 * 2048, np.float32)
    dx = dev(x)
    ql.call("ql_softmax_f32", ptr(dx), out.ptr, 2048, 2048, stream())
    got = out.get((2048, 2048))
    assert np.max(np.abs(got - orc.softmax_reftest_cpu(x))) < 1e-5
    assert np.max(np.abs(got.astype(np.float64).sum(axis=1) - 1.0)) < 1e-5


@pytest.mark.parametrize("f16", [False, True])
# Besides ragged and generic widths, every vector-path variant, exactly filled
# and with a partial last pass: binary16 512, 1024, 1536, 2048, 3000 (one
# wavefront, 1-8 vectors per lane), 6000 (8 wavefronts), 12000, 16384, 32768,
# 40000, 131072 (16 wavefronts, 2-16 vectors); fp32 512, 1024, 1500, 3000, 6000,
# 12000, 16384, 32768, 40000 (1-16 wavefronts, 2-16 vectors).
@pytest.mark.parametrize("rows,cols", [(5, 1), (7, 8), (9, 256), (6, 1000), (3, 8192), (3, 20000),
                                       (2, 65536), (2, 70000), (4, 4097), (1, 3), (5, 512),
                                       (5, 1024), (5, 1500), (5, 1536), (5, 2048), (4, 3000),
                                       (4, 6000), (3, 12000), (3, 16384), (2, 32768), (2, 40000),
                                       (2, 131072)])
def test_softmax_widths(f16, rows, cols):
    x = normal(500 + cols, (rows, cols), sigma=2.0)
    if cols > 3:
        x[0, :3] = -np.inf
    if f16:
        x = _f16(x)
    out = Out(rows * cols, np.uint16 if f16 else np.float32)
    dx = dev(x)
    ql.call("ql_softmax_f16" if f16 else "ql_softmax_f32", ptr(dx), out.ptr, rows, cols, stream())
    want = orc.softmax(x, f16=f16)
    if f16:
        check_f16(out.get((rows, cols)), want, f"softmax f16 {rows}x{cols}")
    else:
        check_close(out.get((rows, cols)), want, RTOL_F32, ATOL_F32, f"softmax f32 {rows}x{cols}")


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("rows,cols,in_off,out_off", [
    (100, 3, 0, 0), (33, 7, 1, 1), (17, 33, 3, 3), (9, 1001, 0, 0), (9, 1001, 5, 5), (6, 4095, 2, 2),
    (5, 4097, 0, 0), (3, 16383, 1, 1), (3, 32001, 0, 0), (2, 50257, 7, 7), (4, 1024, 1, 1),
    (5, 1001, 1, 0), (5, 1001, 0, 3)])   # last two: in and out at different offsets mod 16
def test_softmax_rows_at_any_offset(f16, rows, cols, in_off, out_off):
    # Rows whose starts are not 16-byte aligned (lengths not a multiple of a vector,
    # or offset pointers) take the covering aligned vectors of each row, storing the
    # vectors shared with a neighbouring row element by element; in and out at
    # different offsets take the block-per-row loop.  Guard bands catch stray writes.
    x = normal(900 + cols + in_off, (rows, cols), sigma=2.0)
    if cols > 3:
        x[-1, -3:] = -np.inf
    if f16:
        x = _f16(x)
    out = Out(rows * cols, np.uint16 if f16 else np.float32, offset=out_off)
    dx = dev(x, in_off)
    ql.call("ql_softmax_f16" if f16 else "ql_softmax_f32", ptr(dx), out.ptr, rows, cols, stream())
    want = orc.softmax(x, f16=f16)
    if f16:
        check_f16(out.get((rows, cols)), want, f"softmax f16 {rows}x{cols} +{in_off}/+{out_off}")
    else:
        check_close(out.get((rows, cols)), want, RTOL_F32, ATOL_F32, f"softmax f32 {rows}x{cols} +{in_off}/+{out_off}")


ANY_COLS_F16 = [33, 1001, 2001, 4001, 4095, 8001, 12001, 16001, 24001, 32001, 49001, 65001, 98001, 131001]
ANY_COLS_F32 = [33, 501, 1001, 2001, 4001, 6001, 8001, 12001, 16001, 24001, 32001, 49001, 65001]


@pytest.mark.parametrize("f16,cols", [(True, c) for c in ANY_COLS_F16] + [(False, c) for c in ANY_COLS_F32])
def test_softmax_any_length_every_variant(f16, cols):
    # one length per launch shape of the covering-vector path (vectors per lane x
    # wavefronts per row), so each runs under a check
    rows = 3
    x = normal(960 + cols, (rows, cols), sigma=2.0)
    if f16:
        x = _f16(x)
    out = Out(rows * cols, np.uint16 if f16 else np.float32)
    dx = dev(x)
    ql.call("ql_softmax_f16" if f16 else "ql_softmax_f32", ptr(dx), out.ptr, rows, cols, stream())
    want = orc.softmax(x, f16=f16)
    if f16:
        check_f16(out.get((rows, cols)), want, f"softmax f16 {rows}x{cols}")
    else:
        check_close(out.get((rows, cols)), want, RTOL_F32, ATOL_F32, f"softmax f32 {rows}x{cols}")


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("rows,cols,off", [(9, 1001, 0), (6, 4095, 3), (40, 5, 1)])
def test_softmax_in_place_rows_at_any_offset(f16, rows, cols, off):
    # in place: a row's covering loads read neighbouring rows' elements, which their
    # own workgroups may already have overwritten; those are never used
    x = normal(950 + cols, (rows, cols), sigma=2.0)
    if f16:
        x = _f16(x)
    d = dev(x, off)
    ql.call("ql_softmax_f16" if f16 else "ql_softmax_f32", ptr(d), ptr(d), rows, cols, stream())
    got = host(d, shape=(rows, cols))
    want = orc.softmax(x, f16=f16)
    if f16:
        check_f16(got, want, f"in-place softmax f16 {rows}x{cols}")
    else:
        check_close(got, want, RTOL_F32, ATOL_F32, f"in-place softmax f32 {rows}x{cols}")


@pytest.mark.parametrize("cols", [256, 1001])
def test_softmax_fully_masked_row_is_nan_like_reference(cols):
    x = normal(77, (3, cols))
    x[1] = -np.inf
    out = Out(3 * cols, np.float32)
    dx = dev(x)
    ql.call("ql_softmax_f32", ptr(dx), out.ptr, 3, cols, stream())
    got = out.get((3, cols))
    assert np.all(np.isnan(got[1])) and not np.any(np.isnan(got[[0, 2]]))


# ---- embedding gather -------------------------------------------------------------------------
def test_embed_f16_c5():
    V, D, T = 32000, 4096, 8192
    r = np.random.default_rng(0x51A10056)
    table = r.integers(0, 1 << 16, size=(V, D), dtype=np.uint32).astype(np.uint16)  # any bits
    ids = r.integers(0, V, size=T).astype(np.int32)
    out = Out(T * D, np.uint16)
    dt, di = dev(table), dev(ids)
    ql.call("ql_embed_f16", ptr(dt), ptr(di), T, V, D, out.ptr, stream())
    assert np.array_equal(out.get((T, D)), table[ids])


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("dim,t_off,o_off", [(1, 0, 0), (3, 1, 0), (7, 0, 5), (33, 2, 3), (1001, 0, 0),
                                             (4095, 3, 1), (4096, 1, 1), (2050, 0, 2), (5000, 7, 0)])
def test_embed_rows_at_any_offset(f16, dim, t_off, o_off):
    # rows that are not whole 16-byte vectors or sit at an offset: each output row's
    # covering vectors from two shifted table vectors, the ones shared with the
    # neighbouring rows stored element by element (guard bands around the output);
    # out-of-range ids give zero rows
    V, T = 257, 131
    r = np.random.default_rng(dim + 17 * t_off + o_off)
    table = normal(dim + 5, (V, dim))
    if f16:
        table = _f16(table)
    ids = r.integers(0, V, size=T).astype(np.int32)
    ids[[0, 7, 130]] = [-3, V, 2**31 - 1]
    out = Out(T * dim, np.uint16 if f16 else np.float32, offset=o_off)
    dt, di = dev(table, t_off), dev(ids)
    ql.call("ql_embed_f16" if f16 else "ql_embed_f32", ptr(dt), ptr(di), T, V, dim, out.ptr, stream())
    assert np.array_equal(out.get((T, dim)), orc.embed(table, ids, f16=f16))


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("dim", [1, 7, 64, 1000, 4096])
def test_embed_ragged_and_out_of_range(f16, dim):
    V, T = 300, 77
    r = np.random.default_rng(dim)
    table = normal(dim, (V, dim))
    if f16:
        table = _f16(table)
    ids = r.integers(0, V, size=T).astype(np.int32)
    ids[[0, 5, 9]] = [-1, V, 2**30]
    out = Out(T * dim, np.uint16 if f16 else np.float32)
    dt, di = dev(table), dev(ids)
    ql.call("ql_embed_f16" if f16 else "ql_embed_f32", ptr(dt), ptr(di), T, V, dim, out.ptr,
            stream())
    assert np.array_equal(out.get((T, dim)), orc.embed(table, ids, f16=f16))
    # single-token form (id by value), as launch_fp16_embed / embed_kernel
    one = Out(dim, np.uint16 if f16 else np.float32)
    ql.call("ql_embed_token_f16" if f16 else "ql_embed_token_f32", ptr(dt), 123, dim, one.ptr,
            stream())
    assert np.array_equal(one.get(), table[123])


# ---- KV append ---------------------------------------------------------------------------------
@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("L,S,H,d,T,layer,pos", [(4, 64, 8, 128, 1, 2, 17), (3, 9000, 8, 128, 8192, 1, 100),
                                                 (2, 50, 3, 5, 7, 1, 40), (2, 40, 1, 2, 3, 0, 0)])
def test_kv_append_contiguous(f16, L, S, H, d, T, layer, pos):
    dt = np.uint16 if f16 else np.float32
    r = np.random.default_rng(S + T)
    kn = r.integers(0, 60000, size=(T, H, d)).astype(dt)
    vn = r.integers(0, 60000, size=(T, H, d)).astype(dt)
    n = L * S * H * d
    kc, vc = Out(n, dt), Out(n, dt)
    dkn, dvn = dev(kn), dev(vn)
    ql.call("ql_kv_append_f16" if f16 else "ql_kv_append_f32", kc.ptr, vc.ptr, ptr(dkn), ptr(dvn),
            layer, pos, T, H, d, S, L, stream())
    want_k = np.full(n * np.dtype(dt).itemsize, GUARD_BYTE, np.uint8).view(dt).reshape(L, S, H, d)
    want_v = want_k.copy()
    orc.kv_append_inplace(want_k, want_v, kn, vn, layer, pos, f16=f16)
    assert np.array_equal(kc.get((L, S, H, d)), want_k)
    assert np.array_equal(vc.get((L, S, H, d)), want_v)


def test_paged_kv_append_f16_c5_and_permuted():
    # C5: 8192 tokens -> 512 blocks of 16; block [L,16,8,128]; fresh-pool order 0,1,2,...
    T, H, d, L, layer = 8192, 8, 128, 8, 5
    nb = T // 16
    blk = L * 16 * H * d
    r = np.random.default_rng(0x51A10057)
    kn = r.integers(0, 60000, size=(T, H, d)).astype(np.uint16)
    vn = r.integers(0, 60000, size=(T, H, d)).astype(np.uint16)
    dkn, dvn = dev(kn), dev(vn)
    for order in (np.arange(nb), r.permutation(nb)):
        kpool = empty((nb * blk,), np.uint16, fill_bits=GUARD_BYTE)
        vpool = empty((nb * blk,), np.uint16, fill_bits=GUARD_BYTE)
        kptrs = dev(np.array([kpool.ptr + 2 * blk * b for b in range(nb)], np.int64))
        vptrs = dev(np.array([vpool.ptr + 2 * blk * b for b in range(nb)], np.int64))
        slots = np.array([order[t // 16] * 16 + t % 16 for t in range(T)], np.int32)
        slots[[3, 4000]] = -1                       # padding tokens are skipped
        dsl = dev(slots)
        ql.call("ql_paged_kv_append_f16", ptr(kptrs), ptr(vptrs), nb, ptr(dsl), ptr(dkn), ptr(dvn),
                T, layer, L, H, d, stream())
        wk = np.full(nb * blk, 0xA5A5, np.uint16)
        wv = wk.copy()
        offs = (np.arange(nb) * blk).astype(np.int64)
        orc.paged_kv_append_inplace(wk, wv, offs, slots, kn, vn, layer, L, H, d)
        assert np.array_equal(host(kpool), wk)
        assert np.array_equal(host(vpool), wv)


def test_paged_kv_append_unaligned_rows_and_bad_slots():
    T, H, d, L, layer, nb = 40, 3, 6, 2, 1, 4        # kv = 18 elements: not 16-byte rows
    blk = L * 16 * H * d
    r = np.random.default_rng(9)
    kn = r.integers(0, 60000, size=(T, H, d)).astype(np.uint16)
    vn = r.integers(0, 60000, size=(T, H, d)).astype(np.uint16)
    kpool = empty((nb * blk,), np.uint16, fill_bits=GUARD_BYTE)
    vpool = empty((nb * blk,), np.uint16, fill_bits=GUARD_BYTE)
    kptrs = dev(np.array([kpool.ptr + 2 * blk * b for b in range(nb)], np.int64))
    vptrs = dev(np.array([vpool.ptr + 2 * blk * b for b in range(nb)], np.int64))
    slots = (np.arange(T) + 5).astype(np.int32)
    slots[7] = nb * 16 + 3                            # block beyond the pool: skipped
    dsl, dkn, dvn = dev(slots), dev(kn), dev(vn)
    ql.call("ql_paged_kv_append_f16", ptr(kptrs), ptr(vptrs), nb, ptr(dsl), ptr(dkn), ptr(dvn), T,
            layer, L, H, d, stream())
    wk = np.full(nb * blk, 0xA5A5, np.uint16)
    wv = wk.copy()
    orc.paged_kv_append_inplace(wk, wv, (np.arange(nb) * blk).astype(np.int64), slots, kn, vn,
                                layer, L, H, d)
    assert np.array_equal(host(kpool), wk) and np.array_equal(host(vpool), wv)


@pytest.mark.parametrize("T,H,d,misalign", [(7, 8, 128, 0), (9, 1, 64, 0), (13, 16, 128, 0), (5, 32, 128, 0),
                                             (11, 8, 128, 1), (6, 2, 8, 1), (3, 1, 8, 0)])
def test_paged_kv_append_token_groups_and_misaligned_blocks(T, H, d, misalign):
    # token counts that do not fill the last group of four, rows of 64 .. 4096
    # elements (one, two or four vectors per lane, and the wide-row kernel), and
    # block pointers 2 bytes past 16-byte alignment (element stores)
    L, layer = 3, 2
    nb = (T + 15) // 16 + 2
    blk = L * 16 * H * d
    r = np.random.default_rng(T * 100 + H * d + misalign)
    kn = r.integers(0, 60000, size=(T, H, d)).astype(np.uint16)
    vn = r.integers(0, 60000, size=(T, H, d)).astype(np.uint16)
    kpool = empty((nb * blk + 8,), np.uint16, fill_bits=GUARD_BYTE)
    vpool = empty((nb * blk + 8,), np.uint16, fill_bits=GUARD_BYTE)
    kptrs = dev(np.array([kpool.ptr + 2 * (misalign + blk * b) for b in range(nb)], np.int64))
    vptrs = dev(np.array([vpool.ptr + 2 * (misalign + blk * b) for b in range(nb)], np.int64))
    order = r.permutation(nb)
    slots = np.array([order[t // 16] * 16 + t % 16 for t in range(T)], np.int32)
    slots[T // 2] = -1
    dsl, dkn, dvn = dev(slots), dev(kn), dev(vn)
    ql.call("ql_paged_kv_append_f16", ptr(kptrs), ptr(vptrs), nb, ptr(dsl), ptr(dkn), ptr(dvn), T,
            layer, L, H, d, stream())
    wk = np.full(nb * blk + 8, 0xA5A5, np.uint16)
    wv = wk.copy()
    orc.paged_kv_append_inplace(wk, wv, (np.arange(nb) * blk + misalign).astype(np.int64), slots, kn,
                                vn, layer, L, H, d)
    assert np.array_equal(host(kpool), wk) and np.array_equal(host(vpool), wv)


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("dim", [4096, 4095])
def test_embed_empty_vocab_gives_zero_rows(f16, dim):
    # vocab 0: every id is out of range, so every row is zeros and no table row is read
    T = 9
    dt = np.uint16 if f16 else np.float32
    table = dev(np.ones(8, dt))                      # smaller than one row
    ids = dev(np.arange(T, dtype=np.int32))
    out = Out(T * dim, dt)
    ql.call("ql_embed_f16" if f16 else "ql_embed_f32", table.ptr, ids.ptr, T, 0, dim, out.ptr, stream())
    assert not np.any(out.get((T, dim)))


# ---- fp16 -> fp32 ------------------------------------------------------------------------------
# offsets in elements (input, output): 0 takes the 8-byte-load path, 4 (8-byte but not
# 16-byte aligned) too, 1 against 0 the per-element path; one offset for both: the
# leading elements up to the output's next 128-byte boundary in block 0, then
# vectors (fewer elements than that: the per-element path); n = 3 has no whole
# 4-element vector
@pytest.mark.parametrize("offset,n,out_offset", [(0, 65536, 0), (0, 32000, 0), (0, 13, 0), (4, 32003, 0),
                                                 (1, 1001, 0), (0, 3, 0), (1, 1001, 1), (17, 5000, 17),
                                                 (3, 20, 3), (5, 70001, 5)])
def test_f16_to_f32_bit_exact(offset, n, out_offset):
    h = (np.arange(n, dtype=np.uint32) * 7 % 65536).astype(np.uint16)
    out = Out(n, np.float32, offset=out_offset)
    dh = dev(h, offset)
    ql.call("ql_f16_to_f32", ptr(dh), out.ptr, n, stream())
    got, want = out.get(), orc.f16_to_f32(h)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


# ---- fp32 -> fp16 (the fp32 engine's quantized GEMM bridge) ------------------------------------
def _narrow_inputs():
    h = np.arange(0, 0x7bff, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    mid = ((lo + (h + 1).view(np.float16).astype(np.float64)) / 2).astype(np.float32)   # ties
    bits = np.random.default_rng(9).integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    special = np.array([65504.0, 65519.996, 65520.0, 1e9, 2.0 ** -24, 2.0 ** -25, 2.0 ** -14, -0.0,
                        np.inf, -np.inf, np.nan], np.float32)
    return np.concatenate([mid, -mid, np.nextafter(mid, np.float32(0)), bits.view(np.float32), special])


# (input offset, n, output offset) in elements: 16-byte-aligned input with an
# 8-byte-aligned output takes the vector path; one offset for both the leading
# elements up to the input's next 128-byte boundary in block 0, then vectors;
# different offsets otherwise the per-element path
@pytest.mark.parametrize("offset,n,out_offset", [(0, None, 0), (1, 1001, 1), (0, 13, 0), (0, 4099, 4),
                                                 (4, 2001, 4), (0, 3, 0), (31, 70001, 31), (2, 10, 2),
                                                 (1, 1001, 0)])
def test_f32_to_f16_bit_exact(offset, n, out_offset):
    x = _narrow_inputs()
    if n is not None:
        x = x[-n:]
    out = Out(x.size, np.uint16, offset=out_offset)
    dx = dev(x, offset_elems=offset)
    ql.call("ql_f32_to_f16", ptr(dx), out.ptr, x.size, stream())
    got, want = out.get(), orc.f32_to_f16(x)
    nan = np.isnan(x)
    assert np.all((got[nan] & 0x7c00) == 0x7c00) and np.all((got[nan] & 0x3ff) != 0)
    assert np.array_equal(got[~nan], want[~nan])


# ---- fused RoPE + KV-cache append ----------------------------------------------------------
def _pool(nb, blk, misalign=0):
    """Paged pool of nb blocks (+ slack for a misaligned table) and its device pointer table."""
    pool = empty((nb * blk + 16,), np.uint16, fill_bits=GUARD_BYTE)
    ptrs = dev(np.array([pool.ptr + 2 * misalign + 2 * blk * b for b in range(nb)], np.int64))
    return pool, ptrs


@pytest.mark.parametrize("pairing", [ql.ROPE_HALF, ql.ROPE_INTERLEAVED])
@pytest.mark.parametrize("T,H,HK,d,misalign", [(8192, 32, 8, 128, 0), (37, 4, 2, 64, 0),
                                               (20, 3, 1, 96, 0), (45, 4, 2, 64, 1),
                                               (45, 5, 3, 128, 1), (19, 2, 1, 128, 0),
                                               (33, 6, 2, 128, 0), (5, 120, 8, 128, 0),
                                               (21, 4, 2, 32, 0), (21, 4, 2, 32, 1),
                                               (13, 3, 1, 6, 0), (9, 2, 2, 256, 0)])   # per-pair loop
def test_rope_paged_kv_append_fused(pairing, T, H, HK, d, misalign):
    # One launch == ql_rope_f16 then ql_paged_kv_append_f16, bit for bit; and
    # both agree with the oracle (C5 shape: Q 32x128, K/V 8x128, theta 5e5).
    L, layer, theta = 4, 2, 5e5
    nb = (T + 15) // 16 + 2
    blk = L * 16 * HK * d
    r = np.random.default_rng(T + d)
    q = _f16(normal(T, (T, H * d)))
    k = _f16(normal(T + 1, (T, HK * d)))
    v = _f16(normal(T + 2, (T, HK * d)))
    order = r.permutation(nb)
    slots = np.array([order[t // 16] * 16 + t % 16 for t in range(T)], np.int32)
    slots[T // 3] = -1
    dsl, dv = dev(slots), dev(v)
    # fused
    q1, k1 = dev(q), dev(k)
    kp1, kb1 = _pool(nb, blk, misalign)
    vp1, vb1 = _pool(nb, blk, misalign)
    ql.call("ql_rope_paged_kv_append_f16", q1.ptr, k1.ptr, dv.ptr, T, H, HK, d, H * d, HK * d,
            HK * d, None, 0, theta, pairing, kb1.ptr, vb1.ptr, nb, dsl.ptr, layer, L, stream())
    # two steps
    q2, k2 = dev(q), dev(k)
    kp2, kb2 = _pool(nb, blk, misalign)
    vp2, vb2 = _pool(nb, blk, misalign)
    ql.call("ql_rope_f16", q2.ptr, k2.ptr, T, H, HK, d, H * d, HK * d, None, 0, theta, pairing,
            stream())
    ql.call("ql_paged_kv_append_f16", kb2.ptr, vb2.ptr, nb, dsl.ptr, k2.ptr, dv.ptr, T, layer, L,
            HK, d, stream())
    gq, gk = host(q1, shape=(T, H * d)), host(k1, shape=(T, HK * d))
    assert np.array_equal(gq, host(q2, shape=(T, H * d)))
    assert np.array_equal(gk, host(k2, shape=(T, HK * d)))
    assert np.array_equal(host(kp1), host(kp2)) and np.array_equal(host(vp1), host(vp2))
    # oracle: rotation within tolerance; cache rows are exact copies of the rotated K and V
    check_f16(gq, orc.rope(q, H, d, theta, pairing, f16=True), "fused rope q")
    check_f16(gk, orc.rope(k, HK, d, theta, pairing, f16=True), "fused rope k")
    wk = np.full(nb * blk + 16, 0xA5A5, np.uint16)
    wv = wk.copy()
    offs = (np.arange(nb) * blk + misalign).astype(np.int64)
    orc.paged_kv_append_inplace(wk, wv, offs, slots, gk, v, layer, L, HK, d)
    assert np.array_equal(host(kp1), wk) and np.array_equal(host(vp1), wv)


@pytest.mark.parametrize("pairing", [ql.ROPE_HALF, ql.ROPE_INTERLEAVED])
@pytest.mark.parametrize("T,H,HK,d,misalign", [(8192, 32, 8, 128, 0), (45, 5, 3, 128, 1),
                                               (37, 4, 2, 64, 0), (20, 3, 1, 96, 0)])
def test_rope_q_paged_kv_append_leaves_k(pairing, T, H, HK, d, misalign):
    # ql_rope_q_paged_kv_append_f16: Q and both pools exactly as the fused entry
    # point writes them; the caller's K rows are read and left unrotated.
    L, layer, theta = 4, 1, 5e5
    nb = (T + 15) // 16 + 1
    blk = L * 16 * HK * d
    q = _f16(normal(3 * T, (T, H * d)))
    k = _f16(normal(3 * T + 1, (T, HK * d)))
    v = _f16(normal(3 * T + 2, (T, HK * d)))
    order = np.random.default_rng(T).permutation(nb)
    slots = np.array([order[t // 16] * 16 + t % 16 for t in range(T)], np.int32)
    dsl, dv = dev(slots), dev(v)
    outs = []
    for name in ("ql_rope_paged_kv_append_f16", "ql_rope_q_paged_kv_append_f16"):
        dq, dk = dev(q), dev(k)
        kp, kb = _pool(nb, blk, misalign)
        vp, vb = _pool(nb, blk, misalign)
        ql.call(name, dq.ptr, dk.ptr, dv.ptr, T, H, HK, d, H * d, HK * d, HK * d, None, 0, theta,
                pairing, kb.ptr, vb.ptr, nb, dsl.ptr, layer, L, stream())
        outs.append((host(dq, shape=(T, H * d)), host(dk, shape=(T, HK * d)), host(kp), host(vp)))
    (q1, k1, kp1, vp1), (q2, k2, kp2, vp2) = outs
    assert np.array_equal(q1, q2) and np.array_equal(kp1, kp2) and np.array_equal(vp1, vp2)
    assert np.array_equal(k2, k), "K rows must be left as read"
    check_f16(k1, orc.rope(k, HK, d, theta, pairing, f16=True), "fused rope k")


# Q, K and V rows that interleave in one buffer (a fused QKV projection's output)
# run the plane kernel on an interleaved grid (every 16 token blocks of one plane
# group, then the same blocks of the next group); separate buffers keep the planes
# along the grid's y.  Both mappings must give the same bits: each case runs the
# entry point on views of one fused [T, (H + 2*HK)*d] buffer and on contiguous
# copies of the three planes, then checks the fused result against the oracle.
# T covers a partial last token block and a partial last group of 16 blocks.
@pytest.mark.parametrize("pairing", [ql.ROPE_HALF, ql.ROPE_INTERLEAVED])
@pytest.mark.parametrize("entry,T,H,HK,d", [
    ("paged", 8192, 32, 8, 128), ("paged", 77, 4, 2, 64), ("paged", 300, 8, 2, 128), ("paged", 1, 4, 1, 128),
    ("paged_q", 301, 8, 2, 128), ("paged_q", 65, 6, 2, 64),
    ("f32", 300, 8, 2, 128), ("f32", 77, 5, 5, 64), ("f16", 130, 8, 4, 64)])
def test_rope_on_fused_qkv_rows_matches_separate_buffers(entry, pairing, T, H, HK, d):
    L, layer, theta = 3, 1, 5e5
    row = (H + 2 * HK) * d
    f16 = entry != "f32"
    qkv = normal(T + d + H, (T, row))
    if f16:
        qkv = _f16(qkv)
    dt = np.uint16 if f16 else np.float32
    esz = np.dtype(dt).itemsize
    planes = [np.ascontiguousarray(qkv[:, a:b]) for a, b in ((0, H * d), (H * d, (H + HK) * d), ((H + HK) * d, row))]
    nb = (T + 15) // 16 + 1
    blk = L * 16 * HK * d
    slots = np.array([(nb - 1 - t // 16) * 16 + t % 16 for t in range(T)], np.int32)
    dsl = dev(slots)
    outs = []
    for fused in (True, False):
        if fused:
            base = dev(qkv)
            qp, kp, vp = base.ptr, base.ptr + H * d * esz, base.ptr + (H + HK) * d * esz
            qs = ks = vs = row
        else:
            bufs = [dev(x) for x in planes]
            qp, kp, vp = (b.ptr for b in bufs)
            qs, ks, vs = H * d, HK * d, HK * d
        pools = []
        if entry.startswith("paged"):
            kpool, kb = _pool(nb, blk)
            vpool, vb = _pool(nb, blk)
            pools = [kpool, vpool]
            name = "ql_rope_paged_kv_append_f16" if entry == "paged" else "ql_rope_q_paged_kv_append_f16"
            ql.call(name, qp, kp, vp, T, H, HK, d, qs, ks, vs, None, 0, theta, pairing, kb.ptr, vb.ptr, nb,
                    dsl.ptr, layer, L, stream())
        else:
            ql.call("ql_rope_f16" if f16 else "ql_rope_f32", qp, kp, T, H, HK, d, qs, ks, None, 0, theta,
                    pairing, stream())
        if fused:
            got = host(base, shape=(T, row))
            res = [got[:, :H * d], got[:, H * d:(H + HK) * d], got[:, (H + HK) * d:]]
        else:
            res = [host(b, shape=x.shape) for b, x in zip(bufs, planes)]
        outs.append([np.ascontiguousarray(x) for x in res] + [host(pp) for pp in pools])
    for i, (a, b) in enumerate(zip(*outs)):
        assert np.array_equal(a, b), f"output {i} differs between the fused and the separate layout"
    q_got, k_got, v_got = outs[0][:3]
    assert np.array_equal(v_got, planes[2])   # V is read, never written
    wq = orc.rope(planes[0], H, d, theta, pairing, f16=f16)
    if f16:
        check_f16(q_got, wq, "rope q on fused rows")
    else:
        check_abs(q_got, wq, ATOL_ROPE_F32, "rope q on fused rows")
    if entry == "paged_q":
        assert np.array_equal(k_got, planes[1]), "K rows must be left as read"
    else:
        wk = orc.rope(planes[1], HK, d, theta, pairing, f16=f16)
        if f16:
            check_f16(k_got, wk, "rope k on fused rows")
        else:
            check_abs(k_got, wk, ATOL_ROPE_F32, "rope k on fused rows")


@pytest.mark.parametrize("f16", [True, False])
@pytest.mark.parametrize("pairing", [ql.ROPE_HALF, ql.ROPE_INTERLEAVED])
@pytest.mark.parametrize("T,H,HK,d", [(300, 8, 2, 128), (33, 4, 4, 64), (17, 2, 1, 6),
                                      (29, 3, 3, 64), (31, 7, 1, 128), (23, 4, 2, 32), (11, 2, 1, 256)])
def test_rope_kv_append_fused_contiguous_from_fused_qkv(f16, pairing, T, H, HK, d):
    # Q, K, V are views into one fused [T, (H + 2*HK)*d] QKV buffer (strided rows);
    # the cache is [L, S, HK, d], tokens written at positions pos..pos+T-1.
    L, S, layer, pos, theta = 3, T + 40, 1, 25, 1e4
    row = (H + 2 * HK) * d
    qkv = normal(T * d, (T, row))
    if f16:
        qkv = _f16(qkv)
    dt = np.uint16 if f16 else np.float32
    esz = np.dtype(dt).itemsize
    base = dev(qkv)
    qp, kp, vp = base.ptr, base.ptr + H * d * esz, base.ptr + (H + HK) * d * esz
    n = L * S * HK * d
    kc, vc = Out(n, dt), Out(n, dt)
    name = "ql_rope_kv_append_f16" if f16 else "ql_rope_kv_append_f32"
    ql.call(name, qp, kp, vp, T, H, HK, d, row, row, row, None, pos, theta, pairing, kc.ptr, vc.ptr,
            layer, pos, S, L, stream())
    got = host(base, shape=(T, row))
    # reference: contiguous copies through the two separate entry points
    qc, kc2, vc2 = (np.ascontiguousarray(qkv[:, :H * d]), np.ascontiguousarray(qkv[:, H * d:(H + HK) * d]),
                    np.ascontiguousarray(qkv[:, (H + HK) * d:]))
    dq, dk, dvv = dev(qc), dev(kc2), dev(vc2)
    ql.call("ql_rope_f16" if f16 else "ql_rope_f32", dq.ptr, dk.ptr, T, H, HK, d, H * d, HK * d,
            None, pos, theta, pairing, stream())
    kref, vref = Out(n, dt), Out(n, dt)
    ql.call("ql_kv_append_f16" if f16 else "ql_kv_append_f32", kref.ptr, vref.ptr, dk.ptr, dvv.ptr,
            layer, pos, T, HK, d, S, L, stream())
    assert np.array_equal(got[:, :H * d], host(dq, shape=(T, H * d)))
    assert np.array_equal(got[:, H * d:(H + HK) * d], host(dk, shape=(T, HK * d)))
    assert np.array_equal(got[:, (H + HK) * d:], qkv[:, (H + HK) * d:])  # V untouched
    assert np.array_equal(kc.get(), kref.get()) and np.array_equal(vc.get(), vref.get())
    # and against the oracle
    wq = orc.rope(qc, H, d, theta, pairing, pos_offset=pos, f16=f16)
    if f16:
        check_f16(got[:, :H * d], wq, "fused contiguous q")
    else:
        check_abs(got[:, :H * d], wq, ATOL_ROPE_F32, "fused contiguous q")
