"""ql_paged_decode_attention_f16_noalloc: the split decode with its partials in
the library's static device array instead of a caller workspace.  Checked
through the C ABI against ql_paged_decode_attention_f16 given the queried
workspace (same split, same kernels: bit for bit) and against the oracle, on
calls in a row whose second (and third) input is smaller, so stale partials of
an earlier call must not leak into a later one."""
import ctypes

import numpy as np
import pytest

import oracle as orc
import quantlib_amd as ql
from helpers import Out, dev, empty, stream
from test_gpu_attention import _decode_setup, check_attn

pytestmark = pytest.mark.gpu


def _split_bytes(S, h, hkv, d, C):
    size = ctypes.c_size_t()
    ql.call("ql_paged_decode_workspace_size", S, h, hkv, d, C, ctypes.addressof(size))
    return size.value


def _run(entry, case, with_ws):
    pool, bt, ks, vs, q, ctx, h, hkv, d, L, layer = case
    S = len(ctx)
    dq, dctx, dbt = dev(q), dev(np.array(ctx, np.int32)), dev(bt)
    out = Out(S * h * d, np.uint16)
    args = [dq.ptr, out.ptr, h * d, h * d, S, dctx.ptr, max(ctx), dbt.ptr, bt.shape[1],
            pool.kptrs.ptr, pool.vptrs.ptr, pool.nb, layer, L, h, hkv, d]
    if with_ws:
        n = _split_bytes(S, h, hkv, d, max(ctx))
        ws = empty((max(n, 16),), np.uint8, fill_bits=0x7F)
        args += [ws.ptr if n else None, n]
    ql.call(entry, *args, stream())
    return out.get((S, h, d))


def _case(ctx, h, hkv, d, seed, L=2, layer=1):
    pool, bt, ks, vs, q = _decode_setup(ctx, h, hkv, d, L, layer, seed)
    return (pool, bt, ks, vs, q, ctx, h, hkv, d, L, layer)


def test_noalloc_decode_matches_workspace_entry_point():
    cases = [
        _case([4096 - 61 * i for i in range(8)], 32, 8, 128, 0x51A100A1),   # 8 splits
        _case([1000, 17, 513], 32, 8, 128, 0x51A100A2),                     # smaller: 4 splits
        _case([300, 1, 0, 40], 8, 2, 64, 0x51A100A3),                       # head_dim 64, 2 splits
        _case([64 + i for i in range(64)], 32, 8, 128, 0x51A100A4),         # one pass, no scratch
    ]
    for i, case in enumerate(cases):
        pool, bt, ks, vs, q, ctx, h, hkv, d, L, layer = case
        assert _split_bytes(len(ctx), h, hkv, d, max(ctx)) <= ql.DECODE_SCRATCH_BYTES
        got = _run("ql_paged_decode_attention_f16_noalloc", case, False)
        ref = _run("ql_paged_decode_attention_f16", case, True)
        assert np.array_equal(got, ref), f"call {i}: differs from the workspace entry point"
        for s in range(len(ctx)):
            want = orc.attention(q[s:s + 1], ks[s], vs[s], h, hkv, True, f16=True)
            check_attn(got[s:s + 1], want, vs[s], f"noalloc call {i} seq {s} ctx {ctx[s]}")
    # the first case again after the smaller ones: same bits
    assert np.array_equal(_run("ql_paged_decode_attention_f16_noalloc", cases[0], False),
                          _run("ql_paged_decode_attention_f16", cases[0], True))


def test_noalloc_decode_rejects_splits_beyond_the_scratch():
    # 511 sequences x 16 query heads on one KV head at head_dim 128: two splits of
    # 511*16*130 floats each exceed the array; refused on the host, nothing launched
    S, h, hkv, d, C = 511, 16, 1, 128, 4096
    assert _split_bytes(S, h, hkv, d, C) > ql.DECODE_SCRATCH_BYTES
    P = 4096
    rc = ql.raw("ql_paged_decode_attention_f16_noalloc", P, P, h * d, h * d, S, P, C, P, 256,
                P, P, 4096, 0, 1, h, hkv, d, None)
    assert rc == ql.HIP_ERROR_INVALID_VALUE
