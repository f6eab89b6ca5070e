"""GPU parity of the fp16 attention entry points (ql_flash_attention_f16,
ql_attention_f16, ql_paged_attention_f16 and the launch_flash_attention shim)
against the CPU oracle (double-precision softmax . V) on the same seeded
binary16 inputs.

Tolerance, |got - want| <= RTOL_ATTN*|want| + ATOL_ATTN*max|V|: the kernel
multiplies V by the probabilities rounded to binary16 (relative error <= 2^-11
each; the row sum uses the same rounded values, so the output is a convex
combination whose weights are off by <= 2^-10 relative, i.e. <= 2^-10*max|V|
absolute), accumulates in fp32 and rounds the result to binary16 (2^-11
relative).  Probabilities below the binary16 subnormal range add at most
kv_len*2^-25 of weight, well inside the bound at these sizes.

Paged and contiguous K/V run the same arithmetic, so their outputs must agree
bit for bit.  At the C5 shape (8192 tokens, 32 query heads, 8 KV heads,
head_dim 128, causal) the oracle checks sampled rows: query i of a causal
prefill equals a one-query problem over keys 0..i."""
import ctypes

import numpy as np
import pytest

import oracle as orc
import quantlib_amd as ql
from helpers import (GUARD_BYTE, Out, check_close, dev, empty, f16_bits_to_f32, host, normal,
                     ptr, stream, to_f16_bits)
from test_abi import COMPAT_MANGLED

pytestmark = pytest.mark.gpu

RTOL_ATTN = 2e-3
ATOL_ATTN = 2e-3   # times max|V|


def check_attn(got, want, v, what):
    vmax = float(np.abs(f16_bits_to_f32(v)).max()) if v.size else 1.0
    return check_close(f16_bits_to_f32(got), f16_bits_to_f32(want), RTOL_ATTN,
                       ATOL_ATTN * max(vmax, 1e-3), what)


def qkv(seed, q_len, kv_len, h, hkv, d, q_sigma=1.0):
    return (to_f16_bits(normal(seed, (q_len, h, d), q_sigma)),
            to_f16_bits(normal(seed + 1, (kv_len, hkv, d))),
            to_f16_bits(normal(seed + 2, (kv_len, hkv, d))))


# ---- reference semantics (launch_flash_attention) -------------------------------------------
@pytest.mark.parametrize("seq,h,hkv,d,causal,q_sigma", [
    (1, 4, 2, 64, 1, 1.0), (7, 4, 1, 128, 1, 1.0), (64, 8, 2, 64, 0, 1.0),
    (100, 32, 8, 128, 1, 1.0), (129, 6, 4, 64, 1, 3.0), (257, 4, 4, 128, 0, 3.0),
    (300, 8, 8, 128, 1, 0.3), (513, 32, 8, 128, 1, 1.0), (200, 32, 4, 64, 1, 1.0)])
def test_flash_attention_matches_oracle(seq, h, hkv, d, causal, q_sigma):
    q, k, v = qkv(seq * 7 + d, seq, seq, h, hkv, d, q_sigma)
    out = Out(seq * h * d, np.uint16)
    dq, dk, dv = dev(q), dev(k), dev(v)
    ql.call("ql_flash_attention_f16", ptr(dq), ptr(dk), ptr(dv), out.ptr, seq, h, hkv, d, causal,
            stream())
    want = orc.attention(q, k, v, h, hkv, bool(causal), f16=True)
    check_attn(out.get((seq, h, d)), want, v, f"flash attention seq={seq} h={h}/{hkv} d={d}")


def test_flash_attention_passes_reference_test():
    # tests/test_attention.cu:60-141: srand(99) U(-0.5,0.5) [128, 32, 128], no mask,
    # max abs error < 1e-3 against its fp32 CPU loop (inputs here rounded to binary16)
    seq, h, d = 128, 32, 128
    q, k, v = orc.reftest_attention_inputs(seq, h, d, 99)
    qb, kb, vb = to_f16_bits(q), to_f16_bits(k), to_f16_bits(v)
    out = Out(seq * h * d, np.uint16)
    dq, dk, dv = dev(qb), dev(kb), dev(vb)
    ql.call("ql_flash_attention_f16", ptr(dq), ptr(dk), ptr(dv), out.ptr, seq, h, h, d, 0, stream())
    got = out.get((seq, h, d))
    err = float(np.abs(f16_bits_to_f32(got) - orc.attention_reftest_cpu(q, k, v, h)).max())
    assert err < 1e-3, err
    check_attn(got, orc.attention(qb, kb, vb, h, h, False, f16=True), vb, "reference test")


def test_launch_flash_attention_shim_tinyllama_shape():
    # the reference's own shape: TinyLlama 32 query heads, 4 KV heads, head_dim 64
    seq, h, hkv, d = 77, 32, 4, 64
    f = getattr(ql.lib(), COMPAT_MANGLED["launch_flash_attention"])
    f.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 5 + [ctypes.c_void_p]
    f.restype = None
    q, k, v = qkv(77, seq, seq, h, hkv, d)
    dq, dk, dv = dev(q), dev(k), dev(v)
    o1, o2 = Out(seq * h * d, np.uint16), Out(seq * h * d, np.uint16)
    f(ptr(dq), ptr(dk), ptr(dv), o1.ptr, seq, h, hkv, d, 1, stream())
    ql.call("ql_flash_attention_f16", ptr(dq), ptr(dk), ptr(dv), o2.ptr, seq, h, hkv, d, 1,
            stream())
    g1 = o1.get((seq, h, d))
    assert np.array_equal(g1, o2.get((seq, h, d)))
    check_attn(g1, orc.attention(q, k, v, h, hkv, True, f16=True), v, "launch_flash_attention")


# ---- head_dims below 64 (the reference kernel's range) ---------------------------------------
# The reference's launch_flash_attention takes any head_dim <= 64
# (kernels/flash_attention.cu:25-27,64-66); 64 and 128 run on the matrix cores, and
# so does a prefill over heads of a multiple of 8 (zero-padded to 64 in the tiles);
# every other value, and one-query calls, run attn_small, whose probabilities stay
# fp32 (tighter than the bound above).  The shim and the C ABI must give the same bits.
@pytest.mark.parametrize("seq,h,hkv,d,causal", [
    (1, 4, 2, 32, 1), (77, 32, 4, 32, 1), (300, 8, 2, 48, 1), (129, 6, 3, 40, 0),
    (513, 4, 4, 16, 1), (65, 2, 1, 8, 1), (100, 3, 1, 63, 0), (257, 4, 2, 1, 1), (64, 4, 1, 33, 1),
    (200, 6, 2, 24, 1), (131, 4, 4, 56, 0), (1000, 8, 1, 32, 1), (2, 3, 3, 8, 0), (90, 4, 2, 20, 1)])
def test_flash_attention_small_head_dims(seq, h, hkv, d, causal):
    f = getattr(ql.lib(), COMPAT_MANGLED["launch_flash_attention"])
    f.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 5 + [ctypes.c_void_p]
    f.restype = None
    q, k, v = qkv(seq * 11 + d, seq, seq, h, hkv, d)
    dq, dk, dv = dev(q), dev(k), dev(v)
    o1, o2 = Out(seq * h * d, np.uint16), Out(seq * h * d, np.uint16)
    f(ptr(dq), ptr(dk), ptr(dv), o1.ptr, seq, h, hkv, d, causal, stream())
    ql.call("ql_flash_attention_f16", ptr(dq), ptr(dk), ptr(dv), o2.ptr, seq, h, hkv, d, causal,
            stream())
    g1 = o1.get((seq, h, d))
    assert np.array_equal(g1, o2.get((seq, h, d)))
    check_attn(g1, orc.attention(q, k, v, h, hkv, bool(causal), f16=True), v,
               f"head_dim {d} seq={seq} h={h}/{hkv}")


def test_flash_attention_small_head_dim_reference_test_inputs():
    # tests/test_attention.cu's srand(99) U(-0.5,0.5) inputs and 1e-3 bar at head_dim 32
    seq, h, d = 128, 8, 32
    q, k, v = orc.reftest_attention_inputs(seq, h, d, 99)
    qb, kb, vb = to_f16_bits(q), to_f16_bits(k), to_f16_bits(v)
    out = Out(seq * h * d, np.uint16)
    dq, dk, dv = dev(qb), dev(kb), dev(vb)
    ql.call("ql_flash_attention_f16", ptr(dq), ptr(dk), ptr(dv), out.ptr, seq, h, h, d, 0, stream())
    got = out.get((seq, h, d))
    err = float(np.abs(f16_bits_to_f32(got) - orc.attention_reftest_cpu(q, k, v, h)).max())
    assert err < 1e-3, err


@pytest.mark.parametrize("q_len,kv_len,causal", [(1, 1000, 1), (5, 77, 1), (130, 333, 0), (3, 0, 1)])
def test_attention_small_head_dim_strided_unaligned(q_len, kv_len, causal):
    # head_dim 40 with row strides that are not multiples of 8 elements and base
    # pointers 2 bytes past a 16-byte boundary; out padding stays untouched
    h, hkv, d = 6, 2, 40
    qrow, kvrow, orow = h * d + 3, hkv * d + 5, h * d + 7
    qbuf = to_f16_bits(normal(q_len + 5, (q_len * qrow + 1,)))
    kbuf = to_f16_bits(normal(kv_len + 6, (max(kv_len, 1) * kvrow + 1,)))
    vbuf = to_f16_bits(normal(kv_len + 7, (max(kv_len, 1) * kvrow + 1,)))
    dq, dk, dv = dev(qbuf), dev(kbuf), dev(vbuf)
    out = Out(q_len * orow + 1, np.uint16)
    ql.call("ql_attention_f16", ptr(dq) + 2, ptr(dk) + 2, ptr(dv) + 2, out.ptr + 2, q_len, kv_len, h, hkv,
            d, qrow, kvrow, orow, causal, stream())
    got = out.get()
    body = got[1:].reshape(q_len, orow)
    assert got[0] == np.frombuffer(bytes([GUARD_BYTE] * 2), np.uint16)[0]
    assert np.all(body[:, h * d:].view(np.uint8) == GUARD_BYTE), "padding columns written"
    q = qbuf[1:].reshape(q_len, qrow)[:, :h * d].reshape(q_len, h, d)
    k = kbuf[1:1 + kv_len * kvrow].reshape(kv_len, kvrow)[:, :hkv * d].reshape(kv_len, hkv, d)
    v = vbuf[1:1 + kv_len * kvrow].reshape(kv_len, kvrow)[:, :hkv * d].reshape(kv_len, hkv, d)
    want = orc.attention(np.ascontiguousarray(q), np.ascontiguousarray(k), np.ascontiguousarray(v), h, hkv,
                         bool(causal), f16=True)
    check_attn(body[:, :h * d].reshape(q_len, h, d), want, v, f"head_dim 40 q={q_len} kv={kv_len}")


@pytest.mark.parametrize("d", [16, 32, 48, 8, 56, 12, 20, 36])
def test_paged_attention_small_head_dims(d):
    # prefill, decode and a chunk over permuted blocks with a hole in one table,
    # through ql_paged_attention_f16, then every sequence decoding through both
    # paged decode entry points (one pass, no workspace at these head_dims)
    h, hkv, L, layer = 8, 2, 3, 2
    ctx, qn = [150, 70, 33], [150, 1, 9]
    need = [(c + 15) // 16 for c in ctx]
    nb = sum(need) + 2
    perm = np.random.default_rng(d).permutation(nb)
    max_blocks = max(need) + 1
    bt = np.full((3, max_blocks), -1, np.int32)
    o = 0
    for s, n in enumerate(need):
        bt[s, :n] = perm[o:o + n]
        o += n
    pool = PagedPool(nb, L, hkv, d)
    ks, vs, qs = [], [], []
    for s, c in enumerate(ctx):
        ks.append(to_f16_bits(normal(400 + s + d, (c, hkv, d))))
        vs.append(to_f16_bits(normal(500 + s + d, (c, hkv, d))))
        pool.append(bt[s], ks[s], vs[s], layer)
        qs.append(to_f16_bits(normal(600 + s + d, (qn[s], h, d))))
    bt[0, 3] = -1          # sequence 0: keys 48..63 read as zero rows
    kz, vz = [k.copy() for k in ks], [v.copy() for v in vs]
    kz[0][48:64] = 0
    vz[0][48:64] = 0
    cu = np.concatenate([[0], np.cumsum(qn)]).astype(np.int32)
    rows = int(cu[-1])
    dq, dcu, dctx, dbt = dev(np.concatenate(qs)), dev(cu), dev(np.array(ctx, np.int32)), dev(bt)
    out = Out(rows * h * d, np.uint16)
    ql.call("ql_paged_attention_f16", dq.ptr, out.ptr, h * d, h * d, rows, 3, dcu.ptr, dctx.ptr, max(qn),
            dbt.ptr, max_blocks, pool.kptrs.ptr, pool.vptrs.ptr, nb, layer, L, h, hkv, d, 1, stream())
    got = out.get((rows, h, d))
    for s in range(3):
        check_attn(got[cu[s]:cu[s + 1]], orc.attention(qs[s], kz[s], vz[s], h, hkv, True, f16=True), vs[s],
                   f"paged head_dim {d} sequence {s}")
    # decode: one query per sequence (row s), against all ctx[s] keys
    qd = to_f16_bits(normal(700 + d, (3, h, d)))
    dqd = dev(qd)
    size = ctypes.c_size_t(1)
    ql.call("ql_paged_decode_workspace_size", 3, h, hkv, d, max(ctx), ctypes.addressof(size))
    assert size.value == 0
    o1, o2 = Out(3 * h * d, np.uint16), Out(3 * h * d, np.uint16)
    ql.call("ql_paged_decode_attention_f16", dqd.ptr, o1.ptr, h * d, h * d, 3, dctx.ptr, max(ctx), dbt.ptr,
            max_blocks, pool.kptrs.ptr, pool.vptrs.ptr, nb, layer, L, h, hkv, d, None, 0, stream())
    ql.call("ql_paged_decode_attention_f16_noalloc", dqd.ptr, o2.ptr, h * d, h * d, 3, dctx.ptr, max(ctx),
            dbt.ptr, max_blocks, pool.kptrs.ptr, pool.vptrs.ptr, nb, layer, L, h, hkv, d, stream())
    g1 = o1.get((3, h, d))
    assert np.array_equal(g1, o2.get((3, h, d)))
    for s in range(3):
        check_attn(g1[s:s + 1], orc.attention(qd[s:s + 1], kz[s], vz[s], h, hkv, True, f16=True), vs[s],
                   f"paged decode head_dim {d} sequence {s}")


@pytest.mark.parametrize("h,hkv,d,kv", [(16, 4, 32, 3000), (8, 8, 8, 65), (32, 8, 16, 1), (6, 2, 24, 500),
                                        (12, 3, 40, 4097), (4, 1, 48, 33), (20, 4, 56, 2000), (16, 4, 36, 700)])
def test_contiguous_decode_small_head_dim(h, hkv, d, kv):
    # ql_decode_attention_f16 (no workspace needed) equals ql_attention_f16 with one
    # query, and the oracle: heads of a multiple of 8 on the head_dim-64 decode
    # kernel, zero-padded; 36 on attn_small
    q, k, v = qkv(31, 1, kv, h, hkv, d)
    dq, dk, dv = dev(q), dev(k), dev(v)
    o1, o2 = Out(h * d, np.uint16), Out(h * d, np.uint16)
    ql.call("ql_decode_attention_f16", dq.ptr, dk.ptr, dv.ptr, o1.ptr, kv, h, hkv, d, hkv * d, None, 0,
            stream())
    ql.call("ql_attention_f16", dq.ptr, dk.ptr, dv.ptr, o2.ptr, 1, kv, h, hkv, d, h * d, hkv * d, h * d, 1,
            stream())
    g1 = o1.get((1, h, d))
    assert np.array_equal(g1, o2.get((1, h, d)))
    check_attn(g1, orc.attention(q, k, v, h, hkv, True, f16=True), v, f"decode head_dim {d} kv={kv}")


# ---- decode / chunked prefill over a contiguous cache, strided rows -----------------------
@pytest.mark.parametrize("q_len,kv_len", [(1, 1), (1, 1000), (5, 77), (130, 333), (64, 64),
                                          (3, 0)])
@pytest.mark.parametrize("causal", [1, 0])
def test_attention_last_positions_strided(q_len, kv_len, causal):
    # Q rows inside a fused [q_len, (H + 2*HK)*d] QKV buffer; K/V one layer of a
    # [L, S, HK, d] cache; out rows padded (the padding must stay untouched)
    h, hkv, d, L, S, layer = 8, 2, 128, 3, max(kv_len, 1) + 16, 1
    qrow = (h + 2 * hkv) * d
    orow = h * d + 64
    qkvbuf = to_f16_bits(normal(q_len + kv_len, (q_len, qrow)))
    kc = to_f16_bits(normal(kv_len + 1, (L, S, hkv, d)))
    vc = to_f16_bits(normal(kv_len + 2, (L, S, hkv, d)))
    dq, dk, dv = dev(qkvbuf), dev(kc), dev(vc)
    layer_off = 2 * layer * S * hkv * d
    out = Out(q_len * orow, np.uint16)
    ql.call("ql_attention_f16", ptr(dq), ptr(dk) + layer_off, ptr(dv) + layer_off, out.ptr, q_len,
            kv_len, h, hkv, d, qrow, hkv * d, orow, causal, stream())
    got = out.get((q_len, orow))
    assert np.all(got[:, h * d:].view(np.uint8) == GUARD_BYTE), "padding columns written"
    q = np.ascontiguousarray(qkvbuf[:, :h * d]).reshape(q_len, h, d)
    k, v = kc[layer, :kv_len], vc[layer, :kv_len]
    want = orc.attention(q, k, v, h, hkv, bool(causal), f16=True)
    check_attn(got[:, :h * d].reshape(q_len, h, d), want, v, f"attention q={q_len} kv={kv_len}")


# ---- paged KV cache -------------------------------------------------------------------------
class PagedPool:
    """Device pool of nb blocks [L, 16, HK, d] (K and V), written through
    ql_paged_kv_append_f16 from per-sequence block tables."""

    def __init__(self, nb, L, hkv, d, offset_elems=0):
        # offset_elems > 0 starts every block that many elements past a 16-byte
        # boundary (a caller-provided pool with misaligned block pointers)
        self.nb, self.L, self.hkv, self.d = nb, L, hkv, d
        self.blk = L * 16 * hkv * d
        self.kpool = empty((nb * self.blk + offset_elems,), np.uint16, fill_bits=GUARD_BYTE)
        self.vpool = empty((nb * self.blk + offset_elems,), np.uint16, fill_bits=GUARD_BYTE)
        self.kptrs = dev(np.array([self.kpool.ptr + 2 * (self.blk * b + offset_elems) for b in range(nb)],
                                  np.int64))
        self.vptrs = dev(np.array([self.vpool.ptr + 2 * (self.blk * b + offset_elems) for b in range(nb)],
                                  np.int64))

    def append(self, table, k, v, layer):
        n = k.shape[0]
        if n == 0:
            return
        slots = np.array([table[t // 16] * 16 + t % 16 for t in range(n)], np.int32)
        dsl, dk, dv = dev(slots), dev(k), dev(v)
        ql.call("ql_paged_kv_append_f16", self.kptrs.ptr, self.vptrs.ptr, self.nb, dsl.ptr, dk.ptr,
                dv.ptr, n, layer, self.L, self.hkv, self.d, stream())


@pytest.mark.parametrize("h,hkv,d", [(32, 8, 128), (8, 2, 64), (4, 4, 128)])
def test_paged_attention_varlen_matches_contiguous_and_oracle(h, hkv, d):
    # three sequences in one launch: a 200-token prefill, a decode step at
    # context 333, a 17-token chunk at context 150; permuted physical blocks
    L, layer = 4, 3
    ctx = [200, 333, 150]
    qn = [200, 1, 17]
    r = np.random.default_rng(h * d)
    need = [(c + 15) // 16 for c in ctx]
    nb = sum(need) + 3
    perm = r.permutation(nb)
    tables, o = [], 0
    for n in need:
        tables.append(perm[o:o + n])
        o += n
    max_blocks = max(need) + 2
    bt = np.full((len(ctx), max_blocks), -1, np.int32)
    for s, t in enumerate(tables):
        bt[s, :len(t)] = t
    pool = PagedPool(nb, L, hkv, d)
    ks, vs, qs = [], [], []
    for s, c in enumerate(ctx):
        k = to_f16_bits(normal(100 + s, (c, hkv, d)))
        v = to_f16_bits(normal(200 + s, (c, hkv, d)))
        pool.append(bt[s], k, v, layer)
        ks.append(k)
        vs.append(v)
        qs.append(to_f16_bits(normal(300 + s, (qn[s], h, d))))
    cu = np.concatenate([[0], np.cumsum(qn)]).astype(np.int32)
    rows = int(cu[-1])
    qall = np.concatenate(qs)
    dq = dev(qall)
    out = Out(rows * h * d, np.uint16)
    dcu, dctx, dbt = dev(cu), dev(np.array(ctx, np.int32)), dev(bt)
    ql.call("ql_paged_attention_f16", dq.ptr, out.ptr, h * d, h * d, rows, len(ctx), dcu.ptr,
            dctx.ptr, max(qn), dbt.ptr, max_blocks, pool.kptrs.ptr, pool.vptrs.ptr, nb, layer, L,
            h, hkv, d, 1, stream())
    got = out.get((rows, h, d))
    for s in range(len(ctx)):
        mine = got[cu[s]:cu[s + 1]]
        # same sequence through the contiguous entry point: bit-identical
        dqs, dks, dvs = dev(qs[s]), dev(ks[s]), dev(vs[s])
        ref = Out(qn[s] * h * d, np.uint16)
        ql.call("ql_attention_f16", dqs.ptr, dks.ptr, dvs.ptr, ref.ptr, qn[s], ctx[s], h, hkv, d,
                h * d, hkv * d, h * d, 1, stream())
        if qn[s] > 1:   # (a one-query call runs the decode kernel: compared to the oracle only)
            assert np.array_equal(mine, ref.get((qn[s], h, d))), f"paged != contiguous, sequence {s}"
        want = orc.attention(qs[s], ks[s], vs[s], h, hkv, True, f16=True)
        check_attn(mine, want, vs[s], f"paged attention sequence {s}")


def test_paged_attention_skips_bad_rows_and_missing_blocks():
    # sequence 0 claims rows beyond n_q_rows: skipped (its rows keep the guard);
    # sequence 1's table has a hole (-1): those 16 keys read as zero rows
    h, hkv, d, L, layer = 4, 2, 64, 1, 0
    pool = PagedPool(4, L, hkv, d)
    k = to_f16_bits(normal(1, (40, hkv, d)))
    v = to_f16_bits(normal(2, (40, hkv, d)))
    table = np.array([2, 0, 3], np.int32)
    pool.append(table, k, v, layer)
    bt = np.array([[1, -1, -1], [2, -1, 3]], np.int32)
    cu = np.array([3, 9, 4], np.int32)     # seq 0: rows 3..8 (> n_q_rows 4); seq 1: rows 9..3 (empty)
    q = to_f16_bits(normal(3, (4, h, d)))
    dq, dcu = dev(q), dev(cu)
    dctx, dbt = dev(np.array([40, 40], np.int32)), dev(bt)
    out = Out(4 * h * d, np.uint16)
    ql.call("ql_paged_attention_f16", dq.ptr, out.ptr, h * d, h * d, 4, 2, dcu.ptr, dctx.ptr, 8,
            dbt.ptr, 3, pool.kptrs.ptr, pool.vptrs.ptr, 4, layer, L, h, hkv, d, 1, stream())
    assert np.all(out.get().view(np.uint8) == GUARD_BYTE)
    # one valid sequence over the holed table: keys 16..31 are zeros
    cu = np.array([0, 4], np.int32)
    dcu = dev(cu)
    dbt = dev(np.array([[2, -1, 3]], np.int32))
    ql.call("ql_paged_attention_f16", dq.ptr, out.ptr, h * d, h * d, 4, 1, dcu.ptr, dctx.ptr, 4,
            dbt.ptr, 3, pool.kptrs.ptr, pool.vptrs.ptr, 4, layer, L, h, hkv, d, 1, stream())
    kz, vz = k.copy(), v.copy()
    kz[16:32] = 0
    vz[16:32] = 0
    check_attn(out.get((4, h, d)), orc.attention(q, kz, vz, h, hkv, True, f16=True), v, "holed table")


@pytest.mark.parametrize("d", [64, 128, 32])
def test_paged_prefill_tile_with_one_missing_page(d):
    # 200-token causal prefill over 13 permuted blocks whose table misses page 5
    # (keys 80..95, the second page of the second 64-key tile): in that tile one
    # wavefront's page takes the checked loads and reads zero rows while the
    # other three load their pages unchecked; the last tile is partial (keys
    # 192..199).  Oracle: the same attention with K/V rows 80..95 zeroed.
    h, hkv, L, layer, n = 8, 2, 2, 1, 200
    pool = PagedPool(16, L, hkv, d)
    k = to_f16_bits(normal(71 + d, (n, hkv, d)))
    v = to_f16_bits(normal(72 + d, (n, hkv, d)))
    table = np.random.default_rng(d).permutation(16)[:13].astype(np.int32)
    pool.append(table, k, v, layer)
    bt = table.copy()
    bt[5] = -1
    q = to_f16_bits(normal(73 + d, (n, h, d)))
    dq, dcu, dctx, dbt = dev(q), dev(np.array([0, n], np.int32)), dev(np.array([n], np.int32)), dev(bt[None, :])
    out = Out(n * h * d, np.uint16)
    ql.call("ql_paged_attention_f16", dq.ptr, out.ptr, h * d, h * d, n, 1, dcu.ptr, dctx.ptr, n,
            dbt.ptr, 13, pool.kptrs.ptr, pool.vptrs.ptr, 16, layer, L, h, hkv, d, 1, stream())
    kz, vz = k.copy(), v.copy()
    kz[80:96] = 0
    vz[80:96] = 0
    check_attn(out.get((n, h, d)), orc.attention(q, kz, vz, h, hkv, True, f16=True), v,
               f"d={d} tile with one missing page")


@pytest.mark.parametrize("d", [64, 128, 24])
def test_paged_attention_misaligned_block_pointers(d):
    # block pointers 2 bytes past a 16-byte boundary take the element-wise load
    # path: prefill and decode give the same bits as over an aligned pool, and
    # match the oracle (holes in the table still read as zero rows)
    h, hkv, L, layer = 8, 2, 2, 1
    ctx, qn = [150, 77, 40], [150, 20, 1]
    need = [(c + 15) // 16 for c in ctx]
    nb = sum(need) + 1
    perm = np.random.default_rng(d).permutation(nb)
    bt = np.full((len(ctx), max(need) + 1), -1, np.int32)
    o = 0
    for s, n in enumerate(need):
        bt[s, :n] = perm[o:o + n]
        o += n
    bt[2, 1] = -1   # sequence 2: keys 16..31 have no block
    ks = [to_f16_bits(normal(400 + s, (c, hkv, d))) for s, c in enumerate(ctx)]
    vs = [to_f16_bits(normal(500 + s, (c, hkv, d))) for s, c in enumerate(ctx)]
    qs = [to_f16_bits(normal(600 + s, (n, h, d))) for s, n in enumerate(qn)]
    cu = np.concatenate([[0], np.cumsum(qn)]).astype(np.int32)
    rows = int(cu[-1])
    dq, dcu, dctx, dbt = dev(np.concatenate(qs)), dev(cu), dev(np.array(ctx, np.int32)), dev(bt)
    dq1 = dev(np.stack([q[-1] for q in qs]))   # each sequence's last query, for the decode call
    got = {}
    for off in (0, 1):
        pool = PagedPool(nb, L, hkv, d, offset_elems=off)
        for s in range(len(ctx)):
            pool.append(bt[s], ks[s], vs[s], layer)
        out = Out(rows * h * d, np.uint16)
        ql.call("ql_paged_attention_f16", dq.ptr, out.ptr, h * d, h * d, rows, len(ctx), dcu.ptr,
                dctx.ptr, max(qn), dbt.ptr, bt.shape[1], pool.kptrs.ptr, pool.vptrs.ptr, nb, layer, L,
                h, hkv, d, 1, stream())
        dec = Out(len(ctx) * h * d, np.uint16)
        ql.call("ql_paged_decode_attention_f16", dq1.ptr, dec.ptr, h * d, h * d, len(ctx), dctx.ptr,
                max(ctx), dbt.ptr, bt.shape[1], pool.kptrs.ptr, pool.vptrs.ptr, nb, layer, L, h, hkv,
                d, None, 0, stream())
        got[off] = (out.get((rows, h, d)), dec.get((len(ctx), h, d)))
    assert np.array_equal(got[0][0], got[1][0]), "prefill: misaligned pool != aligned pool"
    assert np.array_equal(got[0][1], got[1][1]), "decode: misaligned pool != aligned pool"
    for s in range(len(ctx)):
        k, v = ks[s].copy(), vs[s].copy()
        if s == 2:
            k[16:32] = 0
            v[16:32] = 0
        want = orc.attention(qs[s], k, v, h, hkv, True, f16=True)
        check_attn(got[1][0][cu[s]:cu[s + 1]], want, v, f"misaligned pool prefill seq {s}")
        check_attn(got[1][1][s:s + 1], want[-1:], v, f"misaligned pool decode seq {s}")


# ---- C5 shape: 8192-token causal prefill, GQA 32/8, head_dim 128 ---------------------------
def test_attention_c5_prefill_sampled_rows_and_paged_equivalence():
    T, h, hkv, d, L, layer = 8192, 32, 8, 128, 2, 1
    q, k, v = qkv(0x51A10070, T, T, h, hkv, d)
    dq, dk, dv = dev(q), dev(k), dev(v)
    out = Out(T * h * d, np.uint16)
    ql.call("ql_flash_attention_f16", ptr(dq), ptr(dk), ptr(dv), out.ptr, T, h, hkv, d, 1,
            stream())
    got = out.get((T, h, d))
    rows = [0, 1, 31, 32, 63, 64, 127, 128, 1000, 4095, 4096, 6143, 8190, 8191]
    rows += list(np.random.default_rng(5).integers(0, T, 6))
    for i in rows:
        want = orc.attention(q[i:i + 1], k[:i + 1], v[:i + 1], h, hkv, True, f16=True)
        check_attn(got[i:i + 1], want, v, f"C5 prefill row {i}")
    # the same K/V in a paged pool (fresh-pool block order) gives identical bits
    nb = T // 16
    pool = PagedPool(nb, L, hkv, d)
    table = np.arange(nb, dtype=np.int32)
    pool.append(table, k, v, layer)
    out2 = Out(T * h * d, np.uint16)
    dcu, dctx, dbt = dev(np.array([0, T], np.int32)), dev(np.array([T], np.int32)), dev(table)
    ql.call("ql_paged_attention_f16", dq.ptr, out2.ptr, h * d, h * d, T, 1, dcu.ptr, dctx.ptr, T,
            dbt.ptr, nb, pool.kptrs.ptr, pool.vptrs.ptr, nb, layer, L, h, hkv, d, 1, stream())
    assert np.array_equal(out2.get((T, h, d)), got)


# ---- decode (one query per sequence) ------------------------------------------------------
@pytest.mark.parametrize("h,hkv,d", [(32, 8, 128), (32, 1, 128), (6, 4, 64), (4, 4, 64),
                                     (40, 8, 128)])
@pytest.mark.parametrize("kv_len", [1, 31, 32, 33, 500, 2049])
def test_decode_contiguous_gqa_groups(h, hkv, d, kv_len):
    # q_len = 1 runs the decode kernel: query heads grouped per KV head (32/1: two
    # 16-head column chunks; 6/4: groups of 2,1,2,1 heads; 40/8: 5 per group)
    q, k, v = qkv(kv_len * 3 + h, 1, kv_len, h, hkv, d, 2.0)
    out = Out(h * d, np.uint16)
    dq, dk, dv = dev(q), dev(k), dev(v)
    ql.call("ql_attention_f16", ptr(dq), ptr(dk), ptr(dv), out.ptr, 1, kv_len, h, hkv, d, h * d,
            hkv * d, h * d, 1, stream())
    check_attn(out.get((1, h, d)), orc.attention(q, k, v, h, hkv, True, f16=True), v,
               f"decode h={h}/{hkv} d={d} kv={kv_len}")


@pytest.mark.parametrize("h,hkv,d", [(32, 8, 128), (8, 2, 64), (32, 1, 128), (6, 4, 64)])
@pytest.mark.parametrize("kv_len,row_pad", [(1, 0), (300, 0), (1000, 8), (8192, 0), (4097, 16)])
def test_contiguous_decode_key_split(h, hkv, d, kv_len, row_pad):
    """ql_decode_attention_f16: with the queried workspace the keys are split over
    workgroups (then combined); against the oracle, bit-identical to the paged split
    decode over the same keys (identity block table, same workspace size), and with
    no workspace bit-identical to ql_attention_f16's single pass.  row_pad: K/V rows
    strided past n_kv_heads*d."""
    q, k, v = qkv(kv_len + 7 * h + d, 1, kv_len, h, hkv, d, 2.0)
    stride = hkv * d + row_pad
    kp = np.zeros((kv_len, stride), np.uint16)
    vp = np.zeros((kv_len, stride), np.uint16)
    kp[:, :hkv * d] = k.reshape(kv_len, -1)
    vp[:, :hkv * d] = v.reshape(kv_len, -1)
    dq, dk, dv = dev(q), dev(kp), dev(vp)
    size = ctypes.c_size_t()
    ql.call("ql_decode_attention_workspace_size", h, hkv, d, kv_len, ctypes.addressof(size))
    ws = empty((max(size.value, 16),), np.uint8, fill_bits=0x7F)
    split = Out(h * d, np.uint16)
    ql.call("ql_decode_attention_f16", ptr(dq), ptr(dk), ptr(dv), split.ptr, kv_len, h, hkv, d, stride,
            ws.ptr if size.value else None, size.value, stream())
    got = split.get((1, h, d))
    check_attn(got, orc.attention(q, k, v, h, hkv, True, f16=True), v,
               f"split decode h={h}/{hkv} d={d} kv={kv_len}")
    # no workspace: the single pass of ql_attention_f16
    one, ref1 = Out(h * d, np.uint16), Out(h * d, np.uint16)
    ql.call("ql_decode_attention_f16", ptr(dq), ptr(dk), ptr(dv), one.ptr, kv_len, h, hkv, d, stride,
            None, 0, stream())
    ql.call("ql_attention_f16", ptr(dq), ptr(dk), ptr(dv), ref1.ptr, 1, kv_len, h, hkv, d, h * d, stride,
            h * d, 1, stream())
    assert np.array_equal(one.get(), ref1.get())
    # the paged split decode over the same keys (blocks in order) runs the same split
    L, layer = 2, 1
    nbs = (kv_len + 15) // 16
    pool = PagedPool(nbs, L, hkv, d)
    bt = np.arange(nbs, dtype=np.int32)
    pool.append(bt, k, v, layer)
    psize = ctypes.c_size_t()
    ql.call("ql_paged_decode_workspace_size", 1, h, hkv, d, kv_len, ctypes.addressof(psize))
    assert psize.value == size.value
    pws = empty((max(psize.value, 16),), np.uint8, fill_bits=0x7F)
    paged = Out(h * d, np.uint16)
    dctx, dbt = dev(np.array([kv_len], np.int32)), dev(bt)
    ql.call("ql_paged_decode_attention_f16", ptr(dq), paged.ptr, h * d, h * d, 1,
            dctx.ptr, kv_len, dbt.ptr, nbs, pool.kptrs.ptr,
            pool.vptrs.ptr, pool.nb, layer, L, h, hkv, d, pws.ptr if psize.value else None, psize.value,
            stream())
    assert np.array_equal(paged.get((1, h, d)), got)


def _decode_setup(ctx, h, hkv, d, L, layer, seed):
    r = np.random.default_rng(seed)
    need = [(c + 15) // 16 for c in ctx]
    nb = sum(need) + 2
    perm = r.permutation(nb)
    max_blocks = max(need + [1])
    bt = np.full((len(ctx), max_blocks), -1, np.int32)
    o = 0
    pool = PagedPool(nb, L, hkv, d)
    ks, vs = [], []
    for s, c in enumerate(ctx):
        bt[s, :need[s]] = perm[o:o + need[s]]
        o += need[s]
        k = to_f16_bits(normal(seed + 10 * s + 1, (c, hkv, d)))
        v = to_f16_bits(normal(seed + 10 * s + 2, (c, hkv, d)))
        pool.append(bt[s], k, v, layer)
        ks.append(k)
        vs.append(v)
    q = to_f16_bits(normal(seed + 5, (len(ctx), h, d), 2.0))
    return pool, bt, ks, vs, q


@pytest.mark.parametrize("h,hkv,d", [(32, 8, 128), (8, 2, 64), (32, 1, 128)])
def test_paged_decode_splits_and_one_pass_agree_with_oracle(h, hkv, d):
    ctx = [0, 1, 17, 100, 1000, 4096, 33, 130]
    L, layer = 3, 2
    pool, bt, ks, vs, q = _decode_setup(ctx, h, hkv, d, L, layer, h * d + hkv)
    S, max_blocks = len(ctx), bt.shape[1]
    dq, dctx, dbt = dev(q), dev(np.array(ctx, np.int32)), dev(bt)
    size = ctypes.c_size_t()
    ql.call("ql_paged_decode_workspace_size", S, h, hkv, d, max(ctx), ctypes.addressof(size))
    assert size.value > 0
    results = {}
    for label, nbytes in [("one pass", 0), ("full", size.value), ("partial", size.value // 3)]:
        ws = empty((max(nbytes, 1),), np.uint8, fill_bits=0x7F) if nbytes else None
        out = Out(S * h * d, np.uint16)
        ql.call("ql_paged_decode_attention_f16", dq.ptr, out.ptr, h * d, h * d, S, dctx.ptr,
                max(ctx), dbt.ptr, max_blocks, pool.kptrs.ptr, pool.vptrs.ptr, pool.nb, layer, L,
                h, hkv, d, ws.ptr if ws else None, nbytes, stream())
        got = out.get((S, h, d))
        for s in range(S):
            want = orc.attention(q[s:s + 1], ks[s], vs[s], h, hkv, True, f16=True)
            check_attn(got[s:s + 1], want, vs[s], f"decode {label} seq {s} ctx {ctx[s]}")
        results[label] = got
    # the varlen entry point with one query per sequence runs the same one-pass kernel
    out = Out(S * h * d, np.uint16)
    dcu = dev(np.arange(S + 1, dtype=np.int32))
    ql.call("ql_paged_attention_f16", dq.ptr, out.ptr, h * d, h * d, S, S, dcu.ptr, dctx.ptr, 1,
            dbt.ptr, max_blocks, pool.kptrs.ptr, pool.vptrs.ptr, pool.nb, layer, L, h, hkv, d, 1,
            stream())
    assert np.array_equal(out.get((S, h, d)), results["one pass"])


@pytest.mark.parametrize("h,hkv,d", [(32, 8, 128), (8, 2, 64)])
@pytest.mark.parametrize("split", [False, True])
def test_paged_decode_holed_tables(h, hkv, d, split):
    # decode steps over block tables with a hole (-1) and a block index past the
    # pool: the keys of those pages read as zero rows (score 0, value 0), as in
    # the prefill kernel; ragged context lengths end steps inside a page
    ctx = [75, 40, 130]
    L, layer = 2, 1
    pool, bt, ks, vs, q = _decode_setup(ctx, h, hkv, d, L, layer, 0x51A100A0)
    bt = bt.copy()
    bt[0, 1] = -1
    bt[2, 3] = pool.nb + 5
    kz, vz = [k.copy() for k in ks], [v.copy() for v in vs]
    kz[0][16:32] = 0
    vz[0][16:32] = 0
    kz[2][48:64] = 0
    vz[2][48:64] = 0
    S = len(ctx)
    dq, dctx, dbt = dev(q), dev(np.array(ctx, np.int32)), dev(bt)
    size = ctypes.c_size_t()
    ql.call("ql_paged_decode_workspace_size", S, h, hkv, d, max(ctx), ctypes.addressof(size))
    nbytes = size.value if split else 0
    ws = empty((max(nbytes, 1),), np.uint8, fill_bits=0x7F) if nbytes else None
    out = Out(S * h * d, np.uint16)
    ql.call("ql_paged_decode_attention_f16", dq.ptr, out.ptr, h * d, h * d, S, dctx.ptr, max(ctx),
            dbt.ptr, bt.shape[1], pool.kptrs.ptr, pool.vptrs.ptr, pool.nb, layer, L, h, hkv, d,
            ws.ptr if ws else None, nbytes, stream())
    got = out.get((S, h, d))
    for s in range(S):
        want = orc.attention(q[s:s + 1], kz[s], vz[s], h, hkv, True, f16=True)
        check_attn(got[s:s + 1], want, vs[s], f"holed decode seq {s} ctx {ctx[s]} split {split}")


def test_paged_decode_batch_c5_heads_long_context():
    # 16 sequences x 4096-token contexts, Llama-3-8B heads, split over the workspace
    S, C, h, hkv, d, L, layer = 16, 4096, 32, 8, 128, 2, 1
    ctx = [C - 37 * i for i in range(S)]
    pool, bt, ks, vs, q = _decode_setup(ctx, h, hkv, d, L, layer, 0x51A10080)
    dq, dctx, dbt = dev(q), dev(np.array(ctx, np.int32)), dev(bt)
    size = ctypes.c_size_t()
    ql.call("ql_paged_decode_workspace_size", S, h, hkv, d, C, ctypes.addressof(size))
    ws = empty((size.value,), np.uint8)
    out = Out(S * h * d, np.uint16)
    ql.call("ql_paged_decode_attention_f16", dq.ptr, out.ptr, h * d, h * d, S, dctx.ptr, C,
            dbt.ptr, bt.shape[1], pool.kptrs.ptr, pool.vptrs.ptr, pool.nb, layer, L, h, hkv, d,
            ws.ptr, size.value, stream())
    got = out.get((S, h, d))
    for s in range(S):
        check_attn(got[s:s + 1], orc.attention(q[s:s + 1], ks[s], vs[s], h, hkv, True, f16=True),
                   vs[s], f"decode seq {s}")
