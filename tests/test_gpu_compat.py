"""The reference's own tests, rerun against the drop-in shims that keep the
reference's names and signatures (include/quantlib_compat.h), on the GPU."""
import ctypes
import pathlib

import numpy as np
import pytest

import oracle as orc
import quantlib_amd as ql
from helpers import (ATOL_ROPE_F32, RTOL_F32, ATOL_F32, check_abs, check_close, check_f16, dev,
                     empty, f16_bits_to_f32, host, normal, ptr, stream, to_f16_bits, uniform)
from test_abi import COMPAT_MANGLED

pytestmark = pytest.mark.gpu

_p, _i, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float


class KVCache(ctypes.Structure):  # include/kv_cache.h:12-20
    _fields_ = [("k_cache", _p), ("v_cache", _p), ("n_layers", _i), ("max_seq_len", _i),
                ("n_heads", _i), ("head_dim", _i), ("current_len", _i)]


class PagedKVCache(ctypes.Structure):  # include/paged_kvcache.h:9-25
    _fields_ = [("k_blocks", _p), ("v_blocks", _p), ("n_blocks", _i), ("n_layers", _i),
                ("n_kv_heads", _i), ("head_dim", _i), ("free_blocks", ctypes.POINTER(_i)),
                ("free_count", _i), ("block_tables", ctypes.POINTER(ctypes.POINTER(_i))),
                ("max_seqs", _i), ("max_blocks_per_seq", _i)]


def fn(name, argtypes, restype=None):
    f = getattr(ql.lib(), COMPAT_MANGLED[name])
    f.argtypes, f.restype = argtypes, restype
    return f


def sync():
    ql.synchronize()


_hip = None


def d2h(dst_addr: int, src_addr: int, nbytes: int) -> None:
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [_p, _p, ctypes.c_size_t, ctypes.c_int]
        _hip.hipMemcpy.restype = ctypes.c_int
    assert _hip.hipMemcpy(dst_addr, src_addr, nbytes, 2) == 0  # hipMemcpyDeviceToHost


def test_reference_test_softmax_via_launch_softmax():
    # tests/test_softmax.cu:35-110
    launch_softmax = fn("launch_softmax", [_p, _p, _i, _i, _p])
    rows = cols = 2048
    x = orc.reftest_softmax_inputs(rows, cols, 7)
    din, dout = dev(x), empty((rows * cols,), np.float32)
    launch_softmax(ptr(din), ptr(dout), rows, cols, stream())
    got = host(dout, shape=(rows, cols))
    cpu = orc.softmax_reftest_cpu(x)
    assert np.max(np.abs(got - cpu)) < 1e-5
    assert np.max(np.abs(got.astype(np.float64).sum(axis=1) - 1)) < 1e-5


def test_reference_test_rope_norm_via_launch_rope():
    # tests/test_attention.cu:60-121: srand(99)-style U(-0.5,0.5) [128,32,128], theta 1e4;
    # the reference checks the norm to 1e-4; this also checks every element (pos = row).
    launch_rope = fn("launch_rope", [_p, _i, _i, _i, _f, _p])
    T, H, d = 128, 32, 128
    q = uniform(99, (T, H * d), -0.5, 0.5)
    dq = dev(q)
    launch_rope(ptr(dq), T, H, d, 1e4, stream())
    got = host(dq, shape=(T, H * d))
    n0 = np.linalg.norm(q.reshape(T, H, d).astype(np.float64), axis=2)
    n1 = np.linalg.norm(got.reshape(T, H, d).astype(np.float64), axis=2)
    assert np.max(np.abs(n0 - n1)) < 1e-4
    check_abs(got, orc.rope(q, H, d, 1e4, 0), ATOL_ROPE_F32, "launch_rope")


def test_reference_test_kvcache_readback():
    # tests/test_kvcache.cu:27-70 through kvcache_create / kvcache_append / kvcache_get_k
    create = fn("kvcache_create", [_i, _i, _i, _i], ctypes.POINTER(KVCache))
    append = fn("kvcache_append", [ctypes.POINTER(KVCache), _i, _p, _p, _p])
    get_k = fn("kvcache_get_k", [ctypes.POINTER(KVCache), _i], _p)
    get_v = fn("kvcache_get_v", [ctypes.POINTER(KVCache), _i], _p)
    free = fn("kvcache_free", [ctypes.POINTER(KVCache)])
    L, S, H, d = 32, 256, 32, 128
    slice_ = H * d
    c = create(L, S, H, d)
    assert c and c.contents.current_len == 0
    try:
        for tok in range(16):
            hk = np.float32(tok) + np.arange(slice_, dtype=np.float32) / np.float32(slice_)
            hv = np.full(slice_, -tok, np.float32)
            dk, dv = dev(hk), dev(hv)
            for layer in range(L):
                append(c, layer, ptr(dk), ptr(dv), stream())
            sync()
            c.contents.current_len += 1
        back = np.empty(slice_, np.float32)
        k0 = get_k(c, 0)
        d2h(back.ctypes.data, k0 + 7 * slice_ * 4, slice_ * 4)
        assert abs(back[0] - 7.0) < 1e-6
        np.testing.assert_array_equal(back, np.float32(7) + np.arange(slice_, dtype=np.float32) / np.float32(slice_))
        v5 = get_v(c, 5)
        d2h(back.ctypes.data, v5 + 9 * slice_ * 4, slice_ * 4)
        assert np.all(back == -9.0)
        d2h(back.ctypes.data, k0 + 16 * slice_ * 4, slice_ * 4)
        assert np.all(back == 0.0)  # created zeroed, untouched beyond current_len
    finally:
        free(c)


def test_fp16_shims_match_oracle():
    s = stream()
    rows, dim = 4, 4096
    x = to_f16_bits(normal(1, (rows, dim)))
    w = to_f16_bits(uniform(2, dim, 0.5, 1.5))
    dx, dw, do = dev(x), dev(w), empty((rows * dim,), np.uint16)
    fn("launch_fp16_rmsnorm", [_p, _p, _p, _i, _i, _f, _p])(ptr(dx), ptr(dw), ptr(do), rows, dim, 1e-5, s)
    check_f16(host(do, shape=(rows, dim)), orc.rmsnorm(x, w, 1e-5, f16=True), "launch_fp16_rmsnorm")

    q = to_f16_bits(normal(3, (1, 32 * 128)))
    dq = dev(q)
    fn("launch_fp16_rope", [_p, _i, _i, _i, _f, _p])(ptr(dq), 1, 32, 128, 1e4, s)
    assert np.array_equal(host(dq, shape=(1, 32 * 128)), q)  # decode: seq_len=1 -> pos 0 -> identity
    q = to_f16_bits(normal(4, (9, 8 * 64)))
    dq = dev(q)
    fn("launch_fp16_rope", [_p, _i, _i, _i, _f, _p])(ptr(dq), 9, 8, 64, 1e4, s)
    check_f16(host(dq, shape=(9, 8 * 64)), orc.rope(q, 8, 64, 1e4, 0, f16=True), "launch_fp16_rope")

    g, u = to_f16_bits(normal(5, 5632, clip=8)), to_f16_bits(normal(6, 5632, clip=8))
    dg, du, do = dev(g), dev(u), empty((5632,), np.uint16)
    fn("launch_fp16_swiglu", [_p, _p, _p, _i, _i, _p])(ptr(dg), ptr(du), ptr(do), 1, 5632, s)
    check_f16(host(do), orc.swiglu(g, u, f16=True), "launch_fp16_swiglu")

    table = to_f16_bits(normal(7, (100, 4096)))
    dt, do = dev(table), empty((4096,), np.uint16)
    fn("launch_fp16_embed", [_p, _p, _i, _i, _p])(ptr(dt), ptr(do), 42, 4096, s)
    assert np.array_equal(host(do), table[42])

    a, b = to_f16_bits(normal(8, 4096)), to_f16_bits(normal(9, 4096))
    da, db = dev(a), dev(b)
    fn("launch_fp16_add", [_p, _p, _i, _p])(ptr(da), ptr(db), 4096, s)
    assert np.array_equal(host(da), orc.add(a, b, f16=True))

    dl, do = dev(a), empty((4096,), np.float32)
    fn("launch_fp16_to_fp32", [_p, _p, _i, _p])(ptr(dl), ptr(do), 4096, s)
    assert np.array_equal(host(do), orc.f16_to_f32(a))

    L, S, H, d, layer, pos = 4, 32, 8, 128, 3, 11
    kc, vc = empty((L * S * H * d,), np.uint16, fill_bits=0), empty((L * S * H * d,), np.uint16, fill_bits=0)
    kn, vn = to_f16_bits(normal(10, H * d)), to_f16_bits(normal(11, H * d))
    dkn, dvn = dev(kn), dev(vn)
    fn("launch_fp16_kvcache_append", [_p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p])(
        ptr(kc), ptr(vc), ptr(dkn), ptr(dvn), layer, pos, H, d, S, L, s)
    wk, wv = np.zeros((L, S, H, d), np.uint16), np.zeros((L, S, H, d), np.uint16)
    orc.kv_append_inplace(wk, wv, kn.reshape(1, H, d), vn.reshape(1, H, d), layer, pos, f16=True)
    assert np.array_equal(host(kc, shape=(L, S, H, d)), wk)
    assert np.array_equal(host(vc, shape=(L, S, H, d)), wv)


class FP16KVCache(ctypes.Structure):  # src/fp16_forward.cu:115-120
    _fields_ = [("k_cache", _p), ("v_cache", _p), ("n_layers", _i), ("max_seq", _i),
                ("n_kv_heads", _i), ("head_dim", _i), ("current_len", _i)]


def test_fp16_kvcache_create_append_free():
    # the fp16 layer's cache lifecycle (src/fp16_forward.cu:122-145, appends as at
    # :194-199): create, one launch_fp16_kvcache_append per layer per token at
    # position current_len, read the written rows back, free
    create = fn("fp16_kvcache_create", [_i, _i, _i, _i], ctypes.POINTER(FP16KVCache))
    free = fn("fp16_kvcache_free", [ctypes.POINTER(FP16KVCache)])
    append = fn("launch_fp16_kvcache_append", [_p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p])
    L, S, H, d, T = 3, 40, 8, 128, 5
    assert not create(0, S, H, d) and not create(L, S, H, -1)
    c = create(L, S, H, d)
    assert c
    try:
        cc = c.contents
        assert (cc.n_layers, cc.max_seq, cc.n_kv_heads, cc.head_dim, cc.current_len) == (L, S, H, d, 0)
        kn = to_f16_bits(normal(30, (T, L, H, d)))
        vn = to_f16_bits(normal(31, (T, L, H, d)))
        for t in range(T):
            for layer in range(L):
                dk, dv = dev(kn[t, layer]), dev(vn[t, layer])
                append(cc.k_cache, cc.v_cache, ptr(dk), ptr(dv), layer, cc.current_len, H, d, S, L,
                       stream())
                sync()
            cc.current_len += 1
        row = H * d * 2
        for layer in range(L):
            for t in range(T):
                gk, gv = np.empty(H * d, np.uint16), np.empty(H * d, np.uint16)
                off = ((layer * S) + t) * row
                d2h(gk.ctypes.data, cc.k_cache + off, row)
                d2h(gv.ctypes.data, cc.v_cache + off, row)
                assert np.array_equal(gk, kn[t, layer].reshape(-1))
                assert np.array_equal(gv, vn[t, layer].reshape(-1))
    finally:
        free(c)


def test_fp32_shims_match_oracle():
    s = stream()
    rows, dim = 3, 2048
    x, w = normal(20, (rows, dim)), uniform(21, dim, 0.5, 1.5)
    dx, dw, do = dev(x), dev(w), empty((rows * dim,), np.float32)
    fn("launch_rmsnorm", [_p, _p, _p, _i, _i, _f, _p])(ptr(dx), ptr(dw), ptr(do), rows, dim, 1e-5, s)
    check_close(host(do, shape=(rows, dim)), orc.rmsnorm(x, w, 1e-5), RTOL_F32, ATOL_F32, "launch_rmsnorm")

    g, u = normal(22, (32, 5632), clip=8), normal(23, (32, 5632), clip=8)
    dg, du, do = dev(g), dev(u), empty((32 * 5632,), np.float32)
    fn("launch_swiglu", [_p, _p, _p, _i, _i, _p])(ptr(dg), ptr(du), ptr(do), 32, 5632, s)
    check_close(host(do, shape=(32, 5632)), orc.swiglu(g, u), RTOL_F32, ATOL_F32, "launch_swiglu")

    a, b = normal(24, 4096), normal(25, 4096)
    da, db = dev(a), dev(b)
    fn("add_residual", [_p, _p, _i, _p])(ptr(da), ptr(db), 4096, s)
    assert np.array_equal(host(da), orc.add(a, b))

    table = normal(26, (50, 2048))
    dt, do = dev(table), empty((2048,), np.float32)
    fn("launch_embed", [_p, _p, _i, _i, _p])(ptr(do), ptr(dt), 17, 2048, s)
    assert np.array_equal(host(do), table[17])


def test_paged_allocator_lifo_and_pool_layout():
    # src/paged_kvcache.cu:16-98: fresh pool hands out 0,1,2,...; -1 when empty;
    # block i of each pool at pool + i * (n_layers*16*H_kv*d) halves.
    create = fn("paged_kv_create", [_i, _i, _i, _i, _i, _i], ctypes.POINTER(PagedKVCache))
    alloc = fn("paged_kv_allocate_block", [ctypes.POINTER(PagedKVCache)], _i)
    release = fn("paged_kv_free_block", [ctypes.POINTER(PagedKVCache), _i])
    free = fn("paged_kv_free", [ctypes.POINTER(PagedKVCache)])
    nb, L, H, d = 6, 4, 8, 128
    c = create(nb, L, H, d, 3, 10)
    assert c
    try:
        assert [alloc(c) for _ in range(nb)] == list(range(nb))
        assert alloc(c) == -1
        release(c, 4)
        release(c, 1)
        assert alloc(c) == 1 and alloc(c) == 4
        assert all(c.contents.block_tables[s][j] == -1 for s in range(3) for j in range(10))
        ptrs = (ctypes.c_uint64 * nb)()
        d2h(ctypes.addressof(ptrs), c.contents.k_blocks, 8 * nb)
        blk_bytes = L * 16 * H * d * 2
        assert [ptrs[i] - ptrs[0] for i in range(nb)] == [i * blk_bytes for i in range(nb)]

        # append through the ql_ paged kernel into this cache's pool
        T, layer = 40, 2
        table = (ctypes.c_int32 * 3)(5, 0, 3)
        slots = (ctypes.c_int32 * T)()
        assert ql.raw("ql_paged_slot_mapping", ctypes.addressof(table), 3, 0, T, ctypes.addressof(slots)) == 0
        slots_np = np.frombuffer(slots, np.int32).copy()
        kn = to_f16_bits(normal(30, (T, H, d)))
        vn = to_f16_bits(normal(31, (T, H, d)))
        dsl, dkn, dvn = dev(slots_np), dev(kn), dev(vn)
        ql.call("ql_paged_kv_append_f16", c.contents.k_blocks, c.contents.v_blocks, nb, ptr(dsl),
                ptr(dkn), ptr(dvn), T, layer, L, H, d, stream())
        sync()
        pool = np.empty(nb * L * 16 * H * d, np.uint16)
        d2h(pool.ctypes.data, ptrs[0], pool.nbytes)
        pool = pool.reshape(nb, L, 16, H, d)
        for t in range(T):
            b, o = slots_np[t] // 16, slots_np[t] % 16
            assert np.array_equal(pool[b, layer, o], kn[t]), t
    finally:
        free(c)


# ---- quantlib FP8 (quantlib_src/tests/test_fp8.cu) -------------------------------------------
class QuantParams(ctypes.Structure):   # quant_types.h:23-29
    _fields_ = [("scales", _p), ("zeros", _p), ("group_size", _i), ("granularity", _i),
                ("n_scales", _i)]


class QuantMatrix(ctypes.Structure):   # quant_types.h:32-39
    _fields_ = [("data", _p), ("params", QuantParams), ("rows", _i), ("cols", _i), ("bits", _i),
                ("format", ctypes.c_char * 16)]


def test_reference_fp8_test_via_quantlib_shims():
    # quantlib_src/tests/test_fp8.cu:24-100: 1024x1024 U(-1,1) weights (rand(), default
    # seed), E4M3 per-group 128, E5M2 per-channel, E4M3 per-tensor; max abs error < 0.25.
    to_e4m3 = fn("quantlib_fp16_to_fp8_e4m3", [_p, _i, _i, _i, _i, _p], QuantMatrix)
    to_e5m2 = fn("quantlib_fp16_to_fp8_e5m2", [_p, _i, _i, _i, _i, _p], QuantMatrix)
    to_f16 = fn("quantlib_fp8_to_fp16", [ctypes.POINTER(QuantMatrix), _p, _p])
    qerr = fn("quantlib_quant_error", [_p, _p, _i], ctypes.c_float)
    qfree = fn("quantlib_free", [ctypes.POINTER(QuantMatrix)])
    stats = fn("quantlib_print_stats", [ctypes.POINTER(QuantMatrix)])
    rows = cols = 1024
    x = to_f16_bits(orc.reftest_fp8_inputs(rows, cols, 1))
    dx = dev(x)
    deq = empty((rows * cols,), np.uint16)
    for conv, fmt, gran, gs in [(to_e4m3, 0, 2, 128), (to_e5m2, 1, 1, 0), (to_e4m3, 0, 0, 0)]:
        qm = conv(ptr(dx), rows, cols, gran, gs, stream())
        assert qm.bits == 8 and qm.format == (b"E4M3" if fmt == 0 else b"E5M2")
        stats(ctypes.byref(qm))
        to_f16(ctypes.byref(qm), ptr(deq), stream())
        sync()
        err = qerr(ptr(dx), ptr(deq), rows * cols)
        assert err < 0.25, err
        q_want, sc_want = orc.fp8_quantize(x, fmt, gran, gs, 0)   # the reference's algorithm
        codes = np.empty(rows * cols, np.uint8)
        scales = np.empty(qm.params.n_scales, np.float32)
        d2h(codes.ctypes.data, qm.data, codes.nbytes)
        d2h(scales.ctypes.data, qm.params.scales, scales.nbytes)
        assert np.array_equal(scales, sc_want) and np.array_equal(codes.reshape(rows, cols), q_want)
        assert np.array_equal(host(deq, shape=(rows, cols)),
                              orc.fp8_dequantize(q_want, sc_want, fmt, gran, gs, 0))
        assert abs(err - float(np.abs(f16_bits_to_f32(host(deq)) - f16_bits_to_f32(x).ravel()).max())) == 0
        qfree(ctypes.byref(qm))
        assert qm.data is None and qm.params.scales is None


def test_reference_gemm_test_via_quantlib_shims():
    # quantlib_src/tests/test_gemm.cu:29-85: A [32 x 64] and W [64 x 64] from srand(7)
    # U(-0.1, 0.1), W quantized E4M3 in groups of 64 (quantlib_fp16_to_fp8_e4m3),
    # C = quantlib_fp8_gemm; its bar: max abs error < 1.0 against its fp32 CPU GEMM
    # of the unquantized weights.  Tighter here: the same against the product of the
    # dequantized weights within the GEMM bound, and the quantization error alone
    # explains the distance to the unquantized product.
    to_e4m3 = fn("quantlib_fp16_to_fp8_e4m3", [_p, _i, _i, _i, _i, _p], QuantMatrix)
    gemm = fn("quantlib_fp8_gemm", [_p, ctypes.POINTER(QuantMatrix), _p, _i, _i, _i, _p])
    qfree = fn("quantlib_free", [ctypes.POINTER(QuantMatrix)])
    M, N, K = 32, 64, 64
    a32, w32 = orc.reftest_gemm_inputs(M, N, K, 7)
    a, w = to_f16_bits(a32), to_f16_bits(w32)
    da, dw = dev(a), dev(w)
    qm = to_e4m3(ptr(dw), N, K, 2, 64, stream())
    out = empty((M * N,), np.uint16)
    gemm(ptr(da), ctypes.byref(qm), ptr(out), M, N, K, stream())
    sync()
    got = f16_bits_to_f32(host(out, shape=(M, N))).astype(np.float64)
    ref = orc.gemm_reftest_cpu(a, w).astype(np.float64)
    err = float(np.abs(got - ref).max())
    assert err < 1.0, err
    q, sc = orc.fp8_quantize(w, 0, 2, 64, 0)
    wd = orc.fp8_dequantize(q, sc, 0, 2, 64, 0)
    af, wdf = f16_bits_to_f32(a).astype(np.float64), f16_bits_to_f32(wd).astype(np.float64)
    s = af @ wdf.T
    bound = 2.0 ** -10 * (np.abs(s) + np.abs(af) @ np.abs(wdf).T)
    assert np.all(np.abs(got - s) <= bound)
    wf = f16_bits_to_f32(w).astype(np.float64)
    qerr = np.abs(af) @ np.abs(wdf - wf).T
    assert np.all(np.abs(got - ref) <= qerr + bound + K * 2.0 ** -23 * (np.abs(af) @ np.abs(wf).T))
    qfree(ctypes.byref(qm))


@pytest.mark.parametrize("M", [16, 128])
def test_quantlib_fp8_gemm_shim(M):
    to_e4m3 = fn("quantlib_fp16_to_fp8_e4m3", [_p, _i, _i, _i, _i, _p], QuantMatrix)
    gemm = fn("quantlib_fp8_gemm", [_p, ctypes.POINTER(QuantMatrix), _p, _i, _i, _i, _p])
    qfree = fn("quantlib_free", [ctypes.POINTER(QuantMatrix)])
    N, K = 256, 512
    w = to_f16_bits(normal(5, (N, K), K ** -0.5))
    a = to_f16_bits(normal(6, (M, K)))
    dw, da = dev(w), dev(a)
    qm = to_e4m3(ptr(dw), N, K, 2, 128, stream())
    out = empty((M * N,), np.uint16)
    gemm(ptr(da), ctypes.byref(qm), ptr(out), M, N, K, stream())
    sync()
    q, sc = orc.fp8_quantize(w, 0, 2, 128, 0)
    wd = orc.fp8_dequantize(q, sc, 0, 2, 128, 0)
    want = orc.matmul(a, wd)
    bound = 2.0 ** -10 * (np.abs(f16_bits_to_f32(want)) +
                          np.abs(f16_bits_to_f32(a)).astype(np.float64) @ np.abs(f16_bits_to_f32(wd)).T)
    assert np.all(np.abs(f16_bits_to_f32(host(out, shape=(M, N))) - f16_bits_to_f32(want)) <= bound)
    qfree(ctypes.byref(qm))


def test_quantlib_fp8_gemm_shim_on_two_streams():
    """Two quantlib_fp8_gemm calls in flight at once on two streams, one on the
    split-K register path (16 rows) and one on the dequantize path (128 rows):
    each stream has its own workspace, so both match the oracle.  Repeated so
    the second round reuses the grown buffers."""
    to_e4m3 = fn("quantlib_fp16_to_fp8_e4m3", [_p, _i, _i, _i, _i, _p], QuantMatrix)
    gemm = fn("quantlib_fp8_gemm", [_p, ctypes.POINTER(QuantMatrix), _p, _i, _i, _i, _p])
    qfree = fn("quantlib_free", [ctypes.POINTER(QuantMatrix)])
    s2 = ctypes.c_void_p()
    ql.hip_check(ql.hip().hipStreamCreate(ctypes.byref(s2)), "hipStreamCreate")
    N, K = 1024, 4096
    w = to_f16_bits(normal(15, (N, K), K ** -0.5))
    dw = dev(w)
    qm = to_e4m3(ptr(dw), N, K, 2, 128, stream())
    sync()
    q, sc = orc.fp8_quantize(w, 0, 2, 128, 0)
    wd = orc.fp8_dequantize(q, sc, 0, 2, 128, 0)
    cases = []
    for M, s in ((16, stream()), (128, s2.value)):
        a = to_f16_bits(normal(16 + M, (M, K)))
        want = orc.matmul(a, wd)
        bound = 2.0 ** -10 * (np.abs(f16_bits_to_f32(want)) +
                              np.abs(f16_bits_to_f32(a)).astype(np.float64) @ np.abs(f16_bits_to_f32(wd)).T)
        cases.append((M, s, dev(a), empty((M * N,), np.uint16), want, bound))
    for _ in range(2):
        for M, s, da, out, _, _ in cases:
            out.fill_bytes(0xFF)
        for rep in range(3):      # interleave enqueues on the two streams
            for M, s, da, out, _, _ in cases:
                gemm(ptr(da), ctypes.byref(qm), ptr(out), M, N, K, s)
        ql.hip_check(ql.hip().hipStreamSynchronize(s2.value), "hipStreamSynchronize")
        sync()
        for M, s, da, out, want, bound in cases:
            got = f16_bits_to_f32(host(out, shape=(M, N)))
            assert np.all(np.abs(got - f16_bits_to_f32(want)) <= bound), M
    qfree(ctypes.byref(qm))
    h = ql.hip()
    h.hipStreamDestroy.argtypes, h.hipStreamDestroy.restype = [_p], ctypes.c_int
    ql.hip_check(h.hipStreamDestroy(s2.value), "hipStreamDestroy")


@pytest.mark.parametrize("M", [1, 100])
def test_fp32_quantized_gemm_bridge(M):
    """The fp32 engine's quantized GEMM (sgemm, src/forward.cu:52-70) through the
    shims: launch_fp32_to_fp16 on A, quantlib_fp8_gemm, launch_fp16_to_fp32 on C.
    The narrowed A is bit-exact (RNE), C within the FP8 GEMM bound, and the widened
    C is exactly the binary16 C."""
    to_e4m3 = fn("quantlib_fp16_to_fp8_e4m3", [_p, _i, _i, _i, _i, _p], QuantMatrix)
    gemm = fn("quantlib_fp8_gemm", [_p, ctypes.POINTER(QuantMatrix), _p, _i, _i, _i, _p])
    qfree = fn("quantlib_free", [ctypes.POINTER(QuantMatrix)])
    narrow = fn("launch_fp32_to_fp16", [_p, _p, _i, _p])
    widen = fn("launch_fp16_to_fp32", [_p, _p, _i, _p])
    N, K = 512, 1024
    w = to_f16_bits(normal(25, (N, K), K ** -0.5))
    a32 = normal(26 + M, (M, K))
    dw, da32 = dev(w), dev(a32)
    qm = to_e4m3(ptr(dw), N, K, 2, 128, stream())
    ha, hc = empty((M * K,), np.uint16), empty((M * N,), np.uint16)
    c32 = empty((M * N,), np.float32)
    narrow(ptr(da32), ptr(ha), M * K, stream())
    gemm(ptr(ha), ctypes.byref(qm), ptr(hc), M, N, K, stream())
    widen(ptr(hc), ptr(c32), M * N, stream())
    sync()
    a16 = orc.f32_to_f16(a32)
    assert np.array_equal(host(ha, shape=(M, K)), a16)
    q, sc = orc.fp8_quantize(w, 0, 2, 128, 0)
    wd = orc.fp8_dequantize(q, sc, 0, 2, 128, 0)
    want = orc.matmul(a16, wd)
    bound = 2.0 ** -10 * (np.abs(f16_bits_to_f32(want)) +
                          np.abs(f16_bits_to_f32(a16)).astype(np.float64) @ np.abs(f16_bits_to_f32(wd)).T)
    c16 = host(hc, shape=(M, N))
    assert np.all(np.abs(f16_bits_to_f32(c16) - f16_bits_to_f32(want)) <= bound)
    assert np.array_equal(host(c32, shape=(M, N)), f16_bits_to_f32(c16))
    qfree(ctypes.byref(qm))


@pytest.mark.parametrize("vocab", [1, 255, 32000, 128256])
def test_fp16_greedy_sample_shim(vocab):
    # src/fp16_forward.cu:285-297: the index of the largest logit, as a host int.
    # Logits come from binary16 (the engine widens them), so ties are likely at
    # this vocab size; the first index of the maximum is the answer (the
    # reference's own tie order depends on a race between its warps).
    f = fn("fp16_greedy_sample", [_p, _i, _p], _i)
    r = np.random.default_rng(vocab)
    for trial in range(3):
        x = f16_bits_to_f32(to_f16_bits(r.standard_normal(vocab).astype(np.float32) * 3.0))
        if trial == 1:
            x[r.integers(0, vocab, size=min(vocab, 4))] = x.max()   # planted ties
        if trial == 2:
            x = -np.abs(x) - 1.0                                    # every logit negative
        d = dev(x.astype(np.float32))
        got = f(d.ptr, vocab, stream())
        assert got == int(np.argmax(x)), (vocab, trial, got, int(np.argmax(x)))
        assert got == int(orc.argmax(x[None, :])[0])
    assert f(None, 0, stream()) == 0   # empty scan: index 0, no launch


def test_dropin_caller_program_runs():
    """The C++ caller of tests/dropin/caller.cpp (reference-style call sites,
    linked against libquantlib_amd.so, built by build()) run as a child process:
    every closed-form check it makes passes."""
    import subprocess
    exe = pathlib.Path(__file__).resolve().parent / "dropin" / "caller"
    assert exe.exists(), f"{exe} is not built: run __graft_entry__.build() (make -C tests/dropin)"
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "dropin caller: ok" in r.stdout, r.stdout + r.stderr
