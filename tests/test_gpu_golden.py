"""GPU: every committed golden fixture (tests/golden/) through the C ABI.

Each fixture's inputs go through the HIP library's entry point and the outputs
are compared with the fixture's expected outputs at the op's tolerance
(manifest.json "tol": fp32 rtol 1e-5, fp32 RoPE abs 1e-6, binary16 rtol 2e-3,
attention rtol 2e-3 + 2e-3 max|V|, index ops bit-exact).  Outputs sit between
guard bands, caches and pools start from a guard pattern that untouched slots
must keep."""
import numpy as np
import pytest

import quantlib_amd as ql
from golden import make_golden as mg
from helpers import Out, check_close, dev, empty, f16_bits_to_f32, host, ptr, stream

pytestmark = pytest.mark.gpu


def _check(got, want, tol, what, vmax=None):
    if tol == "exact":
        assert got.dtype == want.dtype and got.tobytes() == want.tobytes(), f"{what}: not bit-exact"
        return
    f16 = want.dtype == np.uint16
    g = f16_bits_to_f32(got) if f16 else got
    w = f16_bits_to_f32(want) if f16 else want
    if tol == "attention":
        check_close(g, w, 2e-3, 2e-3 * max(vmax, 1e-3), what)
    else:
        t = mg.TOL[tol]
        check_close(g, w, t["rtol"], t["atol"], what)


def _pool(nb, blk, guard):
    kp = empty((nb * blk,), np.uint16)
    vp = empty((nb * blk,), np.uint16)
    kp.upload(np.full(nb * blk, guard, np.uint16))
    vp.upload(np.full(nb * blk, guard, np.uint16))
    kptr = dev(np.array([kp.ptr + 2 * blk * b for b in range(nb)], np.int64))
    vptr = dev(np.array([vp.ptr + 2 * blk * b for b in range(nb)], np.int64))
    return kp, vp, kptr, vptr


@pytest.mark.parametrize("name", mg.names())
def test_golden_fixture(name):
    p, a = mg.load(name)
    op, tol, s = p["op"], p["tol"], stream()
    held = []           # device inputs stay allocated until the test ends

    def D(arr):
        t = dev(arr)
        held.append(t)
        return t.ptr

    if op in ("rmsnorm_f32", "rmsnorm_f16"):
        x = a["in_x"]
        out = Out(x.size, x.dtype)
        ql.call(f"ql_{op}", D(x), D(a["in_w"]), out.ptr, x.shape[0], x.shape[1],
                p["eps"], s)
        _check(out.get(x.shape), a["want_out"], tol, name)

    elif op in ("add_rmsnorm_f32", "add_rmsnorm_f16"):
        x = a["in_x"]
        dx, out = dev(x), Out(x.size, x.dtype)
        ql.call(f"ql_{op}", ptr(dx), D(a["in_d"]), D(a["in_w"]), out.ptr, x.shape[0],
                x.shape[1], p["eps"], s)
        _check(host(dx, shape=x.shape), a["want_x"], "exact", f"{name} x'")
        _check(out.get(x.shape), a["want_out"], tol, name)

    elif op in ("rope_f32", "rope_f16"):
        q, k = a["in_q"], a["in_k"]
        dq, dk = dev(q), dev(k)
        pos = dev(a["in_positions"]) if "in_positions" in a else None
        ql.call(f"ql_{op}", ptr(dq), ptr(dk), q.shape[0], p["n_heads"], p["n_kv_heads"],
                p["head_dim"], q.shape[1], k.shape[1], None if pos is None else ptr(pos),
                p["pos_offset"], p["theta"], p["pairing"], s)
        _check(host(dq, shape=q.shape), a["want_q"], tol, f"{name} q")
        _check(host(dk, shape=k.shape), a["want_k"], tol, f"{name} k")

    elif op in ("swiglu_f32", "swiglu_f16"):
        g = a["in_gate"]
        out = Out(g.size, g.dtype)
        ql.call(f"ql_{op}", D(g), D(a["in_up"]), out.ptr, g.shape[0], g.shape[1], s)
        _check(out.get(g.shape), a["want_out"], tol, name)

    elif op in ("softmax_f32", "softmax_f16"):
        x = a["in_x"]
        out = Out(x.size, x.dtype)
        ql.call(f"ql_{op}", D(x), out.ptr, x.shape[0], x.shape[1], s)
        got = out.get(x.shape)
        _check(got, a["want_out"], tol, name)
        if "want_reftest_cpu" in a:       # tests/test_softmax.cu:88-106
            assert np.abs(got - a["want_reftest_cpu"]).max() < 1e-5
            assert np.abs(got.astype(np.float64).sum(axis=1) - 1.0).max() < 1e-5

    elif op in ("embed_f16", "embed_f32"):
        t, ids = a["in_table"], a["in_ids"]
        out = Out(ids.size * t.shape[1], t.dtype)
        ql.call(f"ql_{op}", D(t), D(ids), ids.size, t.shape[0], t.shape[1], out.ptr, s)
        _check(out.get((ids.size, t.shape[1])), a["want_out"], tol, name)

    elif op == "kv_append_f32_tokens":
        # tests/test_kvcache.cu:47-60: one token at a time into every layer
        L, S, H, d = p["n_layers"], p["max_seq"], p["n_kv_heads"], p["head_dim"]
        kc, vc = empty((L * S * H * d,), np.float32, 0), empty((L * S * H * d,), np.float32, 0)
        for tok in range(a["in_k"].shape[0]):
            dk, dv = dev(a["in_k"][tok]), dev(a["in_v"][tok])
            for layer in range(L):
                ql.call("ql_kv_append_f32", kc.ptr, vc.ptr, dk.ptr, dv.ptr, layer, tok, 1, H, d, S,
                        L, s)
            ql.synchronize()
        _check(host(kc, shape=(L, S, H, d)), a["want_k_cache"], tol, f"{name} k")
        _check(host(vc, shape=(L, S, H, d)), a["want_v_cache"], tol, f"{name} v")
        assert host(kc, shape=(L, S, H, d))[0, 7, 0, 0] == 7.0    # the reference's known answer

    elif op == "kv_append_f16":
        L, S, H, d = p["n_layers"], p["max_seq"], p["n_kv_heads"], p["head_dim"]
        n = L * S * H * d
        kc, vc = empty((n,), np.uint16), empty((n,), np.uint16)
        kc.upload(np.full(n, p["guard"], np.uint16))
        vc.upload(np.full(n, p["guard"], np.uint16))
        kn = a["in_k"]
        ql.call("ql_kv_append_f16", kc.ptr, vc.ptr, D(kn), D(a["in_v"]), p["layer"],
                p["pos"], kn.shape[0], H, d, S, L, s)
        _check(host(kc, shape=(L, S, H, d)), a["want_k_cache"], tol, f"{name} k")
        _check(host(vc, shape=(L, S, H, d)), a["want_v_cache"], tol, f"{name} v")

    elif op == "paged_kv_append_f16":
        nb, L, H, d = p["n_blocks"], p["n_layers"], p["n_kv_heads"], p["head_dim"]
        kp, vp, kptr, vptr = _pool(nb, L * 16 * H * d, p["guard"])
        kn = a["in_k"]
        ql.call("ql_paged_kv_append_f16", kptr.ptr, vptr.ptr, nb, D(a["in_slots"]),
                D(kn), D(a["in_v"]), kn.shape[0], p["layer"], L, H, d, s)
        _check(host(kp), a["want_k_pool"], tol, f"{name} k pool")
        _check(host(vp), a["want_v_pool"], tol, f"{name} v pool")

    elif op == "rope_paged_kv_append_f16":
        nb, L, H, HK, d = (p[k] for k in ("n_blocks", "n_layers", "n_heads", "n_kv_heads",
                                          "head_dim"))
        kp, vp, kptr, vptr = _pool(nb, L * 16 * HK * d, p["guard"])
        q, k, v = a["in_q"], a["in_k"], a["in_v"]
        dq, dk = dev(q), dev(k)
        ql.call("ql_rope_paged_kv_append_f16", dq.ptr, dk.ptr, D(v), q.shape[0], H, HK, d,
                q.shape[1], k.shape[1], v.shape[1], D(a["in_positions"]), 0, p["theta"],
                p["pairing"], kptr.ptr, vptr.ptr, nb, D(a["in_slots"]), p["layer"], L, s)
        _check(host(dq, shape=q.shape), a["want_q"], tol, f"{name} q")
        got_k = host(dk, shape=k.shape)
        _check(got_k, a["want_k"], tol, f"{name} k")
        # the pool holds exactly the rotated K rows the call left in k, and V bit for bit
        want_kp = a["want_k_pool"].copy()
        blk_rows = want_kp.reshape(nb, L, 16, HK * d)
        for t, sl in enumerate(a["in_slots"]):
            if 0 <= sl < nb * 16:
                blk_rows[sl // 16, p["layer"], sl % 16] = got_k[t]
        _check(host(kp), want_kp, "exact", f"{name} k pool")
        _check(host(vp), a["want_v_pool"], "exact", f"{name} v pool")

    elif op == "f16_to_f32":
        x = a["in_x"]
        out = Out(x.size, np.float32)
        ql.call("ql_f16_to_f32", D(x), out.ptr, x.size, s)
        got, want = out.get(), a["want_out"]
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert got[~nan].tobytes() == want[~nan].tobytes()

    elif op == "flash_attention_f16":
        q, k, v = a["in_q"], a["in_k"], a["in_v"]
        out = Out(q.size, np.uint16)
        ql.call("ql_flash_attention_f16", D(q), D(k), D(v), out.ptr,
                q.shape[0], p["n_heads"], p["n_kv_heads"], p["head_dim"], p["causal"], s)
        _check(out.get(q.shape), a["want_out"], tol, name,
               vmax=float(np.abs(f16_bits_to_f32(v)).max()))

    elif op == "fp8_quantize":
        x = a["in_x"]
        rows, cols = x.shape
        dx = dev(x)
        for fmt, mode, gran, gs in p["variants"]:
            tag = f"f{fmt}_m{mode}"
            want_sc = a[f"want_scales_{tag}"]
            q, sc = empty((x.size,), np.uint8), empty((want_sc.size,), np.float32)
            ql.call("ql_fp8_quantize", dx.ptr, rows, cols, fmt, gran, gs, mode, q.ptr, sc.ptr, s)
            _check(host(q, shape=x.shape), a[f"want_codes_{tag}"], tol, f"{name} codes {tag}")
            _check(host(sc), want_sc, tol, f"{name} scales {tag}")
            out = Out(x.size, np.uint16)
            ql.call("ql_fp8_dequantize", q.ptr, sc.ptr, rows, cols, fmt, gran, gs, mode, out.ptr, s)
            _check(out.get(x.shape), a[f"want_deq_{tag}"], tol, f"{name} dequantized {tag}")

    else:
        raise KeyError(op)
