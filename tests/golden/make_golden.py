"""Golden fixtures for the hot-path ops: small inputs with their expected outputs.

Each fixture is one `.npz` (plain arrays, no pickled objects) holding the inputs
(`in_*`) and expected outputs (`want_*`) of one C-ABI call, with its scalar
arguments and tolerance in `manifest.json` beside a sha256 of the file.

Where the expected outputs come from:
  * the CPU oracle (oracle/oracle.c) computes them, and
  * before a fixture is written, `independent_check` recomputes them with a
    float64 numpy formulation of the reference formula (cited per op) and
    requires agreement within the op's tolerance; index ops (gather, KV
    appends, widening) are checked bit for bit against numpy indexing.
Two fixtures carry the reference's own test data:
  * softmax_f32_reftest: the first rows of tests/test_softmax.cu:38-47
    (srand(7), U(-2,2), 2048 columns, glibc rand() sequence) with the result of
    its cpu_softmax (:19-30) next to the oracle's;
  * kv_append_f32_readback: the fill of tests/test_kvcache.cu:47-60
    (k[i] = tok + i/slice, v = -tok, 16 tokens into every layer) at a smaller
    head count, with its known answer layer 0 / token 7 / k[0] = 7.0.

Run `python tests/golden/make_golden.py` to rewrite the fixtures and manifest.
tests/test_golden.py (CPU) re-verifies them and tests/test_gpu_golden.py runs
each through the HIP library.
"""
from __future__ import annotations

import hashlib
import json
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent.parent
for _p in (ROOT, ROOT / "tests"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

import oracle as orc                                        # noqa: E402

MANIFEST = HERE / "manifest.json"
ROPE_INTERLEAVED, ROPE_HALF = 0, 1     # pairing values of ql_rope_* ((2i, 2i+1), rotate-half)

# tolerances of the north star: |got - want| <= rtol*|want| + atol
TOL = {
    "f32": {"rtol": 1e-5, "atol": 2.0 ** -126},
    "rope_f32": {"rtol": 0.0, "atol": 1e-6},
    "f16": {"rtol": 2e-3, "atol": 2.0 ** -24},
    "exact": {"rtol": 0.0, "atol": 0.0},
}


def _rng(seed):
    return np.random.default_rng(seed)


def _normal(seed, shape, sigma=1.0, clip=None):
    x = _rng(seed).standard_normal(size=shape, dtype=np.float32) * np.float32(sigma)
    if clip is not None:
        np.clip(x, -clip, clip, out=x)
    return x


def _uniform(seed, shape, lo, hi):
    return _rng(seed).uniform(lo, hi, size=shape).astype(np.float32)


def _h(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def _w(h):
    """binary16 bits -> float64 values"""
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float64)


def _causal(x, first_pos=0):
    """-inf where column > the row's position (row r sits at first_pos + r)."""
    r, c = x.shape
    x[np.triu_indices(r, k=1 + first_pos, m=c)] = -np.inf
    return x


# ---- cases -----------------------------------------------------------------------------------
def case_rmsnorm_f32():
    x = _normal(101, (6, 1000))
    x[0] = 0.75                                     # constant row
    x[1] = 0.0
    x[1, 17] = 3.0                                  # one-hot row
    w = _uniform(102, 1000, 0.5, 1.5)
    return {"op": "rmsnorm_f32", "eps": 1e-5, "tol": "f32"}, {
        "in_x": x, "in_w": w, "want_out": orc.rmsnorm(x, w, 1e-5)}


def case_rmsnorm_f16():
    x, w = _h(_normal(103, (5, 520))), _h(_uniform(104, 520, 0.5, 1.5))
    return {"op": "rmsnorm_f16", "eps": 1e-5, "tol": "f16"}, {
        "in_x": x, "in_w": w, "want_out": orc.rmsnorm(x, w, 1e-5, f16=True)}


def case_add_rmsnorm_f32():
    x, d, w = _normal(105, (4, 256)), _normal(106, (4, 256)), _uniform(107, 256, 0.5, 1.5)
    xs, y = orc.add_rmsnorm(x, d, w, 1e-5)
    return {"op": "add_rmsnorm_f32", "eps": 1e-5, "tol": "f32"}, {
        "in_x": x, "in_d": d, "in_w": w, "want_x": xs, "want_out": y}


def case_add_rmsnorm_f16():
    # hidden 4096: the width of the Llama-3-8B-shaped layer
    x, d = _h(_normal(108, (3, 4096))), _h(_normal(109, (3, 4096)))
    w = _h(_uniform(110, 4096, 0.5, 1.5))
    xs, y = orc.add_rmsnorm(x, d, w, 1e-5, f16=True)
    return {"op": "add_rmsnorm_f16", "eps": 1e-5, "tol": "f16"}, {
        "in_x": x, "in_d": d, "in_w": w, "want_x": xs, "want_out": y}


def _rope_case(name, f16, T, H, HK, d, theta, pairing, seed, positions=None, pos_offset=0):
    conv = _h if f16 else (lambda a: a)
    q, k = conv(_normal(seed, (T, H * d))), conv(_normal(seed + 1, (T, HK * d)))
    pos = None if positions is None else np.asarray(positions, np.int32)
    arrays = {"in_q": q, "in_k": k,
              "want_q": orc.rope(q, H, d, theta, pairing, pos, pos_offset, f16=f16),
              "want_k": orc.rope(k, HK, d, theta, pairing, pos, pos_offset, f16=f16)}
    if pos is not None:
        arrays["in_positions"] = pos
    return {"op": name, "n_heads": H, "n_kv_heads": HK, "head_dim": d, "theta": theta,
            "pairing": pairing, "pos_offset": pos_offset,
            "tol": "f16" if f16 else "rope_f32"}, arrays


def case_rope_f32_half():
    # TinyLlama head shape of the RoPE config, positions 0..32
    return _rope_case("rope_f32", False, 33, 4, 2, 64, 1e4, ROPE_HALF, 111)


def case_rope_f32_interleaved_positions():
    # the reference's own pairing, positions up to 2^17 (large fp32 angles)
    pos = _rng(113).integers(0, 131072, size=21)
    return _rope_case("rope_f32", False, 21, 4, 2, 64, 1e4, ROPE_INTERLEAVED, 114, positions=pos)


def case_rope_f32_llama3_tail():
    # head_dim 128, theta 5e5, the last positions of an 8192-token prompt
    return _rope_case("rope_f32", False, 16, 2, 1, 128, 5e5, ROPE_HALF, 116, pos_offset=8176)


def case_rope_f16_llama3():
    # Q 32 x 128 / K 8 x 128, theta 5e5, positions 8183..8191
    return _rope_case("rope_f16", True, 9, 32, 8, 128, 5e5, ROPE_HALF, 118, pos_offset=8183)


def case_rope_f16_interleaved():
    return _rope_case("rope_f16", True, 12, 4, 1, 64, 1e4, ROPE_INTERLEAVED, 120)


def case_swiglu_f32():
    g, u = _normal(121, (3, 700), clip=8.0), _normal(122, (3, 700), clip=8.0)
    g[0, :12] = [0.0, -0.0, 1e-30, -1e-30, 8.0, -8.0, 80.0, -80.0, 100.0, -100.0, 3e4, -3e4]
    u[0, :12] = 1.0
    return {"op": "swiglu_f32", "tol": "f32"}, {"in_gate": g, "in_up": u,
                                               "want_out": orc.swiglu(g, u)}


def case_swiglu_f16():
    # ffn width of the SwiGLU config
    g, u = _h(_normal(123, (3, 5632), clip=8.0)), _h(_normal(124, (3, 5632), clip=8.0))
    return {"op": "swiglu_f16", "tol": "f16"}, {"in_gate": g, "in_up": u,
                                               "want_out": orc.swiglu(g, u, f16=True)}


def case_softmax_f32_reftest():
    x = orc.reftest_softmax_inputs(2048, 2048, 7)[:4].copy()
    return {"op": "softmax_f32", "tol": "f32"}, {
        "in_x": x, "want_out": orc.softmax(x), "want_reftest_cpu": orc.softmax_reftest_cpu(x)}


def case_softmax_f32_causal():
    # rows 0..7 and the last 8 rows of a 300 x 300 causal score matrix
    x = _normal(125, (16, 300), sigma=2.0)
    _causal(x[:8])
    _causal(x[8:], first_pos=292)
    return {"op": "softmax_f32", "tol": "f32"}, {"in_x": x, "want_out": orc.softmax(x)}


def case_softmax_f16_causal():
    # the last 8 rows of the 4096 x 4096 causal softmax config
    x = _causal(_normal(126, (8, 4096), sigma=2.0), first_pos=4088)
    xh = _h(x)
    return {"op": "softmax_f16", "tol": "f16"}, {"in_x": xh, "want_out": orc.softmax(xh, f16=True)}


def _table_bits(seed, shape):
    t = _rng(seed).integers(0, 1 << 16, size=shape).astype(np.uint16)
    return np.where((t & 0x7C00) == 0x7C00, t & 0x3FFF, t).astype(np.uint16)   # no inf/NaN


def case_embed_f16():
    table = _table_bits(127, (40, 64))
    ids = np.array([3, 0, 39, 3, -1, 40, 12345, 17, 8], np.int32)   # 3 out of range -> zero rows
    return {"op": "embed_f16", "tol": "exact"}, {
        "in_table": table, "in_ids": ids, "want_out": orc.embed(table, ids, f16=True)}


def case_embed_f32():
    table = _normal(128, (40, 96))
    ids = _rng(129).integers(0, 40, size=11).astype(np.int32)
    return {"op": "embed_f32", "tol": "exact"}, {
        "in_table": table, "in_ids": ids, "want_out": orc.embed(table, ids)}


def case_kv_append_f32_readback():
    L, S, H, d = 4, 32, 2, 64
    slice_ = H * d
    kc = np.zeros((L, S, H, d), np.float32)
    vc = np.zeros((L, S, H, d), np.float32)
    ks, vs = [], []
    for tok in range(16):
        k = (np.float32(tok) + np.arange(slice_, dtype=np.float32) / np.float32(slice_))
        v = np.full(slice_, -np.float32(tok), np.float32)
        ks.append(k)
        vs.append(v)
        for layer in range(L):
            orc.kv_append_inplace(kc, vc, k.reshape(1, H, d), v.reshape(1, H, d), layer, tok)
    return {"op": "kv_append_f32_tokens", "n_layers": L, "max_seq": S, "n_kv_heads": H,
            "head_dim": d, "tol": "exact"}, {
        "in_k": np.stack(ks), "in_v": np.stack(vs), "want_k_cache": kc, "want_v_cache": vc}


def case_kv_append_f16():
    L, S, H, d, layer, pos, T = 3, 12, 2, 64, 1, 3, 5
    kn, vn = _table_bits(130, (T, H, d)), _table_bits(131, (T, H, d))
    kc = np.full((L, S, H, d), 0xA5A5, np.uint16)
    vc = kc.copy()
    orc.kv_append_inplace(kc, vc, kn, vn, layer, pos, f16=True)
    return {"op": "kv_append_f16", "n_layers": L, "max_seq": S, "n_kv_heads": H, "head_dim": d,
            "layer": layer, "pos": pos, "guard": 0xA5A5, "tol": "exact"}, {
        "in_k": kn, "in_v": vn, "want_k_cache": kc, "want_v_cache": vc}


def _paged_slots(block_table, start, T):
    p = start + np.arange(T)
    return (np.asarray(block_table)[p // 16] * 16 + p % 16).astype(np.int32)


def case_paged_kv_append_f16():
    L, H, d, layer, nb = 2, 2, 64, 1, 6
    T, start = 40, 3
    slots = _paged_slots([4, 1, 5], start, T)      # tokens 3..42 of a sequence
    slots[9] = -1                                  # padding token: skipped
    slots[30] = nb * 16 + 2                        # block beyond the pool: skipped
    kn, vn = _table_bits(132, (T, H, d)), _table_bits(133, (T, H, d))
    blk = L * 16 * H * d
    kp = np.full(nb * blk, 0xA5A5, np.uint16)
    vp = kp.copy()
    orc.paged_kv_append_inplace(kp, vp, np.arange(nb, dtype=np.int64) * blk, slots, kn, vn,
                                layer, L, H, d)
    return {"op": "paged_kv_append_f16", "n_blocks": nb, "n_layers": L, "layer": layer,
            "n_kv_heads": H, "head_dim": d, "guard": 0xA5A5, "tol": "exact"}, {
        "in_k": kn, "in_v": vn, "in_slots": slots, "want_k_pool": kp, "want_v_pool": vp}


def case_rope_paged_kv_append_f16():
    # fused RoPE + paged append: Q rotated in place, rotated K and V into the pool
    L, H, HK, d, layer, nb, T, start, theta = 2, 4, 2, 128, 0, 5, 20, 14, 5e5
    q, k, v = (_h(_normal(134 + i, (T, n * d))) for i, n in enumerate((H, HK, HK)))
    slots = _paged_slots([3, 0, 4], start, T)
    pos = (start + np.arange(T)).astype(np.int32)
    wq = orc.rope(q, H, d, theta, ROPE_HALF, pos, 0, f16=True)
    wk = orc.rope(k, HK, d, theta, ROPE_HALF, pos, 0, f16=True)
    blk = L * 16 * HK * d
    kp = np.full(nb * blk, 0xA5A5, np.uint16)
    vp = kp.copy()
    orc.paged_kv_append_inplace(kp, vp, np.arange(nb, dtype=np.int64) * blk, slots, wk, v, layer,
                                L, HK, d)
    return {"op": "rope_paged_kv_append_f16", "n_heads": H, "n_kv_heads": HK, "head_dim": d,
            "theta": theta, "pairing": ROPE_HALF, "n_blocks": nb, "n_layers": L, "layer": layer,
            "guard": 0xA5A5, "tol": "f16"}, {
        "in_q": q, "in_k": k, "in_v": v, "in_positions": pos, "in_slots": slots,
        "want_q": wq, "want_k": wk, "want_k_pool": kp, "want_v_pool": vp}


def case_f16_to_f32():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)     # every binary16 value
    return {"op": "f16_to_f32", "tol": "exact"}, {"in_x": h, "want_out": orc.f16_to_f32(h)}


def case_flash_attention_f16():
    seq, H, HK, d = 24, 4, 2, 64
    q, k, v = (_h(_normal(140 + i, (seq, n, d))) for i, n in enumerate((H, HK, HK)))
    return {"op": "flash_attention_f16", "n_heads": H, "n_kv_heads": HK, "head_dim": d,
            "causal": 1, "tol": "attention"}, {
        "in_q": q, "in_k": k, "in_v": v, "want_out": orc.attention(q, k, v, H, HK, True, f16=True)}


def case_fp8_quantize():
    x = _h(_normal(150, (4, 256)) * np.float32(3.0))
    out = {}
    for fmt in (0, 1):
        for mode, gran, gs in ((0, 2, 128), (1, 1, 0)):
            tag = f"f{fmt}_m{mode}"
            q, sc = orc.fp8_quantize(x, fmt, gran, gs, mode)
            out[f"want_codes_{tag}"] = q
            out[f"want_scales_{tag}"] = sc
            out[f"want_deq_{tag}"] = orc.fp8_dequantize(q, sc, fmt, gran, gs, mode)
    out["in_x"] = x
    return {"op": "fp8_quantize", "tol": "exact",
            "variants": [[fmt, mode, gran, gs] for fmt in (0, 1)
                         for mode, gran, gs in ((0, 2, 128), (1, 1, 0))]}, out


CASES = {f.__name__[5:]: f for f in (
    case_rmsnorm_f32, case_rmsnorm_f16, case_add_rmsnorm_f32, case_add_rmsnorm_f16,
    case_rope_f32_half, case_rope_f32_interleaved_positions, case_rope_f32_llama3_tail,
    case_rope_f16_llama3, case_rope_f16_interleaved, case_swiglu_f32, case_swiglu_f16,
    case_softmax_f32_reftest, case_softmax_f32_causal, case_softmax_f16_causal,
    case_embed_f16, case_embed_f32, case_kv_append_f32_readback, case_kv_append_f16,
    case_paged_kv_append_f16, case_rope_paged_kv_append_f16, case_f16_to_f32,
    case_flash_attention_f16, case_fp8_quantize)}


# ---- independent float64 checks ------------------------------------------------------------
def _within(got, want, rtol, atol, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    same_inf = np.isinf(want) & (got == want)
    err = np.where(same_inf, 0.0, np.abs(got - want))
    bound = rtol * np.abs(np.where(np.isinf(want), 0.0, want)) + atol
    bad = ~(err <= bound)
    assert not bad.any(), f"{what}: {int(bad.sum())} values outside tolerance, max err {err.max():.3e}"
    return float(err.max()) if err.size else 0.0


def _f64(a, f16):
    return _w(a) if f16 else np.asarray(a, np.float64)


def _rmsnorm64(x, w, eps):
    return x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + eps) * w


def _rope64(x, n_heads, d, theta, pairing, positions):
    """kernels/rope.cu:33-41 in float64, with the fp32 angle of the reference:
    inv_freq = fp32(1 / fp32(theta^fp32(2i/d))), angle = fp32(pos * inv_freq)."""
    T = x.shape[0]
    x = x.reshape(T, -1)[:, :n_heads * d].reshape(T, n_heads, d)
    i = np.arange(d // 2)
    expo = (np.float32(2.0) * i.astype(np.float32)) / np.float32(d)
    inv = np.float32(1.0) / np.power(np.float64(theta), expo.astype(np.float64)).astype(np.float32)
    ang = (np.asarray(positions, np.float32)[:, None] * inv[None, :]).astype(np.float64)
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    if pairing == ROPE_HALF:
        x0, x1 = x[..., : d // 2], x[..., d // 2:]
    else:
        x0, x1 = x[..., 0::2], x[..., 1::2]
    y0, y1 = x0 * c - x1 * s, x0 * s + x1 * c
    y = np.empty_like(x)
    if pairing == ROPE_HALF:
        y[..., : d // 2], y[..., d // 2:] = y0, y1
    else:
        y[..., 0::2], y[..., 1::2] = y0, y1
    return y.reshape(T, n_heads * d)


def _softmax64(x):
    m = np.max(x, axis=1, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=1, keepdims=True)


def _attention64(q, k, v, H, HK, causal):
    seq, _, d = q.shape
    out = np.zeros_like(q)
    for h in range(H):
        g = h * HK // H
        s = q[:, h, :] @ k[:, g, :].T / np.sqrt(np.float32(d)).astype(np.float64)
        if causal:
            s = np.where(np.tril(np.ones((seq, k.shape[0]), bool), k.shape[0] - seq), s, -np.inf)
        out[:, h, :] = _softmax64(s) @ v[:, g, :]
    return out


def _ocp_decode(code, fmt):
    """OCP 8-bit floating point specification, E4M3FN (bias 7) and E5M2 (bias 15)."""
    code = np.asarray(code, np.int64)
    mbits, bias = (3, 7) if fmt == 0 else (2, 15)
    sign = np.where(code & 0x80, -1.0, 1.0)
    e = (code >> mbits) & ((1 << (7 - mbits)) - 1)
    m = code & ((1 << mbits) - 1)
    val = np.where(e == 0, m * 2.0 ** (1 - bias - mbits),
                   (1 + m / 2.0 ** mbits) * 2.0 ** (e.astype(np.float64) - bias))
    return sign * val


def independent_check(params, arrays):
    """Recompute the fixture's expected outputs without the oracle; returns the
    largest deviation seen (0 for bit-exact ops)."""
    op, a = params["op"], arrays
    f16 = op.endswith("_f16") or op == "fp8_quantize"
    tol = TOL.get(params["tol"])
    if op in ("rmsnorm_f32", "rmsnorm_f16"):
        # kernels/rmsnorm.cu:27-48, kernels/fp16_ops.cu:18-41
        want = _rmsnorm64(_f64(a["in_x"], f16), _f64(a["in_w"], f16), params["eps"])
        return _within(_f64(a["want_out"], f16), want, tol["rtol"], tol["atol"], op)
    if op in ("add_rmsnorm_f32", "add_rmsnorm_f16"):
        # src/fp16_forward.cu:213-216 (add) then rmsnorm of the stored sum
        xs = _f64(a["in_x"], f16) + _f64(a["in_d"], f16)
        if f16:
            xs16 = xs.astype(np.float16)                    # one rounding of an exact sum
            assert np.array_equal(xs16.view(np.uint16), a["want_x"]), op
            xs = xs16.astype(np.float64)
        else:
            assert np.array_equal(xs.astype(np.float32), a["want_x"]), op
        want = _rmsnorm64(xs, _f64(a["in_w"], f16), params["eps"])
        return _within(_f64(a["want_out"], f16), want, tol["rtol"], tol["atol"], op)
    if op in ("rope_f32", "rope_f16"):
        T = a["in_q"].shape[0]
        pos = a["in_positions"] if "in_positions" in a else params["pos_offset"] + np.arange(T)
        m = 0.0
        for nm, heads in (("q", params["n_heads"]), ("k", params["n_kv_heads"])):
            want = _rope64(_f64(a[f"in_{nm}"], f16), heads, params["head_dim"], params["theta"],
                           params["pairing"], pos)
            m = max(m, _within(_f64(a[f"want_{nm}"], f16), want, tol["rtol"], tol["atol"],
                               f"{op} {nm}"))
        return m
    if op in ("swiglu_f32", "swiglu_f16"):
        # kernels/feedforward.cu:4-6,21-24: silu(g) * u
        g, u = _f64(a["in_gate"], f16), _f64(a["in_up"], f16)
        with np.errstate(over="ignore"):
                return _within(_f64(a["want_out"], f16), g / (1.0 + np.exp(-g)) * u, tol["rtol"],
                           tol["atol"], op)
    if op in ("softmax_f32", "softmax_f16"):
        # kernels/softmax.cu:44-85
        want = _softmax64(_f64(a["in_x"], f16))
        m = _within(_f64(a["want_out"], f16), want, tol["rtol"], tol["atol"], op)
        if "want_reftest_cpu" in a:
            # tests/test_softmax.cu:88-106: max abs error < 1e-5 against its cpu_softmax
            assert np.abs(a["want_out"] - a["want_reftest_cpu"]).max() < 1e-5
            assert np.abs(a["want_reftest_cpu"].astype(np.float64).sum(axis=1) - 1).max() < 1e-5
        return m
    if op in ("embed_f16", "embed_f32"):
        t, ids = a["in_table"], a["in_ids"]
        ok = (ids >= 0) & (ids < t.shape[0])
        want = np.zeros((ids.size, t.shape[1]), t.dtype)
        want[ok] = t[ids[ok]]
        assert np.array_equal(want.view(np.uint8), a["want_out"].view(np.uint8)), op
        return 0.0
    if op == "kv_append_f32_tokens":
        L, S, H, d = (params[k] for k in ("n_layers", "max_seq", "n_kv_heads", "head_dim"))
        n = a["in_k"].shape[0]
        kc = np.zeros((L, S, H * d), np.float32)
        vc = np.zeros((L, S, H * d), np.float32)
        kc[:, :n], vc[:, :n] = a["in_k"][None], a["in_v"][None]
        assert np.array_equal(kc.reshape(a["want_k_cache"].shape), a["want_k_cache"])
        assert np.array_equal(vc.reshape(a["want_v_cache"].shape), a["want_v_cache"])
        assert a["want_k_cache"][0, 7, 0, 0] == 7.0           # tests/test_kvcache.cu:63-68
        return 0.0
    if op == "kv_append_f16":
        kc = np.full(a["want_k_cache"].shape, params["guard"], np.uint16)
        vc = kc.copy()
        p, T = params["pos"], a["in_k"].shape[0]
        kc[params["layer"], p:p + T], vc[params["layer"], p:p + T] = a["in_k"], a["in_v"]
        assert np.array_equal(kc, a["want_k_cache"]) and np.array_equal(vc, a["want_v_cache"])
        return 0.0
    if op in ("paged_kv_append_f16", "rope_paged_kv_append_f16"):
        nb, L, H, d, layer = (params[k] for k in ("n_blocks", "n_layers", "n_kv_heads",
                                                  "head_dim", "layer"))
        kp = np.full((nb, L, 16, H * d), params["guard"], np.uint16)
        vp = kp.copy()
        knew = a["want_k"] if op.startswith("rope") else a["in_k"]
        for t, s in enumerate(a["in_slots"]):
            if 0 <= s < nb * 16:                              # include/paged_kvcache.h:9-25
                kp[s // 16, layer, s % 16] = knew[t].reshape(-1)
                vp[s // 16, layer, s % 16] = a["in_v"][t].reshape(-1)
        assert np.array_equal(kp.reshape(-1), a["want_k_pool"]), op
        assert np.array_equal(vp.reshape(-1), a["want_v_pool"]), op
        if op.startswith("rope"):
            m = 0.0
            for nm, heads in (("q", params["n_heads"]), ("k", params["n_kv_heads"])):
                want = _rope64(_w(a[f"in_{nm}"]), heads, d, params["theta"], params["pairing"],
                               a["in_positions"])
                m = max(m, _within(_w(a[f"want_{nm}"]), want, tol["rtol"], tol["atol"], nm))
            return m
        return 0.0
    if op == "f16_to_f32":
        h = a["in_x"].view(np.float16).astype(np.float32)
        nan = np.isnan(h)
        assert np.array_equal(np.isnan(a["want_out"]), nan)
        assert np.array_equal(h[~nan].view(np.uint32), a["want_out"][~nan].view(np.uint32))
        return 0.0
    if op == "flash_attention_f16":
        # kernels/flash_attention.cu:29-182 in float64
        q, k, v = (_w(a[n]) for n in ("in_q", "in_k", "in_v"))
        want = _attention64(q, k, v, params["n_heads"], params["n_kv_heads"], params["causal"])
        return _within(_w(a["want_out"]), want, 2e-3, 2e-3 * np.abs(v).max(), op)
    if op == "fp8_quantize":
        # quantlib_src/kernels/fp8_convert.cu:15-173: scale = fmax / max|x| over the group
        # (the reference's max sees offsets < 32 mod 128 of each group); OCP codes are
        # the nearest representable value
        x = _w(a["in_x"])
        m = 0.0
        for fmt, mode, gran, gs in params["variants"]:
            tag = f"f{fmt}_m{mode}"
            fmax = 448.0 if fmt == 0 else 57344.0
            sc, q = a[f"want_scales_{tag}"], a[f"want_codes_{tag}"]
            if gran == 2:
                g = np.abs(x.reshape(-1, gs))
                seen = g[:, (np.arange(gs) % 128) < 32] if mode == 0 else g
                want_sc = (np.float32(fmax) / seen.max(axis=1).astype(np.float32))
            else:
                want_sc = np.float32(fmax) / np.abs(x).max(axis=1).astype(np.float32)
            assert np.array_equal(sc, want_sc.astype(np.float32)), tag
            if mode == 1:
                per = np.repeat(sc, x.size // sc.size).reshape(x.shape).astype(np.float64)
                scaled = (x.astype(np.float32) * per.astype(np.float32)).astype(np.float64)
                dec = _ocp_decode(q, fmt)
                grid = _ocp_decode(np.arange(256), fmt)
                grid = grid[np.isfinite(grid)]
                nearest = np.abs(scaled[..., None] - grid).min(axis=-1)
                assert np.all(np.abs(dec - np.clip(scaled, -fmax, fmax)) <= nearest + 1e-12), tag
                deq = _w(a[f"want_deq_{tag}"])
                m = max(m, _within(deq, dec / per, 2.0 ** -10, 2.0 ** -24, f"deq {tag}"))
        return m
    raise KeyError(op)


# ---- files -----------------------------------------------------------------------------------
def _sha256(path: pathlib.Path) -> str:
    return hashlib.sha256(path.read_bytes()).hexdigest()


def load(name: str):
    """(params, arrays) of one committed fixture."""
    man = json.loads(MANIFEST.read_text())
    params = man["fixtures"][name]["params"]
    with np.load(HERE / f"{name}.npz", allow_pickle=False) as z:
        arrays = {k: z[k] for k in z.files}
    return params, arrays


def names():
    return sorted(json.loads(MANIFEST.read_text())["fixtures"])


def main():
    fixtures = {}
    for name, fn in CASES.items():
        params, arrays = fn()
        dev = independent_check(params, arrays)
        path = HERE / f"{name}.npz"
        np.savez_compressed(path, **arrays)
        fixtures[name] = {"file": path.name, "sha256": _sha256(path), "params": params,
                          "max_dev_vs_float64": dev}
        print(f"{name:40s} {path.stat().st_size:8d} B  max dev vs float64 {dev:.3e}")
    MANIFEST.write_text(json.dumps({"generator": "tests/golden/make_golden.py",
                                    "fixtures": fixtures}, indent=1, sort_keys=True) + "\n")


if __name__ == "__main__":
    main()
