"""GPU parity of greedy sampling (ql_argmax_*) and of the decoder-layer engine
(ql_engine_*): a small fp16 Llama-style layer run on batcher steps (a mixed
prefill step, then an all-decode step that takes the split-decode path) against
the oracle composed in the same order -- rmsnorm, x W^T, RoPE at the step's
positions, causal attention over each sequence's K/V history, residual add,
SwiGLU -- with a binary16 rounding after every stage, as the engine stores them.
The FP8-weight layer (ql_engine_layer_fp8) is checked the same way against the
oracle layer on the oracle codec's dequantized weights.

Layer tolerance, |got - want| <= 2e-2*|want| + 1e-2*max|want|: both sides round
every stage to binary16 (2^-11 relative) but accumulate GEMMs in different
orders (fp32 in hipBLASLt, double in the oracle), so single-ulp differences in
intermediate values propagate through up to six dependent stages."""
import ctypes

import numpy as np
import pytest

import oracle as orc
import quantlib_amd as ql
from helpers import check_close, dev, empty, f16_bits_to_f32, host, normal, stream, to_f16_bits
from test_gpu_attention import PagedPool

pytestmark = pytest.mark.gpu


# ---- argmax --------------------------------------------------------------------------------
@pytest.mark.parametrize("rows,cols,pad", [(1, 5, 0), (7, 32000, 0), (3, 128256, 0), (5, 1001, 3),
                                           (64, 4096, 8)])
@pytest.mark.parametrize("f16", [False, True])
def test_argmax_matches_oracle(rows, cols, pad, f16):
    ld = cols + pad
    x = normal(rows * cols + pad, (rows, ld), 3.0)
    if rows >= 3:
        x[0, :] = -np.inf
        x[1, :cols // 2] = np.nan
        x[2, 7 % cols] = x[2, (cols - 1)] = 50.0          # tie: first index wins
    if rows >= 5 and not f16:
        # the scan's start value -1e20f (src/continuous_batch.cu:15): a row at or
        # below it gives 0; in the next one the last value is the first above it
        x[3, :] = -1e20
        x[3, cols // 3] = -np.inf
        x[4, :] = -2e20
        x[4, cols - 1] = -9.9e19
    if f16:
        xb = to_f16_bits(x)
        want = orc.argmax(f16_bits_to_f32(xb)[:, :cols])
    else:
        xb = x
        want = orc.argmax(x[:, :cols])
    out = empty((rows,), np.int32)
    d = dev(xb)
    ql.call("ql_argmax_f16" if f16 else "ql_argmax_f32", d.ptr, rows, cols, ld, out.ptr, stream())
    assert list(host(out)) == list(want)


# ---- decoder layer -------------------------------------------------------------------------
H, HK, HD, DM, FF = 4, 2, 64, 256, 512
THETA, EPS, PAIR = 1e4, 1e-5, ql.ROPE_HALF


def layer_weights(seed):
    r = lambda s, shape, scale: to_f16_bits(normal(seed + s, shape, scale))
    qkv_out = (H + 2 * HK) * HD
    return {"attn_norm": to_f16_bits(np.random.default_rng(seed).uniform(0.5, 1.5, DM).astype(np.float32)),
            "wqkv": r(1, (qkv_out, DM), DM ** -0.5), "wo": r(2, (DM, H * HD), (H * HD) ** -0.5),
            "ffn_norm": to_f16_bits(np.random.default_rng(seed + 3).uniform(0.5, 1.5, DM).astype(np.float32)),
            "w_gate": r(4, (FF, DM), DM ** -0.5), "w_up": r(5, (FF, DM), DM ** -0.5),
            "w_down": r(6, (DM, FF), FF ** -0.5)}


def oracle_layer(x, delta_in, w, plan, hist):
    """One layer on the host; hist[req] holds (K rows, V rows) of earlier steps."""
    if delta_in is None:
        x1, y = x, orc.rmsnorm(x, w["attn_norm"], EPS, f16=True)
    else:
        x1, y = orc.add_rmsnorm(x, delta_in, w["attn_norm"], EPS, f16=True)
    qkv = orc.matmul(y, w["wqkv"])
    q = np.ascontiguousarray(qkv[:, :H * HD])
    k = np.ascontiguousarray(qkv[:, H * HD:(H + HK) * HD])
    v = np.ascontiguousarray(qkv[:, (H + HK) * HD:])
    pos = plan["positions"]
    q = orc.rope(q, H, HD, THETA, PAIR, positions=pos, f16=True)
    k = orc.rope(k, HK, HD, THETA, PAIR, positions=pos, f16=True)
    attn = np.zeros((plan["n_rows"], H * HD), np.uint16)
    cu = plan["cu_q_lens"]
    for i, rid in enumerate(plan["req_ids"]):
        sl = slice(cu[i], cu[i + 1])
        ks, vs = hist.setdefault(int(rid), ([], []))
        ks.extend(k[sl])
        vs.extend(v[sl])
        kk = np.stack(ks).reshape(-1, HK, HD)
        vv = np.stack(vs).reshape(-1, HK, HD)
        attn[sl] = orc.attention(q[sl].reshape(-1, H, HD), kk, vv, H, HK, True, f16=True).reshape(-1, H * HD)
    o = orc.matmul(attn, w["wo"])
    x2 = orc.add(x1, o, f16=True)
    y2 = orc.rmsnorm(x2, w["ffn_norm"], EPS, f16=True)
    mid = orc.swiglu(orc.matmul(y2, w["w_gate"]), orc.matmul(y2, w["w_up"]), f16=True)
    return x2, orc.matmul(mid, w["w_down"])


def check_layer(got, want, what):
    g, wv = f16_bits_to_f32(got), f16_bits_to_f32(want)
    check_close(g, wv, 2e-2, 1e-2 * float(np.abs(wv).max()), what)


def step_device(plan, pool, L, keep):
    arrs = {k: dev(np.ascontiguousarray(plan[k], np.int32)) for k in
            ("positions", "slot_mapping", "cu_q_lens", "ctx_lens")}
    arrs["block_tables"] = dev(np.ascontiguousarray(plan["block_tables"], np.int32).reshape(-1))
    keep.append(arrs)
    return ql.StepDevice(plan["n_rows"], plan["n_seqs"], plan["max_q_len"], plan["max_ctx_len"],
                         plan["max_blocks"], arrs["positions"].ptr, arrs["slot_mapping"].ptr,
                         arrs["cu_q_lens"].ptr, arrs["ctx_lens"].ptr, arrs["block_tables"].ptr,
                         pool.kptrs.ptr, pool.vptrs.ptr, pool.nb, L)


def run_engine_steps(eng, layer_call, weights, prompts, n_steps, max_gen=8):
    """Batcher steps through the engine's layers (layer_call(l, x, delta_in, delta_out, sd))
    and logits, each stage checked against the oracle layer on `weights` (fp16 bits)."""
    L, nblk, vocab = len(weights), 32, 512
    final_norm = to_f16_bits(np.random.default_rng(9).uniform(0.5, 1.5, DM).astype(np.float32))
    lm_head = to_f16_bits(normal(10, (vocab, DM), DM ** -0.5))
    d_final, d_lm = dev(final_norm), dev(lm_head)
    pool = PagedPool(nblk, L, HK, HD)
    b = ql.Batcher(nblk, 4)
    for rid, n in prompts.items():
        b.add(rid, np.arange(n, dtype=np.int32), max_gen)
    hist = [dict() for _ in range(L)]
    keep = []
    for step in range(n_steps):
        plan = b.plan()
        T = plan["n_rows"]
        sd = step_device(plan, pool, L, keep)
        x = to_f16_bits(normal(500 + step, (T, DM)))
        dx = dev(x)
        deltas = [empty((T * DM,), np.uint16) for _ in range(L)]
        xo, delta = x, None
        for l in range(L):
            layer_call(l, dx.ptr, deltas[l - 1].ptr if l else None, deltas[l].ptr, sd)
            xo, delta = oracle_layer(xo, delta, weights[l], plan, hist[l])
            check_layer(host(dx, shape=(T, DM)), xo, f"step {step} layer {l} residual")
            check_layer(host(deltas[l], shape=(T, DM)), delta, f"step {step} layer {l} mlp out")
            xo = host(dx, shape=(T, DM)).copy()      # continue from the GPU's stream
            delta = host(deltas[l], shape=(T, DM)).copy()
        # logits of the sampled rows and greedy tokens
        n = plan["n_seqs"]
        rows_d = dev(plan["sample_rows"])
        logits = empty((n * vocab,), np.uint16)
        toks = empty((n,), np.int32)
        ql.call("ql_engine_logits_f16", eng, dx.ptr, deltas[-1].ptr, d_final.ptr, d_lm.ptr, vocab,
                rows_d.ptr, n, T, logits.ptr, toks.ptr, stream())
        xf = orc.add(xo, delta, f16=True)
        yf = orc.rmsnorm(xf, final_norm, EPS, f16=True)
        want = orc.matmul(yf[plan["sample_rows"]], lm_head)
        got = host(logits, shape=(n, vocab))
        check_layer(got, want, f"step {step} logits")
        assert list(host(toks)) == list(orc.argmax(f16_bits_to_f32(got)))
        b.commit(host(toks))
        assert step == 0 or plan["max_q_len"] == 1        # later steps are all decodes


@pytest.mark.parametrize("prompts", [{0: 20, 1: 33, 2: 5},    # mixed prefill, then decodes
                                     {0: 45}])                 # one fresh prompt: contiguous attention
def test_engine_layers_steps_and_logits_match_oracle(prompts):
    L = 2
    weights = [layer_weights(100 * (l + 1)) for l in range(L)]
    dw = [{k: dev(v) for k, v in w.items()} for w in weights]
    lw = [ql.LayerWeights(*(d[k].ptr for k in ("attn_norm", "wqkv", "wo", "ffn_norm", "w_gate", "w_up",
                                               "w_down"))) for d in dw]
    dims = ql.LayerDims(DM, H, HK, HD, FF, THETA, EPS, PAIR)
    eng = ctypes.c_void_p()
    ql.call("ql_engine_create", ctypes.byref(dims), 64, 8, 256, ctypes.byref(eng))
    try:
        run_engine_steps(eng, lambda l, x, di, do, sd: ql.call(
            "ql_engine_layer_f16", eng, ctypes.byref(lw[l]), l, x, di, do, ctypes.byref(sd), stream()),
            weights, prompts, 3)
    finally:
        ql.call("ql_engine_destroy", eng)


MATS = ("wqkv", "wo", "w_gate", "w_up", "w_down")


@pytest.mark.parametrize("fmt,gran,gs,mode,prompts", [
    # the reference's quantize_model: E4M3, groups of 128, its own codec; a 58-row prefill
    (ql.FP8_E4M3, ql.QUANT_PER_GROUP, 128, ql.FP8_MODE_REFERENCE, {0: 20, 1: 33, 2: 5}),
    # per-channel OCP codes; a 100-row prefill takes the dequantize + library GEMM path
    (ql.FP8_E4M3, ql.QUANT_PER_CHANNEL, 0, ql.FP8_MODE_OCP, {0: 70, 1: 30}),
    # reference codes checked free of the codes whose reference decode differs
    (ql.FP8_E4M3, ql.QUANT_PER_GROUP, 128, ql.FP8_MODE_REFERENCE_CLEAN, {0: 9, 1: 4})])
def test_engine_fp8_layers_match_oracle(fmt, gran, gs, mode, prompts):
    L = 2
    src = [layer_weights(100 * (l + 1)) for l in range(L)]
    qmode = ql.FP8_MODE_REFERENCE if mode == ql.FP8_MODE_REFERENCE_CLEAN else mode
    count = empty((1,), np.uint64)
    deq, keep, lw = [], [], []
    for w in src:
        d = dict(w)
        fw = {}
        for k in MATS:
            q, sc = orc.fp8_quantize(w[k], fmt, gran, gs, qmode)
            d[k] = orc.fp8_dequantize(q, sc, fmt, gran, gs, qmode)
            dq, ds = dev(q), dev(sc)
            if mode == ql.FP8_MODE_REFERENCE_CLEAN:
                ql.call("ql_fp8_count_ref_special", dq.ptr, q.size, fmt, count.ptr, stream())
                assert int(host(count)[0]) == 0
            keep += [dq, ds]
            fw[k] = ql.FP8Weight(dq.ptr, ds.ptr)
        deq.append(d)
        dn, fn = dev(w["attn_norm"]), dev(w["ffn_norm"])
        keep += [dn, fn]
        lw.append(ql.LayerWeightsFP8(dn.ptr, fw["wqkv"], fw["wo"], fn.ptr, fw["w_gate"], fw["w_up"],
                                     fw["w_down"], fmt, gran, gs, mode))
    dims = ql.LayerDims(DM, H, HK, HD, FF, THETA, EPS, PAIR)
    eng = ctypes.c_void_p()
    ql.call("ql_engine_create_fp8", ctypes.byref(dims), 128, 8, 256, gran, gs, ctypes.byref(eng))
    try:
        run_engine_steps(eng, lambda l, x, di, do, sd: ql.call(
            "ql_engine_layer_fp8", eng, ctypes.byref(lw[l]), l, x, di, do, ctypes.byref(sd), stream()),
            deq, prompts, 3)
    finally:
        ql.call("ql_engine_destroy", eng)


def fp8_layer(w, keep, fmt=ql.FP8_E4M3, gran=ql.QUANT_PER_GROUP, gs=128, mode=ql.FP8_MODE_REFERENCE):
    """ql_layer_weights_fp8 of one layer's fp16 weights, quantized by the oracle codec."""
    fw = {}
    for k in MATS:
        q, sc = orc.fp8_quantize(w[k], fmt, gran, gs, mode)
        dq, ds = dev(q), dev(sc)
        keep += [dq, ds]
        fw[k] = ql.FP8Weight(dq.ptr, ds.ptr)
    dn, fn = dev(w["attn_norm"]), dev(w["ffn_norm"])
    keep += [dn, fn]
    return ql.LayerWeightsFP8(dn.ptr, fw["wqkv"], fw["wo"], fn.ptr, fw["w_gate"], fw["w_up"], fw["w_down"],
                              fmt, gran, gs, mode)


@pytest.mark.parametrize("kind", ["f16", "fp8"])
def test_decode_step_graph_replays_match_eager(kind):
    """A 2-layer decode step captured with ql_graph_begin/end and replayed three
    times, with eager work and synchronisations between the replays: every
    replay reproduces the eager step bit for bit (residual stream, MLP outputs)."""
    L = 2
    weights = [layer_weights(100 * (l + 1)) for l in range(L)]
    keep = []
    if kind == "f16":
        dw = [{k: dev(v) for k, v in w.items()} for w in weights]
        keep += dw
        lw = [ql.LayerWeights(*(d[k].ptr for k in ("attn_norm", "wqkv", "wo", "ffn_norm", "w_gate", "w_up",
                                                   "w_down"))) for d in dw]
        fn = "ql_engine_layer_f16"
    else:
        lw = [fp8_layer(w, keep) for w in weights]
        fn = "ql_engine_layer_fp8"
    dims = ql.LayerDims(DM, H, HK, HD, FF, THETA, EPS, PAIR)
    eng = ctypes.c_void_p()
    ql.call("ql_engine_create_fp8", ctypes.byref(dims), 64, 8, 256, ql.QUANT_PER_GROUP, 128, ctypes.byref(eng))
    pool = PagedPool(32, L, HK, HD)
    b = ql.Batcher(32, 4)
    for rid, n in {0: 20, 1: 33, 2: 5}.items():
        b.add(rid, np.arange(n, dtype=np.int32), 8)
    st = stream()
    graph = ctypes.c_void_p()

    def run_step(sd, dx, deltas):
        for l in range(L):
            ql.call(fn, eng, ctypes.byref(lw[l]), l, dx.ptr, deltas[l - 1].ptr if l else None, deltas[l].ptr,
                    ctypes.byref(sd), st)
    try:
        # prefill step, eagerly (fills the K/V history)
        plan = b.plan()
        sd = step_device(plan, pool, L, keep)
        dx = dev(to_f16_bits(normal(1, (plan["n_rows"], DM))))
        deltas = [empty((plan["n_rows"] * DM,), np.uint16) for _ in range(L)]
        run_step(sd, dx, deltas)
        b.commit(np.zeros(plan["n_seqs"], np.int32))
        # decode step: eager reference (also the warm-up of its GEMM shapes)
        plan = b.plan()
        assert plan["max_q_len"] == 1
        T = plan["n_rows"]
        sd = step_device(plan, pool, L, keep)
        x0 = to_f16_bits(normal(2, (T, DM)))
        dx = dev(x0)
        deltas = [empty((T * DM,), np.uint16) for _ in range(L)]
        run_step(sd, dx, deltas)
        want_x = host(dx, shape=(T, DM)).copy()
        want_d = [host(d, shape=(T, DM)).copy() for d in deltas]
        # capture the same step
        dx.upload(x0)
        ql.call("ql_graph_begin", st)
        try:
            run_step(sd, dx, deltas)
        finally:
            ql.call("ql_graph_end", st, ctypes.byref(graph))
        scratch = [dev(to_f16_bits(normal(3, (T, FF)))) for _ in range(3)]
        for rep in range(3):
            dx.upload(x0)
            for d in deltas:
                d.fill_bytes(0)
            # eager work between replays on the same stream
            ql.call("ql_swiglu_f16", scratch[0].ptr, scratch[1].ptr, scratch[2].ptr, T, FF, st)
            ql.call("ql_graph_launch", graph, st)
            ql.synchronize()
            assert np.array_equal(host(dx, shape=(T, DM)), want_x), f"replay {rep}: residual stream"
            for l in range(L):
                assert np.array_equal(host(deltas[l], shape=(T, DM)), want_d[l]), f"replay {rep}: layer {l}"
    finally:
        if graph.value:
            ql.call("ql_graph_destroy", graph)
        ql.call("ql_engine_destroy", eng)


# ---- tuned library GEMM plans ----------------------------------------------------------------
@pytest.mark.parametrize("M,N,K", [(1, 1536, 512), (5, 512, 1536), (64, 1024, 256)])
def test_gemm_tune_keeps_results_within_tolerance(M, N, K):
    x = to_f16_bits(normal(71 + M, (M, K)))
    w = to_f16_bits(normal(72 + N, (N, K)) * np.float32(K ** -0.5))
    dx, dw = dev(x), dev(w)
    want = orc.matmul(x, w)
    outs = []
    # the untuned plan, then tuned twice in a row (timing may pick another candidate
    # the second time), then the last plan once more
    for tune in (False, True, True, False):
        if tune:
            ql.call("ql_gemm_tune_f16", M, N, K, stream())
        y = empty((M * N,), np.uint16)
        ql.call("ql_gemm_f16", dx.ptr, dw.ptr, y.ptr, M, N, K, stream())
        got = host(y, shape=(M, N))
        # fp32 accumulation in any order, one binary16 rounding of the result
        bound = 2.0 ** -10 * np.abs(f16_bits_to_f32(want)) + 2.0 ** -10 * (
            np.abs(f16_bits_to_f32(x)).astype(np.float64) @ np.abs(f16_bits_to_f32(w)).T.astype(np.float64))
        err = np.abs(f16_bits_to_f32(got).astype(np.float64) - f16_bits_to_f32(want))
        assert np.all(err <= bound), f"gemm {M}x{N}x{K} tuned={tune}: max err {err.max():.3e}"
        outs.append(got)
    assert np.array_equal(outs[2], outs[3])   # one plan: identical results
    for bad in ((0, N, K), (M, -1, K), (M, N, 0)):
        with pytest.raises(ql.QLError):
            ql.call("ql_gemm_tune_f16", *bad, stream())


def test_engine_layers_after_tuning_match_oracle():
    L = 2
    prompts = {0: 20, 1: 33, 2: 5}           # a 58-row prefill, then 3-row decodes
    weights = [layer_weights(100 * (l + 1)) for l in range(L)]
    dw = [{k: dev(v) for k, v in w.items()} for w in weights]
    lw = [ql.LayerWeights(*(d[k].ptr for k in ("attn_norm", "wqkv", "wo", "ffn_norm", "w_gate", "w_up",
                                               "w_down"))) for d in dw]
    dims = ql.LayerDims(DM, H, HK, HD, FF, THETA, EPS, PAIR)
    eng = ctypes.c_void_p()
    ql.call("ql_engine_create", ctypes.byref(dims), 64, 8, 256, ctypes.byref(eng))
    try:
        for rows in (58, 3):
            ql.call("ql_engine_tune", eng, rows, stream())
        with pytest.raises(ql.QLError):
            ql.call("ql_engine_tune", eng, 65, stream())    # beyond the engine's max_rows
        run_engine_steps(eng, lambda l, x, di, do, sd: ql.call(
            "ql_engine_layer_f16", eng, ctypes.byref(lw[l]), l, x, di, do, ctypes.byref(sd), stream()),
            weights, prompts, 3)
    finally:
        ql.call("ql_engine_destroy", eng)


# ---- the engine at the benched layer shape ------------------------------------------------
# Llama-3-8B-shaped layer of fp16_layer_forward (src/fp16_forward.cu:167-223): hidden 4096,
# 32 query / 8 KV heads of 128, ffn 14336, rotate-half RoPE at theta 5e5.  The oracle GEMMs
# at these widths take ~0.7 s per 400 M multiply-adds, so every row goes through the QKV
# product (attention needs all K/V rows) but only sampled rows through attention, the output
# projection and the MLP.
C5 = {"DM": 4096, "H": 32, "HK": 8, "HD": 128, "FF": 14336, "THETA": 5e5}


def c5_weights(seed):
    c = C5
    r = lambda s, shape, scale: to_f16_bits(normal(seed + s, shape, scale))
    return {"attn_norm": to_f16_bits(np.random.default_rng(seed).uniform(0.5, 1.5, c["DM"]).astype(np.float32)),
            "wqkv": r(1, ((c["H"] + 2 * c["HK"]) * c["HD"], c["DM"]), c["DM"] ** -0.5),
            "wo": r(2, (c["DM"], c["H"] * c["HD"]), (c["H"] * c["HD"]) ** -0.5),
            "ffn_norm": to_f16_bits(np.random.default_rng(seed + 3).uniform(0.5, 1.5, c["DM"]).astype(np.float32)),
            "w_gate": r(4, (c["FF"], c["DM"]), c["DM"] ** -0.5), "w_up": r(5, (c["FF"], c["DM"]), c["DM"] ** -0.5),
            "w_down": r(6, (c["DM"], c["FF"]), c["FF"] ** -0.5)}


def oracle_layer_rows(x, delta_in, w, plan, hist, rows):
    """The oracle layer of oracle_layer at the C5 dims, returning the residual
    stream and MLP output of `rows` only; hist[req] gains every row's K and V."""
    c = C5
    H_, HK_, HD_ = c["H"], c["HK"], c["HD"]
    if delta_in is None:
        x1, y = x, orc.rmsnorm(x, w["attn_norm"], EPS, f16=True)
    else:
        x1, y = orc.add_rmsnorm(x, delta_in, w["attn_norm"], EPS, f16=True)
    qkv = orc.matmul(y, w["wqkv"])
    pos = plan["positions"]
    q = orc.rope(np.ascontiguousarray(qkv[:, :H_ * HD_]), H_, HD_, c["THETA"], PAIR, positions=pos, f16=True)
    k = orc.rope(np.ascontiguousarray(qkv[:, H_ * HD_:(H_ + HK_) * HD_]), HK_, HD_, c["THETA"], PAIR,
                 positions=pos, f16=True)
    v = np.ascontiguousarray(qkv[:, (H_ + HK_) * HD_:])
    cu = plan["cu_q_lens"]
    seq_of = np.searchsorted(cu, np.arange(plan["n_rows"]), side="right") - 1
    before = {}
    for i, rid in enumerate(plan["req_ids"]):
        ks, vs = hist.setdefault(int(rid), ([], []))
        before[i] = len(ks)
        ks.extend(k[cu[i]:cu[i + 1]])
        vs.extend(v[cu[i]:cu[i + 1]])
    attn = np.zeros((len(rows), H_ * HD_), np.uint16)
    for j, r in enumerate(rows):
        i = int(seq_of[r])
        ks, vs = hist[int(plan["req_ids"][i])]
        n = before[i] + (r - cu[i]) + 1          # keys up to this row's position (causal)
        kk = np.stack(ks[:n]).reshape(n, HK_, HD_)
        vv = np.stack(vs[:n]).reshape(n, HK_, HD_)
        attn[j] = orc.attention(q[r:r + 1].reshape(1, H_, HD_), kk, vv, H_, HK_, True, f16=True).reshape(-1)
    x2 = orc.add(x1[rows], orc.matmul(attn, w["wo"]), f16=True)
    y2 = orc.rmsnorm(x2, w["ffn_norm"], EPS, f16=True)
    mid = orc.swiglu(orc.matmul(y2, w["w_gate"]), orc.matmul(y2, w["w_up"]), f16=True)
    return x2, orc.matmul(mid, w["w_down"])


@pytest.mark.parametrize("prompts", [{0: 64},            # one fresh prompt: contiguous attention
                                     {0: 40, 1: 24}])    # two prompts: paged prefill attention
def test_engine_layer_c5_shape_prefill_and_decode(prompts):
    """One C5-shaped layer (ql_engine_layer_f16) for a prefill step and then an
    all-decode step (split decode over the paged pool), sampled rows of the
    residual stream and of the MLP output against the oracle-composed layer."""
    c = C5
    w = c5_weights(300)
    dw = {k: dev(v) for k, v in w.items()}
    lw = ql.LayerWeights(*(dw[k].ptr for k in ("attn_norm", "wqkv", "wo", "ffn_norm", "w_gate", "w_up",
                                               "w_down")))
    dims = ql.LayerDims(c["DM"], c["H"], c["HK"], c["HD"], c["FF"], c["THETA"], EPS, PAIR)
    eng = ctypes.c_void_p()
    ql.call("ql_engine_create", ctypes.byref(dims), 64, 4, 256, ctypes.byref(eng))
    pool = PagedPool(16, 1, c["HK"], c["HD"])
    b = ql.Batcher(16, 4)
    for rid, n in prompts.items():
        b.add(rid, np.arange(n, dtype=np.int32), 4)
    hist, keep = {}, []
    try:
        for step in range(2):
            plan = b.plan()
            T = plan["n_rows"]
            assert (step == 0) == (plan["max_q_len"] > 1)
            sd = step_device(plan, pool, 1, keep)
            x = to_f16_bits(normal(900 + step, (T, c["DM"])))
            dx, dd = dev(x), empty((T * c["DM"],), np.uint16)
            ql.call("ql_engine_layer_f16", eng, ctypes.byref(lw), 0, dx.ptr, None, dd.ptr, ctypes.byref(sd),
                    stream())
            rows = [0, 17, 39, 40, T - 1] if T > 1 else [0]
            rows = sorted(set(r for r in rows if r < T))
            wx, wd = oracle_layer_rows(x, None, w, plan, hist, rows)
            check_layer(host(dx, shape=(T, c["DM"]))[rows], wx, f"C5 step {step} residual")
            check_layer(host(dd, shape=(T, c["DM"]))[rows], wd, f"C5 step {step} mlp out")
            b.commit(np.full(plan["n_seqs"], 7, np.int32))
    finally:
        ql.call("ql_engine_destroy", eng)
