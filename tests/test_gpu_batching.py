"""Serving steps end to end on the GPU: the batcher's plans drive the paged KV
append and the paged attention (mixed prefill + decode steps, then decode-only
steps), and every sequence's attention output is checked against the oracle
over that sequence's whole K/V history.  Q/K/V rows stand in for the
projections: seeded per (request, position), so a position's K/V row is the
same whichever step writes it."""
import numpy as np
import pytest

import oracle as orc
import quantlib_amd as ql
from helpers import Out, dev, normal, stream, to_f16_bits
from test_gpu_attention import PagedPool, check_attn

pytestmark = pytest.mark.gpu


def rows_for(kind, rid, positions, width):
    base = {"q": 1, "k": 2, "v": 3}[kind] * 1_000_003 + rid * 10_007
    return np.stack([to_f16_bits(normal(base + int(p), (width,))) for p in positions])


@pytest.mark.parametrize("h,hkv,d,nblk,max_active", [(8, 2, 64, 64, 4), (32, 8, 128, 12, 3)])
def test_batched_serving_steps_match_oracle(h, hkv, d, nblk, max_active):
    L, layer = 2, 1
    pool = PagedPool(nblk, L, hkv, d)
    b = ql.Batcher(nblk, max_active)
    reqs = {0: (20, 6), 1: (1, 10), 2: (35, 4), 3: (16, 8), 4: (50, 5), 5: (3, 12)}
    for rid, (plen, gen) in reqs.items():
        b.add(rid, np.arange(plen, dtype=np.int32) + 10, gen)
    hist_k, hist_v = {}, {}
    steps = decode_only = 0
    while True:
        c = b.counts()
        if c["n_active"] == 0 and c["n_pending"] == 0:
            break
        p = b.plan()
        n, rows = p["n_seqs"], p["n_rows"]
        steps += 1
        if n == 0:
            b.commit(np.zeros(0, np.int32))
            continue
        decode_only += int(p["max_q_len"] == 1)
        cu = p["cu_q_lens"]
        q = np.zeros((rows, h * d), np.uint16)
        k = np.zeros((rows, hkv * d), np.uint16)
        v = np.zeros((rows, hkv * d), np.uint16)
        for i in range(n):
            rid, sl = int(p["req_ids"][i]), slice(cu[i], cu[i + 1])
            pos = p["positions"][sl]
            q[sl] = rows_for("q", rid, pos, h * d)
            k[sl] = rows_for("k", rid, pos, hkv * d)
            v[sl] = rows_for("v", rid, pos, hkv * d)
        dk, dv, dq, dsl = dev(k), dev(v), dev(q), dev(p["slot_mapping"])
        ql.call("ql_paged_kv_append_f16", pool.kptrs.ptr, pool.vptrs.ptr, nblk, dsl.ptr, dk.ptr,
                dv.ptr, rows, layer, L, hkv, d, stream())
        out = Out(rows * h * d, np.uint16)
        dcu, dctx = dev(cu), dev(p["ctx_lens"])
        dbt = dev(np.ascontiguousarray(p["block_tables"]))
        ql.call("ql_paged_attention_f16", dq.ptr, out.ptr, h * d, h * d, rows, n, dcu.ptr, dctx.ptr,
                p["max_q_len"], dbt.ptr, p["max_blocks"], pool.kptrs.ptr, pool.vptrs.ptr, nblk, layer,
                L, h, hkv, d, 1, stream())
        got = out.get((rows, h, d))
        for i in range(n):
            rid, sl = int(p["req_ids"][i]), slice(cu[i], cu[i + 1])
            hist_k.setdefault(rid, []).extend(k[sl])
            hist_v.setdefault(rid, []).extend(v[sl])
            kk = np.stack(hist_k[rid]).reshape(-1, hkv, d)
            vv = np.stack(hist_v[rid]).reshape(-1, hkv, d)
            assert kk.shape[0] == p["ctx_lens"][i]
            want = orc.attention(q[sl].reshape(-1, h, d), kk, vv, h, hkv, True, f16=True)
            check_attn(got[sl], want, vv, f"step {steps} request {rid}")
        b.commit(np.full(n, 7, np.int32))
    assert decode_only > 0 and steps > 3
    ev = []
    while (e := b.pop_finished()) is not None:
        ev.append(e)
    assert sorted(e[0] for e in ev) == sorted(reqs)
    assert b.counts()["free_blocks"] == nblk
