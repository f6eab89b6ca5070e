"""CPU checks of the continuous-batching bookkeeping (ql_batcher_*): the
reference scheduler's own scenario (tests/test_continuous_batch.cu) traced by
hand, each rule of src/continuous_batch.cu on a small case, the kernel-input
arrays of a plan against their definitions, and pool invariants over a random
workload.  No GPU is used."""
import ctypes

import numpy as np
import pytest

import quantlib_amd as ql

EOS = 2


def run_ticks(b, sampler, max_ticks=100):
    """Drive plan/commit until nothing is active or pending; returns the plans."""
    plans = []
    for _ in range(max_ticks):
        c = b.counts()
        if c["n_active"] == 0 and c["n_pending"] == 0:
            break
        p = b.plan()
        plans.append(p)
        b.commit(sampler(p))
    return plans


def drain(b):
    out = []
    while (ev := b.pop_finished()) is not None:
        out.append(ev)
    return out


def zeros(p):
    return np.zeros(p["n_seqs"], np.int32)


def test_reference_continuous_batch_scenario():
    # tests/test_continuous_batch.cu:6-28: 10 blocks of 16, max 4 active, requests
    # (id, prompt, max_gen) = (1,30,20) (2,50,15) (3,60,10) (4,20,10); the sampled
    # token is never the end token.  Trace derived by hand from the rules:
    b = ql.Batcher(10, 4)
    for rid, plen, gen in [(1, 30, 20), (2, 50, 15), (3, 60, 10), (4, 20, 10)]:
        b.add(rid, np.full(plen, rid, np.int32), gen)
    plans = run_ticks(b, zeros)
    seqs = [list(p["req_ids"]) for p in plans]
    # tick 1: 1, 2, 3 admitted (2+4+4 blocks), 4 waits at the head (0 free)
    assert seqs[0] == [1, 2, 3] and list(plans[0]["is_prefill"]) == [1, 1, 1]
    assert plans[0]["n_rows"] == 140
    assert [list(t[t >= 0]) for t in plans[0]["block_tables"]] == [[0, 1], [2, 3, 4, 5], [6, 7, 8, 9]]
    # ticks 2-3: three decodes; tick 4: request 1 needs a block for position 32, none
    # free -> evicted before running
    assert seqs[1] == seqs[2] == [1, 2, 3]
    assert seqs[3] == [2, 3]
    # tick 5: request 1's blocks (returned 0 then 1, LIFO) admit request 4 -> blocks [1, 0];
    # the active list became [3, 2] by swap-with-last, then 4 is appended
    assert seqs[4] == [3, 2, 4] and list(plans[4]["is_prefill"]) == [0, 0, 1]
    assert list(plans[4]["block_tables"][2][:2]) == [1, 0]
    # tick 6: request 3 needs a block for position 64 -> evicted; active becomes [4, 2]
    assert seqs[5] == [2, 4]
    assert all(s == [4, 2] for s in seqs[6:13])
    # tick 14: request 4 reaches 20 + 10 tokens; tick 15: request 2 reaches 50 + 15
    assert seqs[13] == [4, 2] and seqs[14] == [2] and len(plans) == 15
    ev = drain(b)
    assert [(e[0], e[1], len(e[3])) for e in ev] == [
        (1, ql.FINISH_EVICTED, 33), (3, ql.FINISH_EVICTED, 65),
        (4, ql.FINISH_LENGTH, 30), (2, ql.FINISH_LENGTH, 65)]
    assert b.counts() == {"n_active": 0, "n_pending": 0, "free_blocks": 10, "n_finished": 0}


def test_growth_at_block_boundary_and_slots():
    b = ql.Batcher(8, 2)
    b.add(7, np.arange(100, 116, dtype=np.int32), 40)   # exactly one block of prompt
    p = b.plan()
    assert p["n_rows"] == 16 and list(p["slot_mapping"]) == list(range(16))
    assert list(p["positions"]) == list(range(16)) and list(p["token_ids"]) == list(range(100, 116))
    b.commit([555])
    assert b.counts()["free_blocks"] == 7
    p = b.plan()   # decode of position 16 (token 555) needs block 1
    assert b.counts()["free_blocks"] == 6
    assert list(p["token_ids"]) == [555] and list(p["positions"]) == [16]
    assert list(p["slot_mapping"]) == [1 * 16 + 0] and list(p["ctx_lens"]) == [17]
    assert list(p["block_tables"][0]) == [0, 1]
    b.commit([556])
    p = b.plan()
    assert list(p["slot_mapping"]) == [17] and b.counts()["free_blocks"] == 6


def test_eos_finishes_and_frees():
    b = ql.Batcher(4, 2)
    b.add(1, [9, 9, 9], 50)
    b.plan()
    b.commit([11])
    b.plan()
    b.commit([EOS])
    assert b.counts()["n_active"] == 0 and b.counts()["free_blocks"] == 4
    rid, reason, plen, toks = b.pop_finished()
    assert (rid, reason, plen, list(toks)) == (1, ql.FINISH_EOS, 3, [9, 9, 9, 11, EOS])


def test_custom_eos_token():
    b = ql.Batcher(4, 2, eos_token=77)
    b.add(1, [3], 5)
    b.plan()
    b.commit([EOS])           # 2 is an ordinary token here
    b.plan()
    b.commit([77])
    assert b.pop_finished()[1] == ql.FINISH_EOS


def test_head_of_line_blocking_and_max_active():
    b = ql.Batcher(6, 2)
    b.add(1, np.zeros(40, np.int32), 3)   # 3 blocks
    b.add(2, np.zeros(60, np.int32), 3)   # 4 blocks: does not fit while 1 runs
    b.add(3, np.zeros(5, np.int32), 3)    # 1 block: fits, but waits behind 2
    p = b.plan()
    assert list(p["req_ids"]) == [1] and b.counts()["n_pending"] == 2
    b.commit([1])
    p = b.plan()
    assert list(p["req_ids"]) == [1]
    # max_active: three small requests, two admitted
    b2 = ql.Batcher(10, 2)
    for r in range(3):
        b2.add(r, [1, 2], 4)
    assert list(b2.plan()["req_ids"]) == [0, 1] and b2.counts()["n_pending"] == 1


def test_plan_arrays_match_their_definitions():
    b = ql.Batcher(64, 8)
    rng = np.random.default_rng(3)
    prompts = {r: rng.integers(3, 1000, size=int(n)).astype(np.int32)
               for r, n in zip(range(5), [17, 1, 33, 48, 5])}
    for r, pr in prompts.items():
        b.add(r, pr, 30)
    history = {r: list(pr) for r, pr in prompts.items()}
    for tick in range(6):
        p = b.plan()
        n, cu = p["n_seqs"], p["cu_q_lens"]
        assert cu[0] == 0 and cu[-1] == p["n_rows"] and np.all(np.diff(cu) > 0)
        assert p["max_q_len"] == np.diff(cu).max() and p["max_ctx_len"] == p["ctx_lens"].max()
        for i in range(n):
            r, rows = p["req_ids"][i], slice(cu[i], cu[i + 1])
            pos, toks, slots = p["positions"][rows], p["token_ids"][rows], p["slot_mapping"][rows]
            table = p["block_tables"][i]
            nb = int((table >= 0).sum())
            assert np.all(table[nb:] == -1)
            assert nb == -(-p["ctx_lens"][i] // 16)                 # ceil(ctx / 16) blocks
            assert pos[-1] + 1 == p["ctx_lens"][i] and p["sample_rows"][i] == cu[i + 1] - 1
            if p["is_prefill"][i]:
                assert list(pos) == list(range(len(prompts[r])))
            else:
                assert len(pos) == 1 and pos[0] == len(history[r]) - 1
            assert list(toks) == [history[r][q] for q in pos]
            assert list(slots) == [table[q // 16] * 16 + q % 16 for q in pos]
        live = p["block_tables"][p["block_tables"] >= 0]
        assert len(set(live.tolist())) == live.size                 # no block shared
        samp = rng.integers(3, 1000, size=n).astype(np.int32)
        for i in range(n):
            history[p["req_ids"][i]].append(int(samp[i]))
        b.commit(samp)


def test_random_workload_pool_invariants():
    rng = np.random.default_rng(11)
    nblk = 40
    b = ql.Batcher(nblk, 6)
    gen_budget = {}
    for r in range(60):
        n = int(rng.integers(1, 90))
        gen_budget[r] = int(rng.integers(1, 40))
        b.add(r, rng.integers(3, 100, size=n).astype(np.int32), gen_budget[r])

    def sampler(p):
        return np.where(rng.random(p["n_seqs"]) < 0.05, EOS, 7).astype(np.int32)

    for p in run_ticks(b, sampler, max_ticks=2000):
        held = p["block_tables"][p["block_tables"] >= 0]
        assert len(set(held.tolist())) == held.size and held.size <= nblk
    assert b.counts() == {"n_active": 0, "n_pending": 0, "free_blocks": nblk, "n_finished": 60}
    ev = drain(b)
    assert sorted(e[0] for e in ev) == list(range(60))
    for rid, reason, plen, toks in ev:
        gen = len(toks) - plen
        if reason == ql.FINISH_LENGTH:
            assert gen == gen_budget[rid]
        elif reason == ql.FINISH_EOS:
            assert toks[-1] == EOS and gen <= gen_budget[rid]
        else:
            assert reason == ql.FINISH_EVICTED and gen < gen_budget[rid]


def test_borrowed_stack_is_the_paged_kv_free_list():
    # the free_blocks / free_count pair of a PagedKVCache (fresh pool: n-1 .. 0, count n)
    n = 6
    stack = np.arange(n - 1, -1, -1, dtype=np.int32)
    count = np.array([n], np.int32)
    b = ql.Batcher(n, 2, stack=stack, free_count=count)
    b.add(1, np.zeros(20, np.int32), 2)   # 2 blocks: pops 0 then 1
    p = b.plan()
    assert list(p["block_tables"][0]) == [0, 1] and count[0] == 4
    b.commit([5])
    b.plan()
    b.commit([5])                       # length reached: blocks pushed back 0, 1
    assert count[0] == 6 and list(stack[4:6]) == [0, 1]
    b.close()


def test_argument_validation():
    h = ctypes.c_void_p()
    assert ql.raw("ql_batcher_create", 4, 0, 2, ctypes.byref(h)) == ql.HIP_ERROR_INVALID_VALUE
    assert ql.raw("ql_batcher_create", -1, 2, 2, ctypes.byref(h)) == ql.HIP_ERROR_INVALID_VALUE
    b = ql.Batcher(4, 2)
    p = np.zeros(4, np.int32)
    assert ql.raw("ql_batcher_add_request", b.h, 1, p.ctypes.data, 0, 5) == ql.HIP_ERROR_INVALID_VALUE
    assert ql.raw("ql_batcher_add_request", b.h, 1, p.ctypes.data, 4, 0) == ql.HIP_ERROR_INVALID_VALUE
    # commit before plan, plan twice, commit with the wrong count
    assert ql.raw("ql_batcher_commit", b.h, None, 0) == ql.HIP_ERROR_INVALID_VALUE
    b.add(1, p, 3)
    plan = ql.StepPlan()
    assert ql.raw("ql_batcher_plan", b.h, ctypes.byref(plan)) == 0
    assert ql.raw("ql_batcher_plan", b.h, ctypes.byref(plan)) == ql.HIP_ERROR_INVALID_VALUE
    assert ql.raw("ql_batcher_commit", b.h, p.ctypes.data, 2) == ql.HIP_ERROR_INVALID_VALUE
    assert ql.raw("ql_batcher_commit", b.h, p.ctypes.data, 1) == 0
    assert ql.raw("ql_batcher_destroy", None) == 0
