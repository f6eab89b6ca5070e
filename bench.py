#!/usr/bin/env python3
"""Throughput of the fused per-layer kernels on one MI355X.

Workload ("C5"): the memory-bound chain of one
Llama-3-8B-shaped decoder layer in fp16 over a T=8192-token batch, in the order
of the reference's fp16_layer_forward (src/fp16_forward.cu:167-223), GEMMs
and attention excluded:

  1. residual add + attention RMSNorm   x[8192,4096] += d; y = rmsnorm(x)
  2. RoPE on Q and K + paged KV append  Q[8192,32,128], K,V[8192,8,128], theta 5e5, rotate-half;
     (one fused launch)                 rotated K and V -> 512 blocks of 16 (pool of 32 layers)
  3. residual add + FFN RMSNorm         as 1
  4. SwiGLU                             gate, up [8192,14336] -> out

One step = one pass of that chain.  The unfused RoPE and paged-append kernels
are timed separately under "kernels" for comparison, each kernel beside a plain
copy of its byte count (copy_same_bytes, vs_copy).  Inputs are synthetic (seeded normal values
made on the host and uploaded once) and resident in HBM before timing.  Three
device buffer sets (~1 GB each) are rotated step to step so no input is still
in the 256 MB MALL; the KV append rotates over the 32 pool layers.  The
single-kernel passes of the smaller kernels rotate more: the RoPE and KV-append
kernels over 12 sets of Q, K, V (96 MiB each), the embedding gather over 4
tables (250 MB each) with their own ids.
value = algorithmic bytes of the chain (each input read once, each output
written once) / wall time per step.  Before the timed steps, whatever --warmup
asks, ~30 ms of copies and then >= 30 ms of chain steps run untimed (the
clocks take ~20 ms of sustained load to ramp up), then the --warmup steps, then
the timed region once with one step (the first timed region of a process pays
~45 us of one-time host cost); every single-kernel pass starts after ~30 ms of
untimed device work as well.

The embedding gather and the final RMSNorm (once per forward, not per layer)
are timed separately and reported under "kernels".  The roofline entry is for the dominant kernel,
SwiGLU fp16 [8192 x 14336]: 3 x 8192 x 14336 x 2 B = 704,643,072 B per launch,
timed after the timed steps in a pass of its own: back-to-back launches on the
work stream between one pair of HIP events.  The timed steps themselves carry
no instrumentation: one event pair and a host clock at their edges only.

`--all-configs` times every BASELINE config (C1-C5) one kernel at a time, each
beside a plain copy of its byte count, and
adds the attention that consumes the path's output: causal prefill over the
8192 tokens (contiguous, and over the paged pool the chain writes), reported in
TFLOP/s against the dense fp16 matrix peak, and paged decode (64 sequences x
4096 tokens; 1 sequence x 8192 tokens with the key-split workspace), HBM-bound
on the K/V rows, and one whole decoder layer through the engine (hipBLASLt
GEMMs + the fused kernels + attention) for that prefill and those decode steps,
on fp16 weights and on FP8 weights (the reference's quantized forward; the
decode steps also as a 32-layer step captured in one HIP graph), plus the
FP8-weight GEMM at decode row counts against the fp16 GEMM and the FP8 codec,
the decode of one sequence over the contiguous cache (one pass and key split),
and the reference's own kernel benchmark (tests/benchmark_all.cu: its shapes,
its timing method, through the drop-in shims) beside its published times.
Matrix-core-bound passes warm up for ~60 ms on their own kernel rather than on
copies (the clocks need it after a memory-bound pass).

Device memory, the stream and events come from libamdhip64 through the
library's own binding (quant-lib_amd/quantlib_amd.py); no framework runtime is
loaded.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "quant-lib_amd"))

PEAK_HBM_GBS = 8000.0          # MI355X HBM3E peak, GB/s
PEAK_MFMA_F16_TFLOPS = 2500.0  # MI355X dense fp16 matrix peak, TFLOP/s
T, D, HQ, HKV, HD, F = 8192, 4096, 32, 8, 128, 14336
VOCAB, THETA, EPS, L_POOL, PAGE = 32000, 5e5, 1e-5, 32, 16
NSETS = 3
# single-kernel passes of the RoPE / KV-append kernels rotate over more sets:
# one set of Q, K, V is 96 MiB, and three would partly stay in the 256 MB MALL
NROPE = 12
NTABLES = 4   # embedding tables (250 MB each) rotated by the gather pass
# warm-up launches of a single-kernel pass: one full rotation of every set it
# cycles through (buffer sets, tables, the 32 pool layers), so no timed launch
# is the first to touch a buffer (first touches also pay address translation)
WARM = 32
# untimed device work before the timed steps, whatever --warmup says: half
# copies, half chain steps (the clocks ramp over ~20 ms of sustained load)
CLOCK_WARMUP_MS = 60.0

BYTES = {
    "add_rmsnorm_f16": 4 * T * D * 2 + 2 * D,                     # read x,d; write x',y; w
    "rmsnorm_f16": 2 * T * D * 2 + 2 * D,                         # final norm: read x; write y; w
    "rope_f16": 2 * T * (HQ + HKV) * HD * 2,                      # in-place read+write Q,K
    "paged_kv_append_f16": 4 * T * HKV * HD * 2 + 4 * T,          # read K,V; write K,V; slots
    "swiglu_f16": 3 * T * F * 2,                                  # read gate,up; write out
    "embed_f16": 2 * T * D * 2 + 4 * T,                           # read rows; write out; ids
    # Q read+write; K read, write in place, write to cache; V read, write to cache; slots
    "rope_paged_kv_append_f16": 2 * T * HQ * HD * 2 + 5 * T * HKV * HD * 2 + 4 * T,
    # opt-in variant: rotated K to the cache only (no in-place K write), not in the chain
    "rope_q_paged_kv_append_f16": 2 * T * HQ * HD * 2 + 4 * T * HKV * HD * 2 + 4 * T,
}
COPY_TOKENS = 131072                                              # 256 MiB per K and V
COPY_ELEMS = COPY_TOKENS * HKV * HD
BYTES["copy_calibration"] = 2 * 2 * COPY_ELEMS * 2                # read + write, K and V
CHAIN = ["add_rmsnorm_f16", "rope_paged_kv_append_f16", "add_rmsnorm_f16", "swiglu_f16"]
# the same layer with RoPE and the paged append as two launches (reference order)
CHAIN_UNFUSED = ["add_rmsnorm_f16", "rope_f16", "paged_kv_append_f16", "add_rmsnorm_f16",
                 "swiglu_f16"]
CHAIN_BYTES = sum(BYTES[k] for k in CHAIN)


def parse():
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # untimed steps after the time-based clock warm-up (CLOCK_WARMUP_MS)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--breakdown-reps", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="target CPU time of the oracle baseline sample (0 = skip)")
    ap.add_argument("--traffic-file", default=str(ROOT / "profiles" / "pmc_traffic.json"))
    ap.add_argument("--all-configs", action="store_true",
                    help="time every BASELINE config (C1..C5) and print a table instead of the JSON line")
    ap.add_argument("--reps", type=int, default=50, help="launches per config in --all-configs")
    ap.add_argument("--only", default="",
                    help="--all-configs row groups to time, comma-separated: "
                         "configs, refbench, kv, attention, layer, fp8 (default: all)")
    return ap.parse_args()


class Chain:
    """Device buffers of the C5 layer chain and the launches of one step."""

    def __init__(self, ql, np):
        self.ql = ql
        r = np.random.default_rng(0x51A10005)

        def randn(*shape, clip=None):
            a = r.standard_normal(size=shape, dtype=np.float32)
            if clip is not None:
                np.clip(a, -clip, clip, out=a)
            return a.astype(np.float16).view(np.uint16)

        up = ql.DeviceArray.from_numpy
        # one host copy of every input, uploaded into NSETS distinct device sets
        host = {"x": randn(T, D), "d1": randn(T, D), "d2": randn(T, D),
                "q": randn(T, HQ * HD), "k": randn(T, HKV * HD), "v": randn(T, HKV * HD),
                "gate": randn(T, F, clip=8.0), "up": randn(T, F, clip=8.0)}
        self.sets = []
        for _ in range(NSETS):
            s = {k: up(v) for k, v in host.items()}
            s["y"] = ql.DeviceArray((T, D), np.uint16)
            s["out"] = ql.DeviceArray((T, F), np.uint16)
            self.sets.append(s)
        del host
        self.w_attn = up(r.uniform(0.5, 1.5, D).astype(np.float16).view(np.uint16))
        self.w_ffn = up(r.uniform(0.5, 1.5, D).astype(np.float16).view(np.uint16))
        # paged pool: 512 blocks of [32 layers, 16, 8, 128] fp16 (1 MiB each) per K and V
        self.nb = T // PAGE
        blk = L_POOL * PAGE * HKV * HD
        self.kpool = ql.DeviceArray((self.nb * blk,), np.uint16).fill_bytes(0)
        self.vpool = ql.DeviceArray((self.nb * blk,), np.uint16).fill_bytes(0)
        self.kptrs = up(np.array([self.kpool.ptr + 2 * blk * b for b in range(self.nb)], np.int64))
        self.vptrs = up(np.array([self.vpool.ptr + 2 * blk * b for b in range(self.nb)], np.int64))
        # fresh-pool block order 0,1,2,... (LIFO allocator of src/paged_kvcache.cu:49-53)
        self.slots = up(np.arange(T, dtype=np.int32))
        # Q, K, V sets for the single-kernel RoPE / append passes (12 x 96 MiB)
        qh, kh, vh = randn(T, HQ * HD), randn(T, HKV * HD), randn(T, HKV * HD)
        self.rope_sets = [{"q": up(qh), "k": up(kh), "v": up(vh)} for _ in range(NROPE)]
        del qh, kh, vh
        # embedding tables and ids (gather timed separately): each launch gathers
        # from another table with other ids, so no row is still in the MALL
        tab = randn(VOCAB, D)
        self.tables = [up(tab) for _ in range(NTABLES)]
        del tab
        self.ids = [up(r.integers(0, VOCAB, size=T).astype(np.int32)) for _ in range(NTABLES)]
        self.emb_out = [ql.DeviceArray((T, D), np.uint16) for _ in range(NSETS)]
        # plain-copy reference: 2 x 256 MiB copied by the contiguous KV-append kernel
        self.cp_src = [ql.DeviceArray((COPY_ELEMS,), np.uint16) for _ in range(2)]
        self.cp_dst = [ql.DeviceArray((COPY_ELEMS,), np.uint16) for _ in range(2)]
        self.stream = ql.stream()
        self.step_no = 0
        ql.synchronize()

    # one launch per kernel of the chain --------------------------------------------------
    def k_add_rmsnorm(self, s, which):
        w = self.w_attn if which == "d1" else self.w_ffn
        self.ql.call("ql_add_rmsnorm_f16", s["x"].ptr, s[which].ptr, w.ptr, s["y"].ptr, T, D, EPS,
                     self.stream)

    def k_rmsnorm(self, s):
        self.ql.call("ql_rmsnorm_f16", s["x"].ptr, self.w_ffn.ptr, s["y"].ptr, T, D, EPS, self.stream)

    def k_rope(self, s):
        self.ql.call("ql_rope_f16", s["q"].ptr, s["k"].ptr, T, HQ, HKV, HD, HQ * HD, HKV * HD, None,
                     0, THETA, self.ql.ROPE_HALF, self.stream)

    def k_paged(self, s, layer):
        self.ql.call("ql_paged_kv_append_f16", self.kptrs.ptr, self.vptrs.ptr, self.nb,
                     self.slots.ptr, s["k"].ptr, s["v"].ptr, T, layer, L_POOL, HKV, HD, self.stream)

    def k_rope_paged(self, s, layer):
        self.ql.call("ql_rope_paged_kv_append_f16", s["q"].ptr, s["k"].ptr, s["v"].ptr, T, HQ, HKV, HD,
                     HQ * HD, HKV * HD, HKV * HD, None, 0, THETA, self.ql.ROPE_HALF, self.kptrs.ptr,
                     self.vptrs.ptr, self.nb, self.slots.ptr, layer, L_POOL, self.stream)

    def k_rope_q_paged(self, s, layer):
        self.ql.call("ql_rope_q_paged_kv_append_f16", s["q"].ptr, s["k"].ptr, s["v"].ptr, T, HQ, HKV,
                     HD, HQ * HD, HKV * HD, HKV * HD, None, 0, THETA, self.ql.ROPE_HALF, self.kptrs.ptr,
                     self.vptrs.ptr, self.nb, self.slots.ptr, layer, L_POOL, self.stream)

    def k_swiglu(self, s):
        self.ql.call("ql_swiglu_f16", s["gate"].ptr, s["up"].ptr, s["out"].ptr, T, F, self.stream)

    def k_embed(self, i):
        self.ql.call("ql_embed_f16", self.tables[i % NTABLES].ptr, self.ids[i % NTABLES].ptr, T, VOCAB, D,
                     self.emb_out[i % NSETS].ptr, self.stream)

    def k_copy(self):
        # [COPY_TOKENS, 8, 128] fp16 per K and V: a pure 16-byte copy of known size
        self.ql.call("ql_kv_append_f16", self.cp_dst[0].ptr, self.cp_dst[1].ptr, self.cp_src[0].ptr,
                     self.cp_src[1].ptr, 0, 0, COPY_TOKENS, HKV, HD, COPY_TOKENS, 1, self.stream)

    def k_copy_bytes(self, nbytes, i):
        """A plain copy moving `nbytes` in all (half read, half written) with the
        same kernel as k_copy, at offsets that rotate through the 2 x 256 MiB
        source and destination pool so a small copy is not served from the MALL."""
        tokens = max(1, nbytes // (8 * HKV * HD))      # 2 KiB read + 2 KiB written per token, K and V
        elems = tokens * HKV * HD
        nrot = max(1, COPY_ELEMS // elems)
        off = 2 * (i % nrot) * elems                   # bytes
        self.ql.call("ql_kv_append_f16", self.cp_dst[0].ptr + off, self.cp_dst[1].ptr + off,
                     self.cp_src[0].ptr + off, self.cp_src[1].ptr + off, 0, 0, tokens, HKV, HD, tokens, 1,
                     self.stream)
        return 8 * elems                               # bytes moved: K and V, 2 B each, read and written

    def step(self):
        i = self.step_no
        self.step_no += 1
        s = self.sets[i % NSETS]
        self.k_add_rmsnorm(s, "d1")
        self.k_rope_paged(s, i % L_POOL)
        self.k_add_rmsnorm(s, "d2")
        self.k_swiglu(s)

    def kernel_launcher(self, name):
        return {
            "add_rmsnorm_f16": lambda i: self.k_add_rmsnorm(self.sets[i % NSETS], "d1"),
            "rmsnorm_f16": lambda i: self.k_rmsnorm(self.sets[i % NSETS]),
            "rope_f16": lambda i: self.k_rope(self.rope_sets[i % NROPE]),
            "paged_kv_append_f16": lambda i: self.k_paged(self.rope_sets[i % NROPE], i % L_POOL),
            "rope_paged_kv_append_f16": lambda i: self.k_rope_paged(self.rope_sets[i % NROPE], i % L_POOL),
            "rope_q_paged_kv_append_f16": lambda i: self.k_rope_q_paged(self.rope_sets[i % NROPE],
                                                                        i % L_POOL),
            "swiglu_f16": lambda i: self.k_swiglu(self.sets[i % NSETS]),
            "embed_f16": lambda i: self.k_embed(i),
            "copy_calibration": lambda i: self.k_copy(),
        }[name]


_HEAT = []


def timed_region(ql, chain, steps):
    """`steps` chain steps between a synchronisation on each side: (host seconds,
    event milliseconds) from the first launch to the end of the last."""
    t_all0, t_all1 = ql.Event(), ql.Event()
    ql.synchronize()
    t0 = time.perf_counter()
    t_all0.record(chain.stream)
    for _ in range(steps):
        chain.step()
    t_all1.record(chain.stream)
    ql.synchronize()
    wall = time.perf_counter() - t0
    return wall, t_all0.elapsed_ms(t_all1)


def heat(ql, stream, ms=30.0):
    """About `ms` of untimed device work (a 2 x 64 MiB copy, ~40 us a launch)
    before a timed pass.  The clocks ramp up over the first ~20 ms of sustained
    load (a kernel trace of this bench shows the chain step settle from 236 to
    229 us), so a pass that follows host work (data generation, the CPU
    baseline) or a pass of short launches would otherwise run partly cold."""
    import numpy as np
    if not _HEAT:
        n = 32 << 20   # fp16 elements: 64 MiB per buffer
        _HEAT.extend(ql.DeviceArray((n,), np.uint16).fill_bytes(0) for _ in range(4))
    tokens = _HEAT[0].size // (HKV * HD)
    for _ in range(int(ms * 1e3 / 40.0) + 1):
        ql.call("ql_kv_append_f16", _HEAT[2].ptr, _HEAT[3].ptr, _HEAT[0].ptr, _HEAT[1].ptr, 0, 0, tokens,
                HKV, HD, tokens, 1, stream)
    ql.synchronize()


def warm_on(ql, stream, launch, ms=60.0):
    """About `ms` of untimed launches of the workload itself before a timed pass
    of a matrix-core-bound kernel.  Under sustained matrix-core load the clocks
    go through a transient: a kernel trace of the C5 prefill attention shows
    ~630 us for the first launches, ~800 us around the fifth (after 30 ms of
    copies), then a slow settle to a steady 605-660 us (box to box) after
    ~40 ms; timed inside that window it read 700 us.  The launch count is
    sized from the second launch (the first one also loads the code object)."""
    launch(0)
    ql.synchronize()
    a, b = ql.Event(), ql.Event()
    a.record(stream)
    launch(1)
    b.record(stream)
    ql.synchronize()
    per_ms = max(a.elapsed_ms(b), 1e-3)
    n = int(ms / per_ms) + 2
    for i in range(2, n):
        launch(i)
    ql.synchronize()
    return n


def percentiles(us):
    """Median, p10 and p90 of a list of durations (us)."""
    v = sorted(us)
    at = lambda f: v[min(len(v) - 1, int(f * len(v)))]
    return {"us_median": round(at(0.5), 2), "us_p10": round(at(0.1), 2), "us_p90": round(at(0.9), 2)}


def breakdown(chain, ql, reps):
    """Duration of each kernel on the work stream, two ways.

    us_mean: `reps` launches back to back (rotating buffer sets) between one
    pair of HIP events, divided by reps -- the kernel's duration plus the
    dispatch gap, which is what a rocprofv3 kernel trace averages to within
    about 1%.  events_per_launch: a second pass with an event pair around
    every launch (each pair adds the events' own cost, a few us), kept for
    its spread.

    copy_same_bytes: the plain copy of copy_calibration, resized to move the
    kernel's algorithmic bytes (half read, half written) and timed the same way.
    A launch carries a fixed cost (ramp-up and drain, ~2 us) besides its
    bytes, so a 67 MB copy runs at ~5.3 TB/s and a 1 GB one at ~6.5-6.7: the
    copy of the same size is the kernel's practical ceiling, and vs_copy =
    copy us / kernel us (1.0 = as fast as a copy of its bytes)."""
    def back_to_back(launch):
        heat(ql, chain.stream)   # every pass starts on ramped clocks
        for i in range(WARM):
            launch(i)
        ql.synchronize()
        a0, a1 = ql.Event(), ql.Event()
        a0.record(chain.stream)
        for i in range(reps):
            launch(i)
        a1.record(chain.stream)
        ql.synchronize()
        return a0.elapsed_ms(a1) * 1e3 / reps

    out = {}
    for name in ["add_rmsnorm_f16", "rope_paged_kv_append_f16", "rope_q_paged_kv_append_f16",
                 "rope_f16", "paged_kv_append_f16", "swiglu_f16", "embed_f16", "rmsnorm_f16",
                 "copy_calibration"]:
        launch = chain.kernel_launcher(name)
        mean = back_to_back(launch)
        evs = [(ql.Event(), ql.Event()) for _ in range(reps)]
        for i, (a, b) in enumerate(evs):
            a.record(chain.stream)
            launch(i)
            b.record(chain.stream)
        ql.synchronize()
        us = sorted(a.elapsed_ms(b) * 1e3 for a, b in evs)
        gbs = BYTES[name] / (mean * 1e-6) / 1e9
        out[name] = {"us_mean": round(mean, 2), "bytes": BYTES[name], "GBps": round(gbs, 1),
                     "frac_peak": round(gbs / PEAK_HBM_GBS, 4),
                     "events_per_launch": percentiles(us)}
        if name != "copy_calibration":
            moved = chain.k_copy_bytes(BYTES[name], 0)
            cp = back_to_back(lambda i: chain.k_copy_bytes(BYTES[name], i))
            out[name]["copy_same_bytes"] = {"bytes": moved, "us_mean": round(cp, 2),
                                            "GBps": round(moved / (cp * 1e-6) / 1e9, 1)}
            out[name]["vs_copy"] = round(cp * BYTES[name] / moved / mean, 3)
    return out


def host_cpu():
    """CPU model and the cores this process may run on (the box's share)."""
    model = "unknown"
    try:
        for ln in pathlib.Path("/proc/cpuinfo").read_text().splitlines():
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return {"cpu_model": model, "nproc": usable, "os_cpu_count": os.cpu_count()}


def cpu_baseline(seconds, threads=1):
    """The oracle (scalar C) on a bounded sample of the same chain: the C5 shapes
    restricted to 512 tokens per thread, repeated until `seconds` elapse.  With
    threads > 1 every thread runs its own 512-token slice (own buffers) at the
    same time; ctypes releases the interpreter lock during each C call, so the
    slices run on separate host cores."""
    import threading
    import numpy as np
    sys.path.insert(0, str(ROOT))
    import oracle as orc

    lib = orc.lib()
    n = 512
    sample_bytes = CHAIN_BYTES * n // T  # the fused chain's bytes; the oracle runs rope then append

    def P(a):
        return a.ctypes.data

    def make(seed):
        r = np.random.default_rng(seed)

        def h(*shape, clip=None):
            a = r.standard_normal(size=shape, dtype=np.float32)
            if clip:
                np.clip(a, -clip, clip, out=a)
            return a.astype(np.float16).view(np.uint16)

        nb = n // PAGE
        blk = L_POOL * PAGE * HKV * HD
        b = {"x": h(n, D), "d1": h(n, D), "d2": h(n, D), "y": np.empty((n, D), np.uint16),
             "w": r.uniform(0.5, 1.5, D).astype(np.float16).view(np.uint16),
             "q": h(n, HQ * HD), "k": h(n, HKV * HD), "v": h(n, HKV * HD),
             "gate": h(n, F, clip=8), "up": h(n, F, clip=8), "out": np.empty((n, F), np.uint16),
             "kpool": np.empty(nb * blk, np.uint16), "vpool": np.empty(nb * blk, np.uint16),
             "offs": (np.arange(nb) * blk).astype(np.int64), "slots": np.arange(n, dtype=np.int32)}
        b["nb"] = nb
        return b

    def one(b, layer):
        lib.or_add_rmsnorm_f16(P(b["x"]), P(b["d1"]), P(b["w"]), P(b["y"]), n, D, EPS)
        lib.or_rope_f16(P(b["q"]), n, HQ, HD, HQ * HD, None, 0, THETA, 1)
        lib.or_rope_f16(P(b["k"]), n, HKV, HD, HKV * HD, None, 0, THETA, 1)
        lib.or_paged_kv_append_f16(P(b["kpool"]), P(b["vpool"]), P(b["offs"]), b["nb"], P(b["slots"]),
                                   P(b["k"]), P(b["v"]), n, layer, L_POOL, HKV, HD)
        lib.or_add_rmsnorm_f16(P(b["x"]), P(b["d2"]), P(b["w"]), P(b["y"]), n, D, EPS)
        lib.or_swiglu_f16(P(b["gate"]), P(b["up"]), P(b["out"]), n * F)

    bufs = [make(1 + i) for i in range(threads)]
    for b in bufs:
        one(b, 0)
    passes = [0] * threads
    start = threading.Barrier(threads + 1)
    stop = [0.0]

    def worker(i):
        start.wait()
        while time.perf_counter() < stop[0]:
            one(bufs[i], passes[i] % L_POOL)
            passes[i] += 1

    ts = [threading.Thread(target=worker, args=(i,)) for i in range(threads)]
    for t in ts:
        t.start()
    t0 = time.perf_counter()
    stop[0] = t0 + seconds
    start.wait()
    for t in ts:
        t.join()
    el = time.perf_counter() - t0
    reps = sum(passes)
    gbs = sample_bytes * reps / el / 1e9
    how = "1 thread" if threads == 1 else f"{threads} threads, one 512-token slice each"
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"oracle/oracle.c scalar C (gcc -O2, {how}) running the same layer chain on "
                      f"{n}-token slices of the {T} tokens (C5 shapes), {reps} passes in {el:.1f} s; "
                      f"{sample_bytes / 1e6:.1f} MB of algorithmic traffic per pass; "
                      f"= {el / reps * T / n * 1e6:.0f} us per decoder layer at T=8192"}


def all_configs(ql, np, reps, only=()):
    """Every BASELINE config: device time per launch, back to back on one stream
    with enough rotating buffer sets that each launch reads data last touched
    >= 1 GiB earlier (defeats the 256 MB MALL).  Returns a list of rows."""
    r = np.random.default_rng(7)
    st = ql.stream()
    rows = []
    want = lambda group: not only or group in only
    if want("refbench"):
        rows += refbench_rows(ql, np, st)
    if want("kv"):
        rows += kvcache_append_rows(ql, np, st)
    if not want("configs") and not want("attention") and not want("layer"):
        return rows + (fp8_rows(ql, np, reps) if want("fp8") else [])

    def sets_for(nbytes):
        return max(2, min(64, -(-(1 << 30) // max(nbytes, 1))))

    def upload(a):
        return ql.DeviceArray.from_numpy(a)

    def f16(a):
        return a.astype(np.float16).view(np.uint16)

    def time_it(name, cfg, nbytes, nsets, make, launch):
        bufs = [make() for _ in range(nsets)]
        heat(ql, st)
        for i in range(max(3, nsets)):   # every set once before timing
            launch(bufs[i % nsets])
        ql.synchronize()
        a, b = ql.Event(), ql.Event()
        a.record(st)
        for i in range(reps):
            launch(bufs[i % nsets])
        b.record(st)
        us = a.elapsed_ms(b) * 1e3 / reps
        gbs = nbytes / (us * 1e-6) / 1e9
        rows.append({"config": cfg, "kernel": name, "bytes": nbytes, "us": round(us, 2),
                     "GBps": round(gbs, 1), "frac_peak": round(gbs / PEAK_HBM_GBS, 4),
                     **copy_same(nbytes, us)})
        del bufs

    def copy_same(nbytes, us):
        """A plain copy of the row's byte count, timed the same way (see breakdown)."""
        moved = chain.k_copy_bytes(nbytes, 0)
        for i in range(WARM):
            chain.k_copy_bytes(nbytes, i)
        ql.synchronize()
        a, b = ql.Event(), ql.Event()
        a.record(st)
        for i in range(reps):
            chain.k_copy_bytes(nbytes, i)
        b.record(st)
        cp = a.elapsed_ms(b) * 1e3 / reps
        return {"copy_same_bytes_us": round(cp, 2), "vs_copy": round(cp * nbytes / moved / us, 3)}

    def randn(*shape, clip=None, sigma=1.0):
        x = r.standard_normal(size=shape, dtype=np.float32) * np.float32(sigma)
        if clip:
            np.clip(x, -clip, clip, out=x)
        return x

    chain = Chain(ql, np)
    if not want("configs"):
        rows += attention_rows(ql, np, chain, reps) if want("attention") else []
        rows += layer_rows(ql, np, chain, reps) if want("layer") else []
        del chain
        return rows + (fp8_rows(ql, np, reps) if want("fp8") else [])
    # C1: RMSNorm fp32 2048x2048
    R_, C_ = 2048, 2048
    x1, w1 = randn(R_, C_), r.uniform(0.5, 1.5, C_).astype(np.float32)
    nb = 2 * R_ * C_ * 4 + C_ * 4
    dw1 = upload(w1)
    time_it("rmsnorm_f32", "C1 2048x2048", nb, sets_for(nb),
            lambda: (upload(x1), ql.DeviceArray((R_, C_), np.float32)),
            lambda b: ql.call("ql_rmsnorm_f32", b[0].ptr, dw1.ptr, b[1].ptr, R_, C_, 1e-5, st))
    # C2: RoPE fp32 Q[2048,32,64] + K[2048,4,64], both pairings
    q2, k2 = randn(2048, 32 * 64), randn(2048, 4 * 64)
    nb = 2 * (q2.nbytes + k2.nbytes)
    for pairing, pname in ((ql.ROPE_HALF, "rotate-half"), (ql.ROPE_INTERLEAVED, "interleaved")):
        time_it(f"rope_f32 {pname}", "C2 Q[2048,32,64]+K[2048,4,64]", nb, sets_for(nb),
                lambda: (upload(q2), upload(k2)),
                lambda b, p=pairing: ql.call("ql_rope_f32", b[0].ptr, b[1].ptr, 2048, 32, 4, 64,
                                             32 * 64, 4 * 64, None, 0, 1e4, p, st))
    # C3: SwiGLU fp32 and fp16, rows x 5632
    for rows_ in (1, 32, 128, 512):
        g3, u3 = randn(rows_, 5632, clip=8.0), randn(rows_, 5632, clip=8.0)
        for prec in ("f32", "f16"):
            gg, uu = (g3, u3) if prec == "f32" else (f16(g3), f16(u3))
            nb = 3 * gg.nbytes
            time_it(f"swiglu_{prec}", f"C3 {rows_}x5632", nb, sets_for(nb),
                    lambda gg=gg, uu=uu: (upload(gg), upload(uu), ql.DeviceArray(gg.shape, gg.dtype)),
                    lambda b, prec=prec, rows_=rows_: ql.call(f"ql_swiglu_{prec}", b[0].ptr, b[1].ptr,
                                                             b[2].ptr, rows_, 5632, st))
    # C4: softmax fp32 and fp16, 4096x4096 causal, N(0, sigma=2)
    x4 = randn(4096, 4096, sigma=2.0)
    x4[np.triu_indices(4096, k=1)] = -np.inf
    for prec in ("f32", "f16"):
        xx = x4 if prec == "f32" else f16(x4)
        nb = 2 * xx.nbytes
        time_it(f"softmax_{prec}", "C4 4096x4096 causal", nb, sets_for(nb),
                lambda xx=xx: (upload(xx), ql.DeviceArray(xx.shape, xx.dtype)),
                lambda b, prec=prec: ql.call(f"ql_softmax_{prec}", b[0].ptr, b[1].ptr, 4096, 4096, st))
    rows.append(cpu_softmax_row(np, x4))
    del x4
    # C5: the layer-chain kernels (one launch each, as in the default mode)
    for name in ["embed_f16", "add_rmsnorm_f16", "rmsnorm_f16", "rope_f16", "paged_kv_append_f16",
                 "rope_paged_kv_append_f16", "rope_q_paged_kv_append_f16", "swiglu_f16",
                 "copy_calibration"]:
        launch = chain.kernel_launcher(name)
        heat(ql, st)
        for i in range(WARM):
            launch(i)
        ql.synchronize()
        a, b = ql.Event(), ql.Event()
        a.record(st)
        for i in range(reps):
            launch(i)
        b.record(st)
        us = a.elapsed_ms(b) * 1e3 / reps
        gbs = BYTES[name] / (us * 1e-6) / 1e9
        rows.append({"config": "C5 T=8192 llama3-8b", "kernel": name, "bytes": BYTES[name],
                     "us": round(us, 2), "GBps": round(gbs, 1), "frac_peak": round(gbs / PEAK_HBM_GBS, 4),
                     **(copy_same(BYTES[name], us) if name != "copy_calibration" else {})})
    rows += attention_rows(ql, np, chain, reps) if want("attention") else []
    rows += layer_rows(ql, np, chain, reps) if want("layer") else []
    del chain
    rows += fp8_rows(ql, np, reps) if want("fp8") else []
    return rows


def cpu_softmax_row(np, x):
    """The reference's only CPU loop on the path, cpu_softmax of
    tests/test_softmax.cu:19-30 (3 passes, expf, one thread), restated in the
    oracle as or_softmax_reftest_cpu, on the C4 input; median of 3 runs."""
    sys.path.insert(0, str(ROOT))
    import oracle as orc
    lib = orc.lib()
    rows_, cols = x.shape
    xin = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(xin)
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        lib.or_softmax_reftest_cpu(xin.ctypes.data, out.ctypes.data, rows_, cols)
        ts.append(time.perf_counter() - t0)
    us = sorted(ts)[1] * 1e6
    nb = 2 * xin.nbytes
    info = host_cpu()
    return {"config": "C4 4096x4096 causal", "bytes": nb, "us": round(us, 1),
            "GBps": round(nb / (us * 1e-6) / 1e9, 2), "frac_peak": None,
            "kernel": f"CPU baseline: cpu_softmax (tests/test_softmax.cu:19-30) restated in "
                      f"oracle/oracle.c, gcc -O2, 1 thread of {info['nproc']} ({info['cpu_model']})"}


def refbench_rows(ql, np, st):
    """The reference's own kernel benchmark (tests/benchmark_all.cu:89-262) on
    this build, the reference's way: the drop-in shims of include/quantlib_compat.h
    (launch_softmax, launch_rmsnorm, launch_rope, launch_swiglu), one untimed
    launch, then `reps` back-to-back launches on the same buffers between one
    event pair (500 / 1000 / 1000 / 5000, as there).  Inputs are seeded N(0,1)
    (the reference times uninitialised buffers); ~30 ms of copies warm the clocks
    before each shape.  Published times: RTX 2060 Max-Q, README.md:25-64.
    Bytes: this repo's algorithmic model (each input read once, each output
    written once); the reference's own GB/s counts RMSNorm's x twice."""
    from quantlib_amd import lib as _lib
    p_, i_, f_ = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    L = _lib()
    softmax = L._Z14launch_softmaxPKfPfiiP12ihipStream_t
    softmax.argtypes, softmax.restype = [p_, p_, i_, i_, p_], None
    rmsnorm = L._Z14launch_rmsnormPKfS0_PfiifP12ihipStream_t
    rmsnorm.argtypes, rmsnorm.restype = [p_, p_, p_, i_, i_, f_, p_], None
    rope = L._Z11launch_ropePfiiifP12ihipStream_t
    rope.argtypes, rope.restype = [p_, i_, i_, i_, f_, p_], None
    swiglu = L._Z13launch_swigluPKfS0_PfiiP12ihipStream_t
    swiglu.argtypes, swiglu.restype = [p_, p_, p_, i_, i_, p_], None
    r = np.random.default_rng(17)
    up = lambda *shape: ql.DeviceArray.from_numpy(r.standard_normal(shape, dtype=np.float32))
    out = []

    def timed(launch, reps):
        heat(ql, st)
        launch()
        ql.synchronize()
        a, b = ql.Event(), ql.Event()
        a.record(st)
        for _ in range(reps):
            launch()
        b.record(st)
        ql.synchronize()
        return a.elapsed_ms(b) * 1e3 / reps

    def row(what, shape, nbytes, us, ref_ms, where):
        out.append({"config": f"reference benchmark ({where}) {shape}",
                    "kernel": f"{what} (reference RTX 2060: {ref_ms * 1e3:.1f} us; {ref_ms * 1e3 / us:.1f}x faster)",
                    "bytes": nbytes, "us": round(us, 2), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
                    "frac_peak": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
                    "reference_us": round(ref_ms * 1e3, 1), "speedup_vs_reference": round(ref_ms * 1e3 / us, 1)})

    for n, ref_ms in ((512, 0.0136), (1024, 0.0377), (2048, 0.1430), (4096, 0.6598)):
        x, y = up(n, n), ql.DeviceArray((n, n), np.float32)
        us = timed(lambda: softmax(x.ptr, y.ptr, n, n, st), 500)
        row("launch_softmax", f"{n}x{n}", 2 * n * n * 4, us, ref_ms, "tests/benchmark_all.cu:89-118")
        del x, y
    for dim, ref_ms in ((512, 0.0390), (1024, 0.0755), (2048, 0.1494), (4096, 0.3757)):
        x, w, y = up(2048, dim), up(dim), ql.DeviceArray((2048, dim), np.float32)
        us = timed(lambda: rmsnorm(x.ptr, w.ptr, y.ptr, 2048, dim, 1e-5, st), 1000)
        row("launch_rmsnorm", f"2048x{dim}", 2 * 2048 * dim * 4 + dim * 4, us, ref_ms,
            "tests/benchmark_all.cu:121-153")
        del x, w, y
    for seq, ref_ms in ((128, 0.0113), (512, 0.0729), (1024, 0.1429), (2048, 0.2842)):
        x = up(seq, 32 * 128)
        us = timed(lambda: rope(x.ptr, seq, 32, 128, 1e4, st), 1000)
        row("launch_rope (32 heads x 128, in place)", f"seq {seq}", 2 * seq * 32 * 128 * 4, us, ref_ms,
            "tests/benchmark_all.cu:190-222")
        del x
    for rows_, ref_ms in ((1, 0.0339), (32, 0.0110), (128, 0.0377), (512, 0.1434)):
        g, u, o = up(rows_, 5632), up(rows_, 5632), ql.DeviceArray((rows_, 5632), np.float32)
        us = timed(lambda: swiglu(g.ptr, u.ptr, o.ptr, rows_, 5632, st), 5000)
        row("launch_swiglu", f"{rows_}x5632", 3 * rows_ * 5632 * 4, us, ref_ms,
            "tests/benchmark_all.cu:225-262")
        del g, u, o
    return out


def kvcache_append_rows(ql, np, st):
    """The reference's per-token KV-cache benchmark (tests/benchmark_all.cu:265-291,
    README.md:66-73): an fp32 KVCache of n_layers x 512 positions x 4 kv heads x
    64, one kvcache_append per layer per token (the drop-in shim of
    include/quantlib_compat.h, one kernel per call), current_len advanced after
    each token, 1000 tokens.  The loop is driven from Python through ctypes, so
    host time per call includes the interpreter's call cost."""
    from quantlib_amd import lib as _lib
    p_, i_ = ctypes.c_void_p, ctypes.c_int

    class KVCache(ctypes.Structure):  # include/kv_cache.h:12-20
        _fields_ = [("k_cache", p_), ("v_cache", p_), ("n_layers", i_), ("max_seq_len", i_),
                    ("n_heads", i_), ("head_dim", i_), ("current_len", i_)]

    L = _lib()
    create = L._Z14kvcache_createiiii
    create.argtypes, create.restype = [i_, i_, i_, i_], ctypes.POINTER(KVCache)
    append = L._Z14kvcache_appendP7KVCacheiPKfS2_P12ihipStream_t
    append.argtypes, append.restype = [ctypes.POINTER(KVCache), i_, p_, p_, p_], None
    free = L._Z12kvcache_freeP7KVCache
    free.argtypes, free.restype = [ctypes.POINTER(KVCache)], None
    out = []
    for n_layers, n_kv, hd in ((4, 4, 64), (8, 4, 64), (16, 4, 64), (32, 4, 64)):
        cache = create(n_layers, 512, n_kv, hd)
        if not cache:
            raise RuntimeError("kvcache_create failed")
        dk = ql.DeviceArray.from_numpy(np.ones(n_kv * hd, np.float32))
        dv = ql.DeviceArray.from_numpy(np.ones(n_kv * hd, np.float32))
        ql.synchronize()
        reps = 1000
        a, b = ql.Event(), ql.Event()
        t0 = time.perf_counter()
        a.record(st)
        for _ in range(reps):
            for layer in range(n_layers):
                append(cache, layer, dk.ptr, dv.ptr, st)
            cache.contents.current_len = (cache.contents.current_len + 1) % 256
        b.record(st)
        ql.synchronize()
        host_ms = (time.perf_counter() - t0) * 1e3 / reps
        ms = a.elapsed_ms(b) / reps
        nb = 4 * n_layers * n_kv * hd * 4  # per token: read K,V slices, write them, every layer
        out.append({"config": f"KV cache {n_layers} layers, kv={n_kv}, hd={hd}",
                    "kernel": "kvcache_append shim, ms per token (reference README.md:66-73: "
                              "0.2751 / 0.5461 / 1.0679 / 0.7727)",
                    "bytes": nb, "us": round(ms * 1e3, 2), "ms_per_token": round(ms, 4),
                    "host_ms_per_token": round(host_ms, 4),
                    "us_per_append": round(ms * 1e3 / n_layers, 2),
                    "GBps": round(nb / (ms * 1e-3) / 1e9, 3), "frac_peak": None})
        free(cache)
        del dk, dv
    return out


def layer_rows(ql, np, chain, reps):
    """One whole Llama-3-8B-shaped decoder layer through the engine -- fp16 weights
    (ql_engine_layer_f16: hipBLASLt GEMMs + the fused kernels + attention) and FP8
    weights (ql_engine_layer_fp8: the reference's quantize_model config, E4M3 in
    groups of 128 with its own codec) -- for a 8192-token prefill of one sequence,
    a decode step of 64 sequences at 4096 keys and a one-sequence decode step
    (the reference's quantized generation).  Weights are seeded N(0, 1/fan_in);
    the step rotates over several weight sets (>= 600 MB) so that none is still
    in the 256 MB MALL, as the layers of a model stream theirs."""
    st = chain.stream
    up = ql.DeviceArray.from_numpy
    r = np.random.default_rng(21)
    QKV = (HQ + 2 * HKV) * HD
    shapes = {"wqkv": (QKV, D), "wo": (D, HQ * HD), "w_gate": (F, D), "w_up": (F, D), "w_down": (D, F)}
    host = {k: (r.standard_normal(sh, dtype=np.float32) * np.float32(sh[1] ** -0.5)).astype(np.float16)
            .view(np.uint16) for k, sh in shapes.items()}
    norm = up(np.ones(D, np.float16).view(np.uint16))
    f16_sets = [{k: up(v) for k, v in host.items()} for _ in range(3)]
    del host
    lw16 = [ql.LayerWeights(norm.ptr, w["wqkv"].ptr, w["wo"].ptr, norm.ptr, w["w_gate"].ptr, w["w_up"].ptr,
                            w["w_down"].ptr) for w in f16_sets]
    fmt, gran, gs, mode = ql.FP8_E4M3, ql.QUANT_PER_GROUP, 128, ql.FP8_MODE_REFERENCE
    fp8_sets, lw8 = [], []
    for i in range(6):
        src = f16_sets[i % 3]
        w8 = {}
        for k, (n_, k_) in shapes.items():
            codes = ql.DeviceArray((n_ * k_,), np.uint8)
            scales = ql.DeviceArray((n_ * k_ // gs,), np.float32)
            ql.call("ql_fp8_quantize", src[k].ptr, n_, k_, fmt, gran, gs, mode, codes.ptr, scales.ptr, st)
            w8[k] = (codes, scales)
        fp8_sets.append(w8)
        fw = {k: ql.FP8Weight(c.ptr, sc.ptr) for k, (c, sc) in w8.items()}
        # static weights: decode as QL_FP8_MODE_REFERENCE_CLEAN when the scan finds
        # none of the codes whose reference decode differs (same results)
        dmode = ql.FP8_MODE_REFERENCE_CLEAN if all(
            ref_special_count(ql, np, w8[k][0], n_ * k_, fmt, st) == 0 for k, (n_, k_) in shapes.items()) else mode
        lw8.append(ql.LayerWeightsFP8(norm.ptr, fw["wqkv"], fw["wo"], norm.ptr, fw["w_gate"], fw["w_up"],
                                      fw["w_down"], fmt, gran, gs, dmode))
    ql.synchronize()
    dims = ql.LayerDims(D, HQ, HKV, HD, F, THETA, EPS, ql.ROPE_HALF)
    rows = []
    gemm_flops = lambda m: 2.0 * m * D * (QKV + HQ * HD + 3 * F)
    w_bytes = sum(n_ * k_ for n_, k_ in shapes.values())
    for label, S, C, q_len in (("prefill 1 seq x 8192 tokens", 1, T, T),
                               ("decode 64 seq x 4096 ctx", 64, 4096, 1),
                               ("decode 1 seq x 4096 ctx", 1, 4096, 1)):
        nbs = C // PAGE
        nb = S * nbs
        blk = L_POOL * PAGE * HKV * HD
        kpool = ql.DeviceArray((nb * blk,), np.uint16)
        vpool = ql.DeviceArray((nb * blk,), np.uint16)
        kpool.fill_bytes(0x3C)
        vpool.fill_bytes(0x3C)
        kp = up(np.array([kpool.ptr + 2 * blk * b for b in range(nb)], np.int64))
        vp = up(np.array([vpool.ptr + 2 * blk * b for b in range(nb)], np.int64))
        n_rows = S * q_len
        if q_len == 1:   # one decode row per sequence at position C-1
            pos = np.full(S, C - 1, np.int32)
            tables = r.permutation(nb).astype(np.int32).reshape(S, nbs)
            slots = (tables[:, (C - 1) // PAGE] * PAGE + (C - 1) % PAGE).astype(np.int32)
        else:
            pos = np.arange(C, dtype=np.int32)
            tables = np.arange(nb, dtype=np.int32).reshape(1, nb)
            slots = (tables[0, pos // PAGE] * PAGE + pos % PAGE).astype(np.int32)
        arrs = {"pos": up(pos), "slots": up(slots), "cu": up(np.arange(S + 1, dtype=np.int32) * q_len),
                "ctx": up(np.full(S, C, np.int32)), "bt": up(tables.reshape(-1))}
        sd = ql.StepDevice(n_rows, S, q_len, C, nbs, arrs["pos"].ptr, arrs["slots"].ptr, arrs["cu"].ptr,
                           arrs["ctx"].ptr, arrs["bt"].ptr, kp.ptr, vp.ptr, nb, L_POOL)
        eng = ctypes.c_void_p()
        ql.call("ql_engine_create_fp8", ctypes.byref(dims), n_rows, S, C, gran, gs, ctypes.byref(eng))
        x = up(r.standard_normal((n_rows, D), dtype=np.float32).astype(np.float16).view(np.uint16))
        deltas = [ql.DeviceArray((n_rows, D), np.uint16) for _ in range(2)]
        fp8_kind = "fp8 e4m3 g128" + (" (reference codes, checked clean)"
                                      if lw8[0].mode == ql.FP8_MODE_REFERENCE_CLEAN else "")
        passes = [("fp16", "ql_engine_layer_f16", lw16, 2 * w_bytes, False),
                  (fp8_kind, "ql_engine_layer_fp8", lw8, w_bytes + 4 * w_bytes // gs, False)]
        if q_len == 1:   # decode steps again after ql_engine_tune picked the GEMM plans
            passes.insert(1, ("fp16", "ql_engine_layer_f16", lw16, 2 * w_bytes, True))
        for kind, fn, lws, wb, tuned in passes:
            if tuned:
                ql.call("ql_engine_tune", eng, n_rows, st)
                kind += " (GEMM plans tuned)"

            def launch(i, fn=fn, lws=lws):
                ql.call(fn, eng, ctypes.byref(lws[i % len(lws)]), i % L_POOL, x.ptr,
                        deltas[(i + 1) % 2].ptr if i else None, deltas[i % 2].ptr, ctypes.byref(sd), st)
            if q_len > 1:
                warm_on(ql, st, launch)   # prefill layers are matrix-core bound
            else:
                heat(ql, st)
            for i in range(max(3, 2 * len(lws))):   # every weight set before timing
                launch(i)
            ql.synchronize()
            n = max(6, reps // 10)
            a, b = ql.Event(), ql.Event()
            a.record(st)
            for i in range(n):
                launch(i + 3)
            b.record(st)
            us = a.elapsed_ms(b) * 1e3 / n
            fl = gemm_flops(n_rows) + (4.0 * (C * (C + 1) / 2) * HD * HQ if q_len > 1 else 4.0 * S * C * HD * HQ)
            rows.append({"config": f"C5 decoder layer, {label}, {kind} weights", "kernel": fn[3:],
                         "bytes": 0, "us": round(us, 2), "GBps": 0.0, "frac_peak": 0.0,
                         "weight_bytes": wb,
                         "tflops": round(fl / (us * 1e-6) / 1e12, 1),
                         "frac_mfma_peak": round(fl / (us * 1e-6) / 1e12 / PEAK_MFMA_F16_TFLOPS, 4),
                         "tokens_per_s_per_layer": round(n_rows / (us * 1e-6), 1)})
            if q_len == 1:
                # the whole 32-layer decode step captured once and replayed
                # (ql_graph_*): one submission instead of ~16 launches per layer
                graph = ctypes.c_void_p()
                ql.call("ql_graph_begin", st)
                try:
                    for l in range(L_POOL):
                        launch(l)
                finally:
                    ql.call("ql_graph_end", st, ctypes.byref(graph))
                heat(ql, st)
                for _ in range(2):
                    ql.call("ql_graph_launch", graph, st)
                ql.synchronize()
                ng = max(3, reps // 20)
                a, b = ql.Event(), ql.Event()
                a.record(st)
                for _ in range(ng):
                    ql.call("ql_graph_launch", graph, st)
                b.record(st)
                us_g = a.elapsed_ms(b) * 1e3 / (ng * L_POOL)
                ql.call("ql_graph_destroy", graph)
                rows.append({"config": f"C5 decoder layer, {label}, {kind} weights, {L_POOL}-layer step "
                                       "in one HIP graph (per layer)", "kernel": fn[3:],
                             "bytes": 0, "us": round(us_g, 2), "GBps": 0.0, "frac_peak": 0.0,
                             "weight_bytes": wb, "weight_GBps": round(wb / (us_g * 1e-6) / 1e9, 1),
                             "tflops": round(fl / (us_g * 1e-6) / 1e12, 1),
                             "frac_mfma_peak": round(fl / (us_g * 1e-6) / 1e12 / PEAK_MFMA_F16_TFLOPS, 4),
                             "tokens_per_s_per_layer": round(n_rows / (us_g * 1e-6), 1)})
        ql.call("ql_engine_destroy", eng)
        del kpool, vpool
    del f16_sets, fp8_sets
    return rows


def ref_special_count(ql, np, codes, n, fmt, st):
    """ql_fp8_count_ref_special of n codes (device), read back."""
    cnt = ql.DeviceArray((1,), np.uint64)
    ql.call("ql_fp8_count_ref_special", codes.ptr, n, fmt, cnt.ptr, st)
    ql.synchronize()
    return int(cnt.numpy()[0])


def fp8_rows(ql, np, reps):
    """The FP8 weight path on Llama-3-8B FFN shapes: the skinny FP8-weight GEMM
    (ql_fp8_gemm_f16) at decode row counts next to the fp16 library GEMM on the
    same shape, and the codec (quantize = scales + encode, dequantize) on a
    14336 x 4096 matrix.  Each launch reads a weight copy last touched >= 600 MB
    earlier (rotating copies), so the weights stream from HBM.  Algorithmic bytes:
    codes (1 B per weight) + scales + activations in + outputs out."""
    st = ql.stream()
    r = np.random.default_rng(31)
    rows = []

    def rotating(n_bytes):
        return max(2, -(-(640 << 20) // n_bytes))

    def timed(launch, n):
        # at least 30 launches per pass (a 10-launch pass moved by up to 60% between
        # runs at 15-30 us per launch), the median of three passes
        n = max(n, 30)
        heat(ql, st)
        for i in range(n):   # as many warm-up launches as timed ones: every rotated copy once
            launch(i)
        ql.synchronize()
        passes = []
        for _ in range(3):
            a, b = ql.Event(), ql.Event()
            a.record(st)
            for i in range(n):
                launch(i + 3)
            b.record(st)
            passes.append(a.elapsed_ms(b) * 1e3 / n)
        return sorted(passes)[1]

    for N, K, what in ((F, D, "gate/up 14336x4096"), (D, F, "down 4096x14336")):
        w16 = (r.standard_normal((N, K), dtype=np.float32) * np.float32(K ** -0.5)).astype(np.float16)
        d16 = [ql.DeviceArray.from_numpy(w16.view(np.uint16)) for _ in range(rotating(2 * N * K))]
        del w16
        for M in (1, 64):
            a = ql.DeviceArray.from_numpy(r.standard_normal((M, K), dtype=np.float32).astype(np.float16)
                                          .view(np.uint16))
            out = ql.DeviceArray((M, N), np.uint16)
            us16 = timed(lambda i: ql.call("ql_gemm_f16", a.ptr, d16[i % len(d16)].ptr, out.ptr, M, N, K, st),
                         max(6, reps // 5))
            for fmt, gran, gs, mode, label in (
                    (ql.FP8_E4M3, ql.QUANT_PER_GROUP, 128, ql.FP8_MODE_REFERENCE, "e4m3 g128 reference codec"),
                    (ql.FP8_E4M3, ql.QUANT_PER_GROUP, 128, ql.FP8_MODE_REFERENCE_CLEAN,
                     "e4m3 g128 reference codes, checked clean"),
                    (ql.FP8_E4M3, ql.QUANT_PER_CHANNEL, 0, ql.FP8_MODE_OCP, "e4m3 per-channel OCP")):
                n_sc = N * K // 128 if gs else N
                codes = [(ql.DeviceArray((N * K,), np.uint8), ql.DeviceArray((n_sc,), np.float32))
                         for _ in range(rotating(N * K))]
                qmode = ql.FP8_MODE_REFERENCE if mode == ql.FP8_MODE_REFERENCE_CLEAN else mode
                for i, (c, sc) in enumerate(codes):
                    ql.call("ql_fp8_quantize", d16[i % len(d16)].ptr, N, K, fmt, gran, gs, qmode, c.ptr, sc.ptr, st)
                if mode == ql.FP8_MODE_REFERENCE_CLEAN:
                    assert all(ref_special_count(ql, np, c, N * K, fmt, st) == 0 for c, _ in codes)
                size = ctypes.c_size_t()
                ql.call("ql_fp8_gemm_workspace_size", M, N, K, gran, gs, ctypes.byref(size))
                ws = ql.DeviceArray((max(size.value, 16),), np.uint8)
                us = timed(lambda i: ql.call("ql_fp8_gemm_f16", a.ptr, codes[i % len(codes)][0].ptr,
                                             codes[i % len(codes)][1].ptr, M, N, K, fmt, gran, gs, mode,
                                             out.ptr, ws.ptr, size.value, st), max(6, reps // 5))
                nbytes = N * K + 4 * n_sc + 2 * M * K + 2 * M * N
                gbs = nbytes / (us * 1e-6) / 1e9
                rows.append({"config": f"FP8 GEMM {what}, {M} rows, {label}", "kernel": "fp8_gemm_f16",
                             "bytes": nbytes, "us": round(us, 2), "GBps": round(gbs, 1),
                             "frac_peak": round(gbs / PEAK_HBM_GBS, 4), "fp16_gemm_us": round(us16, 2),
                             "speedup_vs_fp16": round(us16 / us, 2), "workspace_bytes": size.value})
                del codes, ws
        del d16
    # codec on one 14336 x 4096 matrix
    N, K = F, D
    x = (r.standard_normal((N, K), dtype=np.float32)).astype(np.float16).view(np.uint16)
    xs = [ql.DeviceArray.from_numpy(x) for _ in range(rotating(2 * N * K))]
    del x
    nsets = len(xs)
    qs = [(ql.DeviceArray((N * K,), np.uint8), ql.DeviceArray((N * K // 128,), np.float32)) for _ in range(nsets)]
    for mode, mname in ((ql.FP8_MODE_REFERENCE, "reference codec"), (ql.FP8_MODE_OCP, "OCP")):
        # per tensor reads the matrix twice (its one scale first): 5 bytes an element
        for gran, gs, glabel, n_sc in ((ql.QUANT_PER_GROUP, 128, "g128", N * K // 128),
                                       (ql.QUANT_PER_CHANNEL, 0, "per channel", N),
                                       (ql.QUANT_PER_TENSOR, 0, "per tensor", 1)):
            us = timed(lambda i: ql.call("ql_fp8_quantize", xs[i % nsets].ptr, N, K, ql.FP8_E4M3, gran, gs, mode,
                                         qs[i % nsets][0].ptr, qs[i % nsets][1].ptr, st),
                       max(6, reps // 5))
            nbytes = 3 * N * K + 4 * n_sc
            gbs = nbytes / (us * 1e-6) / 1e9
            rows.append({"config": f"FP8 quantize 14336x4096 e4m3 {glabel}, {mname}", "kernel": "fp8_quantize",
                         "bytes": nbytes, "us": round(us, 2), "GBps": round(gbs, 1),
                         "frac_peak": round(gbs / PEAK_HBM_GBS, 4)})
        nbytes = 3 * N * K + 4 * N * K // 128
        us = timed(lambda i: ql.call("ql_fp8_dequantize", qs[i % nsets][0].ptr, qs[i % nsets][1].ptr, N, K,
                                     ql.FP8_E4M3, ql.QUANT_PER_GROUP, 128, mode, xs[(i + 1) % nsets].ptr, st),
                   max(6, reps // 5))
        gbs = nbytes / (us * 1e-6) / 1e9
        rows.append({"config": f"FP8 dequantize 14336x4096 e4m3 g128, {mname}", "kernel": "fp8_dequantize",
                     "bytes": nbytes, "us": round(us, 2), "GBps": round(gbs, 1),
                     "frac_peak": round(gbs / PEAK_HBM_GBS, 4)})
    del xs, qs
    return rows


def attention_rows(ql, np, chain, reps):
    """Attention over the C5 shapes: causal prefill of the 8192 tokens (contiguous
    Q/K/V and the paged pool the chain writes) -- MFMA-bound, reported in TFLOP/s
    against the dense fp16 peak -- and paged decode, HBM-bound on the K/V rows."""
    st = chain.stream
    rows = []

    def timed(launch, n, compute_bound=False):
        if compute_bound:
            warm_on(ql, st, launch)   # matrix-core bound: warm on the kernel itself
        else:
            heat(ql, st)
            for i in range(n):   # as many warm-up launches as timed ones: every rotated copy once
                launch(i)
            ql.synchronize()
        a, b = ql.Event(), ql.Event()
        a.record(st)
        for i in range(n):
            launch(i)
        b.record(st)
        return a.elapsed_ms(b) * 1e3 / n

    for layer in range(L_POOL):   # every layer of the pool holds K/V rows
        chain.k_paged(chain.sets[layer % NSETS], layer)
    flops = 4.0 * (T * (T + 1) / 2) * HD * HQ
    io = 2 * T * HQ * HD * 2 + 2 * T * HKV * HD * 2
    out = [ql.DeviceArray((T, HQ * HD), np.uint16) for _ in range(2)]
    up = ql.DeviceArray.from_numpy
    cu, ctx, table = up(np.array([0, T], np.int32)), up(np.array([T], np.int32)), \
        up(np.arange(chain.nb, dtype=np.int32))
    n_att = max(3, reps // 10)
    n_pre = max(20, reps // 2)   # prefill: ~15 ms timed after the warm-up on the kernel
    us = timed(lambda i: ql.call("ql_flash_attention_f16", chain.sets[i % NSETS]["q"].ptr,
                                 chain.sets[i % NSETS]["k"].ptr, chain.sets[i % NSETS]["v"].ptr,
                                 out[i % 2].ptr, T, HQ, HKV, HD, 1, st), n_pre, compute_bound=True)
    rows.append({"config": "C5 attention prefill T=8192 causal", "kernel": "flash_attention_f16",
                 "bytes": io, "us": round(us, 2), "GBps": round(io / (us * 1e-6) / 1e9, 1),
                 "frac_peak": round(io / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
                 "tflops": round(flops / (us * 1e-6) / 1e12, 1),
                 "frac_mfma_peak": round(flops / (us * 1e-6) / 1e12 / PEAK_MFMA_F16_TFLOPS, 4)})
    us = timed(lambda i: ql.call("ql_paged_attention_f16", chain.sets[i % NSETS]["q"].ptr,
                                 out[i % 2].ptr, HQ * HD, HQ * HD, T, 1, cu.ptr, ctx.ptr, T, table.ptr,
                                 chain.nb, chain.kptrs.ptr, chain.vptrs.ptr, chain.nb, i % L_POOL,
                                 L_POOL, HQ, HKV, HD, 1, st), n_pre, compute_bound=True)
    rows.append({"config": "C5 attention prefill T=8192 causal", "kernel": "paged_attention_f16",
                 "bytes": io, "us": round(us, 2), "GBps": round(io / (us * 1e-6) / 1e9, 1),
                 "frac_peak": round(io / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
                 "tflops": round(flops / (us * 1e-6) / 1e12, 1),
                 "frac_mfma_peak": round(flops / (us * 1e-6) / 1e12 / PEAK_MFMA_F16_TFLOPS, 4)})
    del out
    # decode: S sequences x C context tokens, Llama-3-8B heads, pool of L_POOL layers
    r = np.random.default_rng(11)
    for S, C in ((64, 4096), (1, 8192)):
        nbs = C // PAGE
        nb = S * nbs
        blk = L_POOL * PAGE * HKV * HD
        kpool = ql.DeviceArray((nb * blk,), np.uint16)
        vpool = ql.DeviceArray((nb * blk,), np.uint16)
        kpool.fill_bytes(0x3C)   # every element 1.0078125: finite, no NaN from unwritten rows
        vpool.fill_bytes(0x3C)
        kp = up(np.array([kpool.ptr + 2 * blk * b for b in range(nb)], np.int64))
        vp = up(np.array([vpool.ptr + 2 * blk * b for b in range(nb)], np.int64))
        q = up(r.standard_normal((S, HQ * HD), dtype=np.float32).astype(np.float16).view(np.uint16))
        o = ql.DeviceArray((S, HQ * HD), np.uint16)
        ctxs = up(np.full(S, C, np.int32))
        bt = up(r.permutation(nb).astype(np.int32).reshape(S, nbs))
        size = ctypes.c_size_t()
        ql.call("ql_paged_decode_workspace_size", S, HQ, HKV, HD, C, ctypes.addressof(size))
        ws = ql.DeviceArray((max(size.value, 16),), np.uint8)
        kv_bytes = S * C * HKV * HD * 2 * 2
        us = timed(lambda i: ql.call("ql_paged_decode_attention_f16", q.ptr, o.ptr, HQ * HD, HQ * HD, S,
                                     ctxs.ptr, C, bt.ptr, nbs, kp.ptr, vp.ptr, nb, i % L_POOL, L_POOL,
                                     HQ, HKV, HD, ws.ptr, size.value, st), max(3, reps // 5))
        gbs = (kv_bytes + 2 * S * HQ * HD * 2) / (us * 1e-6) / 1e9
        rows.append({"config": f"decode {S} seq x {C} ctx (paged, {L_POOL}-layer blocks)",
                     "kernel": "paged_decode_attention_f16", "bytes": kv_bytes + 2 * S * HQ * HD * 2,
                     "us": round(us, 2), "GBps": round(gbs, 1), "frac_peak": round(gbs / PEAK_HBM_GBS, 4),
                     "splits_workspace_bytes": size.value})
        del kpool, vpool, ws
    # decode over the contiguous cache of the reference's fp16 layer (one sequence,
    # src/fp16_forward.cu:202-209): the single pass of ql_attention_f16 against the
    # key split of ql_decode_attention_f16; K/V rows [8192, 8 x 128], 4 rotating copies
    C = 8192
    kvs = [(up(r.standard_normal((C, HKV * HD), dtype=np.float32).astype(np.float16).view(np.uint16)),
            up(r.standard_normal((C, HKV * HD), dtype=np.float32).astype(np.float16).view(np.uint16)))
           for _ in range(4)]
    q = up(r.standard_normal((1, HQ * HD), dtype=np.float32).astype(np.float16).view(np.uint16))
    o = ql.DeviceArray((1, HQ * HD), np.uint16)
    size = ctypes.c_size_t()
    ql.call("ql_decode_attention_workspace_size", HQ, HKV, HD, C, ctypes.addressof(size))
    ws = ql.DeviceArray((max(size.value, 16),), np.uint8)
    nbytes = C * HKV * HD * 2 * 2 + 2 * HQ * HD * 2
    for label, fn in (("attention_f16 (q_len 1, one pass)",
                       lambda i: ql.call("ql_attention_f16", q.ptr, kvs[i % 4][0].ptr, kvs[i % 4][1].ptr, o.ptr,
                                         1, C, HQ, HKV, HD, HQ * HD, HKV * HD, HQ * HD, 1, st)),
                      ("decode_attention_f16 (key split + combine)",
                       lambda i: ql.call("ql_decode_attention_f16", q.ptr, kvs[i % 4][0].ptr, kvs[i % 4][1].ptr,
                                         o.ptr, C, HQ, HKV, HD, HKV * HD, ws.ptr, size.value, st))):
        us = timed(fn, max(3, reps // 5))
        gbs = nbytes / (us * 1e-6) / 1e9
        rows.append({"config": f"decode 1 seq x {C} ctx (contiguous cache)", "kernel": label, "bytes": nbytes,
                     "us": round(us, 2), "GBps": round(gbs, 1), "frac_peak": round(gbs / PEAK_HBM_GBS, 4)})
    del kvs, ws
    return rows


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); "
              "every kernel is independent per token/row, see DESIGN.md for how it shards",
              file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import quantlib_amd as ql

    ql.lib()  # raises if the HIP library is not built
    if ql.device_count() < 1:
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.all_configs:
        rows = all_configs(ql, np, args.reps, tuple(g for g in args.only.split(",") if g))
        print("| config | kernel | algorithmic bytes | us per launch | GB/s | % of 8 TB/s | vs a copy of the same bytes |")
        print("|---|---|---|---|---|---|---|")
        for r_ in rows:
            extra = (f" ({r_['tflops']:.0f} TFLOP/s, {100 * r_['frac_mfma_peak']:.1f}% of fp16 MFMA peak)"
                     if "tflops" in r_ else "")
            frac = "-" if r_["frac_peak"] is None else f"{100 * r_['frac_peak']:.1f}"
            vs = f"{r_['vs_copy']:.3f} (copy {r_['copy_same_bytes_us']:.2f} us)" if "vs_copy" in r_ else "-"
            print(f"| {r_['config']} | {r_['kernel']}{extra} | {r_['bytes']:,} | {r_['us']:.2f} | "
                  f"{r_['GBps']:.2f} | {frac} | {vs} |", flush=True)
        print(json.dumps({"all_configs": rows}), flush=True)
        return
    chain = Chain(ql, np)

    # clock warm-up by time, independent of --warmup: the clocks need ~20 ms of
    # sustained load to ramp (a kernel trace shows the step settle from 236 to
    # ~230 us), so ~30 ms of copies and then >= 30 ms of chain steps run first
    heat(ql, chain.stream, CLOCK_WARMUP_MS / 2)
    warm_steps = warm_on(ql, chain.stream, lambda i: chain.step(), CLOCK_WARMUP_MS / 2)
    for _ in range(args.warmup):
        chain.step()
    ql.synchronize()

    # timed region: K steps and nothing else, one event pair at its edges.  The
    # same region runs once first with one untimed step: the first such region
    # in a process costs ~45 us more host time than later ones (a probe of this
    # bench: 61 us of host clock over its events in the first region, 15 us in
    # every later one), which at the driver's 20 steps is 2 us a step
    timed_region(ql, chain, 1)
    wall, ev_ms = timed_region(ql, chain, args.steps)

    ms_per_step = wall / args.steps * 1e3
    ev_ms_per_step = ev_ms / args.steps
    # per-kernel durations, each kernel in its own bracketed pass after the timed region
    kernels = breakdown(chain, ql, args.breakdown_reps)
    sw = kernels["swiglu_f16"]
    sw_us = sw["us_mean"]
    sw_gbs = BYTES["swiglu_f16"] / (sw_us * 1e-6) / 1e9

    traffic = None
    tf = pathlib.Path(args.traffic_file)
    if tf.exists():
        try:
            traffic = json.loads(tf.read_text()).get("swiglu_f16_c5", {}).get("hbm_bytes_per_launch")
        except (ValueError, AttributeError):
            traffic = None

    cpu_info = host_cpu()
    cpu = cpu_baseline(args.cpu_seconds) if args.cpu_seconds > 0 else None
    # all usable host cores, labelled separately (the GPU box's share is 16 cores)
    n_cores = min(16, cpu_info["nproc"])
    cpu_all = cpu_baseline(args.cpu_seconds, n_cores) if args.cpu_seconds > 0 and n_cores > 1 else None
    for c in (cpu, cpu_all):
        if c is not None:
            c.update(cpu_info)

    chain_gbs = CHAIN_BYTES / (ms_per_step * 1e-3) / 1e9
    line = {
        "metric": "achieved HBM GB/s (% of MI355X peak) per fused kernel; us per decoder layer",
        "value": round(chain_gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "clock_warmup_ms": CLOCK_WARMUP_MS,
        "clock_warmup": f"{CLOCK_WARMUP_MS / 2:.0f} ms of copies, then {warm_steps} untimed chain steps "
                        f"(>= {CLOCK_WARMUP_MS / 2:.0f} ms), then the --warmup steps, then one untimed "
                        "one-step run of the timed region's code",
        "ms_per_step": round(ms_per_step, 4),
        "us_per_decoder_layer": round(ms_per_step * 1e3, 1),
        "us_per_decoder_layer_events": round(ev_ms_per_step * 1e3, 1),
        "frac_peak": round(chain_gbs / PEAK_HBM_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) fp16; gate/up clipped to [-8,8]; w ~ U(0.5,1.5))",
        "config": {"workload": "C5 llama3-8b-shaped fp16 decoder-layer chain: add+rmsnorm, "
                               "rope q+k fused with paged kv append, add+rmsnorm, swiglu",
                   "tokens": T, "hidden": D, "heads": HQ, "kv_heads": HKV, "head_dim": HD,
                   "ffn": F, "rope_theta": THETA, "rope_pairing": "rotate-half", "kv_block": PAGE,
                   "kv_pool_layers": L_POOL, "buffer_sets": NSETS,
                   "chain_bytes_per_step": CHAIN_BYTES,
                   "chain_bytes_unfused": sum(BYTES[k] for k in CHAIN_UNFUSED),
                   "math": "fp32 with fp16 I/O"},
        "roofline": {"kernel": "swiglu_f16 [8192 x 14336]", "bound": "hbm",
                     "achieved": round(sw_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(sw_gbs / PEAK_HBM_GBS, 4), "traffic": traffic,
                     "traffic_source": "not measured in this run: rocprofv3 --pmc FETCH_SIZE and "
                                       "WRITE_SIZE of this kernel, copy-calibrated, read from "
                                       + os.path.relpath(tf, ROOT),
                     "algorithmic_bytes": BYTES["swiglu_f16"], "us_per_launch": sw_us,
                     "timing": f"{args.breakdown_reps} back-to-back launches on the work stream "
                               "between one pair of HIP events, after the timed steps",
                     "events_per_launch": sw["events_per_launch"]},
        "kernels": kernels,
        "cpu_baseline": cpu,
        "cpu_baseline_all_cores": cpu_all,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
