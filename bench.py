#!/usr/bin/env python3
"""QSA KV-cache hot path benchmark on one MI355X.

Workload ("step" = one decode token through the KV path of the 12 QSA
layers): each layer owns a 262144-token q8_0 K and V cache (2 KV heads x
256 dims, 272-byte rows); the step appends the new token's K/V rows (q8_0
quantise at its position) and runs sparse attention for 16 query heads over
a per-KV-head selection of 2051 sorted positions (3 sinks + 512 recent +
1536 uniform). Inputs are synthetic (device-generated N(0,1) with 4 outlier
channels x8), resident in HBM before timing. 16 selection sets with
different decode positions rotate across steps so the 27 MB a step gathers
is not served from the 256 MB Infinity Cache.

Modes:
  batched    -- all 12 layers' steps in one q4_hip_qsa_step_batch call: the
                appends and the split-KV attention in one launch, then the
                split merge (headline `value`).
  sequential -- per layer append + attention launches, captured into one
                hipGraph per step (what a batch-1 decode executes).

Prints one JSON line: metric, value (GB/s of algorithmic bytes), roofline of the
fused step kernel and the CPU baseline.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
PKG = ROOT / "suzuqu-engine-4exp_amd"
for _p in (PKG, ROOT / "tests"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

import q4kv  # noqa: E402

METRIC = "QSA decode µs/layer + achieved HBM GB/s (% of peak) at 262K q8_0 ctx, 1 GPU"
PEAK_GBS = 8000.0
CTX, N_KVH, HD, N_HEAD, WIDTH = 262144, 2, 256, 16, 2051
OUTLIERS = (3, 77, 150, 201)
ROW = HD // 32 * 34                       # 272 B per (position, kv head)
BPT = N_KVH * ROW                         # 544 B per token
GATHER_B = 2 * N_KVH * WIDTH * ROW        # K+V rows gathered per layer
IDX_B = N_KVH * WIDTH * 4
QO_B = N_HEAD * HD * 4
APPEND_B = 2 * N_KVH * HD * 4 + 2 * BPT   # read fp32 K,V rows + write q8 rows
# algorithmic bytes of one layer's step: gather + lists + q in / out + append
LAYER_B = GATHER_B + IDX_B + 2 * QO_B + APPEND_B  # 2 285 848 B
# what the fused append + split-KV kernel must move per layer (its partials
# stay on chip up to the merge, which is not counted here)
SPLIT_KERNEL_B = GATHER_B + IDX_B + QO_B + APPEND_B


def uniform_rows(rng, lo, hi, k):
    """Per row r, k distinct positions drawn uniformly from [lo, hi[r]),
    sorted. Vectorised: oversample with replacement, keep the distinct
    values (a uniform random subset given its size), then a uniform random
    k of them; rows with too few distinct draws are drawn again."""
    hi = np.asarray(hi, np.int64)
    out = np.empty((hi.size, k), np.int64)
    todo = np.arange(hi.size)
    while todo.size:
        span = hi[todo] - lo
        assert (span >= k).all()
        m = k + k // 4 + 64
        x = rng.integers(0, span[:, None], size=(todo.size, m), dtype=np.int64)
        x.sort(axis=1)
        dup = x[:, 1:] == x[:, :-1]
        keys = rng.random(x.shape, dtype=np.float32)
        keys[:, 1:][dup] = 2.0  # repeated values are never picked
        ok = (~dup).sum(axis=1) + 1 >= k
        pick = np.argpartition(keys, k - 1, axis=1)[:, :k]
        pick.sort(axis=1)
        rows = np.take_along_axis(x, pick, axis=1) + lo
        out[todo[ok]] = rows[ok]
        todo = todo[~ok]
    return out


def selection(rng, pos):
    n_uni = WIDTH - 3 - 512
    uni = rng.choice(pos - 512 - 2, size=n_uni, replace=False).astype(np.int64) + 3
    return np.concatenate([np.arange(3), np.sort(uni),
                           np.arange(pos - 511, pos + 1)]).astype(np.int32)


class Bench:
    def __init__(self, layers: int, sets: int):
        self.L, self.R = layers, sets
        self.rt = rt = q4kv.Runtime()
        self.lib = lib = rt.lib
        self.synth = synth = C.CDLL(str(PKG / "lib" / "libq4kv_synth.so"))
        synth.q4kv_synth_heads.restype = C.c_int
        synth.q4kv_synth_heads.argtypes = [C.c_void_p, C.c_uint64, C.c_uint32, C.c_uint64,
                                           C.c_int, C.c_int, C.c_int, C.c_int]
        synth.q4kv_gather_probe_us.restype = C.c_double
        synth.q4kv_gather_probe_us.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32,
                                               C.c_uint32, C.c_uint32, C.c_uint32, C.c_int]

        def gen(ptr, n, seed):
            # the generator launches on the null stream, which does not order
            # against the library's non-blocking stream: drain that first so
            # no queued kernel still reads the buffer being rewritten
            rt.sync()
            assert synth.q4kv_synth_heads(ptr, n, HD, seed, *OUTLIERS) == 0

        self.gen = gen
        n = CTX * N_KVH * HD
        scratch = rt.alloc(n * 4)
        self.kc, self.vc = [], []
        for layer in range(self.L):
            for lst, seed in ((self.kc, 2 * layer + 1), (self.vc, 2 * layer + 2)):
                cache = rt.alloc(CTX * BPT)
                gen(scratch, n, 1000 + seed)
                assert lib.q4_hip_f32_to_q8(cache, scratch, n)
                lst.append(cache)
        rt.sync()
        rt.free(scratch)
        # per-set decode positions, selections and fresh q / new K,V rows
        self.pos = [CTX - 1 - 600 * s for s in range(self.R)]
        rng = np.random.default_rng(1235)
        sel = np.empty((self.R, self.L, N_KVH, WIDTH), np.int32)
        for s in range(self.R):
            for layer in range(self.L):
                for kh in range(N_KVH):
                    sel[s, layer, kh] = selection(rng, self.pos[s])
        self.sel_host = sel
        self.d_sel = rt.upload(sel)
        self.d_q = rt.alloc(self.R * self.L * N_HEAD * HD * 4)
        self.d_nk = rt.alloc(self.R * self.L * N_KVH * HD * 4)
        self.d_nv = rt.alloc(self.R * self.L * N_KVH * HD * 4)
        gen(self.d_q, self.R * self.L * N_HEAD * HD, 77)
        gen(self.d_nk, self.R * self.L * N_KVH * HD, 78)
        gen(self.d_nv, self.R * self.L * N_KVH * HD, 79)
        self.d_out = rt.alloc(self.L * N_HEAD * HD * 4)
        seq = (q4kv.SeqDesc * (self.R * self.L))()
        step = (q4kv.StepDesc * (self.R * self.L))()
        for s in range(self.R):
            for layer in range(self.L):
                i = s * self.L + layer
                seq[i] = q4kv.SeqDesc(self.kc[layer], self.vc[layer], self.q_ptr(s, layer),
                                      None, self.d_out + layer * QO_B,
                                      self.sel_ptr(s, layer), WIDTH, WIDTH, CTX, 0)
                step[i] = q4kv.StepDesc(seq[i], self.row_ptr(self.d_nk, s, layer),
                                        self.row_ptr(self.d_nv, s, layer), self.pos[s])
        self.d_seq = rt.alloc(C.sizeof(seq))
        self.d_step = rt.alloc(C.sizeof(step))
        assert lib.q4_hip_h2d(self.d_seq, C.addressof(seq), C.sizeof(seq))
        assert lib.q4_hip_h2d(self.d_step, C.addressof(step), C.sizeof(step))
        self.graphs = None
        self.bgraphs = None

    def q_ptr(self, s, layer):
        return self.d_q + (s * self.L + layer) * QO_B

    def sel_ptr(self, s, layer):
        return self.d_sel + (s * self.L + layer) * IDX_B

    def row_ptr(self, base, s, layer):
        return base + (s * self.L + layer) * N_KVH * HD * 4

    # ---- one step -----------------------------------------------------------
    def _enqueue_batched(self, s):
        return self.lib.q4_hip_qsa_step_batch(
            self.d_step + s * self.L * C.sizeof(q4kv.StepDesc), self.L, N_HEAD, N_KVH, HD,
            1.0 / 16, q4kv.KV_Q8, WIDTH)

    def step_batched(self, s):
        """One decode step of all layers: one q4_hip_qsa_step_batch call (the
        fused append + split-KV kernel, then the merge) enqueued directly on
        the library stream."""
        assert self._enqueue_batched(s)

    def step_batched_graph(self, s):
        """The same step replayed from a captured graph (one per selection
        set)."""
        if self.bgraphs is None:
            self.bgraphs = _graphs(self.lib, self._enqueue_batched, self.R)
        assert self.lib.q4_hip_graph_launch(self.bgraphs[s])

    def _enqueue_sequential(self, s):
        lib = self.lib
        ok = True
        for layer in range(self.L):
            ok = ok and lib.q4_hip_kv_append_d(self.kc[layer], self.vc[layer],
                                               self.row_ptr(self.d_nk, s, layer),
                                               self.row_ptr(self.d_nv, s, layer),
                                               N_KVH * HD, BPT, q4kv.KV_Q8)
            ok = ok and lib.q4_hip_qsa_decode_idx_kv(
                self.q_ptr(s, layer), self.kc[layer], self.vc[layer], None,
                self.d_out + layer * QO_B, self.sel_ptr(s, layer), WIDTH, N_KVH * WIDTH,
                WIDTH, N_HEAD, N_KVH, HD, 1, CTX, 1.0 / 16, q4kv.KV_Q8)
        return ok

    def step_sequential(self, s):
        """Per layer: q4_hip_kv_append_d then q4_hip_qsa_decode_idx_kv (the
        reference's call sequence, src/q4_fwd.c:891,922), enqueued directly."""
        self.lib.q4_hip_pos_push(self.pos[s])
        assert self._enqueue_sequential(s)

    def step_sequential_graph(self, s):
        """The same per-layer calls replayed from a captured graph."""
        if self.graphs is None:
            self.graphs = _graphs(self.lib, self._enqueue_sequential, self.R)
        self.lib.q4_hip_pos_push(self.pos[s])
        assert self.lib.q4_hip_graph_launch(self.graphs[s])

    def timed(self, step, steps, warmup, prof=False):
        # every selection set (and its graph, where one is used) runs at least
        # once before the timed region, whatever the warmup count
        for i in range(max(warmup, self.R)):
            step(i % self.R)
        self.rt.sync()
        if prof:
            assert self.lib.q4kv_prof_begin(min(steps, 4096))
        assert self.lib.q4kv_timer_begin(0)
        t0 = time.perf_counter()
        for i in range(steps):
            step(i % self.R)
        self.rt.sync()
        wall = time.perf_counter() - t0
        gpu_ms = self.lib.q4kv_timer_end_ms(0)
        kern = None
        if prof:
            tot = C.c_double()
            n = self.lib.q4kv_prof_end(C.byref(tot))
            kern = tot.value / n if n > 0 else None
        return wall, gpu_ms / 1e3, kern

    def gather_ceiling(self, iters=400):
        """The same rows the batched step gathers, DMA'd with no compute: the
        practical roofline of this access pattern on this GPU."""
        n = self.R * self.L
        kc = (C.c_void_p * n)(*[self.kc[i % self.L] for i in range(n)])
        vc = (C.c_void_p * n)(*[self.vc[i % self.L] for i in range(n)])
        ix = (C.c_void_p * n)(*[self.sel_ptr(i // self.L, i % self.L) for i in range(n)])
        d = [self.rt.alloc(8 * n) for _ in range(3)]
        for dp, arr in zip(d, (kc, vc, ix)):
            assert self.lib.q4_hip_h2d(dp, C.addressof(arr), 8 * n)
        self.rt.sync()
        us = self.synth.q4kv_gather_probe_us(d[0], d[1], d[2], self.L, self.R, N_KVH, WIDTH,
                                             iters)
        return us, self.L * GATHER_B / (us * 1e-6) / 1e9

    # ---- parity of the last batched step vs the oracle (layer 0) ------------
    def check_and_cpu(self, cpu_seconds, threads):
        from oracle_ffi import Oracle
        from synth import assert_attn_close

        orc = Oracle()
        rt, s, layer = self.rt, 0, 0
        self.rt.sync()
        kb = rt.download(self.kc[layer], CTX * BPT)
        vb = rt.download(self.vc[layer], CTX * BPT)
        q = rt.download(self.q_ptr(s, layer), QO_B, np.float32).reshape(1, N_HEAD, HD)
        nk = rt.download(self.row_ptr(self.d_nk, s, layer), N_KVH * HD * 4, np.float32)
        nv = rt.download(self.row_ptr(self.d_nv, s, layer), N_KVH * HD * 4, np.float32)
        self.step_batched(s)
        rt.sync()
        got = rt.download(self.d_out + layer * QO_B, QO_B, np.float32).reshape(1, N_HEAD, HD)
        # the downloaded caches already hold set 0's appended row: re-append on
        # the host copy, and check those bytes against the oracle's quantiser
        hk, hv = kb.copy(), vb.copy()
        pos = self.pos[s]
        orc.lib.orc_kv_append(hk.ctypes.data, hv.ctypes.data, nk.ctypes.data, nv.ctypes.data,
                              N_KVH * HD, BPT, 2, pos)
        rows_ok = bool(np.array_equal(hk[pos * BPT:(pos + 1) * BPT], kb[pos * BPT:(pos + 1) * BPT])
                       and np.array_equal(hv[pos * BPT:(pos + 1) * BPT],
                                          vb[pos * BPT:(pos + 1) * BPT]))
        sel = self.sel_host[s, layer].ravel()
        kw = dict(idx=sel, width=WIDTH, tok_stride=N_KVH * WIDTH, kvh_stride=WIDTH, max_kv=CTX)
        want = orc.attn(q, hk, hv, 2, N_HEAD, N_KVH, HD, 1, **kw)
        err = assert_attn_close(got, want, what="bench parity")
        res = {"parity_max_abs_err": err, "append_rows_bit_exact": rows_ok}
        if cpu_seconds <= 0:
            return res, None

        def run(nthreads, budget):
            n, t0 = 0, time.perf_counter()
            while True:
                orc.lib.orc_kv_append(hk.ctypes.data, hv.ctypes.data, nk.ctypes.data,
                                      nv.ctypes.data, N_KVH * HD, BPT, 2, pos)
                orc.attn(q, hk, hv, 2, N_HEAD, N_KVH, HD, 1, dbl=False, threads=nthreads, **kw)
                n += 1
                el = time.perf_counter() - t0
                if el >= budget:
                    return n, el

        n1, el1 = run(1, cpu_seconds)
        nt, elt = run(threads, max(2.0, cpu_seconds / 3))
        cpu = {
            "value": round(n1 * LAYER_B / el1 / 1e9, 4), "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": (f"{n1} single-layer decode steps (q8_0 append + sparse attention of "
                       f"16 heads over 2x2051 rows of one 262144-token q8_0 layer cache), "
                       f"fp32 C restatement of src/q4_fwd.c:330-407, 1 thread, {el1:.1f} s"),
            "us_per_layer": round(el1 / n1 * 1e6, 1),
            "openmp": {"threads": threads, "value": round(nt * LAYER_B / elt / 1e9, 4),
                       "us_per_layer": round(elt / nt * 1e6, 1)},
            "host_cpu": _cpu_model(),
            "host_nproc": len(os.sched_getaffinity(0)),
            "host_logical_cpus": os.cpu_count(),
        }
        return res, cpu


# ---------------------------------------------------------------------------
# The other BASELINE configurations, measured beside the headline (extra keys
# under "configs"; the headline `value` stays config 1).


def _graphs(lib, enqueue, n):
    """One captured graph per set (the reference's decode-graph pattern)."""
    out = []
    for r in range(n):
        assert lib.q4_hip_graph_begin() == 1
        ok = enqueue(r)
        g = lib.q4_hip_graph_end()
        assert ok and g, "graph capture failed"
        out.append(g)
    return out


def _time_graphs(b, graphs, steps):
    lib = b.lib
    for i in range(max(8, len(graphs))):
        assert lib.q4_hip_graph_launch(graphs[i % len(graphs)])
    b.rt.sync()
    t0 = time.perf_counter()
    for i in range(steps):
        assert lib.q4_hip_graph_launch(graphs[i % len(graphs)])
    b.rt.sync()
    wall = time.perf_counter() - t0
    for g in graphs:
        lib.q4_hip_graph_free(g)
    return wall / steps


def _time_direct(b, enqueue, n_sets, steps):
    """Seconds per step with each step's calls enqueued directly (no graph)."""
    for i in range(max(8, n_sets)):
        assert enqueue(i % n_sets)
    b.rt.sync()
    t0 = time.perf_counter()
    for i in range(steps):
        assert enqueue(i % n_sets)
    b.rt.sync()
    return (time.perf_counter() - t0) / steps


USE_GRAPHS = True  # --graphs 0: direct launches only (profiling runs)
CPU_BUDGET = 3.0   # seconds of CPU baseline per extra configuration (0: none)


def _cpu_rate(fn, budget):
    """Seconds per call of fn on this host, from calls repeated for about
    `budget` seconds (at least twice)."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget and n >= 2:
            return el / n


def _oracle():
    from oracle_ffi import Oracle
    return Oracle()


def _time_both(b, enqueue, n_sets, steps):
    """(direct, graph) seconds per step (graph None with --graphs 0)."""
    t_d = _time_direct(b, enqueue, n_sets, steps)
    t_g = _time_graphs(b, _graphs(b.lib, enqueue, n_sets), steps) if USE_GRAPHS else None
    return t_d, t_g


def _time_steps(b, enqueue, n_sets, steps):
    """Seconds per step, replayed from captured graphs (the reference's decode
    pattern) or, with --graphs 0, enqueued directly."""
    if USE_GRAPHS:
        return _time_graphs(b, _graphs(b.lib, enqueue, n_sets), steps)
    return _time_direct(b, enqueue, n_sets, steps)


def _us(t, div=1):
    return None if t is None else round(t / div * 1e6, 3)


def _fill(b, ptr, n_tok, kind, seed):
    """Synthetic K or V rows for n_tok tokens written at ptr in width kind."""
    rt, lib = b.rt, b.lib
    n = n_tok * N_KVH * HD
    tmp = rt.alloc(n * 4)
    b.gen(tmp, n, seed)
    if kind == q4kv.KV_Q8:
        assert lib.q4_hip_f32_to_q8(ptr, tmp, n)
    elif kind == q4kv.KV_F16:
        assert lib.q4_hip_f32_to_f16(ptr, tmp, n)
    else:
        assert lib.q4_hip_copy(ptr, tmp, n)
    rt.sync()
    rt.free(tmp)


def config2(b, steps=200, sets=10):
    """Config 2: 32 sequences, contexts log-uniform in [8192, 131072], own
    q8_0 caches; one step = every sequence's append + sparse attention
    (q4_hip_qsa_step_batch)."""
    rt, lib = b.rt, b.lib
    rng = np.random.default_rng(1236)
    n_seq = 32
    lens = np.exp(rng.uniform(np.log(8192), np.log(131072), n_seq)).astype(np.int64)
    ptrs = []
    caches = []
    for s_ in range(n_seq):
        L = int(lens[s_])
        kc, vc = rt.alloc(L * BPT), rt.alloc(L * BPT)
        _fill(b, kc, L, q4kv.KV_Q8, 3000 + 2 * s_)
        _fill(b, vc, L, q4kv.KV_Q8, 3001 + 2 * s_)
        caches.append((kc, vc, L))
    dq = rt.alloc(sets * n_seq * QO_B)
    dnk = rt.alloc(sets * n_seq * N_KVH * HD * 4)
    dnv = rt.alloc(sets * n_seq * N_KVH * HD * 4)
    b.gen(dq, sets * n_seq * N_HEAD * HD, 3500)
    b.gen(dnk, sets * n_seq * N_KVH * HD, 3501)
    b.gen(dnv, sets * n_seq * N_KVH * HD, 3502)
    dout = rt.alloc(n_seq * QO_B)
    sel = np.empty((sets, n_seq, N_KVH, WIDTH), np.int32)
    for r in range(sets):
        for s_, (_, _, L) in enumerate(caches):
            for h in range(N_KVH):
                sel[r, s_, h] = selection(rng, L - 1 - 7 * r)
    dsel = rt.upload(sel)
    steps_d = (q4kv.StepDesc * (sets * n_seq))()
    for r in range(sets):
        for s_, (kc, vc, L) in enumerate(caches):
            i = r * n_seq + s_
            seq = q4kv.SeqDesc(kc, vc, dq + i * QO_B, None, dout + s_ * QO_B,
                               dsel + i * IDX_B, WIDTH, WIDTH, L, 0)
            row = i * N_KVH * HD * 4
            steps_d[i] = q4kv.StepDesc(seq, dnk + row, dnv + row, L - 1 - 7 * r)
    dd = rt.alloc(C.sizeof(steps_d))
    assert lib.q4_hip_h2d(dd, C.addressof(steps_d), C.sizeof(steps_d))
    sz = C.sizeof(q4kv.StepDesc)
    t, t_graph = _time_both(b, lambda r: lib.q4_hip_qsa_step_batch(
        dd + r * n_seq * sz, n_seq, N_HEAD, N_KVH, HD, 1.0 / 16, q4kv.KV_Q8, WIDTH), sets, steps)
    byts = n_seq * LAYER_B
    # the gather ceiling of this step's rows: the same K/V rows of every
    # sequence DMA'd to LDS with no compute, one launch per step, the sets
    # rotating as in the timed steps
    n = sets * n_seq
    tabs = [(C.c_void_p * n)(*[caches[i % n_seq][j] for i in range(n)]) for j in (0, 1)]
    tabs.append((C.c_void_p * n)(*[dsel + i * IDX_B for i in range(n)]))
    dtabs = [rt.alloc(8 * n) for _ in range(3)]
    for dp, arr in zip(dtabs, tabs):
        assert lib.q4_hip_h2d(dp, C.addressof(arr), 8 * n)
    rt.sync()
    g_us = b.synth.q4kv_gather_probe_us(dtabs[0], dtabs[1], dtabs[2], n_seq, sets, N_KVH, WIDTH,
                                        400)
    for dp in dtabs:
        rt.free(dp)
    cpu = None
    if CPU_BUDGET > 0:
        # the oracle's fp32 path (1 thread) on 4 of the 32 sequences (their
        # caches read back), each an append + attention; the step's time is
        # the sample's mean per sequence x 32 (the work per sequence does not
        # depend on its context length)
        orc = _oracle()
        sample = [0, 9, 18, 27]
        per = []
        for s_ in sample:
            kc, vc, L = caches[s_]
            hk, hv = rt.download(kc, L * BPT), rt.download(vc, L * BPT)
            q = rt.download(dq + s_ * QO_B, QO_B, np.float32).reshape(1, N_HEAD, HD)
            row = s_ * N_KVH * HD * 4
            nk = rt.download(dnk + row, N_KVH * HD * 4, np.float32)
            nv = rt.download(dnv + row, N_KVH * HD * 4, np.float32)
            idx = sel[0, s_].ravel()

            def one():
                orc.lib.orc_kv_append(hk.ctypes.data, hv.ctypes.data, nk.ctypes.data,
                                      nv.ctypes.data, N_KVH * HD, BPT, 2, L - 1)
                orc.attn(q, hk, hv, 2, N_HEAD, N_KVH, HD, 1, idx=idx, width=WIDTH,
                         tok_stride=N_KVH * WIDTH, kvh_stride=WIDTH, max_kv=L, scale=1.0 / 16,
                         dbl=False, threads=1)
            per.append(_cpu_rate(one, CPU_BUDGET / len(sample)))
        t_cpu = float(np.mean(per)) * n_seq
        cpu = {"us_per_step": round(t_cpu * 1e6, 1), "gbs": round(byts / t_cpu / 1e9, 4),
               "cores": 1, "kind": "port",
               "sample": f"sequences {sample} (append + attention each, fp32 C restatement, "
                         f"1 thread); extrapolated x32 to the step"}
    for kc, vc, _ in caches:
        rt.free(kc)
        rt.free(vc)
    for p_ in (dq, dnk, dnv, dout, dsel, dd):
        rt.free(p_)
    return {"cpu_baseline": cpu,
            "what": "32 sequences (ctx log-uniform 8192-131072, seed 1236), one batched decode "
                    "step each: q8_0 append + sparse attention over 2x2051 positions",
            "us_per_step": round(t * 1e6, 2), "graph_us_per_step": _us(t_graph),
            "bytes_per_step": byts,
            "gbs": round(byts / t / 1e9, 1), "pct_of_peak": round(100 * byts / t / 1e9 / PEAK_GBS, 2),
            "steps": steps, "selection_sets": sets,
            "gathered_bytes_rotated": sets * byts,
            "gather_ceiling": {"us_per_step": round(g_us, 2),
                               "gbs": round(n_seq * GATHER_B / (g_us * 1e-6) / 1e9, 1),
                               "frac_reached": round(g_us * 1e-6 / t, 3),
                               "what": "the step's K/V rows DMA'd to LDS with no compute, one "
                                       "launch per step (the headline's probe)"},
            "note": "sets rotate so the rows gathered across sets exceed the 256 MB Infinity Cache"}


def config3(b, reps=4):
    """Config 3: chunked prefill -- a 16384-token q8_0 cache, an 8192-token
    fp32 chunk quantised and appended, then every chunk token attends its own
    list per KV head: 3 sinks + 512 recent + 1536 earlier positions."""
    rt, lib = b.rt, b.lib
    ctx0, chunk = 16384, 8192
    max_kv = ctx0 + chunk
    kc, vc = rt.alloc(max_kv * BPT), rt.alloc(max_kv * BPT)
    _fill(b, kc, ctx0, q4kv.KV_Q8, 4000)
    _fill(b, vc, ctx0, q4kv.KV_Q8, 4001)
    nk, nv = rt.alloc(chunk * N_KVH * HD * 4), rt.alloc(chunk * N_KVH * HD * 4)
    b.gen(nk, chunk * N_KVH * HD, 4002)
    b.gen(nv, chunk * N_KVH * HD, 4003)
    dq, dout = rt.alloc(chunk * QO_B), rt.alloc(chunk * QO_B)
    b.gen(dq, chunk * N_HEAD * HD, 4004)
    # lists: 3 sinks + 1536 distinct positions drawn uniformly from
    # [3, pos - 511) + the 512 most recent, per query and KV head (the rule
    # tests/synth.py:selection applies)
    rng = np.random.default_rng(1237)
    pos = ctx0 + np.arange(chunk, dtype=np.int64)
    sel = np.empty((chunk, N_KVH, WIDTH), np.int32)
    for h in range(N_KVH):
        sel[:, h, :3] = np.arange(3)
        sel[:, h, 3:1539] = uniform_rows(rng, 3, pos - 511, 1536)
        sel[:, h, 1539:] = pos[:, None] - 511 + np.arange(512)[None, :]
    dsel = rt.upload(sel)
    off = ctx0 * BPT
    n = chunk * N_KVH * HD

    def run():
        ok = lib.q4_hip_f32_to_q8(kc + off, nk, n) and lib.q4_hip_f32_to_q8(vc + off, nv, n)
        return ok and lib.q4_hip_qsa_decode_idx_kv(dq, kc, vc, None, dout, dsel, WIDTH,
                                                   N_KVH * WIDTH, WIDTH, N_HEAD, N_KVH, HD,
                                                   chunk, max_kv, 1.0 / 16, q4kv.KV_Q8)
    assert run()
    rt.sync()
    assert lib.q4kv_timer_begin(0)
    t0 = time.perf_counter()
    for _ in range(reps):
        assert run()
    rt.sync()
    wall = (time.perf_counter() - t0) / reps
    flop = chunk * N_HEAD * WIDTH * HD * 4
    cpu = None
    if CPU_BUDGET > 0:
        # the oracle (fp32 path, 1 thread): the chunk's q8_0 quantisation
        # timed whole, the attention on 32 sampled queries; the layer's time is
        # quantisation + per-query time x 8192
        orc = _oracle()
        hk, hv = rt.download(kc, max_kv * BPT), rt.download(vc, max_kv * BPT)
        xk = rt.download(nk, n * 4, np.float32)
        xv = rt.download(nv, n * 4, np.float32)
        ts = np.random.default_rng(7).choice(chunk, 32, replace=False)
        qs = [rt.download(dq + int(t) * QO_B, QO_B, np.float32).reshape(1, N_HEAD, HD) for t in ts]
        t_q = _cpu_rate(lambda: (orc.quant_q8(xk), orc.quant_q8(xv)), CPU_BUDGET / 3)
        k = [0]

        def one():
            i = k[0] % len(ts)
            k[0] += 1
            orc.attn(qs[i], hk, hv, 2, N_HEAD, N_KVH, HD, 1, idx=sel[ts[i]].ravel(), width=WIDTH,
                     tok_stride=N_KVH * WIDTH, kvh_stride=WIDTH, max_kv=max_kv, scale=1.0 / 16,
                     dbl=False, threads=1)
        t_a = _cpu_rate(one, 2 * CPU_BUDGET / 3)
        t_cpu = t_q + t_a * chunk
        cpu = {"us_per_layer": round(t_cpu * 1e6, 1), "tflops": round(flop / t_cpu / 1e12, 5),
               "cores": 1, "kind": "port",
               "sample": "q8_0 quantisation of the whole chunk + attention of 32 sampled "
                         "queries (fp32 C restatement, 1 thread), extrapolated to 8192 queries"}
    for p_ in (kc, vc, nk, nv, dq, dout, dsel):
        rt.free(p_)
    return {"cpu_baseline": cpu,
            "what": "8192-token q8_0 chunk appended to a 16384-token cache, then 8192 "
                    "queries x 16 heads over per-KV-head lists of 2051 (3 sinks + 512 recent "
                    "+ 1536 distinct uniform earlier positions)",
            "us_per_layer": round(wall * 1e6, 1), "gflop": round(flop / 1e9, 1),
            "tflops": round(flop / wall / 1e12, 2),
            "pct_of_fp16_mfma_peak": round(100 * flop / wall / 2.5e15, 2), "reps": reps}


def config4(b, steps=100, sets=16, layers=12):
    """Config 4: config 1's decode step on f16 and f32 caches, and the
    restore of a 100000-token x 12-layer q8_0 session image from pinned host
    memory."""
    rt, lib = b.rt, b.lib
    # the descriptors address the Bench's per-(set, layer) rows and outputs
    layers, sets = min(layers, b.L), min(sets, b.R)
    out = {}
    for kind, name in ((q4kv.KV_F16, "f16"), (q4kv.KV_F32, "f32")):
        bpt = q4kv.token_bytes(kind, N_KVH, HD)
        kcs = [rt.alloc(CTX * bpt) for _ in range(layers)]
        vcs = [rt.alloc(CTX * bpt) for _ in range(layers)]
        for li in range(layers):
            _fill(b, kcs[li], CTX, kind, 5000 + 2 * li)
            _fill(b, vcs[li], CTX, kind, 5001 + 2 * li)
        steps_d = (q4kv.StepDesc * (sets * layers))()
        for r in range(sets):
            for li in range(layers):
                i = r * layers + li
                seq = q4kv.SeqDesc(kcs[li], vcs[li], b.q_ptr(r, li), None,
                                   b.d_out + li * QO_B, b.sel_ptr(r, li), WIDTH, WIDTH, CTX, 0)
                steps_d[i] = q4kv.StepDesc(seq, b.row_ptr(b.d_nk, r, li),
                                           b.row_ptr(b.d_nv, r, li), b.pos[r])
        dd = rt.alloc(C.sizeof(steps_d))
        assert lib.q4_hip_h2d(dd, C.addressof(steps_d), C.sizeof(steps_d))
        sz = C.sizeof(q4kv.StepDesc)
        t, t_graph = _time_both(b, lambda r: lib.q4_hip_qsa_step_batch(
            dd + r * layers * sz, layers, N_HEAD, N_KVH, HD, 1.0 / 16, kind, WIDTH), sets, steps)
        byts = 2 * N_KVH * WIDTH * (bpt // N_KVH) + IDX_B + 2 * QO_B + 2 * N_KVH * HD * 4 + 2 * bpt
        out[name] = {"us_per_layer": _us(t, layers), "graph_us_per_layer": _us(t_graph, layers),
                     "bytes_per_layer": byts,
                     "gbs": round(byts * layers / t / 1e9, 1), "layers_per_step": layers,
                     "selection_sets": sets, "gathered_bytes_rotated": sets * layers * byts}
        if CPU_BUDGET > 0:
            # the oracle's fp32 path, 1 thread: one layer's append + attention
            # over that width's cache (layer 0, set 0)
            orc = _oracle()
            hk, hv = rt.download(kcs[0], CTX * bpt), rt.download(vcs[0], CTX * bpt)
            q = rt.download(b.q_ptr(0, 0), QO_B, np.float32).reshape(1, N_HEAD, HD)
            nk = rt.download(b.row_ptr(b.d_nk, 0, 0), N_KVH * HD * 4, np.float32)
            nv = rt.download(b.row_ptr(b.d_nv, 0, 0), N_KVH * HD * 4, np.float32)
            idx = b.sel_host[0, 0].ravel()

            def one():
                orc.lib.orc_kv_append(hk.ctypes.data, hv.ctypes.data, nk.ctypes.data,
                                      nv.ctypes.data, N_KVH * HD, bpt, kind, b.pos[0])
                orc.attn(q, hk, hv, kind, N_HEAD, N_KVH, HD, 1, idx=idx, width=WIDTH,
                         tok_stride=N_KVH * WIDTH, kvh_stride=WIDTH, max_kv=CTX,
                         scale=1.0 / 16, dbl=False, threads=1)
            t_cpu = _cpu_rate(one, CPU_BUDGET / 2)
            del hk, hv
            out[name]["cpu_baseline"] = {
                "us_per_layer": round(t_cpu * 1e6, 1), "gbs": round(byts / t_cpu / 1e9, 4),
                "cores": 1, "kind": "port",
                "sample": "one layer's append + attention (fp32 C restatement, 1 thread)"}
        for p_ in kcs + vcs + [dd]:
            rt.free(p_)
    # session restore: 12 layers x 100000 tokens of q8_0 K and V from pinned memory
    c = q4kv.KvCache()
    n_img = 100000
    assert lib.q4kv_cache_open(C.byref(c), q4kv.KV_Q8, 12, N_KVH, HD, n_img)
    nb = lib.q4kv_image_bytes(C.byref(c), n_img)
    host = lib.q4_hip_host_alloc(nb)
    assert host
    C.memset(host, 0x5A, nb)
    assert lib.q4kv_image_restore(C.byref(c), host, n_img, True)
    t0 = time.perf_counter()
    reps = 3
    for _ in range(reps):
        assert lib.q4kv_image_restore(C.byref(c), host, n_img, True)
    t = (time.perf_counter() - t0) / reps
    lib.q4_hip_host_free(host)
    out["restore"] = {"what": "12 layers x 100000 tokens q8_0 K+V image, pinned host -> "
                              "device cache layout (host link bound)",
                      "bytes": nb, "ms": round(t * 1e3, 2), "gbs": round(nb / t / 1e9, 2)}
    # the same image through a file (page cache), streamed through the pipe
    path = os.path.join(os.environ.get("TMPDIR", "/tmp"), f"q4kv_bench_{os.getpid()}.img")
    try:
        c.n_kv = n_img
        t0 = time.perf_counter()
        ok = lib.q4kv_image_save_file(C.byref(c), path.encode())
        t_save = time.perf_counter() - t0
        t0 = time.perf_counter()
        n_back = lib.q4kv_image_restore_file(C.byref(c), path.encode())
        t_file = time.perf_counter() - t0
        if ok and n_back == n_img:
            out["file_save"] = {"what": "device cache -> image file (D2H overlapped with the "
                                        "writes, 32 MiB pinned chunks)", "bytes": nb,
                                "ms": round(t_save * 1e3, 2), "gbs": round(nb / t_save / 1e9, 2)}
            out["file_restore"] = {"what": "image file (page cache) -> device cache (reads "
                                           "overlapped with the DMA)", "bytes": nb,
                                   "ms": round(t_file * 1e3, 2),
                                   "gbs": round(nb / t_file / 1e9, 2)}
    finally:
        if os.path.exists(path):
            os.remove(path)
    lib.q4kv_cache_close(C.byref(c))
    return out



def config_prep(b, steps=200, sets=4, rot=64, base=1.0e7, eps=1.0e-6):
    """Config 1's 12-layer decode step with the query/key preparation
    (RMSNorm + RoPE of 16 query heads with their gates and of the 2 new key
    rows) fused into the step kernel (q4_hip_qsa_step_prep_batch), against
    the same step done as q_prep + k_prep per layer then the batched step."""
    rt, lib = b.rt, b.lib
    assert b.R >= sets, "config_prep needs a Bench of >= 4 sets"
    L = b.L
    qg = rt.alloc(sets * L * N_HEAD * 2 * HD * 4)
    b.gen(qg, sets * L * N_HEAD * 2 * HD, 91)
    wq, wk = rt.alloc(HD * 4), rt.alloc(HD * 4)
    b.gen(wq, HD, 92)
    b.gen(wk, HD, 93)
    gbuf = rt.alloc(L * N_HEAD * HD * 4)
    qtmp = rt.alloc(L * N_HEAD * HD * 4)
    ktmp = rt.alloc(sets * L * N_KVH * HD * 4)
    preps = (q4kv.PrepStepDesc * (sets * L))()
    steps_d = (q4kv.StepDesc * (sets * L))()
    for r in range(sets):
        for li in range(L):
            i = r * L + li
            qgp = qg + i * N_HEAD * 2 * HD * 4
            out = b.d_out + li * QO_B
            seq = q4kv.SeqDesc(b.kc[li], b.vc[li], qgp, gbuf + li * QO_B, out,
                               b.sel_ptr(r, li), WIDTH, WIDTH, CTX, 0)
            preps[i] = q4kv.PrepStepDesc(q4kv.StepDesc(seq, b.row_ptr(b.d_nk, r, li),
                                                       b.row_ptr(b.d_nv, r, li), b.pos[r]),
                                         wq, wk)
            seq2 = q4kv.SeqDesc(b.kc[li], b.vc[li], qtmp + li * QO_B, gbuf + li * QO_B, out,
                                b.sel_ptr(r, li), WIDTH, WIDTH, CTX, 0)
            steps_d[i] = q4kv.StepDesc(seq2, ktmp + i * N_KVH * HD * 4,
                                       b.row_ptr(b.d_nv, r, li), b.pos[r])
    dp, ds = rt.alloc(C.sizeof(preps)), rt.alloc(C.sizeof(steps_d))
    assert lib.q4_hip_h2d(dp, C.addressof(preps), C.sizeof(preps))
    assert lib.q4_hip_h2d(ds, C.addressof(steps_d), C.sizeof(steps_d))
    psz, ssz = C.sizeof(q4kv.PrepStepDesc), C.sizeof(q4kv.StepDesc)

    def fused(r):
        return lib.q4_hip_qsa_step_prep_batch(dp + r * L * psz, L, N_HEAD, N_KVH, HD, 1.0 / 16,
                                              q4kv.KV_Q8, WIDTH, rot, base, eps)

    def separate(r):
        ok = True
        for li in range(L):
            i = r * L + li
            ok &= lib.q4_hip_qsa_q_prep(qg + i * N_HEAD * 2 * HD * 4, wq, qtmp + li * QO_B,
                                        gbuf + li * QO_B, N_HEAD, HD, rot, b.pos[r], base, eps)
            ok &= lib.q4_hip_copy(ktmp + i * N_KVH * HD * 4, b.row_ptr(b.d_nk, r, li),
                                  N_KVH * HD)
            ok &= lib.q4_hip_qsa_k_prep(ktmp + i * N_KVH * HD * 4, wk, N_KVH, HD, rot,
                                        b.pos[r], base, eps)
        return ok and lib.q4_hip_qsa_step_batch(ds + r * L * ssz, L, N_HEAD, N_KVH, HD,
                                                 1.0 / 16, q4kv.KV_Q8, WIDTH)

    out = {"what": f"{L}-layer decode step with Q/K RMSNorm + RoPE (n_rot {rot}) of 16 query "
                   "heads (+ gates) and the 2 new key rows",
           "launches": {"fused": 2, "separate": 3 * L + 2}}
    for name, fn in (("fused", fused), ("separate", separate)):
        t = _time_steps(b, fn, sets, steps) / L
        out[f"{name}_us_per_layer"] = round(t * 1e6, 3)
    for p_ in (qg, wq, wk, gbuf, qtmp, ktmp, dp, ds):
        rt.free(p_)
    return out


def config_out(b, steps=100, sets=4, n_embd=4096):
    """Config 1's 12-layer decode step followed by each layer's q8_0
    attention output projection (W_o [n_embd][16 x 256], synthetic weights):
    the merge epilogue fused with the GEMV (q4_hip_qsa_step_out_batch)
    against the batched step then one q4_hip_gemv_dd per layer."""
    rt, lib = b.rt, b.lib
    L = b.L
    ncols = N_HEAD * HD
    wbytes = n_embd * ncols // 32 * 34
    tmp = rt.alloc(n_embd * ncols * 4)
    ws = []
    for li in range(L):
        wq = rt.alloc(wbytes)
        b.gen(tmp, n_embd * ncols, 300 + li)
        assert lib.q4_hip_f32_to_q8(wq, tmp, n_embd * ncols)
        ws.append(wq)
    rt.sync()
    rt.free(tmp)
    ys = rt.alloc(L * n_embd * 4)
    outs = (q4kv.OutDesc * L)()
    for li in range(L):
        outs[li] = q4kv.OutDesc(ws[li], ys + li * n_embd * 4)
    dd = rt.alloc(C.sizeof(outs))
    assert lib.q4_hip_h2d(dd, C.addressof(outs), C.sizeof(outs))
    ssz = C.sizeof(q4kv.StepDesc)

    def fused(r):
        return lib.q4_hip_qsa_step_out_batch(b.d_step + r * L * ssz, dd, L, N_HEAD, N_KVH, HD,
                                             1.0 / 16, q4kv.KV_Q8, WIDTH, n_embd, 1.0)

    def separate(r):
        ok = b._enqueue_batched(r)
        for li in range(L):
            ok &= lib.q4_hip_gemv_dd(8, ws[li], n_embd, ncols, b.d_out + li * QO_B,
                                     ys + li * n_embd * 4, 1.0)
        return ok

    out = {"what": f"{L}-layer decode step + attn_output projection per layer (q8_0 "
                   f"[{n_embd}][{ncols}], {wbytes} B per layer)",
           "launches": {"fused": 2, "separate": 2 + L}}
    for name, fn in (("fused", fused), ("separate", separate)):
        t = _time_steps(b, fn, min(sets, b.R), steps) / L
        out[f"{name}_us_per_layer"] = round(t * 1e6, 3)
    # the GEMV alone: one launch per layer, W streamed from HBM (12 x 17.8 MB)
    t = _time_steps(b, lambda r: all(lib.q4_hip_gemv_dd(8, ws[li], n_embd, ncols,
                                                        b.d_out + li * QO_B,
                                                        ys + li * n_embd * 4, 1.0)
                                     for li in range(L)), 1, steps) / L
    out["gemv_us_per_layer"] = round(t * 1e6, 3)
    out["gemv_gbs"] = round((wbytes + ncols * 4 + n_embd * 4) / t / 1e9, 1)
    for p_ in ws + [ys, dd]:
        rt.free(p_)
    return out


def config_gqa12(b, steps=200, n_head=24):
    """The reference's production head layout (24 query heads over 2 KV heads,
    12 per KV head, the model the reference ships for) on config 1's 12-layer
    decode step:
    q8_0 append + sparse attention over the same caches and selections,
    through q4_hip_qsa_step_batch (one fused launch + the merge)."""
    rt, lib = b.rt, b.lib
    L, R = b.L, b.R
    qb = n_head * HD * 4
    dq = rt.alloc(R * L * qb)
    b.gen(dq, R * L * n_head * HD, 95)
    dout = rt.alloc(L * qb)
    steps_d = (q4kv.StepDesc * (R * L))()
    for r in range(R):
        for li in range(L):
            i = r * L + li
            seq = q4kv.SeqDesc(b.kc[li], b.vc[li], dq + i * qb, None, dout + li * qb,
                               b.sel_ptr(r, li), WIDTH, WIDTH, CTX, 0)
            steps_d[i] = q4kv.StepDesc(seq, b.row_ptr(b.d_nk, r, li), b.row_ptr(b.d_nv, r, li),
                                       b.pos[r])
    dd = rt.alloc(C.sizeof(steps_d))
    assert lib.q4_hip_h2d(dd, C.addressof(steps_d), C.sizeof(steps_d))
    sz = C.sizeof(q4kv.StepDesc)
    t, t_graph = _time_both(b, lambda r: lib.q4_hip_qsa_step_batch(
        dd + r * L * sz, L, n_head, N_KVH, HD, 1.0 / 16, q4kv.KV_Q8, WIDTH), R, steps)
    byts = GATHER_B + IDX_B + 2 * qb + APPEND_B
    for p_ in (dq, dout, dd):
        rt.free(p_)
    return {"what": f"{L}-layer decode step, {n_head} query heads / {N_KVH} KV heads "
                    f"(gqa {n_head // N_KVH}), same caches and selections as the headline",
            "us_per_layer": _us(t, L), "graph_us_per_layer": _us(t_graph, L),
            "bytes_per_layer": byts, "gbs": round(byts * L / t / 1e9, 1),
            "selection_sets": R}


def config0(b, steps=300, ctx=4096):
    """Config 0: one layer, batch 1, a 4096-token q8_0 cache, 16 Q / 2 KV
    heads: append the new token (q4_hip_kv_append_d, at position 4096), then
    dense decode attention over all 4097 positions (q4_hip_qsa_decode), with
    a gate. The call pair is timed per step; the oracle's fp32 path beside
    it."""
    rt, lib = b.rt, b.lib
    max_kv = ctx + 1
    kc, vc = rt.alloc(max_kv * BPT), rt.alloc(max_kv * BPT)
    _fill(b, kc, ctx, q4kv.KV_Q8, 6000)
    _fill(b, vc, ctx, q4kv.KV_Q8, 6001)
    nk, nv = rt.alloc(N_KVH * HD * 4), rt.alloc(N_KVH * HD * 4)
    dq, dg, dout = rt.alloc(QO_B), rt.alloc(QO_B), rt.alloc(QO_B)
    b.gen(nk, N_KVH * HD, 6002)
    b.gen(nv, N_KVH * HD, 6003)
    b.gen(dq, N_HEAD * HD, 6004)
    b.gen(dg, N_HEAD * HD, 6005)
    lib.q4_hip_pos_push(ctx)

    def enqueue(_r):
        return (lib.q4_hip_kv_append_d(kc, vc, nk, nv, N_KVH * HD, BPT, q4kv.KV_Q8) and
                lib.q4_hip_qsa_decode(dq, kc, vc, dg, dout, N_HEAD, N_KVH, HD, max_kv, max_kv,
                                      1.0 / 16, q4kv.KV_Q8))
    t, t_graph = _time_both(b, enqueue, 1, steps)
    byts = 2 * max_kv * BPT + 2 * QO_B + QO_B + APPEND_B  # K, V rows, q, gate, out, append
    res = {"what": "one layer: q8_0 append at position 4096, then dense decode attention of "
                   "16 heads over 4097 positions (4096-token cache, gated), per call pair",
           "us_per_step": _us(t), "graph_us_per_step": _us(t_graph), "bytes_per_step": byts,
           "gbs": round(byts / t / 1e9, 1)}
    if CPU_BUDGET > 0:
        orc = _oracle()
        rt.sync()
        hk, hv = rt.download(kc, max_kv * BPT), rt.download(vc, max_kv * BPT)
        q = rt.download(dq, QO_B, np.float32).reshape(1, N_HEAD, HD)
        g = rt.download(dg, QO_B, np.float32).reshape(1, N_HEAD, HD)
        xk = rt.download(nk, N_KVH * HD * 4, np.float32)
        xv = rt.download(nv, N_KVH * HD * 4, np.float32)

        def one():
            orc.lib.orc_kv_append(hk.ctypes.data, hv.ctypes.data, xk.ctypes.data,
                                  xv.ctypes.data, N_KVH * HD, BPT, 2, ctx)
            orc.attn(q, hk, hv, 2, N_HEAD, N_KVH, HD, 1, gate=g, kv_base=ctx, max_kv=max_kv,
                     scale=1.0 / 16, dbl=False, threads=1)
        t_cpu = _cpu_rate(one, CPU_BUDGET)
        res["cpu_baseline"] = {"us_per_step": round(t_cpu * 1e6, 1),
                               "gbs": round(byts / t_cpu / 1e9, 4), "cores": 1, "kind": "port",
                               "sample": "the whole call pair (fp32 C restatement, 1 thread)"}
    for p_ in (kc, vc, nk, nv, dq, dg, dout):
        rt.free(p_)
    return res


def config_ref24(b, steps=200, n_head=24):
    """The reference's one published kernel figure, like for like: its
    production head layout (24 query / 2 KV heads) through its own per-layer
    calls, q4_hip_kv_append_d then q4_hip_qsa_decode_idx (one shared 2051-entry
    list, gated), on config 1's 12 layers of 262144-token q8_0 caches,
    enqueued directly one layer after the other (and replayed from a
    captured graph per step). The reference quotes 82 us per decode_idx call
    on an RX 7900 XTX (its DESIGN.md:130-133)."""
    rt, lib = b.rt, b.lib
    L, R = b.L, b.R
    qb = n_head * HD * 4
    dq, dg = rt.alloc(R * L * qb), rt.alloc(R * L * qb)
    b.gen(dq, R * L * n_head * HD, 96)
    b.gen(dg, R * L * n_head * HD, 97)
    dout = rt.alloc(L * qb)

    def enqueue(r):
        ok = True
        for li in range(L):
            i = r * L + li
            ok = ok and lib.q4_hip_kv_append_d(b.kc[li], b.vc[li], b.row_ptr(b.d_nk, r, li),
                                               b.row_ptr(b.d_nv, r, li), N_KVH * HD, BPT,
                                               q4kv.KV_Q8)
            # the shared list: KV head 0's selection of this (set, layer)
            ok = ok and lib.q4_hip_qsa_decode_idx(dq + i * qb, b.kc[li], b.vc[li], dg + i * qb,
                                                  dout + li * qb, b.sel_ptr(r, li), WIDTH,
                                                  n_head, N_KVH, HD, 1, CTX, 1.0 / 16,
                                                  q4kv.KV_Q8)
        return ok

    def step(r):
        lib.q4_hip_pos_push(b.pos[r])
        return enqueue(r)
    t = _time_direct(b, step, R, steps)
    t_graph = None
    if USE_GRAPHS:
        graphs = _graphs(lib, enqueue, R)
        for i in range(max(8, R)):
            lib.q4_hip_pos_push(b.pos[i % R])
            assert lib.q4_hip_graph_launch(graphs[i % R])
        b.rt.sync()
        t0 = time.perf_counter()
        for i in range(steps):
            lib.q4_hip_pos_push(b.pos[i % R])
            assert lib.q4_hip_graph_launch(graphs[i % R])
        b.rt.sync()
        t_graph = (time.perf_counter() - t0) / steps
        for g in graphs:
            lib.q4_hip_graph_free(g)
    for p_ in (dq, dg, dout):
        rt.free(p_)
    return {"what": f"per layer q4_hip_kv_append_d + q4_hip_qsa_decode_idx (shared list, "
                    f"gated), {n_head} Q / {N_KVH} KV heads, {L} layers one after the other",
            "us_per_layer": _us(t, L), "graph_us_per_layer": _us(t_graph, L),
            "reference_us_per_call": 82.0,
            "reference_source": "reference DESIGN.md:130-133, RX 7900 XTX, decode_idx alone"}


IDX_RATIO, IDX_KBLK, IDX_HEADS, IDX_DIM = 4, 512, 4, 128
IDX_ROT, IDX_BASE, IDX_EPS = 64, 1.0e7, 1.0e-6


def config_indexer(b, steps=100, layers=12):
    """QSA indexer of the decode step at a full 262144-token context
    (src/q4_fwd.c:895-925): per layer the raw indexer key store, the pooling
    of the block it completes, the indexer query's RMSNorm + RoPE, the scores
    of all 65536 visible blocks and the exact top-512 selection expanded to
    2051 positions. One graph per step covers `layers` layers, each with its
    own 64 MiB fp16 key buffer and 32 MiB pool, so the pools (403 MB) stream
    from HBM. Also times the prefill pool rebuild of one layer."""
    rt, lib = b.rt, b.lib
    max_blocks = CTX // IDX_RATIO
    # a position whose visible blocks (65386) do not fill the top-k's 65536-key
    # load exactly, as almost every decode position
    pos = CTX - 601
    raws, pools, scs, sels, qs, ks = [], [], [], [], [], []
    tmp = rt.alloc(CTX * IDX_DIM * 4)
    wn = rt.alloc(IDX_DIM * 4)
    b.gen(wn, IDX_DIM, 77)
    for li in range(layers):
        raw = rt.alloc(CTX * IDX_DIM * 2)
        b.gen(tmp, CTX * IDX_DIM, 9000 + li)
        assert lib.q4_hip_f32_to_f16(raw, tmp, CTX * IDX_DIM)
        raws.append(raw)
        pools.append(rt.alloc(max_blocks * IDX_DIM * 4))
        scs.append(rt.alloc(max_blocks * 4))
        sels.append(rt.alloc(WIDTH * 4))
        q = rt.alloc(IDX_HEADS * IDX_DIM * 4)
        b.gen(q, IDX_HEADS * IDX_DIM, 9100 + li)
        qs.append(q)
        k = rt.alloc(IDX_DIM * 4)
        b.gen(k, IDX_DIM, 9200 + li)
        ks.append(k)
    rt.sync()
    rt.free(tmp)
    # prefill-style rebuild of every complete block (timed on one layer)
    for li in range(layers):
        assert lib.q4_hip_qsa_pool(raws[li], pools[li], wn, IDX_DIM, IDX_RATIO, 0, max_blocks,
                                   IDX_ROT, IDX_BASE, IDX_EPS)
    rt.sync()
    t0 = time.perf_counter()
    reps = 10
    for _ in range(reps):
        assert lib.q4_hip_qsa_pool(raws[0], pools[0], wn, IDX_DIM, IDX_RATIO, 0, max_blocks,
                                   IDX_ROT, IDX_BASE, IDX_EPS)
    rt.sync()
    t_pool = (time.perf_counter() - t0) / reps
    lib.q4_hip_pos_push(pos)
    rt.sync()

    def step(parts):
        ok = True
        for li in range(layers):
            if "store" in parts:
                ok &= lib.q4_hip_f32_to_f16_d(raws[li], IDX_DIM, ks[li], IDX_DIM)
                ok &= lib.q4_hip_qsa_pool_d(raws[li], pools[li], wn, IDX_DIM, IDX_RATIO,
                                            IDX_ROT, IDX_BASE, IDX_EPS)
            if "prep" in parts:
                ok &= lib.q4_hip_qsa_k_prep_d(qs[li], wn, IDX_HEADS, IDX_DIM, IDX_ROT,
                                              IDX_BASE, IDX_EPS)
            if "fused" in parts:
                ok &= lib.q4_hip_qsa_index_score_d(raws[li], pools[li], wn, ks[li], qs[li], wn,
                                                   scs[li], max_blocks, IDX_HEADS, IDX_DIM,
                                                   IDX_RATIO, IDX_ROT, IDX_BASE, IDX_EPS)
            if "score" in parts:
                ok &= lib.q4_hip_qsa_score_d(qs[li], pools[li], scs[li], max_blocks, IDX_HEADS,
                                             IDX_DIM, IDX_RATIO)
            if "topk" in parts:
                ok &= lib.q4_hip_qsa_topk_d(scs[li], sels[li], max_blocks, IDX_KBLK, IDX_RATIO,
                                            WIDTH)
        return ok

    descs = (q4kv.IndexDesc * layers)()
    for li in range(layers):
        descs[li] = q4kv.IndexDesc(raws[li], pools[li], wn, ks[li], qs[li], wn, scs[li],
                                   sels[li], pos)
    dd = rt.alloc(C.sizeof(descs))
    assert lib.q4_hip_h2d(dd, C.addressof(descs), C.sizeof(descs))

    def batched(r):
        return lib.q4_hip_qsa_index_batch(dd, layers, max_blocks, IDX_HEADS, IDX_DIM, IDX_RATIO,
                                          IDX_ROT, IDX_BASE, IDX_EPS, IDX_KBLK, WIDTH)

    out = {"what": f"decode indexer, {layers} layers x 65536 visible blocks (ctx {CTX}), "
                   "4 heads x 128 dims, top-512 of 4-position blocks -> 2051 positions",
           "launches_per_layer": {"full": 5, "fused": 2, "batched": 2.0 / layers}}
    out["batched_us_per_layer"] = round(_time_steps(b, batched, 2, steps) / layers * 1e6, 3)
    for name, parts in (("full", ("store", "prep", "score", "topk")), ("score", ("score",)),
                        ("topk", ("topk",)), ("fused", ("fused", "topk"))):
        t = _time_steps(b, lambda r, parts=parts: step(parts), 2, steps) / layers
        out[f"{name}_us_per_layer"] = round(t * 1e6, 3)
    score_b = max_blocks * (IDX_DIM * 4 + 4) + IDX_HEADS * IDX_DIM * 4
    out["score_bytes_per_layer"] = score_b
    out["score_gbs"] = round(score_b / (out["score_us_per_layer"] * 1e-6) / 1e9, 1)
    out["score_pct_of_peak"] = round(100 * out["score_gbs"] / PEAK_GBS, 2)
    out["pool_rebuild_ms"] = round(t_pool * 1e3, 3)
    pool_b = CTX * IDX_DIM * 2 + max_blocks * IDX_DIM * 4
    out["pool_rebuild_gbs"] = round(pool_b / t_pool / 1e9, 1)
    for p_ in raws + pools + scs + sels + qs + ks + [wn, dd]:
        rt.free(p_)
    return out


def config_layer(b, steps=100):
    """One decode token's whole QSA KV path per layer, in the reference's call
    order (src/q4_fwd.c:891-922): q4_hip_kv_append_d of the new K/V rows, the
    indexer (the raw key store, the pooling of the block it completes, the
    indexer query's RMSNorm + RoPE, scores of the 65536 visible blocks, the
    top-512 selection expanded to 2051 positions), then
    q4_hip_qsa_decode_idx over that shared list (16 query / 2 KV heads,
    gated) on config 1's 262144-token q8_0 caches; the layers one after the
    other. "separate": the reference's five indexer calls; "fused": the
    indexer's store, pool, prep and scores in one q4_hip_qsa_index_score_d.
    The held append rides in the indexer's first launch either way."""
    rt, lib = b.rt, b.lib
    L, R = b.L, b.R
    max_blocks = CTX // IDX_RATIO
    raws, pools, scs, sels, qs, ks = [], [], [], [], [], []
    tmp = rt.alloc(CTX * IDX_DIM * 4)
    wn = rt.alloc(IDX_DIM * 4)
    b.gen(wn, IDX_DIM, 78)
    for li in range(L):
        raw = rt.alloc(CTX * IDX_DIM * 2)
        b.gen(tmp, CTX * IDX_DIM, 9400 + li)
        assert lib.q4_hip_f32_to_f16(raw, tmp, CTX * IDX_DIM)
        raws.append(raw)
        pools.append(rt.alloc(max_blocks * IDX_DIM * 4))
        assert lib.q4_hip_qsa_pool(raw, pools[-1], wn, IDX_DIM, IDX_RATIO, 0, max_blocks,
                                   IDX_ROT, IDX_BASE, IDX_EPS)
        scs.append(rt.alloc(max_blocks * 4))
        sels.append(rt.alloc(WIDTH * 4))
        q = rt.alloc(R * IDX_HEADS * IDX_DIM * 4)
        b.gen(q, R * IDX_HEADS * IDX_DIM, 9500 + li)
        qs.append(q)
        k = rt.alloc(R * IDX_DIM * 4)
        b.gen(k, R * IDX_DIM, 9600 + li)
        ks.append(k)
    rt.sync()
    rt.free(tmp)
    dg = rt.alloc(R * L * QO_B)
    b.gen(dg, R * L * N_HEAD * HD, 98)
    qsz, ksz = IDX_HEADS * IDX_DIM * 4, IDX_DIM * 4

    def enqueue(r, fused):
        ok = True
        for li in range(L):
            ok = ok and lib.q4_hip_kv_append_d(b.kc[li], b.vc[li], b.row_ptr(b.d_nk, r, li),
                                               b.row_ptr(b.d_nv, r, li), N_KVH * HD, BPT,
                                               q4kv.KV_Q8)
            iq, ik = qs[li] + r * qsz, ks[li] + r * ksz
            if fused:
                ok = ok and lib.q4_hip_qsa_index_score_d(raws[li], pools[li], wn, ik, iq, wn,
                                                         scs[li], max_blocks, IDX_HEADS,
                                                         IDX_DIM, IDX_RATIO, IDX_ROT, IDX_BASE,
                                                         IDX_EPS)
            else:
                ok = ok and lib.q4_hip_f32_to_f16_d(raws[li], IDX_DIM, ik, IDX_DIM)
                ok = ok and lib.q4_hip_qsa_pool_d(raws[li], pools[li], wn, IDX_DIM, IDX_RATIO,
                                                  IDX_ROT, IDX_BASE, IDX_EPS)
                ok = ok and lib.q4_hip_qsa_k_prep_d(iq, wn, IDX_HEADS, IDX_DIM, IDX_ROT,
                                                    IDX_BASE, IDX_EPS)
                ok = ok and lib.q4_hip_qsa_score_d(iq, pools[li], scs[li], max_blocks,
                                                   IDX_HEADS, IDX_DIM, IDX_RATIO)
            ok = ok and lib.q4_hip_qsa_topk_d(scs[li], sels[li], max_blocks, IDX_KBLK,
                                              IDX_RATIO, WIDTH)
            ok = ok and lib.q4_hip_qsa_decode_idx(b.q_ptr(r, li), b.kc[li], b.vc[li],
                                                  dg + (r * L + li) * QO_B,
                                                  b.d_out + li * QO_B, sels[li], WIDTH, N_HEAD,
                                                  N_KVH, HD, 1, CTX, 1.0 / 16, q4kv.KV_Q8)
        return ok

    out = {"what": f"per layer: q4_hip_kv_append_d, the indexer (65536 visible blocks, "
                   f"top-512 -> 2051 positions), q4_hip_qsa_decode_idx over its list (gated, "
                   f"{N_HEAD} Q / {N_KVH} KV heads, ctx {CTX}); {L} layers one after the other",
           "launches_per_layer": {"separate": 7, "fused": 4}}
    for name, fused in (("separate", False), ("fused", True)):
        def step(r, fused=fused):
            lib.q4_hip_pos_push(b.pos[r])
            return enqueue(r, fused)
        out[f"{name}_us_per_layer"] = _us(_time_direct(b, step, R, steps), L)
        if USE_GRAPHS:
            graphs = _graphs(lib, lambda r, fused=fused: enqueue(r, fused), R)
            for i in range(max(8, R)):
                lib.q4_hip_pos_push(b.pos[i % R])
                assert lib.q4_hip_graph_launch(graphs[i % R])
            rt.sync()
            t0 = time.perf_counter()
            for i in range(steps):
                lib.q4_hip_pos_push(b.pos[i % R])
                assert lib.q4_hip_graph_launch(graphs[i % R])
            rt.sync()
            out[f"{name}_graph_us_per_layer"] = _us((time.perf_counter() - t0) / steps, L)
            for g in graphs:
                lib.q4_hip_graph_free(g)
    for p_ in raws + pools + scs + sels + qs + ks + [wn, dg]:
        rt.free(p_)
    return out


def config_indexer_prefill(b, cache=16384, chunk=8192, slice_=512, reps=3):
    """The indexer of config 3's chunked prefill (src/q4_fwd.c:740-770, sliced by 512
    tokens as src/q4_fwd.c:1744-1754): for each 512-token slice of an 8192-token
    chunk after a 16384-token cache, the indexer queries' RMSNorm + RoPE
    (q4_hip_qsa_k_prep_n), the scores of every visible block (bf16x3 split on MFMA), and the
    top-512 selection of every token expanded to 2051 positions. The pool of all
    6144 blocks is rebuilt first (q4_hip_qsa_pool), as a new chunk's keys arrive."""
    rt, lib = b.rt, b.lib
    n_pos = cache + chunk
    nb = n_pos // IDX_RATIO
    raw = rt.alloc(n_pos * IDX_DIM * 2)
    tmp = rt.alloc(max(n_pos * IDX_DIM, chunk * IDX_HEADS * IDX_DIM) * 4)
    b.gen(tmp, n_pos * IDX_DIM, 9300)
    assert lib.q4_hip_f32_to_f16(raw, tmp, n_pos * IDX_DIM)
    pool = rt.alloc(nb * IDX_DIM * 4)
    wn = rt.alloc(IDX_DIM * 4)
    b.gen(wn, IDX_DIM, 9301)
    q = rt.alloc(chunk * IDX_HEADS * IDX_DIM * 4)
    score = rt.alloc(slice_ * nb * 4)
    sel = rt.alloc(slice_ * WIDTH * 4)
    rt.sync()

    def run():
        # the chunk's raw indexer queries, as their projection would leave them
        # (one copy: q4_hip_copy blocks until it lands, so per-slice copies
        # would time host round trips, not the indexer)
        ok = lib.q4_hip_copy(q, tmp, chunk * IDX_HEADS * IDX_DIM)
        ok &= lib.q4_hip_qsa_pool(raw, pool, wn, IDX_DIM, IDX_RATIO, 0, nb, IDX_ROT, IDX_BASE,
                                  IDX_EPS)
        for s0 in range(0, chunk, slice_):
            pos0 = cache + s0
            qs = q + s0 * IDX_HEADS * IDX_DIM * 4
            ok &= lib.q4_hip_qsa_k_prep_n(qs, wn, IDX_HEADS, IDX_DIM, IDX_ROT, pos0, IDX_BASE,
                                          IDX_EPS, slice_)
            n_blocks = (pos0 + slice_) // IDX_RATIO
            ok &= lib.q4_hip_qsa_score(qs, pool, score, slice_, n_blocks, nb, IDX_HEADS,
                                       IDX_DIM, pos0, IDX_RATIO)
            ok &= lib.q4_hip_qsa_topk(score, sel, slice_, n_blocks, nb, IDX_KBLK, IDX_RATIO,
                                      pos0, WIDTH)
        return ok

    b.gen(tmp, chunk * IDX_HEADS * IDX_DIM, 9302)
    assert run()
    rt.sync()
    t0 = time.perf_counter()
    for _ in range(reps):
        assert run()
    rt.sync()
    t = (time.perf_counter() - t0) / reps
    flop = sum(2.0 * slice_ * IDX_HEADS * IDX_DIM * ((cache + s0 + slice_) // IDX_RATIO)
               for s0 in range(0, chunk, slice_))
    for p_ in (raw, tmp, pool, wn, q, score, sel):
        rt.free(p_)
    return {"what": f"indexer of an {chunk}-token prefill chunk after a {cache}-token cache, "
                    f"{slice_}-token slices: pool rebuild ({nb} blocks), query prep, scores "
                    "(bf16x3 split on MFMA), top-512 + expansion per token",
            "us_per_layer": round(t * 1e6, 1), "us_per_token": round(t * 1e6 / chunk, 3),
            "score_gflop": round(flop / 1e9, 1)}


ONLY = {"config0": config0, "ref24": config_ref24, "config2": config2, "config3": config3, "config4": config4, "prep": config_prep,
        "gqa12": config_gqa12,
        "out": config_out, "indexer": config_indexer,
        "indexer_prefill": config_indexer_prefill, "layer": config_layer}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--layers", type=int, default=12)
    ap.add_argument("--sets", type=int, default=16)
    ap.add_argument("--mode", choices=["batched", "sequential", "both"], default="both")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--graphs", type=int, default=1,
                    help="also time graph-replayed variants (0: direct launches only, as in "
                         "profiling runs)")
    ap.add_argument("--configs", type=int, default=1,
                    help="also measure configs 2, 3 and 4 (0 to skip)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a device-to-device copy of MIB MiB (PMC calibration)")
    ap.add_argument("--only", choices=sorted(ONLY), default=None,
                    help="only measure one of the extra configurations and print its JSON "
                         "(for profiling)")
    args = ap.parse_args()
    global USE_GRAPHS, CPU_BUDGET
    USE_GRAPHS = bool(args.graphs)
    if args.cpu_seconds <= 0:
        CPU_BUDGET = 0.0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the QSA KV path runs on a single MI355X "
              "(no collectives); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        rt = q4kv.Runtime()
        n = args.copy_calibration << 20
        src, dst = rt.alloc(n), rt.alloc(n)
        for _ in range(3):
            assert rt.lib.q4_hip_copy(dst, src, n // 4)
        rt.sync()
        print(json.dumps({"copy_bytes": n, "launches": 3}))
        return
    if args.only:
        b = Bench(args.layers, max(args.sets, 4))
        print(json.dumps({args.only: ONLY[args.only](b)}), flush=True)
        return
    b = Bench(args.layers, args.sets)
    res = {}
    kern_ms = None
    if args.mode in ("batched", "both"):
        res["batched"] = b.timed(b.step_batched, args.steps, args.warmup)
        if USE_GRAPHS:
            res["batched_graph"] = b.timed(b.step_batched_graph, args.steps, args.warmup)
        # the fused step kernel's duration, from HIP events the library
        # records around each of its launches on its stream, over a second
        # pass of the same timed steps
        _, _, kern_ms = b.timed(b.step_batched, args.steps, args.warmup, prof=True)
    if args.mode in ("sequential", "both"):
        res["sequential"] = b.timed(b.step_sequential, args.steps, args.warmup)
        if USE_GRAPHS:
            res["sequential_graph"] = b.timed(b.step_sequential_graph, args.steps, args.warmup)
    g_us, g_gbs = b.gather_ceiling()
    configs = None
    if args.configs:
        configs = {"config0_dense_decode": config0(b),
                   "config2_batched_decode": config2(b), "config3_chunked_prefill": config3(b),
                   "config4_widths_restore": config4(b),
                   "production_heads_24_2": config_gqa12(b),
                   "reference_call_24q_2kv": config_ref24(b),
                   "qk_prep_fused_step": config_prep(b),
                   "out_projection_fused": config_out(b),
                   "indexer_decode": config_indexer(b),
                   "indexer_prefill": config_indexer_prefill(b),
                   "reference_layer_sequence": config_layer(b)}
    threads = min(16, len(os.sched_getaffinity(0)))
    parity, cpu = b.check_and_cpu(args.cpu_seconds, threads)
    head = "batched" if "batched" in res else "sequential"
    wall, gpu_s, _ = res[head]
    kern_s = kern_ms if head == "batched" else None
    K, L = args.steps, args.layers
    value = K * L * LAYER_B / wall / 1e9
    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": K,
        "warmup": args.warmup, "ms_per_step": round(wall / K * 1e3, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic (device-generated N(0,1), 4 outlier channels x8 per head)",
        "config": {
            "workload": (f"config1 QSA sparse decode: {L} QSA layers x (q8_0 append + sparse "
                         f"attention), {CTX}-token q8_0 cache per layer, 16 Q / 2 KV heads, "
                         f"hd 256, 2051 selected positions per KV head, one "
                         + ("q4_hip_qsa_step_batch call per step" if head == "batched" else
                            "append + decode call pair per layer") + ", enqueued directly"),
            "kv": "q8_0", "ctx": CTX, "layers_per_step": L, "selection_sets": args.sets,
            "bytes_per_layer": LAYER_B, "parallelism": "single GPU",
        },
        "us_per_layer": round(wall / (K * L) * 1e6, 4),
        "pct_of_peak": round(100 * value / PEAK_GBS, 2),
        "timing_mode": ("direct enqueue of each step's calls on the library stream; the "
                        "captured-graph replay of the same steps is the *_graph_* keys"),
    }
    for mode, (w, g, _) in res.items():
        out[f"{mode}_us_per_layer"] = round(w / (K * L) * 1e6, 4)
        out[f"{mode}_gbs"] = round(K * L * LAYER_B / w / 1e9, 2)
        out[f"{mode}_gpu_event_us_per_layer"] = round(g / (K * L) * 1e6, 4)
    if kern_s:
        ach = L * SPLIT_KERNEL_B / (kern_s / 1e3) / 1e9
        out["roofline"] = {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_GBS,
                           "unit": "GB/s", "frac": round(ach / PEAK_GBS, 4), "traffic": None,
                           "kernel": "qsa_q8d256_k<MODE_STEP>",
                           "kernel_us": round(kern_s * 1e3, 3),
                           "kernel_us_source": "HIP events around each launch over a second "
                                               "pass of the timed steps (library stream)",
                           "bytes_per_launch": L * SPLIT_KERNEL_B}
    if configs:
        out["configs"] = configs
    out["gather_ceiling"] = {
        "gbs": round(g_gbs, 1), "us_per_launch": round(g_us, 3),
        "what": "the same K/V rows of one batched step DMA'd to LDS with no compute "
                "(272-byte rows, 16-byte loads): the practical bound of this access pattern"}
    tfile = ROOT / "profiles" / "qsa_q8d256_batch12_traffic.json"
    if kern_s and tfile.exists() and L == 12:
        t = json.loads(tfile.read_text())
        out["roofline"]["traffic"] = t["hbm_bytes_per_launch"]
        out["roofline"]["traffic_source"] = str(tfile.relative_to(ROOT))
    if kern_s:
        out["roofline"]["frac_of_gather_ceiling"] = round(out["roofline"]["achieved"] / g_gbs, 4)
    out.update(parity)
    out["cpu_baseline"] = cpu
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
