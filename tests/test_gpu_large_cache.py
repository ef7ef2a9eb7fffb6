"""Caches larger than 4 GiB: every position read or written sits past byte
offset 2^32 of its cache, except the three sink positions 0-2 (q8_0: 544
bytes per token, positions from 7.95M of 8.4M; f16: 1024 bytes, from 4.2M
of 4.3M; f32: 2048 bytes, from 2.1M of 2.2M). Only the rows the lists name
are written; the oracle runs on a compact copy of those rows with the
lists renumbered, so the host holds no multi-GiB arrays. Paths: one-token
decode (chunk, slab, f16, f32 and general-shape kernels), the fused step
and q4_hip_kv_append_d appending at the cache's last position, and a
prefill-sized launch (band + slab kernels). A
byte offset computed in 32 bits would read or write the wrong rows here."""
import ctypes

import numpy as np
import pytest

import q4kv
from gpu_util import note
from synth import assert_attn_close, heads
from test_gpu_attn import gpu_idx_kv

pytestmark = pytest.mark.gpu

N_KVH, HD, WIDTH = 2, 256, 2051


def _layout(kind):
    """(bytes per token, max_kv, first far position)."""
    if kind == q4kv.KV_Q8:
        return N_KVH * 272, 8_400_000, 7_950_000
    if kind == q4kv.KV_F16:
        return N_KVH * HD * 2, 4_300_000, 4_200_000
    return N_KVH * HD * 4, 2_200_000, 2_100_000


def _lists(rng, n_tok, max_kv, far, pool):
    """[n_tok, n_kvh, WIDTH]: sinks 0-2, 1536 positions from the shared pool,
    then the 512 positions ending at the token's own (the last token at
    max_kv - 1)."""
    sel = np.empty((n_tok, N_KVH, WIDTH), np.int32)
    for t in range(n_tok):
        pos = max_kv - n_tok + t
        cand = pool[pool < pos - 511]
        for kh in range(N_KVH):
            mid = np.sort(rng.choice(cand, WIDTH - 515, replace=False))
            sel[t, kh] = np.concatenate([np.arange(3), mid, np.arange(pos - 511, pos + 1)])
    assert sel[:, :, 3:].min() >= far
    return sel


class _Cache:
    """K and V caches of max_kv tokens on the device holding rows only at the
    positions `used` (sorted), and their compact host copy."""

    def __init__(self, rt, oracle, rng, kind, max_kv, used):
        bpt = _layout(kind)[0]
        self.rt, self.used, self.bpt = rt, used, bpt
        self.k = heads(rng, (used.size, N_KVH))
        self.v = heads(rng, (used.size, N_KVH))
        self.kb = oracle.encode(self.k, kind).reshape(used.size, bpt)
        self.vb = oracle.encode(self.v, kind).reshape(used.size, bpt)
        self.dk, self.dv = rt.alloc(max_kv * bpt), rt.alloc(max_kv * bpt)
        # one copy per run of consecutive positions
        brk = np.flatnonzero(np.diff(used) != 1) + 1
        for i0, i1 in zip(np.r_[0, brk], np.r_[brk, used.size]):
            off = int(used[i0]) * bpt
            rt.h2d(self.dk + off, self.kb[i0:i1])
            rt.h2d(self.dv + off, self.vb[i0:i1])

    def compact(self, sel):
        """sel renumbered to rows of the compact copy (-1 kept)."""
        out = np.searchsorted(self.used, sel).astype(np.int32)
        out[sel < 0] = -1
        assert np.array_equal(self.used[out[sel >= 0]], sel[sel >= 0])
        return out

    def free(self):
        self.rt.free(self.dk)
        self.rt.free(self.dv)


def _setup(rt, oracle, rng, kind, n_tok, pool_n):
    bpt, max_kv, far = _layout(kind)
    pool = np.sort(rng.choice(np.arange(far, max_kv - n_tok - 600), pool_n, replace=False))
    sel = _lists(rng, n_tok, max_kv, far, pool)
    used = np.unique(sel[sel >= 0])
    return max_kv, sel, _Cache(rt, oracle, rng, kind, max_kv, used)


@pytest.mark.parametrize("kind,n_head,n_tok", [
    (q4kv.KV_Q8, 16, 1),    # chunk kernel
    (q4kv.KV_Q8, 32, 1),    # slab kernel (16 query heads per KV head)
    (q4kv.KV_F16, 16, 1),   # f16 kernel
    (q4kv.KV_F32, 16, 1),   # f32 kernel
    (q4kv.KV_Q8, 40, 1),    # general-shape kernel (20 query heads per KV head)
    (q4kv.KV_Q8, 16, 600),  # prefill-sized: band + slab kernels
])
def test_decode_past_4gib(rt, oracle, kind, n_head, n_tok):
    note(f"large cache decode kind={kind} n_head={n_head} n_tok={n_tok}")
    rng = np.random.default_rng(9500 + kind + n_head + n_tok)
    max_kv, sel, cache = _setup(rt, oracle, rng, kind, n_tok, 4000)
    q = heads(rng, (n_tok, n_head))
    try:
        got = gpu_idx_kv(rt, q, cache.dk, cache.dv, kind, n_head, N_KVH, HD, sel.ravel(), WIDTH,
                         N_KVH * WIDTH, WIDTH, max_kv)
    finally:
        cache.free()
    ts = np.arange(n_tok) if n_tok <= 8 else np.unique(
        np.concatenate([[0, n_tok - 1], rng.choice(n_tok, 30, replace=False)]))
    want = oracle.attn(q[ts], cache.kb, cache.vb, kind, n_head, N_KVH, HD, len(ts),
                       idx=cache.compact(sel[ts]).ravel(), width=WIDTH,
                       tok_stride=N_KVH * WIDTH, kvh_stride=WIDTH, max_kv=cache.used.size,
                       threads=8)
    assert_attn_close(got[ts], want, what=f"past 4 GiB kind={kind} n_head={n_head}")


def test_step_appends_past_4gib(rt, oracle):
    """q4_hip_qsa_step_batch appending at position max_kv - 1 (byte offset
    ~4.57e9) of a q8_0 cache, attending a list that ends there."""
    kind, n_head = q4kv.KV_Q8, 16
    note("large cache step append")
    rng = np.random.default_rng(9600)
    max_kv, sel, cache = _setup(rt, oracle, rng, kind, 1, 4000)
    pos = max_kv - 1
    kn, vn = heads(rng, (N_KVH,)), heads(rng, (N_KVH,))
    q = heads(rng, (1, n_head))
    owned = []
    try:
        dq, dkn, dvn = rt.upload(q), rt.upload(kn), rt.upload(vn)
        di = rt.upload(sel.ravel())
        do = rt.alloc(q.nbytes)
        owned += [dq, dkn, dvn, di, do]
        seq = q4kv.SeqDesc(cache.dk, cache.dv, dq, None, do, di, WIDTH, WIDTH, max_kv, 0)
        steps = (q4kv.StepDesc * 1)(q4kv.StepDesc(seq, dkn, dvn, pos))
        dd = rt.alloc(ctypes.sizeof(steps))
        owned.append(dd)
        assert rt.lib.q4_hip_h2d(dd, ctypes.addressof(steps), ctypes.sizeof(steps))
        assert rt.lib.q4_hip_qsa_step_batch(dd, 1, n_head, N_KVH, HD, 1.0 / 16, kind, WIDTH)
        rt.sync()
        got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
        krow = rt.download(cache.dk + pos * cache.bpt, cache.bpt)
        vrow = rt.download(cache.dv + pos * cache.bpt, cache.bpt)
    finally:
        for p in owned:
            rt.free(p)
        cache.free()
    # the appended rows, bit-exact, at the far position
    kb_new, vb_new = oracle.encode(kn, kind), oracle.encode(vn, kind)
    assert np.array_equal(krow, kb_new) and np.array_equal(vrow, vb_new)
    i = int(np.searchsorted(cache.used, pos))
    assert cache.used[i] == pos
    kb, vb = cache.kb.copy(), cache.vb.copy()
    kb[i], vb[i] = kb_new, vb_new
    want = oracle.attn(q, kb, vb, kind, n_head, N_KVH, HD, 1, idx=cache.compact(sel).ravel(),
                       width=WIDTH, tok_stride=N_KVH * WIDTH, kvh_stride=WIDTH,
                       max_kv=cache.used.size)
    assert_attn_close(got, want, what="past 4 GiB step")


@pytest.mark.parametrize("kind", [q4kv.KV_Q8, q4kv.KV_F16, q4kv.KV_F32])
def test_kv_append_d_past_4gib(rt, oracle, kind):
    """q4_hip_kv_append_d at the device position max_kv - 1 (byte offset
    past 2^32): the bytes land there, bit-exact, and the rows beside it are
    untouched."""
    note(f"large cache kv_append_d kind={kind}")
    bpt, max_kv, _ = _layout(kind)
    rng = np.random.default_rng(9700 + kind)
    pos = max_kv - 1
    kn, vn = heads(rng, (N_KVH,)), heads(rng, (N_KVH,))
    dk, dv = rt.alloc(max_kv * bpt), rt.alloc(max_kv * bpt)
    owned = [dk, dv]
    try:
        guard = np.full(bpt, 0xA5, np.uint8)
        for d in (dk, dv):
            rt.h2d(d + (pos - 1) * bpt, guard)
        dkn, dvn = rt.upload(kn), rt.upload(vn)
        owned += [dkn, dvn]
        rt.lib.q4_hip_pos_push(pos)
        assert rt.lib.q4_hip_kv_append_d(dk, dv, dkn, dvn, N_KVH * HD, bpt, kind)
        rt.sync()
        krows = rt.download(dk + (pos - 1) * bpt, 2 * bpt)
        vrows = rt.download(dv + (pos - 1) * bpt, 2 * bpt)
    finally:
        for p in owned:
            rt.free(p)
    assert np.array_equal(krows[bpt:], oracle.encode(kn, kind))
    assert np.array_equal(vrows[bpt:], oracle.encode(vn, kind))
    assert np.array_equal(krows[:bpt], guard) and np.array_equal(vrows[:bpt], guard)
