"""The held append, on the GPU: q4_hip_kv_append_d of whole q8_0 head rows
is held and performed by the next one-token decode on the same caches
(inside its split-kernel launch), or launched first by any other library
call. Cache bytes bit-exact against the oracle, attention within
|err| <= 2e-3 + 1e-3|ref| of the fp64 oracle."""
import numpy as np
import pytest

import q4kv
from gpu_util import note
from synth import WIDTH, assert_attn_close, heads, selection

pytestmark = pytest.mark.gpu

HD = 256


def _out(rt, nbytes):
    p = rt.alloc(nbytes)
    rt.h2d(p, np.full(nbytes // 4, np.nan, np.float32))
    return p


def _caches(rt, oracle, rng, ctx, n_kvh, filled):
    """q8_0 K/V caches of ctx positions, positions < filled written."""
    bpt = q4kv.token_bytes(2, n_kvh, HD)
    k, v = heads(rng, (ctx, n_kvh)), heads(rng, (ctx, n_kvh))
    hk = np.zeros(ctx * bpt, np.uint8)
    hv = np.zeros(ctx * bpt, np.uint8)
    hk[: filled * bpt] = oracle.quant_q8(k[:filled])
    hv[: filled * bpt] = oracle.quant_q8(v[:filled])
    return k, v, hk, hv, rt.upload(hk), rt.upload(hv), bpt


def _decode_kv(rt, q, kc, vc, sel, width, n_head, n_kvh, ctx, gate=None):
    dq, di = rt.upload(q), rt.upload(sel)
    dg = rt.upload(gate) if gate is not None else None
    do = _out(rt, q.nbytes)
    assert rt.lib.q4_hip_qsa_decode_idx_kv(dq, kc, vc, dg, do, di, width, n_kvh * width, width,
                                           n_head, n_kvh, HD, q.shape[0], ctx, 1.0 / 16, 2)
    return do, (dq, di, dg)


def _want(oracle, q, hk, hv, sel, width, n_head, n_kvh, ctx, gate=None):
    return oracle.attn(q, hk, hv, 2, n_head, n_kvh, HD, q.shape[0], gate=gate, idx=sel,
                       width=width, tok_stride=n_kvh * width, kvh_stride=width, max_kv=ctx)


def _lists(rng, n, pos):
    return np.ascontiguousarray(np.stack([selection(rng, pos) for _ in range(n)]), np.int32)


def _append_oracle(oracle, hk, hv, k, v, n, bpt, pos):
    oracle.lib.orc_kv_append(hk.ctypes.data, hv.ctypes.data, k.ctypes.data, v.ctypes.data, n,
                             bpt, 2, pos)


# 8 query heads per KV head (the chunk kernel), 4 (chunk), 12 (the slab kernel)
@pytest.mark.parametrize("n_head,gated", [(16, False), (16, True), (8, False), (24, True)])
def test_held_append_performed_by_the_decode(rt, oracle, n_head, gated):
    """append_d then decode_idx_kv at consecutive positions: the new rows
    bit-exact in both caches and seen by the decode of the same call pair."""
    note(f"held append absorbed n_head={n_head} gated={gated}")
    rng = np.random.default_rng(7200 + n_head + gated)
    ctx, n_kvh, start = 8192, 2, 5000
    k, v, hk, hv, kc, vc, bpt = _caches(rt, oracle, rng, ctx, n_kvh, start)
    dk, dv = rt.alloc(n_kvh * HD * 4), rt.alloc(n_kvh * HD * 4)
    for pos in range(start, start + 3):
        rt.h2d(dk, k[pos])
        rt.h2d(dv, v[pos])
        q = heads(rng, (1, n_head))
        gate = rng.standard_normal((1, n_head, HD)).astype(np.float32) if gated else None
        sel = _lists(rng, n_kvh, pos).ravel()
        rt.lib.q4_hip_pos_push(pos)
        assert rt.lib.q4_hip_kv_append_d(kc, vc, dk, dv, n_kvh * HD, bpt, 2)
        do, tmp = _decode_kv(rt, q, kc, vc, sel, WIDTH, n_head, n_kvh, ctx, gate)
        rt.sync()
        _append_oracle(oracle, hk, hv, k[pos], v[pos], n_kvh * HD, bpt, pos)
        assert np.array_equal(rt.download(kc, hk.size), hk), "K cache bytes"
        assert np.array_equal(rt.download(vc, hv.size), hv), "V cache bytes"
        got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
        assert_attn_close(got, _want(oracle, q, hk, hv, sel, WIDTH, n_head, n_kvh, ctx, gate),
                          what=f"pos {pos}")
        for p in (do, *tmp):
            if p:
                rt.free(p)
    for p in (kc, vc, dk, dv):
        rt.free(p)


def test_held_append_launched_by_other_calls(rt, oracle):
    """A held append is launched before any other library call: a device
    read of the cache, a decode on other caches, a second append, a
    position push."""
    note("held append flushed")
    rng = np.random.default_rng(7300)
    ctx, n_kvh, n_head, pos = 4096, 2, 16, 3000
    k, v, hk, hv, kc, vc, bpt = _caches(rt, oracle, rng, ctx, n_kvh, pos)
    k2, v2, hk2, hv2, kc2, vc2, _ = _caches(rt, oracle, rng, ctx, n_kvh, pos)
    dk, dv = rt.upload(k[pos]), rt.upload(v[pos])
    dk2, dv2 = rt.upload(k2[pos]), rt.upload(v2[pos])
    n = n_kvh * HD
    rt.lib.q4_hip_pos_push(pos)
    _append_oracle(oracle, hk, hv, k[pos], v[pos], n, bpt, pos)
    _append_oracle(oracle, hk2, hv2, k2[pos], v2[pos], n, bpt, pos)
    # 1. a read of the cache (q4_hip_d2h) sees the row
    assert rt.lib.q4_hip_kv_append_d(kc, vc, dk, dv, n, bpt, 2)
    assert np.array_equal(rt.download(kc, hk.size), hk)
    assert np.array_equal(rt.download(vc, hv.size), hv)
    # 2. append to caches 2, then decode caches 1: the append runs first
    assert rt.lib.q4_hip_kv_append_d(kc2, vc2, dk2, dv2, n, bpt, 2)
    q = heads(rng, (1, n_head))
    sel = _lists(rng, n_kvh, pos).ravel()
    do, tmp = _decode_kv(rt, q, kc, vc, sel, WIDTH, n_head, n_kvh, ctx)
    rt.sync()
    assert np.array_equal(rt.download(kc2, hk2.size), hk2)
    assert np.array_equal(rt.download(vc2, hv2.size), hv2)
    got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
    assert_attn_close(got, _want(oracle, q, hk, hv, sel, WIDTH, n_head, n_kvh, ctx),
                      what="decode after a foreign append")
    # 3. two appends in a row: the first is launched by the second
    p2 = pos + 1
    for dev, x in ((dk, k[p2]), (dv, v[p2]), (dk2, k2[p2]), (dv2, v2[p2])):
        rt.h2d(dev, x)
    rt.lib.q4_hip_pos_push(p2)
    assert rt.lib.q4_hip_kv_append_d(kc, vc, dk, dv, n, bpt, 2)
    assert rt.lib.q4_hip_kv_append_d(kc2, vc2, dk2, dv2, n, bpt, 2)
    rt.lib.q4_hip_stream_sync()
    _append_oracle(oracle, hk, hv, k[p2], v[p2], n, bpt, p2)
    _append_oracle(oracle, hk2, hv2, k2[p2], v2[p2], n, bpt, p2)
    for dev, host in ((kc, hk), (vc, hv), (kc2, hk2), (vc2, hv2)):
        assert np.array_equal(rt.download(dev, host.size), host)
    # 4. a position push between append and decode: the append lands at the
    # position it was issued at
    rt.h2d(dk, k[p2 + 1])
    rt.h2d(dv, v[p2 + 1])
    rt.lib.q4_hip_pos_push(p2 + 1)
    assert rt.lib.q4_hip_kv_append_d(kc, vc, dk, dv, n, bpt, 2)
    rt.lib.q4_hip_pos_push(p2 + 2)
    rt.sync()
    _append_oracle(oracle, hk, hv, k[p2 + 1], v[p2 + 1], n, bpt, p2 + 1)
    assert np.array_equal(rt.download(kc, hk.size), hk)
    for p in (kc, vc, kc2, vc2, dk, dv, dk2, dv2, do, *tmp):
        if p:
            rt.free(p)


def test_held_append_in_graph_replays(rt, oracle):
    """append_d + decode captured together: the append rides in the split
    kernel (split + merge: 2 nodes), replayed at four positions."""
    note("held append in graph")
    rng = np.random.default_rng(7400)
    ctx, n_kvh, n_head, start = 8192, 2, 16, 4000
    k, v, hk, hv, kc, vc, bpt = _caches(rt, oracle, rng, ctx, n_kvh, start)
    dk, dv = rt.alloc(n_kvh * HD * 4), rt.alloc(n_kvh * HD * 4)
    dq, di = rt.alloc(n_head * HD * 4), rt.alloc(n_kvh * WIDTH * 4)
    do = _out(rt, n_head * HD * 4)
    assert rt.lib.q4_hip_graph_begin() == 1
    ok = rt.lib.q4_hip_kv_append_d(kc, vc, dk, dv, n_kvh * HD, bpt, 2)
    ok = ok and rt.lib.q4_hip_qsa_decode_idx_kv(dq, kc, vc, None, do, di, WIDTH, n_kvh * WIDTH,
                                                WIDTH, n_head, n_kvh, HD, 1, ctx, 1.0 / 16, 2)
    g = rt.lib.q4_hip_graph_end()
    assert ok and g
    assert rt.lib.q4_hip_graph_nodes(g) == 2, "the append should ride in the split kernel"
    try:
        for pos in range(start, start + 4):
            q = heads(rng, (1, n_head))
            sel = _lists(rng, n_kvh, pos).ravel()
            for dev, x in ((dk, k[pos]), (dv, v[pos]), (dq, q), (di, sel)):
                rt.h2d(dev, x)
            rt.lib.q4_hip_pos_push(pos)
            assert rt.lib.q4_hip_graph_launch(g)
            rt.sync()
            _append_oracle(oracle, hk, hv, k[pos], v[pos], n_kvh * HD, bpt, pos)
            got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
            assert_attn_close(got, _want(oracle, q, hk, hv, sel, WIDTH, n_head, n_kvh, ctx),
                              what=f"replay {pos}")
        assert np.array_equal(rt.download(kc, hk.size), hk)
        assert np.array_equal(rt.download(vc, hv.size), hv)
    finally:
        rt.lib.q4_hip_graph_free(g)
    for p in (kc, vc, dk, dv, dq, di, do):
        rt.free(p)
