"""The held append, on the GPU: q4_hip_kv_append_d of whole q8_0 head rows
is held and performed by the next one-token decode on the same caches
(inside its split-kernel launch), by the indexer call that follows the
append in the reference's decode order (q4_hip_f32_to_f16_d, or the fused
q4_hip_qsa_index_score_d), or launched first by any other library call. Cache bytes bit-exact against the oracle, attention within
|err| <= 2e-3 + 1e-3|ref| of the fp64 oracle."""
import numpy as np
import pytest

import q4kv
from gpu_util import note
from qsa_util import IDX_DIM, IDX_HEADS, K_BLK, N_ROT, RATIO, RMS_EPS, ROPE_BASE, raw_keys
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


@pytest.mark.parametrize("fused", [False, True])
def test_held_append_carried_by_the_indexer(rt, oracle, fused):
    """The reference's per-layer decode order (src/q4_fwd.c:891-922):
    append_d, then the indexer (f32_to_f16_d + pool_d + k_prep_d + score_d,
    or the fused index_score_d), topk_d, decode_idx. The indexer's first
    launch carries the held append. Everything the layer writes (cache bytes,
    raw key row, pool, scores, selection, attention output) is bit-identical
    to the same calls with the append launched on its own, and the cache rows
    equal the oracle's."""
    note(f"held append carried by the indexer fused={fused}")
    lib = rt.lib
    rng = np.random.default_rng(7500 + fused)
    ctx, n_kvh, n_head, start = 8192, 2, 16, 5000
    n = n_kvh * HD
    k, v, hk, hv, kc0, vc0, bpt = _caches(rt, oracle, rng, ctx, n_kvh, start)
    rt.free(kc0)
    rt.free(vc0)
    max_blocks = ctx // RATIO
    raw = raw_keys(rng, ctx)
    pool0 = (rng.standard_normal((max_blocks, IDX_DIM)) * 0.3).astype(np.float32)
    wn = (1 + 0.2 * rng.standard_normal(IDX_DIM)).astype(np.float32)
    qw = (1 + 0.2 * rng.standard_normal(IDX_DIM)).astype(np.float32)

    def layer(d, pos, held):
        lib.q4_hip_pos_push(pos)
        assert lib.q4_hip_kv_append_d(d["kc"], d["vc"], d["dk"], d["dv"], n, bpt, 2)
        if not held:
            assert lib.q4_hip_stream_sync()  # launches the held append on its own
        if fused:
            assert lib.q4_hip_qsa_index_score_d(d["raw"], d["pool"], d["wn"], d["ik"], d["iq"],
                                                d["qw"], d["sc"], max_blocks, IDX_HEADS,
                                                IDX_DIM, RATIO, N_ROT, ROPE_BASE, RMS_EPS)
        else:
            assert lib.q4_hip_f32_to_f16_d(d["raw"], IDX_DIM, d["ik"], IDX_DIM)
            assert lib.q4_hip_qsa_pool_d(d["raw"], d["pool"], d["wn"], IDX_DIM, RATIO, N_ROT,
                                         ROPE_BASE, RMS_EPS)
            assert lib.q4_hip_qsa_k_prep_d(d["iq"], d["qw"], IDX_HEADS, IDX_DIM, N_ROT,
                                           ROPE_BASE, RMS_EPS)
            assert lib.q4_hip_qsa_score_d(d["iq"], d["pool"], d["sc"], max_blocks, IDX_HEADS,
                                          IDX_DIM, RATIO)
        assert lib.q4_hip_qsa_topk_d(d["sc"], d["sel"], max_blocks, K_BLK, RATIO, WIDTH)
        assert lib.q4_hip_qsa_decode_idx(d["q"], d["kc"], d["vc"], d["g"], d["out"], d["sel"],
                                         WIDTH, n_head, n_kvh, HD, 1, ctx, 1.0 / 16, 2)
        rt.sync()

    sets = []
    for held in (False, True):
        sets.append(dict(kc=rt.upload(hk), vc=rt.upload(hv), dk=rt.alloc(n * 4),
                         dv=rt.alloc(n * 4), raw=rt.upload(raw), pool=rt.upload(pool0),
                         wn=rt.upload(wn), qw=rt.upload(qw), ik=rt.alloc(IDX_DIM * 4),
                         iq=rt.alloc(IDX_HEADS * IDX_DIM * 4), sc=rt.alloc(max_blocks * 4),
                         sel=rt.alloc(WIDTH * 4), q=rt.alloc(n_head * HD * 4),
                         g=rt.alloc(n_head * HD * 4),
                         out=_out(rt, n_head * HD * 4)))
    for pos in range(start, start + 3):
        ik = rng.standard_normal(IDX_DIM).astype(np.float32)
        iq = rng.standard_normal((IDX_HEADS, IDX_DIM)).astype(np.float32)
        q = heads(rng, (1, n_head))
        gate = rng.standard_normal((1, n_head, HD)).astype(np.float32)
        outs = []
        for held, d in zip((False, True), sets):
            for key, x in (("dk", k[pos]), ("dv", v[pos]), ("ik", ik), ("iq", iq), ("q", q),
                           ("g", gate)):
                rt.h2d(d[key], x)
            layer(d, pos, held)
            outs.append([rt.download(d["kc"], hk.size), rt.download(d["vc"], hv.size),
                         rt.download(d["raw"], raw.nbytes), rt.download(d["pool"], pool0.nbytes),
                         rt.download(d["sc"], (pos + 1) // RATIO * 4),  # rows written
                         rt.download(d["sel"], WIDTH * 4),
                         rt.download(d["out"], q.nbytes)])
        _append_oracle(oracle, hk, hv, k[pos], v[pos], n, bpt, pos)
        assert np.array_equal(outs[1][0], hk), f"pos {pos}: K cache bytes"
        assert np.array_equal(outs[1][1], hv), f"pos {pos}: V cache bytes"
        for name, a, b in zip(("K", "V", "raw", "pool", "scores", "selection", "output"),
                              outs[0], outs[1]):
            assert np.array_equal(a, b), f"pos {pos}: {name} differs from the unheld order"
        sel = outs[1][5].view(np.int32)
        got = outs[1][6].view(np.float32).reshape(q.shape)
        want = oracle.attn(q, hk, hv, 2, n_head, n_kvh, HD, 1, gate=gate,
                           idx=np.tile(sel, n_kvh), width=WIDTH, tok_stride=n_kvh * WIDTH, kvh_stride=WIDTH, max_kv=ctx)
        assert_attn_close(got, want, what=f"pos {pos}")
    for d in sets:
        for p in d.values():
            rt.free(p)


@pytest.mark.parametrize("fused", [False, True])
def test_held_append_carried_by_the_indexer_in_graph(rt, oracle, fused):
    """append_d captured with the indexer's first call: one node (the append
    rides in it), and each replay writes the rows at the pushed position."""
    note(f"held append + indexer in graph fused={fused}")
    lib = rt.lib
    rng = np.random.default_rng(7600 + fused)
    ctx, n_kvh, start = 4096, 2, 3000
    n = n_kvh * HD
    k, v, hk, hv, kc, vc, bpt = _caches(rt, oracle, rng, ctx, n_kvh, start)
    max_blocks = ctx // RATIO
    dk, dv = rt.alloc(n * 4), rt.alloc(n * 4)
    d_raw, d_ik = rt.upload(raw_keys(rng, ctx)), rt.alloc(IDX_DIM * 4)
    d_pool = rt.upload(np.zeros((max_blocks, IDX_DIM), np.float32))
    d_wn = rt.upload(np.ones(IDX_DIM, np.float32))
    d_iq = rt.upload(rng.standard_normal((IDX_HEADS, IDX_DIM)).astype(np.float32))
    d_sc = rt.alloc(max_blocks * 4)
    assert lib.q4_hip_graph_begin() == 1
    ok = lib.q4_hip_kv_append_d(kc, vc, dk, dv, n, bpt, 2)
    if fused:
        ok = ok and lib.q4_hip_qsa_index_score_d(d_raw, d_pool, d_wn, d_ik, d_iq, d_wn, d_sc,
                                                 max_blocks, IDX_HEADS, IDX_DIM, RATIO, N_ROT,
                                                 ROPE_BASE, RMS_EPS)
    else:
        ok = ok and lib.q4_hip_f32_to_f16_d(d_raw, IDX_DIM, d_ik, IDX_DIM)
    g = lib.q4_hip_graph_end()
    assert ok and g
    try:
        assert lib.q4_hip_graph_nodes(g) == 1, "the append should ride in the indexer launch"
        for pos in range(start, start + 3):
            rt.h2d(dk, k[pos])
            rt.h2d(dv, v[pos])
            rt.h2d(d_ik, rng.standard_normal(IDX_DIM).astype(np.float32))
            lib.q4_hip_pos_push(pos)
            assert lib.q4_hip_graph_launch(g)
            rt.sync()
            _append_oracle(oracle, hk, hv, k[pos], v[pos], n, bpt, pos)
            assert np.array_equal(rt.download(kc, hk.size), hk), f"replay {pos}: K"
            assert np.array_equal(rt.download(vc, hv.size), hv), f"replay {pos}: V"
    finally:
        lib.q4_hip_graph_free(g)
    for p in (kc, vc, dk, dv, d_raw, d_ik, d_pool, d_wn, d_iq, d_sc):
        rt.free(p)
