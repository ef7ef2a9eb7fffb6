"""q4_hip_qsa_step_batch -- a decode step's K/V append and attention in one
launch -- against the two launches it stands for (q4_hip_kv_append_batch,
then q4_hip_qsa_decode_batch) on the same inputs: cache bytes and outputs
bit-identical, and the outputs against the oracle over the appended cache."""
import ctypes

import numpy as np
import pytest

import q4kv
from gpu_util import note
from synth import WIDTH, assert_attn_close, heads, selection

pytestmark = pytest.mark.gpu

N_HEAD, N_KVH, HD = 16, 2, 256


def _case(rng, oracle, n_seq, ctx, kind, pos_of, sel_of, n_head=N_HEAD):
    """Host data of n_seq items: caches holding positions < pos, the new
    token's rows, queries and per-KV-head lists."""
    bpt = q4kv.token_bytes(kind, N_KVH, HD)
    items = []
    for s in range(n_seq):
        pos = pos_of(s)
        k, v = heads(rng, (ctx, N_KVH)), heads(rng, (ctx, N_KVH))
        k[pos:] = 0.0
        v[pos:] = 0.0
        kn, vn = heads(rng, (N_KVH,)), heads(rng, (N_KVH,))
        q = heads(rng, (1, n_head))
        sel = sel_of(rng, s, pos)
        enc = (lambda x: oracle.encode(x, kind))
        items.append(dict(pos=pos, kc=enc(k), vc=enc(v), kn=kn, vn=vn, q=q, sel=sel,
                          k=k, v=v))
    return items, bpt


def _run(rt, items, ctx, kind, fused, dense=False):
    """Run one step for every item; returns (caches, outputs) downloaded."""
    n_seq = len(items)
    ptrs = []
    before = set(rt._owned)
    steps = (q4kv.StepDesc * n_seq)()
    seqs = (q4kv.SeqDesc * n_seq)()
    apps = (q4kv.AppendDesc * n_seq)()
    for s, it in enumerate(items):
        kc, vc = rt.upload(it["kc"]), rt.upload(it["vc"])
        dkn, dvn, dq = rt.upload(it["kn"]), rt.upload(it["vn"]), rt.upload(it["q"])
        do = rt.alloc(it["q"].nbytes)
        rt.h2d(do, np.full(it["q"].size, np.nan, np.float32))
        di = None if dense else rt.upload(it["sel"])
        n_sel = it["pos"] + 1 if dense else it["sel"].shape[-1]
        stride = 0 if dense else it["sel"].shape[-1]
        seqs[s] = q4kv.SeqDesc(kc, vc, dq, None, do, di, n_sel, stride, ctx, 0)
        steps[s] = q4kv.StepDesc(seqs[s], dkn, dvn, it["pos"])
        apps[s] = q4kv.AppendDesc(kc, vc, dkn, dvn, it["pos"], 0)
        ptrs.append((kc, vc, do))
    max_n = max((it["pos"] + 1) if dense else it["sel"].shape[-1] for it in items)
    lib = rt.lib
    nh = items[0]["q"].shape[1]
    if fused:
        dd = rt.alloc(ctypes.sizeof(steps))
        assert lib.q4_hip_h2d(dd, ctypes.addressof(steps), ctypes.sizeof(steps))
        assert lib.q4_hip_qsa_step_batch(dd, n_seq, nh, N_KVH, HD, 1.0 / 16, kind, max_n)
    else:
        da = rt.alloc(ctypes.sizeof(apps))
        ds = rt.alloc(ctypes.sizeof(seqs))
        assert lib.q4_hip_h2d(da, ctypes.addressof(apps), ctypes.sizeof(apps))
        assert lib.q4_hip_h2d(ds, ctypes.addressof(seqs), ctypes.sizeof(seqs))
        bpt = q4kv.token_bytes(kind, N_KVH, HD)
        assert lib.q4_hip_kv_append_batch(da, n_seq, N_KVH * HD, bpt, kind)
        assert lib.q4_hip_qsa_decode_batch(ds, n_seq, nh, N_KVH, HD, 1.0 / 16, kind, max_n)
    rt.sync()
    caches, outs = [], []
    for (kc, vc, do), it in zip(ptrs, items):
        caches.append((rt.download(kc, it["kc"].nbytes, np.uint8),
                       rt.download(vc, it["vc"].nbytes, np.uint8)))
        outs.append(rt.download(do, it["q"].nbytes, np.float32).reshape(it["q"].shape))
    for p in [p for p in rt._owned if p not in before]:
        rt.free(p)
    return caches, outs


def _check(rt, oracle, items, ctx, kind, dense=False, what=""):
    note(f"step batch {what}")
    c1, o1 = _run(rt, items, ctx, kind, fused=True, dense=dense)
    c2, o2 = _run(rt, items, ctx, kind, fused=False, dense=dense)
    for s, it in enumerate(items):
        assert np.array_equal(c1[s][0], c2[s][0]) and np.array_equal(c1[s][1], c2[s][1]), \
            f"{what}: cache bytes differ, item {s}"
        assert np.array_equal(o1[s], o2[s]), f"{what}: outputs differ, item {s}"
        # the appended row is the encoding of the new token
        bpt = q4kv.token_bytes(kind, N_KVH, HD)
        p = it["pos"]
        assert np.array_equal(c1[s][0][p * bpt:(p + 1) * bpt], oracle.encode(it["kn"], kind))
        k = it["k"].copy()
        v = it["v"].copy()
        k[p], v[p] = it["kn"], it["vn"]
        kq, vq = oracle.encode(k, kind), oracle.encode(v, kind)
        if dense:
            want = oracle.attn(it["q"], kq, vq, kind, it["q"].shape[1], N_KVH, HD, 1, kv_base=p,
                               max_kv=ctx, scale=1.0 / 16)
        else:
            w = it["sel"].shape[-1]
            want = oracle.attn(it["q"], kq, vq, kind, it["q"].shape[1], N_KVH, HD, 1, idx=it["sel"],
                               width=w, tok_stride=N_KVH * w, kvh_stride=w, max_kv=ctx,
                               scale=1.0 / 16)
        assert_attn_close(o1[s], want, what=f"{what} item {s}")


def _sel_kv(rng, s, pos):
    return np.stack([selection(rng, pos) for _ in range(N_KVH)])


# 12 sequences (24 items): two 64-position chunks per workgroup, the
# single-buffer kernel; 32 sequences (64 items): five chunks per workgroup,
# the double-buffered instance (fused step and batched decode alike)
@pytest.mark.parametrize("n_seq", [12, 32])
def test_step_batch_q8_matches_append_then_decode(rt, oracle, n_seq):
    """n_seq layers, new position inside each list (the list's last entry)."""
    rng = np.random.default_rng(900 + n_seq)
    ctx = 16384
    items, _ = _case(rng, oracle, n_seq, ctx, q4kv.KV_Q8, lambda s: ctx - 1 - 300 * s, _sel_kv)
    _check(rt, oracle, items, ctx, q4kv.KV_Q8, what=f"q8 {n_seq} layers")


@pytest.mark.parametrize("kind", [q4kv.KV_Q8, q4kv.KV_F16, q4kv.KV_F32])
def test_step_batch_position_anywhere_in_list(rt, oracle, kind):
    """The new position listed first, in a middle chunk and twice, or not at
    all (then only the cache write shows it)."""
    rng = np.random.default_rng(901 + kind)
    ctx = 8192

    def sel_of(rng, s, pos):
        base = np.stack([selection(rng, pos - 1) for _ in range(N_KVH)])
        if s == 0:
            base[:, 0] = pos                      # first chunk
        elif s == 1:
            base[:, 1000] = pos                   # a middle chunk (another split)
        elif s == 2:
            base[:, 70] = pos                     # twice, two chunks
            base[:, 2000] = pos
        return base                               # s == 3: not listed
    items, _ = _case(rng, oracle, 4, ctx, kind, lambda s: 5000 + 37 * s, sel_of)
    _check(rt, oracle, items, ctx, kind, what=f"position anywhere, width {kind}")


@pytest.mark.parametrize("kind", [q4kv.KV_Q8, q4kv.KV_F16, q4kv.KV_F32])
def test_step_batch_dense_items(rt, oracle, kind):
    """Dense items (no list): positions 0 .. pos, the new one last."""
    rng = np.random.default_rng(902 + kind)
    ctx = 4096
    items, _ = _case(rng, oracle, 3, ctx, kind, lambda s: 1000 + 1500 * s, _sel_kv)
    _check(rt, oracle, items, ctx, kind, dense=True, what=f"dense, width {kind}")


@pytest.mark.parametrize("kind", [q4kv.KV_F16, q4kv.KV_F32])
def test_step_batch_other_widths(rt, oracle, kind):
    """f16 and f32 caches: the fused launch (append inside the attention)
    against the append launch then the attention launch."""
    rng = np.random.default_rng(903 + kind)
    ctx = 4096
    items, _ = _case(rng, oracle, 3, ctx, kind, lambda s: ctx - 1 - 300 * s, _sel_kv)
    _check(rt, oracle, items, ctx, kind, what=f"width {kind}")


@pytest.mark.parametrize("kind", [q4kv.KV_Q8, q4kv.KV_F16, q4kv.KV_F32])
@pytest.mark.parametrize("n_head", [24, 32, 18])
def test_step_batch_more_heads_per_kv_head(rt, oracle, n_head, kind):
    """The production layout (24 query heads over 2 KV heads, 12 per KV head),
    16 per KV head, and an odd 9: the fused step of two head groups against
    append + batched decode, and against the oracle."""
    rng = np.random.default_rng(950 + n_head + 100 * kind)
    ctx = 16384
    items, _ = _case(rng, oracle, 12, ctx, kind, lambda s: ctx - 1 - 300 * s, _sel_kv,
                     n_head=n_head)
    _check(rt, oracle, items, ctx, kind, what=f"width {kind}, 12 layers, {n_head} heads")


@pytest.mark.parametrize("kind", [q4kv.KV_Q8, q4kv.KV_F16, q4kv.KV_F32])
def test_step_batch_more_heads_position_anywhere(rt, oracle, kind):
    """24 heads: the new position first, in a middle split, twice, or not at all."""
    rng = np.random.default_rng(960 + kind)
    ctx = 8192

    def sel_of(rng, s, pos):
        base = np.stack([selection(rng, pos - 1) for _ in range(N_KVH)])
        if s == 0:
            base[:, 0] = pos
        elif s == 1:
            base[:, 1000] = pos
        elif s == 2:
            base[:, 70] = pos
            base[:, 2000] = pos
        return base
    items, _ = _case(rng, oracle, 4, ctx, kind, lambda s: 5000 + 37 * s, sel_of, n_head=24)
    _check(rt, oracle, items, ctx, kind, what=f"24 heads, position anywhere, width {kind}")


@pytest.mark.parametrize("kind,n_seq", [(q4kv.KV_Q8, 3), (q4kv.KV_F16, 3), (q4kv.KV_F32, 3),
                                        (q4kv.KV_Q8, 32), (q4kv.KV_F16, 32)])
def test_step_batch_graph_replays(rt, oracle, kind, n_seq):
    """q4_hip_qsa_step_batch captured once into a graph and replayed four
    times, each replay a new decode position with new rows, queries and
    selections written between replays (descriptors included): every replay
    matches the oracle over the cache as appended so far, and the caches end
    byte-identical to the oracle's appends. 3 sequences take one chunk or
    pass per split; 32 take several (q8_0: the slab kernel)."""
    note(f"graph-captured step_batch kind={kind} n_seq={n_seq}")
    rng = np.random.default_rng(970 + kind + n_seq)
    ctx, base = 6000, 5000
    bpt = q4kv.token_bytes(kind, N_KVH, HD)
    lib = rt.lib
    hk, hv, kcs, vcs = [], [], [], []
    for s in range(n_seq):
        k, v = heads(rng, (ctx, N_KVH)), heads(rng, (ctx, N_KVH))
        k[base:] = 0.0
        v[base:] = 0.0
        hk.append(oracle.encode(k, kind).copy())
        hv.append(oracle.encode(v, kind).copy())
        kcs.append(rt.upload(hk[-1]))
        vcs.append(rt.upload(hv[-1]))
    dq = [rt.alloc(N_HEAD * HD * 4) for _ in range(n_seq)]
    dkn = [rt.alloc(N_KVH * HD * 4) for _ in range(n_seq)]
    dvn = [rt.alloc(N_KVH * HD * 4) for _ in range(n_seq)]
    dsel = [rt.alloc(N_KVH * WIDTH * 4) for _ in range(n_seq)]
    dout = [rt.alloc(N_HEAD * HD * 4) for _ in range(n_seq)]
    dd = rt.alloc(ctypes.sizeof(q4kv.StepDesc) * n_seq)

    def descs(pos):
        steps = (q4kv.StepDesc * n_seq)()
        for s in range(n_seq):
            seq = q4kv.SeqDesc(kcs[s], vcs[s], dq[s], None, dout[s], dsel[s], WIDTH, WIDTH,
                               ctx, 0)
            steps[s] = q4kv.StepDesc(seq, dkn[s], dvn[s], pos)
        assert lib.q4_hip_h2d(dd, ctypes.addressof(steps), ctypes.sizeof(steps))
        rt.sync()

    descs(base)
    assert lib.q4_hip_graph_begin() == 1
    ok = lib.q4_hip_qsa_step_batch(dd, n_seq, N_HEAD, N_KVH, HD, 1.0 / 16, kind, WIDTH)
    g = lib.q4_hip_graph_end()
    assert ok and g
    try:
        for pos in (base, base + 1, base + 2, base + 3):
            qs, sels = [], []
            for s in range(n_seq):
                q = heads(rng, (1, N_HEAD))
                kn, vn = heads(rng, (N_KVH,)), heads(rng, (N_KVH,))
                sel = np.stack([selection(rng, pos) for _ in range(N_KVH)])
                rt.h2d(dq[s], q)
                rt.h2d(dkn[s], kn)
                rt.h2d(dvn[s], vn)
                rt.h2d(dsel[s], sel)
                hk[s][pos * bpt:(pos + 1) * bpt] = oracle.encode(kn, kind)
                hv[s][pos * bpt:(pos + 1) * bpt] = oracle.encode(vn, kind)
                qs.append(q)
                sels.append(sel)
            descs(pos)
            assert lib.q4_hip_graph_launch(g)
            rt.sync()
            for s in range(n_seq):
                got = rt.download(dout[s], qs[s].nbytes, np.float32).reshape(qs[s].shape)
                want = oracle.attn(qs[s], hk[s], hv[s], kind, N_HEAD, N_KVH, HD, 1,
                                   idx=sels[s].ravel(), width=WIDTH, tok_stride=N_KVH * WIDTH,
                                   kvh_stride=WIDTH, max_kv=ctx, scale=1.0 / 16)
                assert_attn_close(got, want, what=f"replay pos {pos} seq {s}")
        for s in range(n_seq):
            assert np.array_equal(rt.download(kcs[s], hk[s].size), hk[s])
            assert np.array_equal(rt.download(vcs[s], hv[s].size), hv[s])
    finally:
        lib.q4_hip_graph_free(g)
        for p in kcs + vcs + dq + dkn + dvn + dsel + dout + [dd]:
            rt.free(p)
