"""Attention shapes outside the MFMA kernels' tiling, which the reference
accepts (src/q4_rocm.cu:7253-7297: any hd <= 256, any number of query heads
per KV head, on its one-block-per-head fallback): head_dim not a multiple of
32 for f16/f32 caches, and more than 16 query heads per KV head for every
width. Each entry point family (dense causal, per-KV-head lists, shared
list, batch, decode step) against the oracle, with the attention bar
|got - ref| <= 2e-3 + 1e-3*|ref|; splits and the merge are exercised by long
lists over few items."""
import ctypes

import numpy as np
import pytest

import q4kv
from gpu_util import note, quantize_on_gpu
from synth import assert_attn_close, heads
from test_gpu_attn import _out, gpu_idx_kv

pytestmark = pytest.mark.gpu


def _lists(rng, n_tok, n_kvh, width, ctx, pad):
    """[n_tok, n_kvh, width] distinct positions, the last `pad` of each -1,
    plus one out-of-range entry per list when there is room."""
    sel = np.full((n_tok, n_kvh, width), -1, np.int32)
    for t in range(n_tok):
        for kh in range(n_kvh):
            n = width - pad
            sel[t, kh, :n] = rng.choice(ctx, n, replace=False)
            if pad:
                sel[t, kh, n] = ctx + 7  # skipped like padding
    return sel


# (kind, hd, n_head, n_kvh): odd and non-32 head dims (f16/f32); 24, 32 and
# 20 query heads per KV head (three, four and three head groups)
IDX_CASES = [
    (1, 80, 16, 2),
    (0, 72, 6, 2),
    (1, 33, 4, 1),
    (0, 200, 3, 3),
    (2, 128, 24, 1),
    (2, 256, 64, 2),
    (1, 64, 40, 2),
]


@pytest.mark.parametrize("kind,hd,n_head,n_kvh", IDX_CASES)
def test_any_shape_indexed(rt, oracle, kind, hd, n_head, n_kvh):
    note(f"any-shape idx_kv kind={kind} hd={hd} n_head={n_head} n_kvh={n_kvh}")
    rng = np.random.default_rng(900 + 7 * kind + hd + n_head)
    ctx, n_tok, width = 9000, 3, 2051
    k = heads(rng, (ctx, n_kvh), hd=hd)
    v = heads(rng, (ctx, n_kvh), hd=hd)
    q = heads(rng, (n_tok, n_head), hd=hd)
    gate = rng.standard_normal((n_tok, n_head, hd)).astype(np.float32)
    kc, _ = quantize_on_gpu(rt, k, kind)
    vc, _ = quantize_on_gpu(rt, v, kind)
    kb, vb = oracle.encode(k, kind), oracle.encode(v, kind)
    sel = _lists(rng, n_tok, n_kvh, width, ctx, pad=37)
    got = gpu_idx_kv(rt, q, kc, vc, kind, n_head, n_kvh, hd, sel.ravel(), width,
                     n_kvh * width, width, ctx, gate=gate)
    want = oracle.attn(q, kb, vb, kind, n_head, n_kvh, hd, n_tok, gate=gate, idx=sel.ravel(),
                       width=width, tok_stride=n_kvh * width, kvh_stride=width, max_kv=ctx,
                       threads=8)
    assert_attn_close(got, want, what=f"idx_kv hd={hd} gqa={n_head // n_kvh}")
    # the reference's shared-list entry point (one list for every KV head)
    shared = sel[:, 0, :].copy()
    dq, dg, di = rt.upload(q), rt.upload(gate), rt.upload(shared.ravel())
    do = _out(rt, q.nbytes)
    assert rt.lib.q4_hip_qsa_decode_idx(dq, kc, vc, dg, do, di, width, n_head, n_kvh, hd,
                                        n_tok, ctx, 1.0 / np.sqrt(hd), kind)
    rt.sync()
    got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
    want = oracle.attn(q, kb, vb, kind, n_head, n_kvh, hd, n_tok, gate=gate,
                       idx=shared.ravel(), width=width, tok_stride=width, kvh_stride=0,
                       max_kv=ctx, threads=8)
    assert_attn_close(got, want, what=f"shared list hd={hd}")
    # all-padding lists give zeros
    empty = np.full(n_tok * n_kvh * 5, -1, np.int32)
    got = gpu_idx_kv(rt, q, kc, vc, kind, n_head, n_kvh, hd, empty, 5, n_kvh * 5, 5, ctx)
    assert not got.any()
    for p in (dq, dg, di, do, kc, vc):
        rt.free(p)


@pytest.mark.parametrize("kind,hd,n_head,n_kvh,n_tok,base", [
    (1, 80, 16, 2, 1, 20000),   # long dense decode: many splits
    (0, 72, 6, 2, 7, 700),      # causal prefill, one split
    (1, 33, 4, 1, 1, 4000),
    (2, 256, 48, 2, 1, 30000),  # 24 heads per KV head
])
def test_any_shape_dense_causal(rt, oracle, kind, hd, n_head, n_kvh, n_tok, base):
    note(f"any-shape dense kind={kind} hd={hd} n_head={n_head} n_tok={n_tok} base={base}")
    rng = np.random.default_rng(950 + kind + hd + n_tok)
    ctx = base + n_tok
    k = heads(rng, (ctx, n_kvh), hd=hd)
    v = heads(rng, (ctx, n_kvh), hd=hd)
    q = heads(rng, (n_tok, n_head), hd=hd)
    gate = rng.standard_normal((n_tok, n_head, hd)).astype(np.float32)
    kc, _ = quantize_on_gpu(rt, k, kind)
    vc, _ = quantize_on_gpu(rt, v, kind)
    kb, vb = oracle.encode(k, kind), oracle.encode(v, kind)
    dq, dg = rt.upload(q), rt.upload(gate)
    do = _out(rt, q.nbytes)
    scale = 1.0 / np.sqrt(hd)
    assert rt.lib.q4_hip_qsa_decode_n(dq, kc, vc, dg, do, n_head, n_kvh, hd, n_tok, base, ctx,
                                      scale, kind)
    rt.sync()
    got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
    want = oracle.attn(q, kb, vb, kind, n_head, n_kvh, hd, n_tok, gate=gate, kv_base=base,
                       max_kv=ctx, threads=8)
    assert_attn_close(got, want, what=f"dense hd={hd} gqa={n_head // n_kvh}")
    if n_tok == 1:  # q4_hip_qsa_decode: the same call by KV length
        do2 = _out(rt, q.nbytes)
        assert rt.lib.q4_hip_qsa_decode(dq, kc, vc, dg, do2, n_head, n_kvh, hd, base + 1, ctx,
                                        scale, kind)
        rt.sync()
        assert np.array_equal(rt.download(do2, q.nbytes, np.float32).reshape(q.shape), got)
        rt.free(do2)
    for p in (dq, dg, do, kc, vc):
        rt.free(p)


@pytest.mark.parametrize("kind,hd,n_head,n_kvh", [(1, 80, 16, 2), (0, 48, 40, 2),
                                                 (2, 64, 36, 2)])
def test_any_shape_step_and_batch(rt, oracle, kind, hd, n_head, n_kvh):
    """q4_hip_qsa_step_batch (append, then attention) and
    q4_hip_qsa_decode_batch over sequences of different lengths, dense and
    indexed; the appended rows are byte-exact."""
    note(f"any-shape step/batch kind={kind} hd={hd} n_head={n_head}")
    rng = np.random.default_rng(990 + kind + hd)
    n_seq, ctx = 4, 6000
    bpt = q4kv.token_bytes(kind, n_kvh, hd)
    lib = rt.lib
    items, owned = [], []
    steps = (q4kv.StepDesc * n_seq)()
    for s in range(n_seq):
        pos = [5999, 70, 3000, 1][s]
        k, v = heads(rng, (ctx, n_kvh), hd=hd), heads(rng, (ctx, n_kvh), hd=hd)
        kn, vn = heads(rng, (n_kvh,), hd=hd), heads(rng, (n_kvh,), hd=hd)
        k[pos], v[pos] = kn, vn
        q = heads(rng, (1, n_head), hd=hd)
        dense = s % 2 == 1
        sel = None if dense else _lists(rng, 1, n_kvh, 700, ctx, pad=11)
        if sel is not None:
            sel[0, :, 0] = pos  # the new token is listed
        kb, vb = oracle.encode(k, kind), oracle.encode(v, kind)
        # caches holding everything but the new token's row
        kc0, vc0 = kb.copy(), vb.copy()
        kc0[pos * bpt:(pos + 1) * bpt] = 0
        vc0[pos * bpt:(pos + 1) * bpt] = 0
        dkc, dvc = rt.upload(kc0), rt.upload(vc0)
        dkn, dvn, dq = rt.upload(kn), rt.upload(vn), rt.upload(q)
        do = _out(rt, q.nbytes)
        di = None if dense else rt.upload(sel.ravel())
        n_sel = pos + 1 if dense else 700
        seq = q4kv.SeqDesc(dkc, dvc, dq, None, do, di, n_sel, 0 if dense else 700, ctx, 0)
        steps[s] = q4kv.StepDesc(seq, dkn, dvn, pos)
        owned += [p for p in (dkc, dvc, dkn, dvn, dq, do, di) if p]
        items.append(dict(pos=pos, q=q, kb=kb, vb=vb, sel=sel, do=do, dkc=dkc, dvc=dvc,
                          seq=seq, dense=dense))
    dd = rt.alloc(ctypes.sizeof(steps))
    assert lib.q4_hip_h2d(dd, ctypes.addressof(steps), ctypes.sizeof(steps))
    scale = 1.0 / np.sqrt(hd)
    assert lib.q4_hip_qsa_step_batch(dd, n_seq, n_head, n_kvh, hd, scale, kind, 6000)
    rt.sync()
    outs = []
    for it in items:
        assert np.array_equal(rt.download(it["dkc"], it["kb"].size), it["kb"])
        assert np.array_equal(rt.download(it["dvc"], it["vb"].size), it["vb"])
        got = rt.download(it["do"], it["q"].nbytes, np.float32).reshape(it["q"].shape)
        outs.append(got)
        if it["dense"]:
            want = oracle.attn(it["q"], it["kb"], it["vb"], kind, n_head, n_kvh, hd, 1,
                               kv_base=it["pos"], max_kv=ctx)
        else:
            want = oracle.attn(it["q"], it["kb"], it["vb"], kind, n_head, n_kvh, hd, 1,
                               idx=it["sel"].ravel(), width=700, tok_stride=n_kvh * 700,
                               kvh_stride=700, max_kv=ctx)
        assert_attn_close(got, want, what=f"step seq pos={it['pos']}")
    # the same sequences through the batch entry point (caches now appended)
    seqs = (q4kv.SeqDesc * n_seq)(*[it["seq"] for it in items])
    for it in items:
        rt.h2d(it["do"], np.full(it["q"].size, np.nan, np.float32))
    ds = rt.alloc(ctypes.sizeof(seqs))
    assert lib.q4_hip_h2d(ds, ctypes.addressof(seqs), ctypes.sizeof(seqs))
    assert lib.q4_hip_qsa_decode_batch(ds, n_seq, n_head, n_kvh, hd, scale, kind, 6000)
    rt.sync()
    for it, o in zip(items, outs):
        got = rt.download(it["do"], it["q"].nbytes, np.float32).reshape(it["q"].shape)
        assert np.array_equal(got, o)
    for p in owned + [dd, ds]:
        rt.free(p)


def test_any_shape_rejections(rt):
    """q8_0 rows are 32-element blocks: hd must be a multiple of 32 there;
    hd > 256 and n_head not a multiple of n_kvh stay refused."""
    note("any-shape rejections")
    buf = rt.alloc(1 << 16)
    lib = rt.lib
    assert not lib.q4_hip_qsa_decode_n(buf, buf, buf, buf, buf, 4, 1, 80, 1, 0, 8, 0.1, 2)
    assert not lib.q4_hip_qsa_decode_n(buf, buf, buf, buf, buf, 4, 1, 288, 1, 0, 8, 0.1, 1)
    assert not lib.q4_hip_qsa_decode_n(buf, buf, buf, buf, buf, 6, 4, 64, 1, 0, 8, 0.1, 1)
    rt.free(buf)


@pytest.mark.parametrize("kind,n_head", [(1, 16), (1, 24), (0, 16), (0, 24)])
def test_wide_prefill_multi_pass(rt, oracle, kind, n_head):
    """f16 / f32 caches at hd 256 with enough items that each split streams
    several passes per wave (the online softmax rescales across passes):
    600 queries x 2 KV heads over 2051-entry lists, sampled rows against the
    oracle, plus dense causal prefill over the same cache."""
    note(f"wide prefill multi-pass kind={kind} n_head={n_head}")
    rng = np.random.default_rng(1300 + kind + n_head)
    n_kvh, hd, n_tok, base = 2, 256, 600, 3000
    ctx = base + n_tok
    k, v = heads(rng, (ctx, n_kvh)), heads(rng, (ctx, n_kvh))
    q = heads(rng, (n_tok, n_head))
    gate = rng.standard_normal((n_tok, n_head, hd)).astype(np.float32)
    kc, _ = quantize_on_gpu(rt, k, kind)
    vc, _ = quantize_on_gpu(rt, v, kind)
    kb, vb = oracle.encode(k, kind), oracle.encode(v, kind)
    width = 2051
    sel = _lists(rng, n_tok, n_kvh, width, ctx, pad=0)
    sel[::5, :, -100:] = -1  # some ragged lists
    got = gpu_idx_kv(rt, q, kc, vc, kind, n_head, n_kvh, hd, sel.ravel(), width,
                     n_kvh * width, width, ctx, gate=gate)
    ts = np.unique(np.concatenate([[0, n_tok - 1], rng.choice(n_tok, 40, replace=False)]))
    want = oracle.attn(q[ts], kb, vb, kind, n_head, n_kvh, hd, len(ts), gate=gate[ts],
                       idx=sel[ts].ravel(), width=width, tok_stride=n_kvh * width,
                       kvh_stride=width, max_kv=ctx, threads=8)
    assert_attn_close(got[ts], want, what=f"wide prefill kind={kind} n_head={n_head}")
    assert np.all(np.isfinite(got))
    dq, dg = rt.upload(q), rt.upload(gate)
    do = _out(rt, q.nbytes)
    assert rt.lib.q4_hip_qsa_decode_n(dq, kc, vc, dg, do, n_head, n_kvh, hd, n_tok, base, ctx,
                                      1.0 / 16, kind)
    rt.sync()
    got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
    # dense causal rows: token t sees 0 .. base + t; check the sampled rows
    for t in ts[:8]:
        w1 = oracle.attn(q[t:t + 1], kb, vb, kind, n_head, n_kvh, hd, 1, gate=gate[t:t + 1],
                         kv_base=base + int(t), max_kv=ctx)
        assert_attn_close(got[t:t + 1], w1, what=f"dense prefill row {t}")
    for p in (dq, dg, do, kc, vc):
        rt.free(p)


@pytest.mark.parametrize("kind,n_head,n_tok,off", [(2, 16, 2, 2), (2, 24, 2, 2), (1, 16, 2, 2),
                                                  (1, 24, 2, 2), (0, 16, 2, 4), (2, 16, 600, 2)])
def test_unaligned_caches(rt, oracle, kind, n_head, n_tok, off):
    """Caches that are not 16-byte aligned (base + off bytes) take kernels that
    read them in smaller pieces; results as for aligned caches. The 600-token
    q8_0 case is prefill-sized (otherwise the band and slab kernels)."""
    note(f"unaligned caches kind={kind} n_head={n_head} n_tok={n_tok} off={off}")
    rng = np.random.default_rng(1400 + kind + n_head + n_tok)
    n_kvh, hd, ctx, width = 2, 256, 5000, 2051
    k, v = heads(rng, (ctx, n_kvh)), heads(rng, (ctx, n_kvh))
    q = heads(rng, (n_tok, n_head))
    gate = rng.standard_normal((n_tok, n_head, hd)).astype(np.float32)
    kb, vb = oracle.encode(k, kind), oracle.encode(v, kind)
    kbuf, vbuf = rt.alloc(kb.nbytes + 64), rt.alloc(vb.nbytes + 64)
    rt.h2d(kbuf + off, kb)
    rt.h2d(vbuf + off, vb)
    sel = _lists(rng, n_tok, n_kvh, width, ctx, pad=20)
    got = gpu_idx_kv(rt, q, kbuf + off, vbuf + off, kind, n_head, n_kvh, hd, sel.ravel(),
                     width, n_kvh * width, width, ctx, gate=gate)
    ts = np.arange(n_tok) if n_tok <= 8 else np.unique(
        np.concatenate([[0, n_tok - 1], rng.choice(n_tok, 30, replace=False)]))
    want = oracle.attn(q[ts], kb, vb, kind, n_head, n_kvh, hd, len(ts), gate=gate[ts],
                       idx=sel[ts].ravel(), width=width, tok_stride=n_kvh * width,
                       kvh_stride=width, max_kv=ctx, threads=8)
    assert_attn_close(got[ts], want, what=f"unaligned kind={kind} n_head={n_head}")
    rt.free(kbuf)
    rt.free(vbuf)
