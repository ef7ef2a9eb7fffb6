"""Seeded randomized sweep of q4_hip_qsa_step_batch (the decode step: append
the token's K/V rows, then attend) against the two launches it stands for
(q4_hip_kv_append_batch, then q4_hip_qsa_decode_batch): cache bytes and
outputs bit-identical, and outputs within 2e-3 + 1e-3*|ref| of the oracle
over the appended cache. Per case: cache width, head_dim, KV heads, query
heads per KV head (fused and unfused shapes), item count; per item: its
position (the last cache row included), dense or listed, and the new
position listed zero, one or two times among the list shapes of the
attention sweep."""
import ctypes

import numpy as np
import pytest

import q4kv
from gpu_util import note
from synth import assert_attn_close, heads
from test_gpu_attn_sweep import _list

pytestmark = pytest.mark.gpu

N_CASES = 40


def _case(seed):
    rng = np.random.default_rng(70000 + seed)
    kind = int(rng.choice([0, 1, 2, 2]))
    hd = 256 if (kind == 2 or rng.random() < 0.7) else int(rng.choice([64, 80, 96, 200]))
    if kind == 2 and rng.random() < 0.2:
        hd = int(rng.choice([64, 128]))
    n_kvh = int(rng.choice([1, 2, 2, 3]))
    gqa = int(rng.choice([1, 4, 8, 8, 12, 16, 20]))
    n_seq = int(rng.choice([1, 3, 12, 20]))
    ctx = int(rng.integers(1200, 5000))
    width = int(rng.choice([17, 129, 700, 2051]))
    return rng, dict(kind=kind, hd=hd, n_kvh=n_kvh, n_head=gqa * n_kvh, n_seq=n_seq, ctx=ctx,
                     width=width)


def _run(rt, items, c, fused):
    kind, hd, n_kvh, n_head, ctx = c["kind"], c["hd"], c["n_kvh"], c["n_head"], c["ctx"]
    bpt = q4kv.token_bytes(kind, n_kvh, hd)
    n = len(items)
    steps, seqs, apps = (q4kv.StepDesc * n)(), (q4kv.SeqDesc * n)(), (q4kv.AppendDesc * n)()
    owned, ptrs = [], []
    for s, it in enumerate(items):
        kc, vc = rt.upload(it["kc"]), rt.upload(it["vc"])
        dkn, dvn, dq = rt.upload(it["kn"]), rt.upload(it["vn"]), rt.upload(it["q"])
        do = rt.alloc(it["q"].nbytes)
        rt.h2d(do, np.full(it["q"].size, np.nan, np.float32))
        di = None if it["sel"] is None else rt.upload(it["sel"])
        n_sel = it["pos"] + 1 if it["sel"] is None else c["width"]
        stride = 0 if it["sel"] is None else c["width"]
        seqs[s] = q4kv.SeqDesc(kc, vc, dq, None, do, di, n_sel, stride, ctx, 0)
        steps[s] = q4kv.StepDesc(seqs[s], dkn, dvn, it["pos"])
        apps[s] = q4kv.AppendDesc(kc, vc, dkn, dvn, it["pos"], 0)
        owned += [p for p in (kc, vc, dkn, dvn, dq, do, di) if p]
        ptrs.append((kc, vc, do))
    max_n = max(c["width"], max(it["pos"] + 1 for it in items))
    lib = rt.lib
    if fused:
        dd = rt.alloc(ctypes.sizeof(steps))
        owned.append(dd)
        assert lib.q4_hip_h2d(dd, ctypes.addressof(steps), ctypes.sizeof(steps))
        assert lib.q4_hip_qsa_step_batch(dd, n, n_head, n_kvh, hd, 1.0 / np.sqrt(hd), kind, max_n)
    else:
        da, ds = rt.alloc(ctypes.sizeof(apps)), rt.alloc(ctypes.sizeof(seqs))
        owned += [da, ds]
        assert lib.q4_hip_h2d(da, ctypes.addressof(apps), ctypes.sizeof(apps))
        assert lib.q4_hip_h2d(ds, ctypes.addressof(seqs), ctypes.sizeof(seqs))
        assert lib.q4_hip_kv_append_batch(da, n, n_kvh * hd, bpt, kind)
        assert lib.q4_hip_qsa_decode_batch(ds, n, n_head, n_kvh, hd, 1.0 / np.sqrt(hd), kind,
                                           max_n)
    rt.sync()
    res = [(rt.download(kc, it["kc"].nbytes), rt.download(vc, it["vc"].nbytes),
            rt.download(do, it["q"].nbytes, np.float32).reshape(it["q"].shape))
           for (kc, vc, do), it in zip(ptrs, items)]
    for p in owned:
        rt.free(p)
    return res


@pytest.mark.parametrize("seed", range(N_CASES))
def test_step_random_case(rt, oracle, seed):
    rng, c = _case(seed)
    kind, hd, n_kvh, n_head, ctx, width = (c["kind"], c["hd"], c["n_kvh"], c["n_head"], c["ctx"],
                                           c["width"])
    note(f"step sweep seed={seed} {c}")
    items = []
    for s in range(c["n_seq"]):
        pos = ctx - 1 if s == 0 else int(rng.integers(0, ctx))
        k, v = heads(rng, (ctx, n_kvh), hd=hd), heads(rng, (ctx, n_kvh), hd=hd)
        kn, vn = heads(rng, (n_kvh,), hd=hd), heads(rng, (n_kvh,), hd=hd)
        if rng.random() < 0.25:
            sel = None  # dense: positions 0 .. pos
        else:
            sel = np.stack([_list(rng, width, ctx, pos) for _ in range(n_kvh)])
            for _ in range(int(rng.integers(0, 3))):  # the new position, 0-2 times
                sel[:, int(rng.integers(0, width))] = pos
        items.append(dict(pos=pos, k=k, v=v, kn=kn, vn=vn, kc=oracle.encode(k, kind),
                          vc=oracle.encode(v, kind), q=heads(rng, (1, n_head), hd=hd), sel=sel))
    fused = _run(rt, items, c, True)
    twice = _run(rt, items, c, False)
    for s, it in enumerate(items):
        assert np.array_equal(fused[s][0], twice[s][0]), f"seed {seed} item {s}: K bytes"
        assert np.array_equal(fused[s][1], twice[s][1]), f"seed {seed} item {s}: V bytes"
        assert np.array_equal(fused[s][2], twice[s][2]), f"seed {seed} item {s}: outputs"
        k, v = it["k"].copy(), it["v"].copy()
        k[it["pos"]], v[it["pos"]] = it["kn"], it["vn"]
        kb, vb = oracle.encode(k, kind), oracle.encode(v, kind)
        assert np.array_equal(fused[s][0], kb), f"seed {seed} item {s}: appended K row"
        if it["sel"] is None:
            want = oracle.attn(it["q"], kb, vb, kind, n_head, n_kvh, hd, 1, kv_base=it["pos"],
                               max_kv=ctx)
        else:
            want = oracle.attn(it["q"], kb, vb, kind, n_head, n_kvh, hd, 1,
                               idx=it["sel"].ravel(), width=width, tok_stride=n_kvh * width,
                               kvh_stride=width, max_kv=ctx)
        assert_attn_close(fused[s][2], want, what=f"step sweep seed {seed} item {s}")
