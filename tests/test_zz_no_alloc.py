"""q4_hip_qsa_step_batch_noalloc -- the decode step whose split partials live
in the library's static device scratch -- against q4_hip_qsa_step_batch on
the same inputs: appended cache bytes and outputs bit-identical (same split
division), outputs within the attention bar of the oracle, on two calls in a
row (the second smaller, so stale scratch from the first must not leak in),
and the rejection of a call whose partials exceed the scratch."""
import ctypes

import numpy as np
import pytest

import q4kv
from gpu_util import note
from synth import assert_attn_close, heads, selection

pytestmark = pytest.mark.gpu

N_HEAD, N_KVH, HD = 16, 2, 256


def _items(rng, oracle, n_seq, ctx, kind):
    out = []
    for s in range(n_seq):
        pos = ctx - 1 - 211 * s
        k, v = heads(rng, (ctx, N_KVH)), heads(rng, (ctx, N_KVH))
        k[pos:] = 0.0
        v[pos:] = 0.0
        out.append(dict(pos=pos, k=k, v=v, kc=oracle.encode(k, kind), vc=oracle.encode(v, kind),
                        kn=heads(rng, (N_KVH,)), vn=heads(rng, (N_KVH,)),
                        q=heads(rng, (1, N_HEAD)),
                        sel=np.stack([selection(rng, pos) for _ in range(N_KVH)])))
    return out


def _step(rt, items, ctx, kind, entry):
    before = set(rt._owned)
    n_seq = len(items)
    steps = (q4kv.StepDesc * n_seq)()
    ptrs = []
    for s, it in enumerate(items):
        kc, vc = rt.upload(it["kc"]), rt.upload(it["vc"])
        dkn, dvn, dq = rt.upload(it["kn"]), rt.upload(it["vn"]), rt.upload(it["q"])
        do = rt.alloc(it["q"].nbytes)
        rt.h2d(do, np.full(it["q"].size, np.nan, np.float32))
        di = rt.upload(it["sel"])
        w = it["sel"].shape[-1]
        steps[s] = q4kv.StepDesc(q4kv.SeqDesc(kc, vc, dq, None, do, di, w, w, ctx, 0),
                                 dkn, dvn, it["pos"])
        ptrs.append((kc, vc, do))
    dd = rt.alloc(ctypes.sizeof(steps))
    assert rt.lib.q4_hip_h2d(dd, ctypes.addressof(steps), ctypes.sizeof(steps))
    max_n = max(it["sel"].shape[-1] for it in items)
    assert getattr(rt.lib, entry)(dd, n_seq, N_HEAD, N_KVH, HD, 1.0 / 16, kind, max_n), entry
    rt.sync()
    res = []
    for (kc, vc, do), it in zip(ptrs, items):
        res.append((rt.download(kc, it["kc"].nbytes), rt.download(vc, it["vc"].nbytes),
                    rt.download(do, it["q"].nbytes, np.float32).reshape(it["q"].shape)))
    for p in [p for p in rt._owned if p not in before]:
        rt.free(p)
    return res


@pytest.mark.parametrize("kind", [q4kv.KV_Q8, q4kv.KV_F16, q4kv.KV_F32])
def test_noalloc_step_matches_step_batch_twice(rt, oracle, kind):
    ctx = 8192
    for call, n_seq in enumerate((12, 3)):
        note(f"noalloc step kind {kind} call {call} n_seq {n_seq}")
        rng = np.random.default_rng(1300 + 10 * kind + call)
        items = _items(rng, oracle, n_seq, ctx, kind)
        ref = _step(rt, items, ctx, kind, "q4_hip_qsa_step_batch")
        got = _step(rt, items, ctx, kind, "q4_hip_qsa_step_batch_noalloc")
        for s, it in enumerate(items):
            assert np.array_equal(got[s][0], ref[s][0]), f"call {call} item {s}: K bytes differ"
            assert np.array_equal(got[s][1], ref[s][1]), f"call {call} item {s}: V bytes differ"
            assert np.array_equal(got[s][2], ref[s][2]), f"call {call} item {s}: outputs differ"
            p = it["pos"]
            k, v = it["k"].copy(), it["v"].copy()
            k[p], v[p] = it["kn"], it["vn"]
            w = it["sel"].shape[-1]
            want = oracle.attn(it["q"], oracle.encode(k, kind), oracle.encode(v, kind), kind,
                               N_HEAD, N_KVH, HD, 1, idx=it["sel"], width=w,
                               tok_stride=N_KVH * w, kvh_stride=w, max_kv=ctx, scale=1.0 / 16)
            assert_attn_close(got[s][2], want, what=f"noalloc call {call} item {s}")


def test_noalloc_rejects_partials_beyond_scratch(rt):
    """255 sequences x 2 KV heads with 16 query heads per KV head would need
    510 x 2 splits x 16 x 258 floats (> 4M): refused before any launch."""
    note("noalloc rejection")
    dummy = rt.alloc(256)
    assert not rt.lib.q4_hip_qsa_step_batch_noalloc(dummy, 255, 32, 2, 256, 1.0 / 16,
                                                    q4kv.KV_Q8, 2051)
    rt.sync()
