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

N_KVH = 2


def _items(rng, oracle, n_seq, ctx, kind, n_head, hd):
    out = []
    for s in range(n_seq):
        pos = ctx - 1 - 211 * s
        k, v = heads(rng, (ctx, N_KVH), hd=hd), heads(rng, (ctx, N_KVH), hd=hd)
        k[pos:] = 0.0
        v[pos:] = 0.0
        out.append(dict(pos=pos, k=k, v=v, kc=oracle.encode(k, kind), vc=oracle.encode(v, kind),
                        kn=heads(rng, (N_KVH,), hd=hd), vn=heads(rng, (N_KVH,), hd=hd),
                        q=heads(rng, (1, n_head), hd=hd),
                        sel=np.stack([selection(rng, pos) for _ in range(N_KVH)])))
    return out


def _step(rt, items, ctx, kind, entry, n_head, hd):
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
    assert getattr(rt.lib, entry)(dd, n_seq, n_head, N_KVH, hd, 1.0 / 16, kind, max_n), entry
    rt.sync()
    res = []
    for (kc, vc, do), it in zip(ptrs, items):
        res.append((rt.download(kc, it["kc"].nbytes), rt.download(vc, it["vc"].nbytes),
                    rt.download(do, it["q"].nbytes, np.float32).reshape(it["q"].shape)))
    for p in [p for p in rt._owned if p not in before]:
        rt.free(p)
    return res


# (kind, query heads, head_dim): the fused step kernels (q8_0 chunk, f16,
# f32), the append launch + split kernel path (f16, hd 128: the generic MFMA
# kernel) and the general-shape kernel (24 query heads per KV head)
@pytest.mark.parametrize("kind,n_head,hd", [(q4kv.KV_Q8, 16, 256), (q4kv.KV_F16, 16, 256),
                                            (q4kv.KV_F32, 16, 256), (q4kv.KV_F16, 16, 128),
                                            (q4kv.KV_Q8, 48, 256)])
def test_noalloc_step_matches_step_batch_twice(rt, oracle, kind, n_head, hd):
    ctx = 8192
    for call, n_seq in enumerate((12, 3)):
        note(f"noalloc step kind {kind} heads {n_head} hd {hd} call {call} n_seq {n_seq}")
        rng = np.random.default_rng(1300 + 10 * kind + call + n_head + hd)
        items = _items(rng, oracle, n_seq, ctx, kind, n_head, hd)
        ref = _step(rt, items, ctx, kind, "q4_hip_qsa_step_batch", n_head, hd)
        got = _step(rt, items, ctx, kind, "q4_hip_qsa_step_batch_noalloc", n_head, hd)
        for s, it in enumerate(items):
            assert np.array_equal(got[s][0], ref[s][0]), f"call {call} item {s}: K bytes differ"
            assert np.array_equal(got[s][1], ref[s][1]), f"call {call} item {s}: V bytes differ"
            assert np.array_equal(got[s][2], ref[s][2]), f"call {call} item {s}: outputs differ"
            p = it["pos"]
            k, v = it["k"].copy(), it["v"].copy()
            k[p], v[p] = it["kn"], it["vn"]
            w = it["sel"].shape[-1]
            want = oracle.attn(it["q"], oracle.encode(k, kind), oracle.encode(v, kind), kind,
                               n_head, N_KVH, hd, 1, idx=it["sel"], width=w,
                               tok_stride=N_KVH * w, kvh_stride=w, max_kv=ctx, scale=1.0 / 16)
            assert_attn_close(got[s][2], want, what=f"noalloc call {call} item {s}")


def test_noalloc_rejects_partials_beyond_scratch(rt):
    """A call whose split partials exceed the 4M-float scratch is refused
    before any launch. The division is the step's: 16 query heads per KV
    head take the slab kernel, whose splits are ceil(512 / items) capped by
    the list's 128-entry passes (17 for 2051 entries); 255 sequences x 2 KV
    heads = 510 items -> 2 splits -> 510 x 2 x 16 x 258 = 4210560 floats."""
    note("noalloc rejection")
    n_seq, gqa, passes = 255, 16, (2051 + 127) // 128
    items = n_seq * N_KVH
    splits = min(-(-512 // items), passes)
    need = items * splits * gqa * 258
    assert need > 4 << 20, need  # the case is beyond the scratch by the formula
    dummy = rt.alloc(256)
    assert not rt.lib.q4_hip_qsa_step_batch_noalloc(dummy, n_seq, N_KVH * gqa, N_KVH, 256,
                                                    1.0 / 16, q4kv.KV_Q8, 2051)
    rt.sync()
