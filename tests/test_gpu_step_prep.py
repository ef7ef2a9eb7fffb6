"""q4_hip_qsa_step_prep_batch -- query/key RMSNorm + RoPE, K/V append and
attention in one launch (plus the merge) -- against the calls it stands for
(q4_hip_qsa_q_prep, q4_hip_qsa_k_prep, q4_hip_qsa_step_batch) on the same
inputs: cache bytes, gate copy and outputs bit-identical; outputs against
the oracle's attention over the prepared query and key."""
import ctypes

import numpy as np
import pytest

import q4kv
from gpu_util import note
from synth import assert_attn_close, heads, selection

pytestmark = pytest.mark.gpu

N_HEAD, N_KVH, HD = 16, 2, 256
N_ROT, BASE, EPS = 64, 1.0e7, 1.0e-6


def _items(rng, oracle, n_seq, ctx, width, n_head=N_HEAD):
    items = []
    for s in range(n_seq):
        pos = ctx - 1 - 97 * s
        k, v = heads(rng, (ctx, N_KVH)), heads(rng, (ctx, N_KVH))
        k[pos:] = 0.0
        v[pos:] = 0.0
        if width:   # short lists that end at the new position
            sel = np.stack([np.append(np.sort(rng.choice(pos, width - 1, replace=False)), pos)
                            for _ in range(N_KVH)])
        else:
            sel = np.stack([selection(rng, pos) for _ in range(N_KVH)])
        q = heads(rng, (n_head,))
        gate = rng.standard_normal((n_head, HD)).astype(np.float32)
        items.append(dict(pos=pos, kc=oracle.encode(k, q4kv.KV_Q8),
                          vc=oracle.encode(v, q4kv.KV_Q8), k=k, v=v,
                          kn=heads(rng, (N_KVH,)) * 3, vn=heads(rng, (N_KVH,)),
                          qg=np.concatenate([q, gate], axis=-1).astype(np.float32),
                          sel=sel.astype(np.int32),
                          wq=(1 + 0.2 * rng.standard_normal(HD)).astype(np.float32),
                          wk=(1 + 0.2 * rng.standard_normal(HD)).astype(np.float32)))
    return items


def _run(rt, items, ctx, fused):
    lib = rt.lib
    before = set(rt._owned)
    n = len(items)
    nh = items[0]["qg"].shape[0]
    steps = (q4kv.StepDesc * n)()
    preps = (q4kv.PrepStepDesc * n)()
    keep = []
    for s, it in enumerate(items):
        kc, vc = rt.upload(it["kc"]), rt.upload(it["vc"])
        dqg, dkn, dvn = rt.upload(it["qg"]), rt.upload(it["kn"]), rt.upload(it["vn"])
        dwq, dwk = rt.upload(it["wq"]), rt.upload(it["wk"])
        dg = rt.upload(np.full((nh, HD), np.nan, np.float32))
        do = rt.upload(np.full((nh, HD), np.nan, np.float32))
        di = rt.upload(it["sel"])
        w = it["sel"].shape[-1]
        if fused:
            seq = q4kv.SeqDesc(kc, vc, dqg, dg, do, di, w, w, ctx, 0)
            preps[s] = q4kv.PrepStepDesc(q4kv.StepDesc(seq, dkn, dvn, it["pos"]), dwq, dwk)
        else:
            dq = rt.alloc(nh * HD * 4)
            dk = rt.upload(it["kn"])                       # k_prep works in place
            assert lib.q4_hip_qsa_q_prep(dqg, dwq, dq, dg, nh, HD, N_ROT, it["pos"], BASE, EPS)
            assert lib.q4_hip_qsa_k_prep(dk, dwk, N_KVH, HD, N_ROT, it["pos"], BASE, EPS)
            seq = q4kv.SeqDesc(kc, vc, dq, dg, do, di, w, w, ctx, 0)
            steps[s] = q4kv.StepDesc(seq, dk, dvn, it["pos"])
        keep.append((kc, vc, dg, do, dkn))
    max_n = max(it["sel"].shape[-1] for it in items)
    arr = preps if fused else steps
    dd = rt.alloc(ctypes.sizeof(arr))
    assert lib.q4_hip_h2d(dd, ctypes.addressof(arr), ctypes.sizeof(arr))
    if fused:
        assert lib.q4_hip_qsa_step_prep_batch(dd, n, nh, N_KVH, HD, 1.0 / 16, q4kv.KV_Q8,
                                              max_n, N_ROT, BASE, EPS)
    else:
        assert lib.q4_hip_qsa_step_batch(dd, n, nh, N_KVH, HD, 1.0 / 16, q4kv.KV_Q8, max_n)
    rt.sync()
    res = []
    for (kc, vc, dg, do, dkn), it in zip(keep, items):
        res.append(dict(kc=rt.download(kc, it["kc"].nbytes, np.uint8),
                        vc=rt.download(vc, it["vc"].nbytes, np.uint8),
                        g=rt.download(dg, nh * HD * 4, np.float32),
                        out=rt.download(do, nh * HD * 4, np.float32).reshape(1, nh, HD),
                        kn=rt.download(dkn, it["kn"].nbytes, np.float32)))
    for p in [p for p in rt._owned if p not in before]:
        rt.free(p)
    return res


# 32 sequences: five chunks per workgroup, the double-buffered instance
# 24 heads over 2 KV heads (12 per KV head): the production layout, two head
# groups per workgroup
@pytest.mark.parametrize("n_seq,ctx,width,n_head", [(12, 16384, 0, 16), (3, 4096, 40, 16),
                                                     (32, 16384, 0, 16), (12, 16384, 0, 24),
                                                     (3, 4096, 40, 24)])
def test_step_prep_matches_prep_then_step(rt, oracle, n_seq, ctx, width, n_head):
    """12 layers of 2051-entry lists (split-KV with a merge), and 40-entry
    lists (one split: the kernel's own epilogue applies the gate)."""
    note(f"step_prep n_seq={n_seq} width={width} n_head={n_head}")
    rng = np.random.default_rng(910 + n_seq + n_head)
    items = _items(rng, oracle, n_seq, ctx, width, n_head)
    a = _run(rt, items, ctx, fused=True)
    b = _run(rt, items, ctx, fused=False)
    for s, it in enumerate(items):
        for key in ("kc", "vc", "g", "out"):
            assert np.array_equal(a[s][key].view(np.uint8), b[s][key].view(np.uint8)), (s, key)
        assert np.array_equal(a[s]["kn"], it["kn"].ravel())     # raw K not modified
        assert np.array_equal(a[s]["g"].reshape(n_head, HD), it["qg"][:, HD:])
        # against the oracle: attention of the prepared query over the cache
        # holding the prepared, quantised key
        p = it["pos"]
        qp = oracle.qsa_prep(it["qg"][None, :, :HD], it["wq"], N_ROT, p, BASE, EPS)
        kp = oracle.qsa_prep(it["kn"][None], it["wk"], N_ROT, p, BASE, EPS)[0]
        k, v = it["k"].copy(), it["v"].copy()
        k[p], v[p] = kp, it["vn"]
        kq, vq = oracle.encode(k, q4kv.KV_Q8), oracle.encode(v, q4kv.KV_Q8)
        w = it["sel"].shape[-1]
        want = oracle.attn(qp, kq, vq, q4kv.KV_Q8, n_head, N_KVH, HD, 1,
                           gate=it["qg"][None, :, HD:], idx=it["sel"], width=w,
                           tok_stride=N_KVH * w, kvh_stride=w, max_kv=ctx, scale=1.0 / 16)
        assert_attn_close(a[s]["out"], want, what=f"step_prep item {s}")
