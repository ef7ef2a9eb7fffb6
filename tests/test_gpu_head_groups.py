"""Decode launches with 9-16 query heads per KV head on a q8_0 / head_dim 256
cache run the chunk kernel in two groups of query heads (grid.z: heads 0-7,
then the rest) over the same rows. Every entry point family against the fp64
oracle (|err| <= 2e-3 and <= 1e-3|ref| where |ref| >= 1), at head counts
whose second group is full, partial and a single head, for one and several
tokens, gated and not; and the held append riding in that launch. Batch
descriptors at these head counts (which keep the slab kernel) are checked
beside them."""
import ctypes

import numpy as np
import pytest

import q4kv
from gpu_util import note, quantize_on_gpu
from synth import WIDTH, assert_attn_close, heads, selection

pytestmark = pytest.mark.gpu

HD, N_KVH, CTX = 256, 2, 6000


def _setup(rt, oracle, rng):
    k, v = heads(rng, (CTX, N_KVH)), heads(rng, (CTX, N_KVH))
    kc, _ = quantize_on_gpu(rt, k, 2)
    vc, _ = quantize_on_gpu(rt, v, 2)
    return k, v, kc, vc, oracle.quant_q8(k), oracle.quant_q8(v)


@pytest.mark.parametrize("gqa", [9, 12, 13, 16])
@pytest.mark.parametrize("n_tok", [1, 3])
def test_head_groups_match_oracle(rt, oracle, gqa, n_tok):
    n_head = gqa * N_KVH
    note(f"head groups gqa={gqa} n_tok={n_tok}")
    rng = np.random.default_rng(8100 + 10 * gqa + n_tok)
    _, _, kc, vc, kb, vb = _setup(rt, oracle, rng)
    lib = rt.lib
    q = heads(rng, (n_tok, n_head))
    gate = rng.standard_normal((n_tok, n_head, HD)).astype(np.float32)
    pos0 = CTX - n_tok
    # per-KV-head lists (q4_hip_qsa_decode_idx_kv), no gate
    sel = np.stack([np.stack([selection(rng, pos0 + t) for _ in range(N_KVH)])
                    for t in range(n_tok)]).astype(np.int32)
    dq, di = rt.upload(q), rt.upload(sel)
    do = rt.alloc(q.nbytes)
    assert lib.q4_hip_qsa_decode_idx_kv(dq, kc, vc, None, do, di, WIDTH, N_KVH * WIDTH, WIDTH,
                                        n_head, N_KVH, HD, n_tok, CTX, 1.0 / 16, 2)
    rt.sync()
    got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
    want = oracle.attn(q, kb, vb, 2, n_head, N_KVH, HD, n_tok, idx=sel.ravel(), width=WIDTH,
                       tok_stride=N_KVH * WIDTH, kvh_stride=WIDTH, max_kv=CTX, scale=1.0 / 16)
    assert_attn_close(got, want, what=f"idx_kv gqa {gqa}")
    # one list shared by the KV heads, gated (q4_hip_qsa_decode_idx)
    shared = np.ascontiguousarray(sel[:, 0, :])
    ds, dg = rt.upload(shared), rt.upload(gate)
    assert lib.q4_hip_qsa_decode_idx(dq, kc, vc, dg, do, ds, WIDTH, n_head, N_KVH, HD, n_tok,
                                     CTX, 1.0 / 16, 2)
    rt.sync()
    got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
    want = oracle.attn(q, kb, vb, 2, n_head, N_KVH, HD, n_tok, gate=gate,
                       idx=np.repeat(shared, N_KVH, axis=0).ravel(), width=WIDTH,
                       tok_stride=N_KVH * WIDTH, kvh_stride=WIDTH, max_kv=CTX, scale=1.0 / 16)
    assert_attn_close(got, want, what=f"idx gated gqa {gqa}")
    # dense causal decode over the cache prefix (q4_hip_qsa_decode_n)
    assert lib.q4_hip_qsa_decode_n(dq, kc, vc, dg, do, n_head, N_KVH, HD, n_tok, pos0, CTX,
                                   1.0 / 16, 2)
    rt.sync()
    got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
    want = oracle.attn(q, kb, vb, 2, n_head, N_KVH, HD, n_tok, gate=gate, kv_base=pos0,
                       max_kv=CTX, scale=1.0 / 16)
    assert_attn_close(got, want, what=f"dense gqa {gqa}")
    for p in (kc, vc, dq, di, do, ds, dg):
        rt.free(p)


def test_head_groups_with_held_append(rt, oracle):
    """append_d then decode_idx_kv at 13 query heads per KV head: the append
    rides in the head-grouped launch (written once, by group 0) and the new
    position is seen by both groups."""
    note("head groups + held append")
    rng = np.random.default_rng(8200)
    gqa, n_head = 13, 13 * N_KVH
    k, v, kc, vc, kb, vb = _setup(rt, oracle, rng)
    pos = CTX - 1
    bpt = N_KVH * 272
    kb, vb = kb.copy(), vb.copy()
    kn, vn = heads(rng, (N_KVH,)), heads(rng, (N_KVH,))
    dk, dv = rt.upload(kn), rt.upload(vn)
    q = heads(rng, (1, n_head))
    sel = np.stack([selection(rng, pos) for _ in range(N_KVH)]).astype(np.int32)
    dq, di = rt.upload(q), rt.upload(sel)
    do = rt.alloc(q.nbytes)
    rt.lib.q4_hip_pos_push(pos)
    assert rt.lib.q4_hip_kv_append_d(kc, vc, dk, dv, N_KVH * HD, bpt, 2)
    assert rt.lib.q4_hip_qsa_decode_idx_kv(dq, kc, vc, None, do, di, WIDTH, N_KVH * WIDTH, WIDTH,
                                           n_head, N_KVH, HD, 1, CTX, 1.0 / 16, 2)
    rt.sync()
    oracle.lib.orc_kv_append(kb.ctypes.data, vb.ctypes.data, kn.ctypes.data, vn.ctypes.data,
                             N_KVH * HD, bpt, 2, pos)
    assert np.array_equal(rt.download(kc, kb.size), kb), "K cache bytes"
    assert np.array_equal(rt.download(vc, vb.size), vb), "V cache bytes"
    got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
    want = oracle.attn(q, kb, vb, 2, n_head, N_KVH, HD, 1, idx=sel.ravel(), width=WIDTH,
                       tok_stride=N_KVH * WIDTH, kvh_stride=WIDTH, max_kv=CTX, scale=1.0 / 16)
    assert_attn_close(got, want, what="held append gqa 13")
    for p in (kc, vc, dk, dv, dq, di, do):
        rt.free(p)


@pytest.mark.parametrize("gqa", [9, 12, 16])
def test_head_groups_batch_descriptors(rt, oracle, gqa):
    """q4_hip_qsa_decode_batch of four sequences sharing the caches, two with
    per-KV-head lists and two with dense prefixes, gated."""
    n_head, n_seq = gqa * N_KVH, 4
    note(f"head groups batch gqa={gqa}")
    rng = np.random.default_rng(8300 + gqa)
    _, _, kc, vc, kb, vb = _setup(rt, oracle, rng)
    q = heads(rng, (n_seq, n_head))
    gate = rng.standard_normal((n_seq, n_head, HD)).astype(np.float32)
    descs = (q4kv.SeqDesc * n_seq)()
    owned, outs, want = [], [], []
    for t in range(n_seq):
        dq1, dg1 = rt.upload(q[t:t + 1]), rt.upload(gate[t:t + 1])
        do1 = rt.alloc(q[t].nbytes)
        owned += [dq1, dg1, do1]
        if t % 2:
            n_sel = CTX - 97 * t
            descs[t] = q4kv.SeqDesc(kc, vc, dq1, dg1, do1, None, n_sel, 0, CTX, 0)
            want.append(oracle.attn(q[t:t + 1], kb, vb, 2, n_head, N_KVH, HD, 1,
                                    gate=gate[t:t + 1], kv_base=n_sel - 1, max_kv=CTX,
                                    scale=1.0 / 16)[0])
        else:
            sel = np.stack([selection(rng, CTX - 1 - t) for _ in range(N_KVH)]).astype(np.int32)
            di1 = rt.upload(sel)
            owned.append(di1)
            descs[t] = q4kv.SeqDesc(kc, vc, dq1, dg1, do1, di1, WIDTH, WIDTH, CTX, 0)
            want.append(oracle.attn(q[t:t + 1], kb, vb, 2, n_head, N_KVH, HD, 1,
                                    gate=gate[t:t + 1], idx=sel.ravel(), width=WIDTH,
                                    tok_stride=N_KVH * WIDTH, kvh_stride=WIDTH, max_kv=CTX,
                                    scale=1.0 / 16)[0])
        outs.append(do1)
    dd = rt.alloc(ctypes.sizeof(descs))
    owned.append(dd)
    assert rt.lib.q4_hip_h2d(dd, ctypes.addressof(descs), ctypes.sizeof(descs))
    assert rt.lib.q4_hip_qsa_decode_batch(dd, n_seq, n_head, N_KVH, HD, 1.0 / 16, 2, CTX)
    rt.sync()
    got = np.stack([rt.download(o, q[0].nbytes, np.float32).reshape(n_head, HD) for o in outs])
    assert_attn_close(got, np.stack(want), what=f"batch gqa {gqa}")
    for p in owned + [kc, vc]:
        rt.free(p)
