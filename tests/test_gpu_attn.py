"""QSA attention on the GPU vs the CPU oracle (double precision over the same
cache bytes): |got - ref| <= 2e-3 + 1e-3*|ref|, the north-star bar."""
import ctypes

import numpy as np
import pytest

import q4kv
from gpu_util import note, quantize_on_gpu
from synth import WIDTH, assert_attn_close, heads, selection

pytestmark = pytest.mark.gpu


def _out(rt, nbytes):
    p = rt.alloc(nbytes)
    rt.h2d(p, np.full(nbytes // 4, np.nan, np.float32))  # catch unwritten outputs
    return p


def gpu_idx_kv(rt, q, kc, vc, kind, n_head, n_kvh, hd, idx, width, tok_stride, kvh_stride,
               max_kv, gate=None):
    n_tok = q.shape[0]
    dq = rt.upload(q)
    dg = rt.upload(gate) if gate is not None else None
    di = rt.upload(idx)
    do = _out(rt, q.nbytes)
    assert rt.lib.q4_hip_qsa_decode_idx_kv(dq, kc, vc, dg, do, di, width, tok_stride,
                                           kvh_stride, n_head, n_kvh, hd, n_tok, max_kv,
                                           1.0 / np.sqrt(hd), kind)
    rt.sync()
    out = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
    for p in (dq, dg, di, do):
        if p:
            rt.free(p)
    return out


# ------------------------------------------------- reference known-answer test
def test_reference_qsa_check_port(rt, oracle):
    """src/q4_test.c:134-238: n_head 2, n_kvh 1, hd 32, n_tok 2, npos 4,
    deterministic inputs, q4_hip_qsa_decode_n for f32/f16/q8 with the
    reference's tolerances vs the unquantised reference, plus the strict bar
    vs the oracle over the stored cache values."""
    note("q4_test port")
    n_head, n_kvh, hd, n_tok, npos = 2, 1, 32, 2, 4
    i = np.arange(npos * hd)
    k = (((i * 17) % 11) * 0.05 - 0.2).astype(np.float32).reshape(npos, 1, hd)
    v = (((i * 13) % 9) * 0.07).astype(np.float32).reshape(npos, 1, hd)
    j = np.arange(n_tok * n_head * hd)
    q = (((j * 3) % 7) * 0.1).astype(np.float32).reshape(n_tok, n_head, hd)
    gate = (((j % 5) - 2) * 0.3).astype(np.float32).reshape(n_tok, n_head, hd)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    ref_unq = oracle.attn(q, k, v, 0, n_head, n_kvh, hd, n_tok, gate=gate, kv_base=0,
                          max_kv=npos, scale=scale)
    dq, dg = rt.upload(q), rt.upload(gate)
    do = _out(rt, q.nbytes)
    for kind, tol in ((0, 1e-3), (1, 2e-2), (2, 8e-2)):
        dk, _ = quantize_on_gpu(rt, k, kind)
        dv, _ = quantize_on_gpu(rt, v, kind)
        assert rt.lib.q4_hip_qsa_decode_n(dq, dk, dv, dg, do, n_head, n_kvh, hd, n_tok, 0,
                                          npos, float(scale), kind)
        rt.sync()
        got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
        assert np.abs(got - ref_unq).max() <= tol, kind
        want = oracle.attn(q, oracle.encode(k, kind), oracle.encode(v, kind), kind, n_head,
                           n_kvh, hd, n_tok, gate=gate, kv_base=0, max_kv=npos, scale=scale)
        assert_attn_close(got, want, what=f"kind {kind}")


def test_null_gate_rejected_by_reference_entry_points(rt):
    p = rt.alloc(4096)
    assert not rt.lib.q4_hip_qsa_decode_n(p, p, p, None, p, 2, 1, 32, 1, 0, 4, 0.17, 0)
    assert not rt.lib.q4_hip_qsa_decode_idx(p, p, p, None, p, p, 2, 2, 1, 32, 1, 4, 0.17, 0)
    assert not rt.lib.q4_hip_qsa_decode_n(p, p, p, p, p, 2, 1, 512, 1, 0, 4, 0.17, 0)


def test_entry_points_refuse_null_and_empty_arguments(rt):
    """The reference's error convention (src/q4_rocm.cu:20-28, 7253-7254):
    false, never a launch, for null buffers, zero counts and bad shapes; the
    output buffer stays untouched."""
    note("argument refusals")
    lib, p = rt.lib, rt.alloc(1 << 20)
    out = _out(rt, 4 * 16 * 256)
    dn = lib.q4_hip_qsa_decode_n
    assert not dn(None, p, p, p, out, 16, 2, 256, 1, 0, 8, 0.06, 2)   # q
    assert not dn(p, None, p, p, out, 16, 2, 256, 1, 0, 8, 0.06, 2)   # K cache
    assert not dn(p, p, None, p, out, 16, 2, 256, 1, 0, 8, 0.06, 2)   # V cache
    assert not dn(p, p, p, p, None, 16, 2, 256, 1, 0, 8, 0.06, 2)     # out
    assert not dn(p, p, p, p, out, 16, 2, 256, 0, 0, 8, 0.06, 2)      # n_tok 0
    assert not dn(p, p, p, p, out, 0, 2, 256, 1, 0, 8, 0.06, 2)       # n_head 0
    assert not dn(p, p, p, p, out, 16, 0, 256, 1, 0, 8, 0.06, 2)      # n_kvh 0
    assert not dn(p, p, p, p, out, 16, 2, 0, 1, 0, 8, 0.06, 2)        # hd 0
    assert not dn(p, p, p, p, out, 16, 3, 256, 1, 0, 8, 0.06, 2)      # n_head % n_kvh
    assert not dn(p, p, p, p, out, 16, 2, 256, 1, 0, 8, 0.06, 3)      # width kind
    assert not lib.q4_hip_qsa_decode(p, p, p, p, out, 16, 2, 256, 0, 8, 0.06, 2)  # n_kv 0
    ik = lib.q4_hip_qsa_decode_idx_kv
    assert not ik(p, p, p, None, out, None, 4, 8, 4, 16, 2, 256, 1, 8, 0.06, 2)  # idx
    assert not ik(p, p, p, None, out, p, 0, 8, 4, 16, 2, 256, 1, 8, 0.06, 2)     # width 0
    assert not ik(p, p, p, None, out, p, 4, 8, 4, 16, 2, 256, 0, 8, 0.06, 2)     # n_tok 0
    assert not lib.q4_hip_qsa_decode_batch(None, 1, 16, 2, 256, 0.06, 2, 8)
    assert not lib.q4_hip_qsa_decode_batch(p, 0, 16, 2, 256, 0.06, 2, 8)
    assert not lib.q4_hip_qsa_decode_batch(p, 1, 16, 2, 256, 0.06, 2, 0)
    assert not lib.q4_hip_qsa_step_batch(None, 1, 16, 2, 256, 0.06, 2, 8)
    assert not lib.q4_hip_qsa_step_batch(p, 0, 16, 2, 256, 0.06, 2, 8)
    rt.sync()
    assert np.isnan(rt.download(out, 4 * 16 * 256, np.float32)).all()
    rt.free(p)
    rt.free(out)


def test_no_visible_position_gives_zero_rows(rt):
    """max_kv 0: no position is visible, so every output row is 0 (sum 0 ->
    out 0, src/q4_rocm.cu:6968-7013), for the dense and the listed entry
    points."""
    note("max_kv 0")
    rng = np.random.default_rng(77)
    q = heads(rng, (1, 16))
    dq, dg = rt.upload(q), rt.upload(np.zeros_like(q))
    kv = rt.alloc(64 * 544)
    rt.h2d(kv, np.zeros(64 * 544, np.uint8))
    sel = rt.upload(np.arange(2 * 8, dtype=np.int32))
    for dense in (True, False):
        do = _out(rt, q.nbytes)
        if dense:
            ok = rt.lib.q4_hip_qsa_decode_n(dq, kv, kv, dg, do, 16, 2, 256, 1, 5, 0, 1.0 / 16, 2)
        else:
            ok = rt.lib.q4_hip_qsa_decode_idx_kv(dq, kv, kv, None, do, sel, 8, 16, 8, 16, 2,
                                                 256, 1, 0, 1.0 / 16, 2)
        assert ok, dense
        rt.sync()
        assert not rt.download(do, q.nbytes, np.float32).any(), dense
        rt.free(do)
    for x in (dq, dg, kv, sel):
        rt.free(x)


# ------------------------------------------------- config 0: dense decode, ctx 4096
def test_config0_dense_decode_after_append(rt, oracle):
    note("config0 dense 4097")
    rng = np.random.default_rng(1234)
    n_head, n_kvh, hd, ctx = 16, 2, 256, 4096
    k, v = heads(rng, (ctx + 1, n_kvh)), heads(rng, (ctx + 1, n_kvh))
    q = heads(rng, (1, n_head))
    gate = rng.standard_normal((1, n_head, hd)).astype(np.float32)
    max_kv = ctx + 1
    bpt = q4kv.token_bytes(2, n_kvh, hd)
    kc, _ = quantize_on_gpu(rt, np.concatenate([k[:ctx], np.zeros_like(k[:1])]), 2)
    vc, _ = quantize_on_gpu(rt, np.concatenate([v[:ctx], np.zeros_like(v[:1])]), 2)
    dk, dv = rt.upload(k[ctx]), rt.upload(v[ctx])
    rt.lib.q4_hip_pos_push(ctx)
    assert rt.lib.q4_hip_kv_append_d(kc, vc, dk, dv, n_kvh * hd, bpt, 2)
    dq, dg = rt.upload(q), rt.upload(gate)
    do = _out(rt, q.nbytes)
    assert rt.lib.q4_hip_qsa_decode(dq, kc, vc, dg, do, n_head, n_kvh, hd, ctx + 1, max_kv,
                                    1.0 / 16, 2)
    rt.sync()
    kb, vb = oracle.quant_q8(k), oracle.quant_q8(v)
    assert np.array_equal(rt.download(kc, kb.size), kb)
    got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
    want = oracle.attn(q, kb, vb, 2, n_head, n_kvh, hd, 1, gate=gate, kv_base=ctx,
                       max_kv=max_kv, scale=1.0 / 16)
    err = assert_attn_close(got, want, what="config0")
    note(f"config0 max abs err {err:.2e}")


# ------------------------------------------------- config 1: QSA sparse decode at 262K
def test_config1_sparse_decode_262k(rt, oracle):
    note("config1 262144 q8 append+sparse decode")
    rng = np.random.default_rng(1235)
    n_head, n_kvh, hd, ctx = 16, 2, 256, 262144
    pos = ctx - 1
    k, v = heads(rng, (ctx, n_kvh)), heads(rng, (ctx, n_kvh))
    q = heads(rng, (1, n_head))
    bpt = q4kv.token_bytes(2, n_kvh, hd)
    # the cache holds positions 0..pos-1; the new token is appended at pos
    kc = rt.alloc(ctx * bpt)
    vc = rt.alloc(ctx * bpt)
    for cache, x in ((kc, k), (vc, v)):
        src = rt.upload(x[:pos])
        assert rt.lib.q4_hip_f32_to_q8(cache, src, pos * n_kvh * hd)
        rt.sync()
        rt.free(src)
    dk, dv = rt.upload(k[pos]), rt.upload(v[pos])
    rt.lib.q4_hip_pos_push(pos)
    assert rt.lib.q4_hip_kv_append_d(kc, vc, dk, dv, n_kvh * hd, bpt, 2)
    sel = np.stack([selection(rng, pos) for _ in range(n_kvh)])
    got = gpu_idx_kv(rt, q, kc, vc, 2, n_head, n_kvh, hd, sel.ravel(), WIDTH, n_kvh * WIDTH,
                     WIDTH, ctx)
    kb, vb = oracle.quant_q8(k), oracle.quant_q8(v)
    assert np.array_equal(rt.download(kc, kb.size), kb), "K cache bytes differ"
    assert np.array_equal(rt.download(vc, vb.size), vb), "V cache bytes differ"
    want = oracle.attn(q, kb, vb, 2, n_head, n_kvh, hd, 1, idx=sel.ravel(), width=WIDTH,
                       tok_stride=n_kvh * WIDTH, kvh_stride=WIDTH, max_kv=ctx)
    err = assert_attn_close(got, want, what="config1")
    note(f"config1 max abs err {err:.2e}")
    rt.free(kc)
    rt.free(vc)


# ------------------------------------------------- widths, GQA, padding, prefill
@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("n_head", [16, 24, 4])
def test_sparse_decode_widths_and_gqa(rt, oracle, kind, n_head):
    note(f"sparse decode kind={kind} n_head={n_head}")
    rng = np.random.default_rng(300 + 10 * kind + n_head)
    n_kvh, hd, ctx = 2, 256, 20000
    k, v = heads(rng, (ctx, n_kvh)), heads(rng, (ctx, n_kvh))
    q = heads(rng, (1, n_head))
    gate = rng.standard_normal((1, n_head, hd)).astype(np.float32)
    kc, _ = quantize_on_gpu(rt, k, kind)
    vc, _ = quantize_on_gpu(rt, v, kind)
    sel = np.stack([selection(rng, ctx - 1) for _ in range(n_kvh)])
    sel[1, ::97] = -1  # padding holes
    sel[0, 5] = ctx + 7  # beyond max_kv: skipped like padding
    got = gpu_idx_kv(rt, q, kc, vc, kind, n_head, n_kvh, hd, sel.ravel(), WIDTH,
                     n_kvh * WIDTH, WIDTH, ctx, gate=gate)
    want = oracle.attn(q, oracle.encode(k, kind), oracle.encode(v, kind), kind, n_head,
                       n_kvh, hd, 1, gate=gate, idx=sel.ravel(), width=WIDTH,
                       tok_stride=n_kvh * WIDTH, kvh_stride=WIDTH, max_kv=ctx)
    assert_attn_close(got, want, what=f"kind {kind} heads {n_head}")
    rt.free(kc)
    rt.free(vc)


def test_shared_list_reference_entry_and_short_lists(rt, oracle):
    note("decode_idx shared list, short widths")
    rng = np.random.default_rng(400)
    n_head, n_kvh, hd, ctx = 16, 2, 256, 3000
    k, v = heads(rng, (ctx, n_kvh)), heads(rng, (ctx, n_kvh))
    kc, _ = quantize_on_gpu(rt, k, 2)
    vc, _ = quantize_on_gpu(rt, v, 2)
    kb, vb = oracle.quant_q8(k), oracle.quant_q8(v)
    for width in (1, 7, 64, 65, 2051):
        q = heads(rng, (3, n_head))
        gate = rng.standard_normal((3, n_head, hd)).astype(np.float32)
        idx = np.stack([rng.choice(ctx, width, replace=False) for _ in range(3)])
        idx = idx.astype(np.int32).ravel()
        dq, dg, di = rt.upload(q), rt.upload(gate), rt.upload(idx)
        do = _out(rt, q.nbytes)
        assert rt.lib.q4_hip_qsa_decode_idx(dq, kc, vc, dg, do, di, width, n_head, n_kvh, hd,
                                            3, ctx, 1.0 / 16, 2)
        rt.sync()
        got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
        want = oracle.attn(q, kb, vb, 2, n_head, n_kvh, hd, 3, gate=gate, idx=idx,
                           width=width, tok_stride=width, kvh_stride=0, max_kv=ctx)
        assert_attn_close(got, want, what=f"width {width}")
    # all-padding list -> zeros
    q = heads(rng, (1, n_head))
    idx = np.full(2 * 70, -1, np.int32)
    got = gpu_idx_kv(rt, q, kc, vc, 2, n_head, n_kvh, hd, idx, 70, 140, 70, ctx)
    assert not got.any()


# 96 tokens (192 items, two splits each); 160 q8_0 tokens (320 items): one
# split per item, 33 chunks per workgroup, the double-buffered instance
@pytest.mark.parametrize("kind,n_tok", [(2, 96), (1, 96), (2, 160)])
def test_prefill_indexed_and_dense_causal(rt, oracle, kind, n_tok):
    note(f"prefill kind={kind} n_tok={n_tok}")
    rng = np.random.default_rng(500 + kind + n_tok)
    n_head, n_kvh, hd, base = 16, 2, 256, 2500
    ctx = base + n_tok
    k, v = heads(rng, (ctx, n_kvh)), heads(rng, (ctx, n_kvh))
    q = heads(rng, (n_tok, n_head))
    gate = rng.standard_normal((n_tok, n_head, hd)).astype(np.float32)
    kc, _ = quantize_on_gpu(rt, k, kind)
    vc, _ = quantize_on_gpu(rt, v, kind)
    kb, vb = oracle.encode(k, kind), oracle.encode(v, kind)
    sel = np.stack([np.stack([selection(rng, base + t) for _ in range(n_kvh)])
                    for t in range(n_tok)])
    got = gpu_idx_kv(rt, q, kc, vc, kind, n_head, n_kvh, hd, sel.ravel(), WIDTH,
                     n_kvh * WIDTH, WIDTH, ctx, gate=gate)
    want = oracle.attn(q, kb, vb, kind, n_head, n_kvh, hd, n_tok, gate=gate,
                       idx=sel.ravel(), width=WIDTH, tok_stride=n_kvh * WIDTH,
                       kvh_stride=WIDTH, max_kv=ctx, threads=8)
    assert_attn_close(got, want, what="prefill indexed")
    # dense causal: token t sees 0 .. base+t
    dq, dg = rt.upload(q), rt.upload(gate)
    do = _out(rt, q.nbytes)
    assert rt.lib.q4_hip_qsa_decode_n(dq, kc, vc, dg, do, n_head, n_kvh, hd, n_tok, base, ctx,
                                      1.0 / 16, kind)
    rt.sync()
    got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
    want = oracle.attn(q, kb, vb, kind, n_head, n_kvh, hd, n_tok, gate=gate, kv_base=base,
                       max_kv=ctx, threads=8)
    assert_attn_close(got, want, what="prefill dense")


# ------------------------------------------------- config 2: batched decode
def test_config2_batched_decode_subset(rt, oracle):
    note("config2 batched decode, 8 sequences")
    rng = np.random.default_rng(1236)
    n_seq, n_head, n_kvh, hd = 8, 16, 2, 256
    lens = np.exp(rng.uniform(np.log(8192), np.log(131072), n_seq)).astype(np.int64)
    descs = (q4kv.SeqDesc * n_seq)()
    keep = []
    for s in range(n_seq):
        L = int(lens[s])
        k, v = heads(rng, (L, n_kvh)), heads(rng, (L, n_kvh))
        q = heads(rng, (1, n_head))
        sel = np.stack([selection(rng, L - 1) for _ in range(n_kvh)]).ravel()
        kc, _ = quantize_on_gpu(rt, k, 2)
        vc, _ = quantize_on_gpu(rt, v, 2)
        dq, di = rt.upload(q), rt.upload(sel)
        do = _out(rt, q.nbytes)
        descs[s] = q4kv.SeqDesc(kc, vc, dq, None, do, di, WIDTH, WIDTH, L, 0)
        keep.append((k, v, q, sel, do, L))
    dd = rt.alloc(ctypes.sizeof(descs))
    assert rt.lib.q4_hip_h2d(dd, ctypes.addressof(descs), ctypes.sizeof(descs))
    assert rt.lib.q4_hip_qsa_decode_batch(dd, n_seq, n_head, n_kvh, hd, 1.0 / 16, 2, WIDTH)
    rt.sync()
    for k, v, q, sel, do, L in keep:
        got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
        want = oracle.attn(q, oracle.quant_q8(k), oracle.quant_q8(v), 2, n_head, n_kvh, hd,
                           1, idx=sel, width=WIDTH, tok_stride=2 * WIDTH, kvh_stride=WIDTH,
                           max_kv=L)
        assert_attn_close(got, want, what=f"seq len {L}")


# ------------------------------------------------- graph capture + device position
def test_graph_captured_append_and_decode_replays(rt, oracle):
    note("graph capture append + decode")
    rng = np.random.default_rng(600)
    n_head, n_kvh, hd, ctx = 16, 2, 256, 8192
    bpt = q4kv.token_bytes(2, n_kvh, hd)
    k, v = heads(rng, (ctx, n_kvh)), heads(rng, (ctx, n_kvh))
    hk = np.concatenate([oracle.quant_q8(k[:4000]), np.zeros((ctx - 4000) * bpt, np.uint8)])
    hv = np.concatenate([oracle.quant_q8(v[:4000]), np.zeros((ctx - 4000) * bpt, np.uint8)])
    kc, vc = rt.upload(hk), rt.upload(hv)
    dk, dv = rt.alloc(n_kvh * hd * 4), rt.alloc(n_kvh * hd * 4)
    dq = rt.alloc(n_head * hd * 4)
    di = rt.alloc(n_kvh * WIDTH * 4)
    do = _out(rt, n_head * hd * 4)
    assert rt.lib.q4_hip_graph_begin() == 1
    ok = rt.lib.q4_hip_kv_append_d(kc, vc, dk, dv, n_kvh * hd, bpt, 2)
    ok = ok and rt.lib.q4_hip_qsa_decode_idx_kv(dq, kc, vc, None, do, di, WIDTH,
                                                n_kvh * WIDTH, WIDTH, n_head, n_kvh, hd, 1,
                                                ctx, 1.0 / 16, 2)
    g = rt.lib.q4_hip_graph_end()
    assert ok and g
    try:
        for pos in (4000, 4001, 4002, 4003):
            q = heads(rng, (1, n_head))
            sel = np.stack([selection(rng, pos) for _ in range(n_kvh)]).ravel()
            rt.h2d(dk, k[pos])
            rt.h2d(dv, v[pos])
            rt.h2d(dq, q)
            rt.h2d(di, sel)
            rt.lib.q4_hip_pos_push(pos)
            assert rt.lib.q4_hip_graph_launch(g)
            rt.sync()
            oracle.lib.orc_kv_append(hk.ctypes.data, hv.ctypes.data, k[pos].ctypes.data,
                                     v[pos].ctypes.data, n_kvh * hd, bpt, 2, pos)
            got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
            want = oracle.attn(q, hk, hv, 2, n_head, n_kvh, hd, 1, idx=sel, width=WIDTH,
                               tok_stride=2 * WIDTH, kvh_stride=WIDTH, max_kv=ctx)
            assert_attn_close(got, want, what=f"replay pos {pos}")
        assert np.array_equal(rt.download(kc, hk.size), hk)
    finally:
        rt.lib.q4_hip_graph_free(g)


# ------------------------------------------------- config 4 widths at full length
@pytest.mark.parametrize("kind", [1, 0])
def test_config4_widths_sparse_decode_262k(rt, oracle, kind):
    note(f"config4 width kind={kind} at 262144")
    rng = np.random.default_rng(1239 + kind)
    n_head, n_kvh, hd, ctx = 16, 2, 256, 262144
    k, v = heads(rng, (ctx, n_kvh)), heads(rng, (ctx, n_kvh))
    q = heads(rng, (1, n_head))
    kc, _ = quantize_on_gpu(rt, k, kind)
    vc, _ = quantize_on_gpu(rt, v, kind)
    sel = np.stack([selection(rng, ctx - 1) for _ in range(n_kvh)])
    got = gpu_idx_kv(rt, q, kc, vc, kind, n_head, n_kvh, hd, sel.ravel(), WIDTH,
                     n_kvh * WIDTH, WIDTH, ctx)
    rt.free(kc)
    rt.free(vc)
    want = oracle.attn(q, oracle.encode(k, kind), oracle.encode(v, kind), kind, n_head,
                       n_kvh, hd, 1, idx=sel.ravel(), width=WIDTH, tok_stride=n_kvh * WIDTH,
                       kvh_stride=WIDTH, max_kv=ctx)
    assert_attn_close(got, want, what=f"width {kind}")


# ------------------------------------------------- config 3: chunked prefill
def test_config3_chunked_prefill_sampled(rt, oracle):
    """16384-token q8_0 cache + an 8192-token fp32 chunk quantised and appended,
    then causal QSA attention for every query of the chunk over its own
    selection (3 sinks + 512 recent causal + up to 1536 uniform earlier). All
    8192 queries run on the GPU; 64 sampled queries are checked against the
    oracle, and the appended chunk's bytes are checked in full."""
    note("config3 prefill 8192 after 16384")
    rng = np.random.default_rng(1237)
    n_head, n_kvh, hd, base, n_tok = 16, 2, 256, 16384, 8192
    ctx = base + n_tok
    k, v = heads(rng, (ctx, n_kvh)), heads(rng, (ctx, n_kvh))
    q = heads(rng, (n_tok, n_head))
    bpt = q4kv.token_bytes(2, n_kvh, hd)
    kc, vc = rt.alloc(ctx * bpt), rt.alloc(ctx * bpt)
    for cache, x in ((kc, k), (vc, v)):
        src = rt.upload(x[:base])
        assert rt.lib.q4_hip_f32_to_q8(cache, src, base * n_kvh * hd)
        chunk = rt.upload(x[base:])
        assert rt.lib.q4_hip_f32_to_q8(cache + base * bpt, chunk, n_tok * n_kvh * hd)
        rt.sync()
        rt.free(src)
        rt.free(chunk)
    sel = np.empty((n_tok, n_kvh, WIDTH), np.int32)
    for t in range(n_tok):
        for kh in range(n_kvh):
            sel[t, kh] = selection(rng, base + t)
    got = gpu_idx_kv(rt, q, kc, vc, 2, n_head, n_kvh, hd, sel.ravel(), WIDTH, n_kvh * WIDTH,
                     WIDTH, ctx)
    kb, vb = oracle.quant_q8(k), oracle.quant_q8(v)
    assert np.array_equal(rt.download(kc, kb.size), kb)
    assert np.array_equal(rt.download(vc, vb.size), vb)
    rt.free(kc)
    rt.free(vc)
    ts = np.sort(rng.choice(n_tok, 64, replace=False))
    ts[0], ts[-1] = 0, n_tok - 1
    want = oracle.attn(q[ts], kb, vb, 2, n_head, n_kvh, hd, len(ts), idx=sel[ts].ravel(),
                       width=WIDTH, tok_stride=n_kvh * WIDTH, kvh_stride=WIDTH, max_kv=ctx,
                       threads=8)
    assert_attn_close(got[ts], want, what="config3 sampled queries")
    assert np.all(np.isfinite(got))
