"""Seeded randomized parity sweep of the attention entry points against the
oracle (|got - ref| <= 2e-3 + 1e-3*|ref|): cache width, head_dim, query heads
per KV head, KV heads, token count, entry point and list shape are drawn per
case, so the kernel choice (chunk, slab, band, f16, f32, general-shape and
generic kernels, one or many splits) varies across cases. Each case is
small enough for the oracle; the case parameters are printed before its GPU
step. List shapes follow the reference's format (src/q4_rocm.cu:7668-7696):
positions, -1 padding, and here also out-of-range entries, duplicates,
leading padding and runs of consecutive positions."""
import ctypes

import numpy as np
import pytest

import q4kv
from gpu_util import note, quantize_on_gpu
from synth import assert_attn_close, heads
from test_gpu_attn import _out, gpu_idx_kv

pytestmark = pytest.mark.gpu

N_CASES = 160


def _case(seed):
    rng = np.random.default_rng(50000 + seed)
    kind = int(rng.choice([0, 1, 2, 2, 2]))
    if kind == 2 or rng.random() < 0.6:
        hd = int(rng.choice([32, 64, 128, 256, 256, 256]))
    else:
        hd = int(rng.integers(8, 257))
    n_kvh = int(rng.choice([1, 2, 2, 3, 4]))
    gqa = int(rng.choice([1, 2, 4, 8, 8, 8, 12, 16, 20]))
    n_tok = int(rng.choice([1, 1, 2, 5, 40, 300]))
    mode = str(rng.choice(["idx_kv", "idx_kv", "idx", "dense", "batch"]))
    width = int(rng.choice([1, 17, 64, 129, 700, 2051]))
    ctx = int(rng.integers(max(width + 64, 600), 6000))
    while n_tok > 1 and n_tok * gqa * n_kvh * width * hd > 1.5e9:  # oracle time
        n_tok //= 2
    return rng, dict(kind=kind, hd=hd, n_kvh=n_kvh, n_head=gqa * n_kvh, n_tok=n_tok, mode=mode,
                     width=width, ctx=ctx)


def _list(rng, width, ctx, end):
    """One list of `width` entries in one of several shapes."""
    shape = rng.integers(0, 7)
    if shape == 0:      # sorted distinct, trailing padding
        n = int(rng.integers(0, min(width, ctx) + 1))
        sel = np.sort(rng.choice(ctx, n, replace=False))
        out = np.full(width, -1, np.int64)
        out[:n] = sel
    elif shape == 1:    # trailing run of consecutive positions ending at `end`
        run = int(rng.integers(1, width + 1))
        pre = np.sort(rng.choice(max(end - run, 1), width - run, replace=True))
        out = np.concatenate([pre, np.arange(end - run + 1, end + 1)])
    elif shape == 2:    # right-aligned: leading padding, then 0 .. n-1
        n = int(rng.integers(0, width + 1))
        out = np.full(width, -1, np.int64)
        out[width - n:] = np.arange(n)
    elif shape == 3:    # unsorted with duplicates
        out = rng.integers(0, ctx, width)
    elif shape == 4:    # out-of-range and negative entries mixed in
        out = rng.integers(-3, ctx + 50, width)
    elif shape == 5:    # all padding
        out = np.full(width, -1, np.int64)
    else:               # sinks, uniform middle, recent run
        ns = min(3, width)
        nr = min(int(rng.integers(0, width - ns + 1)), end + 1)
        nu = width - ns - nr
        mid = rng.choice(np.arange(ns, max(end - nr + 1, ns + 1)), nu, replace=True) if nu else []
        out = np.concatenate([np.arange(ns), np.sort(mid), np.arange(end - nr + 1, end + 1)])
    return np.asarray(out[:width], np.int32)


@pytest.mark.parametrize("seed", range(N_CASES))
def test_attention_random_case(rt, oracle, seed):
    rng, c = _case(seed)
    kind, hd, n_kvh, n_head, n_tok = c["kind"], c["hd"], c["n_kvh"], c["n_head"], c["n_tok"]
    mode, width, ctx = c["mode"], c["width"], c["ctx"]
    note(f"sweep seed={seed} {c}")
    k = heads(rng, (ctx, n_kvh), hd=hd)
    v = heads(rng, (ctx, n_kvh), hd=hd)
    q = heads(rng, (n_tok, n_head), hd=hd)
    gate = rng.standard_normal((n_tok, n_head, hd)).astype(np.float32)
    kc, _ = quantize_on_gpu(rt, k, kind)
    vc, _ = quantize_on_gpu(rt, v, kind)
    kb, vb = oracle.encode(k, kind), oracle.encode(v, kind)
    scale = 1.0 / np.sqrt(hd)
    owned = [kc, vc]
    if mode == "idx_kv":
        sel = np.stack([np.stack([_list(rng, width, ctx, min(ctx - 1, ctx - n_tok + t))
                                  for _ in range(n_kvh)]) for t in range(n_tok)])
        got = gpu_idx_kv(rt, q, kc, vc, kind, n_head, n_kvh, hd, sel.ravel(), width,
                         n_kvh * width, width, ctx, gate=gate)
        want = oracle.attn(q, kb, vb, kind, n_head, n_kvh, hd, n_tok, gate=gate,
                           idx=sel.ravel(), width=width, tok_stride=n_kvh * width,
                           kvh_stride=width, max_kv=ctx, scale=scale, threads=8)
    elif mode == "idx":
        sel = np.stack([_list(rng, width, ctx, ctx - n_tok + t) for t in range(n_tok)])
        dq, dg, di = rt.upload(q), rt.upload(gate), rt.upload(sel.ravel())
        do = _out(rt, q.nbytes)
        owned += [dq, dg, di, do]
        assert rt.lib.q4_hip_qsa_decode_idx(dq, kc, vc, dg, do, di, width, n_head, n_kvh, hd,
                                            n_tok, ctx, scale, kind)
        rt.sync()
        got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
        want = oracle.attn(q, kb, vb, kind, n_head, n_kvh, hd, n_tok, gate=gate,
                           idx=sel.ravel(), width=width, tok_stride=width, kvh_stride=0,
                           max_kv=ctx, scale=scale, threads=8)
    elif mode == "dense":
        base = int(rng.integers(0, ctx - n_tok + 1))
        dq, dg = rt.upload(q), rt.upload(gate)
        do = _out(rt, q.nbytes)
        owned += [dq, dg, do]
        assert rt.lib.q4_hip_qsa_decode_n(dq, kc, vc, dg, do, n_head, n_kvh, hd, n_tok, base,
                                          ctx, scale, kind)
        rt.sync()
        got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
        want = oracle.attn(q, kb, vb, kind, n_head, n_kvh, hd, n_tok, gate=gate, kv_base=base,
                           max_kv=ctx, scale=scale, threads=8)
    else:  # batch: n_tok independent sequences over the same cache, own lists
        descs = (q4kv.SeqDesc * n_tok)()
        sels, outs = [], []
        for t in range(n_tok):
            dense = rng.random() < 0.3
            dq1, dg1 = rt.upload(q[t:t + 1]), rt.upload(gate[t:t + 1])
            do1 = _out(rt, q[t].nbytes)
            owned += [dq1, dg1, do1]
            if dense:
                n_sel = int(rng.integers(1, ctx + 1))
                descs[t] = q4kv.SeqDesc(kc, vc, dq1, dg1, do1, None, n_sel, 0, ctx, 0)
                sels.append(("dense", n_sel))
            else:
                s1 = np.stack([_list(rng, width, ctx, ctx - 1) for _ in range(n_kvh)])
                di1 = rt.upload(s1.ravel())
                owned.append(di1)
                descs[t] = q4kv.SeqDesc(kc, vc, dq1, dg1, do1, di1, width, width, ctx, 0)
                sels.append(("idx", s1))
            outs.append(do1)
        dd = rt.alloc(ctypes.sizeof(descs))
        owned.append(dd)
        assert rt.lib.q4_hip_h2d(dd, ctypes.addressof(descs), ctypes.sizeof(descs))
        assert rt.lib.q4_hip_qsa_decode_batch(dd, n_tok, n_head, n_kvh, hd, scale, kind, max(
            width, ctx))
        rt.sync()
        got = np.stack([rt.download(o, q[0].nbytes, np.float32).reshape(n_head, hd)
                        for o in outs])
        want = np.empty_like(got)
        for t, (kind_s, s1) in enumerate(sels):
            if kind_s == "dense":
                want[t] = oracle.attn(q[t:t + 1], kb, vb, kind, n_head, n_kvh, hd, 1,
                                      gate=gate[t:t + 1], kv_base=s1 - 1, max_kv=ctx,
                                      scale=scale)[0]
            else:
                want[t] = oracle.attn(q[t:t + 1], kb, vb, kind, n_head, n_kvh, hd, 1,
                                      gate=gate[t:t + 1], idx=s1.ravel(), width=width,
                                      tok_stride=n_kvh * width, kvh_stride=width, max_kv=ctx,
                                      scale=scale)[0]
    try:
        assert_attn_close(got, want, what=f"sweep seed {seed} {c}")
    finally:
        for p in owned:
            rt.free(p)
