"""The attention output projection: q4_hip_gemv_dd (q8_0) against the
oracle's float64 GEMV, at the decode shape and at odd shapes (both kernels),
within 2e-3 absolute + 1e-3 relative (normalised by the row's |W| |x|)."""
import numpy as np
import pytest

from gpu_util import note

pytestmark = pytest.mark.gpu


def _check(rt, oracle, nrows, ncols, scale, seed):
    note(f"gemv q8 {nrows}x{ncols}")
    rng = np.random.default_rng(seed)
    wf = rng.standard_normal((nrows, ncols)).astype(np.float32) * 0.05
    w = oracle.quant_q8(wf)
    x = rng.standard_normal(ncols).astype(np.float32)
    dw, dx = rt.upload(w), rt.upload(x)
    dy = rt.upload(np.full(nrows, np.nan, np.float32))
    assert rt.lib.q4_hip_gemv_dd(8, dw, nrows, ncols, dx, dy, scale)
    rt.sync()
    got = rt.download(dy, nrows * 4, np.float32)
    want = oracle.gemv_q8(w, nrows, ncols, x, scale)
    # error relative to the magnitude that enters the sum
    mag = np.abs(oracle.dequant_q8(w, nrows * ncols).reshape(nrows, ncols)) @ np.abs(x) * abs(scale)
    err = np.abs(got.astype(np.float64) - want) / (1.0 + mag)
    assert np.all(np.isfinite(got)) and err.max() < 1e-5, err.max()
    np.testing.assert_allclose(got, want, rtol=1e-3, atol=2e-3)
    for p in (dw, dx, dy):
        rt.free(p)


@pytest.mark.parametrize("nrows,ncols", [(4096, 4096), (4096, 6144), (17, 64), (1000, 8192),
                                         (33, 96), (5, 32), (300, 4128)])
def test_gemv_q8_matches_oracle(rt, oracle, nrows, ncols):
    _check(rt, oracle, nrows, ncols, 0.75, nrows + ncols)


def test_gemv_rejects_other_types(rt):
    d = rt.alloc(4096)
    assert not rt.lib.q4_hip_gemv_dd(1, d, 4, 64, d, d, 1.0)     # f16 weights
    assert not rt.lib.q4_hip_gemv_dd(8, d, 4, 48, d, d, 1.0)     # not whole blocks
    rt.free(d)


# ------------------------------------------------------------ fused epilogue
import ctypes  # noqa: E402

import q4kv  # noqa: E402
from synth import heads, selection  # noqa: E402

N_HEAD, N_KVH, HD = 16, 2, 256


def _step_items(rng, oracle, n_seq, ctx, width, n_embd, n_head=N_HEAD):
    items = []
    for s in range(n_seq):
        pos = ctx - 1 - 131 * s
        k, v = heads(rng, (ctx, N_KVH)), heads(rng, (ctx, N_KVH))
        if width:
            sel = np.stack([np.append(np.sort(rng.choice(pos, width - 1, replace=False)), pos)
                            for _ in range(N_KVH)])
        else:
            sel = np.stack([selection(rng, pos) for _ in range(N_KVH)])
        items.append(dict(pos=pos, kc=oracle.encode(k, q4kv.KV_Q8), vc=oracle.encode(v, q4kv.KV_Q8),
                          kn=heads(rng, (N_KVH,)), vn=heads(rng, (N_KVH,)), q=heads(rng, (n_head,)),
                          gate=rng.standard_normal((n_head, HD)).astype(np.float32),
                          sel=sel.astype(np.int32),
                          w=oracle.quant_q8((rng.standard_normal((n_embd, n_head * HD)) * 0.02)
                                            .astype(np.float32)),
                          y0=rng.standard_normal(n_embd).astype(np.float32)))
    return items


def _run_step(rt, items, ctx, n_embd, fused, y_scale):
    lib = rt.lib
    before = set(rt._owned)
    n = len(items)
    n_head = items[0]["q"].shape[0]
    steps = (q4kv.StepDesc * n)()
    outs = (q4kv.OutDesc * n)()
    keep = []
    for s, it in enumerate(items):
        kc, vc = rt.upload(it["kc"]), rt.upload(it["vc"])
        dq, dg = rt.upload(it["q"]), rt.upload(it["gate"])
        do = rt.upload(np.full((n_head, HD), np.nan, np.float32))
        di = rt.upload(it["sel"])
        dw, dy = rt.upload(it["w"]), rt.upload(it["y0"])
        w = it["sel"].shape[-1]
        seq = q4kv.SeqDesc(kc, vc, dq, dg, do, di, w, w, ctx, 0)
        steps[s] = q4kv.StepDesc(seq, rt.upload(it["kn"]), rt.upload(it["vn"]), it["pos"])
        outs[s] = q4kv.OutDesc(dw, dy)
        keep.append((kc, vc, do, dw, dy))
    max_n = max(it["sel"].shape[-1] for it in items)
    ds, dd = rt.alloc(ctypes.sizeof(steps)), rt.alloc(ctypes.sizeof(outs))
    assert lib.q4_hip_h2d(ds, ctypes.addressof(steps), ctypes.sizeof(steps))
    assert lib.q4_hip_h2d(dd, ctypes.addressof(outs), ctypes.sizeof(outs))
    if fused:
        assert lib.q4_hip_qsa_step_out_batch(ds, dd, n, n_head, N_KVH, HD, 1.0 / 16, q4kv.KV_Q8,
                                             max_n, n_embd, y_scale)
    else:
        assert lib.q4_hip_qsa_step_batch(ds, n, n_head, N_KVH, HD, 1.0 / 16, q4kv.KV_Q8, max_n)
        t = rt.alloc(n_embd * 4)
        for (kc, vc, do, dw, dy) in keep:
            assert lib.q4_hip_gemv_dd(8, dw, n_embd, n_head * HD, do, t, y_scale)
            rt.sync()
            y = rt.download(dy, n_embd * 4, np.float32) + rt.download(t, n_embd * 4, np.float32)
            rt.h2d(dy, y.astype(np.float32))
    rt.sync()
    res = [dict(kc=rt.download(kc, it["kc"].nbytes, np.uint8),
                out=rt.download(do, n_head * HD * 4, np.float32),
                y=rt.download(dy, n_embd * 4, np.float32))
           for (kc, vc, do, dw, dy), it in zip(keep, items)]
    for p in [p for p in rt._owned if p not in before]:
        rt.free(p)
    return res


@pytest.mark.parametrize("n_seq,width,n_embd,n_head", [(12, 0, 4096, 16), (3, 40, 1000, 16),
                                                       (12, 0, 6144, 24), (3, 40, 1000, 24)])
def test_step_out_matches_step_then_gemv(rt, oracle, n_seq, width, n_embd, n_head):
    """Split merge (12 layers, 2051-entry lists) and one-split items: the
    attention output bit-identical to q4_hip_qsa_step_batch's, and y0 + W out
    against q4_hip_gemv_dd + add and the oracle's float64 GEMV."""
    note(f"step_out n_seq={n_seq} width={width} n_embd={n_embd} n_head={n_head}")
    rng = np.random.default_rng(930 + n_seq + n_head)
    ctx = 16384
    items = _step_items(rng, oracle, n_seq, ctx, width, n_embd, n_head)
    a = _run_step(rt, items, ctx, n_embd, True, 0.5)
    b = _run_step(rt, items, ctx, n_embd, False, 0.5)
    for s, it in enumerate(items):
        assert np.array_equal(a[s]["kc"], b[s]["kc"])
        assert np.array_equal(a[s]["out"].view(np.uint32), b[s]["out"].view(np.uint32))
        want = it["y0"].astype(np.float64) + oracle.gemv_q8(it["w"], n_embd, n_head * HD,
                                                             b[s]["out"], 0.5)
        np.testing.assert_allclose(a[s]["y"], b[s]["y"], rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(a[s]["y"], want, rtol=1e-3, atol=2e-3)
