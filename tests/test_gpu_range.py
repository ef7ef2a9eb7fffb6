"""Values of large and small magnitude on the MFMA kernels, against the
oracle (|got - ref| <= 2e-3 + 1e-3*|ref|).

The kernels carry Q as fp16 hi/lo parts after dividing each head's q (times
the softmax scale where a kernel folds it in) by the power of two that
brings its largest magnitude into [0.5, 1), so no range of q is excluded
and the results must not depend on the magnitude:
test_query_magnitude_any runs queries x 1e5 and x 1e-4 through every MFMA
kernel (chunk, slab, band, f16, f32, generic). Here one 32-dimension
block of every head sums to about +704 and another to about -640 (about +63
and -58 after the scale): a kernel that folded the +1152 bias of its
int8 -> fp16 K operands into a product with those sums (-1152 x 63 is
beyond fp16's 65504) would fail. The slab kernel's K operands are exact (no
bias left in the products); the chunk kernel removes the bias through the
accumulator input of each block's MFMA, in fp32."""
import numpy as np
import pytest

from gpu_util import note, quantize_on_gpu
from synth import assert_attn_close, heads, selection
from test_gpu_attn import gpu_idx_kv

pytestmark = pytest.mark.gpu


# (query heads, tokens): decode through the chunk kernel (8 per KV head) and
# the slab kernel (16); prefill-sized launches through the band + slab
# kernels (8 and 16 per KV head)
@pytest.mark.parametrize("n_head,n_tok", [(16, 1), (32, 1), (16, 700), (32, 300)])
def test_large_query_blocks(rt, oracle, n_head, n_tok):
    n_kvh, hd, width = 2, 256, 2051
    note(f"large query blocks n_head={n_head} n_tok={n_tok}")
    rng = np.random.default_rng(9100 + n_head + n_tok)
    base = 6000
    ctx = base + n_tok
    k, v = heads(rng, (ctx, n_kvh)), heads(rng, (ctx, n_kvh))
    q = heads(rng, (n_tok, n_head))
    # block 0 sums to about +704, block 3 to about -640 (not exactly
    # representable sums, as real queries give)
    q[:, :, 0:32] = 22.0 + 3.0 * rng.standard_normal((n_tok, n_head, 32), dtype=np.float32)
    q[:, :, 96:128] = -20.0 + 3.0 * rng.standard_normal((n_tok, n_head, 32), dtype=np.float32)
    kc, _ = quantize_on_gpu(rt, k, 2)
    vc, _ = quantize_on_gpu(rt, v, 2)
    sel = np.stack([np.stack([selection(rng, base + t) for _ in range(n_kvh)])
                    for t in range(n_tok)]).astype(np.int32)
    got = gpu_idx_kv(rt, q, kc, vc, 2, n_head, n_kvh, hd, sel.ravel(), width, n_kvh * width,
                     width, ctx)
    rt.free(kc)
    rt.free(vc)
    kb, vb = oracle.quant_q8(k), oracle.quant_q8(v)
    ts = np.arange(n_tok) if n_tok <= 8 else np.unique(
        np.concatenate([[0, n_tok - 1], rng.choice(n_tok, 40, replace=False)]))
    want = oracle.attn(q[ts], kb, vb, 2, n_head, n_kvh, hd, len(ts), idx=sel[ts].ravel(),
                       width=width, tok_stride=n_kvh * width, kvh_stride=width, max_kv=ctx,
                       threads=8)
    # Outputs here reach |ref| ~ 25 (the softmax concentrates on positions
    # whose outlier V channels are large), and the scores ~1e3: fp32 rounding
    # of those scores alone moves such outputs by ~1e-4 relative (~2.5e-3
    # absolute), so an fp32 reference would miss a 2e-3 max-abs bar against
    # this fp64 oracle too. The bar is the allclose form 2e-3 + 1e-3 |ref|.
    assert_attn_close(got[ts], want, what=f"large query blocks n_head={n_head} n_tok={n_tok}",
                      combined=True)


@pytest.mark.parametrize("n_head,n_tok", [(16, 1), (32, 1), (16, 700), (32, 300)])
def test_large_v_values(rt, oracle, n_head, n_tok):
    """V values up to ~2.4e4 (block scales up to ~190; the band kernel's fp16
    parts of v * scale stay below 65504), K and Q at unit scale. The outputs
    are the unit-scale outputs times 1000, so the bar is the unit-scale bar
    times 1000: |got - ref| <= 2 + 1e-3*|ref|. (The chunk and slab kernels
    carry V as 1152 + v and remove the bias on the MFMA pipe, so their error
    is ~1e-5 of a V block's absmax: ~5e-4 at unit scale, ~0.25 here.)"""
    n_kvh, hd, width = 2, 256, 2051
    note(f"large v values n_head={n_head} n_tok={n_tok}")
    rng = np.random.default_rng(9300 + n_head + n_tok)
    base = 6000
    ctx = base + n_tok
    k = heads(rng, (ctx, n_kvh))
    v = heads(rng, (ctx, n_kvh)) * np.float32(1000.0)
    q = heads(rng, (n_tok, n_head))
    kc, _ = quantize_on_gpu(rt, k, 2)
    vc, _ = quantize_on_gpu(rt, v, 2)
    sel = np.stack([np.stack([selection(rng, base + t) for _ in range(n_kvh)])
                    for t in range(n_tok)]).astype(np.int32)
    got = gpu_idx_kv(rt, q, kc, vc, 2, n_head, n_kvh, hd, sel.ravel(), width, n_kvh * width,
                     width, ctx)
    rt.free(kc)
    rt.free(vc)
    kb, vb = oracle.quant_q8(k), oracle.quant_q8(v)
    ts = np.arange(n_tok) if n_tok <= 8 else np.unique(
        np.concatenate([[0, n_tok - 1], rng.choice(n_tok, 40, replace=False)]))
    want = oracle.attn(q[ts], kb, vb, 2, n_head, n_kvh, hd, len(ts), idx=sel[ts].ravel(),
                       width=width, tok_stride=n_kvh * width, kvh_stride=width, max_kv=ctx,
                       threads=8)
    # the unit-scale bar (2e-3 absolute) scaled by the data's factor 1000:
    # the outputs are 1000x the unit-scale ones, and so are their errors
    assert_attn_close(got[ts], want, atol=2.0, rtol=1e-3,
                      what=f"large v values n_head={n_head} n_tok={n_tok}")


# (kind, head_dim, query heads, tokens): the chunk kernel (q8, 8 per KV
# head), the slab kernel (16), the band + slab prefill kernels, the f16
# kernel (8 and 16), the f32 kernel, the generic MFMA kernel (q8, hd 128)
@pytest.mark.parametrize("kind,hd,n_head,n_tok", [(2, 256, 16, 1), (2, 256, 32, 1),
                                                  (2, 256, 16, 300), (1, 256, 16, 1),
                                                  (1, 256, 32, 1), (0, 256, 16, 1),
                                                  (2, 128, 16, 1)])
@pytest.mark.parametrize("qscale", [1e5, 1e-4])
def test_query_magnitude_any(rt, oracle, kind, hd, n_head, n_tok, qscale):
    """Queries x 1e5 (|q| up to ~4e6, far past fp16's 65504; the softmax is
    then nearly one-hot) and x 1e-4 (nearly uniform weights) against the fp64
    oracle on the same cache bytes, at the unscaled bar."""
    n_kvh, width = 2, 2051
    note(f"query magnitude kind={kind} hd={hd} n_head={n_head} n_tok={n_tok} x{qscale:g}")
    rng = np.random.default_rng(9500 + 7 * kind + hd + n_head + n_tok + int(qscale > 1))
    base = 6000
    ctx = base + n_tok
    k, v = heads(rng, (ctx, n_kvh), hd=hd), heads(rng, (ctx, n_kvh), hd=hd)
    q = heads(rng, (n_tok, n_head), hd=hd) * np.float32(qscale)
    kc, _ = quantize_on_gpu(rt, k, kind)
    vc, _ = quantize_on_gpu(rt, v, kind)
    sel = np.stack([np.stack([selection(rng, base + t) for _ in range(n_kvh)])
                    for t in range(n_tok)]).astype(np.int32)
    got = gpu_idx_kv(rt, q, kc, vc, kind, n_head, n_kvh, hd, sel.ravel(), width,
                     n_kvh * width, width, ctx)
    rt.free(kc)
    rt.free(vc)
    ts = np.arange(n_tok) if n_tok <= 8 else np.unique(
        np.concatenate([[0, n_tok - 1], rng.choice(n_tok, 40, replace=False)]))
    want = oracle.attn(q[ts], oracle.encode(k, kind), oracle.encode(v, kind), kind, n_head,
                       n_kvh, hd, len(ts), idx=sel[ts].ravel(), width=width,
                       tok_stride=n_kvh * width, kvh_stride=width, max_kv=ctx, threads=8)
    assert_attn_close(got[ts], want, what=f"query x{qscale:g} kind {kind} hd {hd}")
