"""Prefill-sized indexed launches (more than 8192 items, one split per item)
with lists built to exercise the recent-window band split: the run of
consecutive positions that ends a list is attended separately and merged
with the rest of the list. Every list shape the split has to get right is
mixed into the same launch, and sampled queries are checked against the
oracle (|got - ref| <= 2e-3 + 1e-3*|ref|):

- runs of 63 (no band), 64, 65, 200 positions and lists that are one run;
- a run followed by -1 padding, or by positions >= max_kv and padding;
- lists with no run, and lists that are all padding (zero output);
- runs ending far from their neighbours' (a token group whose runs span
  more than 1024 positions falls back to the general kernel);
- runs longer than 1024 positions (the band takes their last 1024);
- right-aligned lists (-1 padding first, then a run from position 0);
- a token count that is not a multiple of the 16-token band tile;
- 8, 4 and 1 query heads per KV head, with and without the gate.

src/q4_rocm.cu:6816-6861 is the list semantics (padding and out-of-range
entries are skipped)."""
import numpy as np
import pytest

from gpu_util import note, quantize_on_gpu
from synth import assert_attn_close, heads
from test_gpu_attn import gpu_idx_kv

pytestmark = pytest.mark.gpu

N_TOK = 4200  # 8400 items with two KV heads: one split each; 4200 % 16 == 8


def _prefix(rng, lo, hi, count):
    """count sorted distinct positions in [lo, hi)."""
    if count <= 0:
        return np.empty(0, np.int64)
    return np.sort(rng.choice(hi - lo, size=count, replace=False)) + lo


def band_lists(rng, n_tok, n_kvh, width, base, ctx, long_run):
    """[n_tok, n_kvh, width] int32 lists; token t's query sits at base + t."""
    out = np.full((n_tok, n_kvh, width), -1, np.int32)
    runs = (63, 64, 65, 200, long_run)
    for t in range(n_tok):
        end = base + t
        for kh in range(n_kvh):
            cat = (t + 3 * kh) % 7
            far = cat == 6 and (t // 16) % 3 == 0
            if cat == 6 and not far:
                cat = 0
            if cat == 0:  # prefix + run of rr ending at the query
                rr = min(runs[(t // 7) % len(runs)], width)
                sel = np.concatenate([_prefix(rng, 0, end - rr - 1, width - rr),
                                      np.arange(end - rr + 1, end + 1)])
            elif cat == 1:  # run of 120, then 40 padding entries
                sel = np.concatenate([_prefix(rng, 0, end - 121, width - 160),
                                      np.arange(end - 119, end + 1)])
            elif cat == 2:  # no run
                sel = _prefix(rng, 0, ctx, width)
            elif cat == 3:  # all padding
                sel = np.empty(0, np.int64)
            elif cat == 4:  # run of 100, two out-of-range entries, padding
                sel = np.concatenate([_prefix(rng, 0, end - 101, width - 112),
                                      np.arange(end - 99, end + 1), [ctx + 3, ctx + 10]])
            elif cat == 5:  # run of 90 ending 500 before the query
                e = end - 500
                sel = np.concatenate([_prefix(rng, 0, e - 91, width - 90),
                                      np.arange(e - 89, e + 1)])
            else:  # far: run of 80 ending anywhere in the older context
                e = int(rng.integers(width + 200, base - 2000))
                sel = np.concatenate([_prefix(rng, 0, e - 81, width - 80),
                                      np.arange(e - 79, e + 1)])
            out[t, kh, : sel.size] = sel
            if (t // 16) % 5 == 4:
                # right-aligned: -1 padding first, then positions 0 .. L - 1
                # (a -1 right before a run down to position 0 must not extend it)
                L = 100 + t % 16
                out[t, kh, :] = -1
                out[t, kh, width - L:] = np.arange(L)
    return out


@pytest.mark.parametrize("n_head,width,gated,long_run", [
    (16, 300, True, 300),
    (8, 300, False, 300),
    (2, 300, False, 300),
    (16, 1300, False, 1300),
])
def test_prefill_band_split(rt, oracle, n_head, width, gated, long_run):
    n_kvh, hd = 2, 256
    note(f"band split n_head={n_head} width={width} gated={gated} n_tok={N_TOK}")
    rng = np.random.default_rng(7000 + n_head + width)
    base = width + 4000
    ctx = base + N_TOK
    k, v = heads(rng, (ctx, n_kvh)), heads(rng, (ctx, n_kvh))
    q = heads(rng, (N_TOK, n_head))
    gate = rng.standard_normal((N_TOK, n_head, hd)).astype(np.float32) if gated else None
    kc, _ = quantize_on_gpu(rt, k, 2)
    vc, _ = quantize_on_gpu(rt, v, 2)
    sel = band_lists(rng, N_TOK, n_kvh, width, base, ctx, long_run)
    got = gpu_idx_kv(rt, q, kc, vc, 2, n_head, n_kvh, hd, sel.ravel(), width,
                     n_kvh * width, width, ctx, gate=gate)
    rt.free(kc)
    rt.free(vc)
    kb, vb = oracle.quant_q8(k), oracle.quant_q8(v)
    # three whole 16-token groups (one of them holding a far run), the ragged
    # last group and a random sample
    ts = np.unique(np.concatenate([np.arange(0, 16), np.arange(48, 80), np.arange(160, 176),
                                   np.arange(N_TOK - 8, N_TOK),
                                   rng.choice(N_TOK, 200, replace=False)]))
    want = oracle.attn(q[ts], kb, vb, 2, n_head, n_kvh, hd, len(ts),
                       gate=gate[ts] if gated else None, idx=sel[ts].ravel(), width=width,
                       tok_stride=n_kvh * width, kvh_stride=width, max_kv=ctx, threads=8)
    assert_attn_close(got[ts], want, what=f"band split n_head={n_head} width={width}")
    assert np.all(np.isfinite(got))
    # all-padding lists (both KV heads) give zero rows
    for t in range(N_TOK):
        for kh in range(n_kvh):
            if not (sel[t, kh] >= 0).any():
                g = n_head // n_kvh
                assert not got[t, kh * g:(kh + 1) * g].any(), (t, kh)
