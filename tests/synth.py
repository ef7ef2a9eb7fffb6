"""Seeded synthetic inputs for the BASELINE configurations (tests only).

K, V and Q are fp32 ~N(0,1) with 4 outlier channels per head scaled x8;
selections are 3 sinks + the 512 most recent positions + 1536 distinct
uniform draws from the rest, sorted (dense prefix when the context is
shorter than that)."""
from __future__ import annotations

import numpy as np

OUTLIERS = (3, 77, 150, 201)
N_SINK, N_RECENT, N_UNIFORM = 3, 512, 1536
WIDTH = N_SINK + N_RECENT + N_UNIFORM  # 2051


def heads(rng, shape, hd=256, outliers=OUTLIERS):
    """fp32 normal tensor [..., hd] with outlier channels scaled x8."""
    x = rng.standard_normal(tuple(shape) + (hd,), dtype=np.float32)
    for c in outliers:
        if c < hd:
            x[..., c] *= 8.0
    return x


def selection(rng, pos, width=WIDTH, n_sink=N_SINK, n_recent=N_RECENT):
    """Sorted distinct positions visible to a query at `pos` (inclusive),
    -1 padded to `width`."""
    n_uniform = width - n_sink - n_recent
    if pos + 1 <= width:
        sel = np.arange(pos + 1, dtype=np.int32)
    else:
        lo, hi = n_sink, pos - n_recent + 1  # uniform range [lo, hi)
        uni = rng.choice(hi - lo, size=n_uniform, replace=False).astype(np.int64) + lo
        sel = np.concatenate([np.arange(n_sink), np.sort(uni),
                              np.arange(pos - n_recent + 1, pos + 1)]).astype(np.int32)
    out = np.full(width, -1, dtype=np.int32)
    out[: sel.size] = sel
    return out


def assert_attn_close(got, ref, atol=2e-3, rtol=1e-3, what="", combined=False):
    """The attention bar, both parts of it: max |got - ref| <= atol
    everywhere, and |got - ref| <= rtol * |ref| wherever |ref| >= atol /
    (2 rtol) (1.0 for the default bar: values at the data's unit scale; below
    that the relative bar would ask for less than fp32 rounding of the
    softmax sums gives). Scaled data scale atol with it (the relative floor
    follows). combined=True checks the allclose form |got - ref| <= atol +
    rtol |ref| instead (stress tests whose outputs sit far above unit scale).
    Returns the max abs error."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - ref)
    floor = atol / (2.0 * rtol)
    bad_abs = err > atol
    bad_rel = (np.abs(ref) >= floor) & (err > rtol * np.abs(ref))
    if combined:
        bad_abs = err > atol + rtol * np.abs(ref)
        bad_rel = np.zeros_like(bad_abs)
    bad = bad_abs | bad_rel
    assert not bad.any(), (f"{what}: {bad_abs.sum()} of {bad.size} past max-abs {atol:g}, "
                           f"{bad_rel.sum()} past rel {rtol:g} (|ref| >= {floor:g}); "
                           f"max abs err {err.max():.3e}")
    return float(err.max())
