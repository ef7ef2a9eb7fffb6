"""The split-KV launches with the KV heads of each (token, split) grouped on
one XCD against the plain (split, item) grid (q4kv_xcd_group): the grouping
only places workgroups, so outputs and cache bytes are bit-identical. Covers
the chunk kernel (fused step and batched decode), the batched slab kernel
(many chunks per split) and the slab kernel's two head groups (24 query
heads over 2 KV heads)."""
import numpy as np
import pytest

import q4kv
from gpu_util import note
from test_gpu_step import _case, _run, _sel_kv

pytestmark = pytest.mark.gpu


@pytest.fixture
def grouping(rt):
    assert rt.lib.q4kv_xcd_group(-1) == 1, "grouping is the default"
    yield
    rt.lib.q4kv_xcd_group(1)


@pytest.mark.parametrize("n_seq,n_head", [(1, 16), (12, 16), (32, 16), (4, 24)])
@pytest.mark.parametrize("fused", [True, False])
def test_grouped_launch_bit_identical(rt, oracle, grouping, n_seq, n_head, fused):
    rng = np.random.default_rng(700 + n_seq + n_head)
    ctx = 8192
    items, _ = _case(rng, oracle, n_seq, ctx, q4kv.KV_Q8, lambda s: ctx - 1 - 53 * s, _sel_kv,
                     n_head=n_head)
    note(f"xcd grouping n_seq={n_seq} n_head={n_head} fused={fused}")
    runs = []
    for on in (1, 0):
        assert rt.lib.q4kv_xcd_group(on) == on
        runs.append(_run(rt, items, ctx, q4kv.KV_Q8, fused=fused))
    (c1, o1), (c0, o0) = runs
    for s in range(n_seq):
        assert np.array_equal(c1[s][0], c0[s][0]) and np.array_equal(c1[s][1], c0[s][1]), \
            f"cache bytes differ, item {s}"
        assert np.array_equal(o1[s], o0[s]), f"outputs differ, item {s}"
        assert np.all(np.isfinite(o1[s]))
