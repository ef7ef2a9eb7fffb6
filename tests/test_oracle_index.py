"""Pins of the QSA indexer oracle (CPU only).

Selection is checked against an independent sort-based brute force; pooling,
scoring and Q/K preparation against closed forms, invariants and float64
NumPy arithmetic."""
import math

import numpy as np
import pytest

from qsa_util import (IDX_DIM, K_BLK, N_ROT, RATIO, RMS_EPS, ROPE_BASE, WIDTH,
                      brute_select, keys_of, raw_keys)


# ------------------------------------------------------------------ keys
def test_key_orders_like_floats(oracle):
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(2000).astype(np.float32) * 1e3,
                        np.array([0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-45,
                                  3.4e38, -3.4e38], np.float32)])
    k = keys_of(x)
    for v, kk in zip(x[:64], k[:64]):
        assert oracle.lib.orc_qsa_key(float(v)) == int(kk)
    ok = np.argsort(k, kind="stable")
    xs = x[ok]
    assert np.all(np.diff(xs.astype(np.float64)) >= 0)
    # -0 orders below +0
    assert keys_of(np.float32([-0.0]))[0] < keys_of(np.float32([0.0]))[0]


# ------------------------------------------------------------------ top-k
def _rows(rng, n_vis):
    yield "random", rng.standard_normal(n_vis).astype(np.float32)
    yield "relu-sums", np.maximum(rng.standard_normal(n_vis), 0).astype(np.float32)
    q = np.round(rng.standard_normal(n_vis) * 3).astype(np.float32)  # heavy ties
    yield "ties", q
    z = np.zeros(n_vis, np.float32)
    z[rng.integers(0, n_vis, n_vis // 3)] = -0.0
    z[rng.integers(0, n_vis, 50)] = 1.0
    yield "signed-zeros", z
    c = np.full(n_vis, 2.5, np.float32)
    yield "all-equal", c
    n = rng.standard_normal(n_vis).astype(np.float32)
    n[rng.integers(0, n_vis, 7)] = np.nan
    n[rng.integers(0, n_vis, 5)] = -np.inf
    yield "nan-inf", n


@pytest.mark.parametrize("pos", [0, 2, 3, 4 * K_BLK - 1, 4 * K_BLK, 4 * K_BLK + 3,
                                 5000, 65539, 262143])
def test_topk_matches_brute_force(oracle, pos):
    rng = np.random.default_rng(pos)
    n_vis = (pos + 1) // RATIO
    stride = max(n_vis, 1) + 3
    for name, row in _rows(rng, max(n_vis, 1)):
        sc = np.full((1, stride), 7.0, np.float32)  # beyond n_vis: must be ignored
        sc[0, :row.size] = row
        got = oracle.qsa_topk(sc, 1, stride, K_BLK, RATIO, pos, WIDTH)[0]
        want = brute_select(sc[0], pos, K_BLK, RATIO, WIDTH)
        assert np.array_equal(got, want), (pos, name)


def test_topk_multi_token_rows_and_small_kblk(oracle):
    rng = np.random.default_rng(5)
    pos0, n_tok, k_blk, stride = 700, 9, 37, 300
    sc = rng.standard_normal((n_tok, stride)).astype(np.float32)
    got = oracle.qsa_topk(sc, n_tok, stride, k_blk, RATIO, pos0, 200)
    for t in range(n_tok):
        assert np.array_equal(got[t], brute_select(sc[t], pos0 + t, k_blk, RATIO, 200))


def test_topk_selection_properties(oracle):
    rng = np.random.default_rng(9)
    pos = 40001
    n_vis = (pos + 1) // RATIO
    sc = rng.standard_normal((1, n_vis)).astype(np.float32)
    sel = oracle.qsa_topk(sc, 1, n_vis, K_BLK, RATIO, pos, WIDTH)[0]
    chosen = sel[:K_BLK * RATIO].reshape(K_BLK, RATIO)
    assert np.all(chosen % RATIO == np.arange(RATIO))          # whole blocks
    blocks = chosen[:, 0] // RATIO
    assert np.unique(blocks).size == K_BLK
    # distinct scores: the K_BLK-1 above the threshold ascending, then the threshold block
    assert np.all(np.diff(blocks[:-1]) > 0)
    assert sc[0, blocks[-1]] == sc[0, blocks].min()
    assert sc[0, blocks].min() >= np.sort(sc[0])[-K_BLK]      # the K_BLK largest
    tail = sel[K_BLK * RATIO:]
    ntail = pos - n_vis * RATIO + 1
    assert np.array_equal(tail[:ntail], np.arange(n_vis * RATIO, pos + 1))
    assert np.all(tail[ntail:] == -1)


# ------------------------------------------------------------------ RoPE frequency
def test_rope_freq_correctly_rounded(oracle):
    # powers of two are exact
    for p in range(4):
        assert oracle.lib.orc_rope_freq(16.0, p, 4) == 2.0 ** -p
    for base in (1e4, 1e6, 1e7):
        for p in range(32):
            e = float(-np.float32(p) / np.float32(32))
            exact = base ** e
            f = np.float32(oracle.lib.orc_rope_freq(base, p, 32))
            ulp = np.spacing(f)
            assert abs(float(f) - exact) <= 0.5 * ulp * (1 + 1e-9), (base, p)


# ------------------------------------------------------------------ prep
def test_prep_closed_forms(oracle):
    rng = np.random.default_rng(1)
    hd = 128
    x = rng.standard_normal((3, 4, hd)).astype(np.float32)
    wn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    normed = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True)
                                            + RMS_EPS) * wn
    # position 0: RoPE is the identity
    y0 = oracle.qsa_prep(x[:1], wn, N_ROT, 0, ROPE_BASE, RMS_EPS)
    np.testing.assert_allclose(y0[0], normed[0], rtol=1e-6, atol=1e-6)
    y = oracle.qsa_prep(x, wn, N_ROT, 262141, ROPE_BASE, RMS_EPS)
    # dims >= n_rot untouched by RoPE; pair norms preserved
    np.testing.assert_allclose(y[..., N_ROT:], normed[..., N_ROT:], rtol=1e-6, atol=1e-6)
    pn = lambda a: np.hypot(a[..., 0:N_ROT:2], a[..., 1:N_ROT:2])
    np.testing.assert_allclose(pn(y), pn(normed), rtol=1e-5, atol=1e-6)
    # pair p rotates by the fp32 angle pos*freq_p
    for t in range(3):
        pos = 262141 + t
        for p in (0, 1, 7, 31):
            f = np.float32(oracle.lib.orc_rope_freq(ROPE_BASE, p, N_ROT // 2))
            ang = float(np.float32(pos) * f)
            a0, a1 = normed[t, 0, 2 * p], normed[t, 0, 2 * p + 1]
            want = (a0 * math.cos(ang) - a1 * math.sin(ang), a0 * math.sin(ang) + a1 * math.cos(ang))
            np.testing.assert_allclose(y[t, 0, 2 * p:2 * p + 2], want, rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------------ pool
def test_pool_closed_forms(oracle):
    hd, nb = IDX_DIM, 6
    wn = np.linspace(0.5, 1.5, hd).astype(np.float32)
    c = np.full((nb * RATIO, hd), 3.0, np.float16).view(np.uint16)
    pool = np.full((nb, hd), -9.0, np.float32)
    oracle.qsa_pool(c, pool, wn, hd, RATIO, 1, 4, 0, ROPE_BASE, RMS_EPS)   # no RoPE
    assert np.all(pool[0] == -9.0) and np.all(pool[4:] == -9.0)       # only [b0,b1)
    np.testing.assert_allclose(pool[1:4], np.broadcast_to(wn / np.sqrt(1 + RMS_EPS / 9), (3, hd)),
                               rtol=1e-6)
    rng = np.random.default_rng(2)
    raw = raw_keys(rng, nb * RATIO)
    pool = np.zeros((nb, hd), np.float32)
    oracle.qsa_pool(raw, pool, wn, hd, RATIO, 0, nb, N_ROT, ROPE_BASE, RMS_EPS)
    m = raw.view(np.float16).astype(np.float64).reshape(nb, RATIO, hd).mean(1)
    normed = m / np.sqrt((m ** 2).mean(-1, keepdims=True) + RMS_EPS) * wn
    np.testing.assert_allclose(pool[0], normed[0], rtol=1e-6, atol=1e-7)  # block 0: pos 0
    np.testing.assert_allclose(pool[:, N_ROT:], normed[:, N_ROT:], rtol=1e-6, atol=1e-7)
    pn = lambda a: np.hypot(a[..., 0:N_ROT:2], a[..., 1:N_ROT:2])
    np.testing.assert_allclose(pn(pool), pn(normed), rtol=1e-5, atol=1e-7)


# ------------------------------------------------------------------ score
def test_score_matches_float64(oracle):
    rng = np.random.default_rng(3)
    n_tok, nb, stride, nh, pos0 = 5, 40, 48, 4, 140
    q = rng.standard_normal((n_tok, nh, IDX_DIM)).astype(np.float32)
    pool = rng.standard_normal((nb, IDX_DIM)).astype(np.float32)
    sc = oracle.qsa_score(q, pool, n_tok, nb, stride, nh, IDX_DIM, pos0, RATIO)
    d = np.einsum("thd,bd->thb", q.astype(np.float64), pool.astype(np.float64))
    want = np.maximum(d, 0).sum(1)
    for t in range(n_tok):
        n_vis = (pos0 + t + 1) // RATIO
        np.testing.assert_allclose(sc[t, :n_vis], want[t, :n_vis], rtol=1e-6, atol=1e-5)
        assert np.all(sc[t, n_vis:nb] == np.float32(-1e30))
        assert np.all(np.isnan(sc[t, nb:]))                       # untouched beyond n_blocks
