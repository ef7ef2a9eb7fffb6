"""GPU parity of the QSA indexer and Q/K preparation (src/q4_rocm.cu:6229-6343,
7366-7960) through the C ABI, against the CPU oracle.

Selection is integer work on fp32 bit patterns: given the same scores the
GPU list must equal the oracle's bit for bit. Pooling, scoring and
preparation are fp32 arithmetic, checked within 2e-3 absolute + 1e-3
relative of the oracle's float64 result."""
import numpy as np
import pytest

from gpu_util import note
from qsa_util import (IDX_DIM, IDX_HEADS, K_BLK, N_ROT, RATIO, RMS_EPS, ROPE_BASE, WIDTH,
                      raw_keys)

pytestmark = pytest.mark.gpu
ATOL, RTOL = 2e-3, 1e-3


def _close(got, want, what):
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL, err_msg=what)


def _score_rows(rng, n_vis):
    yield "random", rng.standard_normal(n_vis).astype(np.float32)
    yield "relu-sums", np.maximum(rng.standard_normal(n_vis) * 4, 0).astype(np.float32)
    yield "ties", np.round(rng.standard_normal(n_vis) * 3).astype(np.float32)
    # a few ties around the threshold, with a small candidate set
    yield "near-ties", (np.round(rng.standard_normal(n_vis) * 300) / 300).astype(np.float32)
    # top values far apart (wide candidate range, several radix passes)
    w = rng.standard_normal(n_vis).astype(np.float32)
    w[rng.integers(0, n_vis, 300)] = 1e30
    w[rng.integers(0, n_vis, 300)] = -1e-30
    yield "wide", w
    z = np.zeros(n_vis, np.float32)
    z[rng.integers(0, n_vis, n_vis // 3)] = -0.0
    z[rng.integers(0, n_vis, 40)] = 1.0
    yield "signed-zeros", z
    yield "all-equal", np.full(n_vis, 2.5, np.float32)
    # rising with the index: the whole selection in the last slices of a split row
    yield "ascending", np.linspace(0.0, 1.0, n_vis, dtype=np.float32)
    n = rng.standard_normal(n_vis).astype(np.float32)
    n[rng.integers(0, n_vis, 7)] = np.nan
    n[rng.integers(0, n_vis, 5)] = -np.inf
    yield "nan-inf", n


# ----------------------------------------------------------------- top-k
@pytest.mark.parametrize("cap", ["tight", "wide"])
@pytest.mark.parametrize("pos", [0, 2, 3, 2047, 2048, 2051, 5000, 65539, 262139, 262143, 300001])
def test_topk_d_bit_exact(rt, oracle, pos, cap):
    """Row capacity (stride) just past the visible blocks, or a whole number
    of 65536-key chunks beyond them, which the kernel then loads unmasked;
    either way the 9.0 filler past n_vis must never be selected."""
    lib = rt.lib
    rng = np.random.default_rng(100 + pos)
    n_vis = (pos + 1) // RATIO
    stride = max(n_vis, 1) + 5
    if cap == "wide":
        stride = -(-stride // 65536) * 65536
    for name, row in _score_rows(rng, max(n_vis, 1)):
        note(f"topk_d pos={pos} cap={cap} rows={name}")
        sc = np.full((1, stride), 9.0, np.float32)   # past n_vis: never read as a score
        sc[0, :row.size] = row
        d_sc, d_sel = rt.upload(sc), rt.alloc(WIDTH * 4)
        lib.q4_hip_pos_push(pos)
        assert lib.q4_hip_qsa_topk_d(d_sc, d_sel, stride, K_BLK, RATIO, WIDTH)
        rt.sync()
        got = rt.download(d_sel, WIDTH * 4, np.int32)
        want = oracle.qsa_topk(sc, 1, stride, K_BLK, RATIO, pos, WIDTH)[0]
        rt.free(d_sc)
        rt.free(d_sel)
        assert np.array_equal(got, want), (pos, name, np.flatnonzero(got != want)[:8])


def test_topk_d_split_row_graph_replays(rt, oracle):
    """Rows of 16385-65536 blocks are selected by 8 slice workgroups that hand
    their candidates to the last one through a per-GPU buffer and ticket. A
    captured topk_d replayed at positions filling 3, 8 and 5 slices and a
    dense prefix, with an eager call on another row between replays: every
    list bit-exact against the oracle (the ticket is re-armed by each launch,
    the buffer reused)."""
    lib = rt.lib
    rng = np.random.default_rng(4242)
    stride = 65536
    row = np.maximum(rng.standard_normal(stride) * 6, 0).astype(np.float32)
    other = rng.standard_normal(stride).astype(np.float32)
    d_sc, d_sel = rt.upload(row[None, :]), rt.alloc(WIDTH * 4)
    d_o, d_osel = rt.upload(other[None, :]), rt.alloc(WIDTH * 4)
    lib.q4_hip_pos_push(100000)
    assert lib.q4_hip_graph_begin() == 1
    ok = lib.q4_hip_qsa_topk_d(d_sc, d_sel, stride, K_BLK, RATIO, WIDTH)
    g = lib.q4_hip_graph_end()
    assert ok and g
    try:
        for pos in (80003, 262143, 170001, 1500, 262140):
            note(f"split topk_d graph replay pos={pos}")
            lib.q4_hip_pos_push(pos)
            assert lib.q4_hip_graph_launch(g)
            rt.sync()
            want = oracle.qsa_topk(row[None, :], 1, stride, K_BLK, RATIO, pos, WIDTH)[0]
            got = rt.download(d_sel, WIDTH * 4, np.int32)
            assert np.array_equal(got, want), (pos, np.flatnonzero(got != want)[:8])
            epos = pos // 2 + 40000
            lib.q4_hip_pos_push(epos)
            assert lib.q4_hip_qsa_topk_d(d_o, d_osel, stride, K_BLK, RATIO, WIDTH)
            rt.sync()
            want = oracle.qsa_topk(other[None, :], 1, stride, K_BLK, RATIO, epos, WIDTH)[0]
            got = rt.download(d_osel, WIDTH * 4, np.int32)
            assert np.array_equal(got, want), ("eager", epos, np.flatnonzero(got != want)[:8])
    finally:
        lib.q4_hip_graph_free(g)
    for p_ in (d_sc, d_sel, d_o, d_osel):
        rt.free(p_)


@pytest.mark.parametrize("k_blk,width", [(1, 16), (37, 300), (511, WIDTH)])
def test_topk_d_split_row_small_k(rt, oracle, k_blk, width):
    """The split selection (a row capacity of 16385-65536 blocks) at other
    k_blk and widths: lists shorter than the width take the tail rule, and
    each slice's local candidate bin follows its own need."""
    lib = rt.lib
    rng = np.random.default_rng(4300 + k_blk)
    stride, pos = 60000, 200001
    for name, row in _score_rows(rng, stride):
        note(f"split topk_d k_blk={k_blk} width={width} rows={name}")
        d_sc, d_sel = rt.upload(row[None, :]), rt.alloc(width * 4)
        lib.q4_hip_pos_push(pos)
        assert lib.q4_hip_qsa_topk_d(d_sc, d_sel, stride, k_blk, RATIO, width)
        rt.sync()
        got = rt.download(d_sel, width * 4, np.int32)
        want = oracle.qsa_topk(row[None, :], 1, stride, k_blk, RATIO, pos, width)[0]
        rt.free(d_sc)
        rt.free(d_sel)
        assert np.array_equal(got, want), (k_blk, name, np.flatnonzero(got != want)[:8])


def test_topk_rows_bit_exact(rt, oracle):
    """Prefill form: n_tok rows, one per token at pos0 + t, crossing the
    dense-prefix boundary, with small k_blk and width."""
    lib = rt.lib
    for pos0, n_tok, k_blk, width, stride in [(2040, 20, K_BLK, WIDTH, 600),
                                              (9000, 33, 100, 300, 2300),
                                              (9000, 33, 100, 300, 8192),
                                              (40000, 9, K_BLK, WIDTH, 12000),
                                              (70000, 6, K_BLK, WIDTH, 17503)]:
        note(f"topk rows pos0={pos0} n_tok={n_tok} k_blk={k_blk}")
        rng = np.random.default_rng(pos0)
        sc = np.round(rng.standard_normal((n_tok, stride)) * 8).astype(np.float32)
        d_sc, d_sel = rt.upload(sc), rt.alloc(n_tok * width * 4)
        n_blocks = (pos0 + n_tok) // RATIO
        assert lib.q4_hip_qsa_topk(d_sc, d_sel, n_tok, n_blocks, stride, k_blk, RATIO, pos0,
                                   width)
        rt.sync()
        got = rt.download(d_sel, n_tok * width * 4, np.int32).reshape(n_tok, width)
        want = oracle.qsa_topk(sc, n_tok, stride, k_blk, RATIO, pos0, width)
        rt.free(d_sc)
        rt.free(d_sel)
        assert np.array_equal(got, want), (pos0, np.argwhere(got != want)[:8])


def test_topk_rejects_bad_shapes(rt):
    lib = rt.lib
    d = rt.alloc(4096)
    assert not lib.q4_hip_qsa_topk(d, d, 1, 1, 1, 513, RATIO, 0, WIDTH)   # k_blk > 512
    assert not lib.q4_hip_qsa_topk(d, d, 1, 1, 1, K_BLK, RATIO, 0, 0)     # width 0
    assert not lib.q4_hip_qsa_topk_d(d, d, 1, 0, RATIO, WIDTH)            # k_blk 0
    assert not lib.q4_hip_qsa_score(d, d, d, 1, 1, 1, 4, 64, 0, RATIO)     # hd != 128
    assert not lib.q4_hip_qsa_score(d, d, d, 1, 1, 1, 5, IDX_DIM, 0, RATIO)  # heads > 4
    assert not lib.q4_hip_qsa_pool(d, d, None, 64, RATIO, 0, 1, N_ROT, ROPE_BASE, RMS_EPS)
    rt.free(d)


# ----------------------------------------------------------------- score
@pytest.mark.parametrize("n_tok,pos0,n_head", [(1, 262143, 4), (2, 4097, 3), (5, 1000, 4),
                                                (37, 20000, 4), (16, 123, 2)])
def test_score_matches_oracle(rt, oracle, n_tok, pos0, n_head):
    lib = rt.lib
    note(f"score n_tok={n_tok} pos0={pos0} n_head={n_head}")
    rng = np.random.default_rng(n_tok * 7 + pos0)
    n_blocks = (pos0 + n_tok) // RATIO + 3          # a few blocks past every token's n_vis
    stride = n_blocks + 9
    q = rng.standard_normal((n_tok, n_head, IDX_DIM)).astype(np.float32)
    pool = (rng.standard_normal((n_blocks, IDX_DIM)) * 0.3).astype(np.float32)
    d_q, d_pool = rt.upload(q), rt.upload(pool)
    sentinel = np.full((n_tok, stride), np.nan, np.float32)
    d_sc = rt.upload(sentinel)
    assert lib.q4_hip_qsa_score(d_q, d_pool, d_sc, n_tok, n_blocks, stride, n_head, IDX_DIM,
                                pos0, RATIO)
    rt.sync()
    got = rt.download(d_sc, sentinel.nbytes, np.float32).reshape(n_tok, stride)
    want = oracle.qsa_score(q, pool, n_tok, n_blocks, stride, n_head, IDX_DIM, pos0, RATIO)
    for t in range(n_tok):
        n_vis = (pos0 + t + 1) // RATIO
        _close(got[t, :n_vis], want[t, :n_vis], f"token {t}")
        assert np.all(got[t, n_vis:n_blocks] == np.float32(-1e30))
        assert np.all(np.isnan(got[t, n_blocks:]))
    for p in (d_q, d_pool, d_sc):
        rt.free(p)


@pytest.mark.parametrize("pos", [2, 3, 700, 262143])
def test_score_d_matches_oracle(rt, oracle, pos):
    lib = rt.lib
    note(f"score_d pos={pos}")
    rng = np.random.default_rng(pos)
    stride = 65536
    n_vis = (pos + 1) // RATIO
    q = rng.standard_normal((1, IDX_HEADS, IDX_DIM)).astype(np.float32)
    pool = (rng.standard_normal((stride, IDX_DIM)) * 0.3).astype(np.float32)
    d_q, d_pool = rt.upload(q), rt.upload(pool)
    d_sc = rt.upload(np.full(stride, np.nan, np.float32))
    lib.q4_hip_pos_push(pos)
    assert lib.q4_hip_qsa_score_d(d_q, d_pool, d_sc, stride, IDX_HEADS, IDX_DIM, RATIO)
    rt.sync()
    got = rt.download(d_sc, stride * 4, np.float32)
    want = oracle.qsa_score(q, pool[:max(n_vis, 1)], 1, n_vis, stride, IDX_HEADS, IDX_DIM,
                            pos, RATIO)[0]
    _close(got[:n_vis], want[:n_vis], "visible blocks")
    assert np.all(np.isnan(got[n_vis:]))            # only visible blocks are written
    for p in (d_q, d_pool, d_sc):
        rt.free(p)


# ----------------------------------------------------------------- pool
def test_pool_matches_oracle(rt, oracle):
    lib = rt.lib
    rng = np.random.default_rng(11)
    nb = 65536
    raw = raw_keys(rng, nb * RATIO)
    wn = (1 + 0.2 * rng.standard_normal(IDX_DIM)).astype(np.float32)
    d_raw, d_wn = rt.upload(raw), rt.upload(wn)
    sentinel = np.full((nb, IDX_DIM), np.nan, np.float32)
    d_pool = rt.upload(sentinel)
    for b0, b1 in [(0, 5), (5, 6), (60000, nb)]:
        note(f"pool blocks [{b0},{b1})")
        assert lib.q4_hip_qsa_pool(d_raw, d_pool, d_wn, IDX_DIM, RATIO, b0, b1, N_ROT,
                                   ROPE_BASE, RMS_EPS)
    rt.sync()
    got = rt.download(d_pool, sentinel.nbytes, np.float32).reshape(nb, IDX_DIM)
    want = np.full_like(sentinel, np.nan)
    oracle.qsa_pool(raw, want, wn, IDX_DIM, RATIO, 0, 6, N_ROT, ROPE_BASE, RMS_EPS)
    oracle.qsa_pool(raw, want, wn, IDX_DIM, RATIO, 60000, nb, N_ROT, ROPE_BASE, RMS_EPS)
    for lo, hi in [(0, 6), (60000, nb)]:
        _close(got[lo:hi], want[lo:hi], f"blocks {lo}..{hi}")
    assert np.all(np.isnan(got[6:60000]))
    # no weight vector: RMSNorm alone
    note("pool without wn")
    assert lib.q4_hip_qsa_pool(d_raw, d_pool, None, IDX_DIM, RATIO, 7, 9, N_ROT, ROPE_BASE,
                               RMS_EPS)
    rt.sync()
    got = rt.download(d_pool, sentinel.nbytes, np.float32).reshape(nb, IDX_DIM)
    oracle.qsa_pool(raw, want, None, IDX_DIM, RATIO, 7, 9, N_ROT, ROPE_BASE, RMS_EPS)
    _close(got[7:9], want[7:9], "no wn")
    for p in (d_raw, d_wn, d_pool):
        rt.free(p)


def test_pool_d_and_f16_store_follow_device_position(rt, oracle):
    lib = rt.lib
    rng = np.random.default_rng(12)
    n_pos = 4096
    raw = raw_keys(rng, n_pos)
    wn = (1 + 0.2 * rng.standard_normal(IDX_DIM)).astype(np.float32)
    d_raw, d_wn = rt.upload(raw), rt.upload(wn)
    pool0 = np.full((n_pos // RATIO, IDX_DIM), np.nan, np.float32)
    d_pool = rt.upload(pool0)
    expect = pool0.copy()
    for pos in (0, 1, 2, 3, 4, 7, 1021, 1023, 4095):
        note(f"f32_to_f16_d + pool_d pos={pos}")
        k = rng.standard_normal(IDX_DIM).astype(np.float32) * 3
        d_k = rt.upload(k)
        lib.q4_hip_pos_push(pos)
        assert lib.q4_hip_f32_to_f16_d(d_raw, IDX_DIM, d_k, IDX_DIM)
        assert lib.q4_hip_qsa_pool_d(d_raw, d_pool, d_wn, IDX_DIM, RATIO, N_ROT, ROPE_BASE,
                                     RMS_EPS)
        rt.sync()
        rt.free(d_k)
        raw[pos] = oracle.quant_f16(k)
        if (pos + 1) % RATIO == 0:
            oracle.qsa_pool(raw, expect, wn, IDX_DIM, RATIO, pos // RATIO, pos // RATIO + 1,
                            N_ROT, ROPE_BASE, RMS_EPS)
    got_raw = rt.download(d_raw, raw.nbytes, np.uint16).reshape(raw.shape)
    assert np.array_equal(got_raw, raw)                 # fp16 RNE store, bit-exact
    got = rt.download(d_pool, pool0.nbytes, np.float32).reshape(pool0.shape)
    done = ~np.isnan(expect[:, 0])
    assert done.sum() == 4                              # blocks 0, 1, 255, 1023
    _close(got[done], expect[done], "pooled blocks")
    assert np.all(np.isnan(got[~done]))
    for p in (d_raw, d_wn, d_pool):
        rt.free(p)


# ----------------------------------------------------------------- prep
@pytest.mark.parametrize("hd,n_rot,n_head,n_tok,pos0", [(256, 64, 16, 1, 262143),
                                                        (128, 64, 4, 9, 100000),
                                                        (256, 256, 2, 3, 5),
                                                        (640, 32, 3, 2, 77),
                                                        (128, 64, 4, 515, 20000),
                                                        (640, 32, 3, 400, 77)])
def test_q_k_prep_match_oracle(rt, oracle, hd, n_rot, n_head, n_tok, pos0):
    lib = rt.lib
    note(f"prep hd={hd} n_rot={n_rot} n_head={n_head} n_tok={n_tok} pos0={pos0}")
    rng = np.random.default_rng(hd + n_tok)
    qg = rng.standard_normal((n_tok, n_head, 2 * hd)).astype(np.float32)
    wn = (1 + 0.2 * rng.standard_normal(hd)).astype(np.float32)
    k = rng.standard_normal((n_tok, n_head, hd)).astype(np.float32) * 2
    d_qg, d_wn, d_k = rt.upload(qg), rt.upload(wn), rt.upload(k)
    d_q, d_g = rt.alloc(k.nbytes), rt.alloc(k.nbytes)
    if n_tok == 1:
        assert lib.q4_hip_qsa_q_prep(d_qg, d_wn, d_q, d_g, n_head, hd, n_rot, pos0,
                                     ROPE_BASE, RMS_EPS)
        assert lib.q4_hip_qsa_k_prep(d_k, d_wn, n_head, hd, n_rot, pos0, ROPE_BASE, RMS_EPS)
    else:
        assert lib.q4_hip_qsa_q_prep_n(d_qg, d_wn, d_q, d_g, n_head, hd, n_rot, pos0,
                                       ROPE_BASE, RMS_EPS, n_tok)
        assert lib.q4_hip_qsa_k_prep_n(d_k, d_wn, n_head, hd, n_rot, pos0, ROPE_BASE,
                                       RMS_EPS, n_tok)
    rt.sync()
    got_q = rt.download(d_q, k.nbytes, np.float32).reshape(k.shape)
    got_g = rt.download(d_g, k.nbytes, np.float32).reshape(k.shape)
    got_k = rt.download(d_k, k.nbytes, np.float32).reshape(k.shape)
    _close(got_q, oracle.qsa_prep(qg[..., :hd], wn, n_rot, pos0, ROPE_BASE, RMS_EPS), "q")
    assert np.array_equal(got_g, qg[..., hd:])
    _close(got_k, oracle.qsa_prep(k, wn, n_rot, pos0, ROPE_BASE, RMS_EPS), "k")
    for p in (d_qg, d_wn, d_k, d_q, d_g):
        rt.free(p)


def test_prep_d_follow_device_position(rt, oracle):
    lib = rt.lib
    hd, n_head, pos = 128, IDX_HEADS, 262142
    rng = np.random.default_rng(3)
    qg = rng.standard_normal((1, n_head, 2 * hd)).astype(np.float32)
    k = rng.standard_normal((1, n_head, hd)).astype(np.float32)
    d_qg, d_k = rt.upload(qg), rt.upload(k)
    d_q, d_g = rt.alloc(k.nbytes), rt.alloc(k.nbytes)
    note("q_prep_d / k_prep_d")
    lib.q4_hip_pos_push(pos)
    assert lib.q4_hip_qsa_q_prep_d(d_qg, None, d_q, d_g, n_head, hd, N_ROT, ROPE_BASE, RMS_EPS)
    assert lib.q4_hip_qsa_k_prep_d(d_k, None, n_head, hd, N_ROT, ROPE_BASE, RMS_EPS)
    rt.sync()
    _close(rt.download(d_q, k.nbytes, np.float32).reshape(k.shape),
           oracle.qsa_prep(qg[..., :hd], None, N_ROT, pos, ROPE_BASE, RMS_EPS), "q_d")
    _close(rt.download(d_k, k.nbytes, np.float32).reshape(k.shape),
           oracle.qsa_prep(k, None, N_ROT, pos, ROPE_BASE, RMS_EPS), "k_d")
    for p in (d_qg, d_k, d_q, d_g):
        rt.free(p)


# ----------------------------------------------------------------- chain
def test_decode_indexer_chain(rt, oracle):
    """f32_to_f16_d -> pool_d -> k_prep_d (indexer q) -> score_d -> topk_d at a
    full 262144-position context; the selection equals the oracle's top-k
    of the GPU's own scores, and those scores match the oracle's."""
    lib = rt.lib
    rng = np.random.default_rng(21)
    max_kv = 262144
    max_blocks = max_kv // RATIO
    pos = max_kv - 1
    raw = raw_keys(rng, max_kv)
    wn = (1 + 0.2 * rng.standard_normal(IDX_DIM)).astype(np.float32)
    qw = (1 + 0.2 * rng.standard_normal(IDX_DIM)).astype(np.float32)
    d_raw, d_wn, d_qw = rt.upload(raw), rt.upload(wn), rt.upload(qw)
    d_pool = rt.alloc(max_blocks * IDX_DIM * 4)
    note("chain: pool rebuild")
    assert lib.q4_hip_qsa_pool(d_raw, d_pool, d_wn, IDX_DIM, RATIO, 0, max_blocks - 1, N_ROT,
                               ROPE_BASE, RMS_EPS)
    k = rng.standard_normal(IDX_DIM).astype(np.float32)
    q = rng.standard_normal((1, IDX_HEADS, IDX_DIM)).astype(np.float32)
    d_k, d_q = rt.upload(k), rt.upload(q)
    d_sc, d_sel = rt.alloc(max_blocks * 4), rt.alloc(WIDTH * 4)
    note("chain: decode step")
    lib.q4_hip_pos_push(pos)
    assert lib.q4_hip_f32_to_f16_d(d_raw, IDX_DIM, d_k, IDX_DIM)
    assert lib.q4_hip_qsa_pool_d(d_raw, d_pool, d_wn, IDX_DIM, RATIO, N_ROT, ROPE_BASE, RMS_EPS)
    assert lib.q4_hip_qsa_k_prep_d(d_q, d_qw, IDX_HEADS, IDX_DIM, N_ROT, ROPE_BASE, RMS_EPS)
    assert lib.q4_hip_qsa_score_d(d_q, d_pool, d_sc, max_blocks, IDX_HEADS, IDX_DIM, RATIO)
    assert lib.q4_hip_qsa_topk_d(d_sc, d_sel, max_blocks, K_BLK, RATIO, WIDTH)
    rt.sync()
    sc = rt.download(d_sc, max_blocks * 4, np.float32)
    sel = rt.download(d_sel, WIDTH * 4, np.int32)
    pool = rt.download(d_pool, max_blocks * IDX_DIM * 4, np.float32).reshape(max_blocks, IDX_DIM)
    qp = rt.download(d_q, q.nbytes, np.float32).reshape(q.shape)
    raw[pos] = oracle.quant_f16(k)
    # the GPU's pool (spot rows incl. the one pool_d completed) and q match the oracle
    rows = np.r_[0:4, 30000:30004, max_blocks - 4:max_blocks]
    want_pool = np.zeros((max_blocks, IDX_DIM), np.float32)
    for b in rows:
        oracle.qsa_pool(raw, want_pool, wn, IDX_DIM, RATIO, b, b + 1, N_ROT, ROPE_BASE, RMS_EPS)
    _close(pool[rows], want_pool[rows], "pool")
    _close(qp, oracle.qsa_prep(q, qw, N_ROT, pos, ROPE_BASE, RMS_EPS), "indexer q")
    want_sc = oracle.qsa_score(qp, pool, 1, max_blocks, max_blocks, IDX_HEADS, IDX_DIM, pos,
                               RATIO)[0]
    _close(sc, want_sc, "scores")
    want_sel = oracle.qsa_topk(sc[None, :], 1, max_blocks, K_BLK, RATIO, pos, WIDTH)[0]
    assert np.array_equal(sel, want_sel)
    for p in (d_raw, d_wn, d_qw, d_pool, d_k, d_q, d_sc, d_sel):
        rt.free(p)


@pytest.mark.parametrize("pos", [2, 3, 7, 1001, 262143])
def test_fused_index_score_matches_separate_calls(rt, pos):
    """q4_hip_qsa_index_score_d == f32_to_f16_d + pool_d + k_prep_d + score_d,
    bit for bit (raw row, pool, scores), and q is left unmodified."""
    lib = rt.lib
    note(f"index_score_d pos={pos}")
    rng = np.random.default_rng(pos + 5)
    max_kv = 262144
    max_blocks = max_kv // RATIO
    n_pos = max(pos + 1, 64)
    raw = raw_keys(rng, max_kv)
    wn = (1 + 0.2 * rng.standard_normal(IDX_DIM)).astype(np.float32)
    qw = (1 + 0.2 * rng.standard_normal(IDX_DIM)).astype(np.float32)
    k = rng.standard_normal(IDX_DIM).astype(np.float32)
    q = rng.standard_normal((IDX_HEADS, IDX_DIM)).astype(np.float32)
    pool0 = (rng.standard_normal((max_blocks, IDX_DIM)) * 0.3).astype(np.float32)
    outs = []
    for fused in (False, True):
        d_raw, d_pool, d_wn, d_qw = rt.upload(raw), rt.upload(pool0), rt.upload(wn), rt.upload(qw)
        d_k, d_q = rt.upload(k), rt.upload(q)
        d_sc = rt.upload(np.full(max_blocks, np.nan, np.float32))
        d_sel = rt.alloc(WIDTH * 4)
        lib.q4_hip_pos_push(pos)
        if fused:
            assert lib.q4_hip_qsa_index_score_d(d_raw, d_pool, d_wn, d_k, d_q, d_qw, d_sc,
                                                max_blocks, IDX_HEADS, IDX_DIM, RATIO, N_ROT,
                                                ROPE_BASE, RMS_EPS)
        else:
            assert lib.q4_hip_f32_to_f16_d(d_raw, IDX_DIM, d_k, IDX_DIM)
            assert lib.q4_hip_qsa_pool_d(d_raw, d_pool, d_wn, IDX_DIM, RATIO, N_ROT, ROPE_BASE,
                                         RMS_EPS)
            assert lib.q4_hip_qsa_k_prep_d(d_q, d_qw, IDX_HEADS, IDX_DIM, N_ROT, ROPE_BASE,
                                           RMS_EPS)
            assert lib.q4_hip_qsa_score_d(d_q, d_pool, d_sc, max_blocks, IDX_HEADS, IDX_DIM,
                                          RATIO)
        assert lib.q4_hip_qsa_topk_d(d_sc, d_sel, max_blocks, K_BLK, RATIO, WIDTH)
        rt.sync()
        outs.append((rt.download(d_raw, raw.nbytes, np.uint16)[:n_pos * IDX_DIM],
                     rt.download(d_pool, pool0.nbytes, np.float32),
                     rt.download(d_sc, max_blocks * 4, np.float32),
                     rt.download(d_sel, WIDTH * 4, np.int32),
                     rt.download(d_q, q.nbytes, np.float32)))
        for p in (d_raw, d_pool, d_wn, d_qw, d_k, d_q, d_sc, d_sel):
            rt.free(p)
    (r0, p0, s0, l0, _), (r1, p1, s1, l1, q1) = outs
    assert np.array_equal(r0, r1)
    assert np.array_equal(p0.view(np.uint32), p1.view(np.uint32))
    assert np.array_equal(s0.view(np.uint32), s1.view(np.uint32))
    assert np.array_equal(l0, l1)
    assert np.array_equal(q1.reshape(q.shape), q)      # q untouched by the fused call


def test_index_batch_matches_per_item_calls(rt):
    """q4_hip_qsa_index_batch == per item q4_hip_qsa_index_score_d +
    q4_hip_qsa_topk_d at the item's position, bit for bit, for items of
    different lengths (dense-prefix, completing and non-completing blocks)."""
    import ctypes
    import q4kv
    lib = rt.lib
    rng = np.random.default_rng(77)
    max_kv = 65536 * 4
    max_blocks = max_kv // RATIO
    positions = [2, 1500, 40003, 100007, max_kv - 1]
    items = []
    for pos in positions:
        items.append(dict(pos=pos, raw=raw_keys(rng, max_kv),
                          pool=(rng.standard_normal((max_blocks, IDX_DIM)) * 0.3).astype(np.float32),
                          k=rng.standard_normal(IDX_DIM).astype(np.float32),
                          q=rng.standard_normal((IDX_HEADS, IDX_DIM)).astype(np.float32),
                          wk=(1 + 0.2 * rng.standard_normal(IDX_DIM)).astype(np.float32),
                          wq=(1 + 0.2 * rng.standard_normal(IDX_DIM)).astype(np.float32)))
    results = []
    for batched in (True, False):
        note(f"index batch batched={batched}")
        descs = (q4kv.IndexDesc * len(items))()
        ptrs = []
        for i, it in enumerate(items):
            d = dict(raw=rt.upload(it["raw"]), pool=rt.upload(it["pool"]), wk=rt.upload(it["wk"]),
                     k=rt.upload(it["k"]), q=rt.upload(it["q"]), wq=rt.upload(it["wq"]),
                     sc=rt.upload(np.full(max_blocks, np.nan, np.float32)), sel=rt.alloc(WIDTH * 4))
            ptrs.append(d)
            descs[i] = q4kv.IndexDesc(d["raw"], d["pool"], d["wk"], d["k"], d["q"], d["wq"],
                                      d["sc"], d["sel"], it["pos"])
            if not batched:
                lib.q4_hip_pos_push(it["pos"])
                assert lib.q4_hip_qsa_index_score_d(d["raw"], d["pool"], d["wk"], d["k"], d["q"],
                                                    d["wq"], d["sc"], max_blocks, IDX_HEADS,
                                                    IDX_DIM, RATIO, N_ROT, ROPE_BASE, RMS_EPS)
                assert lib.q4_hip_qsa_topk_d(d["sc"], d["sel"], max_blocks, K_BLK, RATIO, WIDTH)
        if batched:
            dd = rt.alloc(ctypes.sizeof(descs))
            assert lib.q4_hip_h2d(dd, ctypes.addressof(descs), ctypes.sizeof(descs))
            assert lib.q4_hip_qsa_index_batch(dd, len(items), max_blocks, IDX_HEADS, IDX_DIM,
                                              RATIO, N_ROT, ROPE_BASE, RMS_EPS, K_BLK, WIDTH)
        rt.sync()
        res = []
        for d, it in zip(ptrs, items):
            n_vis = (it["pos"] + 1) // RATIO
            res.append((rt.download(d["raw"], it["raw"].nbytes, np.uint16)[
                            it["pos"] * IDX_DIM:(it["pos"] + 1) * IDX_DIM],
                        rt.download(d["pool"], it["pool"].nbytes, np.float32),
                        rt.download(d["sc"], max_blocks * 4, np.float32)[:n_vis],
                        rt.download(d["sel"], WIDTH * 4, np.int32)))
            for p in d.values():
                rt.free(p)
        if batched:
            rt.free(dd)
        results.append(res)
    for i, (a, b) in enumerate(zip(*results)):
        for j in range(4):
            assert np.array_equal(a[j].view(np.uint8), b[j].view(np.uint8)), (positions[i], j)
