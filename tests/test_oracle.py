"""Pins of the CPU oracle (runs on CPU, no GPU).

Each check is independent of the oracle's own formula: hardware F16C, the
reference's own compiled q4_quant.c (oracle/_ref), closed forms and
invariants, so a dropped term, wrong index or transposed operand fails.
"""
import numpy as np
import pytest

from synth import heads, selection, WIDTH

KINDS = (0, 1, 2)


# --------------------------------------------------------------- fp16 codec
def test_f16_encoder_matches_f16c_exhaustively(oracle):
    # every non-NaN float32 bit pattern vs x86 vcvtps2ph (RNE)
    assert oracle.lib.orc_check_f16c(0, 1 << 32, 1) == 0


def test_f16_decoder_matches_reference_all_codes(oracle):
    if oracle.ref is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    for h in range(65536):
        a = oracle.lib.orc_f16_to_f32(h)
        b = oracle.ref.q4_f16_to_f32(h)
        assert (np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32)) or (
            np.isnan(a) and np.isnan(b)), hex(h)


def test_f16_roundtrip_identity(oracle):
    for h in range(65536):
        if (h & 0x7C00) == 0x7C00 and (h & 0x3FF):
            continue  # NaN payloads
        assert oracle.lib.orc_f16_from_f32(oracle.lib.orc_f16_to_f32(h)) == h


# --------------------------------------------------------------- q8_0
def _blocks(b):
    b = b.reshape(-1, 34)
    return b[:, :2].copy().view(np.uint16)[:, 0], b[:, 2:].view(np.int8)


def test_q8_zero_block(oracle):
    s, q = _blocks(oracle.quant_q8(np.zeros(32, np.float32)))
    assert s[0] == 0 and not q.any()


def test_q8_ramp_block_closed_form(oracle):
    # x_j = j - 16: amax 16, d = 16/127, q_j = rint((j-16)*127/16)
    x = np.arange(32, dtype=np.float32) - 16
    s, q = _blocks(oracle.quant_q8(x))
    d = np.float32(16) / np.float32(127)
    assert s[0] == np.float16(d).view(np.uint16)
    idv = np.float32(1) / d
    want = np.clip(np.rint((x * idv).astype(np.float32)), -127, 127).astype(np.int8)
    assert np.array_equal(q[0], want)
    assert q[0][0] == -127 and q[0][16] == 0


@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_q8_single_unit_value(oracle, sign):
    x = np.zeros(32, np.float32)
    x[5] = sign
    s, q = _blocks(oracle.quant_q8(x))
    assert s[0] == 0x2008  # fp16(1/127)
    assert q[0][5] == int(sign * 127) and np.count_nonzero(q[0]) == 1


def test_q8_invariants_and_reference_dequant(oracle):
    rng = np.random.default_rng(7)
    x = heads(rng, (4096, 2)).ravel()
    x[:32] *= 1e-30  # tiny block: fp32-subnormal scale, fp16 flushes to 0
    x[32:64] *= 1e4  # large block: fp16 scale near its top
    b = oracle.quant_q8(x)
    s, q = _blocks(b)
    assert q.min() >= -127
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(1)
    d = (amax / np.float32(127)).astype(np.float32)
    assert np.array_equal(s, d.astype(np.float16).view(np.uint16))
    # the max-magnitude element maps to +-127 whenever d > 0
    am = np.abs(xb).argmax(1)
    live = d > 0
    assert np.all(np.abs(q[np.arange(len(q)), am][live]) == 127)
    # |q*(1/d) quantisation error| <= 1/2 step in units of d
    idv = np.where(d > 0, np.float32(1) / np.where(d > 0, d, 1), 0).astype(np.float32)
    err = np.abs(q.astype(np.float64) - (xb * idv[:, None]).astype(np.float64))
    assert err.max() <= 0.5 + 1e-6
    # the oracle's dequantiser equals the reference's own q4_dequant_row(Q8_0)
    n = x.size
    mine = oracle.dequant_q8(b, n)
    if oracle.ref is not None:
        import oracle_ffi

        theirs = np.empty(n, np.float32)
        assert oracle.ref.q4_dequant_row(oracle_ffi.Q4_T_Q8_0, b.ctypes.data, n,
                                         theirs.ctypes.data)
        assert np.array_equal(mine.view(np.uint32), theirs.view(np.uint32))


def test_f16_width_matches_numpy_and_reference(oracle):
    rng = np.random.default_rng(3)
    x = heads(rng, (64, 2)).ravel()
    h = oracle.quant_f16(x)
    assert np.array_equal(h, x.astype(np.float16).view(np.uint16))
    if oracle.ref is not None:
        import oracle_ffi

        back = np.empty(x.size, np.float32)
        assert oracle.ref.q4_dequant_row(oracle_ffi.Q4_T_F16, h.ctypes.data, x.size,
                                         back.ctypes.data)
        assert np.array_equal(back, x.astype(np.float16).astype(np.float32))


def test_layout_constants(oracle):
    # src/q4_fwd.c:644-650 bytes/token and :663-665 width tags at the model shape
    assert oracle.lib.orc_kv_token_bytes(2, 2, 256) == 544
    assert oracle.lib.orc_kv_token_bytes(1, 2, 256) == 1024
    assert oracle.lib.orc_kv_token_bytes(0, 2, 256) == 2048
    assert [oracle.lib.orc_kv_tag(k) for k in (2, 1, 0)] == [8, 2, 4]


# --------------------------------------------------------------- attention
def _cache(oracle, x, kind):
    return oracle.encode(x, kind)


def _deq(oracle, x, kind):
    """Values the cache holds, as float64 [n_pos, n_kvh, hd]."""
    b = oracle.encode(x, kind)
    if kind == 2:
        return oracle.dequant_q8(b, x.size).reshape(x.shape).astype(np.float64)
    if kind == 1:
        return b.view(np.float16).astype(np.float64).reshape(x.shape)
    return x.astype(np.float64)


@pytest.mark.parametrize("kind", KINDS)
def test_attn_single_position_returns_v(oracle, kind):
    rng = np.random.default_rng(1)
    hd, n_kvh, n_head = 64, 2, 4
    k, v = heads(rng, (10, n_kvh), hd), heads(rng, (10, n_kvh), hd)
    q = heads(rng, (1, n_head), hd)
    idx = np.array([[7, -1, -1]] * n_kvh, np.int32).ravel()
    out = oracle.attn(q, _cache(oracle, k, kind), _cache(oracle, v, kind), kind, n_head,
                      n_kvh, hd, 1, idx=idx, width=3, tok_stride=6, kvh_stride=3)
    vd = _deq(oracle, v, kind)
    for h in range(n_head):
        assert np.allclose(out[0, h], vd[7, h // 2], rtol=0, atol=1e-6)


@pytest.mark.parametrize("kind", KINDS)
def test_attn_equal_keys_give_mean_of_v(oracle, kind):
    rng = np.random.default_rng(2)
    hd, n_kvh, n_head, n = 32, 1, 2, 50
    k = np.repeat(heads(rng, (1, n_kvh), hd), n, axis=0)
    v = heads(rng, (n, n_kvh), hd)
    q = heads(rng, (1, n_head), hd)
    idx = np.array([3, 9, 17, 42, -1, 11], np.int32)
    out = oracle.attn(q, _cache(oracle, k, kind), _cache(oracle, v, kind), kind, n_head,
                      n_kvh, hd, 1, idx=idx, width=6, tok_stride=6)
    want = _deq(oracle, v, kind)[[3, 9, 17, 42, 11], 0].mean(0)
    assert np.allclose(out[0, 0], want, atol=1e-6) and np.allclose(out[0, 1], want, atol=1e-6)


def test_attn_two_positions_logistic_closed_form(oracle):
    rng = np.random.default_rng(4)
    hd = 32
    k, v = heads(rng, (2, 1), hd), heads(rng, (2, 1), hd)
    q = heads(rng, (1, 1), hd)
    gate = rng.standard_normal((1, 1, hd)).astype(np.float32)
    out = oracle.attn(q, k, v, 0, 1, 1, hd, 1, gate=gate, idx=np.array([0, 1], np.int32),
                      width=2, tok_stride=2, scale=0.25)
    s = 0.25 * (k[:, 0].astype(np.float64) @ q[0, 0].astype(np.float64))
    p0 = 1.0 / (1.0 + np.exp(s[1] - s[0]))
    want = (p0 * v[0, 0] + (1 - p0) * v[1, 0]) / (1.0 + np.exp(-gate[0, 0].astype(np.float64)))
    assert np.allclose(out[0, 0], want, rtol=1e-6, atol=1e-7)


def test_attn_empty_and_padding(oracle):
    rng = np.random.default_rng(5)
    hd = 32
    k, v = heads(rng, (4, 1), hd), heads(rng, (4, 1), hd)
    q = heads(rng, (1, 2), hd)
    out = oracle.attn(q, k, v, 0, 2, 1, hd, 1, idx=np.full(5, -1, np.int32), width=5,
                      tok_stride=5)
    assert not out.any()
    # positions >= max_kv are skipped like padding
    a = oracle.attn(q, k, v, 0, 2, 1, hd, 1, idx=np.array([1, 3, 2], np.int32), width=3,
                    tok_stride=3, max_kv=3)
    b = oracle.attn(q, k, v, 0, 2, 1, hd, 1, idx=np.array([1, -1, 2], np.int32), width=3,
                    tok_stride=3, max_kv=3)
    assert np.array_equal(a, b)


def test_attn_dense_equals_indexed_prefix_and_permutation(oracle):
    rng = np.random.default_rng(6)
    hd, n_kvh, n_head, n_tok, base = 64, 2, 8, 3, 20
    n = base + n_tok
    k, v = heads(rng, (n, n_kvh), hd), heads(rng, (n, n_kvh), hd)
    q = heads(rng, (n_tok, n_head), hd)
    kc, vc = _cache(oracle, k, 2), _cache(oracle, v, 2)
    dense = oracle.attn(q, kc, vc, 2, n_head, n_kvh, hd, n_tok, kv_base=base)
    idx = np.full((n_tok, n), -1, np.int32)
    for t in range(n_tok):
        perm = rng.permutation(base + t + 1)
        idx[t, : perm.size] = perm
    ind = oracle.attn(q, kc, vc, 2, n_head, n_kvh, hd, n_tok, idx=idx, width=n, tok_stride=n)
    assert np.allclose(dense, ind, atol=1e-6)


def test_attn_linear_in_v_and_gqa_mapping(oracle):
    rng = np.random.default_rng(8)
    hd, n_kvh, n_head, n = 32, 2, 4, 30
    k = heads(rng, (n, n_kvh), hd)
    v1, v2 = heads(rng, (n, n_kvh), hd), heads(rng, (n, n_kvh), hd)
    q = heads(rng, (1, n_head), hd)
    idx = selection(rng, n - 1, width=12, n_sink=2, n_recent=4)
    kw = dict(idx=idx, width=12, tok_stride=12)
    o1 = oracle.attn(q, k, v1, 0, n_head, n_kvh, hd, 1, **kw)
    o2 = oracle.attn(q, k, v2, 0, n_head, n_kvh, hd, 1, **kw)
    o12 = oracle.attn(q, k, v1 + v2, 0, n_head, n_kvh, hd, 1, **kw)
    assert np.allclose(o12, o1 + o2, atol=1e-5)
    # swapping the two KV heads swaps the two query-head groups
    ks, vs = k[:, ::-1].copy(), v1[:, ::-1].copy()
    qs = np.concatenate([q[:, 2:], q[:, :2]], axis=1)
    os_ = oracle.attn(qs, ks, vs, 0, n_head, n_kvh, hd, 1, **kw)
    assert np.allclose(os_[:, :2], o1[:, 2:], atol=1e-6)
    assert np.allclose(os_[:, 2:], o1[:, :2], atol=1e-6)


def test_attn_f32_path_close_to_double(oracle):
    rng = np.random.default_rng(9)
    hd, n_kvh, n_head, n = 256, 2, 16, 3000
    k, v = heads(rng, (n, n_kvh), hd), heads(rng, (n, n_kvh), hd)
    q = heads(rng, (1, n_head), hd)
    kc, vc = _cache(oracle, k, 2), _cache(oracle, v, 2)
    sel = np.stack([selection(rng, n - 1) for _ in range(n_kvh)]).ravel()
    kw = dict(idx=sel, width=WIDTH, tok_stride=2 * WIDTH, kvh_stride=WIDTH)
    a = oracle.attn(q, kc, vc, 2, n_head, n_kvh, hd, 1, dbl=True, **kw)
    b = oracle.attn(q, kc, vc, 2, n_head, n_kvh, hd, 1, dbl=False, threads=4, **kw)
    assert np.allclose(a, b, atol=2e-3, rtol=1e-3)


def test_selection_rule():
    rng = np.random.default_rng(10)
    pos = 262143
    s = selection(rng, pos)
    assert s.size == WIDTH == 2051 and (s >= 0).all()
    assert np.all(np.diff(s) > 0)  # sorted, distinct
    assert list(s[:3]) == [0, 1, 2] and list(s[-512:]) == list(range(pos - 511, pos + 1))
    mid = s[3:-512]
    assert mid.min() >= 3 and mid.max() <= pos - 512
    short = selection(rng, 100)
    assert list(short[:101]) == list(range(101)) and (short[101:] == -1).all()


# --------------------------------------------------------------- q8_0 GEMV
def test_gemv_q8_against_reference_dequant(oracle):
    rng = np.random.default_rng(40)
    nrows, ncols = 37, 320
    wf = rng.standard_normal((nrows, ncols)).astype(np.float32)
    w = oracle.quant_q8(wf)
    x = rng.standard_normal(ncols).astype(np.float32)
    y = oracle.gemv_q8(w, nrows, ncols, x, scale=0.5)
    if oracle.ref is not None:   # the reference's own dequantiser
        deq = np.empty(nrows * ncols, np.float32)
        assert oracle.ref.q4_dequant_row(8, w.ctypes.data, nrows * ncols, deq.ctypes.data)
        want = 0.5 * (deq.reshape(nrows, ncols).astype(np.float64) @ x.astype(np.float64))
    else:
        want = 0.5 * (oracle.dequant_q8(w, nrows * ncols).reshape(nrows, ncols).astype(np.float64)
                      @ x.astype(np.float64))
    np.testing.assert_allclose(y, want, rtol=1e-6, atol=1e-5)
    # closed form: a weight row with one +-1 per block... row r = e_{c} picks x[c] (scale 1/127)
    e = np.zeros((3, ncols), np.float32)
    for r, c in enumerate((0, 77, 319)):
        e[r, c] = 1.0
    ye = oracle.gemv_q8(oracle.quant_q8(e), 3, ncols, x)
    d = np.float32(np.float16(1.0 / 127)) * 127
    np.testing.assert_allclose(ye, d * x[[0, 77, 319]], rtol=1e-6)
