"""KV-cache writes on the GPU vs the CPU oracle: bit-exact bytes."""
import numpy as np
import pytest

import q4kv
from gpu_util import note, quantize_on_gpu
from synth import heads

pytestmark = pytest.mark.gpu


def _tie_block():
    # amax = 127 -> d = 1, 1/d = 1: exact .5 ties exercise round-half-even
    x = np.array([127.0] + [k + 0.5 for k in range(-8, 8)] + [-0.5, 0.5, 2.5, -2.5] +
                 [0.0] * 11, np.float32)
    return x[:32]


def edge_inputs():
    rng = np.random.default_rng(11)
    blocks = [
        np.zeros(32, np.float32),
        -np.zeros(32, np.float32),
        _tie_block(),
        rng.standard_normal(32).astype(np.float32) * np.float32(1e-30),   # scale -> fp16 0
        rng.standard_normal(32).astype(np.float32) * np.float32(1e-6),    # fp16-subnormal scale
        rng.standard_normal(32).astype(np.float32) * np.float32(1e7),     # scale -> fp16 inf
        rng.standard_normal(32).astype(np.float32) * np.float32(6e4),
        np.full(32, -3.25, np.float32),
        np.where(np.arange(32) == 31, 1.0, 1e-3).astype(np.float32),
    ]
    return np.concatenate(blocks)


@pytest.mark.parametrize("n_tok", [1, 8192])
def test_q8_bit_exact_config_distribution(rt, oracle, n_tok):
    note(f"q8 quant n_tok={n_tok}")
    rng = np.random.default_rng(100 + n_tok)
    x = heads(rng, (n_tok, 2))  # config 3 chunk: 8192 x 512 fp32
    dst, nb = quantize_on_gpu(rt, x, q4kv.KV_Q8)
    got = rt.download(dst, nb)
    want = oracle.quant_q8(x)
    assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} bytes differ"


def test_q8_bit_exact_edges_and_ragged(rt, oracle):
    note("q8 quant edges")
    x = edge_inputs()
    rng = np.random.default_rng(12)
    # a ragged length: 33 blocks (not a multiple of the 32-block workgroup)
    x = np.concatenate([x, heads(rng, (1,), 32 * 24).ravel()])
    dst, nb = quantize_on_gpu(rt, x, q4kv.KV_Q8)
    assert np.array_equal(rt.download(dst, nb), oracle.quant_q8(x))


def test_q8_unaligned_buffers(rt, oracle):
    note("q8 quant unaligned")
    rng = np.random.default_rng(13)
    x = heads(rng, (70,), 256).ravel()
    src = rt.upload(np.concatenate([np.zeros(1, np.float32), x]))  # src + 4 B
    dst = rt.alloc(x.size // 32 * 34 + 16)
    assert rt.lib.q4_hip_f32_to_q8(dst + 2, src + 4, x.size)
    rt.sync()
    got = rt.download(dst, x.size // 32 * 34 + 2)[2:]
    assert np.array_equal(got, oracle.quant_q8(x))


def test_q8_rejects_bad_arguments(rt):
    assert not rt.lib.q4_hip_f32_to_q8(None, None, 32)
    p = rt.alloc(64)
    assert not rt.lib.q4_hip_f32_to_q8(p, p, 31)
    assert not rt.lib.q4_hip_f32_to_q8(p, p, 0)


def test_f16_bit_exact(rt, oracle):
    note("f16 quant")
    rng = np.random.default_rng(14)
    x = np.concatenate([heads(rng, (257, 2)).ravel(), edge_inputs(),
                        np.array([65519.0, 65520.0, 1e-8, -6e-8], np.float32)])
    dst, nb = quantize_on_gpu(rt, x, q4kv.KV_F16)
    assert np.array_equal(rt.download(dst, nb, np.uint16), oracle.quant_f16(x))


@pytest.mark.parametrize("kind", [0, 1, 2])
def test_kv_append_at_device_position(rt, oracle, kind):
    note(f"kv_append_d kind={kind}")
    rng = np.random.default_rng(20 + kind)
    n_kvh, hd, max_kv = 2, 256, 64
    bpt = q4kv.token_bytes(kind, n_kvh, hd)
    kc, vc = rt.alloc(max_kv * bpt), rt.alloc(max_kv * bpt)
    hk = np.zeros(max_kv * bpt, np.uint8)
    hv = np.zeros(max_kv * bpt, np.uint8)
    rt.h2d(kc, hk)
    rt.h2d(vc, hv)
    dk, dv = rt.alloc(n_kvh * hd * 4), rt.alloc(n_kvh * hd * 4)
    for pos in (0, 5, 63, 17):
        k, v = heads(rng, (n_kvh,), hd), heads(rng, (n_kvh,), hd)
        rt.h2d(dk, k)
        rt.h2d(dv, v)
        rt.lib.q4_hip_pos_push(pos)
        assert rt.lib.q4_hip_kv_append_d(kc, vc, dk, dv, n_kvh * hd, bpt, kind)
        assert oracle.lib.orc_kv_append(hk.ctypes.data, hv.ctypes.data, k.ctypes.data,
                                        v.ctypes.data, n_kvh * hd, bpt, kind, pos) == 0
    rt.sync()
    assert np.array_equal(rt.download(kc, max_kv * bpt), hk)
    assert np.array_equal(rt.download(vc, max_kv * bpt), hv)


def test_use_stream_roundtrip_keeps_ordering(rt, oracle):
    """q4kv_use_stream(NULL) returns the library to its own stream; pushes of
    the device position keep their order across the pinned staging ring."""
    assert rt.lib.q4kv_use_stream(None)
    n_kvh, hd, max_kv = 2, 256, 40
    bpt = q4kv.token_bytes(2, n_kvh, hd)
    kc, vc = rt.alloc(max_kv * bpt), rt.alloc(max_kv * bpt)
    rt.h2d(kc, np.zeros(max_kv * bpt, np.uint8))
    rt.h2d(vc, np.zeros(max_kv * bpt, np.uint8))
    rng = np.random.default_rng(31)
    hk = np.zeros(max_kv * bpt, np.uint8)
    hv = np.zeros(max_kv * bpt, np.uint8)
    rows = heads(rng, (max_kv, 2, n_kvh))
    dr = rt.upload(rows)
    for pos in range(max_kv):  # more pushes than staging slots, no sync between
        rt.lib.q4_hip_pos_push(pos)
        base = dr + pos * 2 * n_kvh * hd * 4
        assert rt.lib.q4_hip_kv_append_d(kc, vc, base, base + n_kvh * hd * 4, n_kvh * hd,
                                          bpt, 2)
        oracle.lib.orc_kv_append(hk.ctypes.data, hv.ctypes.data, rows[pos, 0].ctypes.data,
                                 rows[pos, 1].ctypes.data, n_kvh * hd, bpt, 2, pos)
    rt.sync()
    assert np.array_equal(rt.download(kc, hk.size), hk)
    assert np.array_equal(rt.download(vc, hv.size), hv)
