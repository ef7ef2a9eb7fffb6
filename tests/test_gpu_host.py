"""The C host layer (include/q4kv_host.h) on the GPU: cache allocation and
addressing, width-dispatched writes, the decode append, attention call
sites, and the session K/V image (save / pinned restore / file guard) --
config 4's restore-then-decode at full size."""
import ctypes as C
import os

import numpy as np
import pytest

import q4kv
from gpu_util import note
from synth import WIDTH, assert_attn_close, heads, selection

pytestmark = pytest.mark.gpu


def _open(rt, kind, n_layer, max_kv, n_kvh=2, hd=256):
    c = q4kv.KvCache()
    assert rt.lib.q4kv_cache_open(C.byref(c), kind, n_layer, n_kvh, hd, max_kv)
    return c


def _cache_bytes(rt, c, is_v, layer, n_tok):
    p = rt.lib.q4kv_at(C.byref(c), is_v, layer, 0)
    return rt.download(p, n_tok * c.bpt)


@pytest.mark.parametrize("kind", [0, 1, 2])
def test_write_chunk_append_and_attend(rt, oracle, kind):
    note(f"host layer kind={kind}")
    rng = np.random.default_rng(700 + kind)
    n_layer, max_kv, n_head, hd, n_kvh = 3, 3000, 16, 256, 2
    c = _open(rt, kind, n_layer, max_kv)
    try:
        assert c.bpt == q4kv.token_bytes(kind, n_kvh, hd)
        layer, n0 = 1, 2500
        k, v = heads(rng, (n0 + 1, n_kvh)), heads(rng, (n0 + 1, n_kvh))
        dk, dv = rt.upload(k[:n0]), rt.upload(v[:n0])
        assert rt.lib.q4kv_write_chunk(C.byref(c), layer, 0, dk, dv, n0)
        # context-full guard (src/q4_fwd.c:813-816 semantics)
        assert not rt.lib.q4kv_write_chunk(C.byref(c), layer, max_kv - 10, dk, dv, 11)
        nk, nv = rt.upload(k[n0]), rt.upload(v[n0])
        rt.lib.q4_hip_pos_push(n0)
        assert rt.lib.q4kv_append_d(C.byref(c), layer, nk, nv)
        rt.sync()
        assert np.array_equal(_cache_bytes(rt, c, 0, layer, n0 + 1), oracle.encode(k, kind))
        assert np.array_equal(_cache_bytes(rt, c, 1, layer, n0 + 1), oracle.encode(v, kind))
        kb, vb = oracle.encode(k, kind), oracle.encode(v, kind)
        q = heads(rng, (1, n_head))
        gate = rng.standard_normal((1, n_head, hd)).astype(np.float32)
        dq, dg, do = rt.upload(q), rt.upload(gate), rt.alloc(q.nbytes)
        # dense decode over 0..n0 (the n_all <= width branch of qsa_attend)
        assert rt.lib.q4kv_attend(C.byref(c), layer, dq, dg, do, n_head, 1, n0, None, 0, 0, 0)
        rt.sync()
        got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
        want = oracle.attn(q, kb, vb, kind, n_head, n_kvh, hd, 1, gate=gate, kv_base=n0,
                           max_kv=max_kv, scale=1.0 / 16)
        assert_attn_close(got, want, what="dense attend")
        # sparse decode over a per-KV-head selection
        sel = np.stack([selection(rng, n0) for _ in range(n_kvh)]).ravel()
        di = rt.upload(sel)
        assert rt.lib.q4kv_attend(C.byref(c), layer, dq, None, do, n_head, 1, n0, di, WIDTH,
                                  n_kvh * WIDTH, WIDTH)
        rt.sync()
        got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
        want = oracle.attn(q, kb, vb, kind, n_head, n_kvh, hd, 1, idx=sel, width=WIDTH,
                           tok_stride=n_kvh * WIDTH, kvh_stride=WIDTH, max_kv=max_kv,
                           scale=1.0 / 16)
        assert_attn_close(got, want, what="sparse attend")
    finally:
        rt.lib.q4kv_cache_close(C.byref(c))


def test_image_file_roundtrip_and_guard(rt, tmp_path):
    note("session image file")
    rng = np.random.default_rng(710)
    c = _open(rt, 2, 2, 512)
    d = _open(rt, 2, 2, 512)
    e = _open(rt, 1, 2, 512)
    try:
        n = 300
        for layer in range(2):
            for is_v in (0, 1):
                x = rng.integers(0, 256, n * c.bpt, dtype=np.uint8)
                rt.h2d(rt.lib.q4kv_at(C.byref(c), is_v, layer, 0), x)
        c.n_kv = n
        path = str(tmp_path / "img.q4kv").encode()
        assert rt.lib.q4kv_image_save_file(C.byref(c), path)
        assert os.path.getsize(path) == 32 + rt.lib.q4kv_image_bytes(C.byref(c), n)
        assert rt.lib.q4kv_image_restore_file(C.byref(d), path) == n and d.n_kv == n
        for layer in range(2):
            for is_v in (0, 1):
                assert np.array_equal(_cache_bytes(rt, c, is_v, layer, n),
                                      _cache_bytes(rt, d, is_v, layer, n))
        # width tag mismatch (q8 image into an f16 cache) is refused, cache left empty
        assert rt.lib.q4kv_image_restore_file(C.byref(e), path) == 0 and e.n_kv == 0
        assert rt.lib.q4kv_image_restore_file(C.byref(d), b"/nonexistent/x") == 0
    finally:
        for x in (c, d, e):
            rt.lib.q4kv_cache_close(C.byref(x))


def test_pipe_streams_odd_chunks_both_ways(rt, tmp_path):
    """The staged file <-> device pipe with a chunk much smaller than the
    sections (many buffer reuses), odd sizes and offsets; a short file fails
    the read and the pipe reports it at finish."""
    note("pipe file <-> device")
    lib = rt.lib
    rng = np.random.default_rng(720)
    sizes = [1, 999, 1000, 1001, 7777, 65536 + 3]
    blobs = [rng.integers(0, 256, n, dtype=np.uint8) for n in sizes]
    path = tmp_path / "pipe.bin"
    hdr = 13
    with open(path, "wb") as f:
        f.write(b"x" * hdr)
        for b in blobs:
            f.write(b.tobytes())
    dst = [rt.alloc(n) for n in sizes]
    p = lib.q4kv_pipe_open(1000)
    assert p
    fd = os.open(path, os.O_RDONLY)
    off = hdr
    for d, n in zip(dst, sizes):
        assert lib.q4kv_pipe_file_to_dev(p, fd, off, d, n)
        off += n
    assert lib.q4kv_pipe_finish(p)
    os.close(fd)
    for d, b in zip(dst, blobs):
        assert np.array_equal(rt.download(d, b.size, np.uint8), b)
    # device -> file at other offsets, read back on the host
    out = tmp_path / "out.bin"
    fd = os.open(out, os.O_WRONLY | os.O_CREAT | os.O_TRUNC, 0o644)
    off = 5
    for d, n in zip(dst, sizes):
        assert lib.q4kv_pipe_dev_to_file(p, fd, off, d, n)
        off += n
    assert lib.q4kv_pipe_finish(p)
    os.close(fd)
    data = np.fromfile(out, np.uint8)
    assert np.array_equal(data[5:], np.concatenate(blobs))
    # a read past the end of the file fails, and finish reports it
    fd = os.open(path, os.O_RDONLY)
    ok = lib.q4kv_pipe_file_to_dev(p, fd, os.path.getsize(path) - 10, dst[-1], sizes[-1])
    assert not ok
    assert not lib.q4kv_pipe_finish(p)           # reports the failure once
    assert lib.q4kv_pipe_finish(p)               # then the pipe is usable again
    os.close(fd)
    lib.q4kv_pipe_close(p)
    for d in dst:
        rt.free(d)


def test_image_file_truncated_body_is_refused(rt, tmp_path):
    note("session image file, truncated")
    rng = np.random.default_rng(711)
    c = _open(rt, 2, 2, 512)
    d = _open(rt, 2, 2, 512)
    try:
        n = 400
        for layer in range(2):
            for is_v in (0, 1):
                rt.h2d(rt.lib.q4kv_at(C.byref(c), is_v, layer, 0),
                       rng.integers(0, 256, n * c.bpt, dtype=np.uint8))
        c.n_kv = n
        path = str(tmp_path / "img.q4kv")
        assert rt.lib.q4kv_image_save_file(C.byref(c), path.encode())
        with open(path, "r+b") as f:
            f.truncate(os.path.getsize(path) - 1)
        d.n_kv = 7
        assert rt.lib.q4kv_image_restore_file(C.byref(d), path.encode()) == 0 and d.n_kv == 0
    finally:
        for x in (c, d):
            rt.lib.q4kv_cache_close(C.byref(x))


def test_config4_restore_100k_image_then_decode(rt, oracle):
    """Config 4: restore a 100000-token q8_0 image of 12 QSA layers from pinned
    host memory into the device layout, then decode 256 tokens (append +
    sparse attention) and check layers 0 and 11 at several tokens."""
    note("config4 restore 100k x 12 layers + 256 decode steps")
    rng = np.random.default_rng(1238)
    n_layer, n_img, n_dec, n_head, hd, n_kvh = 12, 100000, 256, 16, 256, 2
    c = _open(rt, 2, n_layer, n_img + n_dec)
    body_n = rt.lib.q4kv_image_bytes(C.byref(c), n_img)
    assert body_n == 12 * 100000 * 1088
    host = rt.lib.q4_hip_host_alloc(body_n)
    assert host
    try:
        body = np.ctypeslib.as_array(C.cast(host, C.POINTER(C.c_uint8)), shape=(body_n,))
        # real q8_0 bytes for layers 0 and 11 (checked below), random bytes elsewhere
        sec = n_img * c.bpt
        keep = {}
        for layer in range(n_layer):
            for is_v in (0, 1):
                off = (2 * layer + is_v) * sec
                if layer in (0, n_layer - 1):
                    x = heads(rng, (n_img, n_kvh))
                    keep[(layer, is_v)] = x
                    body[off:off + sec] = oracle.quant_q8(x)
                else:
                    body[off:off + sec] = rng.integers(0, 256, sec, dtype=np.uint8)
        assert rt.lib.q4kv_image_restore(C.byref(c), host, n_img, True)
        assert c.n_kv == n_img
        for layer in (0, n_layer - 1):
            for is_v in (0, 1):
                off = (2 * layer + is_v) * sec
                assert np.array_equal(_cache_bytes(rt, c, is_v, layer, n_img),
                                      body[off:off + sec])
        dq, do = rt.alloc(n_head * hd * 4), rt.alloc(n_head * hd * 4)
        dk, dv = rt.alloc(n_kvh * hd * 4), rt.alloc(n_kvh * hd * 4)
        di = rt.alloc(n_kvh * WIDTH * 4)
        hk = {l: oracle.quant_q8(keep[(l, 0)]) for l in (0, n_layer - 1)}
        hv = {l: oracle.quant_q8(keep[(l, 1)]) for l in (0, n_layer - 1)}
        for l in hk:
            hk[l] = np.concatenate([hk[l], np.zeros(n_dec * c.bpt, np.uint8)])
            hv[l] = np.concatenate([hv[l], np.zeros(n_dec * c.bpt, np.uint8)])
        checks = {0, 1, 127, 255}
        for t in range(n_dec):
            pos = n_img + t
            rt.lib.q4_hip_pos_push(pos)
            for layer in range(n_layer):
                k, v = heads(rng, (n_kvh,)), heads(rng, (n_kvh,))
                q = heads(rng, (1, n_head))
                sel = np.stack([selection(rng, pos) for _ in range(n_kvh)]).ravel()
                rt.h2d(dk, k)
                rt.h2d(dv, v)
                rt.h2d(dq, q)
                rt.h2d(di, sel)
                assert rt.lib.q4kv_append_d(C.byref(c), layer, dk, dv)
                assert rt.lib.q4kv_attend(C.byref(c), layer, dq, None, do, n_head, 1, pos, di,
                                          WIDTH, n_kvh * WIDTH, WIDTH)
                if layer in hk:
                    oracle.lib.orc_kv_append(hk[layer].ctypes.data, hv[layer].ctypes.data,
                                             k.ctypes.data, v.ctypes.data, n_kvh * hd, c.bpt,
                                             2, pos)
                    if t in checks:
                        rt.sync()
                        got = rt.download(do, q.nbytes, np.float32).reshape(q.shape)
                        want = oracle.attn(q, hk[layer], hv[layer], 2, n_head, n_kvh, hd, 1,
                                           idx=sel, width=WIDTH, tok_stride=n_kvh * WIDTH,
                                           kvh_stride=WIDTH, max_kv=c.max_kv, scale=1.0 / 16)
                        assert_attn_close(got, want, what=f"token {t} layer {layer}")
        rt.sync()
        for l in hk:
            assert np.array_equal(_cache_bytes(rt, c, 0, l, n_img + n_dec), hk[l])
    finally:
        rt.lib.q4_hip_host_free(host)
        rt.lib.q4kv_cache_close(C.byref(c))
