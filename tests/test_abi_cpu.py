"""The C-ABI library loads and exports every symbol the public headers
declare; host-layer constants match the reference (no GPU calls)."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

import q4kv

ROOT = Path(__file__).resolve().parent.parent
HEADERS = [ROOT / "include" / "q4kv.h", ROOT / "include" / "q4kv_host.h"]


def declared_functions():
    names = set()
    for h in HEADERS:
        src = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(q4\w+)\s*\(", src, flags=re.M):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(q4kv.LIB_PATH))
    names = declared_functions()
    assert len(names) >= 50
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding covers all of them
    assert names <= set(q4kv.SIGNATURES), sorted(names - set(q4kv.SIGNATURES))


def test_binding_loads():
    q4kv.load()


def test_host_layout_functions():
    lib = q4kv.load()
    assert lib.q4kv_kind_of(b"f32") == 0 and lib.q4kv_kind_of(b"fp32") == 0
    assert lib.q4kv_kind_of(b"f16") == 1 and lib.q4kv_kind_of(b"fp16") == 1
    assert lib.q4kv_kind_of(b"q8") == 2 and lib.q4kv_kind_of(b"anything") == 2
    assert [lib.q4kv_token_bytes(k, 2, 256) for k in (2, 1, 0)] == [544, 1024, 2048]
    assert [lib.q4kv_tag(k) for k in (2, 1, 0)] == [8, 2, 4]
    # 12 QSA layers at ctx 262144 in q8_0: 3.2 GiB (the reference repository's DESIGN.md:62-64)
    gib = lib.q4kv_cache_bytes(2, 12, 2, 256, 262144) / 2**30
    assert abs(gib - 3.19) < 0.01
    assert abs(lib.q4kv_cache_bytes(2, 12, 2, 256, 65536) / 2**30 - 0.80) < 0.01


def test_entry_points_reject_bad_arguments_without_gpu():
    lib = q4kv.load()
    # q4_hip_init was never called in this process: every entry point must
    # refuse rather than touch the device
    assert not lib.q4_hip_ok()
    assert not lib.q4_hip_f32_to_q8(None, None, 32)
    assert not lib.q4_hip_qsa_decode_n(None, None, None, None, None, 16, 2, 256, 1, 0, 8,
                                       0.0625, 2)
    assert lib.q4_hip_malloc(16) is None
