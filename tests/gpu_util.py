"""Helpers shared by the GPU tests: upload synthetic caches and run the
library's entry points through the C ABI."""
from __future__ import annotations

import sys

import numpy as np

import q4kv


def note(msg: str) -> None:
    """Name the case before a GPU step (flushed, so a fault still shows it)."""
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


def quantize_on_gpu(rt, x: np.ndarray, kind: int) -> tuple[int, int]:
    """Upload fp32 x, write it as a cache of width kind; returns (ptr, nbytes)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    src = rt.upload(x)
    n = x.size
    nbytes = n // 32 * 34 if kind == q4kv.KV_Q8 else n * (2 if kind == q4kv.KV_F16 else 4)
    dst = rt.alloc(nbytes)
    lib = rt.lib
    if kind == q4kv.KV_Q8:
        assert lib.q4_hip_f32_to_q8(dst, src, n)
    elif kind == q4kv.KV_F16:
        assert lib.q4_hip_f32_to_f16(dst, src, n)
    else:
        assert lib.q4_hip_copy(dst, src, n)
    rt.sync()
    rt.free(src)
    return dst, nbytes
