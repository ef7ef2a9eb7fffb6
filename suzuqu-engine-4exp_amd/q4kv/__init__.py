"""ctypes binding of libq4kv.so, the MI355X QSA KV-cache library.

This is the binding a Python caller (tests, the benchmark) uses; C callers
link the same library through include/q4kv.h and include/q4kv_host.h.
Importing never falls back to anything: if the shared library is missing or
lacks a symbol, loading raises.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent.parent
LIB_PATH = PKG_DIR / "lib" / "libq4kv.so"

KV_F32, KV_F16, KV_Q8 = 0, 1, 2
KV_NAMES = {"f32": KV_F32, "f16": KV_F16, "q8": KV_Q8}

_vp, _fp, _ip = C.c_void_p, C.c_void_p, C.c_void_p
_u32, _u64, _i32, _f32, _b = C.c_uint32, C.c_uint64, C.c_int32, C.c_float, C.c_bool


class SeqDesc(C.Structure):
    """One entry of the q4kv_seq_desc array (64 bytes), see include/q4kv.h.
    The batched kernels fetch cache rows in 16-byte pieces, so the caches a
    descriptor names must be 16-byte aligned (include/q4kv.h); construction
    refuses others (device memory from q4_hip_malloc always is)."""

    _fields_ = [
        ("kcache", _vp), ("vcache", _vp), ("q", _vp), ("gate", _vp), ("out", _vp),
        ("idx", _vp), ("n_sel", _u32), ("idx_kvh_stride", _u32), ("max_kv", _u32),
        ("reserved", _u32),
    ]

    def __init__(self, *args, **kw):
        super().__init__(*args, **kw)
        for name in ("kcache", "vcache"):
            ptr = getattr(self, name) or 0
            if ptr % 16:
                raise ValueError(f"q4kv_seq_desc.{name} must be 16-byte aligned (got {ptr:#x})")


assert C.sizeof(SeqDesc) == 64


class StepDesc(C.Structure):
    """q4kv_step_desc of include/q4kv.h (96 bytes): a SeqDesc plus the
    token's K/V rows and their cache position."""

    _fields_ = [("seq", SeqDesc), ("k", _vp), ("v", _vp), ("pos", _u32),
                ("reserved", _u32 * 3)]


assert C.sizeof(StepDesc) == 96


class PrepStepDesc(C.Structure):
    """q4kv_prep_step_desc of include/q4kv.h (128 bytes)."""

    _fields_ = [("step", StepDesc), ("wn_q", _vp), ("wn_k", _vp),
                ("reserved", C.c_uint64 * 2)]


assert C.sizeof(PrepStepDesc) == 128


class OutDesc(C.Structure):
    """q4kv_out_desc of include/q4kv.h."""

    _fields_ = [("w_o", _vp), ("y", _vp)]


class IndexDesc(C.Structure):
    """q4kv_index_desc of include/q4kv.h (80 bytes)."""

    _fields_ = [("raw", _vp), ("pool", _vp), ("wn_k", _vp), ("k_new", _vp), ("q", _vp),
                ("wn_q", _vp), ("score", _vp), ("sel", _vp), ("pos", _u32),
                ("reserved", _u32 * 3)]


assert C.sizeof(IndexDesc) == 80


class AppendDesc(C.Structure):
    """q4kv_append_desc of include/q4kv.h (40 bytes)."""

    _fields_ = [("kcache", _vp), ("vcache", _vp), ("k", _vp), ("v", _vp), ("pos", _u32),
                ("reserved", _u32)]


class KvCache(C.Structure):
    """q4kv_cache of include/q4kv_host.h."""

    _fields_ = [
        ("kind", C.c_int), ("n_layer", _u32), ("n_kvh", _u32), ("hd", _u32),
        ("max_kv", _u32), ("bpt", _u32), ("n_kv", _u32), ("d_k", _vp), ("d_v", _vp),
    ]


# name -> (restype, argtypes). Every symbol include/q4kv.h and
# include/q4kv_host.h declare.
SIGNATURES = {
    "q4_hip_init": (_b, []),
    "q4_hip_shutdown": (None, []),
    "q4_hip_ok": (_b, []),
    "q4_hip_malloc": (_vp, [C.c_size_t]),
    "q4_hip_free": (None, [_vp]),
    "q4_hip_h2d": (_b, [_vp, _vp, C.c_size_t]),
    "q4_hip_d2h": (_b, [_vp, _vp, C.c_size_t]),
    "q4_hip_sync": (None, []),
    "q4_hip_clear": (None, []),
    "q4_hip_d2h_async": (_b, [_vp, _vp, _u64]),
    "q4_hip_h2d_async": (_b, [_vp, _vp, _u64]),
    "q4_hip_stream_sync": (_b, []),
    "q4_hip_copy": (_b, [_vp, _vp, _u64]),
    "q4_hip_graph_begin": (C.c_int, []),
    "q4_hip_graph_end": (_vp, []),
    "q4_hip_graph_nodes": (_u32, [_vp]),
    "q4_hip_graph_launch": (_b, [_vp]),
    "q4_hip_graph_free": (None, [_vp]),
    "q4_hip_pos_push": (None, [_i32]),
    "q4_hip_capturing": (C.c_int, []),
    "q4_hip_pos_dev_ok": (C.c_int, []),
    "q4_hip_f32_to_q8": (_b, [_vp, _vp, _u64]),
    "q4_hip_f32_to_f16": (_b, [_vp, _vp, _u64]),
    "q4_hip_kv_append_d": (_b, [_vp, _vp, _vp, _vp, _u32, _u32, C.c_int]),
    "q4_hip_qsa_q_prep": (_b, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, C.c_int32, _f32, _f32]),
    "q4_hip_qsa_q_prep_n": (_b, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, C.c_int32, _f32, _f32,
                                 _u32]),
    "q4_hip_qsa_q_prep_d": (_b, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _f32, _f32]),
    "q4_hip_qsa_k_prep": (_b, [_vp, _vp, _u32, _u32, _u32, C.c_int32, _f32, _f32]),
    "q4_hip_qsa_k_prep_n": (_b, [_vp, _vp, _u32, _u32, _u32, C.c_int32, _f32, _f32, _u32]),
    "q4_hip_qsa_k_prep_d": (_b, [_vp, _vp, _u32, _u32, _u32, _f32, _f32]),
    "q4_hip_f32_to_f16_d": (_b, [_vp, _u32, _vp, _u64]),
    "q4_hip_qsa_pool": (_b, [_vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _f32, _f32]),
    "q4_hip_qsa_pool_d": (_b, [_vp, _vp, _vp, _u32, _u32, _u32, _f32, _f32]),
    "q4_hip_qsa_score": (_b, [_vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32]),
    "q4_hip_qsa_score_d": (_b, [_vp, _vp, _vp, _u32, _u32, _u32, _u32]),
    "q4_hip_qsa_topk": (_b, [_vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32]),
    "q4_hip_qsa_topk_d": (_b, [_vp, _vp, _u32, _u32, _u32, _u32]),
    "q4_hip_qsa_step_prep_batch": (_b, [_vp, _u32, _u32, _u32, _u32, _f32, C.c_int, _u32,
                                        _u32, _f32, _f32]),
    "q4_hip_qsa_step_out_batch": (_b, [_vp, _vp, _u32, _u32, _u32, _u32, _f32, C.c_int, _u32,
                                       _u32, _f32]),
    "q4_hip_gemv_dd": (_b, [_u32, _vp, _u64, _u64, _vp, _vp, _f32]),
    "q4kv_pipe_open": (_vp, [C.c_size_t]),
    "q4kv_pipe_close": (None, [_vp]),
    "q4kv_pipe_file_to_dev": (_b, [_vp, C.c_int, _u64, _vp, _u64]),
    "q4kv_pipe_dev_to_file": (_b, [_vp, C.c_int, _u64, _vp, _u64]),
    "q4kv_pipe_finish": (_b, [_vp]),
    "q4_hip_qsa_index_batch": (_b, [_vp, _u32, _u32, _u32, _u32, _u32, _u32, _f32, _f32, _u32,
                                    _u32]),
    "q4_hip_qsa_index_score_d": (_b, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32,
                                      _u32, _f32, _f32]),
    "q4_hip_qsa_decode_n": (_b, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32,
                                 _u32, _f32, C.c_int]),
    "q4_hip_qsa_decode_idx": (_b, [_vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32,
                                   _u32, _u32, _f32, C.c_int]),
    "q4_hip_qsa_decode": (_b, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _f32,
                               C.c_int]),
    "q4_hip_qsa_topk_alloc": (_b, []),
    "q4_hip_qsa_decode_idx_kv": (_b, [_vp, _vp, _vp, _vp, _vp, _vp, _u32, _u64, _u64, _u32,
                                      _u32, _u32, _u32, _u32, _f32, C.c_int]),
    "q4_hip_qsa_decode_batch": (_b, [_vp, _u32, _u32, _u32, _u32, _f32, C.c_int, _u32]),
    "q4_hip_qsa_step_batch": (_b, [_vp, _u32, _u32, _u32, _u32, _f32, C.c_int, _u32]),
    "q4_hip_qsa_step_batch_noalloc": (_b, [_vp, _u32, _u32, _u32, _u32, _f32, C.c_int, _u32]),
    "q4_hip_host_alloc": (_vp, [C.c_size_t]),
    "q4_hip_host_free": (None, [_vp]),
    "q4kv_timer_begin": (_b, [C.c_int]),
    "q4kv_timer_end_ms": (C.c_double, [C.c_int]),
    "q4kv_device_info": (C.c_int, [C.c_char_p, C.c_int, C.POINTER(C.c_int),
                                   C.POINTER(C.c_int)]),
    "q4kv_use_stream": (_b, [_vp]),
    "q4kv_prof_begin": (_b, [C.c_int]),
    "q4kv_prof_end": (C.c_int, [C.POINTER(C.c_double)]),
    "q4kv_xcd_group": (C.c_int, [C.c_int]),
    "q4_hip_kv_append_batch": (_b, [_vp, _u32, _u32, _u32, C.c_int]),
    # host layer (include/q4kv_host.h)
    "q4kv_kind_of": (C.c_int, [C.c_char_p]),
    "q4kv_token_bytes": (_u32, [C.c_int, _u32, _u32]),
    "q4kv_cache_bytes": (_u64, [C.c_int, _u32, _u32, _u32, _u32]),
    "q4kv_tag": (_u32, [C.c_int]),
    "q4kv_cache_open": (_b, [C.POINTER(KvCache), C.c_int, _u32, _u32, _u32, _u32]),
    "q4kv_cache_close": (None, [C.POINTER(KvCache)]),
    "q4kv_at": (_vp, [C.POINTER(KvCache), C.c_int, _u32, _u32]),
    "q4kv_write": (_b, [C.POINTER(KvCache), _vp, _vp, _u64]),
    "q4kv_write_chunk": (_b, [C.POINTER(KvCache), _u32, _u32, _vp, _vp, _u32]),
    "q4kv_append_d": (_b, [C.POINTER(KvCache), _u32, _vp, _vp]),
    "q4kv_attend": (_b, [C.POINTER(KvCache), _u32, _vp, _vp, _vp, _u32, _u32, _u32, _vp,
                         _u32, _u64, _u64]),
    "q4kv_image_bytes": (_u64, [C.POINTER(KvCache), _u32]),
    "q4kv_image_restore": (_b, [C.POINTER(KvCache), _vp, _u32, _b]),
    "q4kv_image_save": (_b, [C.POINTER(KvCache), _vp]),
    "q4kv_image_save_file": (_b, [C.POINTER(KvCache), C.c_char_p]),
    "q4kv_image_restore_file": (_u32, [C.POINTER(KvCache), C.c_char_p]),
}

_lib = None


def load(path: os.PathLike | str | None = None) -> C.CDLL:
    """Load libq4kv.so and bind every declared symbol (raises if absent)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(f"libq4kv.so not built at {p}: run __graft_entry__.build()")
    lib = C.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError if the symbol is missing
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


class Runtime:
    """Device memory helpers over the C ABI (initialises the library)."""

    def __init__(self, lib: C.CDLL | None = None):
        self.lib = lib or load()
        if not self.lib.q4_hip_init():
            raise RuntimeError("q4_hip_init failed (no GPU visible?)")
        self._owned: list[int] = []

    def alloc(self, nbytes: int) -> int:
        p = self.lib.q4_hip_malloc(max(int(nbytes), 1))
        if not p:
            raise MemoryError(f"q4_hip_malloc({nbytes}) failed")
        self._owned.append(p)
        return p

    def upload(self, arr: np.ndarray) -> int:
        arr = np.ascontiguousarray(arr)
        p = self.alloc(arr.nbytes)
        self.h2d(p, arr)
        return p

    def h2d(self, dptr: int, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        if arr.nbytes and not self.lib.q4_hip_h2d(dptr, arr.ctypes.data, arr.nbytes):
            raise RuntimeError("q4_hip_h2d failed")

    def download(self, dptr: int, nbytes: int, dtype=np.uint8) -> np.ndarray:
        out = np.empty(int(nbytes), dtype=np.uint8)
        if nbytes and not self.lib.q4_hip_d2h(out.ctypes.data, dptr, int(nbytes)):
            raise RuntimeError("q4_hip_d2h failed")
        return out.view(dtype)

    def free(self, dptr: int) -> None:
        if dptr in self._owned:
            self._owned.remove(dptr)
        self.lib.q4_hip_free(dptr)

    def free_all(self) -> None:
        for p in self._owned:
            self.lib.q4_hip_free(p)
        self._owned.clear()

    def sync(self) -> None:
        if not self.lib.q4_hip_stream_sync():
            raise RuntimeError("q4_hip_stream_sync failed")


def token_bytes(kind: int, n_kvh: int, hd: int) -> int:
    """Bytes per token of one K or V cache (src/q4_fwd.c:644-650)."""
    kvw = n_kvh * hd
    return (kvw // 32) * 34 if kind == KV_Q8 else kvw * (2 if kind == KV_F16 else 4)
