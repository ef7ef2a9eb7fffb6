"""ctypes binding of the CPU oracle (oracle/build/liboracle.so) and of the
reference's own q4_quant.c build (oracle/_ref/libq4ref.so), for tests only."""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
ORACLE_SO = ROOT / "oracle" / "build" / "liboracle.so"
REF_SO = ROOT / "oracle" / "_ref" / "libq4ref.so"
Q4_T_F16, Q4_T_Q8_0 = 1, 8  # ggml type ids used by src/q4.h


def _ptr(a):
    return None if a is None else a.ctypes.data


class Oracle:
    def __init__(self):
        if not ORACLE_SO.exists():
            subprocess.run(["make", "-C", str(ROOT / "oracle")], check=True,
                           stdout=subprocess.DEVNULL)
        L = self.lib = C.CDLL(str(ORACLE_SO))
        vp, u32, u64, f32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_float
        L.orc_f16_from_f32.restype = C.c_uint16
        L.orc_f16_from_f32.argtypes = [f32]
        L.orc_f16_to_f32.restype = f32
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_quant_q8_0.restype = C.c_int
        L.orc_quant_q8_0.argtypes = [vp, u64, vp]
        L.orc_quant_f16.argtypes = [vp, u64, vp]
        L.orc_dequant_q8_0.argtypes = [vp, u64, vp]
        L.orc_kv_token_bytes.restype = u32
        L.orc_kv_token_bytes.argtypes = [C.c_int, u32, u32]
        L.orc_kv_tag.restype = u32
        L.orc_kv_tag.argtypes = [C.c_int]
        L.orc_kv_append.restype = C.c_int
        L.orc_kv_append.argtypes = [vp, vp, vp, vp, u32, u32, C.c_int, u32]
        L.orc_attn.restype = C.c_int
        L.orc_attn.argtypes = [vp, vp, vp, C.c_int, vp, vp, u32, u32, u32, u32, vp, u32,
                               u64, u64, u32, u32, f32, C.c_int, C.c_int]
        i32 = C.c_int32
        L.orc_qsa_key.restype = u32
        L.orc_qsa_key.argtypes = [f32]
        L.orc_rope_freq.restype = f32
        L.orc_rope_freq.argtypes = [f32, u32, u32]
        L.orc_qsa_prep.restype = C.c_int
        L.orc_qsa_prep.argtypes = [vp, vp, vp, u32, u32, i32, f32, f32]
        L.orc_qsa_pool.restype = C.c_int
        L.orc_qsa_pool.argtypes = [vp, vp, vp, u32, u32, u32, u32, u32, f32, f32]
        L.orc_qsa_score.restype = C.c_int
        L.orc_qsa_score.argtypes = [vp, vp, vp, u32, u32, u32, u32, u32, u32, u32]
        L.orc_qsa_topk.restype = C.c_int
        L.orc_qsa_topk.argtypes = [vp, vp, u32, u32, u32, u32, u32, u32]
        L.orc_gemv_q8_0.restype = C.c_int
        L.orc_gemv_q8_0.argtypes = [vp, u64, u64, vp, vp, f32]
        L.orc_check_f16c.restype = u64
        L.orc_check_f16c.argtypes = [u64, u64, u64]
        self.ref = None
        if REF_SO.exists():
            R = self.ref = C.CDLL(str(REF_SO))
            R.q4_f16_to_f32.restype = f32
            R.q4_f16_to_f32.argtypes = [C.c_uint16]
            R.q4_dequant_row.restype = C.c_bool
            R.q4_dequant_row.argtypes = [u32, vp, u64, vp]

    # --- quantisation -----------------------------------------------------
    def quant_q8(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        out = np.empty(x.size // 32 * 34, dtype=np.uint8)
        assert self.lib.orc_quant_q8_0(_ptr(x), x.size, _ptr(out)) == 0
        return out

    def quant_f16(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        out = np.empty(x.size, dtype=np.uint16)
        self.lib.orc_quant_f16(_ptr(x), x.size, _ptr(out))
        return out

    def dequant_q8(self, b: np.ndarray, n: int) -> np.ndarray:
        b = np.ascontiguousarray(b, dtype=np.uint8)
        out = np.empty(n, dtype=np.float32)
        self.lib.orc_dequant_q8_0(_ptr(b), n, _ptr(out))
        return out

    def encode(self, x: np.ndarray, kind: int) -> np.ndarray:
        """fp32 [..., n] -> cache bytes of width kind (0 f32, 1 f16, 2 q8)."""
        if kind == 2:
            return self.quant_q8(x)
        if kind == 1:
            return self.quant_f16(x).view(np.uint8)
        return np.ascontiguousarray(x, dtype=np.float32).ravel().view(np.uint8)

    # --- attention ----------------------------------------------------------
    def attn(self, q, kc, vc, kind, n_head, n_kvh, hd, n_tok, *, gate=None, idx=None,
             width=0, tok_stride=0, kvh_stride=0, kv_base=0, max_kv=None, scale=None,
             dbl=True, threads=1):
        q = np.ascontiguousarray(q, dtype=np.float32)
        gate = None if gate is None else np.ascontiguousarray(gate, dtype=np.float32)
        idx = None if idx is None else np.ascontiguousarray(idx, dtype=np.int32)
        kc = np.ascontiguousarray(kc)
        vc = np.ascontiguousarray(vc)
        out = np.zeros((n_tok, n_head, hd), dtype=np.float32)
        if scale is None:
            scale = 1.0 / np.sqrt(np.float32(hd))
        if max_kv is None:
            max_kv = 1 << 30
        rc = self.lib.orc_attn(_ptr(q), _ptr(kc), _ptr(vc), kind, _ptr(gate), _ptr(out),
                               n_head, n_kvh, hd, n_tok, _ptr(idx), width, tok_stride,
                               kvh_stride, kv_base, max_kv, float(scale), int(dbl), threads)
        assert rc == 0
        return out

    # --- QSA indexer ----------------------------------------------------------
    def qsa_prep(self, x, wn, n_rot, pos0, base, eps):
        """x [n_tok][n_head][hd] -> RMSNorm*wn + RoPE at pos0+t (per head)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        wn = None if wn is None else np.ascontiguousarray(wn, dtype=np.float32)
        out = np.empty_like(x)
        n_tok, n_head, hd = x.shape
        for t in range(n_tok):
            for h in range(n_head):
                assert self.lib.orc_qsa_prep(_ptr(x[t, h]), _ptr(out[t, h]), _ptr(wn), hd,
                                             n_rot, pos0 + t, base, eps) == 0
        return out

    def qsa_pool(self, raw, pool, wn, hd, ratio, b0, b1, n_rot, base, eps):
        raw = np.ascontiguousarray(raw, dtype=np.uint16)
        wn = None if wn is None else np.ascontiguousarray(wn, dtype=np.float32)
        assert pool.dtype == np.float32 and pool.flags.c_contiguous
        assert self.lib.orc_qsa_pool(_ptr(raw), _ptr(pool), _ptr(wn), hd, ratio, b0, b1,
                                     n_rot, base, eps) == 0
        return pool

    def qsa_score(self, q, pool, n_tok, n_blocks, stride, n_head, hd, pos0, ratio, out=None):
        q = np.ascontiguousarray(q, dtype=np.float32)
        pool = np.ascontiguousarray(pool, dtype=np.float32)
        if out is None:
            out = np.full((n_tok, stride), np.nan, dtype=np.float32)
        assert self.lib.orc_qsa_score(_ptr(q), _ptr(pool), _ptr(out), n_tok, n_blocks,
                                      stride, n_head, hd, pos0, ratio) == 0
        return out

    def qsa_topk(self, score, n_tok, stride, k_blk, ratio, pos0, width):
        score = np.ascontiguousarray(score, dtype=np.float32)
        sel = np.empty((n_tok, width), dtype=np.int32)
        assert self.lib.orc_qsa_topk(_ptr(score), _ptr(sel), n_tok, stride, k_blk, ratio,
                                     pos0, width) == 0
        return sel

    def gemv_q8(self, w, nrows, ncols, x, scale=1.0):
        w = np.ascontiguousarray(w, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(nrows, dtype=np.float32)
        assert self.lib.orc_gemv_q8_0(_ptr(w), nrows, ncols, _ptr(x), _ptr(y), scale) == 0
        return y
