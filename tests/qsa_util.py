"""Independent checks for the QSA indexer: a sort-based brute-force top-k
selection and synthetic indexer inputs. Test infrastructure only."""
from __future__ import annotations

import numpy as np

RATIO, K_BLK, TOPK, IDX_DIM, IDX_HEADS = 4, 512, 2048, 128, 4
WIDTH = TOPK + RATIO - 1          # 2051, src/q4_fwd.c idx_width
ROPE_BASE, RMS_EPS, N_ROT = 1.0e7, 1.0e-6, 64


def keys_of(x: np.ndarray) -> np.ndarray:
    """Order-preserving uint32 image of fp32 values (NumPy bit ops)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return np.where(u & np.uint32(0x80000000), ~u, u | np.uint32(0x80000000)).astype(np.uint32)


def brute_select(row: np.ndarray, pos: int, k_blk: int, ratio: int, width: int) -> np.ndarray:
    """Selection list of one token by full sort: the top `need` blocks under
    (score key descending, block index ascending), emitted as the blocks above
    the need-th key in ascending order, then the blocks equal to it in
    ascending order, each expanded to `ratio` positions; then the causal tail
    n_vis*ratio .. pos; then -1."""
    n_vis = (pos + 1) // ratio
    need = min(n_vis, k_blk)
    w = np.arange(width)
    if need == n_vis:
        return np.where(w <= pos, w, -1).astype(np.int32)
    k = keys_of(row[:n_vis]).astype(np.int64)
    order = np.lexsort((np.arange(n_vis), -k))   # primary: key desc
    top = order[:need]
    thr = k[top[-1]]
    gt = np.sort(top[k[top] > thr])
    eq = np.sort(top[k[top] == thr])
    chosen = np.concatenate([gt, eq])
    exp = (chosen[:, None] * ratio + np.arange(ratio)[None, :]).ravel()
    out = np.full(width, -1, dtype=np.int64)
    m = min(width, exp.size)
    out[:m] = exp[:m]
    tail = n_vis * ratio + (w - exp.size)
    rest = w >= exp.size
    out[rest] = np.where(tail[rest] <= pos, tail[rest], -1)
    return out.astype(np.int32)


def raw_keys(rng: np.random.Generator, n_pos: int, hd: int = IDX_DIM) -> np.ndarray:
    """fp16 raw indexer keys [n_pos][hd] as uint16 bit patterns."""
    return rng.standard_normal((n_pos, hd)).astype(np.float16).view(np.uint16)
