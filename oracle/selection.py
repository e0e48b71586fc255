"""numpy/ctypes front end of the C selection oracle (``oracle/selection.c``).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference anchors: ``saf3r/triton/topk_utils.py:26-29`` (sortable key),
``saf3r/triton/fused_qk_topk.py:73-100`` (composite key, tie rule, frame-major output),
``saf3r/patch/adaptive_block_value.py:16-24`` (population-weighted block mean),
``saf3r/patch/sparse_attention.py:143-186, 256-273`` (q_probe / stride key sets),
``saf3r/patch/utils.py:54-184`` (token top-k from feature scores, :func:`token_topk_from_scores`).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> str:
    """Compile ``liboracle.so`` with the committed Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        i32, i64, p = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p
        lib.oracle_fkey.argtypes = [ctypes.c_uint32]
        lib.oracle_fkey.restype = ctypes.c_uint32
        lib.oracle_block_pool.argtypes = [p, i64, i32, i32, i32, i32, i32, p]
        lib.oracle_block_pool.restype = None
        lib.oracle_block_scores.argtypes = [p, p, i32, i32, i32, p]
        lib.oracle_block_scores.restype = None
        lib.oracle_frame_topk.argtypes = [p, i32, i32, i32, i32, p]
        lib.oracle_frame_topk.restype = i32
        lib.oracle_global_topk.argtypes = [p, i32, i32, i32, p]
        lib.oracle_global_topk.restype = i32
        lib.oracle_probe_chunk.argtypes = [i32]
        lib.oracle_probe_chunk.restype = i32
        lib.oracle_probe_mean.argtypes = [p, i64, i32, i32, p]
        lib.oracle_probe_mean.restype = None
        lib.oracle_probe_scores.argtypes = [p, p, i64, i32, i32, ctypes.c_float, p]
        lib.oracle_probe_scores.restype = None
        lib.oracle_keyset.argtypes = [p, i32, i32, i32, i32, i32, i32, i32, p]
        lib.oracle_keyset.restype = i32
        _lib = lib
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def fkey(x) -> np.ndarray:
    """Sortable uint32 key of fp32 values (vectorised restatement of the C transform)."""
    b = np.ascontiguousarray(np.asarray(x, dtype=np.float32)).view(np.uint32)
    return np.where(b & np.uint32(0x80000000), ~b, b | np.uint32(0x80000000)).astype(np.uint32)


def fkey_c(bits: int) -> int:
    return int(_load().oracle_fkey(ctypes.c_uint32(bits)))


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round fp32 -> bf16 (nearest-even) and return the 16-bit patterns."""
    b = np.ascontiguousarray(np.asarray(x, dtype=np.float32)).view(np.uint32).astype(np.uint64)
    rounded = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    # NaN stays NaN (quiet); none of the oracle inputs are NaN.
    return rounded.astype(np.uint16)


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def block_pool(x_bf16: np.ndarray, frames: int, tokens_per_frame: int, num_special: int,
               block: int = 64) -> np.ndarray:
    """Pooled patch-block means of one head. ``x_bf16``: uint16 [F*T, D] (bf16 bits)."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    n, d = x.shape
    assert n == frames * tokens_per_frame
    p = tokens_per_frame - num_special
    nbf = -(-p // block)
    out = np.zeros((frames * nbf, d), dtype=np.float32)
    _load().oracle_block_pool(_ptr(x), d, frames, tokens_per_frame, num_special, d, block, _ptr(out))
    return out


def block_scores(pq: np.ndarray, pk: np.ndarray) -> np.ndarray:
    """scores[i, j] = sequential-fmaf dot of pooled query block i and pooled key block j."""
    q = np.ascontiguousarray(pq, dtype=np.float32)
    k = np.ascontiguousarray(pk, dtype=np.float32)
    assert q.shape[1] == k.shape[1]
    out = np.zeros((q.shape[0], k.shape[0]), dtype=np.float32)
    _load().oracle_block_scores(_ptr(q), _ptr(k), q.shape[0], k.shape[0], q.shape[1], _ptr(out))
    return out


def frame_topk(scores: np.ndarray, frames: int, k: int) -> np.ndarray:
    """Per-frame top-k over a [NQ, F*C] score matrix -> int32 [NQ, F*min(k, C)]."""
    s = np.ascontiguousarray(scores, dtype=np.float32)
    nq, nc = s.shape
    assert nc % frames == 0
    c = nc // frames
    ke = min(k, c)
    out = np.full((nq, frames * ke), -1, dtype=np.int32)
    rc = _load().oracle_frame_topk(_ptr(s), nq, frames, c, k, _ptr(out))
    if rc != 0:
        raise ValueError(f"oracle_frame_topk failed ({rc})")
    return out


def global_topk(scores: np.ndarray, k: int) -> np.ndarray:
    s = np.ascontiguousarray(scores, dtype=np.float32)
    nq, nc = s.shape
    ke = min(k, nc)
    out = np.full((nq, ke), -1, dtype=np.int32)
    rc = _load().oracle_global_topk(_ptr(s), nq, nc, k, _ptr(out))
    if rc != 0:
        raise ValueError(f"oracle_global_topk failed ({rc})")
    return out


def block_select(q_bf16: np.ndarray, k_bf16: np.ndarray, frames: int, tokens_per_frame: int,
                 num_special: int, topk: int, block: int = 64, scope: str = "frame") -> np.ndarray:
    """Full block-selection pipeline of one head: pool -> score -> top-k."""
    pq = block_pool(q_bf16, frames, tokens_per_frame, num_special, block)
    pk = block_pool(k_bf16, frames, tokens_per_frame, num_special, block)
    s = block_scores(pq, pk)
    if scope == "frame":
        return frame_topk(s, frames, topk)
    return global_topk(s, topk)


KEYSET_STRIDE, KEYSET_TOPK = 0, 1


def probe_chunk(n: int) -> int:
    return int(_load().oracle_probe_chunk(n))


def _as_f32_rows(x: np.ndarray) -> np.ndarray:
    """fp32 rows from fp32 values or bf16 bit patterns (uint16, converted exactly)."""
    x = np.asarray(x)
    if x.dtype == np.uint16:
        return bf16_to_f32(x)
    return np.ascontiguousarray(x, dtype=np.float32)


def probe_mean(q: np.ndarray) -> np.ndarray:
    """Mean query of one head over the given rows [N, D] (fp32 values or bf16 bits), in row order."""
    q = np.ascontiguousarray(_as_f32_rows(q))
    n, d = q.shape
    out = np.zeros(d, dtype=np.float32)
    _load().oracle_probe_mean(_ptr(q), d, n, d, _ptr(out))
    return out


def probe_scores(qbar: np.ndarray, k: np.ndarray, scale: float | None = None) -> np.ndarray:
    """score[t] = sequential-fmaf(qbar . k[t]) * scale (scale defaults to 1/sqrt(D)); k [N, D] fp32 values
    or bf16 bits."""
    qb = np.ascontiguousarray(qbar, dtype=np.float32)
    k = np.ascontiguousarray(_as_f32_rows(k))
    n, d = k.shape
    out = np.zeros(n, dtype=np.float32)
    sc = float(np.float32(1.0 / np.sqrt(d))) if scale is None else float(scale)
    _load().oracle_probe_scores(_ptr(qb), _ptr(k), d, n, d, sc, _ptr(out))
    return out


def keyset(scores, n: int, tokens_per_frame: int, num_special: int, mode: int, param: int, start: int = 0,
           include: bool = False) -> np.ndarray:
    """Sorted key set of one head (see ``oracle_keyset``); ``scores`` may be None for mode 0."""
    s = np.zeros(1, dtype=np.float32) if scores is None else np.ascontiguousarray(scores, dtype=np.float32)
    out = np.zeros(n, dtype=np.int32)
    cnt = _load().oracle_keyset(_ptr(s), n, tokens_per_frame, num_special, mode, param, start, int(bool(include)),
                                _ptr(out))
    if cnt < 0:
        raise ValueError(f"oracle_keyset failed ({cnt})")
    return out[:cnt].copy()


def sortable16(bits: np.ndarray) -> np.ndarray:
    """Order key of bf16 bit patterns: larger score -> larger key, -0.0 below +0.0."""
    b = np.asarray(bits, dtype=np.uint16).astype(np.int64)
    return np.where(b & 0x8000, b ^ 0xFFFF, b ^ 0x8000)


def _best(keys: np.ndarray, idx: np.ndarray, k: int) -> np.ndarray:
    """The k best of (keys, idx) by key, ties to the lower idx, returned in increasing idx order."""
    order = np.lexsort((idx, -keys))[:k]
    return np.sort(idx[order])


def token_topk_from_scores(bits: np.ndarray, frames: int, per_frame: int, topk: int, per_frame_mode: bool = True,
                           exclude_first: bool = False, first_stride: int = 1, cap: int = 0) -> np.ndarray:
    """Selection of ``compute_qk_topk_indices_batched`` (``saf3r/patch/utils.py:54-184``) from bf16 score
    rows ``bits`` uint16 [rows, frames*per_frame]: optional frame-0 samples 0, s, 2s, ... first
    (exclude_first, :94-99, :176-178), then per-frame top-min(topk, P) of frames >= f0
    (:146-156) or the global top-k beyond frame 0 (:157-160), then at most ``cap`` of those (:162-169).
    Order within the kept keys: increasing key index (the reference's sorted=False order is
    unspecified); ties go to the lower key."""
    bits = np.asarray(bits, dtype=np.uint16)
    rows = bits.shape[0]
    f0 = 1 if exclude_first else 0
    keys = sortable16(bits[:, :frames * per_frame])
    first = np.arange(0, per_frame, first_stride, dtype=np.int64) if exclude_first else np.zeros(0, np.int64)
    out = []
    for r in range(rows):
        if per_frame_mode:
            k = min(topk, per_frame)
            parts = [_best(keys[r, f * per_frame:(f + 1) * per_frame], np.arange(per_frame) + f * per_frame, k)
                     for f in range(f0, frames)]
            cand = np.concatenate(parts) if parts else np.zeros(0, np.int64)
        else:
            lo = f0 * per_frame
            n = frames * per_frame - lo
            cand = _best(keys[r, lo:], np.arange(lo, lo + n), min(topk, n))
        if 0 < cap < len(cand):
            cand = _best(keys[r, cand], cand, cap)
        out.append(np.concatenate([first, cand]))
    return np.asarray(out, dtype=np.int32).reshape(rows, -1)

