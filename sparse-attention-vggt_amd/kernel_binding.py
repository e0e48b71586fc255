"""Kernel-level drop-in: the reference's two Triton entry points bound to the C ABI with ctypes.

These are the functions a maintainer would put in place of the reference's Triton call sites, with
the reference's names, arguments and output shapes and dtypes:

- ``fused_sparse_topk_attention(q, k, v, kv_indices, scale=None)`` and its TopK > 2048 variant
  ``fused_sparse_topk_attention_2`` (``saf3r/triton/sparse_topk_attention.py:115-166, 261-286``):
  q [N, D], k [Nk, D], v [Nk, Dv], kv_indices [N, TopK] -> out [N, Dv] in ``v.dtype``; q, k and v are
  used as fp32 (the reference upcasts them), the fp32 result is rounded once to ``v.dtype``.
- ``compute_qk_topk_indices_fused(q, k, topk, num_toks_per_img)``
  (``saf3r/triton/fused_qk_topk.py:120-217``): q [B, Nq, D], k [B, Nk, D] -> int32
  [B, Nq, (Nk / num_toks_per_img) * min(topk, num_toks_per_img)], per-frame top-k of bf16 q.k, frame-major,
  score descending, ties to the lower key. Every batch element is computed (one C call each, on the
  current stream, sharing one score workspace).

This build supports D = Dv = 64 (VGGT's head_dim); other sizes raise ``ValueError`` (the reference
autotunes BLOCK_D for any D). The reference's assertions are ``ValueError``s here; a C-ABI failure
raises ``RuntimeError`` with the library's message. There is no CPU path: tensors must be on the GPU
(the reference's CPU fallback ``_reference_perframe``, ``fused_qk_topk.py:105-117``, is not bound).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib, ops

HEAD_DIM = 64


def _rows(t: torch.Tensor) -> _lib.Rows:
    """A plain [n, 64] row matrix (``saf3r_rows`` {ptr, row stride, 0, all rows one frame, 0})."""
    return _lib.Rows(t.data_ptr(), t.stride(0), 0, 1 << 62, 0)


def _check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(_lib.load().saf3r_last_error().decode(errors="replace"))


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def fused_sparse_topk_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kv_indices: torch.Tensor,
                                scale: float | None = None) -> torch.Tensor:
    """``out[i] = sum_j softmax_j(q[i] . k[idx[i, j]] * scale) v[idx[i, j]]`` (entries < 0 or >= Nk
    are skipped); ``scale`` defaults to 1/sqrt(D). A stride-0 ``kv_indices`` row view shares one list."""
    if not (q.is_cuda and k.is_cuda and v.is_cuda and kv_indices.is_cuda):
        raise ValueError("fused_sparse_topk_attention takes GPU tensors")
    if q.dim() != 2 or k.dim() != 2 or v.dim() != 2 or kv_indices.dim() != 2:
        raise ValueError("q [N, D], k [Nk, D], v [Nk, Dv] and kv_indices [N, TopK] must be 2-D")
    N, D = q.shape
    if D != HEAD_DIM or k.shape[1] != D or v.shape[1] != HEAD_DIM:
        raise ValueError(f"this build supports D = Dv = {HEAD_DIM} (got D {D}, k {k.shape[1]}, Dv {v.shape[1]})")
    if k.shape[0] != v.shape[0] or kv_indices.shape[0] != N:
        raise ValueError("k and v need the same rows, kv_indices one row per query")
    if scale is None:
        scale = 1.0 / (D ** 0.5)
    out_dtype = v.dtype
    if out_dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise ValueError(f"unsupported v dtype {out_dtype}")
    qk32 = not (q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16)
    q = q.to(torch.float32 if qk32 else torch.bfloat16).contiguous()
    k = k.to(torch.float32 if qk32 else torch.bfloat16).contiguous()
    v32 = out_dtype != torch.bfloat16
    v = v.to(torch.float32 if v32 else torch.bfloat16).contiguous()
    idx = kv_indices
    if idx.stride(1) != 1:
        idx = idx.contiguous()
    idx = idx.to(torch.int32)
    out = torch.empty(N, HEAD_DIM, device=q.device, dtype=torch.float32 if v32 else torch.bfloat16)
    if N == 0:
        return out.to(out_dtype)
    flags = (_lib.GATHER_QK_FP32 if qk32 else 0) | (_lib.GATHER_V_FP32 | _lib.GATHER_OUT_FP32 if v32 else 0)
    lib = _lib.load()
    args = (ctypes.byref(_rows(q)), ctypes.byref(_rows(k)), ctypes.byref(_rows(v)), ctypes.c_void_p(idx.data_ptr()),
            idx.stride(0), N, idx.shape[1], k.shape[0], float(scale), flags, ctypes.byref(_rows(out)))
    if ops.gather_sliced(N, idx.shape[1]):  # many rows with long lists: the two-pass kernels
        nbytes = lib.saf3r_gather_attn_workspace_bytes(N, idx.shape[1])
        if nbytes < 0:
            raise RuntimeError(lib.saf3r_last_error().decode(errors="replace"))
        ws = torch.empty(nbytes, device=q.device, dtype=torch.uint8)
        _check(lib.saf3r_gather_attn_fwd_sliced(*args, ctypes.c_void_p(ws.data_ptr()), nbytes, _stream()))
    else:
        _check(lib.saf3r_gather_attn_fwd(*args, _stream()))
    return out if out.dtype == out_dtype else out.to(out_dtype)


# The reference's online-softmax variant for long lists has the same contract; one kernel serves both.
fused_sparse_topk_attention_2 = fused_sparse_topk_attention


def compute_qk_topk_indices_fused(q: torch.Tensor, k: torch.Tensor, topk: int,
                                  num_toks_per_img: int | None = None) -> torch.Tensor:
    """Per-frame top-k key indices of bf16 q.k with fp32 accumulation, for every batch element."""
    if num_toks_per_img is None or num_toks_per_img <= 0:
        raise ValueError("num_toks_per_img must be > 0")
    if q.dim() != 3 or k.dim() != 3 or q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise ValueError("q (B, Nq, D) and k (B, Nk, D) must agree in B and D")
    if k.shape[1] % num_toks_per_img != 0:
        raise ValueError("Nk must be divisible by num_toks_per_img")
    if not (q.is_cuda and k.is_cuda):
        raise ValueError("compute_qk_topk_indices_fused takes GPU tensors")
    B, Nq, D = q.shape
    if D != HEAD_DIM:
        raise ValueError(f"this build supports D = {HEAD_DIM} (got {D})")
    frames = k.shape[1] // num_toks_per_img
    ke = min(topk, num_toks_per_img)
    if topk < 1 or ke > 128:
        raise ValueError("per-frame topk must be in 1 .. 128")
    lib = _lib.load()
    q_bf = q.to(torch.bfloat16).contiguous()
    k_bf = k.to(torch.bfloat16).contiguous()
    out = torch.empty(B, Nq, frames * ke, device=q.device, dtype=torch.int32)
    if B == 0 or Nq == 0:
        return out
    nbytes = lib.saf3r_token_topk_workspace_bytes(Nq, frames, num_toks_per_img, topk)
    if nbytes < 0:
        raise RuntimeError(lib.saf3r_last_error().decode(errors="replace"))
    ws = torch.empty(nbytes, device=q.device, dtype=torch.uint8) if nbytes else None
    for b in range(B):
        _check(lib.saf3r_token_topk(ctypes.byref(_rows(q_bf[b])), ctypes.byref(_rows(k_bf[b])), Nq, frames,
                                    num_toks_per_img, topk, ctypes.c_void_p(out[b].data_ptr()),
                                    ctypes.c_void_p(0 if ws is None else ws.data_ptr()), nbytes, _stream()))
    return out
