"""Token top-k from features: the index source of the non-lazy dino_topk path.

ref: saf3r/patch/utils.py:54-184 (compute_qk_topk_indices_batched), saf3r/patch/patch_vggt.py:313-357
(customized_forward: L2-normalised DINO patch tokens of every frame give every query its keys).

The scores of a block of queries are one bf16 batched product, as in the reference (a plain library
GEMM); the selection (per-frame or global top-k, frame-0 samples, the max_topk cap) is the
``saf3r_frame_topk_scores`` kernel. Within the kept keys the order is increasing key index (the
reference's ``torch.topk(sorted=False)`` leaves it unspecified), and ties go to the lower key.
"""
from __future__ import annotations

import torch

from .. import ops


def output_width(num_keys: int, topk: int, per_frame: bool, num_toks_per_img: int | None, max_topk: int,
                 include_first_frame: bool, first_frame_stride: int) -> tuple[int, int, int]:
    """(F_sel, rest_eff, rest_final) as the reference computes them (utils.py:100-128)."""
    if include_first_frame:
        if not num_toks_per_img or num_keys % num_toks_per_img:
            raise AssertionError("num_toks_per_img is required and must divide the key count")
        first = -(-num_toks_per_img // first_frame_stride)
        if first > max_topk:
            raise AssertionError(f"sampled first-frame tokens ({first}) exceed max_topk ({max_topk})")
        f_excl = num_toks_per_img
    else:
        first, f_excl = 0, 0
    if per_frame:
        if not num_toks_per_img or num_keys % num_toks_per_img:
            raise AssertionError("Nk must be divisible by num_toks_per_img when per_frame=True")
        num_imgs = num_keys // num_toks_per_img
        k = min(topk, num_toks_per_img)
        rest_eff = k * (num_imgs - 1 if include_first_frame else num_imgs)
    else:
        rest_eff = topk
    rest_eff = min(rest_eff, num_keys - f_excl)
    rest_final = min(rest_eff, max_topk - first)
    return first, rest_eff, rest_final


def compute_qk_topk_indices_batched(q: torch.Tensor, k: torch.Tensor, topk: int, per_frame: bool = False,
                                    num_toks_per_img: int | None = None, q_blocksize: int = 4096,
                                    max_topk: int = 2048, include_first_frame: bool = False,
                                    first_frame_stride: int = 4) -> torch.Tensor:
    """int32 [B, Nq, F_sel + rest_final] key indices per query (same arguments and output width as
    the reference function). q [B, Nq, D], k [B, Nk, D] on the GPU."""
    if q.dim() != 3 or k.dim() != 3 or q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise AssertionError("q and k must be (B, N, D) with the same B and D")
    if topk <= 0 or first_frame_stride < 1:
        raise AssertionError("topk must be > 0 and first_frame_stride >= 1")
    B, Nq, _ = q.shape
    Nk = k.shape[1]
    first, rest_eff, rest_final = output_width(Nk, topk, per_frame, num_toks_per_img, max_topk,
                                               include_first_frame, first_frame_stride)
    P = num_toks_per_img if (per_frame or include_first_frame) else Nk
    frames = Nk // P
    qb = q.to(torch.bfloat16)
    # keys padded to a multiple of 8 columns: score rows then start on 16-byte boundaries
    nk8 = -(-Nk // 8) * 8
    kt = torch.zeros(B, k.shape[2], nk8, dtype=torch.bfloat16, device=k.device)
    kt[:, :, :Nk] = k.to(torch.bfloat16).transpose(1, 2)
    out = torch.empty(B, Nq, first + rest_final, dtype=torch.int32, device=q.device)
    cap = rest_final if rest_final < rest_eff else 0
    for b in range(B):
        for qs in range(0, Nq, q_blocksize):
            qe = min(qs + q_blocksize, Nq)
            scores = torch.matmul(qb[b, qs:qe], kt[b])[:, :Nk]  # bf16 [Bq, Nk], row stride nk8
            out[b, qs:qe] = ops.frame_topk_scores(scores, frames, P, topk, per_frame_mode=per_frame,
                                                  exclude_first=include_first_frame,
                                                  first_stride=first_frame_stride, cap=cap)
    return out
