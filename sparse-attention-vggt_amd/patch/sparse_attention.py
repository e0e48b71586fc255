"""Head modes of the sparse-config JSON and their kernel patterns.

ref: saf3r/patch/sparse_attention.py:12-90 (mode dispatch; unknown modes raise ValueError),
     :93-107 (get_separate_indices).

Reference modes          kernel pattern
  full                   DENSE
  global_to_frame        FRAME_LOCAL
  all_to_first           ANCHOR
  skip                   SKIP
  dino_topk              TOKEN_DYNAMIC (special rows dense, image rows gather-attend est_topk_idx)
Block patterns (same JSON format, new mode names)
  dense                  DENSE
  frame_local            FRAME_LOCAL
  anchor_local           ANCHOR_LOCAL (frame 0 and the query's own frame)
  block_topk             BLOCK_DYNAMIC (per-head pooled block scores, top-k blocks per frame)
Reference modes without a kernel in this build: stride, q_probe_topk, broadcast_first -> NotImplementedError.
"""
from __future__ import annotations

import torch

from ..ops import ANCHOR, ANCHOR_LOCAL, BLOCK_DYNAMIC, DENSE, FRAME_LOCAL, SKIP, TOKEN_DYNAMIC

MODE_TO_PATTERN = {
    "full": DENSE,
    "dense": DENSE,
    "global_to_frame": FRAME_LOCAL,
    "frame_local": FRAME_LOCAL,
    "anchor_local": ANCHOR_LOCAL,
    "block_topk": BLOCK_DYNAMIC,
    "dino_topk": TOKEN_DYNAMIC,
    "all_to_first": ANCHOR,
    "skip": SKIP,
}
UNBUILT_MODES = ("stride", "q_probe_topk", "broadcast_first")


def pattern_of(cfg: dict) -> int:
    mode = cfg["mode"]
    if mode in MODE_TO_PATTERN:
        return MODE_TO_PATTERN[mode]
    if mode in UNBUILT_MODES:
        raise NotImplementedError(f"mode {mode!r} has no kernel in this build")
    raise ValueError(f"Unsupported mode: {mode}")


def get_separate_indices(num_imgs: int, num_toks_per_img: int, num_special_tokens: int):
    """Special and image token indices (``saf3r/patch/sparse_attention.py:93-107``)."""
    base = torch.arange(num_imgs) * num_toks_per_img
    spec = (base[:, None] + torch.arange(num_special_tokens)[None, :]).reshape(-1)
    img = (base[:, None] + torch.arange(num_special_tokens, num_toks_per_img)[None, :]).reshape(-1)
    return spec, img
