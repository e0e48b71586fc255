"""Head modes of the sparse-config JSON and their kernel patterns.

ref: saf3r/patch/sparse_attention.py:12-90 (mode dispatch; unknown modes raise ValueError),
     :93-107 (get_separate_indices).

Reference modes          kernel pattern
  full                   DENSE
  global_to_frame        FRAME_LOCAL
  all_to_first           ANCHOR
  skip                   SKIP
  dino_topk              TOKEN_DYNAMIC (special rows dense, image rows gather-attend est_topk_idx);
                         with dino_sp2sp_stride s != 1 TOKEN_DYNAMIC_KEYSET (special rows over keys
                         0, s, 2s, ...)
Block patterns (same JSON format, new mode names)
  dense                  DENSE
  frame_local            FRAME_LOCAL
  anchor_local           ANCHOR_LOCAL (frame 0 and the query's own frame)
  block_topk             BLOCK_DYNAMIC (per-head pooled block scores, top-k blocks per frame)
  stride                 KEYSET (keys start, start + stride, ... plus, with include_as (default
                         True), frame 0 and every special token; start = head % stride with shift)
  q_probe_topk           KEYSET (the N // stride (or min(topk, N), default topk 1024) keys with the
                         best mean-query scores, plus frame 0 and the specials with include_as
                         (default False))
  broadcast_first        BROADCAST (frame 0's attention map applied to every frame's V, :110-131)
q_probe_topk with q_sample_ratio < 1 takes the mean query over the reference's linspace-sampled rows
(``:154-157``); dino_topk with dino_sp2sp_stride != 1 lets its special rows attend every s-th key
(``:199-204``, pattern TOKEN_DYNAMIC_STRIDED over a strided key set).
"""
from __future__ import annotations

import torch

from ..ops import (ANCHOR, ANCHOR_LOCAL, BLOCK_DYNAMIC, BROADCAST, DENSE, FRAME_LOCAL, KEYSET, KEYSET_STRIDE,
                   KEYSET_TOPK, SKIP, TOKEN_DYNAMIC, TOKEN_DYNAMIC_KEYSET, KeySetSpec)

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
    "stride": KEYSET,
    "q_probe_topk": KEYSET,
    "broadcast_first": BROADCAST,
}
UNBUILT_MODES = ()


def pattern_of(cfg: dict) -> int:
    mode = cfg["mode"]
    if mode == "dino_topk" and int(cfg.get("dino_sp2sp_stride", 1)) != 1:
        return TOKEN_DYNAMIC_KEYSET
    if mode in MODE_TO_PATTERN:
        return MODE_TO_PATTERN[mode]
    if mode in UNBUILT_MODES:
        raise NotImplementedError(f"mode {mode!r} has no kernel in this package")
    raise ValueError(f"Unsupported mode: {mode}")


def keyset_spec(cfg: dict, head: int, num_tokens: int) -> KeySetSpec:
    """Key set of a ``stride`` or ``q_probe_topk`` head (``saf3r/patch/sparse_attention.py:56-85``)."""
    mode = cfg["mode"]
    if mode == "stride":
        stride = int(cfg.get("stride", 4))
        start = head % stride if cfg.get("shift", False) else 0
        return KeySetSpec(head, KEYSET_STRIDE, stride, start, bool(cfg.get("include_as", True)))
    if mode == "q_probe_topk":
        if "stride" in cfg:
            k = max(1, num_tokens // int(cfg["stride"]))
        else:
            k = min(int(cfg.get("topk", 1024)), num_tokens)
        return KeySetSpec(head, KEYSET_TOPK, k, 0, bool(cfg.get("include_as", False)),
                          float(cfg.get("q_sample_ratio", 1)))
    if mode == "dino_topk":  # special rows over k[::s] (``sparse_attention.py:199-204``)
        stride = int(cfg.get("dino_sp2sp_stride", 1))
        if stride < 1:
            raise ValueError("dino_sp2sp_stride must be >= 1")
        return KeySetSpec(head, KEYSET_STRIDE, stride, 0, False)
    raise ValueError(f"mode {mode!r} has no key set")


def get_separate_indices(num_imgs: int, num_toks_per_img: int, num_special_tokens: int):
    """Special and image token indices (``saf3r/patch/sparse_attention.py:93-107``)."""
    base = torch.arange(num_imgs) * num_toks_per_img
    spec = (base[:, None] + torch.arange(num_special_tokens)[None, :]).reshape(-1)
    img = (base[:, None] + torch.arange(num_special_tokens, num_toks_per_img)[None, :]).reshape(-1)
    return spec, img
