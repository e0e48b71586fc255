"""Algorithmic work of a layer: attention FLOP from the allowed (query, key) pairs of each head's
pattern, projection FLOP, and the bytes the block selection must move.

Attention FLOP of a head = 4 * d * |allowed pairs| (QK^T and PV, 2 FLOP per multiply-add); padding
slots and masked pairs are not counted. For block-dynamic heads the pairs are counted from the
actual selection lists (the last patch block of a frame holds P - 64*(NBf-1) tokens); for key-set
heads from the member count of their key set.
"""
from __future__ import annotations

import torch

from .layout import BLOCK, HEAD_DIM, Geometry
from .ops import ANCHOR, ANCHOR_LOCAL, BLOCK_DYNAMIC, BROADCAST, DENSE, FRAME_LOCAL, KEYSET, SKIP, TOKEN_DYNAMIC


def block_population(geom: Geometry, block_ids: torch.Tensor) -> torch.Tensor:
    """Tokens in each global patch block id (0 for ids < 0)."""
    last = geom.patches - BLOCK * (geom.blocks_per_frame - 1)
    b = block_ids.long()
    pop = torch.where(b % geom.blocks_per_frame == geom.blocks_per_frame - 1, last, BLOCK)
    return torch.where(b >= 0, pop, torch.zeros_like(pop))


def dynamic_pairs(geom: Geometry, sel: torch.Tensor) -> int:
    """Allowed pairs of one block-dynamic head: special rows see every key; patch rows of query
    block i see the patch tokens of the blocks listed in sel[i]."""
    keys = block_population(geom, sel).sum(dim=-1)  # [NB]
    rows = block_population(geom, torch.arange(geom.num_blocks, device=sel.device))
    S = geom.frames * geom.num_special
    return int((keys * rows).sum().item()) + S * geom.tokens


def head_pairs(pattern: int, geom: Geometry, sel: torch.Tensor | None = None, topk_width: int = 0,
               keyset_count: int = 0) -> int:
    N, F, T = geom.tokens, geom.frames, geom.tokens_per_frame
    S = F * geom.num_special
    if pattern == DENSE:
        return N * N
    if pattern == FRAME_LOCAL:
        return F * T * T
    if pattern == ANCHOR_LOCAL:
        return T * T + (F - 1) * T * 2 * T
    if pattern == ANCHOR:
        return N * T
    if pattern == SKIP:
        return 0
    if pattern == BLOCK_DYNAMIC:
        return dynamic_pairs(geom, sel)
    if pattern == TOKEN_DYNAMIC:
        return S * N + F * geom.patches * topk_width
    if pattern == KEYSET:
        return N * keyset_count
    if pattern == BROADCAST:  # every row weighs frame 0's T keys (its scores taken from frame 0)
        return F * T * T
    raise ValueError(pattern)


def attention_flops(patterns, geom: Geometry, sel: torch.Tensor | None = None, topk_width: int = 0,
                    keyset_counts=None) -> int:
    """Sum over heads; ``sel`` holds one list per BLOCK_DYNAMIC head and ``keyset_counts`` one member
    count per KEYSET head, each in head order."""
    total = 0
    j = jk = 0
    for p in patterns:
        s = None
        c = 0
        if p == BLOCK_DYNAMIC:
            s = sel[j]
            j += 1
        elif p == KEYSET:
            c = int(keyset_counts[jk])
            jk += 1
        total += head_pairs(p, geom, s, topk_width, c)
    return 4 * HEAD_DIM * total


def projection_flops(num_tokens: int, dim: int) -> int:
    """qkv (dim -> 3*dim) and proj (dim -> dim) Linear layers."""
    return 2 * num_tokens * dim * 4 * dim


def selection_bytes(geom: Geometry, n_heads: int, width: int) -> dict:
    """Bytes the block selection must move for ``n_heads`` block-dynamic heads.
    pool: read the packed Q and K patch rows (bf16), write pooled Q and K (fp32).
    select: read pooled Q and K, write the int32 lists."""
    rows = geom.frames * geom.patches
    pooled = geom.num_blocks * HEAD_DIM * 4
    return {
        "pool": n_heads * (2 * rows * HEAD_DIM * 2 + 2 * pooled),
        "select": n_heads * (2 * pooled + geom.num_blocks * width * 4),
        "fused_path": n_heads * (2 * geom.tokens * HEAD_DIM * 2 + geom.num_blocks * width * 4),
    }
