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
from .ops import (ANCHOR, ANCHOR_LOCAL, BLOCK_DYNAMIC, BROADCAST, DENSE, FRAME_LOCAL, KEYSET, KEYSET_PATTERNS, SKIP,
                  TOKEN_DYNAMIC, TOKEN_DYNAMIC_KEYSET)


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
    if pattern == TOKEN_DYNAMIC_KEYSET:  # special rows over the strided key set
        return S * keyset_count + F * geom.patches * topk_width
    if pattern == KEYSET:
        return N * keyset_count
    if pattern == BROADCAST:
        raise ValueError("BROADCAST heads are counted by head_flops (scores once, PV per frame)")
    raise ValueError(pattern)


def attention_flops(patterns, geom: Geometry, sel: torch.Tensor | None = None, topk_width: int = 0,
                    keyset_counts=None) -> int:
    """Sum over heads; ``sel`` holds one list per BLOCK_DYNAMIC head and ``keyset_counts`` one member
    count per key-set head (KEYSET, TOKEN_DYNAMIC_KEYSET), each in head order."""
    total = 0
    j = jk = 0
    for p in patterns:
        s = None
        c = 0
        if p == BLOCK_DYNAMIC:
            s = sel[j]
            j += 1
        elif p in KEYSET_PATTERNS:
            c = int(keyset_counts[jk])
            jk += 1
        total += head_flops(p, geom, s, topk_width, c)
    return total


def head_flops(pattern: int, geom: Geometry, sel: torch.Tensor | None = None, topk_width: int = 0,
               keyset_count: int = 0) -> int:
    """Algorithmic FLOP of one head. broadcast_first (``saf3r/patch/sparse_attention.py:110-131``)
    computes frame 0's T x T scores once (2*d*T^2) and applies the map to every frame's values
    (2*d*F*T^2); every other pattern costs 4*d per allowed pair."""
    if pattern == BROADCAST:
        T = geom.tokens_per_frame
        return 2 * HEAD_DIM * T * T + 2 * HEAD_DIM * geom.frames * T * T
    return 4 * HEAD_DIM * head_pairs(pattern, geom, sel, topk_width, keyset_count)


def executed_tile_flops(patterns, geom: Geometry, sel: torch.Tensor | None = None, keyset_counts=None,
                        token_order=None) -> int:
    """FLOP of the 64 x 64 (query tile, key tile) pairs the attention kernel walks, 4 * d * 64 * 64 per
    pair, padding and masked positions included: set against the algorithmic FLOP it shows the padding
    and masking waste. Query tiles: the special region (ceil(F*ns/64) tiles) and NBf patch tiles per
    frame, or ceil(F*T/64) token-order tiles for DENSE heads packed in token order, or ceil(T/64) tiles
    per frame for frame-relative heads in the framed layout (``token_order`` value 2). Key tiles per query
    tile follow each pattern's walk: the special tiles holding the needed frames' special tokens plus
    those frames' patch tiles for the frame-relative patterns, the listed blocks for block-dynamic
    patch rows, ceil(count/64) compact tiles for key sets, ceil(T/64) for broadcast_first."""
    F, NBf, T, ns = geom.frames, geom.blocks_per_frame, geom.tokens_per_frame, geom.num_special
    S = F * ns
    nst = -(-S // BLOCK)
    NT = nst + F * NBf
    ntt = -(-geom.tokens // BLOCK)

    def sp_tiles(f0, f1):  # special tiles holding the special tokens of frames f0..f1
        return 0 if ns == 0 else ((f1 + 1) * ns - 1) // BLOCK - (f0 * ns) // BLOCK + 1

    def frame_rel(anchor, local):
        total = 0
        for st in range(nst):  # special query tiles: the frames whose specials they hold
            f0, f1 = (st * BLOCK) // ns, (min(S, (st + 1) * BLOCK) - 1) // ns
            keys = (sp_tiles(f0, f1) + (f1 - f0 + 1) * NBf) if local else 0
            if anchor and not (local and f0 == 0):
                keys += sp_tiles(0, 0) + NBf
            total += keys
        for f in range(F):  # patch query tiles of frame f
            keys = (sp_tiles(f, f) + NBf) if local else 0
            if anchor and not (local and f == 0):
                keys += sp_tiles(0, 0) + NBf
            total += NBf * keys
        return total

    nbt = geom.frame_tiles
    tiles = 0
    j = jk = 0
    for h, p in enumerate(patterns):
        lay = int(token_order[h]) if token_order is not None else 0
        if p == DENSE:
            tiles += ntt * ntt if lay else NT * NT
        elif lay == 2 and p in (FRAME_LOCAL, ANCHOR_LOCAL, ANCHOR):
            # framed layout: NBT query tiles per frame, each walking one frame (two for the
            # anchor+local rows of frames 1 .. F-1)
            frames_walked = F + (F - 1) if p == ANCHOR_LOCAL else F
            tiles += nbt * nbt * frames_walked
        elif p == FRAME_LOCAL:
            tiles += frame_rel(False, True)
        elif p == ANCHOR_LOCAL:
            tiles += frame_rel(True, True)
        elif p == ANCHOR:
            tiles += frame_rel(True, False)
        elif p == BLOCK_DYNAMIC:
            s = sel[j]
            j += 1
            tiles += nst * NT + int((s >= 0).sum().item())
        elif p == TOKEN_DYNAMIC:
            tiles += nst * NT
        elif p in KEYSET_PATTERNS:
            c = int(keyset_counts[jk])
            jk += 1
            tiles += (NT if p == KEYSET else nst) * (-(-c // BLOCK))
        elif p == BROADCAST:
            ct = -(-T // BLOCK)
            tiles += F * ct * ct
    return 4 * HEAD_DIM * BLOCK * BLOCK * tiles


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
