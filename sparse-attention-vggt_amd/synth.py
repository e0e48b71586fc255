"""Seeded synthetic workloads of the benchmark configurations (no datasets or checkpoints).

Structured Q/K/V (the 4- and 32-frame single-layer shapes)
    g = torch.Generator().manual_seed(seed); draw order: Bq, Bv ~ N(0,1) [T, H, 64]; then for each
    frame f: Eq_f, Ek_f, Ev_f ~ N(0,1) [T, H, 64].
    Q_f = s*(Bq + 0.3*Eq_f), K_f = s*(Bq + 0.3*Ek_f), V_f = Bv + 0.3*Ev_f, s = sqrt(3/1.09).
    K shares Q's base, so token t of frame f corresponds to token t of every other frame; unrelated
    logits have std 3 after the 1/8 scale. Token order per frame: camera, 4 registers, 37x37 patches.

Head tables
    round_robin_patterns: head h -> [dense, frame-local, anchor+local, dynamic][h % 4].
    seeded_patterns: counts by largest remainder from the fractions (dynamic 40%, frame-local 25%,
    anchor+local 20%, dense 15%; ties to the earlier category), assigned through
    torch.randperm(H) drawn from seed (16 heads -> 7 / 4 / 3 / 2).
    da3_patterns: 50% dynamic, the rest split evenly across the other three (24 heads -> 12/4/4/4).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from .layout import Geometry
from .ops import ANCHOR_LOCAL, BLOCK_DYNAMIC, DENSE, FRAME_LOCAL

VGGT_TOKENS_PER_FRAME = 1374  # 1 camera + 4 registers + 37 x 37 patches (518 x 518 input, patch 14)
VGGT_PATCH_GRID = (37, 37)
NUM_SPECIAL = 5


@dataclass
class QKVWorkload:
    geom: Geometry
    q: torch.Tensor  # [H, N, 64] fp32
    k: torch.Tensor
    v: torch.Tensor


def structured_qkv(frames: int, heads: int = 16, tokens_per_frame: int = VGGT_TOKENS_PER_FRAME,
                   num_special: int = NUM_SPECIAL, seed: int = 0, device="cpu") -> QKVWorkload:
    T = tokens_per_frame
    g = torch.Generator(device=device).manual_seed(seed)
    s = math.sqrt(3.0 / 1.09)
    shape = (T, heads, 64)
    bq = torch.randn(shape, generator=g, device=device)
    bv = torch.randn(shape, generator=g, device=device)
    q = torch.empty(frames * T, heads, 64, device=device)
    k = torch.empty_like(q)
    v = torch.empty_like(q)
    for f in range(frames):
        eq = torch.randn(shape, generator=g, device=device)
        ek = torch.randn(shape, generator=g, device=device)
        ev = torch.randn(shape, generator=g, device=device)
        sl = slice(f * T, (f + 1) * T)
        q[sl] = s * (bq + 0.3 * eq)
        k[sl] = s * (bq + 0.3 * ek)
        v[sl] = bv + 0.3 * ev
    geom = Geometry(frames, T, num_special)
    return QKVWorkload(geom, q.permute(1, 0, 2).contiguous(), k.permute(1, 0, 2).contiguous(),
                       v.permute(1, 0, 2).contiguous())


def round_robin_patterns(heads: int) -> list[int]:
    cycle = [DENSE, FRAME_LOCAL, ANCHOR_LOCAL, BLOCK_DYNAMIC]
    return [cycle[h % 4] for h in range(heads)]


def _largest_remainder(total: int, fractions) -> list[int]:
    raw = [total * f for f in fractions]
    counts = [int(math.floor(r)) for r in raw]
    order = sorted(range(len(raw)), key=lambda i: (-(raw[i] - counts[i]), i))
    for i in order[: total - sum(counts)]:
        counts[i] += 1
    return counts


def seeded_patterns(heads: int = 16, seed: int = 1, fractions=(0.40, 0.25, 0.20, 0.15)) -> list[int]:
    cats = [BLOCK_DYNAMIC, FRAME_LOCAL, ANCHOR_LOCAL, DENSE]
    counts = _largest_remainder(heads, fractions)
    perm = torch.randperm(heads, generator=torch.Generator().manual_seed(seed)).tolist()
    table = [DENSE] * heads
    pos = 0
    for cat, n in zip(cats, counts):
        for h in perm[pos:pos + n]:
            table[h] = cat
        pos += n
    return table


def da3_patterns(heads: int = 24, seed: int = 1) -> list[int]:
    rest = (1.0 - 0.5) / 3
    return seeded_patterns(heads, seed, (0.5, rest, rest, rest))


def vggt_positions(frames: int, patch_h: int = 37, patch_w: int = 37, num_special: int = NUM_SPECIAL,
                   device="cpu") -> torch.Tensor:
    """Global-layer positions (y, x): patches (row+1, col+1) in row-major order, specials (0, 0)
    (``saf3r/models/official_vggt/models/aggregator.py:225-240``). int32 [F*(ns+h*w), 2]."""
    yy, xx = torch.meshgrid(torch.arange(patch_h), torch.arange(patch_w), indexing="ij")
    patch = torch.stack([yy.flatten(), xx.flatten()], dim=-1) + 1
    frame = torch.cat([torch.zeros(num_special, 2, dtype=torch.long), patch], dim=0)
    return frame.repeat(frames, 1).to(device=device, dtype=torch.int32)
