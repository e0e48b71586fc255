"""Token geometry of a global-attention layer and the packed slot layout of the kernels.

Frame f holds tokens [f*T, (f+1)*T); the first ``num_special`` are special (camera + registers,
``saf3r/patch/sparse_attention.py:93-107``), the other P = T - num_special are patch tokens, cut
into NBf = ceil(P/64) blocks per frame. The packed layout puts all special tokens first
(padded to a multiple of 64 slots) and then every frame's patch tokens padded to NBf*64 slots,
so every 64-slot tile belongs to one frame (or to the special region). Two per-head variants
use the same buffers: token order (DENSE heads, slot t = token t) and the framed layout
(frame-relative heads, frame f's T tokens in token order at tile f*ceil(T/64)).
"""
from __future__ import annotations

from dataclasses import dataclass

BLOCK = 64
HEAD_DIM = 64


@dataclass(frozen=True)
class Geometry:
    frames: int
    tokens_per_frame: int
    num_special: int = 5

    def __post_init__(self):
        if self.frames <= 0 or self.tokens_per_frame <= 0 or not (0 <= self.num_special < self.tokens_per_frame):
            raise ValueError(f"invalid geometry {self}")

    @classmethod
    def from_tokens(cls, num_tokens: int, tokens_per_frame: int, num_special: int = 5) -> "Geometry":
        if num_tokens % tokens_per_frame:
            raise ValueError(f"{num_tokens} tokens is not a whole number of {tokens_per_frame}-token frames")
        return cls(num_tokens // tokens_per_frame, tokens_per_frame, num_special)

    @property
    def patches(self) -> int:
        return self.tokens_per_frame - self.num_special

    @property
    def blocks_per_frame(self) -> int:
        return -(-self.patches // BLOCK)

    @property
    def num_blocks(self) -> int:
        return self.frames * self.blocks_per_frame

    @property
    def tokens(self) -> int:
        return self.frames * self.tokens_per_frame

    @property
    def special_slots(self) -> int:
        return -(-(self.frames * self.num_special) // BLOCK) * BLOCK

    @property
    def padded_patches(self) -> int:
        return self.blocks_per_frame * BLOCK

    @property
    def slots(self) -> int:
        """Packed slots per head (L)."""
        return self.special_slots + self.frames * self.padded_patches

    @property
    def tiles(self) -> int:
        return self.slots // BLOCK

    @property
    def frame_tiles(self) -> int:
        """Tiles per frame in the framed layout (NBT = ceil(T/64))."""
        return -(-self.tokens_per_frame // BLOCK)

    @property
    def framed_fits(self) -> bool:
        """The framed layout (frame f's T tokens in token order at tile f*NBT) fits the L slots of a
        head: the special tokens fit the padding of a frame's last patch tile, or there are none."""
        return self.frames * self.frame_tiles * BLOCK <= self.slots
