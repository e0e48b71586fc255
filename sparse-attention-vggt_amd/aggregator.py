"""A VGGT-1B-style aggregator host: DINOv2-L/14 patch embedding, then alternating frame / global
transformer blocks. It is the model the plugin patches in the full-forward workload (64 frames of
518 x 518 images) and in the aggregator tests; its global blocks' ``attn`` modules are what
``patch_model`` replaces.

Shapes and token layout follow the reference's aggregator (read, not imported):
  - ``saf3r/models/official_vggt/models/aggregator.py:49-160`` (constructor: DINOv2 ViT-L/14 with 4
    registers as patch embedding, 24 frame + 24 global ``Block``s of dim 1024 / 16 heads / MLP 4x,
    qk-norm, RoPE base 100, layer scale 0.01, a camera token and 4 register tokens per frame, frame 0
    taking the first of two learned copies),
  - ``aggregator.py:187-322`` (forward: ResNet normalisation, patch tokens from ``x_norm_patchtokens``,
    [camera, registers, patches] per frame, RoPE positions (y+1, x+1) with specials at (0, 0), frame
    blocks over [S, T, C] and global blocks over [1, S*T, C] alternately, every layer's frame and global
    outputs concatenated into the returned list),
  - ``layers/block.py:26-105`` (pre-norm block with layer scale), ``layers/mlp.py`` (Linear-GELU-Linear),
  - ``layers/vision_transformer.py:42-282`` (DINOv2: cls token, learned position embedding, registers
    after cls, final LayerNorm, output dict).
Weights are random (torch's default initialisation, small normal special tokens); there are no
checkpoints in this build.

Frame attention (frame blocks and the DINOv2 blocks: dense attention inside each image) runs on torch's
fused SDPA kernels (flash / memory-efficient only, never the math path), or, with
``frame_attention="saf3r"``, through this package's kernels as the frame-local pattern over the
frames' tokens (identical arithmetic: every token attends to the tokens of its own frame).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import nn

from . import ops
from .layout import HEAD_DIM, Geometry
from .vggt import Attention, RotaryPositionEmbedding2D

RESNET_MEAN = (0.485, 0.456, 0.406)
RESNET_STD = (0.229, 0.224, 0.225)


class LayerScale(nn.Module):
    def __init__(self, dim: int, init_values: float):
        super().__init__()
        self.gamma = nn.Parameter(init_values * torch.ones(dim))

    def forward(self, x):
        return x * self.gamma


class Mlp(nn.Module):
    def __init__(self, dim: int, hidden: int, bias: bool = True):
        super().__init__()
        self.fc1 = nn.Linear(dim, hidden, bias=bias)
        self.act = nn.GELU()
        self.fc2 = nn.Linear(hidden, dim, bias=bias)

    def forward(self, x):
        return self.fc2(self.act(self.fc1(x)))


def frame_local_attention(attn: Attention, x: torch.Tensor, pos, num_special: int) -> torch.Tensor:
    """``attn`` over each frame of x [S, T, C] separately (the frame blocks' attention), through the
    package kernels: qkv Linear, LayerNorm / RoPE packing, the frame-local pattern on every head, proj."""
    S, T, C = x.shape
    H = attn.num_heads
    if attn.head_dim != HEAD_DIM:
        raise NotImplementedError("the kernels are built for head_dim 64")
    geom = Geometry(S, T, num_special)
    qkv = attn.qkv(x.reshape(S * T, C))
    if qkv.dtype != torch.bfloat16:
        qkv = qkv.to(torch.bfloat16)
    qkv = qkv.contiguous()
    ln_q = ln_k = None
    eps = 1e-5
    if isinstance(attn.q_norm, nn.LayerNorm):
        ln_q = (attn.q_norm.weight, attn.q_norm.bias)
        ln_k = (attn.k_norm.weight, attn.k_norm.bias)
        eps = attn.q_norm.eps
    base = p2 = npos = None
    if attn.rope is not None and pos is not None:
        base = float(attn.rope.base_frequency)
        p2 = pos.reshape(-1, 2)
        npos = int(p2.max().item()) + 1
    qp, kp, vp = ops.pack_qkv(qkv, qkv[:, C:], qkv[:, 2 * C:], 3 * C, HEAD_DIM, geom, H, ln_q=ln_q, ln_k=ln_k,
                              ln_eps=eps, pos=p2, rope_base=base, rope_positions=npos)
    out = ops.sparse_attn_fwd(qp, kp, vp, geom, [ops.FRAME_LOCAL] * H)
    y = out.reshape(S, T, C)
    if y.dtype != attn.proj.weight.dtype and not torch.is_autocast_enabled("cuda"):
        y = y.to(attn.proj.weight.dtype)
    return attn.proj_drop(attn.proj(y))


class Block(nn.Module):
    """Pre-norm transformer block: x + ls1(attn(norm1(x))), then x + ls2(mlp(norm2(x)))."""

    def __init__(self, dim: int, num_heads: int, mlp_ratio: float = 4.0, init_values: float | None = None,
                 qk_norm: bool = False, rope=None):
        super().__init__()
        self.norm1 = nn.LayerNorm(dim)
        self.attn = Attention(dim, num_heads, qkv_bias=True, proj_bias=True, qk_norm=qk_norm, rope=rope)
        self.ls1 = LayerScale(dim, init_values) if init_values else nn.Identity()
        self.norm2 = nn.LayerNorm(dim)
        self.mlp = Mlp(dim, int(dim * mlp_ratio))
        self.ls2 = LayerScale(dim, init_values) if init_values else nn.Identity()
        self.frame_attention = "sdpa"  # "saf3r": frame-local pattern of the package kernels (see module doc)
        self.num_special = 0

    def forward(self, x, pos=None):
        h = self.norm1(x)
        if self.frame_attention == "saf3r" and not isinstance(self.attn, Attention):
            raise RuntimeError("frame_attention='saf3r' is for unpatched frame blocks")
        if self.frame_attention == "saf3r":
            a = frame_local_attention(self.attn, h, pos, self.num_special)
        else:
            a = self.attn(h, pos=pos)
        x = x + self.ls1(a)
        return x + self.ls2(self.mlp(self.norm2(x)))


class DinoPatchEmbed(nn.Module):
    """DINOv2 ViT with registers as the aggregator's patch embedding (ViT-L/14: dim 1024, depth 24,
    16 heads, 4 registers; layer scale 1.0, no qk-norm, no RoPE). ``forward`` returns the DINOv2 output
    dict; the aggregator reads ``x_norm_patchtokens``."""

    def __init__(self, img_size: int = 518, patch_size: int = 14, embed_dim: int = 1024, depth: int = 24,
                 num_heads: int = 16, num_register_tokens: int = 4, init_values: float = 1.0):
        super().__init__()
        self.patch_size = patch_size
        self.grid = img_size // patch_size
        self.num_register_tokens = num_register_tokens
        self.proj = nn.Conv2d(3, embed_dim, kernel_size=patch_size, stride=patch_size)
        self.cls_token = nn.Parameter(torch.zeros(1, 1, embed_dim))
        self.pos_embed = nn.Parameter(torch.zeros(1, self.grid * self.grid + 1, embed_dim))
        self.register_tokens = nn.Parameter(torch.zeros(1, num_register_tokens, embed_dim))
        self.blocks = nn.ModuleList([Block(embed_dim, num_heads, 4.0, init_values) for _ in range(depth)])
        for b in self.blocks:
            b.num_special = 1 + num_register_tokens
        self.norm = nn.LayerNorm(embed_dim)
        nn.init.trunc_normal_(self.pos_embed, std=0.02)
        nn.init.normal_(self.cls_token, std=1e-6)
        nn.init.normal_(self.register_tokens, std=1e-6)

    def position_embedding(self, gh: int, gw: int, dtype):
        if gh == self.grid and gw == self.grid:
            return self.pos_embed.to(dtype)
        pe = self.pos_embed.float()
        dim = pe.shape[-1]
        patch = pe[:, 1:].reshape(1, self.grid, self.grid, dim).permute(0, 3, 1, 2)
        patch = F.interpolate(patch, size=(gh, gw), mode="bicubic", antialias=True)
        patch = patch.permute(0, 2, 3, 1).reshape(1, gh * gw, dim)
        return torch.cat([pe[:, :1], patch], dim=1).to(dtype)

    def patchify(self, images: torch.Tensor) -> torch.Tensor:
        """``self.proj`` (a 14x14 convolution with stride 14) as one GEMM over the non-overlapping
        patches: the same weights and the same products, [n, gh*gw, C]. (The convolution path picked a
        direct kernel that took 50 ms for 64 bf16 frames of 518 x 518 on this stack.)"""
        n, c, h, w = images.shape
        p = self.patch_size
        gh, gw = h // p, w // p
        patches = images.reshape(n, c, gh, p, gw, p).permute(0, 2, 4, 1, 3, 5).reshape(n, gh * gw, c * p * p)
        weight = self.proj.weight.reshape(self.proj.out_channels, c * p * p)
        if torch.is_autocast_enabled(patches.device.type):  # autocast casts the operands as for the conv
            return F.linear(patches, weight, self.proj.bias)
        return F.linear(patches, weight.to(patches.dtype), self.proj.bias.to(patches.dtype))

    def forward(self, images: torch.Tensor):
        n, _, h, w = images.shape
        p = self.patch_size
        if h % p or w % p:
            raise AssertionError(f"image size {h}x{w} is not a multiple of the patch size {p}")
        x = self.patchify(images)  # [n, gh*gw, C]
        x = torch.cat([self.cls_token.expand(n, -1, -1).to(x.dtype), x], dim=1)
        x = x + self.position_embedding(h // p, w // p, x.dtype)
        x = torch.cat([x[:, :1], self.register_tokens.expand(n, -1, -1).to(x.dtype), x[:, 1:]], dim=1)
        for blk in self.blocks:
            x = blk(x)
        xn = self.norm(x)
        r = self.num_register_tokens
        return {"x_norm_clstoken": xn[:, 0], "x_norm_regtokens": xn[:, 1:r + 1],
                "x_norm_patchtokens": xn[:, r + 1:], "x_prenorm": x, "masks": None}


def _expand_special(token: torch.Tensor, S: int) -> torch.Tensor:
    """[1, 2, X, C] learned tokens -> [S, X, C]: copy 0 for frame 0, copy 1 for the other frames."""
    first = token[:, 0:1].expand(1, 1, *token.shape[2:])
    rest = token[:, 1:2].expand(1, S - 1, *token.shape[2:])
    return torch.cat([first, rest], dim=1).reshape(S, *token.shape[2:])


class Aggregator(nn.Module):
    def __init__(self, img_size: int = 518, patch_size: int = 14, embed_dim: int = 1024, depth: int = 24,
                 num_heads: int = 16, mlp_ratio: float = 4.0, num_register_tokens: int = 4, rope_freq: float = 100.0,
                 init_values: float = 0.01, dino_depth: int = 24, dino_dim: int = 1024, dino_heads: int = 16,
                 frame_attention: str = "sdpa"):
        super().__init__()
        if dino_dim != embed_dim:
            raise ValueError("the patch embedding width must equal the aggregator width")
        self.patch_embed = DinoPatchEmbed(img_size, patch_size, dino_dim, dino_depth, dino_heads, num_register_tokens)
        self.rope = RotaryPositionEmbedding2D(rope_freq) if rope_freq > 0 else None
        self.frame_blocks = nn.ModuleList([Block(embed_dim, num_heads, mlp_ratio, init_values, True, self.rope)
                                           for _ in range(depth)])
        self.global_blocks = nn.ModuleList([Block(embed_dim, num_heads, mlp_ratio, init_values, True, self.rope)
                                            for _ in range(depth)])
        self.depth = depth
        self.patch_size = patch_size
        self.camera_token = nn.Parameter(torch.randn(1, 2, 1, embed_dim))
        self.register_token = nn.Parameter(torch.randn(1, 2, num_register_tokens, embed_dim))
        nn.init.normal_(self.camera_token, std=1e-6)
        nn.init.normal_(self.register_token, std=1e-6)
        self.patch_start_idx = 1 + num_register_tokens
        self.register_buffer("_resnet_mean", torch.tensor(RESNET_MEAN).view(1, 1, 3, 1, 1), persistent=False)
        self.register_buffer("_resnet_std", torch.tensor(RESNET_STD).view(1, 1, 3, 1, 1), persistent=False)
        self.set_frame_attention(frame_attention)

    def set_frame_attention(self, kind: str):
        """"sdpa" (torch's fused kernels) or "saf3r" (the frame-local pattern of the package kernels) for
        the frame blocks and the patch embedding's blocks."""
        if kind not in ("sdpa", "saf3r"):
            raise ValueError(f"frame attention {kind!r}")
        for b in list(self.frame_blocks) + list(self.patch_embed.blocks):
            b.frame_attention = kind
        for b in self.frame_blocks:
            b.num_special = self.patch_start_idx

    def positions(self, S: int, gh: int, gw: int, device) -> torch.Tensor:
        """[S, T, 2] (y, x): patches (row + 1, col + 1), the special tokens (0, 0)."""
        yy, xx = torch.meshgrid(torch.arange(gh, device=device), torch.arange(gw, device=device), indexing="ij")
        patch = torch.stack([yy.flatten(), xx.flatten()], dim=-1) + 1
        frame = torch.cat([torch.zeros(self.patch_start_idx, 2, dtype=patch.dtype, device=device), patch], dim=0)
        return frame[None].expand(S, -1, -1).contiguous()

    def forward(self, images: torch.Tensor):
        """images [1, S, 3, H, W] in [0, 1] -> (list of [1, S, T, 2C] per layer, patch_start_idx)."""
        B, S, c, H, W = images.shape
        if B != 1:
            raise AssertionError("Currently only support batch size of 1 for simplicity")
        if c != 3:
            raise ValueError(f"Expected 3 input channels, got {c}")
        images = (images - self._resnet_mean.to(images.dtype)) / self._resnet_std.to(images.dtype)
        out = self.patch_embed(images.reshape(S, c, H, W))
        patch_tokens = out["x_norm_patchtokens"] if isinstance(out, dict) else out
        C = patch_tokens.shape[-1]
        dt = patch_tokens.dtype
        tokens = torch.cat([_expand_special(self.camera_token, S).to(dt),
                            _expand_special(self.register_token, S).to(dt), patch_tokens], dim=1)  # [S, T, C]
        T = tokens.shape[1]
        pos = None
        if self.rope is not None:
            pos = self.positions(S, H // self.patch_size, W // self.patch_size, images.device)
        outputs = []
        for i in range(self.depth):
            tokens = self.frame_blocks[i](tokens.reshape(S, T, C), pos=pos)
            frame_out = tokens.reshape(1, S, T, C)
            tokens = self.global_blocks[i](tokens.reshape(1, S * T, C),
                                           pos=None if pos is None else pos.reshape(1, S * T, 2))
            global_out = tokens.reshape(1, S, T, C)
            outputs.append(torch.cat([frame_out, global_out], dim=-1))
        return outputs, self.patch_start_idx


class VGGTAggregatorModel(nn.Module):
    """Holds ``aggregator`` the way VGGT does, so the plugin finds ``model.aggregator.global_blocks``
    and ``model.aggregator.patch_embed``; its forward is the aggregator forward."""

    def __init__(self, **kwargs):
        super().__init__()
        self.aggregator = Aggregator(**kwargs)

    def forward(self, images):
        return self.aggregator(images)


def blurred_frames(frames: int, size: int = 518, sigma: float = 4.0, seed: int = 0, device="cpu",
                   dtype=torch.float32) -> torch.Tensor:
    """[1, frames, 3, size, size] uniform [0, 1] pixels smoothed by a separable Gaussian of ``sigma``
    (radius ceil(3 sigma), reflected borders), from one seeded generator on ``device``."""
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.rand(frames * 3, 1, size, size, generator=g, device=device)
    r = int(math.ceil(3 * sigma))
    t = torch.arange(-r, r + 1, device=device, dtype=torch.float32)
    k = torch.exp(-0.5 * (t / sigma) ** 2)
    k = k / k.sum()
    x = F.conv2d(F.pad(x, (r, r, 0, 0), mode="reflect"), k.view(1, 1, 1, -1))
    x = F.conv2d(F.pad(x, (0, 0, r, r), mode="reflect"), k.view(1, 1, -1, 1))
    return x.reshape(1, frames, 3, size, size).clamp(0, 1).to(dtype)
