"""The VGGT global-attention module shape that the plugin wraps, for hosts without a VGGT model.

``Attention`` exposes the attributes the wrapper reuses (``qkv``, ``q_norm``, ``k_norm``, ``rope``,
``proj``, ``proj_drop``, ``num_heads``, ``head_dim``) with the layout of
``saf3r/models/official_vggt/layers/attention.py:24-80``: qkv Linear(dim, 3*dim) whose output is
read as [N, 3, H, d]; LayerNorm(d) q/k norms; 2-D RoPE with base frequency 100
(``rope.py:62-188``, ``aggregator.py:69,78``). Its own forward is the dense torch computation
(the unpatched layer) and is not on the accelerated path.

``GlobalAttentionStack`` holds ``aggregator.global_blocks[i].attn`` for ``depth`` layers, the part
of the VGGT-1B aggregator the plugin patches.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn
from torch.nn.attention import SDPBackend, sdpa_kernel


class RotaryPositionEmbedding2D(nn.Module):
    def __init__(self, frequency: float = 100.0, scaling_factor: float = 1.0):
        super().__init__()
        self.base_frequency = frequency
        self.scaling_factor = scaling_factor

    def forward(self, tokens: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        d = tokens.shape[-1] // 2
        exps = torch.arange(0, d, 2, device=tokens.device).float() / d
        inv = 1.0 / (self.base_frequency ** exps)
        ang = positions.to(inv.dtype)[..., None] * inv  # [B, N, 2, d/2]
        ang = torch.cat((ang, ang), dim=-1).to(tokens.dtype)
        cos, sin = ang.cos()[:, None], ang.sin()[:, None]  # [B, 1, N, 2, d]

        def one(t, c, s):
            t1, t2 = t[..., : d // 2], t[..., d // 2:]
            return t * c + torch.cat((-t2, t1), dim=-1) * s

        return torch.cat((one(tokens[..., :d], cos[..., 0, :], sin[..., 0, :]),
                          one(tokens[..., d:], cos[..., 1, :], sin[..., 1, :])), dim=-1)


class Attention(nn.Module):
    def __init__(self, dim: int, num_heads: int = 8, qkv_bias: bool = True, proj_bias: bool = True,
                 attn_drop: float = 0.0, proj_drop: float = 0.0, norm_layer=nn.LayerNorm, qk_norm: bool = False,
                 fused_attn: bool = True, rope=None):
        super().__init__()
        assert dim % num_heads == 0
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.scale = self.head_dim ** -0.5
        self.fused_attn = fused_attn
        self.qkv = nn.Linear(dim, dim * 3, bias=qkv_bias)
        self.q_norm = norm_layer(self.head_dim) if qk_norm else nn.Identity()
        self.k_norm = norm_layer(self.head_dim) if qk_norm else nn.Identity()
        self.attn_drop = nn.Dropout(attn_drop)
        self.proj = nn.Linear(dim, dim, bias=proj_bias)
        self.proj_drop = nn.Dropout(proj_drop)
        self.rope = rope

    def forward(self, x: torch.Tensor, pos=None) -> torch.Tensor:
        B, N, C = x.shape
        qkv = self.qkv(x).reshape(B, N, 3, self.num_heads, self.head_dim).permute(2, 0, 3, 1, 4)
        q, k, v = qkv.unbind(0)
        q, k = self.q_norm(q), self.k_norm(k)
        if self.rope is not None:
            q = self.rope(q, pos)
            k = self.rope(k, pos)
        if q.is_cuda:  # torch's fused kernels only: never the unfused math path on the GPU
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                x = F.scaled_dot_product_attention(q, k, v)
        else:
            x = F.scaled_dot_product_attention(q, k, v)
        x = x.transpose(1, 2).reshape(B, N, C)
        return self.proj_drop(self.proj(x))


class _Block(nn.Module):
    def __init__(self, attn: nn.Module):
        super().__init__()
        self.attn = attn


class _Aggregator(nn.Module):
    def __init__(self, blocks):
        super().__init__()
        self.global_blocks = nn.ModuleList(blocks)


class GlobalAttentionStack(nn.Module):
    """``model.aggregator.global_blocks[i].attn`` for i < depth (VGGT-1B: dim 1024, 16 heads, depth 24,
    qk_norm, RoPE base 100)."""

    def __init__(self, depth: int = 24, dim: int = 1024, num_heads: int = 16, rope_freq: float = 100.0):
        super().__init__()
        rope = RotaryPositionEmbedding2D(rope_freq) if rope_freq > 0 else None
        self.aggregator = _Aggregator(
            [_Block(Attention(dim, num_heads, qkv_bias=True, proj_bias=True, qk_norm=True, rope=rope))
             for _ in range(depth)])
