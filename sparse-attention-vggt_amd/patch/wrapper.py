"""Head-wise sparse attention wrapper: head-config parsing and the accelerated layer forward.

ref: saf3r/patch/wrapper.py:8-106 (BaseHeadwiseSparseAttentionWrapper: head_cfg from groups with
     "full" as default and a ValueError for a head listed twice; lazy first-correspondence-head
     top-k; per-head loop), saf3r/patch/patch_vggt.py:494-510 (the lazy indices are shared with
     every later layer), :575-590 (qkv -> q/k norm -> RoPE -> attention -> proj).

One forward of a layer on the GPU:
  qkv Linear (torch) -> saf3r_pack_qkv (LayerNorm + RoPE + packing; block means of the block-dynamic
  heads) -> [block-dynamic heads: saf3r_block_select_pooled] -> [lazy dino_topk: saf3r_token_topk
  once per forward]
  -> saf3r_sparse_attn_fwd (all heads, one launch) -> [dino_topk image rows: saf3r_gather_attn_fwd]
  -> proj Linear (torch).
Instead of a Python loop over heads, every head runs in the single attention launch.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import ops
from ..layout import HEAD_DIM, Geometry
from .sparse_attention import keyset_spec, pattern_of


class SelectionState:
    """Per-model store of the lazily computed token top-k (``est_topk_idx``), shared by every
    dino_topk head; reset by ``update_args_per_forward``."""

    def __init__(self):
        self.reset()

    def reset(self):
        self.est_topk_idx = None
        self.source_layer = None


def _get(cfg, key, default=None):
    if cfg is None:
        return default
    if isinstance(cfg, dict):
        return cfg.get(key, default)
    return getattr(cfg, key, default)


class BaseHeadwiseSparseAttentionWrapper(nn.Module):
    def __init__(self, orig_module, num_special_tokens, num_heads, **kwargs):
        super().__init__()
        self.orig_module = orig_module
        self.num_special_tokens = num_special_tokens
        self.num_heads = num_heads
        self.layer_idx = kwargs.get("layer_idx", None)
        self.patch_width = kwargs.get("patch_width", None)
        self.patch_height = kwargs.get("patch_height", None)
        self.est_topk_idx = torch.empty(0)
        self.lazy_dino_topk = bool(kwargs.get("lazy_dino_topk", False))
        self.dino_topk = int(kwargs.get("dino_topk", 4))
        self.first_dino_flag = False
        self.block_topk = int(kwargs.get("block_topk", 4))
        self.topk_scope = kwargs.get("topk_scope", "frame")
        self.shared = kwargs.get("shared", None) or SelectionState()
        self.last_selection = None
        # keep_attention: hold the pre-projection attention output [N, H*64] of the last forward in
        # last_attention (for inspection and tests; off by default, it keeps the tensor alive)
        self.keep_attention = False
        self.last_attention = None

        cfg = kwargs.get("config", [])
        self.head_cfg = [{"mode": "full"} for _ in range(num_heads)]
        seen = set()
        for group in cfg:
            group = dict(group)
            ids = group.pop("head_ids")
            for h in ids:
                if h in seen:
                    raise ValueError(f"Head {h} assigned to multiple patterns!")
                seen.add(h)
                self.head_cfg[h].update(group)
        self.patterns = [pattern_of(c) for c in self.head_cfg]
        ks = {int(c.get("topk", self.block_topk)) for c, p in zip(self.head_cfg, self.patterns)
              if p == ops.BLOCK_DYNAMIC}
        if len(ks) > 1:
            raise ValueError(f"block_topk heads of one layer must share one k, got {sorted(ks)}")
        self.layer_block_topk = ks.pop() if ks else self.block_topk
        self.dyn_heads = [h for h, p in enumerate(self.patterns) if p == ops.BLOCK_DYNAMIC]
        self.keyset_heads = [h for h, p in enumerate(self.patterns) if p in ops.KEYSET_PATTERNS]
        self.broadcast_heads = [h for h, p in enumerate(self.patterns) if p == ops.BROADCAST]
        self.last_keysets = None
        self.dino_heads = [h for h, p in enumerate(self.patterns) if p in ops.TOKEN_PATTERNS]
        self.first_dino_head = next((h for h in self.dino_heads if self.head_cfg[h].get("is_first_dino", False)), None)
        # heads whose fp32 q / k (after LayerNorm / RoPE) the kernels read, as the reference reads its fp32
        # values under autocast: the q_probe_topk mean and scores (sparse_attention.py:160-166) and the
        # dino_topk gather (sparse_topk_attention.py:74-80)
        probe = {h for h in self.keyset_heads if self.head_cfg[h]["mode"] == "q_probe_topk"}
        self.fp32_heads = sorted(probe | set(self.dino_heads))
        self.fp32_slot = {h: i for i, h in enumerate(self.fp32_heads)}
        # pack Q with the softmax scale folded in (one bf16 rounding of the fp32 q * scale * log2 e), so
        # that the attention walks skip the running maximum; off for tests that compare the plain layout
        self.prescale_q = True

    def q_scaled_heads(self) -> list[bool]:
        """Heads whose packed Q carries ``ops.prescale_factor()``: every head except the first
        correspondence head of a lazy dino_topk layer, whose packed Q the token top-k reads as the
        reference's q (``fused_qk_topk.py:120-217``)."""
        skip = self.first_dino_head if self.lazy_dino_topk else None
        return [self.prescale_q and h != skip for h in range(self.num_heads)]

    # ------------------------------------------------------------------------------------
    def geometry(self, num_tokens: int) -> Geometry:
        if self.patch_height is None or self.patch_width is None:
            raise RuntimeError("patch size unknown: call update_args_per_forward before the forward pass")
        T = self.patch_height * self.patch_width + self.num_special_tokens
        return Geometry.from_tokens(num_tokens, T, self.num_special_tokens)

    def pack(self, qkv: torch.Tensor, pos, geom: Geometry, pool: bool = True):
        """``saf3r_pack_qkv`` of this layer: QK-LayerNorm + RoPE-2D + the per-head layouts, Q with the
        softmax scale where flagged, the fp32 rows of the probe / dino heads, and (``pool``) the block
        means of the block_topk heads. Returns ``ops.pack_qkv``'s tuple."""
        om = self.orig_module
        H = self.num_heads
        C = H * HEAD_DIM
        ln_q = ln_k = None
        eps = 1e-5
        if isinstance(om.q_norm, nn.LayerNorm):
            ln_q = (om.q_norm.weight, om.q_norm.bias)
            ln_k = (om.k_norm.weight, om.k_norm.bias)
            eps = om.q_norm.eps
        elif not isinstance(om.q_norm, nn.Identity):
            raise NotImplementedError(f"q_norm {type(om.q_norm).__name__} is not LayerNorm / Identity")
        base = p2 = npos = None
        if om.rope is not None and pos is not None:
            base = float(om.rope.base_frequency)
            p2 = pos.reshape(-1, 2)
            # table length: the patch grid bounds every position ((y+1, x+1) with specials at 0)
            npos = max(self.patch_height, self.patch_width) + 1 if self.patch_height else None
        # dense heads: unpadded token-order tiles; frame-relative heads: whole frames per tile run
        tord = ops.token_order_heads(self.patterns, geom)
        f32 = [h in self.fp32_slot for h in range(H)] if self.fp32_heads else None
        # block_topk heads: the pack also writes their pooled block records (means of bf16 q / k)
        return ops.pack_qkv(qkv, qkv[:, C:], qkv[:, 2 * C:], 3 * C, HEAD_DIM, geom, H, ln_q=ln_q, ln_k=ln_k,
                            ln_eps=eps, pos=p2, rope_base=base, rope_positions=npos, token_order=tord, fp32_heads=f32,
                            q_scaled=self.q_scaled_heads(), q_scale=ops.prescale_factor(getattr(om, "scale", None)),
                            pool_heads=(self.dyn_heads or None) if pool else None)

    def compute_multihead_attention_packed(self, qkv: torch.Tensor, pos, geom: Geometry) -> torch.Tensor:
        """qkv: bf16 [N, 3*H*64] (the qkv Linear output). Returns bf16 [N, H*64]."""
        om = self.orig_module
        H = self.num_heads
        C = H * HEAD_DIM
        tord = ops.token_order_heads(self.patterns, geom)
        qs = self.q_scaled_heads()
        packed = self.pack(qkv, pos, geom)
        qp, kp, vp = packed[:3]
        qk32 = packed[3] if self.fp32_heads else None
        sel = None
        if self.dyn_heads:
            pooled = packed[-1]
            if self.topk_scope == "frame":
                sel = ops.block_select_pooled(pooled, geom.frames, geom.blocks_per_frame, self.layer_block_topk)
            else:
                sel = ops.block_select(pooled.mean[:, 0], pooled.mean[:, 1], geom.frames, geom.blocks_per_frame,
                                       self.layer_block_topk, self.topk_scope)
        self.last_selection = sel  # block lists of the block_topk heads, in head order
        if self.dino_heads:
            self._lazy_token_topk(qp, kp, geom)
        keysets = None
        if self.keyset_heads:
            keysets = self._keysets(qk32, kp, qkv, geom, C)
        self.last_keysets = keysets
        bcast = None
        if self.broadcast_heads:  # broadcast_first: frame 0's Q/K rows and every frame's V tiles
            bcast = ops.broadcast_gather(qp, kp, geom, self.broadcast_heads, qkv[:, 2 * C:], qkv.stride(0), HEAD_DIM)
        out = ops.sparse_attn_fwd(qp, kp, vp, geom, self.patterns, sel, scale=getattr(om, "scale", None),
                                  keysets=keysets, broadcast=bcast, token_order=tord, q_scaled=qs)
        if self.dino_heads:  # image rows: gather attention over est_topk_idx with the fp32 q / k
            est = self.est_topk_idx
            P, W, T, ns = geom.patches, est.shape[1], geom.tokens_per_frame, geom.num_special
            for h in self.dino_heads:
                s = self.fp32_slot[h]
                qr = ops.rows(qk32[s, 0], 64, ns, P, T)
                kr = ops.rows(qk32[s, 1], 64, ns, P, T)
                vr = ops.rows(qkv, 3 * C, ns, P, T, offset=2 * C + h * HEAD_DIM)
                orr = ops.rows(out, C, ns, P, T, offset=h * HEAD_DIM)
                ops.gather_attn_rows(qr, kr, vr, est, W, geom.frames * P, W, geom.frames * P, None, orr, qk_fp32=True)
        self.last_attention = out if self.keep_attention else None
        return out

    def _keysets(self, qk32, kp, qkv, geom: Geometry, C: int):
        """Shared key sets of the stride / q_probe_topk heads (``sparse_attention.py:143-186, 256-273``):
        probe scores of the top-k heads from their fp32 q / k, members in token order, then the compact
        K / V they attend."""
        specs = [keyset_spec(self.head_cfg[h], h, geom.tokens) for h in self.keyset_heads]
        probe_rows = [i for i, s in enumerate(specs) if s.mode == ops.KEYSET_TOPK]
        scores = None
        if probe_rows:
            ratios = sorted({specs[i].sample_ratio for i in probe_rows})
            if len(ratios) == 1 and len(probe_rows) == len(specs):
                _, scores = ops.probe_scores(qk32, [self.fp32_slot[specs[i].head] for i in probe_rows],
                                             sample=ops.probe_sample(geom.tokens, ratios[0]))
            else:  # one call per sample ratio; rows of stride heads stay unused zeros
                scores = torch.zeros(len(specs), geom.tokens, dtype=torch.float32, device=kp.device)
                for r in ratios:
                    rows_r = [i for i in probe_rows if specs[i].sample_ratio == r]
                    _, sc = ops.probe_scores(qk32, [self.fp32_slot[specs[i].head] for i in rows_r],
                                             sample=ops.probe_sample(geom.tokens, r))
                    scores[rows_r] = sc
        idx, count = ops.keyset_build(specs, geom, scores, kp.device)
        ks = ops.keyset_gather(kp, geom, specs, qkv[:, 2 * C:], qkv.stride(0), HEAD_DIM, idx, count)
        ks.scores = scores
        return ks

    def _lazy_token_topk(self, qp, kp, geom: Geometry):
        """Lazy per-frame token top-k from the first correspondence head (``wrapper.py:42-86``)."""
        if self.lazy_dino_topk and self.first_dino_head is not None and not self.first_dino_flag:
            self.first_dino_flag = True
            h = self.first_dino_head
            P = geom.patches
            r = ops.rows(qp[h], 64, geom.special_slots, P, geom.padded_patches)
            kr = ops.rows(kp[h], 64, geom.special_slots, P, geom.padded_patches)
            idx = ops.token_topk(qp, kp, geom.frames, P, self.dino_topk, qrows=r, krows=kr, n_q=geom.frames * P)
            self.est_topk_idx = idx
            self.shared.est_topk_idx = idx
            self.shared.source_layer = self.layer_idx
        elif self.shared.est_topk_idx is not None:
            self.est_topk_idx = self.shared.est_topk_idx
        if self.est_topk_idx is None or self.est_topk_idx.numel() == 0:
            raise RuntimeError("dino_topk head has no top-k indices: no earlier correspondence head computed them "
                               "and none were provided")
        n_img = geom.frames * geom.patches
        if self.est_topk_idx.shape[0] != n_img or not self.est_topk_idx.is_cuda:
            raise RuntimeError(f"est_topk_idx must be a GPU tensor with {n_img} rows")
        self.est_topk_idx = self.est_topk_idx.to(torch.int32).contiguous()

    def forward(self, *args, **kwargs):
        raise NotImplementedError("This is a base wrapper and should not be used directly.")
