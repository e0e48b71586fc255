"""torch restatement of SAF3R head-wise sparse global attention (a GPU-free reference for the tests).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Token layout (``saf3r/patch/sparse_attention.py:93-107``, ``aggregator.py:225-240``): frame f
holds tokens [f*T, (f+1)*T); the first ``nspec`` of them are special (camera + registers),
the remaining P = T - nspec are patch tokens. Patch tokens of a frame are cut into
NBf = ceil(P/64) blocks of 64 (the last one partial); block b of frame f has the global
block id f*NBf + b.

Patterns (per head; mask M[i, j] = 1 iff query i may attend key j):
  DENSE          always                                 (``saf3r/patch/wrapper.py:99-100``)
  FRAME_LOCAL    frame(j) == frame(i)                   (``sparse_attention.py:234-253``)
  ANCHOR_LOCAL   frame(j) == 0 or frame(j) == frame(i)  (union of ``:134-140`` and ``:234-253``)
  BLOCK_DYNAMIC  special(i): always; patch(i): patch(j) and block(j) in Sel[block(i)]
                 (block analogue of ``dino_topk``, ``:189-231``)
  TOKEN_DYNAMIC  the reference ``dino_topk``: special rows attend every key (or every
                 ``stride``-th key), patch rows attend the image tokens listed in
                 ``est_topk_idx`` (``:189-231``, gather softmax
                 ``saf3r/triton/sparse_topk_attention.py:36-112``)
  ANCHOR         frame(j) == 0 (``all_to_first``, ``:134-140``)
  SKIP           output zero (``:40-41``)
  KEYSET         j in one key set shared by every query of the head (``stride``, ``:256-273``;
                 ``q_probe_topk``, ``:143-186``; the set itself comes from
                 ``oracle.selection.keyset``)
  TOKEN_DYNAMIC_KEYSET  ``dino_topk`` with ``dino_sp2sp_stride`` s != 1: special rows attend keys
                 0, s, 2s, ... (``:199-204``; the list comes from ``oracle.selection.keyset``), image
                 rows as TOKEN_DYNAMIC
  BROADCAST      ``broadcast_first`` (``:110-131``): frame 0's attention map applied to every frame,
                 row f*T + i = sum_j softmax_j(q_i . k_j / sqrt(d)) v_{f*T + j}, i, j < T (not a mask
                 over the row's own q; see :func:`broadcast_attention`)
Scores are q.k / sqrt(d); softmax in the working precision; rows are independent.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

(DENSE, FRAME_LOCAL, ANCHOR_LOCAL, BLOCK_DYNAMIC, TOKEN_DYNAMIC, ANCHOR, SKIP, KEYSET, BROADCAST,
 TOKEN_DYNAMIC_KEYSET) = range(10)


@dataclass(frozen=True)
class Geometry:
    frames: int
    tokens_per_frame: int
    num_special: int = 5
    block: int = 64

    @property
    def patches(self) -> int:
        return self.tokens_per_frame - self.num_special

    @property
    def blocks_per_frame(self) -> int:
        return -(-self.patches // self.block)

    @property
    def tokens(self) -> int:
        return self.frames * self.tokens_per_frame


def token_info(g: Geometry):
    """frame id, special flag and global patch-block id (-1 for specials) of every token."""
    t = torch.arange(g.tokens)
    frame = t // g.tokens_per_frame
    local = t % g.tokens_per_frame
    special = local < g.num_special
    p = (local - g.num_special).clamp(min=0)
    gblock = torch.where(special, torch.full_like(t, -1), frame * g.blocks_per_frame + p // g.block)
    return frame, special, gblock


def image_token_ids(g: Geometry) -> torch.Tensor:
    """Token id of every image (patch) token, in image-index order (``sparse_attention.py:104-106``)."""
    i = torch.arange(g.frames * g.patches)
    return (i // g.patches) * g.tokens_per_frame + g.num_special + i % g.patches


def allowed_mask(pattern: int, rows: torch.Tensor, g: Geometry, sel: torch.Tensor | None = None,
                 sp2sp_stride: int = 1) -> torch.Tensor:
    """Boolean mask [len(rows), N] of the keys each query row may attend.

    ``sel`` is the block selection [F*NBf, W] (global block ids, -1 = empty) for
    BLOCK_DYNAMIC. TOKEN_DYNAMIC patch rows carry multiplicities and are not expressible
    as a mask; use :func:`token_dynamic_attention`.
    """
    frame, special, gblock = token_info(g)
    fq, sq, bq = frame[rows], special[rows], gblock[rows]
    n = g.tokens
    if pattern == DENSE:
        return torch.ones(len(rows), n, dtype=torch.bool)
    if pattern == FRAME_LOCAL:
        return fq[:, None] == frame[None, :]
    if pattern == ANCHOR_LOCAL:
        return (fq[:, None] == frame[None, :]) | (frame[None, :] == 0)
    if pattern == ANCHOR:
        return (frame[None, :] == 0).expand(len(rows), n).clone()
    if pattern == KEYSET:
        assert sel is not None, "KEYSET needs the key set (token ids) as sel"
        member = torch.zeros(n, dtype=torch.bool)
        member[torch.as_tensor(sel).long()] = True
        return member[None, :].expand(len(rows), n).clone()
    if pattern == BLOCK_DYNAMIC:
        assert sel is not None
        m = torch.zeros(len(rows), n, dtype=torch.bool)
        m[sq] = True
        pr = (~sq).nonzero().flatten()
        if len(pr):
            chosen = sel[bq[pr]].long()  # [np, W]
            member = torch.zeros(len(pr), g.frames * g.blocks_per_frame + 1, dtype=torch.bool)
            member.scatter_(1, torch.where(chosen < 0, member.shape[1] - 1, chosen), True)
            member[:, -1] = False
            key_ok = member[:, gblock.clamp(min=0)] & (~special)[None, :]
            m[pr] = key_ok
        return m
    raise ValueError(f"pattern {pattern} has no mask form")


def masked_attention(q, k, v, mask, scale=None, dtype=torch.float64):
    """softmax(q k^T * scale masked) v for one head and a row subset; q [r, d], k/v [n, d]."""
    d = q.shape[-1]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    s = (q.to(dtype) @ k.to(dtype).T) * scale
    s = s.masked_fill(~mask, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return p @ v.to(dtype)


def pattern_attention(q, k, v, pattern, g: Geometry, sel=None, chunk=2048, dtype=torch.float64,
                      scale=None):
    """One head, every query row, by explicit masks (chunked over queries)."""
    n, d = q.shape
    if pattern == SKIP:
        return torch.zeros(n, v.shape[1], dtype=dtype)
    out = torch.empty(n, v.shape[1], dtype=dtype)
    for s0 in range(0, n, chunk):
        rows = torch.arange(s0, min(n, s0 + chunk))
        m = allowed_mask(pattern, rows, g, sel)
        out[rows] = masked_attention(q[rows], k, v, m, scale, dtype)
    return out


def gather_attention(q, k, v, idx, scale=None, dtype=torch.float32):
    """``fused_sparse_topk_attention`` restated (``saf3r/triton/sparse_topk_attention.py:36-112``):
    out[i] = sum_j softmax_j(q_i . k[idx[i, j]] * scale) v[idx[i, j]], entries < 0 skipped.
    Exact max-subtracted softmax, accumulation in ``dtype``; q [n, d], k/v [nk, d], idx [n, W].
    """
    d = q.shape[-1]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    idx = idx.long()
    valid = idx >= 0
    safe = idx.clamp(min=0)
    out = torch.empty(q.shape[0], v.shape[1], dtype=dtype)
    step = 4096
    for s0 in range(0, q.shape[0], step):
        sl = slice(s0, s0 + step)
        kk = k.to(dtype)[safe[sl]]  # [r, W, d]
        vv = v.to(dtype)[safe[sl]]
        s = torch.einsum("rd,rwd->rw", q[sl].to(dtype), kk) * scale
        s = s.masked_fill(~valid[sl], float("-inf"))
        p = torch.softmax(s, dim=-1)
        out[sl] = torch.einsum("rw,rwd->rd", p, vv)
    return out


def token_dynamic_attention(q, k, v, est_topk_idx, g: Geometry, sp2sp_stride=1, dtype=torch.float64,
                            spec_keys=None, gather_qk=None):
    """Reference ``dino_topk_attention`` (``saf3r/patch/sparse_attention.py:189-231``).

    Special rows attend keys 0, s, 2s, ... (s = ``sp2sp_stride``; or the token list ``spec_keys``);
    image rows attend the image tokens ``est_topk_idx[i]`` (indices into the image-token list) and
    never special keys. ``gather_qk`` = (q, k) gives the image rows' gather its own q / k (the fp32
    values the reference's gather kernel reads under autocast); by default it uses ``q`` / ``k``.
    """
    frame, special, _ = token_info(g)
    out = torch.empty(g.tokens, v.shape[1], dtype=dtype)
    spec = special.nonzero().flatten()
    keys = torch.arange(0, g.tokens, sp2sp_stride) if spec_keys is None else torch.as_tensor(spec_keys).long()
    m = torch.ones(len(spec), len(keys), dtype=torch.bool)
    out[spec] = masked_attention(q[spec], k[keys], v[keys], m, dtype=dtype)
    img = image_token_ids(g)
    gq, gk = (q, k) if gather_qk is None else gather_qk
    out[img] = gather_attention(gq[img], gk[img], v[img], est_topk_idx, dtype=dtype)
    return out


def broadcast_attention(q, k, v, g: Geometry, dtype=torch.float64):
    """Reference ``broadcast_anchorframe_attention`` (``saf3r/patch/sparse_attention.py:110-131``):
    A = softmax(q0 k0^T / sqrt(d)) over frame 0's T tokens, then out_f = A v_f for every frame f."""
    T, d = g.tokens_per_frame, q.shape[-1]
    q0, k0 = q[:T].to(dtype), k[:T].to(dtype)
    a = torch.softmax((q0 @ k0.T) / math.sqrt(d), dim=-1)  # [T, T]
    vf = v.to(dtype).reshape(g.frames, T, v.shape[-1])
    return (a[None] @ vf).reshape(g.tokens, v.shape[-1])


def sparse_attention_gathered(q, k, v, pattern, g: Geometry, sel=None, dtype=torch.float32,
                              chunk=4096):
    """Same result as :func:`pattern_attention`, computed on restricted key sets (cost follows
    the pattern's allowed pairs). Used for the larger CPU checks and the CPU baseline."""
    n, d = q.shape
    T = g.tokens_per_frame
    qd, kd, vd = q.to(dtype), k.to(dtype), v.to(dtype)
    scale = 1.0 / math.sqrt(d)
    out = torch.empty(n, v.shape[1], dtype=dtype)

    def attend(rows, keys):
        s = (qd[rows] @ kd[keys].T) * scale
        out[rows] = torch.softmax(s, dim=-1) @ vd[keys]

    if pattern == SKIP:
        return torch.zeros(n, v.shape[1], dtype=dtype)
    if pattern == BROADCAST:
        return broadcast_attention(q, k, v, g, dtype)
    if pattern == DENSE:
        for s0 in range(0, n, chunk):
            attend(slice(s0, min(n, s0 + chunk)), slice(0, n))
        return out
    if pattern in (FRAME_LOCAL, ANCHOR_LOCAL, ANCHOR):
        for f in range(g.frames):
            rows = slice(f * T, (f + 1) * T)
            if pattern == FRAME_LOCAL:
                keys = torch.arange(f * T, (f + 1) * T)
            elif pattern == ANCHOR:
                keys = torch.arange(0, T)
            else:
                keys = torch.arange(0, T) if f == 0 else torch.cat([torch.arange(0, T), torch.arange(f * T, (f + 1) * T)])
            attend(rows, keys)
        return out
    if pattern == BLOCK_DYNAMIC:
        frame, special, gblock = token_info(g)
        spec = special.nonzero().flatten()
        attend(spec, slice(0, n))
        nbf, P = g.blocks_per_frame, g.patches
        for f in range(g.frames):
            for b in range(nbf):
                p0 = b * g.block
                rows = torch.arange(f * T + g.num_special + p0, f * T + g.num_special + min(P, p0 + g.block))
                blocks = sel[f * nbf + b]
                blocks = blocks[blocks >= 0].long()
                keys = []
                for cb in blocks.tolist():
                    cf, cbb = divmod(cb, nbf)
                    c0 = cbb * g.block
                    keys.append(torch.arange(cf * T + g.num_special + c0, cf * T + g.num_special + min(P, c0 + g.block)))
                attend(rows, torch.cat(keys))
        return out
    if pattern == KEYSET:
        keys = torch.as_tensor(sel).long()
        for s0 in range(0, n, chunk):
            attend(slice(s0, min(n, s0 + chunk)), keys)
        return out
    raise ValueError(f"pattern {pattern} has no gathered form")


# ----------------------------------------------------------------------------------------
# Layer pieces: RoPE-2D, QK-LayerNorm, the patched global-attention forward.
# ----------------------------------------------------------------------------------------

def rope_tables(max_pos: int, feature_dim: int = 32, base: float = 100.0):
    """cos/sin tables of ``RotaryPositionEmbedding2D`` (``saf3r/models/official_vggt/layers/rope.py:86-117``)
    for fp32 tokens: angles = pos * inv_freq (fp32), duplicated, then cos/sin."""
    exponents = torch.arange(0, feature_dim, 2).float() / feature_dim
    inv_freq = 1.0 / (base ** exponents)
    positions = torch.arange(max_pos, dtype=inv_freq.dtype)
    angles = positions[:, None] * inv_freq[None, :]
    angles = torch.cat((angles, angles), dim=-1)
    return angles.cos(), angles.sin()


def rope2d(x: torch.Tensor, pos: torch.Tensor, base: float = 100.0) -> torch.Tensor:
    """2-D RoPE (``rope.py:119-188``): first half of the features rotated by the y position,
    second half by x; within each half, rotate(t) = cat(-t2, t1). x [..., N, D] fp32, pos [N, 2]."""
    D = x.shape[-1]
    fd = D // 2
    cos, sin = rope_tables(int(pos.max()) + 1, fd, base)

    def one(t, p):
        c, s = cos[p.long()], sin[p.long()]
        t1, t2 = t[..., : fd // 2], t[..., fd // 2:]
        return t * c + torch.cat((-t2, t1), dim=-1) * s

    return torch.cat((one(x[..., :fd], pos[:, 0]), one(x[..., fd:], pos[:, 1])), dim=-1)


def vggt_positions(frames: int, patch_h: int, patch_w: int, num_special: int = 5) -> torch.Tensor:
    """Positions of the global layer tokens (``aggregator.py:225-240``, ``rope.py:39-59``): patches
    (y+1, x+1) in row-major order, specials (0, 0). Returns int64 [F*(nspec+h*w), 2]."""
    yy, xx = torch.meshgrid(torch.arange(patch_h), torch.arange(patch_w), indexing="ij")
    patch = torch.stack([yy.flatten(), xx.flatten()], dim=-1) + 1
    frame = torch.cat([torch.zeros(num_special, 2, dtype=torch.long), patch], dim=0)
    return frame.repeat(frames, 1)


def qkv_prologue(qkv: torch.Tensor, num_heads: int, ln_q, ln_k, pos, eps=1e-5, rope_base=100.0):
    """From the qkv projection output [N, 3*C] to per-head q, k, v [H, N, 64] as the attention
    kernel sees them: LayerNorm(64) on q and k in fp32, RoPE-2D in fp32, then bf16 rounding
    (``patch_vggt.py:575-583`` under ``autocast(bf16)``: LayerNorm and RoPE run in fp32 and
    SDPA receives bf16)."""
    n = qkv.shape[0]
    x = qkv.float().reshape(n, 3, num_heads, -1).permute(1, 2, 0, 3)  # [3, H, N, d]
    q, k, v = x[0], x[1], x[2]
    d = q.shape[-1]
    q = torch.nn.functional.layer_norm(q, (d,), ln_q[0].float(), ln_q[1].float(), eps)
    k = torch.nn.functional.layer_norm(k, (d,), ln_k[0].float(), ln_k[1].float(), eps)
    if pos is not None:
        q = rope2d(q, pos, rope_base)
        k = rope2d(k, pos, rope_base)
    return q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)


def head_outputs(q, k, v, patterns, g: Geometry, sel_by_head=None, est_topk_idx=None,
                 dtype=torch.float32, gathered=True, gather_qk_by_head=None):
    """Per-head attention of a layer: q/k/v [H, N, d] -> [H, N, d]. ``gather_qk_by_head`` {h: (q, k)}
    gives the image-row gather of token-dynamic heads its own q / k."""
    outs = []
    for h, pat in enumerate(patterns):
        sel = None if sel_by_head is None else sel_by_head.get(h)
        gqk = None if gather_qk_by_head is None else gather_qk_by_head.get(h)
        if pat == TOKEN_DYNAMIC:
            o = token_dynamic_attention(q[h], k[h], v[h], est_topk_idx, g, dtype=dtype, gather_qk=gqk)
        elif pat == TOKEN_DYNAMIC_KEYSET:  # sel: the special rows' key list
            o = token_dynamic_attention(q[h], k[h], v[h], est_topk_idx, g, dtype=dtype, spec_keys=sel, gather_qk=gqk)
        elif pat == BROADCAST:
            o = broadcast_attention(q[h], k[h], v[h], g, dtype=dtype)
        elif gathered:
            o = sparse_attention_gathered(q[h], k[h], v[h], pat, g, sel, dtype=dtype)
        else:
            o = pattern_attention(q[h], k[h], v[h], pat, g, sel, dtype=dtype)
        outs.append(o)
    return torch.stack(outs)


# ----------------------------------------------------------------------------------------
# The patched layer at the reference's own rounding points (autocast bf16)
# ----------------------------------------------------------------------------------------

def _bf16(x):
    return x.to(torch.bfloat16).to(torch.float64)


def reference_layer(x, w_qkv, b_qkv, ln_q, ln_k, w_proj, b_proj, pos, head_cfg, g: Geometry, lazy_topk: int = 4,
                    eps: float = 1e-5, rope_base: float = 100.0, est_topk_idx=None):
    """One patched global layer computed the way the reference computes it under ``autocast(bf16)``
    (``saf3r/patch/patch_vggt.py:575-590``, ``saf3r/patch/wrapper.py:94-106``,
    ``saf3r/patch/sparse_attention.py:12-273``), in fp64 with the reference's rounding points:

    - qkv and proj Linear layers: bf16 inputs and weights, result rounded to bf16;
    - q/k LayerNorm and RoPE in fp32 (autocast runs layer_norm in fp32; RoPE keeps the token dtype);
    - SDPA modes (full, global_to_frame, all_to_first, stride, the q_probe_topk attention, the special
      rows of dino_topk) attend on bf16-rounded q/k/v (autocast casts SDPA inputs);
    - q_probe_topk: mean query and probe scores from the fp32 q/k (``:160-166``), rounded to fp32;
      top-k ties to the lower token;
    - dino_topk image rows: the gather kernel reads the fp32 q/k and the bf16 v
      (``saf3r/triton/sparse_topk_attention.py:74-80``);
    - lazy dino indices: per-frame top-``lazy_topk`` of bf16 q . bf16 k of the first correspondence head
      (``fused_qk_topk.py:175-176``), ties to the lower key;
    - broadcast_first: bf16 matmuls, fp32 softmax (``:110-131``);
    - the head outputs are rounded to bf16 before the projection.

    x [N, C] (bf16 values), head_cfg: one dict per head. Returns (y [N, C] fp64, info) where info
    holds the key sets ({head: token list}) and the lazy indices used."""
    with torch.no_grad():
        return _reference_layer(x, w_qkv, b_qkv, ln_q, ln_k, w_proj, b_proj, pos, head_cfg, g, lazy_topk, eps,
                                rope_base, est_topk_idx)


def _reference_layer(x, w_qkv, b_qkv, ln_q, ln_k, w_proj, b_proj, pos, head_cfg, g, lazy_topk, eps, rope_base,
                     est_topk_idx):
    N, C = x.shape
    H = len(head_cfg)
    d = C // H
    xd = _bf16(x.float())
    qkv = _bf16(xd @ _bf16(w_qkv.float()).T + _bf16(b_qkv.float()))
    qkv = qkv.reshape(N, 3, H, d).permute(1, 2, 0, 3)  # [3, H, N, d]
    q32 = torch.nn.functional.layer_norm(qkv[0], (d,), ln_q[0].double(), ln_q[1].double(), eps).float()
    k32 = torch.nn.functional.layer_norm(qkv[1], (d,), ln_k[0].double(), ln_k[1].double(), eps).float()
    if pos is not None:
        q32 = rope2d(q32, pos, rope_base)
        k32 = rope2d(k32, pos, rope_base)
    v = qkv[2]  # bf16 values in fp64
    qb, kb = _bf16(q32), _bf16(k32)
    scale = 1.0 / math.sqrt(d)
    T, F = g.tokens_per_frame, g.frames
    info = {"keysets": {}, "est_topk_idx": est_topk_idx}
    img = image_token_ids(g)
    _, special, _ = token_info(g)
    spec = special.nonzero().flatten()

    def sdpa(rows, keys, h):
        s = (qb[h][rows] @ kb[h][keys].T) * scale
        return torch.softmax(s, dim=-1) @ v[h][keys]

    if est_topk_idx is None:
        first = next((h for h, c in enumerate(head_cfg) if c["mode"] == "dino_topk" and c.get("is_first_dino")), None)
        if first is not None:
            s = (qb[first][img] @ kb[first][img].T).float().numpy()
            from . import selection as OS
            info["est_topk_idx"] = torch.from_numpy(OS.frame_topk(s, F, lazy_topk))
    outs = []
    for h, cfg in enumerate(head_cfg):
        mode = cfg["mode"]
        o = torch.empty(N, d, dtype=torch.float64)
        if mode == "full":
            o = sdpa(slice(0, N), slice(0, N), h)
        elif mode == "skip":
            o = torch.zeros(N, d, dtype=torch.float64)
        elif mode == "global_to_frame":
            for f in range(F):
                r = slice(f * T, (f + 1) * T)
                o[r] = sdpa(r, r, h)
        elif mode == "all_to_first":
            o = sdpa(slice(0, N), slice(0, T), h)
        elif mode == "broadcast_first":
            a = torch.softmax(_bf16((qb[h][:T] @ kb[h][:T].T) * scale).float(), dim=-1).double()
            o = _bf16(_bf16(a) @ v[h].reshape(F, T, d)).reshape(N, d)
        elif mode in ("stride", "q_probe_topk"):
            include = cfg.get("include_as", mode == "stride")
            if mode == "stride":
                st = int(cfg.get("stride", 4))
                start = h % st if cfg.get("shift", False) else 0
                sel = torch.arange(start, N, st)
            else:
                k_top = max(1, N // int(cfg["stride"])) if "stride" in cfg else min(int(cfg.get("topk", 1024)), N)
                ratio = cfg.get("q_sample_ratio", 1)
                rows = torch.arange(N)
                if ratio < 1:
                    rows = torch.linspace(0, N - 1, steps=max(1, int(N * ratio))).long()
                qbar = q32[h][rows].double().mean(0).float().double()
                scores = ((qbar @ k32[h].double().T) / math.sqrt(d)).float().double()
                order = sorted(range(N), key=lambda t: (-float(scores[t]), t))
                sel = torch.tensor(order[:k_top], dtype=torch.long)
            if include:
                sel = torch.cat([sel, torch.arange(T), spec])
            keys = torch.unique(sel)
            info["keysets"][h] = keys
            o = sdpa(slice(0, N), keys, h)
        elif mode == "dino_topk":
            st = int(cfg.get("dino_sp2sp_stride", 1))
            o[spec] = sdpa(spec, torch.arange(0, N, st), h)
            idx = info["est_topk_idx"].long()
            valid = idx >= 0
            kk = k32[h][img].double()[idx.clamp(min=0)]  # [P, W, d] fp32 keys
            s = torch.einsum("rd,rwd->rw", q32[h][img].double(), kk) * scale
            s = s.masked_fill(~valid, float("-inf"))
            p = torch.softmax(s, dim=-1)
            o[img] = torch.einsum("rw,rwd->rd", p, v[h][img][idx.clamp(min=0)])
        else:
            raise ValueError(f"mode {mode!r} has no reference-semantics restatement")
        outs.append(_bf16(o))
    info["heads"] = torch.stack(outs)  # [H, N, d] head outputs (bf16 values) before the projection
    attn = info["heads"].permute(1, 0, 2).reshape(N, C)
    y = attn @ _bf16(w_proj.float()).T + _bf16(b_proj.float())
    return y, info
