"""torch-facing wrappers of the C-ABI kernels. Buffers are allocated here with torch (the library
never allocates); every call is asynchronous on the current HIP stream.

Tensor conventions: bf16 CUDA tensors, head_dim 64, contiguous unless stated otherwise.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Sequence

import torch

from . import _lib
from .layout import BLOCK, HEAD_DIM, Geometry

# Pattern ids (``enum saf3r_pattern``).
(DENSE, FRAME_LOCAL, ANCHOR_LOCAL, BLOCK_DYNAMIC, TOKEN_DYNAMIC, ANCHOR, SKIP, KEYSET, BROADCAST,
 TOKEN_DYNAMIC_KEYSET) = range(10)
PATTERN_NAMES = {
    DENSE: "dense", FRAME_LOCAL: "frame_local", ANCHOR_LOCAL: "anchor_local",
    BLOCK_DYNAMIC: "block_topk", TOKEN_DYNAMIC: "dino_topk", ANCHOR: "all_to_first", SKIP: "skip",
    KEYSET: "keyset", BROADCAST: "broadcast_first", TOKEN_DYNAMIC_KEYSET: "dino_topk_strided",
}
FIXED_ORDER = 1  # saf3r_attn_flags
LAYOUT_PACKED, LAYOUT_TOKEN, LAYOUT_FRAMED = 0, 1, 2  # saf3r_layout: per-head layouts (token_order arrays)
LOG2E = 1.4426950408889634
KEYSET_PATTERNS = (KEYSET, TOKEN_DYNAMIC_KEYSET)  # heads served from the key-set buffers
TOKEN_PATTERNS = (TOKEN_DYNAMIC, TOKEN_DYNAMIC_KEYSET)  # heads whose patch rows gather-attend est_topk_idx


_recorder = None

# Key-walk order of saf3r_sparse_attn_fwd: "paced" (walks start where the measured step time and the
# wall clock point, for cache reuse; the last output bits vary run to run) or "fixed" (every walk from
# its first tile: run-to-run identical output).
_walk_order = "paced"
_pace_state = {}  # device index -> [int64 tensor of 12 (the library's pacing state), call counter]


def set_walk_order(order: str) -> None:
    """Default key-walk order of ``sparse_attn_fwd``: "paced" or "fixed"."""
    global _walk_order
    if order not in ("paced", "fixed"):
        raise ValueError(f"walk order {order!r}: 'paced' or 'fixed'")
    _walk_order = order


def walk_order() -> str:
    return _walk_order


def _pace(device):
    """(pointer, sequence number) of the per-device pacing state; the counter advances per call."""
    idx = torch.device(device).index or 0
    st = _pace_state.get(idx)
    if st is None:
        st = [torch.zeros(12, dtype=torch.int64, device=device), 0]
        _pace_state[idx] = st
    seq = st[1]
    st[1] = (seq + 1) & 0xFFFFFFFF
    return st[0], seq


def set_event_recorder(recorder) -> None:
    """Install (or clear with None) a callable ``recorder(name, phase)`` invoked right before
    (phase "start") and after (phase "end") each launch of the attention and selection kernels,
    on the launching thread; used by the benchmark to bracket kernels with stream events."""
    global _recorder
    _recorder = recorder


def _mark(name, phase):
    if _recorder is not None:
        _recorder(name, phase)


def _ptr(t: torch.Tensor | None):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _need_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("saf3r kernels take GPU tensors")


def _i32_array(vals: Sequence[int]):
    arr = (ctypes.c_int32 * len(vals))(*[int(v) for v in vals])
    return arr


def _u8_flags(flags: Sequence[bool] | None, n: int):
    """Host uint8 [n] flag array for the C ABI (None: no array)."""
    if flags is None:
        return None
    flags = list(flags)
    if len(flags) != n:
        raise ValueError(f"one flag per head: got {len(flags)} for {n} heads")
    return (ctypes.c_uint8 * n)(*[1 if f else 0 for f in flags])


def _u8_layouts(layouts: Sequence[int] | None, n: int):
    """Host uint8 [n] array of per-head layouts (``LAYOUT_*``; True counts as ``LAYOUT_TOKEN``)."""
    if layouts is None:
        return None
    layouts = [int(x) for x in layouts]
    if len(layouts) != n:
        raise ValueError(f"one layout per head: got {len(layouts)} for {n} heads")
    if any(x not in (LAYOUT_PACKED, LAYOUT_TOKEN, LAYOUT_FRAMED) for x in layouts):
        raise ValueError(f"unknown layout in {layouts}")
    return (ctypes.c_uint8 * n)(*layouts)


FRAMED_PATTERNS = (FRAME_LOCAL, ANCHOR_LOCAL, ANCHOR)  # heads that can take the framed layout


def token_order_heads(patterns: Sequence[int], geom: Geometry | None = None) -> list[int]:
    """Per-head layout for ``pack_qkv`` / ``sparse_attn_fwd`` (``token_order``): DENSE heads take token
    order (no special or per-frame padding, so none of their query or key tiles is partly empty);
    with ``geom`` given and ``geom.framed_fits``, the frame-relative heads take the framed layout
    (each frame's tokens, special ones included, in whole tiles of their own, so every query tile
    walks whole frames with prefix masks only); every other head the packed layout."""
    framed = geom is not None and geom.framed_fits
    return [LAYOUT_TOKEN if int(p) == DENSE else LAYOUT_FRAMED if (framed and int(p) in FRAMED_PATTERNS)
            else LAYOUT_PACKED for p in patterns]


def rope_inv_freq(base: float = 100.0, feature_dim: int = 32) -> torch.Tensor:
    """Inverse frequencies of the 2-D RoPE (``rope.py:103-104``) for fp32 tokens (CPU tensor)."""
    exponents = torch.arange(0, feature_dim, 2).float() / feature_dim
    return 1.0 / (base ** exponents)


_rope_cache = {}


def rope_tables(positions: int, base: float = 100.0, device="cuda"):
    """cos / sin tables [positions, 16] fp32 of the 2-D RoPE for fp32 tokens, computed as
    ``rope.py:100-115`` does (angles = position * inv_freq in fp32, then cos / sin), cached."""
    key = (int(positions), float(base), str(device))
    if key not in _rope_cache:
        inv = rope_inv_freq(base)
        ang = torch.arange(int(positions), dtype=torch.float32)[:, None] * inv[None, :]
        _rope_cache[key] = (ang.cos().contiguous().to(device), ang.sin().contiguous().to(device))
    return _rope_cache[key]


def packed_buffers(geom: Geometry, num_heads: int, device) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    L = geom.slots
    q = torch.empty(num_heads, L, HEAD_DIM, dtype=torch.bfloat16, device=device)
    k = torch.empty_like(q)
    v = torch.empty(num_heads, L // BLOCK, BLOCK, HEAD_DIM, dtype=torch.bfloat16, device=device)
    return q, k, v


def prescale_factor(scale: float | None = None) -> float:
    """The factor ``pack_qkv(q_scaled=...)`` applies to Q for ``sparse_attn_fwd(q_scaled=...)``:
    softmax scale (default 1/sqrt(64)) times log2(e)."""
    return (1.0 / math.sqrt(HEAD_DIM) if scale is None else scale) * LOG2E


@dataclass
class Pooled:
    """Pooled block records of n heads (``saf3r_block_select_pooled``'s input): record
    (s*2 + t)*NB + b for head s, tensor t (0 = q, 1 = k), block b. ``mean`` fp32 [n, 2, NB, 64],
    ``split`` int16 [n, 2, NB, 2, 64] (fp16 bits), ``meta`` fp32 [n, 2, NB, 2]."""
    mean: torch.Tensor
    split: torch.Tensor
    meta: torch.Tensor

    @staticmethod
    def empty(n: int, nb: int, device) -> "Pooled":
        return Pooled(torch.empty(n, 2, nb, HEAD_DIM, dtype=torch.float32, device=device),
                      torch.empty(n, 2, nb, 2, HEAD_DIM, dtype=torch.int16, device=device),
                      torch.empty(n, 2, nb, 2, dtype=torch.float32, device=device))


def pack_qkv(q, k, v, tok_stride: int, head_stride: int, geom: Geometry, num_heads: int,
             ln_q=None, ln_k=None, ln_eps: float = 1e-5, pos=None, rope_base=None, rope_positions=None, out=None,
             token_order: Sequence[int] | None = None, fp32_heads: Sequence[bool] | None = None,
             q_scaled: Sequence[bool] | None = None, q_scale: float | None = None,
             pool_heads: Sequence[int] | None = None):
    """QK-LayerNorm + RoPE-2D + packing (``saf3r_pack_qkv``). ``q``/``k``/``v`` are tensors (or
    views) whose element (t, h, d) is at ``data_ptr + t*tok_stride + h*head_stride + d``.
    RoPE is applied when ``rope_base`` is given; ``rope_positions`` is the table length
    (default: max position + 1, which costs one device-to-host read). ``token_order`` gives each
    head's layout (``LAYOUT_*``, see ``token_order_heads``; True = token order). With ``fp32_heads``
    the call returns a fourth tensor, fp32 [n_flagged, 2, N, 64]: the fp32 q (index 0) and k (1) of
    the flagged heads after LayerNorm / RoPE, in token order and increasing head order. Heads flagged
    in ``q_scaled`` get their packed Q multiplied by ``q_scale`` (default ``prescale_factor()``) in
    fp32 before the one bf16 rounding; pass the same flags to ``sparse_attn_fwd``. With
    ``pool_heads`` (head ids, packed layout) the pack also writes those heads' pooled block records
    (block means of bf16(q) without the scale and of bf16(k), and their split records) and the call
    returns them last, as a :class:`Pooled`."""
    _need_cuda(q, k, v)
    lib = _lib.load()
    qp, kp, vp = out if out is not None else packed_buffers(geom, num_heads, q.device)
    pooled, pool_flags = None, None
    if pool_heads:
        pool_heads = sorted(pool_heads)
        pooled = Pooled.empty(len(pool_heads), geom.num_blocks, q.device)
        pool_flags = [h in pool_heads for h in range(num_heads)]
    qk32 = None
    if fp32_heads is not None and any(fp32_heads):
        qk32 = torch.empty(sum(1 for f in fp32_heads if f), 2, geom.tokens, HEAD_DIM, dtype=torch.float32,
                           device=q.device)
    apply_ln = ln_q is not None
    if apply_ln:  # fp32 device copies (the kernel reads them as device arrays of 64 floats)
        qw, qb = (t.detach().to(device=q.device, dtype=torch.float32).contiguous() for t in ln_q)
        kw, kb = (t.detach().to(device=q.device, dtype=torch.float32).contiguous() for t in ln_k)
        if any(t.numel() != HEAD_DIM for t in (qw, qb, kw, kb)):
            raise ValueError("LayerNorm weight and bias must hold 64 values each")
    else:
        qw = qb = kw = kb = None
    rc = rs = None
    npos = 0
    if rope_base is not None:
        if pos is None:
            raise ValueError("RoPE needs positions")
        pos = pos.to(device=q.device, dtype=torch.int32).contiguous()
        npos = int(rope_positions) if rope_positions is not None else int(pos.max().item()) + 1
        rc, rs = rope_tables(npos, rope_base, q.device)
    _mark("pack_qkv", "start")
    _lib.check(lib.saf3r_pack_qkv(
        _ptr(q), _ptr(k), _ptr(v), tok_stride, head_stride, geom.frames, geom.tokens_per_frame, geom.num_special,
        num_heads, _ptr(qw), _ptr(qb), _ptr(kw), _ptr(kb), float(ln_eps), int(apply_ln),
        _ptr(pos) if rc is not None else None, _ptr(rc), _ptr(rs), npos, _ptr(qp), _ptr(kp), _ptr(vp),
        _u8_layouts(token_order, num_heads), _u8_flags(fp32_heads, num_heads) if qk32 is not None else None,
        _ptr(qk32), _u8_flags(q_scaled, num_heads), float(prescale_factor() if q_scale is None else q_scale),
        _u8_flags(pool_flags, num_heads), _ptr(pooled.mean if pooled else None),
        _ptr(pooled.split if pooled else None), _ptr(pooled.meta if pooled else None), _lib.stream_ptr()))
    _mark("pack_qkv", "end")
    res = (qp, kp, vp) + ((qk32,) if fp32_heads is not None else ()) + ((pooled,) if pooled is not None else ())
    return res


def pack_heads(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, geom: Geometry, **kw):
    """Pack per-head tensors [H, N, 64] (no LayerNorm / RoPE unless requested)."""
    H, N, D = q.shape
    assert D == HEAD_DIM and N == geom.tokens and k.shape == q.shape == v.shape
    q, k, v = (t.to(torch.bfloat16).contiguous() for t in (q, k, v))
    return pack_qkv(q, k, v, HEAD_DIM, N * HEAD_DIM, geom, H, **kw)


def _check_packed(qp, kp, vp, geom: Geometry):
    H = qp.shape[0]
    exp_rows = (H, geom.slots, HEAD_DIM)
    for t in (qp, kp):
        if t is not None and (tuple(t.shape) != exp_rows or t.dtype != torch.bfloat16 or not t.is_contiguous()):
            raise ValueError(f"packed Q/K must be contiguous bf16 {exp_rows}, got {tuple(t.shape)}")
    if vp is not None and (tuple(vp.shape) != (H, geom.tiles, BLOCK, HEAD_DIM) or not vp.is_contiguous()):
        raise ValueError(f"packed V must be contiguous bf16 {(H, geom.tiles, BLOCK, HEAD_DIM)}")


def block_pool(qp: torch.Tensor, kp: torch.Tensor | None, geom: Geometry, heads: Sequence[int]):
    """fp32 block means [n_heads, F*NBf, 64] of packed Q (and K)."""
    _need_cuda(qp, kp)
    lib = _lib.load()
    _check_packed(qp, kp, None, geom)
    H = qp.shape[0]
    n = len(heads)
    pq = torch.empty(n, geom.num_blocks, HEAD_DIM, dtype=torch.float32, device=qp.device)
    pk = torch.empty_like(pq) if kp is not None else None
    hs = _i32_array(heads)
    _mark("block_pool", "start")
    _lib.check(lib.saf3r_block_pool(_ptr(qp), _ptr(kp), geom.frames, geom.tokens_per_frame, geom.num_special, H,
                                    hs, n, _ptr(pq), _ptr(pk), _lib.stream_ptr()))
    _mark("block_pool", "end")
    return pq, pk


def pooled_prepare(mean: torch.Tensor) -> Pooled:
    """Split records of fp32 pooled means [n, 2, NB, 64] (``saf3r_pooled_prepare``)."""
    _need_cuda(mean)
    lib = _lib.load()
    mean = mean.float().contiguous()
    n, two, nb, d = mean.shape
    if two != 2 or d != HEAD_DIM:
        raise ValueError("pooled means must be [n, 2, NB, 64]")
    res = Pooled(mean, torch.empty(n, 2, nb, 2, HEAD_DIM, dtype=torch.int16, device=mean.device),
                 torch.empty(n, 2, nb, 2, dtype=torch.float32, device=mean.device))
    _lib.check(lib.saf3r_pooled_prepare(_ptr(mean), n * 2 * nb, _ptr(res.split), _ptr(res.meta), _lib.stream_ptr()))
    return res


def block_select_pooled(pooled: Pooled, frames: int, blocks_per_frame: int, k: int) -> torch.Tensor:
    """Per-frame block top-k on the matrix cores (``saf3r_block_select_pooled``), bit-identical to
    ``block_select`` on ``pooled.mean``: int32 [n, NB, frames*min(k, NBf)] of global block ids (one
    launch; no workspace)."""
    _need_cuda(pooled.mean, pooled.split, pooled.meta)
    lib = _lib.load()
    n, _, nb, _ = pooled.mean.shape
    if nb != frames * blocks_per_frame:
        raise ValueError("pooled records do not match frames * blocks_per_frame")
    dev = pooled.mean.device
    idx = torch.empty(n, nb, frames * min(k, blocks_per_frame), dtype=torch.int32, device=dev)
    if lib.saf3r_block_select_pooled_workspace_bytes(n, frames, blocks_per_frame, k) < 0:
        raise ValueError(f"unsupported block selection: {n} heads, {frames} frames x {blocks_per_frame} blocks, k {k}")
    _mark("block_select", "start")
    _lib.check(lib.saf3r_block_select_pooled(_ptr(pooled.mean), _ptr(pooled.split), _ptr(pooled.meta), n, frames,
                                             blocks_per_frame, k, _ptr(idx), None, 0, _lib.stream_ptr()))
    _mark("block_select", "end")
    return idx


def topk_from_scores(scores: torch.Tensor, frames: int, k: int) -> torch.Tensor:
    """Per-frame top-k of fp32 scores [..., rows, frames*C] -> int32 [..., rows, frames*min(k, C)]."""
    _need_cuda(scores)
    lib = _lib.load()
    s = scores.float().contiguous()
    rows, ncol = s.shape[-2], s.shape[-1]
    n = s.numel() // (rows * ncol) if s.numel() else 0
    C = ncol // frames
    if C * frames != ncol:
        raise ValueError("columns are not frames * candidates")
    ke = min(k, C)
    idx = torch.empty(*s.shape[:-1], frames * ke, dtype=torch.int32, device=s.device)
    _lib.check(lib.saf3r_topk_from_scores(_ptr(s), max(n, 1), rows, frames, C, k, _ptr(idx), _lib.stream_ptr()))
    return idx


def block_select(pooled_q: torch.Tensor, pooled_k: torch.Tensor, frames: int, blocks_per_frame: int, k: int,
                 scope: str = "frame") -> torch.Tensor:
    """Block top-k from pooled Q/K: int32 [n, NBq, width] of global block ids."""
    _need_cuda(pooled_q, pooled_k)
    lib = _lib.load()
    n, nbq, _ = pooled_q.shape
    if scope == "frame":
        width = frames * min(k, blocks_per_frame)
    elif scope == "global":
        width = min(k, frames * blocks_per_frame)
    else:
        raise ValueError(f"unknown topk scope {scope!r}")
    idx = torch.empty(n, nbq, width, dtype=torch.int32, device=pooled_q.device)
    pq, pk = pooled_q.contiguous(), pooled_k.contiguous()
    _mark("block_select", "start")
    _lib.check(lib.saf3r_block_select(_ptr(pq), _ptr(pk), n, nbq, frames, blocks_per_frame, k,
                                      0 if scope == "frame" else 1, _ptr(idx), _lib.stream_ptr()))
    _mark("block_select", "end")
    return idx


def sparse_attn_fwd(qp, kp, vp, geom: Geometry, patterns: Sequence[int], sel: torch.Tensor | None = None,
                    scale: float | None = None, out: torch.Tensor | None = None,
                    keysets: "KeySets | None" = None, broadcast: "Broadcast | None" = None,
                    token_order: Sequence[int] | None = None, order: str | None = None,
                    q_scaled: Sequence[bool] | None = None) -> torch.Tensor:
    """All heads in one launch. Returns (or fills) ``out`` bf16 [N, H*64] in natural token order.
    ``keysets`` carries the compact K/V of the KEYSET heads and ``broadcast`` the frame-0 / per-frame
    buffers of the BROADCAST heads (each in increasing head order); ``token_order`` gives the layout
    ``pack_qkv`` packed each head in (``token_order_heads``); ``q_scaled`` the heads whose packed Q
    carries ``prescale_factor(scale)`` (``pack_qkv(q_scaled=...)``), which then skip the running
    maximum. ``order`` ("paced" / "fixed", default ``walk_order()``) chooses the key-walk order
    (see ``set_walk_order``)."""
    _need_cuda(qp, kp, vp)
    lib = _lib.load()
    H = qp.shape[0]
    if len(patterns) != H:
        raise ValueError("one pattern per head")
    _check_packed(qp, kp, vp, geom)
    if out is None:
        out = torch.empty(geom.tokens, H * HEAD_DIM, dtype=torch.bfloat16, device=qp.device)
    elif (out.dtype != torch.bfloat16 or out.dim() != 2 or out.shape[0] != geom.tokens
          or out.shape[1] < H * HEAD_DIM or out.stride(1) != 1):
        raise ValueError(f"out must be bf16 [N, >= H*64] with unit column stride, got {tuple(out.shape)}")
    scale = 1.0 / math.sqrt(HEAD_DIM) if scale is None else scale
    width = 0
    n_dyn = sum(1 for p in patterns if p == BLOCK_DYNAMIC)
    if n_dyn:
        if sel is None:
            raise ValueError("block-dynamic heads need a selection list")
        _need_cuda(sel)
        sel = sel.to(torch.int32).contiguous()
        if sel.dim() != 3 or sel.shape[0] != n_dyn or sel.shape[1] != geom.num_blocks:
            raise ValueError(f"sel must be [{n_dyn}, {geom.num_blocks}, W], got {tuple(sel.shape)}")
        width = sel.shape[-1]
    else:
        sel = None
    n_ks = sum(1 for p in patterns if p in KEYSET_PATTERNS)
    ks_k = ks_v = ks_n = None
    ks_cap = 0
    if n_ks:
        if keysets is None or keysets.k.shape[0] != n_ks:
            raise ValueError(f"{n_ks} key-set heads need {n_ks} gathered key sets")
        ks_k, ks_v, ks_n, ks_cap = keysets.k, keysets.v, keysets.count, keysets.capacity
    n_bc = sum(1 for p in patterns if p == BROADCAST)
    bq = bk = bv = None
    if n_bc:
        if broadcast is None or broadcast.q.shape[0] != n_bc:
            raise ValueError(f"{n_bc} BROADCAST heads need {n_bc} gathered frame-0 / per-frame buffers")
        bq, bk, bv = broadcast.q, broadcast.k, broadcast.v
    pat = _i32_array(patterns)
    order = _walk_order if order is None else order
    if order == "fixed":
        flags, pace, seq = FIXED_ORDER, None, 0
    elif order == "paced":
        flags = 0
        pace, seq = _pace(qp.device)
    else:
        raise ValueError(f"walk order {order!r}: 'paced' or 'fixed'")
    _mark("sparse_attn", "start")
    _lib.check(lib.saf3r_sparse_attn_fwd(
        _ptr(qp), _ptr(kp), _ptr(vp), geom.frames, geom.tokens_per_frame, geom.num_special, H,
        pat, _ptr(sel), width, float(scale), _ptr(out), out.stride(0), _ptr(ks_k), _ptr(ks_v), _ptr(ks_n),
        ks_cap, _ptr(bq), _ptr(bk), _ptr(bv), _u8_layouts(token_order, H), _u8_flags(q_scaled, H), flags,
        _ptr(pace), seq, _lib.stream_ptr()))
    _mark("sparse_attn", "end")
    return out


def rows(t: torch.Tensor, row_stride: int | None = None, base_row: int = 0, rows_per_frame: int | None = None,
         frame_row_stride: int = 0, offset: int = 0) -> _lib.Rows:
    """Row descriptor over a bf16 or fp32 tensor (``offset`` and strides in elements of its dtype)."""
    rs = t.stride(-2) if row_stride is None else row_stride
    rpf = (1 << 62) if rows_per_frame is None else rows_per_frame
    return _lib.Rows(t.data_ptr() + t.element_size() * offset, rs, base_row, rpf, frame_row_stride)


def gather_attn_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, idx: torch.Tensor,
                    scale: float | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """``fused_sparse_topk_attention`` (``saf3r/triton/sparse_topk_attention.py:115-166``):
    q [N, 64], k [Nk, 64], v [Nk, 64], idx int32 [N, TopK] (a stride-0 row view shares one list)
    -> out [N, 64] in ``v.dtype``. As the reference's kernel, q, k and v are used as fp32 (upcast
    exactly) and the fp32 result is rounded once to ``v.dtype``; bf16 rows are read as they are.
    head_dim and the value dim must be 64 (the reference autotunes any D; this build raises)."""
    _need_cuda(q, k, v, idx)
    if q.dim() != 2 or k.dim() != 2 or v.dim() != 2 or idx.dim() != 2:
        raise ValueError("q, k, v and kv_indices must be 2-D")
    n, d = q.shape
    if d != HEAD_DIM or k.shape[1] != HEAD_DIM or v.shape[1] != HEAD_DIM:
        raise ValueError(f"head_dim and value dim must be {HEAD_DIM} (got q {d}, k {k.shape[1]}, v {v.shape[1]})")
    if k.shape[0] != v.shape[0]:
        raise ValueError("k and v must hold the same number of rows")
    if idx.shape[0] != n:
        raise ValueError("kv_indices must have one row per query")
    floats = (torch.float32, torch.float16, torch.bfloat16)
    if q.dtype not in floats or k.dtype not in floats or v.dtype not in floats:
        raise TypeError("q, k and v must be float32, float16 or bfloat16")
    qk32 = not (q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16)
    qk_t = torch.float32 if qk32 else torch.bfloat16
    q, k = (t.to(qk_t).contiguous() for t in (q, k))
    out_dtype = v.dtype
    v32 = out_dtype != torch.bfloat16  # fp32 rows (fp16 upcast exactly), fp32 result rounded here
    res_t = torch.float32 if v32 else torch.bfloat16
    v = v.to(res_t).contiguous()
    if idx.stride(-1) != 1:
        idx = idx.contiguous()
    idx = idx.to(torch.int32)
    direct = out is not None and out.dtype == res_t and out.shape == (n, HEAD_DIM) and out.stride(-1) == 1
    res = out if direct else torch.empty(n, HEAD_DIM, dtype=res_t, device=q.device)
    flags = ((_lib.GATHER_QK_FP32 if qk32 else 0) | (_lib.GATHER_V_FP32 | _lib.GATHER_OUT_FP32 if v32 else 0))
    gather_attn_rows(rows(q), rows(k), rows(v), idx, idx.stride(0), n, idx.shape[1], k.shape[0], scale, rows(res),
                     dtype_flags=flags)
    if out is not None and not direct:
        out.copy_(res)
        return out
    return res if res.dtype == out_dtype else res.to(out_dtype)


_gather_ws = {}  # (device, bytes) -> the sliced gather's workspace, kept for the next call of the same size


def gather_sliced(n: int, topk: int) -> bool:
    """Whether a gather of ``n`` rows with ``topk``-entry lists takes the two-pass sliced kernels (many
    rows with long lists, where the rows the lists touch exceed one XCD's L2)."""
    return topk >= 128 and n * topk >= (1 << 22)


def gather_attn_rows(qr, kr, vr, idx, idx_row_stride, n, topk, num_keys, scale, outr, keep=None, qk_fp32=False,
                     dtype_flags=None, sliced=None):
    """``saf3r_gather_attn_fwd`` on row descriptors; ``qk_fp32``: q and k rows are fp32 (or give the
    full ``dtype_flags``). ``sliced`` (default: ``gather_sliced(n, topk)``) runs
    ``saf3r_gather_attn_fwd_sliced`` with a workspace kept per device and size."""
    lib = _lib.load()
    scale = 1.0 / math.sqrt(HEAD_DIM) if scale is None else scale
    flags = (_lib.GATHER_QK_FP32 if qk_fp32 else 0) if dtype_flags is None else dtype_flags
    if sliced is None:
        sliced = gather_sliced(n, topk)
    _mark("gather_attn", "start")
    if sliced and n > 0:
        nbytes = int(lib.saf3r_gather_attn_workspace_bytes(n, topk))
        if nbytes < 0:
            raise RuntimeError(lib.saf3r_last_error().decode(errors="replace"))
        dev = torch.cuda.current_device()
        ws = _gather_ws.get((dev, nbytes))
        if ws is None:
            _gather_ws.clear()  # one size at a time: the dino heads of a forward share one
            ws = _gather_ws[(dev, nbytes)] = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        _lib.check(lib.saf3r_gather_attn_fwd_sliced(ctypes.byref(qr), ctypes.byref(kr), ctypes.byref(vr), _ptr(idx),
                                                    idx_row_stride, n, topk, num_keys, float(scale), int(flags),
                                                    ctypes.byref(outr), _ptr(ws), nbytes, _lib.stream_ptr()))
    else:
        _lib.check(lib.saf3r_gather_attn_fwd(ctypes.byref(qr), ctypes.byref(kr), ctypes.byref(vr), _ptr(idx),
                                             idx_row_stride, n, topk, num_keys, float(scale), int(flags),
                                             ctypes.byref(outr), _lib.stream_ptr()))
    _mark("gather_attn", "end")
    return keep


def token_topk_workspace_bytes(n_q: int, frames: int, per_frame: int, topk: int) -> int:
    """Bytes of the score workspace ``saf3r_token_topk`` takes for these sizes (0 for top-k <= 16)."""
    nbytes = _lib.load().saf3r_token_topk_workspace_bytes(n_q, frames, per_frame, topk)
    if nbytes < 0:
        _lib.check(_lib.SAF3R_ERR_INVALID)  # raises with the library's message
    return int(nbytes)


def token_topk(q: torch.Tensor, k: torch.Tensor, frames: int, per_frame: int, topk: int,
               qrows: _lib.Rows | None = None, krows: _lib.Rows | None = None, n_q: int | None = None,
               workspace: torch.Tensor | None = None):
    """``compute_qk_topk_indices_fused`` (``saf3r/triton/fused_qk_topk.py:120-217``):
    q [Nq, 64], k [frames*per_frame, 64] -> int32 [Nq, frames*min(topk, per_frame)], or with a batch
    dimension q [B, Nq, 64], k [B, frames*per_frame, 64] -> [B, Nq, frames*min(topk, per_frame)]
    (one call per batch element, as the reference's grid dimension 1 runs them; ``:187``). q and k
    are rounded to bf16, as the reference's kernel multiplies bf16 tiles. Above top-16 the score
    workspace is a torch allocation of ``token_topk_workspace_bytes`` (or ``workspace``)."""
    _need_cuda(q, k) if qrows is None or krows is None else _need_cuda(q)
    if qrows is None and krows is None and q.dim() == 3:
        if k is None or k.dim() != 3 or k.shape[0] != q.shape[0]:
            raise ValueError("batched q needs k of the same batch size")
        ws = workspace
        if ws is None:
            nbytes = token_topk_workspace_bytes(q.shape[1], frames, per_frame, topk)
            ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device) if nbytes else None
        return torch.stack([token_topk(q[b], k[b], frames, per_frame, topk, workspace=ws)
                            for b in range(q.shape[0])])
    lib = _lib.load()
    if qrows is None:
        if q.dim() != 2 or q.shape[-1] != HEAD_DIM:
            raise ValueError(f"q must be [Nq, {HEAD_DIM}] or [B, Nq, {HEAD_DIM}]")
        q = q.to(torch.bfloat16).contiguous()
        qrows = rows(q)
        n_q = q.shape[0]
    if krows is None:
        if k.dim() != 2 or k.shape[-1] != HEAD_DIM:
            raise ValueError(f"k must be [Nk, {HEAD_DIM}] like q")
        k = k.to(torch.bfloat16).contiguous()
        if k.shape[0] != frames * per_frame:
            raise ValueError("k must hold frames * per_frame rows")
        krows = rows(k)
    ke = min(topk, per_frame)
    idx = torch.empty(n_q, frames * ke, dtype=torch.int32, device=q.device)
    if workspace is None:
        nbytes = token_topk_workspace_bytes(n_q, frames, per_frame, topk)
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=q.device) if nbytes else None
    _mark("token_topk", "start")
    _lib.check(lib.saf3r_token_topk(ctypes.byref(qrows), ctypes.byref(krows), n_q, frames, per_frame, topk,
                                    _ptr(idx), _ptr(workspace), 0 if workspace is None else workspace.numel(),
                                    _lib.stream_ptr()))
    _mark("token_topk", "end")
    return idx


# ----------------------------------------------------------------------------------------
# Shared key sets of the stride and q_probe_topk modes
# ----------------------------------------------------------------------------------------
KEYSET_STRIDE, KEYSET_TOPK = 0, 1


@dataclass
class KeySetSpec:
    """One KEYSET head: ``mode`` KEYSET_STRIDE (``param`` = stride, first key ``start``) or
    KEYSET_TOPK (``param`` = k best probe scores); ``include`` adds frame 0 and every special token.
    ref: saf3r/patch/sparse_attention.py:56-85."""
    head: int
    mode: int
    param: int
    start: int = 0
    include: bool = False
    sample_ratio: float = 1.0  # KEYSET_TOPK: q_sample_ratio of the mean query (1 = every token)

    def bound(self, geom: Geometry) -> int:
        """Upper bound of the member count (host side, sizes the compact buffers)."""
        n = geom.tokens
        if self.mode == KEYSET_STRIDE:
            m = 0 if self.start >= n else -(-(n - self.start) // self.param)
        else:
            m = min(self.param, n)
        if self.include:
            m += min(n, geom.tokens_per_frame) + geom.frames * geom.num_special
        return min(m, n)


@dataclass
class KeySets:
    """Compact K/V of the KEYSET heads of a layer: ``k`` [n][capacity][64], ``v`` [n][capacity/64][64][64]
    (transposed tiles), ``count`` int32 [n] members, ``idx`` int32 [n][N] members in token order."""
    k: torch.Tensor
    v: torch.Tensor
    count: torch.Tensor
    idx: torch.Tensor
    capacity: int
    scores: torch.Tensor | None = None
    qbar: torch.Tensor | None = None


def probe_scores(qk32: torch.Tensor, slots: Sequence[int], scale: float | None = None,
                 sample: torch.Tensor | None = None, noalloc: bool = False):
    """Mean query and probe scores (``saf3r/patch/sparse_attention.py:150-168``) of the heads stored at
    ``slots`` of ``qk32`` (fp32 [n, 2, N, 64], q and k rows in token order, as ``pack_qkv`` writes them
    for ``fp32_heads``): returns (qbar fp32 [n_sel][64], scores fp32 [n_sel][N]). ``sample`` (int tokens)
    restricts the mean to those query rows, in list order (the reference's ``q_sample_ratio < 1``).
    ``noalloc`` uses the allocation-free entry (its partial sums in the library's static workspace)."""
    _need_cuda(qk32)
    lib = _lib.load()
    if qk32.dtype != torch.float32 or qk32.dim() != 4 or qk32.shape[1] != 2 or qk32.shape[3] != HEAD_DIM \
            or not qk32.is_contiguous():
        raise ValueError("qk32 must be a contiguous fp32 [n, 2, N, 64] tensor")
    N = qk32.shape[2]
    n = len(slots)
    dev = qk32.device
    hs = torch.tensor(list(slots), dtype=torch.int32, device=dev)
    qbar = torch.empty(n, HEAD_DIM, dtype=torch.float32, device=dev)
    scores = torch.empty(n, N, dtype=torch.float32, device=dev)
    scale = 1.0 / math.sqrt(HEAD_DIM) if scale is None else scale
    if sample is not None:
        sample = sample.to(device=dev, dtype=torch.int32).contiguous()
        if sample.dim() != 1 or not 1 <= sample.numel() <= N:
            raise ValueError("sample must list between 1 and N tokens")
    stride = qk32.stride(0)
    args = (_ptr(qk32), ctypes.c_void_p(qk32.data_ptr() + 4 * qk32.stride(1)), stride, N, _ptr(hs), n, _ptr(sample),
            0 if sample is None else sample.numel(), float(scale))
    _mark("probe", "start")
    if noalloc:
        _lib.check(lib.saf3r_probe_scores_noalloc(*args, _ptr(qbar), _ptr(scores), scores.stride(0),
                                                  _lib.stream_ptr()))
    else:
        partial = torch.empty(n, 256, HEAD_DIM, dtype=torch.float32, device=dev)
        _lib.check(lib.saf3r_probe_scores(*args, _ptr(partial), _ptr(qbar), _ptr(scores), scores.stride(0),
                                          _lib.stream_ptr()))
    _mark("probe", "end")
    return qbar, scores


def probe_sample(num_tokens: int, ratio: float) -> torch.Tensor | None:
    """Query rows of the reference's ``q_sample_ratio`` (``sparse_attention.py:154-157``):
    ``torch.linspace(0, N-1, steps=max(1, int(N * ratio))).long()`` for ratio < 1, else None (all rows).
    The list is computed by the same torch call on the host, so it holds the reference's rows."""
    if ratio >= 1:
        return None
    n = max(1, int(num_tokens * ratio))
    return torch.linspace(0, num_tokens - 1, steps=n).long()


def keyset_build(specs: Sequence[KeySetSpec], geom: Geometry, scores: torch.Tensor | None, device):
    """Members of each key set in token order: (idx int32 [n][N], count int32 [n]). ``scores``
    holds one row per spec (rows of KEYSET_STRIDE specs are not read)."""
    lib = _lib.load()
    n = len(specs)
    if any(s.param <= 0 for s in specs):
        raise ValueError("key-set stride / k must be positive")
    arr = torch.tensor([[s.mode, s.param, s.start, int(bool(s.include))] for s in specs], dtype=torch.int32)
    arr = arr.t().contiguous().to(device)
    idx = torch.empty(n, geom.tokens, dtype=torch.int32, device=device)
    count = torch.empty(n, dtype=torch.int32, device=device)
    if scores is not None:
        _need_cuda(scores)
        if scores.dtype != torch.float32 or scores.shape[0] != n or scores.shape[1] < geom.tokens:
            raise ValueError("scores must be fp32 [n_specs, >= N]")
        scores = scores.contiguous()
    _mark("keyset_build", "start")
    _lib.check(lib.saf3r_keyset_build(_ptr(scores), 0 if scores is None else scores.stride(0), n, _ptr(arr[0]),
                                      _ptr(arr[1]), _ptr(arr[2]), _ptr(arr[3]), geom.frames, geom.tokens_per_frame,
                                      geom.num_special, _ptr(idx), idx.stride(0), _ptr(count), _lib.stream_ptr()))
    _mark("keyset_build", "end")
    return idx, count


def keyset_gather(kp: torch.Tensor, geom: Geometry, specs: Sequence[KeySetSpec], v: torch.Tensor,
                  v_tok_stride: int, v_head_stride: int, idx: torch.Tensor, count: torch.Tensor) -> KeySets:
    """Compact K (packed rows) and transposed V tiles of each key set. ``v`` points at head 0's V of
    token 0 in the natural layout; head h, token t at ``v_tok_stride * t + v_head_stride * h``."""
    _need_cuda(kp, v, idx, count)
    lib = _lib.load()
    n = len(specs)
    cap = max(64, -(-max(s.bound(geom) for s in specs) // 64) * 64)
    dev = kp.device
    kc = torch.empty(n, cap, HEAD_DIM, dtype=torch.bfloat16, device=dev)
    vc = torch.empty(n, cap // 64, 64, 64, dtype=torch.bfloat16, device=dev)
    hs = torch.tensor([s.head for s in specs], dtype=torch.int32, device=dev)
    _mark("keyset_gather", "start")
    _lib.check(lib.saf3r_keyset_gather(_ptr(kp), geom.frames, geom.tokens_per_frame, geom.num_special, _ptr(hs), n,
                                       _ptr(v), v_tok_stride, v_head_stride, _ptr(idx), idx.stride(0), _ptr(count),
                                       cap // 64, _ptr(kc), _ptr(vc), cap, _lib.stream_ptr()))
    _mark("keyset_gather", "end")
    return KeySets(kc, vc, count, idx, cap)


@dataclass
class Broadcast:
    """Buffers of the BROADCAST heads of a layer (``broadcast_first``,
    ``saf3r/patch/sparse_attention.py:110-131``), C = ceil(T/64)*64: ``q`` / ``k`` [n][C][64] packed
    rows of frame 0's tokens in token order (zeros past T), ``v`` [n][F][C/64][64][64] the key-set V
    tiles of every frame's tokens."""
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor


def broadcast_gather(qp: torch.Tensor, kp: torch.Tensor, geom: Geometry, heads: Sequence[int], v: torch.Tensor,
                     v_tok_stride: int, v_head_stride: int) -> Broadcast:
    """Frame 0's Q and K rows and every frame's V tiles of ``heads``, through saf3r_keyset_gather
    (one key set per (head, frame): tokens f*T .. f*T+T-1). ``v`` is head 0's V of token 0 in the
    natural layout (head h, token t at ``v_tok_stride * t + v_head_stride * h``)."""
    _need_cuda(qp, kp, v)
    lib = _lib.load()
    n, F, T = len(heads), geom.frames, geom.tokens_per_frame
    cap = -(-T // 64) * 64
    dev = kp.device
    idx = (torch.arange(F, device=dev, dtype=torch.int32)[:, None] * T
           + torch.arange(T, device=dev, dtype=torch.int32)[None, :]).repeat(n, 1).contiguous()
    count = torch.full((n * F,), T, dtype=torch.int32, device=dev)
    hs = torch.tensor([h for h in heads for _ in range(F)], dtype=torch.int32, device=dev)
    kc = torch.empty(n * F, cap, HEAD_DIM, dtype=torch.bfloat16, device=dev)
    vc = torch.empty(n, F, cap // 64, 64, 64, dtype=torch.bfloat16, device=dev)
    _mark("broadcast_gather", "start")
    _lib.check(lib.saf3r_keyset_gather(_ptr(kp), F, T, geom.num_special, _ptr(hs), n * F, _ptr(v), v_tok_stride,
                                       v_head_stride, _ptr(idx), idx.stride(0), _ptr(count), cap // 64, _ptr(kc),
                                       _ptr(vc), cap, _lib.stream_ptr()))
    # frame 0's query rows: the same gather over the packed Q (its V output is not used)
    hs0 = torch.tensor(list(heads), dtype=torch.int32, device=dev)
    idx0 = idx[::F].contiguous()
    qc = torch.empty(n, cap, HEAD_DIM, dtype=torch.bfloat16, device=dev)
    scratch_v = torch.empty(n, cap // 64, 64, 64, dtype=torch.bfloat16, device=dev)
    _lib.check(lib.saf3r_keyset_gather(_ptr(qp), F, T, geom.num_special, _ptr(hs0), n, _ptr(v), v_tok_stride,
                                       v_head_stride, _ptr(idx0), idx0.stride(0), _ptr(count), cap // 64, _ptr(qc),
                                       _ptr(scratch_v), cap, _lib.stream_ptr()))
    kc0 = kc.view(n, F, cap, HEAD_DIM)[:, 0].contiguous()
    _mark("broadcast_gather", "end")
    return Broadcast(qc, kc0, vc)


def frame_topk_scores(scores: torch.Tensor, frames: int, per_frame: int, topk: int, per_frame_mode: bool = True,
                      exclude_first: bool = False, first_stride: int = 1, cap: int = 0) -> torch.Tensor:
    """Token top-k of every row of a bf16 score block [rows, frames*per_frame] (``saf3r_frame_topk_scores``):
    int32 [rows, F_sel + kept], F_sel frame-0 samples first when ``exclude_first``, then the kept keys
    (per frame or per row, at most ``cap`` when ``cap`` > 0) in increasing key order. Ties go to the
    lower key (ref: saf3r/patch/utils.py:54-184)."""
    _need_cuda(scores)
    lib = _lib.load()
    if scores.dtype != torch.bfloat16 or scores.dim() != 2 or scores.stride(1) != 1 or scores.stride(0) % 8:
        raise ValueError("scores must be a bf16 [rows, keys] tensor with unit column stride and row stride % 8")
    rows = scores.shape[0]
    nk = frames * per_frame
    if scores.shape[1] < nk:
        raise ValueError(f"scores have {scores.shape[1]} columns, need {nk}")
    f0 = 1 if exclude_first else 0
    fsel = -(-per_frame // first_stride) if exclude_first else 0
    if per_frame_mode:
        rest = min(topk, per_frame) * (frames - f0)
    else:
        rest = min(topk, nk - f0 * per_frame)
    kept = min(rest, cap) if cap > 0 else rest
    idx = torch.empty(rows, fsel + kept, dtype=torch.int32, device=scores.device)
    cand_i = cand_k = None
    if per_frame_mode and kept < rest:
        cand_i = torch.empty(rows, rest, dtype=torch.int32, device=scores.device)
        cand_k = torch.empty(rows, rest, dtype=torch.int16, device=scores.device)
    _mark("frame_topk", "start")
    _lib.check(lib.saf3r_frame_topk_scores(_ptr(scores), scores.stride(0), rows, frames, per_frame, int(exclude_first),
                                           first_stride if exclude_first else 0, int(per_frame_mode), topk, cap,
                                           _ptr(idx), idx.stride(0), _ptr(cand_i), _ptr(cand_k), _lib.stream_ptr()))
    _mark("frame_topk", "end")
    return idx

