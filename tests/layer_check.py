"""Shared checks of a patched global-attention layer against the oracle (GPU tests only).

``check_layer_output`` recomputes the q/k/v the kernels consumed (the packing is deterministic),
rebuilds every head's key set / block list / token lists with the oracle, runs the oracle's per-head
attention in fp64 and the output projection, and compares the layer output the wrapper returned.
"""
import importlib

import numpy as np
import torch

from oracle import attention as OA
from oracle import selection as OS
from tests.layout_ref import slot_tokens, unpack_rows, unpack_v


def err(a, b):
    e = (a.float() - b.float()).abs()
    return e.max().item(), e.mean().item()


def make_stack(vggt, depth, dim, heads, seed=0):
    """GlobalAttentionStack with non-trivial LayerNorm affine parameters."""
    torch.manual_seed(seed)
    m = vggt.GlobalAttentionStack(depth=depth, dim=dim, num_heads=heads)
    for b in m.aggregator.global_blocks:
        for n in (b.attn.q_norm, b.attn.k_norm):
            torch.nn.init.uniform_(n.weight, 0.5, 1.5)
            torch.nn.init.normal_(n.bias, std=0.1)
    return m


def oracle_keysets(w, qk32, og, ops):
    """Key sets of the wrapper's stride / q_probe_topk heads from the oracle on the kernels' fp32 q / k
    (``qk32`` {head: (q, k)} fp32 [N, 64] rows)."""
    spa = importlib.import_module(type(w).__module__.rsplit(".", 1)[0] + ".sparse_attention")
    out = {}
    for h in w.keyset_heads:
        s = spa.keyset_spec(w.head_cfg[h], h, og.tokens)
        scores = None
        if s.mode == ops.KEYSET_TOPK:
            rows = ops.probe_sample(og.tokens, s.sample_ratio)
            q32, k32 = qk32[h]
            qh = q32 if rows is None else q32[rows]
            qb = OS.probe_mean(qh.numpy())
            scores = OS.probe_scores(qb, k32.numpy())
        out[h] = torch.from_numpy(OS.keyset(scores, og.tokens, og.tokens_per_frame, og.num_special, s.mode, s.param,
                                            s.start, s.include))
    return out


def packed_qkv(w, x, pos, geom, ops, plain=False):
    """The q / k / v [H, N, 64] (bf16, natural token order) the wrapper's kernels consumed for input x
    (Q of the heads in ``w.q_scaled_heads()`` with ``ops.prescale_factor()`` folded in, as packed), and
    {head: (q, k)} fp32 [N, 64] rows of its fp32 heads (probe and dino heads). ``plain``: also the
    bf16 q without the scale (the rows the block means of the block_topk heads are taken from)."""
    N, dim, H = geom.tokens, w.orig_module.qkv.in_features, w.num_heads
    om = w.orig_module
    qkv = om.qkv(x).reshape(N, 3 * dim).to(torch.bfloat16).contiguous()
    f32 = [h in w.fp32_slot for h in range(H)]
    qp, kp, vp, qk32 = ops.pack_qkv(qkv, qkv[:, dim:], qkv[:, 2 * dim:], 3 * dim, 64, geom, H,
                                    ln_q=(om.q_norm.weight, om.q_norm.bias), ln_k=(om.k_norm.weight, om.k_norm.bias),
                                    pos=pos[0], rope_base=100.0, fp32_heads=f32, q_scaled=w.q_scaled_heads())
    torch.cuda.synchronize()
    toks = slot_tokens(geom.frames, geom.tokens_per_frame, geom.num_special)
    q, _ = unpack_rows(qp.cpu(), toks, N)
    k, _ = unpack_rows(kp.cpu(), toks, N)
    v, _ = unpack_v(vp.cpu(), toks, N)
    rows32 = {h: (qk32[s, 0].cpu(), qk32[s, 1].cpu()) for h, s in w.fp32_slot.items()} if qk32 is not None else {}
    if not plain:
        return q, k, v, rows32
    qp0, _, _ = ops.pack_qkv(qkv, qkv[:, dim:], qkv[:, 2 * dim:], 3 * dim, 64, geom, H,
                             ln_q=(om.q_norm.weight, om.q_norm.bias), ln_k=(om.k_norm.weight, om.k_norm.bias),
                             pos=pos[0], rope_base=100.0)
    q0, _ = unpack_rows(qp0.cpu(), toks, N)
    return q, k, v, rows32, q0


def check_layer_output(w, x, pos, y, geom, ops, li, tol=(2e-2, 2e-3)):
    """``y`` (the wrapper's output for input x) against the oracle layer on the kernels' own q/k/v."""
    N, dim = geom.tokens, w.orig_module.qkv.in_features
    om = w.orig_module
    q, k, v, rows32, q_plain = packed_qkv(w, x, pos, geom, ops, plain=True)
    og = OA.Geometry(geom.frames, geom.tokens_per_frame, geom.num_special)
    c = ops.prescale_factor()
    qs = w.q_scaled_heads()
    for h, (q32, k32) in rows32.items():  # the fp32 rows round to the bf16 ones the attention read
        assert torch.equal((q32 * c if qs[h] else q32).to(torch.bfloat16), q[h])
        assert torch.equal(k32.to(torch.bfloat16), k[h])
    # the attention's q: a prescaled head's packed values divided by the factor, in fp32
    q_att = torch.stack([q[h].float() / c if qs[h] else q[h].float() for h in range(w.num_heads)])
    sel = oracle_keysets(w, rows32, og, ops)
    if w.keyset_heads:  # the kernels' key sets are the oracle's, member for member
        ks = w.last_keysets
        for i, h in enumerate(w.keyset_heads):
            c = int(ks.count[i])
            assert torch.equal(ks.idx[i, :c].cpu(), sel[h].to(torch.int32)), f"layer {li} head {h} key set"
    for h in w.dyn_heads:  # block means of the unscaled bf16 q and of k
        sel[h] = torch.from_numpy(OS.block_select(OS.bf16_bits(q_plain[h].float().numpy()),
                                                  OS.bf16_bits(k[h].float().numpy()), geom.frames,
                                                  geom.tokens_per_frame, geom.num_special, w.layer_block_topk))
    if w.dyn_heads:  # the kernels' block lists are the oracle's
        assert torch.equal(w.last_selection.cpu(), torch.stack([sel[h] for h in w.dyn_heads]).to(torch.int32))
    est = w.est_topk_idx.cpu() if w.dino_heads else None
    gqk = {h: rows32[h] for h in w.dino_heads}
    heads = OA.head_outputs(q_att, k.float(), v.float(), list(w.patterns), og, sel, est_topk_idx=est,
                            dtype=torch.float64, gather_qk_by_head=gqk)
    attn = heads.permute(1, 0, 2).reshape(N, dim).to(torch.bfloat16).float()
    if w.last_attention is not None:  # the attention output itself, at the attention tolerance
        amx, amean = err(w.last_attention.reshape(N, dim).cpu(), heads.permute(1, 0, 2).reshape(N, dim))
        print(f"layer {li} attention: max {amx:.3g} mean {amean:.3g}", flush=True)
        assert amx <= tol[0] and amean <= tol[1], (li, "attention", amx, amean)
    yref = attn @ om.proj.weight.float().cpu().T + om.proj.bias.float().cpu()
    mx, mean = err(y.reshape(N, dim).cpu(), yref)
    # y is the bf16 output of the projection: its own rounding (half an ulp, 2^-8 relative) adds to the bound
    ymax, ymean = yref.abs().max().item(), yref.abs().mean().item()
    print(f"layer {li}: max {mx:.3g} mean {mean:.3g} (|y| max {ymax:.3g}, mean {ymean:.3g})", flush=True)
    assert mx <= tol[0] + ymax * 2 ** -8 and mean <= tol[1] + ymean * 2 ** -8, (li, mx, mean)
    return mx, mean


def rows_of(packed, geom, tokens, head):
    """Rows of ``tokens`` of one head from packed [H, L, 64] Q or K (the padded layout)."""
    slot = torch.full((geom.tokens,), -1, dtype=torch.long)
    toks = slot_tokens(geom.frames, geom.tokens_per_frame, geom.num_special)
    valid = toks >= 0
    slot[toks[valid]] = torch.arange(len(toks))[valid]
    return packed[head][slot[tokens].to(packed.device)].float().cpu()


def sample_rows(geom, n_random, seed):
    """Query rows for a sampled check: frame 0's specials, the end of frame 0 and the start of frame 1
    (special and patch rows), the first 70 rows of the last frame, and ``n_random`` random rows."""
    T, N = geom.tokens_per_frame, geom.tokens
    rng = torch.Generator().manual_seed(seed)
    return torch.unique(torch.cat([torch.arange(5), torch.arange(T - 64, T + 5), torch.arange(N - T, N - T + 70),
                                   torch.randint(0, N, (n_random,), generator=rng)]))


def check_sampled_rows(w, x, pos, y, geom, ops, rows, what, tol=(2e-2, 2e-3)):
    """A block-pattern layer (dense / frame-local / anchor+local / block top-k heads) at full size,
    checked on sampled rows: q / k / v recomputed by the packing in the padded layout (deterministic),
    every block list bit-exact against the oracle's selection from the same packed q / k, the attention
    of ``rows`` against the oracle's masked fp64 attention, and y on those rows through the projection."""
    N, dim, H = geom.tokens, w.orig_module.qkv.in_features, w.num_heads
    om = w.orig_module
    qkv = om.qkv(x).reshape(N, 3 * dim).contiguous()
    qs = w.q_scaled_heads()  # Q as the wrapper packed it (softmax scale folded in)
    pk = dict(ln_q=(om.q_norm.weight, om.q_norm.bias), ln_k=(om.k_norm.weight, om.k_norm.bias), pos=pos[0],
              rope_base=100.0)  # every head padded, for reading back
    qp, kp, _ = ops.pack_qkv(qkv, qkv[:, dim:], qkv[:, 2 * dim:], 3 * dim, 64, geom, H, q_scaled=qs, **pk)
    qp0, _, _ = ops.pack_qkv(qkv, qkv[:, dim:], qkv[:, 2 * dim:], 3 * dim, 64, geom, H, **pk)  # unscaled q
    torch.cuda.synchronize()
    toks_all = torch.arange(N)
    T, F_ = geom.tokens_per_frame, geom.frames
    sel_of = {}
    bits = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)
    for i, h in enumerate(w.dyn_heads):  # block means of the unscaled bf16 q and of k
        qh = rows_of(qp0, geom, toks_all, h).to(torch.bfloat16)
        kh = rows_of(kp, geom, toks_all, h).to(torch.bfloat16)
        want = OS.block_select(bits(qh), bits(kh), F_, T, geom.num_special, w.layer_block_topk)
        assert np.array_equal(w.last_selection[i].cpu().numpy(), want), f"{what}: block list of head {h}"
        sel_of[h] = torch.from_numpy(want)
    print(f"{what}: {len(sel_of)} block lists bit-exact", flush=True)
    og = OA.Geometry(F_, T, geom.num_special)
    attn = torch.empty(len(rows), H, 64, dtype=torch.float64)
    vnat = qkv[:, 2 * dim:].reshape(N, H, 64)
    c = ops.prescale_factor()
    for h, pat in enumerate(w.patterns):
        qh = rows_of(qp, geom, rows, h) / (c if qs[h] else 1.0)
        kh = rows_of(kp, geom, toks_all, h)
        vh = vnat[:, h].float().cpu()
        mask = OA.allowed_mask(pat, rows, og, sel_of.get(h))
        attn[:, h] = OA.masked_attention(qh, kh, vh, mask, dtype=torch.float64)
    got_attn = w.last_attention[rows.to(x.device)].float().cpu().reshape(len(rows), H, 64)
    amx, amean = err(got_attn, attn)
    print(f"{what}: attention on {len(rows)} rows: max {amx:.3g} mean {amean:.3g}", flush=True)
    assert amx <= tol[0] and amean <= tol[1], (what, amx, amean)
    a = attn.reshape(len(rows), dim).to(torch.bfloat16).double()
    yref = a @ om.proj.weight.double().cpu().T + om.proj.bias.double().cpu()
    mx, mean = err(y[rows.to(x.device)].cpu(), yref)
    ymax, ymean = yref.abs().max().item(), yref.abs().mean().item()
    print(f"{what}: y on {len(rows)} rows: max {mx:.3g} mean {mean:.3g} (|y| max {ymax:.3g})", flush=True)
    assert mx <= tol[0] + ymax * 2 ** -8 and mean <= tol[1] + ymean * 2 ** -8, (what, mx, mean)
    return amx, amean


def check_layer(w, x, pos, geom, ops, li):
    """Runs one wrapper on x and checks it against the oracle layer."""
    y = w(x, pos)
    torch.cuda.synchronize()
    return check_layer_output(w, x, pos, y[0], geom, ops, li)
