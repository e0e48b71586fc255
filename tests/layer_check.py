"""Shared checks of a patched global-attention layer against the oracle (GPU tests only).

``check_layer_output`` recomputes the q/k/v the kernels consumed (the packing is deterministic),
rebuilds every head's key set / block list / token lists with the oracle, runs the oracle's per-head
attention in fp64 and the output projection, and compares the layer output the wrapper returned.
"""
import importlib

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


def packed_qkv(w, x, pos, geom, ops):
    """The q / k / v [H, N, 64] (bf16, natural token order) the wrapper's kernels consumed for input x
    (Q of the heads in ``w.q_scaled_heads()`` with ``ops.prescale_factor()`` folded in, as packed), and
    {head: (q, k)} fp32 [N, 64] rows of its fp32 heads (probe and dino heads)."""
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
    return q, k, v, rows32


def check_layer_output(w, x, pos, y, geom, ops, li, tol=(2e-2, 2e-3)):
    """``y`` (the wrapper's output for input x) against the oracle layer on the kernels' own q/k/v."""
    N, dim = geom.tokens, w.orig_module.qkv.in_features
    om = w.orig_module
    q, k, v, rows32 = packed_qkv(w, x, pos, geom, ops)
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
    for h in w.dyn_heads:
        sel[h] = torch.from_numpy(OS.block_select(OS.bf16_bits(q[h].float().numpy()),
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


def check_layer(w, x, pos, geom, ops, li):
    """Runs one wrapper on x and checks it against the oracle layer."""
    y = w(x, pos)
    torch.cuda.synchronize()
    return check_layer_output(w, x, pos, y[0], geom, ops, li)
