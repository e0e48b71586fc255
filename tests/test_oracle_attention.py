"""Pins the attention oracle: library SDPA, closed forms, invariances and a per-query brute force."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import attention as A


def _qkv(n, d=64, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(n, d, generator=g, dtype=dtype) for _ in range(3)]


G = A.Geometry(frames=3, tokens_per_frame=5 + 150)  # 150 patches: blocks of 64, 64, 22


def test_dense_is_library_sdpa():
    q, k, v = _qkv(G.tokens)
    got = A.pattern_attention(q, k, v, A.DENSE, G)
    exp = F.scaled_dot_product_attention(q[None, None], k[None, None], v[None, None])[0, 0]
    torch.testing.assert_close(got, exp, rtol=1e-10, atol=1e-10)


def test_frame_local_is_per_frame_sdpa_and_ignores_other_frames():
    q, k, v = _qkv(G.tokens, seed=1)
    got = A.pattern_attention(q, k, v, A.FRAME_LOCAL, G)
    T = G.tokens_per_frame
    for f in range(G.frames):
        s = slice(f * T, (f + 1) * T)
        exp = F.scaled_dot_product_attention(q[s][None], k[s][None], v[s][None])[0]
        torch.testing.assert_close(got[s], exp, rtol=1e-10, atol=1e-10)
    k2, v2 = k.clone(), v.clone()
    k2[T:2 * T] = torch.randn(T, 64, dtype=k.dtype)
    v2[T:2 * T] = torch.randn(T, 64, dtype=k.dtype)
    got2 = A.pattern_attention(q, k2, v2, A.FRAME_LOCAL, G)
    torch.testing.assert_close(got2[2 * T:], got[2 * T:])


def test_anchor_local_frame0_queries_equal_frame_local():
    q, k, v = _qkv(G.tokens, seed=2)
    T = G.tokens_per_frame
    al = A.pattern_attention(q, k, v, A.ANCHOR_LOCAL, G)
    fl = A.pattern_attention(q, k, v, A.FRAME_LOCAL, G)
    torch.testing.assert_close(al[:T], fl[:T])
    # frame 2 queries: keys are frames {0, 2}
    keys = torch.cat([torch.arange(0, T), torch.arange(2 * T, 3 * T)])
    exp = F.scaled_dot_product_attention(q[2 * T:][None], k[keys][None], v[keys][None])[0]
    torch.testing.assert_close(al[2 * T:], exp, rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("pattern", [A.DENSE, A.FRAME_LOCAL, A.ANCHOR_LOCAL, A.ANCHOR, A.BLOCK_DYNAMIC])
def test_equal_keys_give_mean_of_allowed_values(pattern):
    q, _, v = _qkv(G.tokens, seed=3)
    k = torch.ones(G.tokens, 64, dtype=torch.float64)
    nb = G.frames * G.blocks_per_frame
    sel = torch.tensor([[(i + 1) % nb, (i + 4) % nb] for i in range(nb)], dtype=torch.int32)
    got = A.pattern_attention(q, k, v, pattern, G, sel)
    rows = torch.arange(G.tokens)
    m = A.allowed_mask(pattern, rows, G, sel).double()
    exp = (m @ v) / m.sum(1, keepdim=True)
    torch.testing.assert_close(got, exp, rtol=1e-10, atol=1e-10)


def test_block_dynamic_full_selection_is_patch_only_attention():
    q, k, v = _qkv(G.tokens, seed=4)
    nb = G.frames * G.blocks_per_frame
    sel = torch.arange(nb, dtype=torch.int32).repeat(nb, 1)  # every block selected
    got = A.pattern_attention(q, k, v, A.BLOCK_DYNAMIC, G, sel)
    _, special, _ = A.token_info(G)
    patch = (~special).nonzero().flatten()
    exp_patch = F.scaled_dot_product_attention(q[patch][None], k[patch][None], v[patch][None])[0]
    torch.testing.assert_close(got[patch], exp_patch, rtol=1e-10, atol=1e-10)
    dense = A.pattern_attention(q, k, v, A.DENSE, G)
    torch.testing.assert_close(got[special], dense[special])


@pytest.mark.parametrize("pattern", [A.DENSE, A.FRAME_LOCAL, A.ANCHOR_LOCAL, A.ANCHOR, A.BLOCK_DYNAMIC])
def test_gathered_equals_masked(pattern):
    q, k, v = _qkv(G.tokens, seed=5)
    nb = G.frames * G.blocks_per_frame
    g = torch.Generator().manual_seed(9)
    sel = torch.stack([torch.randperm(nb, generator=g)[:4] for _ in range(nb)]).int()
    sel[0, 1] = -1
    got = A.sparse_attention_gathered(q, k, v, pattern, G, sel, dtype=torch.float64)
    exp = A.pattern_attention(q, k, v, pattern, G, sel)
    torch.testing.assert_close(got, exp, rtol=1e-9, atol=1e-9)


def test_gather_attention_brute_force():
    q, k, v = _qkv(40, d=16, seed=6)
    g = torch.Generator().manual_seed(1)
    idx = torch.randint(0, 40, (40, 7), generator=g)
    idx[3, 2] = -1
    got = A.gather_attention(q, k, v, idx, dtype=torch.float64)
    for i in range(40):
        ids = [j for j in idx[i].tolist() if j >= 0]
        s = [float(q[i] @ k[j]) / 4.0 for j in ids]
        m = max(s)
        w = [math.exp(x - m) for x in s]
        tot = sum(w)
        exp = sum((wi / tot) * v[j] for wi, j in zip(w, ids))
        torch.testing.assert_close(got[i], exp, rtol=1e-9, atol=1e-9)


def test_token_dynamic_rows():
    q, k, v = _qkv(G.tokens, seed=7)
    nimg = G.frames * G.patches
    g = torch.Generator().manual_seed(2)
    est = torch.randint(0, nimg, (nimg, 6), generator=g).int()
    got = A.token_dynamic_attention(q, k, v, est, G)
    _, special, _ = A.token_info(G)
    dense = A.pattern_attention(q, k, v, A.DENSE, G)
    torch.testing.assert_close(got[special], dense[special])
    # image rows never see special keys: changing special keys/values leaves them unchanged
    k2, v2 = k.clone(), v.clone()
    k2[special] += 5.0
    v2[special] -= 3.0
    got2 = A.token_dynamic_attention(q, k2, v2, est, G)
    torch.testing.assert_close(got2[~special], got[~special])
    # stride-s special rows attend keys 0, s, 2s, ...
    gs = A.token_dynamic_attention(q, k, v, est, G, sp2sp_stride=3)
    keys = torch.arange(0, G.tokens, 3)
    exp = F.scaled_dot_product_attention(q[special][None], k[keys][None], v[keys][None])[0]
    torch.testing.assert_close(gs[special], exp, rtol=1e-10, atol=1e-10)


def test_rope2d_closed_form():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 30, 64, generator=g)
    pos = torch.randint(0, 38, (30, 2), generator=g)
    pos[0] = 0
    y = A.rope2d(x, pos)
    torch.testing.assert_close(y[:, 0], x[:, 0])  # position (0, 0) is the identity
    # complex-number form: pairs (i, i+16) of each 32-wide half rotate by pos * base^(-2i/32)
    inv = 1.0 / (100.0 ** (torch.arange(0, 32, 2, dtype=torch.float64) / 32))
    for half, axis in ((0, 0), (1, 1)):
        xs = x[..., half * 32:(half + 1) * 32].double()
        z = torch.complex(xs[..., :16], xs[..., 16:])
        rot = z * torch.exp(1j * pos[:, axis, None].double() * inv)
        exp = torch.cat([rot.real, rot.imag], dim=-1)
        torch.testing.assert_close(y[..., half * 32:(half + 1) * 32].double(), exp, rtol=0, atol=2e-5)
    # norm preserving per rotated pair
    torch.testing.assert_close(y.norm(dim=-1), x.norm(dim=-1), rtol=1e-5, atol=1e-5)


def test_vggt_positions_layout():
    pos = A.vggt_positions(2, 3, 4)
    assert pos.shape == (2 * 17, 2)
    assert pos[:5].abs().sum() == 0
    assert pos[5].tolist() == [1, 1] and pos[16].tolist() == [3, 4]
    assert torch.equal(pos[17:], pos[:17])


def test_broadcast_first_pins():
    """broadcast_first (saf3r/patch/sparse_attention.py:110-131): frame 0 is frame-local attention,
    shifting a frame's V by a constant shifts its rows by it (the map's rows sum to one), and a
    per-element loop over the formula agrees on a tiny case."""
    q, k, v = _qkv(G.tokens, seed=11)
    T = G.tokens_per_frame
    got = A.broadcast_attention(q, k, v, G)
    fl = A.pattern_attention(q, k, v, A.FRAME_LOCAL, G)
    torch.testing.assert_close(got[:T], fl[:T], rtol=1e-10, atol=1e-10)
    # frames 1, 2 given frame 0's V plus a constant: rows equal frame 0's rows plus that constant
    shift = torch.randn(G.frames, 64, dtype=torch.float64)
    v2 = v[:T].repeat(G.frames, 1) + shift.repeat_interleave(T, dim=0)
    got2 = A.broadcast_attention(q, k, v2, G)
    for f in range(G.frames):
        torch.testing.assert_close(got2[f * T:(f + 1) * T], got2[:T] - shift[0] + shift[f], rtol=1e-9, atol=1e-9)
    # the rows never read q or k beyond frame 0
    q3, k3 = q.clone(), k.clone()
    q3[T:] = 0.0
    k3[T:] = 7.0
    torch.testing.assert_close(A.broadcast_attention(q3, k3, v, G), got)
    # element loop, 2 frames x 3 tokens, d = 2
    g = A.Geometry(frames=2, tokens_per_frame=3, num_special=1)
    qs, ks, vs = _qkv(6, d=2, seed=12)
    out = A.broadcast_attention(qs, ks, vs, g)
    for f in range(2):
        for i in range(3):
            w = [math.exp(float(qs[i] @ ks[j]) / math.sqrt(2)) for j in range(3)]
            for d in range(2):
                exp = sum(w[j] * float(vs[3 * f + j, d]) for j in range(3)) / sum(w)
                assert abs(float(out[3 * f + i, d]) - exp) < 1e-12
    # the gathered entry point dispatches to it
    torch.testing.assert_close(A.sparse_attention_gathered(q, k, v, A.BROADCAST, G, dtype=torch.float64), got)



# ---- the layer at the reference's rounding points (oracle.attention.reference_layer) ----------

def _layer_inputs(ph=3, pw=4, frames=2, H=4, seed=0):
    g = torch.Generator().manual_seed(seed)
    C = 64 * H
    G2 = A.Geometry(frames=frames, tokens_per_frame=5 + ph * pw)
    x = torch.randn(G2.tokens, C, generator=g).to(torch.bfloat16).float()
    w_qkv = torch.randn(3 * C, C, generator=g) / math.sqrt(C)
    b_qkv = 0.1 * torch.randn(3 * C, generator=g)
    ln = (1 + 0.2 * torch.randn(64, generator=g), 0.1 * torch.randn(64, generator=g))
    w_p = torch.randn(C, C, generator=g) / math.sqrt(C)
    b_p = 0.1 * torch.randn(C, generator=g)
    pos = A.vggt_positions(frames, ph, pw)
    return G2, x, w_qkv, b_qkv, ln, w_p, b_p, pos


def test_reference_layer_all_full_is_the_unpatched_module():
    """Every head 'full': the restatement equals an independent module (torch SDPA, its own RoPE)
    run in fp64 on the same bf16 weights, within the bf16 rounding of q/k/v and head outputs."""
    import importlib
    import __graft_entry__
    vggt = importlib.import_module(__graft_entry__.package().__name__ + ".vggt")
    G2, x, w_qkv, b_qkv, ln, w_p, b_p, pos = _layer_inputs()
    C = x.shape[1]
    m = vggt.Attention(C, 4, qkv_bias=True, proj_bias=True, qk_norm=True, rope=vggt.RotaryPositionEmbedding2D(100.0))
    with torch.no_grad():
        m.qkv.weight.copy_(w_qkv.to(torch.bfloat16).float())
        m.qkv.bias.copy_(b_qkv.to(torch.bfloat16).float())
        m.proj.weight.copy_(w_p.to(torch.bfloat16).float())
        m.proj.bias.copy_(b_p.to(torch.bfloat16).float())
        for n in (m.q_norm, m.k_norm):
            n.weight.copy_(ln[0])
            n.bias.copy_(ln[1])
        m = m.double()
        exp = m(x.double()[None], pos[None])[0]
    y, _ = A.reference_layer(x, w_qkv, b_qkv, ln, ln, w_p, b_p, pos, [{"mode": "full"}] * 4, G2)
    torch.testing.assert_close(y, exp, rtol=0, atol=3e-2)
    assert (y - exp).abs().mean() < 3e-3
    # a transposed head split or a dropped RoPE term is far outside that bound
    y2, _ = A.reference_layer(x, w_qkv, b_qkv, ln, ln, w_p, b_p, torch.zeros_like(pos), [{"mode": "full"}] * 4, G2)
    assert (y2 - exp).abs().max() > 0.1


def test_reference_layer_mode_identities():
    """Key sets that cover every key reduce to 'full'; frame-local rows ignore other frames;
    a skipped head contributes nothing but the projection bias; broadcast_first on one frame is
    'full' up to its bf16 score rounding; dino rows over every image token exclude only specials."""
    G2, x, w_qkv, b_qkv, ln, w_p, b_p, pos = _layer_inputs()
    N, T = G2.tokens, G2.tokens_per_frame
    args = (x, w_qkv, b_qkv, ln, ln, w_p, b_p, pos)
    full, _ = A.reference_layer(*args, [{"mode": "full"}] * 4, G2)
    cover = [{"mode": "stride", "stride": 1}, {"mode": "q_probe_topk", "topk": N},
             {"mode": "q_probe_topk", "stride": 1, "include_as": True}, {"mode": "full"}]
    y, info = A.reference_layer(*args, cover, G2)
    torch.testing.assert_close(y, full, rtol=0, atol=1e-12)
    assert all(len(info["keysets"][h]) == N for h in range(3))
    # the probe key set is the top-k of the fp32 mean-query scores
    few = [{"mode": "q_probe_topk", "topk": 7}] + [{"mode": "full"}] * 3
    _, inf2 = A.reference_layer(*args, few, G2)
    assert len(inf2["keysets"][0]) == 7
    # skip: the head's columns of attn are zero, so y differs from full by that head's share only
    sk = [{"mode": "skip"}] + [{"mode": "full"}] * 3
    ys, _ = A.reference_layer(*args, sk, G2)
    assert (ys - full).abs().max() > 1e-3
    # frame-local rows of frame 1 do not depend on frame 0's tokens
    fl = [{"mode": "global_to_frame"}] * 4
    y1, _ = A.reference_layer(*args, fl, G2)
    x2 = x.clone()
    x2[:T] = torch.randn(T, x.shape[1]).to(torch.bfloat16).float()
    y2, _ = A.reference_layer(x2, *args[1:], fl, G2)
    torch.testing.assert_close(y1[T:], y2[T:], rtol=0, atol=1e-12)
    # broadcast_first with one frame is full attention (bf16 scores and P)
    G1 = A.Geometry(frames=1, tokens_per_frame=T)
    b1, _ = A.reference_layer(x[:T], *args[1:-1], pos[:T], [{"mode": "broadcast_first"}] * 4, G1)
    f1, _ = A.reference_layer(x[:T], *args[1:-1], pos[:T], [{"mode": "full"}] * 4, G1)
    torch.testing.assert_close(b1, f1, rtol=0, atol=5e-2)
    # dino rows listing every image token: image rows attend all image tokens (fp32 q/k), specials all keys
    P = G2.patches
    est = torch.arange(G2.frames * P, dtype=torch.int32)[None].repeat(G2.frames * P, 1)
    dn = [{"mode": "dino_topk"}] * 4
    yd, _ = A.reference_layer(*args, dn, G2, est_topk_idx=est)
    yf, _ = A.reference_layer(*args, [{"mode": "full"}] * 4, G2)
    spec = torch.tensor([f * T + i for f in range(G2.frames) for i in range(5)])
    torch.testing.assert_close(yd[spec], yf[spec], rtol=0, atol=1e-12)
    assert (yd - yf).abs().max() > 1e-4  # image rows exclude the special keys
