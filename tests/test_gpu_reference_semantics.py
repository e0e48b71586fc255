"""The patched layer at real VGGT geometry and at the reference's own rounding points.

- ``test_all_modes_match_reference_semantics``: x -> y of the wrapper (dim 1024, 16 heads, 4 frames of
  37 x 37 patches) against ``oracle.attention.reference_layer``, which keeps q/k in fp32 after
  LayerNorm / RoPE, feeds SDPA modes bf16 q/k/v, computes the q_probe_topk mean and scores in fp32 and
  gathers dino_topk rows with fp32 q/k, as the reference does under autocast. The kernels round q/k to
  bf16 right after LayerNorm / RoPE; the test bounds the effect (max-abs 2e-2, mean-abs 2e-3) and reports
  how many key-set members and lazy indices differ.
- ``test_wired_layer_vggt_geometry``: the same geometry with the benchmark's block-pattern head table
  against the oracle layer on the kernels' own q/k/v.
- ``test_wired_layer_128_frames_sampled_rows``: one wired layer at 128 frames (175,872 tokens) with the
  benchmark's head table; block lists bit-exact against the oracle, sampled output rows of y against
  the oracle's attention rows through the projection.
- ``test_lazy_token_topk_128_frames_sampled``: the lazy per-frame top-4 at 128 x 1369 image tokens for
  sampled queries against fp64 scores.
"""
import importlib

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import selection as OS
from tests.layer_check import check_layer_output, err, make_stack
from tests.layout_ref import slot_tokens

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
PH = PW = 37


@pytest.fixture(scope="module")
def mods(pkg):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return tuple(importlib.import_module(pkg.__name__ + m) for m in (".patch", ".vggt", ".ops", ".synth"))


HEAD_TABLE = [
    {"mode": "full"}, {"mode": "global_to_frame"}, {"mode": "all_to_first"}, {"mode": "broadcast_first"},
    {"mode": "stride", "stride": 4, "include_as": True}, {"mode": "stride", "stride": 128, "shift": True},
    {"mode": "q_probe_topk", "stride": 4}, {"mode": "q_probe_topk", "topk": 200, "include_as": True},
    {"mode": "q_probe_topk", "stride": 8, "q_sample_ratio": 0.25}, {"mode": "dino_topk", "is_first_dino": True},
    {"mode": "dino_topk"}, {"mode": "dino_topk", "dino_sp2sp_stride": 4}, {"mode": "skip"}, {"mode": "full"},
    {"mode": "global_to_frame"}, {"mode": "q_probe_topk", "stride": 16},
]


def _amplify(m):
    """Scale the output projection by 16, so that the layer output has a magnitude (std ~0.5) at which
    an absolute tolerance of 2e-2 is a real bound. The attention outputs keep the scale of V (std ~0.6),
    where a bf16 ulp is far below the tolerance."""
    with torch.no_grad():
        for b in m.aggregator.global_blocks:
            b.attn.proj.weight *= 16
    return m


def _groups(table):
    groups = []
    for h, c in enumerate(table):
        groups.append(dict(c, head_ids=[h]))
    return groups


def test_all_modes_match_reference_semantics(mods, pkg):
    plug, vggt, ops, synth = mods
    F_, H, dim = 4, 16, 1024
    m = _amplify(make_stack(vggt, 1, dim, H, seed=21)).to(DEV).to(torch.bfloat16)
    plug.patch_model(m, "vggt", {"patch_module": {"type": "headsparse", "topk_mode": "token", "lazy_dino_topk": True,
                                                  "topk": 4}, "sparse_config": {"0": _groups(HEAD_TABLE)}})
    plug.update_args_per_forward(m, "vggt", PH * 14, PW * 14)
    geom = pkg.Geometry(F_, PH * PW + 5, 5)
    N = geom.tokens
    g = torch.Generator().manual_seed(22)
    x = torch.randn(1, N, dim, generator=g).to(torch.bfloat16)
    pos = synth.vggt_positions(F_, PH, PW)[None]
    w = m.aggregator.global_blocks[0].attn
    w.keep_attention = True
    with torch.no_grad():
        y = w(x.to(DEV), pos.to(DEV))[0].float().cpu()
        attn = w.last_attention.float().cpu().reshape(N, H, 64).permute(1, 0, 2)
    om = w.orig_module
    og = OA.Geometry(F_, geom.tokens_per_frame, 5)
    cpu = lambda t: t.detach().float().cpu()
    yref, info = OA.reference_layer(x[0].float(), cpu(om.qkv.weight), cpu(om.qkv.bias),
                                    (cpu(om.q_norm.weight), cpu(om.q_norm.bias)),
                                    (cpu(om.k_norm.weight), cpu(om.k_norm.bias)),
                                    cpu(om.proj.weight), cpu(om.proj.bias), pos[0].long(), HEAD_TABLE, og, lazy_topk=4)
    # how far the kernels' selections (from bf16 q/k) are from the reference's (fp32 q/k)
    ks = w.last_keysets
    for i, h in enumerate(w.keyset_heads):
        got = set(ks.idx[i, :int(ks.count[i])].cpu().tolist())
        want = set(info["keysets"][h].tolist()) if h in info["keysets"] else set(range(0, N, HEAD_TABLE[h].get(
            "dino_sp2sp_stride", 1)))
        print(f"head {h} {HEAD_TABLE[h]['mode']}: {len(got)} members, {len(got ^ want)} differ from the "
              f"fp32 reference selection", flush=True)
        assert len(got ^ want) <= max(8, len(want) // 50)
    est, est_ref = w.est_topk_idx.cpu(), info["est_topk_idx"]
    same = (est == est_ref).float().mean().item()
    print(f"lazy indices: {same:.4%} identical to the reference's", flush=True)
    assert same >= 0.99
    worst = []
    for h in range(H):
        hm, hmean = err(attn[h], info["heads"][h])
        print(f"head {h} {HEAD_TABLE[h]['mode']}: attention max {hm:.3g} mean {hmean:.3g}", flush=True)
        worst.append((hm, hmean, h))
    mx, mean = err(y, yref)
    ymax, ymean = yref.abs().max().item(), yref.abs().mean().item()
    print(f"layer vs reference semantics: max {mx:.3g} mean {mean:.3g} (|y| max {ymax:.3g}, mean {ymean:.3g})",
          flush=True)
    for hm, hmean, h in worst:
        assert hm <= 2e-2 and hmean <= 2e-3, f"head {h}: max {hm:.3g} mean {hmean:.3g}"
    assert mx <= 2e-2 + ymax * 2 ** -8 and mean <= 2e-3 + ymean * 2 ** -8


def test_wired_layer_vggt_geometry(mods, pkg):
    """dim 1024, 16 heads, 4 frames x (5 + 37 x 37) tokens, the benchmark's seeded block table."""
    plug, vggt, ops, synth = mods
    F_, H, dim = 4, 16, 1024
    m = _amplify(make_stack(vggt, 1, dim, H, seed=23)).to(DEV).to(torch.bfloat16)
    names = {ops.BLOCK_DYNAMIC: "block_topk", ops.FRAME_LOCAL: "frame_local", ops.ANCHOR_LOCAL: "anchor_local",
             ops.DENSE: "dense"}
    table = synth.seeded_patterns(H, seed=1)
    plug.patch_model(m, "vggt", {"patch_module": {"type": "headsparse", "block_topk": 4},
                                 "sparse_config": {"0": _groups([{"mode": names[p]} for p in table])}})
    plug.update_args_per_forward(m, "vggt", PH * 14, PW * 14)
    geom = pkg.Geometry(F_, PH * PW + 5, 5)
    g = torch.Generator().manual_seed(24)
    x = torch.randn(1, geom.tokens, dim, generator=g).to(torch.bfloat16).to(DEV)
    pos = synth.vggt_positions(F_, PH, PW).to(DEV)[None]
    w = m.aggregator.global_blocks[0].attn
    w.keep_attention = True
    with torch.no_grad():
        y = w(x, pos)
        torch.cuda.synchronize()
        check_layer_output(w, x, pos, y[0], geom, ops, 0)


def _rows_of(packed, geom, tokens, head):
    """Rows of ``tokens`` of one head from packed [H, L, 64] Q or K."""
    slot = torch.full((geom.tokens,), -1, dtype=torch.long)
    toks = slot_tokens(geom.frames, geom.tokens_per_frame, geom.num_special)
    valid = toks >= 0
    slot[toks[valid]] = torch.arange(len(toks))[valid]
    return packed[head][slot[tokens].to(packed.device)].float().cpu()


def test_wired_layer_128_frames_sampled_rows(mods, pkg):
    plug, vggt, ops, synth = mods
    F_, H, dim = 128, 16, 1024
    m = _amplify(make_stack(vggt, 1, dim, H, seed=25)).to(DEV).to(torch.bfloat16)
    table = synth.seeded_patterns(H, seed=1)
    names = {ops.BLOCK_DYNAMIC: "block_topk", ops.FRAME_LOCAL: "frame_local", ops.ANCHOR_LOCAL: "anchor_local",
             ops.DENSE: "dense"}
    plug.patch_model(m, "vggt", {"patch_module": {"type": "headsparse", "block_topk": 4},
                                 "sparse_config": {"0": _groups([{"mode": names[p]} for p in table])}})
    plug.update_args_per_forward(m, "vggt", PH * 14, PW * 14)
    geom = pkg.Geometry(F_, PH * PW + 5, 5)
    N = geom.tokens
    g = torch.Generator(device=DEV).manual_seed(26)
    x = torch.randn(1, N, dim, generator=g, device=DEV).to(torch.bfloat16)
    pos = synth.vggt_positions(F_, PH, PW).to(DEV)[None]
    w = m.aggregator.global_blocks[0].attn
    w.keep_attention = True
    om = w.orig_module
    with torch.no_grad():
        y = w(x, pos)
        qkv = om.qkv(x).reshape(N, 3 * dim).contiguous()
        tord = ops.token_order_heads(w.patterns)
        qs = w.q_scaled_heads()  # Q as the wrapper packed it (softmax scale folded in)
        qp, kp, vp = ops.pack_qkv(qkv, qkv[:, dim:], qkv[:, 2 * dim:], 3 * dim, 64, geom, H,
                                  ln_q=(om.q_norm.weight, om.q_norm.bias), ln_k=(om.k_norm.weight, om.k_norm.bias),
                                  pos=pos[0], rope_base=100.0, q_scaled=qs)  # every head padded, for reading back
        torch.cuda.synchronize()
    print("128-frame wired layer ran", flush=True)
    # block lists: bit-exact against the oracle's selection from the same packed q/k
    toks_all = torch.arange(N)
    sel_of = {}
    for i, h in enumerate(w.dyn_heads):
        qh = _rows_of(qp, geom, toks_all, h).to(torch.bfloat16)
        kh = _rows_of(kp, geom, toks_all, h).to(torch.bfloat16)
        bits = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)
        want = OS.block_select(bits(qh), bits(kh), F_, geom.tokens_per_frame, 5, 4)
        assert np.array_equal(w.last_selection[i].cpu().numpy(), want), f"block list of head {h}"
        sel_of[h] = torch.from_numpy(want)
    print(f"{len(sel_of)} block lists bit-exact", flush=True)
    rng = torch.Generator().manual_seed(27)
    T = geom.tokens_per_frame
    rows = torch.unique(torch.cat([torch.arange(5), torch.arange(T - 64, T + 5), torch.arange(N - T, N - T + 70),
                                   torch.randint(0, N, (160,), generator=rng)]))
    og = OA.Geometry(F_, T, 5)
    attn = torch.empty(len(rows), H, 64, dtype=torch.float64)
    vnat = qkv[:, 2 * dim:].reshape(N, H, 64)
    c = ops.prescale_factor()
    for h, pat in enumerate(w.patterns):
        qh = _rows_of(qp, geom, rows, h) / (c if qs[h] else 1.0)
        kh = _rows_of(kp, geom, toks_all, h)
        vh = vnat[:, h].float().cpu()
        mask = OA.allowed_mask(pat, rows, og, sel_of.get(h))
        attn[:, h] = OA.masked_attention(qh, kh, vh, mask, dtype=torch.float64)
    got_attn = w.last_attention[rows.to(DEV)].float().cpu().reshape(len(rows), H, 64)
    amx, amean = err(got_attn, attn)
    print(f"128-frame wired layer attention, {len(rows)} rows: max {amx:.3g} mean {amean:.3g}", flush=True)
    assert amx <= 2e-2 and amean <= 2e-3
    a = attn.reshape(len(rows), dim).to(torch.bfloat16).double()
    yref = a @ om.proj.weight.double().cpu().T + om.proj.bias.double().cpu()
    mx, mean = err(y[0][rows.to(DEV)].cpu(), yref)
    ymax, ymean = yref.abs().max().item(), yref.abs().mean().item()
    print(f"128-frame wired layer y, {len(rows)} rows: max {mx:.3g} mean {mean:.3g} (|y| max {ymax:.3g})", flush=True)
    assert mx <= 2e-2 + ymax * 2 ** -8 and mean <= 2e-3 + ymean * 2 ** -8
    del tord


def test_lazy_token_topk_128_frames_sampled(mods, pkg):
    """The lazy per-frame top-4 over 128 x 1369 image tokens (175,232 queries and keys), for 96 sampled
    queries: every selected key's fp64 score equals the fp64 top-4 score of its frame within 1e-4
    (near ties may pick either key), and at least 99% of the indices are identical."""
    plug, vggt, ops, synth = mods
    F_, P = 128, 1369
    g = torch.Generator(device=DEV).manual_seed(28)
    q = (torch.randn(F_ * P, 64, generator=g, device=DEV) * 0.6).to(torch.bfloat16)
    k = (torch.randn(F_ * P, 64, generator=g, device=DEV) * 0.6).to(torch.bfloat16)
    k[P:] += 0.5 * k[:P].repeat(F_ - 1, 1)  # correlated frames, as corresponding tokens are
    idx = ops.token_topk(q, k, F_, P, 4)
    torch.cuda.synchronize()
    rng = torch.Generator().manual_seed(29)
    qs = torch.randint(0, F_ * P, (96,), generator=rng)
    s = (q[qs.to(DEV)].double() @ k.double().T).cpu().numpy()  # [96, F*P]
    ref = OS.frame_topk(s.astype(np.float32), F_, 4)
    got = idx[qs.to(DEV)].cpu().numpy()
    gs = np.take_along_axis(s, got.astype(np.int64), 1)
    rs = np.take_along_axis(s, ref.astype(np.int64), 1)
    same = (got == ref).mean()
    print(f"lazy top-4 at 128 x 1369: {same:.4%} identical, max score gap {np.abs(gs - rs).max():.3g}", flush=True)
    assert np.allclose(gs, rs, atol=1e-4) and same >= 0.99
