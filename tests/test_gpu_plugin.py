"""GPU parity of the patched global-attention layer (qkv -> LayerNorm/RoPE -> sparse heads -> proj)."""
import importlib

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import selection as OS
from tests.layer_check import check_layer, check_layer_output, err, make_stack
from tests.layout_ref import slot_tokens, unpack_rows, unpack_v

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def mods(pkg):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return tuple(importlib.import_module(pkg.__name__ + m) for m in (".patch", ".vggt", ".ops", ".synth"))


_err = err
_make = make_stack


def test_layer_matches_oracle_all_modes(mods, pkg):
    plug, vggt, ops, synth = mods
    ph, pw, F_, H = 7, 9, 4, 8
    dim = 64 * H
    m = _make(vggt, 2, dim, H).to(DEV).to(torch.bfloat16)
    cfg = {"patch_module": {"type": "headsparse", "topk_mode": "token", "lazy_dino_topk": True, "topk": 3,
                            "block_topk": 2},
           "sparse_config": {
               "0": [{"mode": "global_to_frame", "head_ids": [1]}, {"mode": "all_to_first", "head_ids": [2]},
                     {"mode": "dino_topk", "head_ids": [3], "is_first_dino": True, "dino_sp2sp_stride": 1},
                     {"mode": "anchor_local", "head_ids": [4]}, {"mode": "block_topk", "head_ids": [5, 6]},
                     {"mode": "skip", "head_ids": [7]}],
               "1": [{"mode": "dino_topk", "head_ids": [0, 5]}, {"mode": "block_topk", "head_ids": [2]}]}}
    plug.patch_model(m, "vggt", cfg)
    plug.update_args_per_forward(m, "vggt", ph * 14, pw * 14)
    T = ph * pw + 5
    geom = pkg.Geometry(F_, T, 5)
    N = geom.tokens
    g = torch.Generator().manual_seed(3)
    x = torch.randn(1, N, dim, generator=g).to(torch.bfloat16).to(DEV)
    pos = synth.vggt_positions(F_, ph, pw).to(DEV)[None]
    toks = slot_tokens(F_, T, 5)
    og = OA.Geometry(F_, T, 5)
    with torch.no_grad():
        for li in range(2):
            w = m.aggregator.global_blocks[li].attn
            y = w(x, pos)
            torch.cuda.synchronize()
            om = w.orig_module
            qkv = om.qkv(x).reshape(N, 3 * dim).contiguous()
            # exact q/k/v the kernels consumed (packing is deterministic)
            qp, kp, vp = ops.pack_qkv(qkv, qkv[:, dim:], qkv[:, 2 * dim:], 3 * dim, 64, geom, H,
                                      ln_q=(om.q_norm.weight, om.q_norm.bias), ln_k=(om.k_norm.weight, om.k_norm.bias),
                                      pos=pos[0], rope_base=100.0)
            torch.cuda.synchronize()
            q, _ = unpack_rows(qp.cpu(), toks, N)
            k, _ = unpack_rows(kp.cpu(), toks, N)
            v, _ = unpack_v(vp.cpu(), toks, N)
            # the packed values agree with the oracle prologue (fp32 LayerNorm + RoPE, bf16 rounding)
            lnq = (om.q_norm.weight.float().cpu(), om.q_norm.bias.float().cpu())
            lnk = (om.k_norm.weight.float().cpu(), om.k_norm.bias.float().cpu())
            qr, kr, vr = OA.qkv_prologue(qkv.cpu(), H, lnq, lnk, pos[0].cpu())
            assert torch.equal(v, vr)
            assert _err(q, qr)[0] < 0.05 and _err(k, kr)[0] < 0.05
            est = w.est_topk_idx.cpu()
            if li == 0:  # lazy indices from head 3: near-tie tolerant check against the oracle
                qi = q[3][OA.image_token_ids(og)].double()
                s = (qi @ k[3][OA.image_token_ids(og)].double().T).float().numpy()
                ref = OS.frame_topk(s, F_, 3)
                gs = np.take_along_axis(s, est.numpy().astype(np.int64), 1)
                rs = np.take_along_axis(s, ref.astype(np.int64), 1)
                assert np.allclose(gs, rs, atol=1e-3)
            else:  # shared from layer 0
                assert torch.equal(est, m.aggregator.global_blocks[0].attn.est_topk_idx.cpu())
            # every head against the oracle layer (block lists bit-exact, dino rows over the fp32 q / k)
            check_layer_output(w, x, pos, y[0], geom, ops, li)


def test_all_full_equals_unpatched_module(mods, pkg):
    plug, vggt, ops, synth = mods
    ph, pw, F_, H = 5, 6, 3, 4
    dim = 64 * H
    m = _make(vggt, 1, dim, H, seed=1)
    ref_mod = vggt.GlobalAttentionStack(depth=1, dim=dim, num_heads=H)
    ref_mod.load_state_dict(m.state_dict())
    m = m.to(DEV).to(torch.bfloat16)
    plug.patch_model(m, "vggt", {"patch_module": {"type": "headsparse"}, "sparse_config": {"0": []}})
    plug.update_args_per_forward(m, "vggt", ph * 14, pw * 14)
    N = F_ * (ph * pw + 5)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(1, N, dim, generator=g).to(torch.bfloat16)
    pos = synth.vggt_positions(F_, ph, pw)[None].long()
    with torch.no_grad():
        y = m.aggregator.global_blocks[0].attn(x.to(DEV), pos.to(DEV))
        yref = ref_mod.aggregator.global_blocks[0].attn(x.float(), pos)  # fp32 on the CPU
    mx, mean = _err(y[0].cpu(), yref[0])
    print(f"all-full vs unpatched: max {mx:.3g} mean {mean:.3g}", flush=True)
    assert mx <= 2e-2 and mean <= 2e-3


def test_autocast_fp32_module(mods, pkg):
    """The reference runs fp32 weights under autocast(bf16); the wrapper accepts that setting too."""
    plug, vggt, ops, synth = mods
    ph, pw, F_, H = 4, 4, 2, 2
    dim = 64 * H
    m = _make(vggt, 1, dim, H, seed=2).to(DEV)
    plug.patch_model(m, "vggt", {"patch_module": {"type": "headsparse"},
                                 "sparse_config": {"0": [{"mode": "global_to_frame", "head_ids": [1]}]}})
    plug.update_args_per_forward(m, "vggt", ph * 14, pw * 14)
    N = F_ * (ph * pw + 5)
    x = torch.randn(1, N, dim, device=DEV)
    pos = synth.vggt_positions(F_, ph, pw).to(DEV)[None]
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        y = m.aggregator.global_blocks[0].attn(x, pos)
    with torch.no_grad():
        y32 = m.aggregator.global_blocks[0].attn(x, pos)
    assert y.shape == (1, N, dim) and torch.isfinite(y.float()).all()
    assert y32.dtype == torch.float32
    assert _err(y, y32)[0] < 5e-2


_check_layer = check_layer


def test_layer_keyset_modes(mods, pkg):
    plug, vggt, ops, synth = mods
    ph, pw, F_, H = 7, 9, 4, 8
    dim = 64 * H
    m = _make(vggt, 1, dim, H, seed=5).to(DEV).to(torch.bfloat16)
    cfg = {"patch_module": {"type": "headsparse"},
           "sparse_config": {"0": [
               {"mode": "stride", "head_ids": [0], "stride": 4, "include_as": True, "is_base": True},
               {"mode": "stride", "head_ids": [1], "stride": 128, "include_as": True},
               {"mode": "q_probe_topk", "head_ids": [2, 3], "stride": 4},
               {"mode": "q_probe_topk", "head_ids": [4], "topk": 100, "include_as": True},
               {"mode": "stride", "head_ids": [5], "stride": 3, "shift": True, "include_as": False},
               {"mode": "global_to_frame", "head_ids": [6]},
               {"mode": "broadcast_first", "head_ids": [7]}]}}
    plug.patch_model(m, "vggt", cfg)
    plug.update_args_per_forward(m, "vggt", ph * 14, pw * 14)
    geom = pkg.Geometry(F_, ph * pw + 5, 5)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(1, geom.tokens, dim, generator=g).to(torch.bfloat16).to(DEV)
    pos = synth.vggt_positions(F_, ph, pw).to(DEV)[None]
    with torch.no_grad():
        _check_layer(m.aggregator.global_blocks[0].attn, x, pos, geom, ops, 0)


def test_layer_sampled_probe_and_strided_dino(mods, pkg):
    """q_probe_topk with q_sample_ratio < 1 and dino_topk with dino_sp2sp_stride != 1 (special rows over
    keys 0, s, 2s, ...; sparse_attention.py:154-157, 199-204) against the oracle layer."""
    plug, vggt, ops, synth = mods
    ph, pw, F_, H = 7, 9, 4, 8
    dim = 64 * H
    m = _make(vggt, 2, dim, H, seed=9).to(DEV).to(torch.bfloat16)
    cfg = {"patch_module": {"type": "headsparse", "topk_mode": "token", "lazy_dino_topk": True, "topk": 3},
           "sparse_config": {"0": [
               {"mode": "dino_topk", "head_ids": [0], "is_first_dino": True, "dino_sp2sp_stride": 1},
               {"mode": "dino_topk", "head_ids": [1], "dino_sp2sp_stride": 4},
               {"mode": "q_probe_topk", "head_ids": [2], "stride": 4, "q_sample_ratio": 0.25},
               {"mode": "q_probe_topk", "head_ids": [3], "topk": 50, "q_sample_ratio": 0.05, "include_as": True},
               {"mode": "q_probe_topk", "head_ids": [4], "stride": 8},
               {"mode": "stride", "head_ids": [5], "stride": 16}],
               "1": [{"mode": "dino_topk", "head_ids": [2, 6], "dino_sp2sp_stride": 3},
                     {"mode": "dino_topk", "head_ids": [7]}]}}
    plug.patch_model(m, "vggt", cfg)
    plug.update_args_per_forward(m, "vggt", ph * 14, pw * 14)
    geom = pkg.Geometry(F_, ph * pw + 5, 5)
    g = torch.Generator().manual_seed(10)
    x = torch.randn(1, geom.tokens, dim, generator=g).to(torch.bfloat16).to(DEV)
    pos = synth.vggt_positions(F_, ph, pw).to(DEV)[None]
    w0 = m.aggregator.global_blocks[0].attn
    assert w0.patterns[1] == ops.TOKEN_DYNAMIC_KEYSET and w0.patterns[0] == ops.TOKEN_DYNAMIC
    with torch.no_grad():
        for li in range(2):
            _check_layer(m.aggregator.global_blocks[li].attn, x, pos, geom, ops, li)


def test_reference_profile_layers(mods, pkg):
    """Layers 11-13 of the reference's VGGT head profile (stride, q_probe_topk, all_to_first,
    global_to_frame and lazily shared dino_topk heads) at a small frame/patch shape."""
    import json
    import os
    plug, vggt, ops, synth = mods
    with open(os.path.join(os.path.dirname(__file__), "golden", "vggt_eth3d_profile.json")) as f:
        prof = json.load(f)
    ph, pw, F_, H = 6, 8, 3, 16
    dim = 64 * H
    m = _make(vggt, 24, dim, H, seed=7).to(DEV).to(torch.bfloat16)
    plug.patch_model(m, "vggt", {"patch_module": {"type": "headsparse", "topk_mode": "token", "lazy_dino_topk": True,
                                                  "topk": 4}, "sparse_config": prof})
    plug.update_args_per_forward(m, "vggt", ph * 14, pw * 14)
    geom = pkg.Geometry(F_, ph * pw + 5, 5)
    g = torch.Generator().manual_seed(8)
    x = torch.randn(1, geom.tokens, dim, generator=g).to(torch.bfloat16).to(DEV)
    pos = synth.vggt_positions(F_, ph, pw).to(DEV)[None]
    with torch.no_grad():
        for li in (11, 12, 13):
            _check_layer(m.aggregator.global_blocks[li].attn, x, pos, geom, ops, li)


def test_headprofile_records_oracle_nmse(mods, pkg):
    """headprofile on one layer: the layer returns full attention, and every recorded candidate error
    is the oracle's NMSE of that candidate against full attention (saf3r/patch/wrapper.py:163-205)."""
    plug, vggt, ops, synth = mods
    ph, pw, F_, H = 6, 7, 3, 4
    dim = 64 * H
    m = _make(vggt, 13, dim, H, seed=11).to(DEV).to(torch.bfloat16)
    cfg = {"patch_module": {"type": "headprofile", "topk": 6, "per_frame_topk": True, "max_topk": 2048,
                            "include_first_frame": False}}
    plug.patch_model(m, "vggt", cfg)
    plug.update_args_per_forward(m, "vggt", ph * 14, pw * 14)
    geom = pkg.Geometry(F_, ph * pw + 5, 5)
    g = torch.Generator().manual_seed(12)
    tokens = torch.randn(F_, ph * pw, 1024, generator=g).to(DEV)
    plug.set_dino_topk_from_features(m, tokens, cfg)
    x = torch.randn(1, geom.tokens, dim, generator=g).to(torch.bfloat16).to(DEV)
    pos = synth.vggt_positions(F_, ph, pw).to(DEV)[None]
    prof = m.aggregator.global_blocks[12].attn
    with torch.no_grad():
        y = prof(x, pos)
        yd = prof.full(x, pos)  # the all-dense wrapper
    assert _err(y, yd)[0] <= 2e-2  # the same full attention (walk order may differ in the last bits)
    N = geom.tokens
    om = prof.orig_module
    qkv = om.qkv(x).reshape(N, 3 * dim).contiguous()
    qp, kp, vp, qk32 = ops.pack_qkv(qkv, qkv[:, dim:], qkv[:, 2 * dim:], 3 * dim, 64, geom, H,
                                    ln_q=(om.q_norm.weight, om.q_norm.bias), ln_k=(om.k_norm.weight, om.k_norm.bias),
                                    pos=pos[0], rope_base=100.0, fp32_heads=[True] * H)
    toks = slot_tokens(geom.frames, geom.tokens_per_frame, geom.num_special)
    q, _ = unpack_rows(qp.cpu(), toks, N)
    k, _ = unpack_rows(kp.cpu(), toks, N)
    v, _ = unpack_v(vp.cpu(), toks, N)
    rows32 = {h: (qk32[h, 0].cpu(), qk32[h, 1].cpu()) for h in range(H)}  # the dino gather reads fp32 q / k
    og = OA.Geometry(geom.frames, geom.tokens_per_frame, geom.num_special)
    dense = OA.head_outputs(q.float(), k.float(), v.float(), [ops.DENSE] * H, og, dtype=torch.float64)
    energy = (dense ** 2).mean(dim=(1, 2))
    est = prof.shared.est_topk_idx.cpu()
    checked = 0
    for i, (c, w) in enumerate(zip(prof.cfgs, prof.candidates)):
        sel = {}
        if w.keyset_heads:
            ks = w.last_keysets
            sel = {h: ks.idx[j, :int(ks.count[j])].cpu() for j, h in enumerate(w.keyset_heads)}
        out = OA.head_outputs(q.float(), k.float(), v.float(), list(w.patterns), og, sel, est_topk_idx=est,
                              dtype=torch.float64, gather_qk_by_head=rows32)
        nmse = ((out - dense) ** 2).mean(dim=(1, 2)) / energy
        for h in range(H):
            got = prof.head_errors[h][i]["mse"][0]
            want = float(nmse[h])
            print(f"cand {i} {c['mode']} head {h}: kernel {got:.5f} oracle {want:.5f}", flush=True)
            assert abs(got - want) <= 1e-3 + 0.05 * want, (i, h)
            checked += 1
    assert checked == H * len(prof.cfgs)
