"""GPU parity of the token top-k from feature scores (saf3r_frame_topk_scores and the host mirror of
saf3r/patch/utils.py:54-184) against the oracle: bit-exact indices from identical bf16 scores."""
import importlib

import numpy as np
import pytest
import torch

from oracle import selection as OS

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def mods(pkg):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return tuple(importlib.import_module(pkg.__name__ + m) for m in (".ops", ".patch.utils", ".patch"))


def _bits(x: torch.Tensor) -> np.ndarray:
    return x.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


CASES = [  # frames, per_frame, topk, per_frame_mode, exclude_first, first_stride, cap
    (4, 1369, 4, True, False, 1, 0),
    (6, 37, 5, True, True, 4, 0),
    (5, 100, 64, True, False, 1, 150),
    (3, 1296, 16, True, True, 1, 1000),
    (2, 4096, 7, True, False, 1, 0),
    (4, 70, 50, False, False, 1, 0),
    (3, 200, 90, False, True, 8, 40),
    (1, 9, 20, True, False, 1, 0),
    (3, 1369, 64, True, False, 1, 0),
    (2, 1369, 100, True, True, 2, 0),
]


@pytest.mark.parametrize("F,P,k,pf,ex,st,cap", CASES)
def test_frame_topk_scores_bit_exact(mods, F, P, k, pf, ex, st, cap):
    ops = mods[0]
    g = torch.Generator().manual_seed(F * P + k)
    rows = 37
    # integer-valued scores: many ties, decided by the lower key
    x = torch.randint(-6, 7, (rows, F * P), generator=g).to(torch.bfloat16)
    x[:, ::11] = -0.0
    xd = torch.full((rows, -(-F * P // 8) * 8 + 8), 7.0, dtype=torch.bfloat16, device=DEV)  # padded row stride
    xd[:, :F * P] = x.to(DEV)
    got = ops.frame_topk_scores(xd[:, :F * P], F, P, k, per_frame_mode=pf, exclude_first=ex, first_stride=st,
                                cap=cap)
    torch.cuda.synchronize()
    want = OS.token_topk_from_scores(_bits(x), F, P, k, per_frame_mode=pf, exclude_first=ex, first_stride=st,
                                     cap=cap)
    assert got.shape == want.shape
    assert np.array_equal(got.cpu().numpy(), want)


@pytest.mark.parametrize("per_frame,include_first,max_topk", [(True, False, 2048), (True, True, 100),
                                                              (False, False, 2048), (True, False, 40)])
def test_compute_qk_topk_indices_batched(mods, per_frame, include_first, max_topk):
    """The host mirror on L2-normalised features (D = 1024): every block's indices equal the oracle's
    selection from the same block's bf16 scores."""
    ops, U, _ = mods
    S, P, D = 5, 121, 1024
    g = torch.Generator().manual_seed(int(per_frame) + 2 * int(include_first) + max_topk)
    feat = torch.nn.functional.normalize(torch.randn(1, S * P, D, generator=g), dim=-1).to(DEV)
    idx = U.compute_qk_topk_indices_batched(feat, feat, topk=8, per_frame=per_frame, num_toks_per_img=P,
                                            q_blocksize=256, max_topk=max_topk, include_first_frame=include_first,
                                            first_frame_stride=4)
    torch.cuda.synchronize()
    first, rest_eff, rest_final = U.output_width(S * P, 8, per_frame, P, max_topk, include_first, 4)
    assert idx.shape == (1, S * P, first + rest_final)
    q = feat.to(torch.bfloat16)[0]
    kt = torch.zeros(D, -(-S * P // 8) * 8, dtype=torch.bfloat16, device=DEV)
    kt[:, :S * P] = feat.to(torch.bfloat16)[0].t()
    Pm = P if (per_frame or include_first) else S * P
    for qs in range(0, S * P, 256):
        scores = torch.matmul(q[qs:qs + 256], kt)[:, :S * P]
        want = OS.token_topk_from_scores(_bits(scores), (S * P) // Pm, Pm, 8, per_frame_mode=per_frame,
                                         exclude_first=include_first, first_stride=4,
                                         cap=rest_final if rest_final < rest_eff else 0)
        assert np.array_equal(idx[0, qs:qs + 256].cpu().numpy(), want), f"block {qs}"


def test_non_lazy_layer_uses_feature_indices(mods, pkg):
    """A layer with dino_topk heads fed by set_dino_topk_from_features matches the oracle layer."""
    _, U, plug = mods
    vggt = importlib.import_module(pkg.__name__ + ".vggt")
    synth = importlib.import_module(pkg.__name__ + ".synth")
    from tests.test_gpu_plugin import _check_layer, _make
    ph, pw, F_, H = 6, 7, 3, 4
    dim = 64 * H
    m = _make(vggt, 1, dim, H, seed=9).to(DEV).to(torch.bfloat16)
    cfg = {"patch_module": {"type": "headsparse", "topk_mode": "token", "lazy_dino_topk": False, "topk": 5,
                            "per_frame_topk": True, "max_topk": 2048, "include_first_frame": True,
                            "first_frame_stride": 3},
           "sparse_config": {"0": [{"mode": "dino_topk", "head_ids": [1, 2]}, {"mode": "global_to_frame", "head_ids": [3]}]}}
    plug.patch_model(m, "vggt", cfg)
    plug.update_args_per_forward(m, "vggt", ph * 14, pw * 14)
    geom = pkg.Geometry(F_, ph * pw + 5, 5)
    g = torch.Generator().manual_seed(10)
    tokens = torch.randn(F_, ph * pw, 1024, generator=g).to(DEV)
    pv = importlib.import_module(pkg.__name__ + ".patch.patch_vggt")
    idx = pv.set_dino_topk_from_features(m, tokens, cfg)
    assert idx.shape == (F_ * ph * pw, 14 + 2 * 5)
    x = torch.randn(1, geom.tokens, dim, generator=g).to(torch.bfloat16).to(DEV)
    pos = synth.vggt_positions(F_, ph, pw).to(DEV)[None]
    with torch.no_grad():
        _check_layer(m.aggregator.global_blocks[0].attn, x, pos, geom, importlib.import_module(pkg.__name__ + ".ops"), 0)
