"""GPU parity of the key-set path of the `stride` and `q_probe_topk` modes
(saf3r/patch/sparse_attention.py:143-186, 256-273) against the oracle on the same inputs.

Bars: mean query, probe scores, key-set members and the gathered K rows are bit-exact; attention
over the key sets is within max-abs 2e-2 / mean-abs 2e-3 of the fp64 oracle."""
import importlib

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import selection as OS
from tests.layout_ref import slot_tokens, unpack_rows, unpack_v

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
ATOL_MAX, ATOL_MEAN = 2e-2, 2e-3


@pytest.fixture(scope="module")
def ops(pkg):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return importlib.import_module(pkg.__name__ + ".ops")


def _qkv(H, N, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(H, N, 64, generator=g) * scale).to(torch.bfloat16) for _ in range(3)]


def _bits(x: torch.Tensor) -> np.ndarray:
    return x.contiguous().view(torch.int16).numpy().view(np.uint16)


def _qk32(H, N, seed, scale=2.0):
    """fp32 q / k rows [H, 2, N, 64] in the layout pack_qkv writes for fp32 heads (not bf16-exact values)."""
    g = torch.Generator().manual_seed(seed)
    return torch.randn(H, 2, N, 64, generator=g) * scale + 0.3


@pytest.mark.parametrize("N", [3 * 155, 4 * 1374, 128, 70])
def test_probe_scores_bit_exact(ops, pkg, N):
    """The mean query and probe scores from fp32 q / k rows, both probe entries, against the oracle."""
    qk = _qk32(3, N, seed=N)
    qk_dev = qk.to(DEV).contiguous()
    slots = [2, 0]
    for noalloc in (False, True):
        qbar, scores = ops.probe_scores(qk_dev, slots, noalloc=noalloc)
        torch.cuda.synchronize()
        for i, h in enumerate(slots):
            want_q = OS.probe_mean(qk[h, 0].numpy())
            assert np.array_equal(qbar[i].cpu().numpy().view(np.uint32), want_q.view(np.uint32)), f"qbar slot {h}"
            want_s = OS.probe_scores(want_q, qk[h, 1].numpy())
            assert np.array_equal(scores[i].cpu().numpy().view(np.uint32), want_s.view(np.uint32)), f"scores {h}"


@pytest.mark.parametrize("N,ratio", [(3 * 155, 0.1), (4 * 1374, 0.3), (128, 0.5), (70, 0.001)])
def test_probe_scores_sampled_rows_bit_exact(ops, pkg, N, ratio):
    """q_sample_ratio < 1: the mean query over the reference's linspace rows (sparse_attention.py:154-157)."""
    qk = _qk32(2, N, seed=N + 1)
    rows = ops.probe_sample(N, ratio)
    assert rows is not None and len(rows) == max(1, int(N * ratio))
    qbar, scores = ops.probe_scores(qk.to(DEV).contiguous(), [1, 0], sample=rows)
    torch.cuda.synchronize()
    for i, h in enumerate([1, 0]):
        want_q = OS.probe_mean(qk[h, 0][rows].numpy())
        assert np.array_equal(qbar[i].cpu().numpy().view(np.uint32), want_q.view(np.uint32)), f"qbar slot {h}"
        want_s = OS.probe_scores(want_q, qk[h, 1].numpy())
        assert np.array_equal(scores[i].cpu().numpy().view(np.uint32), want_s.view(np.uint32)), f"scores slot {h}"
    # the sampled mean is the fp64 mean of those rows to fp32 accuracy, and not the all-row mean
    ref = qk[0, 0][rows].double().mean(0).float()
    assert torch.allclose(qbar[1].cpu(), ref, atol=1e-5)


def test_pack_writes_fp32_rows_of_flagged_heads(ops, pkg):
    """pack_qkv's fp32 rows (after LayerNorm / RoPE, before the bf16 rounding): token order, flagged heads
    in increasing head order, and they round to exactly the packed bf16 rows."""
    geom = pkg.Geometry(3, 5 + 6 * 7, 5)
    H, N = 4, geom.tokens
    C = 64 * H
    g = torch.Generator().manual_seed(31)
    qkv = torch.randn(N, 3 * C, generator=g).to(torch.bfloat16).to(DEV)
    ln = (torch.rand(64, generator=g) + 0.5, 0.1 * torch.randn(64, generator=g))
    pos = OA.vggt_positions(3, 6, 7)
    qp, kp, vp, qk32 = ops.pack_qkv(qkv, qkv[:, C:], qkv[:, 2 * C:], 3 * C, 64, geom, H, ln_q=ln, ln_k=ln,
                                    pos=pos.to(DEV), rope_base=100.0, fp32_heads=[False, True, False, True])
    torch.cuda.synchronize()
    toks = slot_tokens(geom.frames, geom.tokens_per_frame, geom.num_special)
    q, _ = unpack_rows(qp.cpu(), toks, N)
    k, _ = unpack_rows(kp.cpu(), toks, N)
    assert tuple(qk32.shape) == (2, 2, N, 64)
    qr, kr, _ = OA.qkv_prologue(qkv.cpu(), H, (ln[0], ln[1]), (ln[0], ln[1]), pos)
    for s, h in enumerate((1, 3)):
        assert torch.equal(qk32[s, 0].cpu().to(torch.bfloat16), q[h]) and torch.equal(qk32[s, 1].cpu().to(torch.bfloat16), k[h])
        # the fp32 values themselves: the oracle prologue's fp32 LayerNorm + RoPE within fp32 rounding
        ref_q = OA.rope2d(torch.nn.functional.layer_norm(qkv.cpu().float().reshape(N, 3, H, 64)[:, 0, h], (64,),
                                                         ln[0], ln[1], 1e-5), pos)
        assert torch.allclose(qk32[s, 0].cpu(), ref_q, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("F,T,ns", [(3, 155, 5), (4, 1374, 5), (2, 64, 0), (5, 37, 5), (200, 1374, 5)])
def test_keyset_build_bit_exact(ops, pkg, F, T, ns):
    """Key sets bit-exact against the oracle: stride sets (several starts and strides), top-k sets on
    normal and heavily tied scores, k above the token count; frames shorter than 64 tokens, and
    274,800 tokens (more than one 262,144-token segment of the build kernel)."""
    geom = pkg.Geometry(F, T, ns)
    n = geom.tokens
    rng = np.random.default_rng(n)
    specs = [ops.KeySetSpec(0, ops.KEYSET_STRIDE, 4, 0, True), ops.KeySetSpec(1, ops.KEYSET_TOPK, n // 4, 0, False),
             ops.KeySetSpec(2, ops.KEYSET_TOPK, 37, 0, True), ops.KeySetSpec(3, ops.KEYSET_STRIDE, 128, 3, False),
             ops.KeySetSpec(4, ops.KEYSET_TOPK, n + 5, 0, False), ops.KeySetSpec(5, ops.KEYSET_STRIDE, 7, 2, True)]
    scores = np.zeros((len(specs), n), np.float32)
    scores[1] = rng.standard_normal(n).astype(np.float32)
    scores[2] = rng.integers(-3, 4, n).astype(np.float32)  # ties decided by the lower token
    scores[2][::5] = -0.0
    scores[4] = rng.standard_normal(n).astype(np.float32)
    idx, count = ops.keyset_build(specs, geom, torch.from_numpy(scores).to(DEV), DEV)
    torch.cuda.synchronize()
    idx, count = idx.cpu().numpy(), count.cpu().numpy()
    for i, s in enumerate(specs):
        want = OS.keyset(scores[i], n, T, ns, s.mode, s.param, s.start, s.include)
        assert count[i] == len(want) <= s.bound(geom), f"spec {i}"
        assert np.array_equal(idx[i, :count[i]], want), f"spec {i}"


def test_keyset_gather_rows_and_tiles(ops, pkg):
    geom = pkg.Geometry(3, 155, 5)
    n, H = geom.tokens, 4
    q, k, v = _qkv(H, n, seed=5)
    qp, kp, vp = ops.pack_heads(q.to(DEV), k.to(DEV), v.to(DEV), geom)
    specs = [ops.KeySetSpec(3, ops.KEYSET_STRIDE, 3, 1, True), ops.KeySetSpec(1, ops.KEYSET_STRIDE, 50, 0, False)]
    idx, count = ops.keyset_build(specs, geom, None, DEV)
    vnat = v.permute(1, 0, 2).contiguous().to(DEV)  # [N, H, 64]: head stride 64, token stride H*64
    ks = ops.keyset_gather(kp, geom, specs, vnat, H * 64, 64, idx, count)
    torch.cuda.synchronize()
    kc, vc, cnt, ix = ks.k.cpu(), ks.v.cpu(), count.cpu(), idx.cpu()
    for i, s in enumerate(specs):
        c = int(cnt[i])
        keys = ix[i, :c].long()
        assert torch.equal(kc[i, :c], k[s.head][keys])
        tiles = -(-c // 64)
        assert (kc[i, c:tiles * 64] == 0).all()
        toks = torch.arange(tiles * 64)
        toks = torch.where(toks < c, toks, torch.full_like(toks, -1))
        nat, pad = unpack_v(vc[i:i + 1, :tiles], toks, c)
        assert torch.equal(nat[0], v[s.head][keys]) and (pad == 0).all()


@pytest.mark.parametrize("F,T,ns", [(3, 155, 5), (4, 1374, 5), (1, 70, 5), (2, 64, 0)])
def test_keyset_attention_in_one_launch(ops, pkg, F, T, ns):
    geom = pkg.Geometry(F, T, ns)
    n = geom.tokens
    patterns = [ops.KEYSET, ops.DENSE, ops.KEYSET, ops.FRAME_LOCAL, ops.KEYSET, ops.ANCHOR]
    H = len(patterns)
    q, k, v = _qkv(H, n, seed=F * 3 + T, scale=1.5)
    qp, kp, vp, qk32 = ops.pack_heads(q.to(DEV), k.to(DEV), v.to(DEV), geom, fp32_heads=[h == 2 for h in range(H)])
    specs = [ops.KeySetSpec(0, ops.KEYSET_STRIDE, 4, 0, True), ops.KeySetSpec(2, ops.KEYSET_TOPK, max(1, n // 4)),
             ops.KeySetSpec(4, ops.KEYSET_STRIDE, 128, 0, True)]
    _, sc = ops.probe_scores(qk32, [0])
    scores = torch.zeros(3, n, device=DEV)
    scores[1] = sc[0]
    idx, count = ops.keyset_build(specs, geom, scores, DEV)
    vnat = v.permute(1, 0, 2).contiguous().to(DEV)
    ks = ops.keyset_gather(kp, geom, specs, vnat, H * 64, 64, idx, count)
    out = ops.sparse_attn_fwd(qp, kp, vp, geom, patterns, keysets=ks)
    torch.cuda.synchronize()
    og = OA.Geometry(F, T, ns)
    got = out.float().cpu().reshape(n, H, 64).permute(1, 0, 2)
    ks_of = {s.head: idx[i, :int(count[i])].cpu() for i, s in enumerate(specs)}
    for h, pat in enumerate(patterns):
        ref = OA.sparse_attention_gathered(q[h].float(), k[h].float(), v[h].float(), pat, og, ks_of.get(h),
                                           dtype=torch.float64)
        err = (got[h] - ref.float()).abs()
        print(f"F{F} T{T} head {h} pattern {pat}: max {err.max().item():.3g} mean {err.mean().item():.3g}", flush=True)
        assert err.max().item() <= ATOL_MAX and err.mean().item() <= ATOL_MEAN


@pytest.mark.parametrize("F,T,ns", [(3, 155, 5), (4, 1374, 5), (2, 64, 0), (1, 70, 5), (5, 37, 5)])
def test_broadcast_first_in_one_launch(ops, pkg, F, T, ns):
    """broadcast_first heads (saf3r/patch/sparse_attention.py:110-131) next to other patterns: the
    gathered frame-0 rows and V tiles are exact copies, the outputs within the attention bars."""
    geom = pkg.Geometry(F, T, ns)
    n = geom.tokens
    patterns = [ops.BROADCAST, ops.DENSE, ops.KEYSET, ops.BROADCAST, ops.FRAME_LOCAL]
    H = len(patterns)
    q, k, v = _qkv(H, n, seed=F * 5 + T, scale=1.5)
    qp, kp, vp = ops.pack_heads(q.to(DEV), k.to(DEV), v.to(DEV), geom)
    specs = [ops.KeySetSpec(2, ops.KEYSET_STRIDE, 3, 1, True)]
    idx, count = ops.keyset_build(specs, geom, None, DEV)
    vnat = v.permute(1, 0, 2).contiguous().to(DEV)
    ks = ops.keyset_gather(kp, geom, specs, vnat, H * 64, 64, idx, count)
    bc = ops.broadcast_gather(qp, kp, geom, [0, 3], vnat, H * 64, 64)
    out = ops.sparse_attn_fwd(qp, kp, vp, geom, patterns, keysets=ks, broadcast=bc)
    torch.cuda.synchronize()
    C = -(-T // 64) * 64
    for b, h in enumerate((0, 3)):
        for buf, src in ((bc.q, q), (bc.k, k)):
            rows = buf[b].cpu()
            assert torch.equal(rows[:T], src[h][:T]) and (rows[T:C] == 0).all(), f"head {h} frame-0 rows"
        toks = torch.arange(C)
        toks = torch.where(toks < T, toks, torch.full_like(toks, -1))
        for f in (0, F - 1):
            nat, pad = unpack_v(bc.v[b, f:f + 1].cpu(), toks, T)
            assert torch.equal(nat[0], v[h][f * T:(f + 1) * T]) and (pad == 0).all(), f"head {h} frame {f} V"
    og = OA.Geometry(F, T, ns)
    got = out.float().cpu().reshape(n, H, 64).permute(1, 0, 2)
    ks_of = {2: idx[0, :int(count[0])].cpu()}
    for h, pat in enumerate(patterns):
        ref = OA.sparse_attention_gathered(q[h].float(), k[h].float(), v[h].float(), pat, og, ks_of.get(h),
                                           dtype=torch.float64)
        err = (got[h] - ref.float()).abs()
        print(f"F{F} T{T} head {h} pattern {pat}: max {err.max().item():.3g} mean {err.mean().item():.3g}", flush=True)
        assert err.max().item() <= ATOL_MAX and err.mean().item() <= ATOL_MEAN



@pytest.mark.parametrize("phase", ["fixed", "paced"])
def test_keyset_broadcast_prescaled_out_of_range(ops, pkg, phase):
    """KEYSET, BROADCAST and TOKEN_DYNAMIC_KEYSET heads with the softmax scale packed into Q, whose
    scores leave the range of the walk without a running maximum: outlier keys 69 and 173 log2 units
    above the rest in frame 0 (heads 0-2: a partial row sum beyond 2^64), and every score about 72 units
    below 0 (heads 3-5: row sums below 2^-64). The fixup launch must find the marked items of these
    walks too; every written row matches the oracle in both walk orders."""
    geom = pkg.Geometry(3, 155, 5)
    P = ops
    patterns = [P.KEYSET, P.BROADCAST, P.TOKEN_DYNAMIC_KEYSET, P.KEYSET, P.BROADCAST, P.TOKEN_DYNAMIC_KEYSET]
    H, N, T = len(patterns), geom.tokens, geom.tokens_per_frame
    g = torch.Generator().manual_seed(16)
    q = (0.5 + 0.1 * torch.randn(H, N, 64, generator=g)).to(torch.bfloat16)
    k = (0.3 * torch.randn(H, N, 64, generator=g)).to(torch.bfloat16)
    v = torch.randn(H, N, 64, generator=g).to(torch.bfloat16)
    k[:3, 40] = 12.0   # frame-0 tokens 40 and 100: members of every key set below (stride 4 from 0, or frame 0)
    k[:3, 100] = 30.0
    q[3:] = (2.5 + 0.05 * torch.randn(3, N, 64, generator=g)).to(torch.bfloat16)
    k[3:] = (-2.5 + 0.05 * torch.randn(3, N, 64, generator=g)).to(torch.bfloat16)
    flags = [True] * H
    qp, kp, vp = ops.pack_heads(q.to(DEV), k.to(DEV), v.to(DEV), geom, q_scaled=flags)
    specs = [ops.KeySetSpec(0, ops.KEYSET_STRIDE, 3, 1, True), ops.KeySetSpec(2, ops.KEYSET_STRIDE, 4, 0, False),
             ops.KeySetSpec(3, ops.KEYSET_STRIDE, 3, 1, True), ops.KeySetSpec(5, ops.KEYSET_STRIDE, 4, 0, False)]
    idx, count = ops.keyset_build(specs, geom, None, DEV)
    vnat = v.permute(1, 0, 2).contiguous().to(DEV)
    ks = ops.keyset_gather(kp, geom, specs, vnat, H * 64, 64, idx, count)
    bc = ops.broadcast_gather(qp, kp, geom, [1, 4], vnat, H * 64, 64)
    out = torch.zeros(N, H * 64, dtype=torch.bfloat16, device=DEV)
    for _ in range(2 if phase == "paced" else 1):  # paced: the second call paces by measured step times
        ops.sparse_attn_fwd(qp, kp, vp, geom, patterns, keysets=ks, broadcast=bc, out=out, q_scaled=flags,
                            order=phase)
    torch.cuda.synchronize()
    c = ops.prescale_factor()
    q_used = (q.float() * c).to(torch.bfloat16).float() / c  # the packed Q in unscaled units
    og = OA.Geometry(3, 155, 5)
    got = out.float().cpu().reshape(N, H, 64).permute(1, 0, 2)
    assert torch.isfinite(got).all()
    ks_of = {s.head: idx[i, :int(count[i])].cpu() for i, s in enumerate(specs)}
    assert all(40 in ks_of[h].tolist() and 100 in ks_of[h].tolist() for h in (0, 2))
    special = torch.tensor([f * T + s for f in range(3) for s in range(5)])
    for h, pat in enumerate(patterns):
        ref_pat = P.KEYSET if pat == P.TOKEN_DYNAMIC_KEYSET else pat
        ref = OA.sparse_attention_gathered(q_used[h], k[h].float(), v[h].float(), ref_pat, og, ks_of.get(h),
                                           dtype=torch.float64)
        rows = special if pat == P.TOKEN_DYNAMIC_KEYSET else torch.arange(N)  # its patch rows are the gather's
        e = (got[h][rows] - ref[rows].float()).abs()
        print(f"{phase} head {h} pattern {pat}: max {e.max().item():.3g} mean {e.mean().item():.3g}", flush=True)
        assert e.max().item() <= ATOL_MAX and e.mean().item() <= ATOL_MEAN
