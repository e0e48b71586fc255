"""GPU parity of every kernel against the CPU oracle on the same seeded inputs.

Bars: packing without LayerNorm/RoPE, pooling, top-k and block selection are bit-exact; attention
outputs are within max-abs 2e-2 and mean-abs 2e-3 (bf16 kernel vs fp32/fp64 oracle on identical
bf16 inputs and identical index lists); LayerNorm+RoPE packing is within 1 bf16 ulp-scale error.
"""
import importlib

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import selection as OS
from tests.layout_ref import framed_slot_tokens, slot_tokens, unpack_rows, unpack_v

pytestmark = pytest.mark.gpu
ATOL_MAX, ATOL_MEAN = 2e-2, 2e-3


@pytest.fixture(scope="module")
def ops(pkg):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return importlib.import_module(pkg.__name__ + ".ops")


DEV = "cuda:0"
GEOMS = [(3, 155, 5), (4, 1374, 5), (2, 64, 0), (1, 70, 5), (14, 60, 5), (3, 65, 1)]


def _qkv(H, N, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(H, N, 64, generator=g) * scale).to(torch.bfloat16) for _ in range(3)]


def _check_close(got, ref, what):
    err = (got.float() - ref.float()).abs()
    print(f"{what}: max {err.max().item():.3g} mean {err.mean().item():.3g}", flush=True)
    assert err.max().item() <= ATOL_MAX, f"{what}: max abs {err.max().item()}"
    assert err.mean().item() <= ATOL_MEAN, f"{what}: mean abs {err.mean().item()}"


@pytest.mark.parametrize("F,T,ns", GEOMS)
def test_pack_layout_bit_exact(ops, pkg, F, T, ns):
    geom = pkg.Geometry(F, T, ns)
    H = 3
    q, k, v = _qkv(H, geom.tokens, seed=F * 7 + T)
    qp, kp, vp = ops.pack_heads(q.to(DEV), k.to(DEV), v.to(DEV), geom)
    torch.cuda.synchronize()
    toks = slot_tokens(F, T, ns)
    for src, pk in ((q, qp), (k, kp)):
        nat, pad = unpack_rows(pk.cpu(), toks, geom.tokens)
        assert torch.equal(nat, src) and (pad == 0).all()
    nat, pad = unpack_v(vp.cpu(), toks, geom.tokens)
    assert torch.equal(nat, v) and (pad == 0).all()


@pytest.mark.parametrize("F,T,ns", GEOMS)
def test_pack_token_order_bit_exact(ops, pkg, F, T, ns):
    """Flagged heads: slot t holds token t, zeros past F*T; the others keep the padded layout."""
    geom = pkg.Geometry(F, T, ns)
    H = 3
    q, k, v = _qkv(H, geom.tokens, seed=F * 5 + T)
    flags = [True, False, True]
    qp, kp, vp = ops.pack_heads(q.to(DEV), k.to(DEV), v.to(DEV), geom, token_order=flags)
    torch.cuda.synchronize()
    padded = slot_tokens(F, T, ns)
    tokord = torch.tensor([t if t < geom.tokens else -1 for t in range(geom.slots)])
    for h, fl in enumerate(flags):
        toks = tokord if fl else padded
        for src, pk in ((q, qp), (k, kp)):
            nat, pad = unpack_rows(pk[h:h + 1].cpu(), toks, geom.tokens)
            assert torch.equal(nat[0], src[h]) and (pad == 0).all()
        nat, pad = unpack_v(vp[h:h + 1].cpu(), toks, geom.tokens)
        assert torch.equal(nat[0], v[h]) and (pad == 0).all()


@pytest.mark.parametrize("F,T,ns", GEOMS)
def test_pack_framed_bit_exact(ops, pkg, F, T, ns):
    """Framed heads: frame f's tokens in order from tile f*ceil(T/64), zeros elsewhere; the other heads
    keep their layouts. Where the framed layout does not fit the head, packing it is refused."""
    geom = pkg.Geometry(F, T, ns)
    H = 3
    q, k, v = _qkv(H, geom.tokens, seed=F * 7 + T)
    lay = [ops.LAYOUT_FRAMED, ops.LAYOUT_PACKED, ops.LAYOUT_TOKEN]
    if not geom.framed_fits:
        with pytest.raises(RuntimeError, match="framed layout"):
            ops.pack_heads(q.to(DEV), k.to(DEV), v.to(DEV), geom, token_order=lay)
        return
    qp, kp, vp = ops.pack_heads(q.to(DEV), k.to(DEV), v.to(DEV), geom, token_order=lay)
    torch.cuda.synchronize()
    tokord = torch.tensor([t if t < geom.tokens else -1 for t in range(geom.slots)])
    for h, toks in enumerate((framed_slot_tokens(F, T, ns), slot_tokens(F, T, ns), tokord)):
        for src, pk in ((q, qp), (k, kp)):
            nat, pad = unpack_rows(pk[h:h + 1].cpu(), toks, geom.tokens)
            assert torch.equal(nat[0], src[h]) and (pad == 0).all()
        nat, pad = unpack_v(vp[h:h + 1].cpu(), toks, geom.tokens)
        assert torch.equal(nat[0], v[h]) and (pad == 0).all()


def test_pack_layernorm_rope(ops, pkg):
    geom = pkg.Geometry(3, 5 + 7 * 9, 5)
    H, N = 4, geom.tokens
    g = torch.Generator().manual_seed(11)
    qkv = (torch.randn(N, 3 * H * 64, generator=g) * 2 + 0.5).to(torch.bfloat16)
    lnq = (torch.rand(64, generator=g) + 0.5, torch.randn(64, generator=g) * 0.1)
    lnk = (torch.rand(64, generator=g) + 0.5, torch.randn(64, generator=g) * 0.1)
    pos = OA.vggt_positions(geom.frames, 7, 9)
    d = qkv.to(DEV)
    C = H * 64
    qp, kp, vp = ops.pack_qkv(d, d[:, C:], d[:, 2 * C:], 3 * C, 64, geom, H,
                              ln_q=[t.to(DEV) for t in lnq], ln_k=[t.to(DEV) for t in lnk], ln_eps=1e-5,
                              pos=pos.to(DEV), rope_base=100.0)
    torch.cuda.synchronize()
    qr, kr, vr = OA.qkv_prologue(qkv, H, lnq, lnk, pos)
    toks = slot_tokens(geom.frames, geom.tokens_per_frame, 5)
    qn, _ = unpack_rows(qp.cpu(), toks, N)
    kn, _ = unpack_rows(kp.cpu(), toks, N)
    vn, _ = unpack_v(vp.cpu(), toks, N)
    assert torch.equal(vn, vr)
    for got, ref, nm in ((qn, qr, "q"), (kn, kr, "k")):
        err = (got.float() - ref.float()).abs()
        tol = ref.float().abs() * 2 ** -7 + 1e-3  # one bf16 ulp of rounding-point difference
        assert (err <= tol).all(), f"{nm}: worst {err.max()}"


@pytest.mark.parametrize("F,T,ns", GEOMS)
def test_block_pool_bit_exact(ops, pkg, F, T, ns):
    geom = pkg.Geometry(F, T, ns)
    H = 3
    q, k, v = _qkv(H, geom.tokens, seed=5 + F)
    qp, kp, _ = ops.pack_heads(q.to(DEV), k.to(DEV), v.to(DEV), geom)
    pq, pk = ops.block_pool(qp, kp, geom, [2, 0])
    torch.cuda.synchronize()
    for slot, h in enumerate([2, 0]):
        for src, got in ((q, pq), (k, pk)):
            ref = OS.block_pool(OS.bf16_bits(src[h].float().numpy()), F, T, ns)
            assert np.array_equal(got[slot].cpu().numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("frames,C,k", [(4, 22, 4), (128, 22, 4), (3, 7, 8), (2, 1369, 4), (5, 9, 32), (1, 33, 16)])
def test_topk_from_scores_bit_exact(ops, frames, C, k):
    rng = np.random.default_rng(frames * 31 + C)
    s = rng.integers(-4, 5, size=(2, 37, frames * C)).astype(np.float32)  # ties everywhere
    s[0, 0, :4] = [-0.0, 0.0, np.inf, -np.inf]
    s[1, 3] = rng.standard_normal(frames * C).astype(np.float32)
    got = ops.topk_from_scores(torch.from_numpy(s).to(DEV), frames, k).cpu().numpy()
    for b in range(2):
        assert np.array_equal(got[b], OS.frame_topk(s[b], frames, k))


@pytest.mark.parametrize("frames,nbf,k,scope", [(4, 22, 4, "frame"), (32, 22, 4, "frame"), (6, 21, 8, "frame"),
                                                 (3, 5, 8, "frame"), (4, 22, 4, "global"), (7, 3, 16, "global")])
def test_block_select_bit_exact(ops, frames, nbf, k, scope):
    rng = np.random.default_rng(frames + nbf + k)
    pq = rng.standard_normal((2, frames * nbf, 64)).astype(np.float32)
    pk = rng.standard_normal((2, frames * nbf, 64)).astype(np.float32)
    pk[1, 3] = pk[1, 5]  # exact duplicate candidates: tie -> lower block id
    got = ops.block_select(torch.from_numpy(pq).to(DEV), torch.from_numpy(pk).to(DEV), frames, nbf, k, scope)
    got = got.cpu().numpy()
    for h in range(2):
        s = OS.block_scores(pq[h], pk[h])
        ref = OS.frame_topk(s, frames, k) if scope == "frame" else OS.global_topk(s, k)
        assert np.array_equal(got[h], ref)


def _pooled_case(case, n, rows, rng):
    x = rng.standard_normal((n, rows, 64)).astype(np.float32) * np.float32(0.2)
    if case == "zeros":  # every score 0: no order is certain, every pair takes the sequential path
        x[:] = 0
    elif case == "wide":  # magnitudes 1e-30 .. 1e30 across rows and features
        x *= (10.0 ** rng.uniform(-30, 30, size=(n, rows, 64))).astype(np.float32)
    elif case == "tiny":  # values at and below the fp32 / bf16 normal range
        x *= np.float32(1e-37)
        x[:, ::3] *= np.float32(1e-3)
    elif case == "nonfinite":
        x.reshape(-1)[rng.integers(0, x.size, 40)] = np.inf
        x.reshape(-1)[rng.integers(0, x.size, 40)] = -np.inf
        x.reshape(-1)[rng.integers(0, x.size, 40)] = np.nan
    return x


_ADV_CASES = ["normal", "ties", "zeros", "wide", "tiny", "nonfinite"]


@pytest.mark.parametrize("frames,nbf,k,case",
                         [(f, b, kk, c) for (f, b, kk) in [(4, 22, 4), (5, 32, 8), (3, 1, 1), (6, 21, 3), (2, 7, 8),
                                                          (9, 17, 2)] for c in _ADV_CASES]
                         + [(128, 22, 4, "normal")])
def test_block_select_adversarial_bit_exact(ops, frames, nbf, k, case):
    """Block selection against the oracle on pooled inputs that stress the order: exact ties (equal
    candidates, equal query blocks, 1-ulp neighbours), all-zero scores, 60 decades of magnitude,
    values below the normal range, infinities and NaNs."""
    rng = np.random.default_rng(frames * 7 + nbf * 3 + k + len(case))
    n, nb = 2, frames * nbf
    pq = _pooled_case(case, n, nb, rng)
    pk = _pooled_case(case, n, nb, rng)
    if case == "ties":
        pk[:, 1::nbf] = pk[:, 0::nbf][:, :pk[:, 1::nbf].shape[1]]
        pq[:, 1::2] = pq[:, 0::2][:, :pq[:, 1::2].shape[1]]
        if nbf > 3:
            pk[0, 2::nbf] = np.nextafter(pk[0, 3::nbf], np.float32(np.inf))
    got = ops.block_select(torch.from_numpy(pq).to(DEV), torch.from_numpy(pk).to(DEV), frames, nbf, k).cpu().numpy()
    for h in range(n):
        ref = OS.frame_topk(OS.block_scores(pq[h], pk[h]), frames, k)
        assert np.array_equal(got[h], ref), f"{case}: head {h} differs from the oracle"


@pytest.mark.parametrize("frames,nbf,k,case",
                         [(f, b, kk, c) for (f, b, kk) in [(4, 22, 4), (5, 32, 8), (3, 1, 1), (6, 21, 3), (2, 7, 8),
                                                          (9, 17, 2)] for c in _ADV_CASES]
                         + [(128, 22, 4, "normal"), (3, 5, 8, "ties"), (5, 4, 4, "normal"), (3, 3, 8, "ties"),
                            (2, 32, 16, "normal"), (2, 9, 1, "ties"), (3, 22, 20, "normal")])
def test_block_select_pooled_adversarial_bit_exact(ops, frames, nbf, k, case):
    """The matrix-core block selection (split records, certified order, exact pass for the rest)
    against the oracle's sequential scores on the adversarial pooled inputs, including k = NBf
    (whole frames), k + 1 > NBf, 32 blocks per frame and k > 16 (the sequential kernel)."""
    rng = np.random.default_rng(frames * 11 + nbf * 5 + k + len(case))
    n, nb = 2, frames * nbf
    pq = _pooled_case(case, n, nb, rng)
    pk = _pooled_case(case, n, nb, rng)
    if case == "ties":
        pk[:, 1::nbf] = pk[:, 0::nbf][:, :pk[:, 1::nbf].shape[1]]
        pq[:, 1::2] = pq[:, 0::2][:, :pq[:, 1::2].shape[1]]
        if nbf > 3:
            pk[0, 2::nbf] = np.nextafter(pk[0, 3::nbf], np.float32(np.inf))
    mean = torch.from_numpy(np.stack([pq, pk], axis=1)).to(DEV)  # [n, 2, NB, 64]
    pooled = ops.pooled_prepare(mean)
    got = ops.block_select_pooled(pooled, frames, nbf, k).cpu().numpy()
    for h in range(n):
        ref = OS.frame_topk(OS.block_scores(pq[h], pk[h]), frames, k)
        assert np.array_equal(got[h], ref), f"{case}: head {h} differs from the oracle"


@pytest.mark.parametrize("frames,nbf,k", [(24, 22, 4), (12, 21, 8), (9, 32, 4), (16, 6, 2)])
def test_block_select_pooled_many_listed_pairs(ops, frames, nbf, k):
    """Pooled means in {-1/4, 0, 1/4}: exact score ties everywhere, so about 4 in 5 (query block,
    frame) pairs are listed and a work-group's exact pass holds more candidates than its LDS space
    (several batches); bit-identical to the oracle's sequential selection."""
    rng = np.random.default_rng(frames * 13 + nbf + k)
    n, nb = 2, frames * nbf
    mean = (rng.integers(-1, 2, size=(n, 2, nb, 64)).astype(np.float32) * np.float32(0.25))
    pooled = ops.pooled_prepare(torch.from_numpy(mean).to(DEV))
    got = ops.block_select_pooled(pooled, frames, nbf, k).cpu().numpy()
    for h in range(n):
        ref = OS.frame_topk(OS.block_scores(mean[h, 0], mean[h, 1]), frames, k)
        assert np.array_equal(got[h], ref), f"head {h}"


def test_block_select_pooled_128_frames(ops):
    """128 frames x 22 blocks of N(0, 1/64)-like pooled means (the benchmark's scale), 3 heads: the
    matrix-core selection is bit-identical to the oracle's sequential selection."""
    rng = np.random.default_rng(77)
    frames, nbf, n = 128, 22, 3
    base = rng.standard_normal((n, 1, 64)).astype(np.float32) * np.float32(0.3)  # a shared component
    mean = (base[:, None] + rng.standard_normal((n, 2, frames * nbf, 64)).astype(np.float32) * np.float32(0.12))
    pooled = ops.pooled_prepare(torch.from_numpy(mean).to(DEV))
    got = ops.block_select_pooled(pooled, frames, nbf, 4).cpu().numpy()
    for h in range(n):
        ref = OS.frame_topk(OS.block_scores(mean[h, 0], mean[h, 1]), frames, 4)
        assert np.array_equal(got[h], ref), f"head {h}"


def test_block_select_pooled_unaligned_output(ops, pkg):
    """The C entry takes any 4-byte aligned int32 output: lists written at an address 4 bytes past a
    16-byte boundary (per-element stores in place of 16-byte ones) equal those of an aligned buffer,
    and the words on either side stay untouched."""
    from importlib import import_module
    lib = import_module(pkg.__name__ + "._lib")
    rng = np.random.default_rng(5)
    frames, nbf, n, k = 12, 22, 2, 4
    mean = rng.standard_normal((n, 2, frames * nbf, 64)).astype(np.float32) * np.float32(0.125)
    pooled = ops.pooled_prepare(torch.from_numpy(mean).to(DEV))
    want = ops.block_select_pooled(pooled, frames, nbf, k)
    buf = torch.full((want.numel() + 8,), -7, dtype=torch.int32, device=DEV)
    assert buf.data_ptr() % 16 == 0
    L = lib.load()
    rc = L.saf3r_block_select_pooled(pooled.mean.data_ptr(), pooled.split.data_ptr(), pooled.meta.data_ptr(), n,
                                     frames, nbf, k, buf.data_ptr() + 4, None, 0, lib.stream_ptr())
    assert rc == 0, lib.load().saf3r_last_error()
    got = buf.cpu()
    assert torch.equal(got[1:1 + want.numel()], want.flatten().cpu())
    assert int(got[0]) == -7 and bool((got[1 + want.numel():] == -7).all())


def test_pooled_prepare_split_is_exact(ops):
    """The split record: x * 2^s == h1 + h2 + r with |r| <= 2^-22 |x 2^s| (fp16 normal range), the row's
    largest magnitude times 2^s in [2^14, 2^15), meta = (a norm bound >= the norm, 2^-s); rows outside
    the covered range (non-finite, largest magnitude beyond [2^-50, 2^50]) carry +inf."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((1, 2, 6, 64)).astype(np.float32)
    x[0, 0, 1] *= np.float32(1e-6)
    x[0, 0, 2] = 0
    x[0, 0, 3, 5] = np.inf
    x[0, 1, 0] *= np.float32(1e20)  # largest magnitude above 2^50
    x[0, 1, 1] *= np.float32(1e-20)  # below 2^-50
    pooled = ops.pooled_prepare(torch.from_numpy(x).to(DEV))
    split = pooled.split.cpu().numpy().view(np.float16).astype(np.float64)
    meta = pooled.meta.cpu().numpy()
    for t in range(2):
        for r in range(6):
            row = x[0, t, r].astype(np.float64)
            norm, inv = meta[0, t, r]
            finite = np.isfinite(row).all()
            mx = np.abs(row).max() if finite else np.inf
            safe = finite and (mx == 0 or 2.0 ** -50 <= mx <= 2.0 ** 50)
            if not safe:
                assert norm == np.inf, (t, r)
                continue
            assert norm >= np.sqrt((row ** 2).sum())
            if mx == 0:
                assert inv == 1 and (split[0, t, r] == 0).all()
                continue
            xs = row / inv
            assert 2.0 ** 14 <= np.abs(xs).max() < 2.0 ** 15
            h1, h2 = split[0, t, r, 0], split[0, t, r, 1]
            assert np.array_equal(h1, xs.astype(np.float16).astype(np.float64))
            resid = xs - h1 - h2
            ok = np.abs(resid) <= 2.0 ** -22 * np.abs(xs) + 2.0 ** -25  # fp16 subnormal spacing / 2
            assert ok.all(), (t, r, resid[~ok])


def test_pack_pools_unscaled_rows_bit_exact(ops, pkg):
    """Pooled records from the pack: the block means of bf16(q) (without the Q scale) and bf16(k) equal
    the oracle's pooling of those rows bit for bit, the split records equal saf3r_pooled_prepare's of
    the same means, and the selection from them equals the oracle's."""
    geom = pkg.Geometry(3, 155, 5)
    H = 4
    q, k, v = _qkv(H, geom.tokens, seed=12, scale=1.3)
    qs = [True, False, True, True]
    qp, kp, vp, pooled = ops.pack_heads(q.to(DEV), k.to(DEV), v.to(DEV), geom, q_scaled=qs, pool_heads=[3, 1])
    torch.cuda.synchronize()
    for slot, h in enumerate([1, 3]):
        for t, src in enumerate((q, k)):
            ref = OS.block_pool(OS.bf16_bits(src[h].float().numpy()), geom.frames, geom.tokens_per_frame, 5)
            assert np.array_equal(pooled.mean[slot, t].cpu().numpy().view(np.uint32), ref.view(np.uint32)), (h, t)
    again = ops.pooled_prepare(pooled.mean.clone())
    assert torch.equal(again.split, pooled.split) and torch.equal(again.meta, pooled.meta)
    sel = ops.block_select_pooled(pooled, geom.frames, geom.blocks_per_frame, 2).cpu().numpy()
    for slot, h in enumerate([1, 3]):
        ref = OS.block_select(OS.bf16_bits(q[h].float().numpy()), OS.bf16_bits(k[h].float().numpy()),
                              geom.frames, geom.tokens_per_frame, 5, 2)
        assert np.array_equal(sel[slot], ref)


def _run_layer(ops, pkg, geom, q, k, v, patterns, k_sel=2):
    qp, kp, vp = ops.pack_heads(q.to(DEV), k.to(DEV), v.to(DEV), geom)
    dyn = [h for h, p in enumerate(patterns) if p == ops.BLOCK_DYNAMIC]
    sel = None
    if dyn:
        pq, pk = ops.block_pool(qp, kp, geom, dyn)
        sel = ops.block_select(pq, pk, geom.frames, geom.blocks_per_frame, k_sel)
    out = ops.sparse_attn_fwd(qp, kp, vp, geom, patterns, sel)
    torch.cuda.synchronize()
    return out, sel, dyn


@pytest.mark.parametrize("F,T,ns", GEOMS)
def test_sparse_attention_all_patterns(ops, pkg, F, T, ns):
    geom = pkg.Geometry(F, T, ns)
    patterns = [ops.DENSE, ops.FRAME_LOCAL, ops.ANCHOR_LOCAL, ops.BLOCK_DYNAMIC, ops.ANCHOR, ops.SKIP,
                ops.BLOCK_DYNAMIC, ops.FRAME_LOCAL]
    H = len(patterns)
    q, k, v = _qkv(H, geom.tokens, seed=F * 13 + T, scale=1.5)
    out, sel, dyn = _run_layer(ops, pkg, geom, q, k, v, patterns)
    og = OA.Geometry(F, T, ns)
    sel_by_head = {h: sel[i].cpu() for i, h in enumerate(dyn)}
    got = out.float().cpu().reshape(geom.tokens, H, 64).permute(1, 0, 2)
    for h, pat in enumerate(patterns):
        ref = OA.sparse_attention_gathered(q[h].float(), k[h].float(), v[h].float(), pat, og, sel_by_head.get(h),
                                           dtype=torch.float64)
        _check_close(got[h], ref, f"F{F} T{T} ns{ns} head {h} pattern {pat}")


@pytest.mark.parametrize("F,T,ns", GEOMS)
def test_sparse_attention_token_order_dense(ops, pkg, F, T, ns):
    """DENSE heads in the token-order layout, in one launch with padded-layout heads."""
    geom = pkg.Geometry(F, T, ns)
    patterns = [ops.DENSE, ops.FRAME_LOCAL, ops.DENSE, ops.BLOCK_DYNAMIC, ops.DENSE]
    H = len(patterns)
    q, k, v = _qkv(H, geom.tokens, seed=F * 17 + T, scale=1.5)
    flags = ops.token_order_heads(patterns)
    qp, kp, vp = ops.pack_heads(q.to(DEV), k.to(DEV), v.to(DEV), geom, token_order=flags)
    pq, pk = ops.block_pool(qp, kp, geom, [3])
    sel = ops.block_select(pq, pk, geom.frames, geom.blocks_per_frame, 2)
    out = ops.sparse_attn_fwd(qp, kp, vp, geom, patterns, sel, token_order=flags)
    torch.cuda.synchronize()
    og = OA.Geometry(F, T, ns)
    got = out.float().cpu().reshape(geom.tokens, H, 64).permute(1, 0, 2)
    for h, pat in enumerate(patterns):
        ref = OA.sparse_attention_gathered(q[h].float(), k[h].float(), v[h].float(), pat, og,
                                           sel[0].cpu() if h == 3 else None, dtype=torch.float64)
        _check_close(got[h], ref, f"token order F{F} T{T} ns{ns} head {h} pattern {pat}")


@pytest.mark.parametrize("F,T,ns", GEOMS)
@pytest.mark.parametrize("prescaled", [False, True])
def test_sparse_attention_framed(ops, pkg, F, T, ns, prescaled):
    """Frame-relative heads in the framed layout (the plugin's layouts: token order for dense heads),
    with packed-layout heads in the same launch, against the oracle. Where the framed layout does not
    fit, token_order_heads leaves those heads packed and the same check covers that path."""
    geom = pkg.Geometry(F, T, ns)
    patterns = [ops.FRAME_LOCAL, ops.ANCHOR_LOCAL, ops.DENSE, ops.ANCHOR, ops.BLOCK_DYNAMIC, ops.FRAME_LOCAL,
                ops.ANCHOR_LOCAL]
    H = len(patterns)
    q, k, v = _qkv(H, geom.tokens, seed=F * 19 + T, scale=1.5)
    tord = ops.token_order_heads(patterns, geom)
    want_lay = ops.LAYOUT_FRAMED if geom.framed_fits else ops.LAYOUT_PACKED
    assert [tord[h] for h in (0, 1, 3, 5, 6)] == [want_lay] * 5 and tord[2] == ops.LAYOUT_TOKEN
    flags = [prescaled] * H
    qp, kp, vp = ops.pack_heads(q.to(DEV), k.to(DEV), v.to(DEV), geom, token_order=tord, q_scaled=flags)
    pq, pk = ops.block_pool(qp, kp, geom, [4])
    sel = ops.block_select(pq, pk, geom.frames, geom.blocks_per_frame, 2)
    og = OA.Geometry(F, T, ns)
    c = ops.prescale_factor()
    for order in ("fixed", "paced"):
        out = ops.sparse_attn_fwd(qp, kp, vp, geom, patterns, sel, token_order=tord, q_scaled=flags, order=order)
        torch.cuda.synchronize()
        got = out.float().cpu().reshape(geom.tokens, H, 64).permute(1, 0, 2)
        for h, pat in enumerate(patterns):
            qh = (q[h].float() * c).to(torch.bfloat16).float() / c if prescaled else q[h].float()
            ref = OA.sparse_attention_gathered(qh, k[h].float(), v[h].float(), pat, og,
                                               sel[0].cpu() if h == 4 else None, dtype=torch.float64)
            _check_close(got[h], ref, f"framed F{F} T{T} ns{ns} prescaled={prescaled} {order} head {h} pattern {pat}")


@pytest.mark.parametrize("phase", ["fixed", "paced"])
@pytest.mark.parametrize("framed", [False, True])
def test_sparse_attention_outrun_reference(ops, pkg, phase, framed):
    """Keys whose scores exceed the lazily moved reference maximum by more than 2^64 in P (and one
    beyond the fp32 exponent range) must take the exact path: rescale O and l, recompute P. Every
    pattern must still match the oracle. In the fixed walk order every walk starts at its first
    tile, so the outliers (last frame) are met late."""
    geom = pkg.Geometry(3, 155, 5)
    patterns = [ops.DENSE, ops.DENSE, ops.BLOCK_DYNAMIC, ops.FRAME_LOCAL, ops.ANCHOR_LOCAL]
    H = len(patterns)
    g = torch.Generator().manual_seed(5)
    N = geom.tokens
    q = (0.5 + 0.1 * torch.randn(H, N, 64, generator=g)).to(torch.bfloat16)
    k = (0.3 * torch.randn(H, N, 64, generator=g)).to(torch.bfloat16)
    v = torch.randn(H, N, 64, generator=g).to(torch.bfloat16)
    last = (geom.frames - 1) * geom.tokens_per_frame
    k[:, last + 40] = 12.0   # q.k ~ 384: about 69 log2 units above the first steps
    k[:, last + 100] = 30.0  # about 173 log2 units: exp2 overflows fp32 in the fast pass
    # dense head 0 token order, head 1 packed; the frame-relative heads packed or framed
    F2 = ops.LAYOUT_FRAMED if framed else ops.LAYOUT_PACKED
    flags = [ops.LAYOUT_TOKEN, ops.LAYOUT_PACKED, ops.LAYOUT_PACKED, F2, F2]
    qp, kp, vp = ops.pack_heads(q.to(DEV), k.to(DEV), v.to(DEV), geom, token_order=flags)
    pq, pk = ops.block_pool(qp, kp, geom, [2])
    sel = ops.block_select(pq, pk, geom.frames, geom.blocks_per_frame, 2)
    out = ops.sparse_attn_fwd(qp, kp, vp, geom, patterns, sel, token_order=flags, order=phase)
    torch.cuda.synchronize()
    og = OA.Geometry(3, 155, 5)
    got = out.float().cpu().reshape(N, H, 64).permute(1, 0, 2)
    assert torch.isfinite(got).all()
    for h, pat in enumerate(patterns):
        ref = OA.sparse_attention_gathered(q[h].float(), k[h].float(), v[h].float(), pat, og,
                                           sel[0].cpu() if h == 2 else None, dtype=torch.float64)
        _check_close(got[h], ref, f"outrun phase={phase} framed={framed} head {h} pattern {pat}")


def _prescaled_run(ops, pkg, geom, q, k, v, patterns, flags, order=None, k_sel=2, framed=False):
    """Packs every head with the softmax scale folded into Q and runs the attention on it; returns the
    output, the block lists, and the q the kernels consumed in unscaled units (fp32: packed / factor).
    ``framed``: frame-relative heads in the framed layout."""
    c = ops.prescale_factor()
    H = len(patterns)
    tord = ops.token_order_heads(patterns, geom if framed else None)
    qp, kp, vp = ops.pack_heads(q.to(DEV), k.to(DEV), v.to(DEV), geom, token_order=tord, q_scaled=flags)
    dyn = [h for h, p in enumerate(patterns) if p == ops.BLOCK_DYNAMIC]
    sel = None
    if dyn:
        pq, pk = ops.block_pool(qp, kp, geom, dyn)
        sel = ops.block_select(pq, pk, geom.frames, geom.blocks_per_frame, k_sel)
    out = ops.sparse_attn_fwd(qp, kp, vp, geom, patterns, sel, token_order=tord, q_scaled=flags, order=order)
    torch.cuda.synchronize()
    # the packed Q of a flagged head is bf16(q * c) (one rounding of the fp32 product)
    q_used = torch.stack([(q[h].float() * c).to(torch.bfloat16).float() / c if flags[h] else q[h].float()
                          for h in range(H)])
    return out, sel, dyn, q_used


@pytest.mark.parametrize("F,T,ns", [(3, 155, 5), (4, 1374, 5), (2, 64, 0), (3, 65, 1)])
def test_sparse_attention_prescaled_q(ops, pkg, F, T, ns):
    """Heads packed with the softmax scale in Q walk without a running maximum (exp2 of the MFMA
    result); every pattern and both layouts of DENSE heads match the oracle on the q they consumed,
    next to unflagged heads in the same launch."""
    geom = pkg.Geometry(F, T, ns)
    patterns = [ops.DENSE, ops.FRAME_LOCAL, ops.ANCHOR_LOCAL, ops.BLOCK_DYNAMIC, ops.ANCHOR, ops.SKIP,
                ops.DENSE, ops.FRAME_LOCAL]
    flags = [True, True, True, True, True, True, False, False]
    H = len(patterns)
    q, k, v = _qkv(H, geom.tokens, seed=F * 19 + T, scale=1.5)
    out, sel, dyn, q_used = _prescaled_run(ops, pkg, geom, q, k, v, patterns, flags)
    og = OA.Geometry(F, T, ns)
    got = out.float().cpu().reshape(geom.tokens, H, 64).permute(1, 0, 2)
    for h, pat in enumerate(patterns):
        ref = OA.sparse_attention_gathered(q_used[h], k[h].float(), v[h].float(), pat, og,
                                           sel[dyn.index(h)].cpu() if h in dyn else None, dtype=torch.float64)
        _check_close(got[h], ref, f"prescaled F{F} T{T} ns{ns} head {h} pattern {pat}")


@pytest.mark.parametrize("phase", ["fixed", "paced"])
@pytest.mark.parametrize("framed", [False, True])
def test_sparse_attention_prescaled_out_of_range(ops, pkg, phase, framed):
    """Prescaled heads whose scores leave the range of the walk without a running maximum: keys 69
    and 173 log2 units above the rest (partial row sums beyond 2^64), and rows whose every score lies
    more than 64 units below 0 (row sums below 2^-64). The main launch marks those items and the
    launch after it walks them with the exact maximum; every row matches the oracle."""
    geom = pkg.Geometry(3, 155, 5)
    patterns = [ops.DENSE, ops.DENSE, ops.BLOCK_DYNAMIC, ops.FRAME_LOCAL, ops.ANCHOR_LOCAL, ops.DENSE]
    H = len(patterns)
    g = torch.Generator().manual_seed(6)
    N = geom.tokens
    q = (0.5 + 0.1 * torch.randn(H, N, 64, generator=g)).to(torch.bfloat16)
    k = (0.3 * torch.randn(H, N, 64, generator=g)).to(torch.bfloat16)
    v = torch.randn(H, N, 64, generator=g).to(torch.bfloat16)
    last = (geom.frames - 1) * geom.tokens_per_frame
    k[:5, last + 40] = 12.0   # heads 0-4: outliers in the last frame (overflow)
    k[:5, last + 100] = 30.0
    # head 5: q.k about -400, about -72 log2 units after the scale, for every pair (underflow)
    q[5] = (2.5 + 0.05 * torch.randn(N, 64, generator=g)).to(torch.bfloat16)
    k[5] = (-2.5 + 0.05 * torch.randn(N, 64, generator=g)).to(torch.bfloat16)
    flags = [True] * H
    out, sel, dyn, q_used = _prescaled_run(ops, pkg, geom, q, k, v, patterns, flags, order=phase, framed=framed)
    og = OA.Geometry(3, 155, 5)
    got = out.float().cpu().reshape(N, H, 64).permute(1, 0, 2)
    assert torch.isfinite(got).all()
    for h, pat in enumerate(patterns):
        ref = OA.sparse_attention_gathered(q_used[h], k[h].float(), v[h].float(), pat, og,
                                           sel[0].cpu() if h == 2 else None, dtype=torch.float64)
        _check_close(got[h], ref, f"prescaled out of range phase={phase} framed={framed} head {h} pattern {pat}")


def test_walk_order_paced_and_fixed(ops, pkg):
    """The paced walk order (the product default: walks start where the measured step time and the
    wall clock point) matches the oracle on every pattern over repeated calls, whose pace state
    carries a measured step time from the second call on; the fixed order is bitwise reproducible."""
    geom = pkg.Geometry(24, 1374, 5)
    patterns = [ops.DENSE, ops.BLOCK_DYNAMIC, ops.FRAME_LOCAL, ops.ANCHOR_LOCAL, ops.BLOCK_DYNAMIC, ops.DENSE]
    H = len(patterns)
    q, k, v = _qkv(H, geom.tokens, seed=99, scale=1.5)
    flags = ops.token_order_heads(patterns, geom)  # the plugin's layouts
    qp, kp, vp = ops.pack_heads(q.to(DEV), k.to(DEV), v.to(DEV), geom, token_order=flags)
    dyn = [1, 4]
    pq, pk = ops.block_pool(qp, kp, geom, dyn)
    sel = ops.block_select(pq, pk, geom.frames, geom.blocks_per_frame, 4)
    outs = [ops.sparse_attn_fwd(qp, kp, vp, geom, patterns, sel, token_order=flags, order="paced").clone()
            for _ in range(4)]
    fixed = [ops.sparse_attn_fwd(qp, kp, vp, geom, patterns, sel, token_order=flags, order="fixed").clone()
             for _ in range(2)]
    torch.cuda.synchronize()
    assert torch.equal(fixed[0], fixed[1])
    pace = ops._pace_state[0][0].cpu()
    assert int(pace[1::2].sum()) > 0  # the walks measured their step times
    og = OA.Geometry(geom.frames, geom.tokens_per_frame, geom.num_special)
    rows = torch.cat([torch.arange(0, 200), torch.arange(geom.tokens - 1500, geom.tokens, 7),
                      torch.randint(0, geom.tokens, (300,), generator=torch.Generator().manual_seed(1))])
    for h, pat in enumerate(patterns):
        s = sel[dyn.index(h)].cpu() if h in dyn else None
        m = OA.allowed_mask(pat, rows, og, s)
        ref = OA.masked_attention(q[h][rows].float(), k[h].float(), v[h].float(), m)
        for i, o in enumerate(outs + fixed):
            got = o[rows.to(DEV)].float().cpu().reshape(len(rows), H, 64)[:, h]
            _check_close(got, ref, f"walk order call {i} head {h} pattern {pat}")


def test_sparse_attention_selection_edge_cases(ops, pkg):
    """Hand-made selection lists: -1 entries, a single block, whole-frame selections."""
    geom = pkg.Geometry(3, 155, 5)
    nb = geom.num_blocks
    H = 2
    q, k, v = _qkv(H, geom.tokens, seed=77)
    qp, kp, vp = ops.pack_heads(q.to(DEV), k.to(DEV), v.to(DEV), geom)
    sel = torch.full((2, nb, 5), -1, dtype=torch.int32)
    for b in range(nb):
        sel[0, b, 0] = (b * 5) % nb
        sel[0, b, 3] = (b + 1) % nb if (b + 1) % nb != (b * 5) % nb else -1
        sel[1, b, :3] = torch.tensor([b % 3, 3 + b % 3, 6 + b % 3])
    out = ops.sparse_attn_fwd(qp, kp, vp, geom, [ops.BLOCK_DYNAMIC, ops.BLOCK_DYNAMIC], sel.to(DEV))
    torch.cuda.synchronize()
    og = OA.Geometry(3, 155, 5)
    got = out.float().cpu().reshape(geom.tokens, H, 64).permute(1, 0, 2)
    for h in range(H):
        ref = OA.pattern_attention(q[h].float(), k[h].float(), v[h].float(), OA.BLOCK_DYNAMIC, og, sel[h])
        _check_close(got[h], ref, f"edge head {h}")


@pytest.mark.parametrize("layouts", [False, True])
def test_sparse_attention_structured_c1(ops, pkg, layouts):
    """The 4-frame VGGT shape (5,496 tokens, 16 heads) with the structured generator and round-robin
    patterns: every head in the packed layout, or with the plugin's layouts and prescaled Q."""
    synth = importlib.import_module(pkg.__name__ + ".synth")
    H = 16
    wl = synth.structured_qkv(frames=4, heads=H, seed=0)
    geom = wl.geom
    patterns = synth.round_robin_patterns(H)
    q, k, v = (t.to(torch.bfloat16) for t in (wl.q, wl.k, wl.v))
    if layouts:
        out, sel, dyn, q_used = _prescaled_run(ops, pkg, geom, q, k, v, patterns, [True] * H, k_sel=4, framed=True)
    else:
        out, sel, dyn = _run_layer(ops, pkg, geom, q, k, v, patterns, k_sel=4)
        q_used = q.float()
    og = OA.Geometry(geom.frames, geom.tokens_per_frame, geom.num_special)
    got = out.float().cpu().reshape(geom.tokens, H, 64).permute(1, 0, 2)
    # the selection is bit-exact against the oracle pipeline on the packed Q (prescaled: bf16(q * c))
    c = ops.prescale_factor()
    for i, h in enumerate(dyn):
        qsel = (q[h].float() * c).to(torch.bfloat16) if layouts else q[h]
        ref_sel = OS.block_select(OS.bf16_bits(qsel.float().numpy()), OS.bf16_bits(k[h].float().numpy()),
                                  geom.frames, geom.tokens_per_frame, geom.num_special, 4)
        assert np.array_equal(sel[i].cpu().numpy(), ref_sel)
    sel_by_head = {h: sel[i].cpu() for i, h in enumerate(dyn)}
    for h, pat in enumerate(patterns):
        ref = OA.sparse_attention_gathered(q_used[h], k[h].float(), v[h].float(), pat, og, sel_by_head.get(h),
                                           dtype=torch.float64)
        _check_close(got[h], ref, f"C1 layouts={layouts} head {h} pattern {pat}")


@pytest.mark.parametrize("n,nk,topk", [(100, 300, 7), (37, 64, 64), (64, 5000, 512), (5, 3000, 2100)])
def test_gather_attention(ops, n, nk, topk):
    g = torch.Generator().manual_seed(n + topk)
    q, k, v = (torch.randn(m, 64, generator=g).to(torch.bfloat16) for m in (n, nk, nk))
    idx = torch.randint(0, nk, (n, topk), generator=g, dtype=torch.int32)
    idx[0, :3] = -1
    got = ops.gather_attn_fwd(q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV))
    torch.cuda.synchronize()
    ref = OA.gather_attention(q.float(), k.float(), v.float(), idx, dtype=torch.float64)
    _check_close(got.cpu(), ref, f"gather n{n} topk{topk}")


@pytest.mark.parametrize("n,nk,topk", [(100, 300, 7), (64, 5000, 512), (5, 3000, 2100)])
def test_gather_attention_fp32_qk(ops, n, nk, topk):
    """fp32 q / k rows (the reference's gather reads fp32 q / k under autocast): the scores are fp32 dot
    products of the fp32 values, which bf16 rounding of q / k would move."""
    g = torch.Generator().manual_seed(n + topk + 1)
    q, k = (3.0 * torch.randn(m, 64, generator=g) for m in (n, nk))
    v = torch.randn(nk, 64, generator=g).to(torch.bfloat16)
    idx = torch.randint(0, nk, (n, topk), generator=g, dtype=torch.int32)
    idx[0, :3] = -1
    got = ops.gather_attn_fwd(q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV))
    torch.cuda.synchronize()
    ref = OA.gather_attention(q.double(), k.double(), v.float(), idx, dtype=torch.float64)
    _check_close(got.cpu(), ref, f"gather fp32 q/k n{n} topk{topk}")
    ref_bf = OA.gather_attention(q.to(torch.bfloat16).float(), k.to(torch.bfloat16).float(), v.float(), idx,
                                 dtype=torch.float64)
    if topk <= 512:  # concentrated softmax: bf16-rounded q / k would be much further off than the kernel is
        assert (ref_bf - ref).abs().max() > 2 * (got.cpu().float() - ref).abs().max()


def test_gather_attention_shared_list(ops):
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(m, 64, generator=g).to(torch.bfloat16) for m in (50, 400, 400))
    lst = torch.randperm(400, generator=g)[:96].int()
    idx = lst[None, :].expand(50, 96)  # stride-0 rows
    got = ops.gather_attn_fwd(q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV))
    torch.cuda.synchronize()
    ref = OA.gather_attention(q.float(), k.float(), v.float(), idx.contiguous(), dtype=torch.float64)
    _check_close(got.cpu(), ref, "gather shared list")


@pytest.mark.parametrize("n,nk,topk,rpf", [(100, 300, 5, 300), (70, 3000, 300, 300), (3000, 40 * 137, 160, 137)])
def test_gather_attention_sliced(ops, n, nk, topk, rpf):
    """The two-pass sliced gather (lists cut into 8 slices, partial softmax merged): against the fp64
    reference, and within fp32 rounding of the one-pass kernel. Covers slices left empty (topk 5 < 8),
    masked and out-of-range entries, a row with no valid entry, fp32 q / k, and key rows addressed
    frame by frame (rows_per_frame < the key count, skipping 3 junk rows per stored frame)."""
    g = torch.Generator().manual_seed(n + topk + 7)
    q = 3.0 * torch.randn(n, 64, generator=g)
    k = 3.0 * torch.randn(nk, 64, generator=g)
    v = torch.randn(nk, 64, generator=g).to(torch.bfloat16)
    idx = torch.randint(0, nk, (n, topk), generator=g, dtype=torch.int32)
    idx[0, :3] = -1
    idx[1, :] = -1            # no valid entry: zeros
    idx[2, -1] = nk + 5       # out of range: skipped
    pad = 3
    kst = torch.randn(nk // rpf, pad + rpf, 64, generator=g)
    kst[:, pad:] = k.view(-1, rpf, 64)
    vst = torch.randn(nk // rpf, pad + rpf, 64, generator=g).to(torch.bfloat16)
    vst[:, pad:] = v.view(-1, rpf, 64)
    qd, kd, vd, idd = q.to(DEV), kst.to(DEV).view(-1, 64), vst.to(DEV).view(-1, 64), idx.to(DEV)
    kr = ops.rows(kd, base_row=pad, rows_per_frame=rpf, frame_row_stride=pad + rpf)
    vr = ops.rows(vd, base_row=pad, rows_per_frame=rpf, frame_row_stride=pad + rpf)
    outs = {}
    for sliced in (True, False):
        out = torch.full((n, 64), 7.0, dtype=torch.bfloat16, device=DEV)
        ops.gather_attn_rows(ops.rows(qd), kr, vr, idd, topk, n, topk, nk, None, ops.rows(out), qk_fp32=True,
                             sliced=sliced)
        outs[sliced] = out.cpu()
    torch.cuda.synchronize()
    ref = OA.gather_attention(q.double(), k.double(), v.float(), idx.clamp(max=nk - 1).where(idx < nk, -1),
                              dtype=torch.float64)
    ref[1] = 0.0  # the reference's softmax over no entry is NaN; the kernels write zeros
    _check_close(outs[True], ref, f"sliced gather n{n} topk{topk}")
    assert torch.all(outs[True][1] == 0)
    # the same sums in another order: one bf16 ulp (of the larger value) apart at most, beside values
    # near zero that cancellation leaves (an absolute 1e-4, far below the outputs' scale of 1)
    a, b = outs[True].float(), outs[False].float()
    assert ((a - b).abs() <= torch.maximum(a.abs(), b.abs()) * 2 ** -7 + 1e-4).all(), (a - b).abs().max()


@pytest.mark.parametrize("n", [65536 + 777, 2 * 65536 + 5])
def test_gather_attention_sliced_row_chunks(ops, n):
    """The sliced gather runs rows in chunks of 65536 (both kernels per chunk, one chunk's partials in
    the workspace): 2 and 3 chunks, the last one partial. Every row against the one-pass kernel, and
    rows at the chunk boundaries and the ends against the fp64 reference."""
    nk, topk = 4000, 24
    g = torch.Generator().manual_seed(11)
    q = 3.0 * torch.randn(n, 64, generator=g)
    k = 3.0 * torch.randn(nk, 64, generator=g)
    v = torch.randn(nk, 64, generator=g).to(torch.bfloat16)
    idx = torch.randint(0, nk, (n, topk), generator=g, dtype=torch.int32)
    qd, kd, vd, idd = q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV)
    outs = {}
    for sliced in (True, False):
        out = torch.full((n, 64), 7.0, dtype=torch.bfloat16, device=DEV)
        ops.gather_attn_rows(ops.rows(qd), ops.rows(kd), ops.rows(vd), idd, topk, n, topk, nk, None, ops.rows(out),
                             qk_fp32=True, sliced=sliced)
        outs[sliced] = out.cpu()
    torch.cuda.synchronize()
    a, b = outs[True].float(), outs[False].float()
    assert ((a - b).abs() <= torch.maximum(a.abs(), b.abs()) * 2 ** -7 + 1e-4).all(), (a - b).abs().max()
    rows = torch.tensor(sorted({0, 1, 65534, 65535, 65536, 65537, 131071, 131072, n - 2, n - 1} & set(range(n))))
    ref = OA.gather_attention(q[rows].double(), k.double(), v.float(), idx[rows], dtype=torch.float64)
    _check_close(outs[True][rows], ref, "sliced gather across row chunks")


@pytest.mark.parametrize("layout", ["framed", "paired"])
def test_token_topk_key_row_layouts(ops, layout):
    """Key rows described frame by frame (rows_per_frame == per_frame: the plugin's packed layout)
    and with two key frames per stored frame (the general row map) select what the flat rows do."""
    frames, P, topk, pad = 4, 100, 4, 3
    g = torch.Generator().manual_seed(11)
    q = torch.randn(200, 64, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(frames * P, 64, generator=g).to(torch.bfloat16)
    want = ops.token_topk(q, k.to(DEV), frames, P, topk).cpu()
    rpf = P if layout == "framed" else 2 * P
    store = torch.randn(frames * P // rpf, pad + rpf, 64, generator=g).to(torch.bfloat16)
    store[:, pad:] = k.view(-1, rpf, 64)  # junk rows ahead of every stored frame
    store = store.to(DEV)
    kr = ops.rows(store.view(-1, 64), base_row=pad, rows_per_frame=rpf, frame_row_stride=pad + rpf)
    got = ops.token_topk(q, None, frames, P, topk, krows=kr).cpu()
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("topk", [1, 4, 16])
def test_token_topk_mass_ties(ops, topk):
    """Key frames made of three repeated rows: a third of a frame's scores tie exactly at the
    frame's best value, so far more candidates than fit a lane's buffer reach the threshold; the
    lowest indices of the best value win, as in the reference's composite key."""
    frames, P, nq = 3, 700, 260
    g = torch.Generator().manual_seed(5)
    base = torch.randn(3, 64, generator=g).to(torch.bfloat16)
    k = base[torch.randint(0, 3, (frames * P,), generator=g)]
    q = torch.randn(nq, 64, generator=g).to(torch.bfloat16)
    got = ops.token_topk(q.to(DEV), k.to(DEV), frames, P, topk).cpu()
    torch.cuda.synchronize()
    s = (q.double() @ k.double().T).float().numpy()
    ref = OS.frame_topk(s, frames, topk)
    assert np.array_equal(got.numpy(), ref)


@pytest.mark.parametrize("frames,P,topk", [(3, 1369, 128), (2, 200, 100), (4, 70, 17), (2, 50, 300)])
def test_token_topk_large_k(ops, frames, P, topk):
    """16 < min(topk, P) <= 128 (the reference's range): scores of a chunk of queries, then a radix
    selection per (query, frame); also topk > P (every key of a frame, best first)."""
    g = torch.Generator().manual_seed(frames * P + topk)
    nq = 300
    q = torch.randn(nq, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(frames * P, 64, generator=g).to(torch.bfloat16)
    got = ops.token_topk(q.to(DEV), k.to(DEV), frames, P, topk).cpu()
    torch.cuda.synchronize()
    s = (q.double() @ k.double().T).float().numpy()
    ref = OS.frame_topk(s, frames, topk)
    assert got.shape == ref.shape
    gs = np.take_along_axis(s, got.numpy().astype(np.int64), axis=1)
    rs = np.take_along_axis(s, ref.astype(np.int64), axis=1)
    assert np.allclose(gs, rs, atol=1e-4, rtol=0), "selected scores differ beyond rounding noise"
    assert (got.numpy() == ref).mean() >= 0.99
    # within a frame: distinct keys of that frame, scores non-increasing
    ke = min(topk, P)
    gi = got.numpy().reshape(nq, frames, ke)
    for f in range(frames):
        blk = gi[:, f]
        assert ((blk >= f * P) & (blk < (f + 1) * P)).all()
        assert all(len(set(row)) == ke for row in blk)


def test_token_topk_large_k_ties_and_layout(ops):
    """Mass ties (three repeated key rows) at k = 64 through the general row map: bit-exact with the
    oracle, lowest indices first among equal scores."""
    frames, P, topk, pad = 4, 150, 64, 5
    g = torch.Generator().manual_seed(8)
    base = torch.randn(3, 64, generator=g).to(torch.bfloat16)
    k = base[torch.randint(0, 3, (frames * P,), generator=g)]
    q = torch.randn(130, 64, generator=g).to(torch.bfloat16)
    store = torch.zeros(frames * P // (2 * P), pad + 2 * P, 64, dtype=torch.bfloat16)
    store[:, pad:] = k.view(-1, 2 * P, 64)
    store = store.to(DEV)  # kept alive: the row descriptor holds a raw pointer
    kr = ops.rows(store.view(-1, 64), base_row=pad, rows_per_frame=2 * P, frame_row_stride=pad + 2 * P)
    got = ops.token_topk(q.to(DEV), None, frames, P, topk, krows=kr).cpu()
    torch.cuda.synchronize()
    s = (q.double() @ k.double().T).float().numpy()
    assert np.array_equal(got.numpy(), OS.frame_topk(s, frames, topk))


def test_token_topk_large_k_chunks(ops):
    """128 frames x 1369 keys, top-32 for 3000 queries: the score workspace (1 GiB at most) takes
    the queries in three chunks; sampled rows at the chunk edges against the oracle."""
    frames, P, topk, nq = 128, 1369, 32, 3000
    g = torch.Generator().manual_seed(21)
    q = torch.randn(nq, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(frames * P, 64, generator=g).to(torch.bfloat16)
    got = ops.token_topk(q.to(DEV), k.to(DEV), frames, P, topk).cpu()
    torch.cuda.synchronize()
    rows = [0, 1, 1407, 1408, 1409, 2815, 2816, 2999]
    s = (q[rows].double() @ k.double().T).float().numpy()
    ref = OS.frame_topk(s, frames, topk)
    g_ = got[rows].numpy()
    gs = np.take_along_axis(s, g_.astype(np.int64), axis=1)
    rs = np.take_along_axis(s, ref.astype(np.int64), axis=1)
    assert np.allclose(gs, rs, atol=1e-4, rtol=0)
    assert (g_ == ref).mean() >= 0.99


@pytest.mark.parametrize("frames,P,topk", [(4, 1369, 4), (3, 100, 8), (2, 30, 16), (5, 64, 1)])
def test_token_topk(ops, frames, P, topk):
    g = torch.Generator().manual_seed(frames * P)
    nq = 300
    q = torch.randn(nq, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(frames * P, 64, generator=g).to(torch.bfloat16)
    got = ops.token_topk(q.to(DEV), k.to(DEV), frames, P, topk).cpu()
    torch.cuda.synchronize()
    s = (q.double() @ k.double().T).float().numpy()  # exact products, fp32-rounded sums
    ref = OS.frame_topk(s, frames, topk)
    ke = min(topk, P)
    assert got.shape == ref.shape
    # identical except where the oracle's scores are within fp32 accumulation noise of a tie
    gs = np.take_along_axis(s, got.numpy().astype(np.int64), axis=1)
    rs = np.take_along_axis(s, ref.astype(np.int64), axis=1)
    assert np.allclose(gs, rs, atol=1e-4, rtol=0), "selected scores differ beyond rounding noise"
    same = (got.numpy() == ref).mean()
    assert same > 0.99, f"only {same:.4f} of the indices agree"
    for f in range(frames):  # frame-major: entries of frame f index frame f's keys
        blk = got[:, f * ke:(f + 1) * ke]
        assert ((blk // P) == f).all()
