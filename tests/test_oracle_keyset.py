"""Pins the key-set oracle of the `stride` and `q_probe_topk` modes
(saf3r/patch/sparse_attention.py:56-85, 143-186, 256-273) with checks that do not restate it:
set algebra of the strided key range, brute-force sorts with ties, float64 means and dot
products, a crafted fused-versus-unfused multiply-add case, and equality of the key-set
attention with library SDPA over the gathered keys."""
import math

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import selection as sel


def _include_set(n, T, ns):
    return set(range(min(n, T))) | {t for t in range(n) if t % T < ns}


@pytest.mark.parametrize("frames,T,ns,stride,start,include", [
    (4, 155, 5, 4, 0, True), (3, 70, 5, 128, 0, True), (2, 64, 0, 3, 2, False), (5, 37, 5, 7, 6, True),
    (1, 1374, 5, 4, 1, False)])
def test_stride_keyset_is_set_union(frames, T, ns, stride, start, include):
    n = frames * T
    got = sel.keyset(None, n, T, ns, sel.KEYSET_STRIDE, stride, start, include)
    want = set(range(start, n, stride)) | (_include_set(n, T, ns) if include else set())
    assert got.tolist() == sorted(want)


@pytest.mark.parametrize("n,k,include", [(300, 17, False), (300, 299, True), (1000, 250, False), (64, 200, False)])
def test_topk_keyset_matches_brute_force_with_ties(n, k, include):
    rng = np.random.default_rng(n + k)
    scores = rng.integers(-4, 5, n).astype(np.float32)  # heavy ties
    scores[::7] = -0.0
    scores[3::11] = 0.0
    T, ns = 50, 5
    got = sel.keyset(scores, n, T, ns, sel.KEYSET_TOPK, k, 0, include)
    keys = sel.fkey(scores)
    order = sorted(range(n), key=lambda t: (-int(keys[t]), t))
    want = set(order[:min(k, n)]) | (_include_set(n, T, ns) if include else set())
    assert got.tolist() == sorted(want)


def test_topk_keyset_agrees_with_library_topk_on_distinct_scores():
    rng = np.random.default_rng(1)
    scores = rng.standard_normal(5000).astype(np.float32)
    k = 1234
    got = sel.keyset(scores, 5000, 100, 5, sel.KEYSET_TOPK, k)
    want = torch.topk(torch.from_numpy(scores), k, sorted=False).indices.sort().values.numpy()
    assert np.array_equal(got, want)


def test_probe_mean_is_the_mean_in_chunk_order():
    rng = np.random.default_rng(2)
    n, d = 3000, 64
    x = rng.standard_normal((n, d)).astype(np.float32)
    q = sel.bf16_bits(x)
    got = sel.probe_mean(q)
    xf = sel.bf16_to_f32(q)
    np.testing.assert_allclose(got, xf.astype(np.float64).mean(0), rtol=0, atol=2e-6)
    # the exact order: chunk partial sums (sequential), then the chunk sums in order, then / n
    r = sel.probe_chunk(n)
    assert r == math.ceil(n / 256)
    want = np.zeros(d, np.float32)
    for c0 in range(0, n, r):
        part = np.zeros(d, np.float32)
        for t in range(c0, min(n, c0 + r)):
            part = (part + xf[t]).astype(np.float32)
        want = (want + part).astype(np.float32)
    want = (want / np.float32(n)).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_probe_scores_use_sequential_fma_and_exact_scale():
    rng = np.random.default_rng(3)
    n, d = 500, 64
    k = sel.bf16_bits(rng.standard_normal((n, d)).astype(np.float32))
    qbar = rng.standard_normal(d).astype(np.float32)
    got = sel.probe_scores(qbar, k)
    ref = (sel.bf16_to_f32(k).astype(np.float64) @ qbar.astype(np.float64)) / 8.0
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
    # crafted: term 0 is exact, term 1's product q1*k1 = 1 + 2^-7 + 2^-23 + 2^-30 is not
    # representable; fused into the accumulator it leaves exactly 2^-30, while a separate
    # multiply (rounding away 2^-30) and add would give 0
    qb = np.zeros(d, np.float32)
    qb[0] = -np.float32(1.0 + 2.0 ** -7 + 2.0 ** -23)
    qb[1] = np.float32(1.0 + 2.0 ** -23)
    krow = np.zeros((1, d), np.float32)
    krow[0, 0] = 1.0
    krow[0, 1] = 1.0 + 2.0 ** -7  # bf16-exact
    s = sel.probe_scores(qb, sel.bf16_bits(krow), scale=1.0)
    assert s[0] == np.float32(2.0 ** -30)
    # the scale is a power of two, so scaling is exact
    s8 = sel.probe_scores(qb, sel.bf16_bits(krow), scale=0.125)
    assert s8[0] == np.float32(2.0 ** -33)


def test_keyset_attention_is_sdpa_over_the_gathered_keys():
    torch.manual_seed(0)
    g = OA.Geometry(3, 70, 5)
    n = g.tokens
    q, k, v = (torch.randn(n, 64) for _ in range(3))
    keys = torch.from_numpy(sel.keyset(None, n, 70, 5, sel.KEYSET_STRIDE, 4, 1, True))
    got = OA.pattern_attention(q, k, v, OA.KEYSET, g, keys, dtype=torch.float64)
    ref = torch.nn.functional.scaled_dot_product_attention(q[None].double(), k[keys][None].double(),
                                                           v[keys][None].double())[0]
    torch.testing.assert_close(got, ref, rtol=1e-10, atol=1e-10)
    got2 = OA.sparse_attention_gathered(q, k, v, OA.KEYSET, g, keys, dtype=torch.float64)
    torch.testing.assert_close(got2, ref, rtol=1e-10, atol=1e-10)
