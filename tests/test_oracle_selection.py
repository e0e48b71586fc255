"""Pins the C selection oracle (sortable key, pooling, scoring, top-k) with checks that do not
restate its formulas: brute-force sorts, float comparison, exact small-integer arithmetic and a
crafted case where a fused multiply-add and a separate multiply+add differ."""
import math

import numpy as np
import pytest

from oracle import selection as sel


def _brute_frame_topk(scores, frames, k):
    nq, nc = scores.shape
    c = nc // frames
    ke = min(k, c)
    keys = sel.fkey(scores)
    out = np.full((nq, frames * ke), -1, np.int32)
    for i in range(nq):
        for f in range(frames):
            cand = list(range(f * c, (f + 1) * c))
            cand.sort(key=lambda j: (-int(keys[i, j]), j))
            out[i, f * ke:(f + 1) * ke] = cand[:ke]
    return out


def test_fkey_orders_like_floats():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(2000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 2000),
        np.array([0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-45, np.finfo(np.float32).max,
                  -np.finfo(np.float32).max, np.finfo(np.float32).tiny], np.float32),
    ]).astype(np.float32)
    keys = sel.fkey(vals)
    order_by_key = np.argsort(keys, kind="stable")
    srt = vals[order_by_key]
    assert np.all(np.diff(srt.astype(np.float64)) >= 0)
    # -0.0 sorts strictly below +0.0; -inf is the smallest non-NaN, +inf the largest.
    assert sel.fkey(np.float32(-0.0)) < sel.fkey(np.float32(0.0))
    assert sel.fkey(np.float32(-np.inf)) == keys.min()
    assert sel.fkey(np.float32(np.inf)) == keys.max()
    # C transform agrees with the vectorised one, including NaN payloads.
    for b in [0x00000000, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00000, 0x3F800000, 0xBF800000]:
        assert sel.fkey_c(b) == int(sel.fkey(np.array([b], np.uint32).view(np.float32))[0])
    # Positive NaN ranks above +inf, negative NaN below -inf.
    assert sel.fkey_c(0x7FC00000) > sel.fkey_c(0x7F800000)
    assert sel.fkey_c(0xFFC00000) < sel.fkey_c(0xFF800000)


@pytest.mark.parametrize("frames,c,k", [(1, 5, 2), (3, 22, 4), (4, 7, 7), (2, 9, 16), (5, 33, 8)])
def test_frame_topk_matches_brute_force_with_ties(frames, c, k):
    rng = np.random.default_rng(frames * 100 + c)
    # small integers force many exact ties; signed zeros and infinities included
    s = rng.integers(-3, 4, size=(6, frames * c)).astype(np.float32)
    s[0, :3] = [-0.0, 0.0, -0.0]
    s[1, 1] = np.inf
    s[2, 0] = -np.inf
    got = sel.frame_topk(s, frames, k)
    assert np.array_equal(got, _brute_frame_topk(s, frames, k))


def test_frame_topk_whole_frame_and_tie_to_lowest_index():
    s = np.zeros((1, 6), np.float32)  # all equal -> lowest indices first, per frame
    assert sel.frame_topk(s, 2, 2).tolist() == [[0, 1, 3, 4]]
    assert sel.frame_topk(s, 2, 10).tolist() == [[0, 1, 2, 3, 4, 5]]  # k >= C: whole frame
    s = np.array([[1, 3, 2, 3]], np.float32)
    assert sel.frame_topk(s, 1, 3).tolist() == [[1, 3, 2]]  # descending, tie -> lower index
    s = np.array([[-0.0, 0.0]], np.float32)
    assert sel.frame_topk(s, 1, 1).tolist() == [[1]]  # +0.0 beats -0.0


def test_global_topk_matches_brute_force():
    rng = np.random.default_rng(3)
    s = rng.integers(-2, 3, size=(5, 40)).astype(np.float32)
    got = sel.global_topk(s, 6)
    keys = sel.fkey(s)
    for i in range(5):
        exp = sorted(range(40), key=lambda j: (-int(keys[i, j]), j))[:6]
        assert got[i].tolist() == exp


def test_block_pool_is_population_mean():
    rng = np.random.default_rng(1)
    F, T, ns, D = 3, 5 + 150, 5, 8  # 150 patches -> blocks of 64, 64, 22
    x = rng.standard_normal((F * T, D)).astype(np.float32)
    xb = sel.bf16_bits(x)
    xf = sel.bf16_to_f32(xb)
    got = sel.block_pool(xb, F, T, ns)
    assert got.shape == (F * 3, D)
    for f in range(F):
        for b, (p0, p1) in enumerate([(0, 64), (64, 128), (128, 150)]):
            rows = xf[f * T + ns + p0:f * T + ns + p1].astype(np.float64)
            np.testing.assert_allclose(got[f * 3 + b], rows.mean(0), rtol=0, atol=2e-6)
    # exact on data whose partial sums are exact in fp32
    xi = rng.integers(-8, 9, size=(F * T, D)).astype(np.float32)
    got = sel.block_pool(sel.bf16_bits(xi), F, T, ns)
    for f in range(F):
        rows = xi[f * T + ns + 128:f * T + ns + 150]
        assert np.array_equal(got[f * 3 + 2], (rows.sum(0) / np.float32(22)).astype(np.float32))


def test_block_pool_summation_order_is_grouped_by_16_rows():
    """The block mean's fp32 order: groups of 16 rows, each summed in row order, the group sums added
    in group order. Closed forms on values where every other order rounds differently: 8 rows of
    2^21 then ones (ulp 2 at 2^24, ties to even drop single ones)."""
    F, T, ns, D = 1, 64, 0, 2
    x = np.ones((64, D), np.float32)
    x[:8] = 2.0 ** 21
    got = sel.block_pool(sel.bf16_bits(x), F, T, ns)
    # group 0: 2^24 (its 8 ones are each lost); groups 1..3: 16 each, added exactly
    assert np.all(got == np.float32((2 ** 24 + 48) / 64))
    # (sequential: 2^24 / 64; groups of 8: (2^24 + 56) / 64; groups of 32: (2^24 + 32) / 64)
    assert got[0, 0] not in (np.float32(2 ** 24 / 64), np.float32((2 ** 24 + 56) / 64), np.float32((2 ** 24 + 32) / 64))
    # group sums in order: 2^24 + 1 + 1 + 2 rounds to 2^24 + 2 (reversed it would be 2^24 + 4)
    y = np.zeros((64, D), np.float32)
    y[:8] = 2.0 ** 21
    y[16], y[32], y[48] = 1.0, 1.0, 2.0
    got = sel.block_pool(sel.bf16_bits(y), F, T, ns)
    assert np.all(got == np.float32((2 ** 24 + 2) / 64))
    # a partial block of 22 rows: 8 rows of 2^21, 14 ones -> group 0 = 2^24, group 1 = 6
    F, T, ns = 1, 64 + 22 + 5, 5
    z = np.ones((T, D), np.float32)
    z[ns + 64:ns + 72] = 2.0 ** 21
    got = sel.block_pool(sel.bf16_bits(z), F, T, ns)
    assert np.all(got[1] == np.float32(np.float32(2 ** 24 + 6) / np.float32(22)))


def test_block_scores_use_sequential_fma():
    rng = np.random.default_rng(2)
    q = rng.integers(-5, 6, size=(4, 64)).astype(np.float32)
    k = rng.integers(-5, 6, size=(7, 64)).astype(np.float32)
    assert np.array_equal(sel.block_scores(q, k), (q.astype(np.int64) @ k.T.astype(np.int64)).astype(np.float32))
    # a = 1 + 2^-12: fl(a*a) = 1 + 2^-11 (the 2^-24 term rounds away); then fma(a, -a, fl(a*a))
    # is exactly -2^-24 whereas a separate multiply and add would give 0.
    a = np.float32(1 + 2.0 ** -12)
    got = sel.block_scores(np.array([[a, a]], np.float32), np.array([[a, -a]], np.float32))
    assert got[0, 0] == np.float32(-(2.0 ** -24))
    # agreement with float64 on random data
    qa = rng.standard_normal((9, 64)).astype(np.float32)
    ka = rng.standard_normal((11, 64)).astype(np.float32)
    np.testing.assert_allclose(sel.block_scores(qa, ka), qa.astype(np.float64) @ ka.T.astype(np.float64), atol=1e-4)


def test_bf16_rounding_is_nearest_even():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9, -2.5, 65504.0], np.float32)
    got = sel.bf16_to_f32(sel.bf16_bits(x))
    import torch
    exp = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(got, exp)


def test_block_select_pipeline_shapes():
    rng = np.random.default_rng(4)
    F, T, ns = 2, 5 + 130, 5
    q = sel.bf16_bits(rng.standard_normal((F * T, 64)).astype(np.float32))
    k = sel.bf16_bits(rng.standard_normal((F * T, 64)).astype(np.float32))
    idx = sel.block_select(q, k, F, T, ns, topk=2)
    assert idx.shape == (F * 3, F * 2)
    assert idx.min() >= 0 and idx.max() < F * 3
    for f in range(F):  # frame-major: entries of frame f lie in frame f's block range
        assert np.all(idx[:, 2 * f:2 * f + 2] // 3 == f)
    assert math.isfinite(float(np.abs(sel.block_pool(q, F, T, ns)).max()))
