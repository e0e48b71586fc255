"""Pins the token top-k from feature scores (oracle.selection.token_topk_from_scores,
saf3r/patch/utils.py:54-184): library top-k on distinct scores, whole frames when k >= P, the tie
rule, the sortable order of signed zeros, frame-0 exclusion with samples, the cap, and the width
arithmetic of compute_qk_topk_indices_batched."""
import numpy as np
import pytest
import torch

from oracle import selection as OS


def _distinct_bits(rows, n, seed):
    rng = np.random.default_rng(seed)
    vals = rng.permutation(np.arange(n * rows) - n * rows // 2).astype(np.float32) / 64.0
    x = torch.from_numpy(vals.reshape(rows, n)).to(torch.bfloat16)
    assert all(len(np.unique(x[r].float().numpy())) == n for r in range(rows))  # exact in bf16
    return x.view(torch.int16).numpy().view(np.uint16), x


def test_per_frame_matches_library_topk_on_distinct_scores():
    F, P, k = 3, 40, 5
    bits, x = _distinct_bits(4, F * P, 0)
    got = OS.token_topk_from_scores(bits, F, P, k)
    assert got.shape == (4, F * k)
    for r in range(4):
        for f in range(F):
            want = torch.topk(x[r, f * P:(f + 1) * P].float(), k).indices.numpy() + f * P
            assert np.array_equal(got[r, f * k:(f + 1) * k], np.sort(want))


def test_global_mode_and_whole_frames():
    F, P = 2, 30
    bits, x = _distinct_bits(3, F * P, 1)
    got = OS.token_topk_from_scores(bits, F, P, 7, per_frame_mode=False)
    for r in range(3):
        assert np.array_equal(got[r], np.sort(torch.topk(x[r].float(), 7).indices.numpy()))
    whole = OS.token_topk_from_scores(bits, F, P, P + 9)  # k >= P: every key of every frame
    assert np.array_equal(whole, np.tile(np.arange(F * P), (3, 1)))


def test_ties_go_to_the_lower_key_and_signed_zeros_order():
    P = 8
    row = np.array([0x3F80] * 5 + [0x0000, 0x8000, 0x4000], dtype=np.uint16)  # 1 x5, +0, -0, 2
    got = OS.token_topk_from_scores(row[None], 1, P, 3)
    assert got.tolist() == [[0, 1, 7]]  # 2.0 first, then the two lowest of the tied ones
    got = OS.token_topk_from_scores(row[None], 1, P, 7)
    assert got.tolist() == [[0, 1, 2, 3, 4, 5, 7]]  # +0.0 beats -0.0


def test_first_frame_samples_and_cap():
    F, P, k = 4, 20, 3
    bits, x = _distinct_bits(2, F * P, 2)
    got = OS.token_topk_from_scores(bits, F, P, k, exclude_first=True, first_stride=6)
    assert got.shape == (2, 4 + 3 * k)
    assert (got[:, :4] == [0, 6, 12, 18]).all() and (got[:, 4:] >= P).all()
    capped = OS.token_topk_from_scores(bits, F, P, k, exclude_first=True, first_stride=6, cap=5)
    for r in range(2):
        cand = got[r, 4:]
        best = cand[np.argsort(-x[r, cand].float().numpy(), kind="stable")[:5]]
        assert np.array_equal(capped[r, 4:], np.sort(best))
        assert np.array_equal(capped[r, :4], [0, 6, 12, 18])


def test_output_width_follows_the_reference_arithmetic(pkg):
    import importlib
    U = importlib.import_module(pkg.__name__ + ".patch.utils")
    assert U.output_width(128 * 1369, 4, True, 1369, 2048, False, 4) == (0, 512, 512)
    assert U.output_width(700 * 1369, 64, True, 1369, 44800, False, 4) == (0, 44800, 44800)
    assert U.output_width(10 * 100, 64, True, 100, 300, True, 4) == (25, 576, 275)
    assert U.output_width(1000, 50, False, 100, 2048, True, 1) == (100, 50, 50)
    with pytest.raises(AssertionError):
        U.output_width(1000, 4, True, 100, 10, True, 1)  # 100 samples exceed max_topk
