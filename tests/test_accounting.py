"""The work accounting behind the bench's TFLOP/s and GB/s figures (CPU only): allowed-pair counts
against the oracle's masks counted element by element, the closed forms of the patterns without a
mask form, the executed-tile count against the algorithmic one, and the selection path's bytes at
the bench's shape."""
import pytest
import torch

from oracle import attention as OA


@pytest.fixture(scope="module")
def acc(pkg):
    from importlib import import_module
    return import_module(pkg.__name__ + ".accounting")


@pytest.fixture(scope="module")
def ops(pkg):
    from importlib import import_module
    return import_module(pkg.__name__ + ".ops")


GEOMS = [(3, 155, 5), (2, 64, 0), (4, 70, 5)]


def _mask_pairs(pattern, og, sel=None):
    rows = torch.arange(og.tokens)
    return int(OA.allowed_mask(pattern, rows, og, sel).sum())


@pytest.mark.parametrize("F,T,ns", GEOMS)
def test_pattern_pairs_match_the_oracle_masks(acc, ops, pkg, F, T, ns):
    g, og = pkg.Geometry(F, T, ns), OA.Geometry(F, T, ns)
    for p in (ops.DENSE, ops.FRAME_LOCAL, ops.ANCHOR_LOCAL, ops.ANCHOR):
        assert acc.head_pairs(p, g) == _mask_pairs(p, og), p
    assert acc.head_pairs(ops.SKIP, g) == 0
    # a key set: every query attends the same members
    members = torch.arange(0, og.tokens, 3)
    assert acc.head_pairs(ops.KEYSET, g, keyset_count=len(members)) == _mask_pairs(ops.KEYSET, og, members)


@pytest.mark.parametrize("F,T,ns", GEOMS)
def test_block_dynamic_pairs_match_the_oracle_mask(acc, ops, pkg, F, T, ns):
    """Listed blocks of different populations (the last block of a frame is partial), empty slots,
    and repeated frames: the pair count is the mask's."""
    g, og = pkg.Geometry(F, T, ns), OA.Geometry(F, T, ns)
    nbf = og.blocks_per_frame
    gen = torch.Generator().manual_seed(F * T)
    W = F * min(2, nbf)
    sel = torch.stack([torch.cat([torch.randperm(nbf, generator=gen)[:min(2, nbf)] + f * nbf for f in range(F)])
                       for _ in range(F * nbf)]).int()
    sel[0, 0] = -1  # an empty slot
    assert sel.shape == (F * nbf, W)
    assert acc.head_pairs(ops.BLOCK_DYNAMIC, g, sel) == _mask_pairs(ops.BLOCK_DYNAMIC, og, sel)


def test_closed_forms(acc, ops, pkg):
    g = pkg.Geometry(5, 37, 5)
    N, F, T, S, P, d = g.tokens, 5, 37, 25, 32, 64
    # dino_topk: special rows dense, each patch row over its listed keys (with multiplicity)
    assert acc.head_pairs(ops.TOKEN_DYNAMIC, g, topk_width=F * 4) == S * N + F * P * F * 4
    assert acc.head_pairs(ops.TOKEN_DYNAMIC_KEYSET, g, topk_width=8, keyset_count=11) == S * 11 + F * P * 8
    # broadcast_first: frame 0's scores once, the map applied to every frame's values
    assert acc.head_flops(ops.BROADCAST, g) == 2 * d * T * T + 2 * d * F * T * T
    assert acc.head_flops(ops.DENSE, g) == 4 * d * N * N
    # qkv (dim -> 3 dim) and proj (dim -> dim), 2 FLOP per multiply-add
    assert acc.projection_flops(N, 1024) == 2 * N * 1024 * 3 * 1024 + 2 * N * 1024 * 1024


@pytest.mark.parametrize("F,T,ns", GEOMS)
def test_executed_tiles_cover_the_algorithmic_work(acc, ops, pkg, F, T, ns):
    """Padding and masking only add work: the executed 64 x 64 tile FLOP bound the algorithmic FLOP of
    every pattern, and a token-order dense head runs exactly ceil(N / 64)^2 tiles."""
    g = pkg.Geometry(F, T, ns)
    nbf = g.blocks_per_frame
    sel = torch.stack([torch.arange(F) * nbf for _ in range(F * nbf)]).int()  # each frame's first block
    pats = [ops.DENSE, ops.FRAME_LOCAL, ops.ANCHOR_LOCAL, ops.ANCHOR, ops.BLOCK_DYNAMIC]
    for h, p in enumerate(pats):
        s = sel[None] if p == ops.BLOCK_DYNAMIC else None
        alg = acc.attention_flops([p], g, s)
        exe = acc.executed_tile_flops([p], g, s)
        assert exe >= alg > 0, p
    ntt = -(-g.tokens // 64)
    assert acc.executed_tile_flops([ops.DENSE], g, token_order=[1]) == 4 * 64 * 64 * 64 * ntt * ntt


def test_selection_bytes_at_the_bench_shape(acc, pkg):
    """The fused selection path's algorithmic bytes at 128 frames x 1374 tokens, 7 block-top-4 heads:
    read Q and K of the heads (bf16, 128 B per token each), write the int32 lists (128 frames x 4
    entries per query block)."""
    g = pkg.Geometry(128, 1374, 5)
    b = acc.selection_bytes(g, 7, 128 * 4)
    assert b["fused_path"] == 7 * (2 * 175872 * 128 + 128 * 22 * 512 * 4) == 355532800
