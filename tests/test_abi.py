"""CPU-side checks of the C ABI: the library loads, exports exactly what the header declares,
validates arguments before touching a GPU, and reports injected failures."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "saf3r_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(saf3r_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(pkg):
    from importlib import import_module
    lib_mod = import_module(pkg.__name__ + "._lib")
    lib = lib_mod.load()
    names = _declared()
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(lib_mod.EXPORTS)
    assert lib.saf3r_abi_version() == lib_mod.ABI_VERSION == 13


def test_packed_slots_matches_layout(pkg):
    from importlib import import_module
    lib = import_module(pkg.__name__ + "._lib").load()
    for F, T, ns in [(4, 1374, 5), (128, 1374, 5), (3, 155, 5), (2, 64, 0), (96, 1301, 5), (1, 6, 5)]:
        g = pkg.Geometry(F, T, ns)
        assert lib.saf3r_packed_slots(F, T, ns) == g.slots
    assert pkg.Geometry(128, 1374).slots == 640 + 128 * 1408
    assert lib.saf3r_packed_slots(0, 10, 1) == -1
    assert lib.saf3r_packed_slots(2, 5, 5) == -1


def test_invalid_arguments_fail_before_launch(pkg):
    from importlib import import_module
    L = import_module(pkg.__name__ + "._lib")
    lib = L.load()
    pat = (ctypes.c_int32 * 2)(0, 0)
    rc = lib.saf3r_sparse_attn_fwd(None, None, None, 2, 100, 5, 2, pat, None, 0, 0.125, None, 128, None, None, None,
                                   0, None, None, None, None, None, 0, None, 0, None)
    assert rc == 1 and b"null" in lib.saf3r_last_error()
    bad = (ctypes.c_int32 * 1)(10)
    dev = ctypes.c_void_p(16)
    rc = lib.saf3r_sparse_attn_fwd(dev, dev, dev, 2, 100, 5, 1, bad, None, 0, 0.125, dev, 64, None, None, None, 0,
                                   None, None, None, None, None, 0, None, 0, None)
    assert rc == 1 and b"unknown pattern" in lib.saf3r_last_error()
    ks = (ctypes.c_int32 * 1)(7)  # KEYSET without its buffers
    rc = lib.saf3r_sparse_attn_fwd(dev, dev, dev, 2, 100, 5, 1, ks, None, 0, 0.125, dev, 64, None, None, None, 0,
                                   None, None, None, None, None, 0, None, 0, None)
    assert rc == 1 and b"key-set" in lib.saf3r_last_error()
    tks = (ctypes.c_int32 * 1)(9)  # strided dino special rows without the key-set buffers
    rc = lib.saf3r_sparse_attn_fwd(dev, dev, dev, 2, 100, 5, 1, tks, None, 0, 0.125, dev, 64, None, None, None, 0,
                                   None, None, None, None, None, 0, None, 0, None)
    assert rc == 1 and b"key-set" in lib.saf3r_last_error()
    rc = lib.saf3r_sparse_attn_fwd(dev, dev, dev, 2, 100, 5, 1, ks, None, 0, 0.125, dev, 64, dev, dev, dev, 100,
                                   None, None, None, None, None, 0, None, 0, None)
    assert rc == 1 and b"multiple of 64" in lib.saf3r_last_error()
    bc = (ctypes.c_int32 * 1)(8)  # BROADCAST without its buffers
    rc = lib.saf3r_sparse_attn_fwd(dev, dev, dev, 2, 100, 5, 1, bc, None, 0, 0.125, dev, 64, None, None, None, 0,
                                   None, dev, dev, None, None, 0, None, 0, None)
    assert rc == 1 and b"BROADCAST" in lib.saf3r_last_error()
    fl = (ctypes.c_int32 * 1)(1)  # token order on a FRAME_LOCAL head
    tord = (ctypes.c_uint8 * 1)(1)
    rc = lib.saf3r_sparse_attn_fwd(dev, dev, dev, 2, 100, 5, 1, fl, None, 0, 0.125, dev, 64, None, None, None, 0,
                                   None, None, None, tord, None, 0, None, 0, None)
    assert rc == 1 and b"only DENSE" in lib.saf3r_last_error()
    dn = (ctypes.c_int32 * 1)(0)
    framed = (ctypes.c_uint8 * 1)(2)  # the framed layout on a DENSE head
    rc = lib.saf3r_sparse_attn_fwd(dev, dev, dev, 2, 100, 5, 1, dn, None, 0, 0.125, dev, 64, None, None, None, 0,
                                   None, None, None, framed, None, 0, None, 0, None)
    assert rc == 1 and b"framed layout" in lib.saf3r_last_error()
    # the framed layout where the special tokens do not fit a frame's last patch tile (P = 64, ns = 5)
    rc = lib.saf3r_sparse_attn_fwd(dev, dev, dev, 2, 69, 5, 1, fl, None, 0, 0.125, dev, 64, None, None, None, 0,
                                   None, None, None, framed, None, 0, None, 0, None)
    assert rc == 2 and b"does not fit" in lib.saf3r_last_error()
    rc = lib.saf3r_sparse_attn_fwd(dev, dev, dev, 2, 100, 5, 1, fl, None, 0, 0.125, dev, 64, None, None, None, 0,
                                   None, None, None, (ctypes.c_uint8 * 1)(3), None, 0, None, 0, None)
    assert rc == 1 and b"unknown layout" in lib.saf3r_last_error()
    rc = lib.saf3r_sparse_attn_fwd(dev, dev, dev, 2, 100, 5, 1, dn, None, 0, 0.125, dev, 64, None, None, None, 0,
                                   None, None, None, None, None, 6, None, 0, None)
    assert rc == 1 and b"unknown flags" in lib.saf3r_last_error()
    rc = lib.saf3r_sparse_attn_fwd(dev, dev, dev, 2, 100, 5, 1, dn, None, 0, 0.125, dev, 64, None, None, None, 0,
                                   None, None, None, None, None, 0, ctypes.c_void_p(20), 0, None)
    assert rc == 1 and b"8-byte" in lib.saf3r_last_error()
    rc = lib.saf3r_keyset_build(None, 0, 1, dev, dev, dev, dev, 2, 100, 5, dev, 50, dev, None)
    assert rc == 1 and b"idx_stride" in lib.saf3r_last_error()
    rc = lib.saf3r_keyset_gather(dev, 2, 100, 5, dev, 1, dev, 3072, 64, dev, 200, dev, 3, dev, dev, 128, None)
    assert rc == 1 and b"max_tiles" in lib.saf3r_last_error()
    rc = lib.saf3r_frame_topk_scores(dev, 50, 2, 2, 30, 0, 0, 1, 4, 0, dev, 8, None, None, None)
    assert rc == 1 and b"score stride" in lib.saf3r_last_error()
    rc = lib.saf3r_frame_topk_scores(dev, 64, 2, 2, 30, 0, 0, 1, 4, 0, dev, 7, None, None, None)
    assert rc == 1 and b"idx_stride" in lib.saf3r_last_error()
    rc = lib.saf3r_frame_topk_scores(dev, 60, 2, 2, 30, 0, 0, 1, 4, 0, dev, 8, None, None, None)
    assert rc == 1 and b"16-byte" in lib.saf3r_last_error()
    rc = lib.saf3r_frame_topk_scores(dev, 64, 2, 2, 30, 0, 0, 1, 4, 5, dev, 8, None, None, None)
    assert rc == 1 and b"candidate" in lib.saf3r_last_error()
    rc = lib.saf3r_frame_topk_scores(dev, 9000, 2, 2, 4500, 0, 0, 1, 4, 0, dev, 8, None, None, None)
    assert rc == 2  # frames beyond 4096 keys
    rc = lib.saf3r_probe_scores(dev, dev, 200 * 64, 200, dev, 1, None, 0, 0.125, dev, dev, dev, 10, None)
    assert rc == 1 and b"scores_stride" in lib.saf3r_last_error()
    rc = lib.saf3r_probe_scores(dev, dev, 100 * 64, 200, dev, 1, None, 0, 0.125, dev, dev, dev, 200, None)
    assert rc == 1 and b"slot_stride" in lib.saf3r_last_error()
    rc = lib.saf3r_probe_scores(dev, dev, 200 * 64, 200, dev, 1, dev, 201, 0.125, dev, dev, dev, 200, None)
    assert rc == 1 and b"n_samples" in lib.saf3r_last_error()
    rc = lib.saf3r_probe_scores(dev, dev, 200 * 64, 200, dev, 1, None, 0, 0.125, None, dev, dev, 200, None)
    assert rc == 1 and b"workspace" in lib.saf3r_last_error()
    rc = lib.saf3r_probe_scores_noalloc(dev, dev, 200 * 64, 200, dev, 65, None, 0, 0.125, dev, dev, 200, None)
    assert rc == 2 and b"static workspace" in lib.saf3r_last_error()
    rows = L.Rows(16, 64, 0, 1 << 40, 0)
    rc = lib.saf3r_gather_attn_fwd(ctypes.byref(rows), ctypes.byref(rows), ctypes.byref(rows), dev, 4, 1, 4, 10, 0.125,
                                   8, ctypes.byref(rows), None)
    assert rc == 1 and b"dtype flags" in lib.saf3r_last_error()
    # fp32 V / out rows (dtype flags 2 and 4) need a row stride % 4
    rc = lib.saf3r_gather_attn_fwd(ctypes.byref(rows), ctypes.byref(rows), ctypes.byref(rows6 := L.Rows(16, 6, 0, 1 << 40, 0)),
                                   dev, 4, 1, 4, 10, 0.125, 2, ctypes.byref(rows), None)
    assert rc == 1 and b"v must be" in lib.saf3r_last_error()
    rc = lib.saf3r_gather_attn_fwd(ctypes.byref(rows), ctypes.byref(rows), ctypes.byref(rows), dev, 4, 1, 4, 10, 0.125,
                                   4, ctypes.byref(rows6), None)
    assert rc == 1 and b"out must be" in lib.saf3r_last_error()
    rows6 = L.Rows(16, 6, 0, 1 << 40, 0)  # fp32 rows need a row stride % 4, bf16 rows % 8
    rc = lib.saf3r_gather_attn_fwd(ctypes.byref(rows6), ctypes.byref(rows6), ctypes.byref(rows), dev, 4, 1, 4, 10,
                                   0.125, 1, ctypes.byref(rows), None)
    assert rc == 1 and b"row stride % 4" in lib.saf3r_last_error()
    rc = lib.saf3r_block_select(ctypes.c_void_p(16), ctypes.c_void_p(16), 1, 4, 2, 2, 33, 0, ctypes.c_void_p(16), None)
    assert rc == 2  # k beyond the supported range
    # token top-k above k = 16 takes the caller's workspace: none, or one too small for 128 queries, fails
    krows = L.Rows(16, 64, 0, 1 << 40, 0)
    rc = lib.saf3r_token_topk(ctypes.byref(krows), ctypes.byref(krows), 100, 2, 50, 32, dev, None, 0, None)
    assert rc == 1 and b"workspace" in lib.saf3r_last_error()
    rc = lib.saf3r_token_topk(ctypes.byref(krows), ctypes.byref(krows), 100, 2, 50, 32, dev, dev, 2 * 64 * 4 * 127,
                              None)
    assert rc == 1 and b"at least 65536 bytes" in lib.saf3r_last_error()
    rc = lib.saf3r_token_topk(ctypes.byref(krows), ctypes.byref(krows), 100, 2, 50, 32, dev, dev, -1, None)
    assert rc == 1 and b"negative" in lib.saf3r_last_error()
    rc = lib.saf3r_token_topk(ctypes.byref(krows), ctypes.byref(krows), 100, 2, 200, 129, dev, None, 0, None)
    assert rc == 2 and b"128" in lib.saf3r_last_error()
    rc = lib.saf3r_pack_qkv(None, None, None, 64, 64, 0, 10, 1, 1, None, None, None, None, 1e-5, 0, None, None,
                            None, 0, None, None, None, None, None, None, None, 1.0, None, None, None, None, None)
    assert rc == 1 and b"geometry" in lib.saf3r_last_error()
    flags = (ctypes.c_uint8 * 65)(*([0] * 64 + [1]))  # token order beyond head 63
    rc = lib.saf3r_pack_qkv(dev, dev, dev, 64, 64, 2, 100, 5, 65, None, None, None, None, 1e-5, 0, None, None,
                            None, 0, dev, dev, dev, flags, None, None, None, 1.0, None, None, None, None, None)
    assert rc == 2 and b"token order" in lib.saf3r_last_error()
    rc = lib.saf3r_pack_qkv(dev, dev, dev, 64, 64, 2, 69, 5, 1, None, None, None, None, 1e-5, 0, None, None,
                            None, 0, dev, dev, dev, framed, None, None, None, 1.0, None, None, None, None, None)
    assert rc == 2 and b"framed layout" in lib.saf3r_last_error()
    rc = lib.saf3r_pack_qkv(dev, dev, dev, 64, 64, 2, 100, 5, 1, None, None, None, None, 1e-5, 0, None, None,
                            None, 0, dev, dev, dev, (ctypes.c_uint8 * 1)(7), None, None, None, 1.0, None, None, None, None, None)
    assert rc == 1 and b"unknown layout" in lib.saf3r_last_error()
    rc = lib.saf3r_pack_qkv(dev, dev, dev, 64, 64, 2, 100, 5, 65, None, None, None, None, 1e-5, 0, None, None,
                            None, 0, dev, dev, dev, None, flags, dev, None, 1.0, None, None, None, None, None)
    assert rc == 2 and b"fp32 rows" in lib.saf3r_last_error()
    one = (ctypes.c_uint8 * 2)(0, 1)
    rc = lib.saf3r_pack_qkv(dev, dev, dev, 64, 64, 2, 100, 5, 2, None, None, None, None, 1e-5, 0, None, None,
                            None, 0, dev, dev, dev, None, one, None, None, 1.0, None, None, None, None, None)
    assert rc == 1 and b"qk32" in lib.saf3r_last_error()
    rc = lib.saf3r_pack_qkv(dev, dev, dev, 64, 64, 2, 100, 5, 65, None, None, None, None, 1e-5, 0, None, None,
                            None, 0, dev, dev, dev, None, None, None, flags, 0.18, None, None, None, None, None)
    assert rc == 2 and b"scaled Q" in lib.saf3r_last_error()
    for bad_scale in (0.0, -1.0, float("inf")):
        rc = lib.saf3r_pack_qkv(dev, dev, dev, 64, 64, 2, 100, 5, 2, None, None, None, None, 1e-5, 0, None, None,
                                None, 0, dev, dev, dev, None, None, None, one, bad_scale, None, None, None, None, None)
        assert rc == 1 and b"q_scale" in lib.saf3r_last_error()
    one_pool = (ctypes.c_uint8 * 2)(1, 0)
    rc = lib.saf3r_pack_qkv(dev, dev, dev, 64, 64, 2, 100, 5, 2, None, None, None, None, 1e-5, 0, None, None,
                            None, 0, dev, dev, dev, (ctypes.c_uint8 * 2)(1, 0), None, None, None, 1.0, one_pool,
                            dev, dev, dev, None)
    assert rc == 1 and b"packed layout" in lib.saf3r_last_error()  # a pooled head in token order
    rc = lib.saf3r_pack_qkv(dev, dev, dev, 64, 64, 2, 100, 5, 2, None, None, None, None, 1e-5, 0, None, None,
                            None, 0, dev, dev, dev, None, None, None, None, 1.0, one_pool, dev, None, dev, None)
    assert rc == 1 and b"pool_mean" in lib.saf3r_last_error()
    rc = lib.saf3r_pooled_prepare(dev, 10, ctypes.c_void_p(24), dev, None)
    assert rc == 1 and b"16-byte" in lib.saf3r_last_error()
    rc = lib.saf3r_pooled_prepare(dev, -1, dev, dev, None)
    assert rc == 1
    rc = lib.saf3r_block_select_pooled(dev, dev, dev, 1, 4, 33, 4, dev, None, 0, None)
    assert rc == 2 and b"32 blocks" in lib.saf3r_last_error()
    rc = lib.saf3r_block_select_pooled(dev, dev, dev, 1, 4, 22, 33, dev, None, 0, None)
    assert rc == 2 and b"k must be" in lib.saf3r_last_error()
    rc = lib.saf3r_block_select_pooled(dev, None, dev, 1, 4, 22, 4, dev, None, 0, None)
    assert rc == 1 and b"null" in lib.saf3r_last_error()
    assert lib.saf3r_block_select_pooled_workspace_bytes(7, 128, 22, 4) == 0  # the selection needs no workspace
    assert lib.saf3r_block_select_pooled_workspace_bytes(1, 4, 22, 20) == 0  # k > 16: the sequential kernel
    assert lib.saf3r_block_select_pooled_workspace_bytes(1, 4, 33, 4) == -1
    with pytest.raises(L.Saf3rError):
        L.check(1)


def test_token_topk_workspace_size_query(pkg):
    """The score workspace of the top-k > 16 path: rows of frames x roundup(per_frame, 64) fp32
    scores for whole work-groups of 128 queries, at most 1 GiB (one chunk), 0 for top-k <= 16."""
    from importlib import import_module
    lib = import_module(pkg.__name__ + "._lib").load()
    ws = lib.saf3r_token_topk_workspace_bytes
    row = 128 * 1408 * 4  # 128 frames x 1369 patches, padded to 1408
    assert ws(175232, 128, 1369, 4) == 0
    assert ws(175232, 128, 1369, 16) == 0
    assert ws(175232, 128, 1369, 17) == (2 ** 30 // row // 128 * 128) * row == 1408 * row
    assert ws(175232, 128, 1369, 17) <= 2 ** 30
    assert ws(100, 2, 50, 32) == 128 * 2 * 64 * 4  # min(32, 50) > 16: one work-group of 128 queries
    assert ws(100, 2, 10, 32) == 0  # min(32, 10) = 10 <= 16
    assert ws(300, 3, 100, 64) == 384 * 3 * 128 * 4
    assert ws(0, 3, 100, 64) == 0
    assert ws(100, 2, 200, 129) == -1  # beyond the reference's limit of 128
    assert ws(100, 2, 5000, 32) == -1  # frames above 4096 keys on the k > 16 path
    assert ws(-1, 2, 50, 4) == -1


def test_gather_workspace_size_query(pkg):
    from importlib import import_module
    lib = import_module(pkg.__name__ + "._lib").load()
    assert lib.saf3r_gather_attn_workspace_bytes(175232, 512) == 65536 * 8 * 66 * 4  # one chunk: 8 slices x 66 floats
    assert lib.saf3r_gather_attn_workspace_bytes(1000, 512) == 1000 * 8 * 66 * 4
    assert lib.saf3r_gather_attn_workspace_bytes(0, 512) == 0
    assert lib.saf3r_gather_attn_workspace_bytes(-1, 512) == -1
    assert lib.saf3r_gather_attn_workspace_bytes(10, 0) == -1


def test_fault_injection_is_reported(pkg, monkeypatch):
    from importlib import import_module
    lib = import_module(pkg.__name__ + "._lib").load()
    monkeypatch.setenv("SAF3R_FAULT_INJECT", "saf3r_block_select")
    rc = lib.saf3r_block_select(None, None, 1, 1, 1, 1, 1, 0, None, None)
    assert rc == 4 and b"injected" in lib.saf3r_last_error()
    monkeypatch.setenv("SAF3R_FAULT_INJECT", "")
    rc = lib.saf3r_block_select(None, None, 1, 1, 1, 1, 1, 0, None, None)
    assert rc == 1


def test_geometry_derived_sizes(pkg):
    g = pkg.Geometry(128, 1374, 5)
    assert (g.patches, g.blocks_per_frame, g.num_blocks, g.tokens) == (1369, 22, 2816, 175872)
    # framed layout: 22 tiles per frame (25 patches + 5 specials in the last), inside the 2826 packed tiles
    assert (g.frame_tiles, g.framed_fits, g.tiles) == (22, True, 2826)
    assert pkg.Geometry(2, 69, 5).framed_fits is False  # 64 patches fill their tile: no room for the specials
    assert pkg.Geometry(3, 64, 0).framed_fits is True
    assert pkg.Geometry(96, 1301, 5).framed_fits is True  # DA3 504^2: 1296 % 64 = 16, + 5
    g5 = pkg.Geometry(96, 1301, 5)
    assert (g5.blocks_per_frame, g5.num_blocks, g5.tokens) == (21, 2016, 124896)
    with pytest.raises(ValueError):
        pkg.Geometry.from_tokens(100, 30)


def test_kernel_binding_validates_before_any_gpu_call(pkg):
    """The reference-signature binding raises ValueError for CPU tensors and malformed shapes."""
    from importlib import import_module
    import torch
    kb = import_module(pkg.__name__ + ".kernel_binding")
    q = torch.randn(4, 64)
    with pytest.raises(ValueError, match="GPU"):
        kb.fused_sparse_topk_attention(q, q, q, torch.zeros(4, 2, dtype=torch.int32))
    with pytest.raises(ValueError, match="num_toks_per_img"):
        kb.compute_qk_topk_indices_fused(q[None], q[None], 2, None)
    with pytest.raises(ValueError, match="agree"):
        kb.compute_qk_topk_indices_fused(q[None], q[None].expand(2, 4, 64), 2, 2)
    with pytest.raises(ValueError, match="GPU"):
        kb.compute_qk_topk_indices_fused(q[None], q[None], 2, 2)
