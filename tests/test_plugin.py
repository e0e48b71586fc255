"""CPU checks of the plugin surface: config parsing, module replacement, per-forward geometry, and
the error behaviour the reference defines (duplicate head, unknown mode, batch size, model name)."""
import json
import os
from types import SimpleNamespace

import pytest
import torch

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def plug(pkg):
    import importlib
    return importlib.import_module(pkg.__name__ + ".patch")


@pytest.fixture(scope="module")
def vggt(pkg):
    import importlib
    return importlib.import_module(pkg.__name__ + ".vggt")


def _model(vggt, depth=3, dim=64, heads=4):
    return vggt.GlobalAttentionStack(depth=depth, dim=dim, num_heads=heads)


def test_head_cfg_defaults_and_groups(plug, vggt, pkg):
    import importlib
    ops = importlib.import_module(pkg.__name__ + ".ops")
    m = _model(vggt, depth=2, dim=256, heads=4)
    cfg = {"patch_module": {"type": "headsparse", "topk_mode": "token", "lazy_dino_topk": True, "topk": 4},
           "sparse_config": {"0": [{"mode": "global_to_frame", "head_ids": [1]},
                                   {"mode": "block_topk", "head_ids": [2, 3], "topk": 8}],
                             "1": [{"mode": "all_to_first", "head_ids": [0]}]}}
    group = cfg["sparse_config"]["0"][0]
    plug.patch_model(m, "vggt", cfg)
    w0 = m.aggregator.global_blocks[0].attn
    assert isinstance(w0, plug.HeadwiseSparseAttentionWrapper)
    assert [c["mode"] for c in w0.head_cfg] == ["full", "global_to_frame", "block_topk", "block_topk"]
    assert w0.patterns == [ops.DENSE, ops.FRAME_LOCAL, ops.BLOCK_DYNAMIC, ops.BLOCK_DYNAMIC]
    assert w0.layer_block_topk == 8 and w0.dyn_heads == [2, 3]
    assert "head_ids" in group  # the caller's config is not mutated
    w1 = m.aggregator.global_blocks[1].attn
    assert w1.patterns == [ops.ANCHOR, ops.DENSE, ops.DENSE, ops.DENSE]
    assert w1.shared is w0.shared is m.saf3r_selection_state


def test_errors_follow_reference(plug, vggt):
    m = _model(vggt)
    dup = {"patch_module": {"type": "headsparse"},
           "sparse_config": {"0": [{"mode": "skip", "head_ids": [1]}, {"mode": "all_to_first", "head_ids": [1]}]}}
    with pytest.raises(ValueError, match="multiple"):
        plug.patch_model(m, "vggt", dup)
    bad = {"patch_module": {"type": "headsparse"}, "sparse_config": {"0": [{"mode": "bogus", "head_ids": [0]}]}}
    with pytest.raises(ValueError, match="Unsupported mode"):
        plug.patch_model(_model(vggt), "vggt", bad)
    with pytest.raises(ValueError, match="Unsupported model"):
        plug.patch_model(_model(vggt), "pi3x", bad)
    with pytest.raises(NotImplementedError):
        plug.patch_model(_model(vggt), "vggt", {"patch_module": {"type": "headcache"}, "sparse_config": {}})
    with pytest.raises(AssertionError):
        plug.patch_model(_model(vggt), "vggt", {"patch_module": {"type": "headsparse", "topk_mode": "global"},
                                               "sparse_config": {"0": [{"mode": "dino_topk", "head_ids": [0]}]}})


def test_update_args_per_forward_sets_geometry(plug, vggt):
    m = _model(vggt, depth=2, dim=256, heads=4)
    cfg = {"patch_module": {"type": "headsparse", "lazy_dino_topk": True, "topk": 4},
           "sparse_config": {"0": [{"mode": "dino_topk", "head_ids": [0], "is_first_dino": True}], "1": []}}
    plug.patch_model(m, "vggt", cfg)
    w = m.aggregator.global_blocks[0].attn
    w.first_dino_flag = True
    m.saf3r_selection_state.est_topk_idx = torch.zeros(1)
    plug.update_args_per_forward(m, "vggt", 518, 518)
    for b in m.aggregator.global_blocks:
        assert b.attn.patch_height == b.attn.patch_width == 37
        assert b.attn.first_dino_flag is False
    assert m.saf3r_selection_state.est_topk_idx is None
    g = w.geometry(4 * 1374)
    assert (g.frames, g.tokens_per_frame, g.patches) == (4, 1374, 1369)
    with pytest.raises(ValueError):
        w.geometry(1000)


def test_wrapper_refuses_cpu_and_batches(plug, vggt):
    m = _model(vggt, depth=1, dim=256, heads=4)
    plug.patch_model(m, "vggt", {"patch_module": {"type": "headsparse"}, "sparse_config": {"0": []}})
    plug.update_args_per_forward(m, "vggt", 28, 28)
    w = m.aggregator.global_blocks[0].attn
    with pytest.raises(AssertionError):
        w(torch.randn(2, 18, 256))
    with pytest.raises(RuntimeError, match="GPU"):
        w(torch.randn(1, 18, 256))


def test_reference_vggt_profile_fixture(plug, vggt):
    """The reference's VGGT head profile (24 layers x 16 heads, each head exactly once)."""
    with open(os.path.join(GOLDEN, "vggt_eth3d_profile.json")) as f:
        prof = json.load(f)
    assert set(prof) == {str(i) for i in range(24)}
    for groups in prof.values():
        assert sorted(h for g in groups for h in g["head_ids"]) == list(range(16))
    firsts = [(k, g["head_ids"]) for k, gs in prof.items() for g in gs if g.get("is_first_dino")]
    assert firsts == [("11", [14])]
    # the whole profile patches: every mode it uses has a kernel
    m = _model(vggt, depth=24, dim=1024, heads=16)
    plug.patch_model(m, "vggt", {"patch_module": {"type": "headsparse", "topk_mode": "token",
                                                  "lazy_dino_topk": True, "topk": 4}, "sparse_config": prof})
    wrappers = [b.attn for b in m.aggregator.global_blocks]
    assert sum(len(w.keyset_heads) for w in wrappers) == 212 + 75
    assert [w.layer_idx for w in wrappers if w.first_dino_head is not None] == [11]
    # key sets of the profile's groups at the 128-frame shape
    from importlib import import_module
    spa = import_module(plug.__name__ + ".sparse_attention")
    ops = import_module(plug.__name__.rsplit(".", 1)[0] + ".ops")
    n = 128 * 1374
    s4 = spa.keyset_spec({"mode": "stride", "stride": 4, "include_as": True, "is_base": True}, 3, n)
    assert (s4.mode, s4.param, s4.start, s4.include) == (ops.KEYSET_STRIDE, 4, 0, True)
    qp = spa.keyset_spec({"mode": "q_probe_topk", "stride": 4, "is_base": False}, 5, n)
    assert (qp.mode, qp.param, qp.include) == (ops.KEYSET_TOPK, n // 4, False)
    assert spa.keyset_spec({"mode": "q_probe_topk"}, 0, n).param == 1024
    assert spa.keyset_spec({"mode": "stride", "stride": 3, "shift": True}, 7, n).start == 1
    assert spa.keyset_spec({"mode": "q_probe_topk", "q_sample_ratio": 0.5}, 0, n).sample_ratio == 0.5
    # q_sample_ratio < 1: the reference's linspace rows (sparse_attention.py:154-157)
    rows = ops.probe_sample(1000, 0.1)
    assert rows.tolist() == torch.linspace(0, 999, steps=100).long().tolist() and rows[0] == 0 and rows[-1] == 999
    assert ops.probe_sample(1000, 1) is None and ops.probe_sample(5, 0.01).tolist() == [0]
    # dino_topk with dino_sp2sp_stride != 1: special rows over keys 0, s, 2s, ... (:199-204)
    sd = spa.keyset_spec({"mode": "dino_topk", "dino_sp2sp_stride": 3}, 2, n)
    assert (sd.mode, sd.param, sd.start, sd.include) == (ops.KEYSET_STRIDE, 3, 0, False)
    assert spa.pattern_of({"mode": "dino_topk", "dino_sp2sp_stride": 3}) == ops.TOKEN_DYNAMIC_KEYSET
    assert spa.pattern_of({"mode": "dino_topk", "dino_sp2sp_stride": 1}) == ops.TOKEN_DYNAMIC
    m = _model(vggt, depth=1, dim=128, heads=2)
    plug.patch_model(m, "vggt", {"patch_module": {"type": "headsparse"},
                                 "sparse_config": {"0": [{"mode": "broadcast_first", "head_ids": [0]}]}})
    w = m.aggregator.global_blocks[0].attn
    assert w.patterns == [ops.BROADCAST, ops.DENSE] and w.broadcast_heads == [0]


def test_headprofile_candidates_and_json(plug, vggt, pkg, tmp_path):
    """headprofile patching and the JSON writer (saf3r/patch/wrapper.py:163-190,
    saf3r/patch/patch_vggt.py:521-566): candidate list per layer, lowest mean error per head,
    heads grouped per chosen candidate, the first dino_topk head marked."""
    import importlib
    prof = importlib.import_module(plug.__name__ + ".profiler")
    c3 = prof.candidate_configs(3)
    c12 = prof.candidate_configs(12)
    assert len(c3) == 16 and c3[0] == {"mode": "stride", "stride": 128, "include_as": True, "is_base": True}
    assert c12[0]["stride"] == 4 and [c["stride"] for c in c12[4:9]] == [8, 16, 32, 64, 128]
    assert [c["stride"] for c in c12[9:15]] == [4, 8, 16, 32, 64, 128] and c12[15]["mode"] == "dino_topk"
    m = _model(vggt, depth=2, dim=256, heads=4)
    plug.patch_model(m, "vggt", {"patch_module": {"type": "headprofile"}})
    p0, p1 = (b.attn for b in m.aggregator.global_blocks)
    assert isinstance(p0, plug.SparseAttentionProfiler) and p0.heads == [0, 1, 2, 3]
    plug.update_args_per_forward(m, "vggt", 28, 42)
    assert (p0.patch_height, p0.patch_width) == (2, 3)
    # synthetic errors over two samples: head -> candidate -> [e1, e2]
    errs = {0: {2: [0.1, 0.3], 5: [0.2, 0.1]}, 1: {15: [0.01, 0.02], 2: [0.5, 0.5]},
            2: {5: [0.05, 0.1], 15: [0.2, 0.2]}, 3: {2: [0.0, 0.1], 15: [0.3, 0.3]}}
    for h, d in errs.items():
        p0.head_errors[h] = {i: {"cfg": p0.cfgs[i], "mse": v} for i, v in d.items()}
    p1.head_errors = {1: {15: {"cfg": p1.cfgs[15], "mse": [0.0]}}}
    res = plug.save_profile_results(m, str(tmp_path / "prof.json"), "cmp_mse")
    import json
    saved = json.load(open(tmp_path / "prof.json"))
    assert set(saved) == {"0", "1"}
    by_mode = {c["mode"]: c for c in saved["0"]}
    assert by_mode["stride"]["head_ids"] == [0, 2] and by_mode["stride"]["stride"] == 4 * 128
    assert by_mode["dino_topk"]["head_ids"] == [1] and by_mode["dino_topk"]["is_first_dino"] is True
    assert by_mode["all_to_first"]["head_ids"] == [3]
    assert saved["1"] == [dict(p1.cfgs[15], head_ids=[1])]  # only the first dino head is marked
    assert res[0] == saved["0"]

