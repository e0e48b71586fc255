"""``headprofile``: the offline head profiler that writes the head-profile JSON.

ref: saf3r/patch/wrapper.py:112-205 (BaseSparseAttentionProfiler: per head, every candidate
     configuration against full attention, error = NMSE = mse / (mean(full^2) + 1e-10) accumulated
     over calibration samples), saf3r/patch/patch_vggt.py:225-272 (patching: profiled heads per
     layer from profile_config_path or every head; DINO-feature top-k for the dino_topk candidate),
     :521-566 (save_profile_results: per head the candidate with the lowest mean error, grouped per
     layer, the first dino_topk head marked is_first_dino).

The dino_topk candidate reads the DINO-feature top-k of the forward, which the forward hook installed on
``aggregator.patch_embed`` computes (``patch_vggt.install_feature_topk``), as the reference's rebound
aggregator forward does; it is scored for every profiled head, as in the reference.

Every candidate runs through the same kernels as the sparse model: the profiled heads of a layer
take the candidate's mode together (one sparse-attention launch per candidate), the other heads are
skipped, and the layer returns full attention, as the reference profiler does.
"""
from __future__ import annotations

import json
import math

import numpy as np
import torch
from torch import Tensor, nn

from .. import ops
from ..layout import HEAD_DIM
from .wrapper import BaseHeadwiseSparseAttentionWrapper, _get


def candidate_configs(layer_idx: int, upper_stride: int = 128, lower_stride: int = 4, switch_layer: int = 9):
    """The candidate list of ``profile_attention_cmp_mse`` (``saf3r/patch/wrapper.py:163-190``)."""
    base = upper_stride if int(layer_idx) < switch_layer else lower_stride
    cfgs = [{"mode": "stride", "stride": base, "include_as": True, "is_base": True},
            {"mode": "broadcast_first", "is_base": False},
            {"mode": "all_to_first", "is_base": False},
            {"mode": "global_to_frame", "is_base": False}]
    for mul in range(1, 6):
        cfgs.append({"mode": "stride", "stride": base * (2 ** mul), "is_base": False})
    for mul in range(6):
        cfgs.append({"mode": "q_probe_topk", "stride": base * (2 ** mul), "is_base": False})
    cfgs.append({"mode": "dino_topk", "topk": 32768, "dino_sp2sp_stride": 1, "is_base": False})
    return cfgs


class SparseAttentionProfiler(nn.Module):
    """Replaces ``aggregator.global_blocks.{i}.attn`` under ``patch_module.type = headprofile``."""

    def __init__(self, orig_module, layer_idx: int, heads, num_special_tokens: int, shared, verbose=True,
                 profile_metric="cmp_mse", upper_stride=128, lower_stride=4, switch_layer=9,
                 wrapper_cls=None):
        super().__init__()
        if profile_metric != "cmp_mse":
            raise NotImplementedError(f"profile_metric {profile_metric!r}: only cmp_mse is built")
        self.orig_module = orig_module
        self.layer_idx = layer_idx
        self.num_heads = orig_module.num_heads
        self.heads = sorted(int(h) for h in heads)
        self.verbose = verbose
        self.shared = shared
        self.patch_height = self.patch_width = None
        self.cfgs = candidate_configs(layer_idx, upper_stride, lower_stride, switch_layer)
        self.head_errors = {h: {} for h in self.heads}
        # one sparse wrapper per candidate (the profiled heads in that mode, the rest skipped) and
        # one all-dense wrapper for the reference output
        skip = [h for h in range(self.num_heads) if h not in self.heads]

        def wrapper(groups):
            return wrapper_cls(orig_module, layer_idx=layer_idx, config=groups, shared=shared, lazy_dino_topk=False)

        self.full = wrapper([])
        self.candidates = nn.ModuleList()
        for c in self.cfgs:
            groups = [dict(c, head_ids=list(self.heads))]
            if skip:
                groups.append({"mode": "skip", "head_ids": skip})
            self.candidates.append(wrapper(groups))

    def forward(self, x: Tensor, pos=None) -> Tensor:
        B, N, C = x.shape
        if B != 1:
            raise AssertionError("Currently only support batch size of 1 for simplicity")
        om = self.orig_module
        for w in (self.full, *self.candidates):
            w.patch_height, w.patch_width = self.patch_height, self.patch_width
        geom = self.full.geometry(N)
        qkv = om.qkv(x).reshape(N, 3 * C).to(torch.bfloat16).contiguous()
        p = None if pos is None else pos[0]
        full = self.full.compute_multihead_attention_packed(qkv, p, geom)
        ref = full.float().reshape(N, self.num_heads, HEAD_DIM)
        energy = (ref ** 2).mean(dim=(0, 2)) + 1e-10
        for i, (cfg, w) in enumerate(zip(self.cfgs, self.candidates)):
            if cfg["mode"] == "dino_topk" and self.shared.est_topk_idx is None:
                raise RuntimeError("headprofile scores the dino_topk candidate from DINO-feature indices: run the "
                                   "model through aggregator.patch_embed (the forward hook computes them) or call "
                                   "set_dino_topk_from_features before this layer")
            out = w.compute_multihead_attention_packed(qkv, p, geom).float().reshape(N, self.num_heads, HEAD_DIM)
            mse = ((out - ref) ** 2).mean(dim=(0, 2)) / energy
            for h in self.heads:
                e = float(mse[h])
                rec = self.head_errors[h].setdefault(i, {"cfg": cfg, "mse": []})
                rec["mse"].append(e)
                if self.verbose:
                    print(f"[L{self.layer_idx:>2} | H{h:>2}] config {cfg}, MSE={e:.6f}")
        y = full.reshape(B, N, C)
        if not torch.is_autocast_enabled("cuda") and y.dtype != om.proj.weight.dtype:
            y = y.to(om.proj.weight.dtype)
        return om.proj_drop(om.proj(y))


def profile_results(model, metric: str = "cmp_mse") -> dict:
    """{layer: [cfg with head_ids, ...]}: per head the candidate with the lowest mean error
    (``save_profile_results``, ``saf3r/patch/patch_vggt.py:521-560``)."""
    err_metric = metric.split("_")[-1]
    results = {}
    first_dino = False
    for i, block in enumerate(model.aggregator.global_blocks):
        attn = block.attn
        if not isinstance(attn, SparseAttentionProfiler):
            continue
        layer = {}
        for h, cfgs in attn.head_errors.items():
            best_idx, best_cfg, best = None, None, math.inf
            for idx, rec in cfgs.items():
                m = float(np.mean(rec[err_metric]))
                if m < best:
                    best_idx, best_cfg, best = idx, rec["cfg"], m
            if best_idx is None:
                continue
            if best_idx not in layer:
                best_cfg = dict(best_cfg)
                if best_cfg["mode"] == "dino_topk" and not first_dino:
                    first_dino = True
                    best_cfg["is_first_dino"] = True
                best_cfg["head_ids"] = [h]
                layer[best_idx] = best_cfg
            else:
                layer[best_idx]["head_ids"].append(h)
        results[i] = [c for _, c in layer.items()]
    return results


def save_profile_results(model, save_path: str, metric: str = "cmp_mse") -> dict:
    res = profile_results(model, metric)
    with open(save_path, "w") as f:
        json.dump({str(k): v for k, v in res.items()}, f, indent=4)
    return res


def patch_model_profile(model, model_cfg, wrapper_cls, num_special_tokens: int, num_heads: int, num_layers: int,
                        state):
    """``headprofile`` patching (``saf3r/patch/patch_vggt.py:225-272``)."""
    pm = _get(model_cfg, "patch_module")
    path = _get(model_cfg, "profile_config_path")
    if path:
        with open(path) as f:
            config = json.load(f)
    else:
        config = {str(i): list(range(num_heads)) for i in range(num_layers)}
    blocks = model.aggregator.global_blocks
    for layer_key, heads in config.items():
        i = int(layer_key)
        if i >= len(blocks):
            raise ValueError(f"Failed to get module aggregator.global_blocks.{i}.attn from the model.")
        blocks[i].attn = SparseAttentionProfiler(
            blocks[i].attn, i, heads, num_special_tokens, state, verbose=bool(_get(pm, "verbose", False)),
            profile_metric=_get(pm, "profile_metric", "cmp_mse"), upper_stride=_get(pm, "upper_stride", 128),
            lower_stride=_get(pm, "lower_stride", 4), switch_layer=_get(pm, "switch_layer", 9),
            wrapper_cls=wrapper_cls)
    model.saf3r_selection_state = state
    return model
