"""VGGT plugin: ``headsparse`` patching of the global attention layers.

ref: saf3r/patch/patch_vggt.py:178-222 (headsparse branch: read the sparse-config JSON, require
     topk_mode == "token" when a dino_topk head exists, choose lazy / precomputed top-k, replace
     ``aggregator.global_blocks.{i}.attn``), :274-310 (update_args_per_forward: patch grid from
     the image size, reset of the lazy flag), :571-590 (HeadwiseSparseAttentionWrapper.forward).

Configuration (plain dict or attribute object, as the reference's addict ``model_cfg``):
    sparse_config_path | sparse_config     JSON path or the parsed {layer: [group, ...]} mapping
    patch_module.type                      "headsparse"
    patch_module.topk_mode                 "token" (required when a dino_topk head exists)
    patch_module.lazy_dino_topk            indices from the first correspondence head (True), or
                                           from DINO patch features each forward (False): a forward
                                           hook on ``aggregator.patch_embed`` runs
                                           ``set_dino_topk_from_features`` with per_frame_topk,
                                           max_topk, include_first_frame, first_frame_stride
    patch_module.topk                      per-frame token top-k of dino_topk heads
    patch_module.block_topk                per-frame block top-k of block_topk heads (default 4)
    patch_module.topk_scope                "frame" (default) or "global" for block_topk heads
The lazy indices are shared through one ``SelectionState`` per model instead of rebinding the
aggregator forward: every dino_topk layer after the one holding the first correspondence head
reads them, exactly the layers the reference copies them to. The non-lazy indices (and the DINO
candidate of ``headprofile``) come from a forward hook on the aggregator's patch embedding, which sees
the same post-norm patch tokens the reference's rebound ``Aggregator.forward`` reads
(``patch_vggt.py:195-207, 226-240, 313-357``).
"""
from __future__ import annotations

import json

import torch
from torch import Tensor

from ..layout import HEAD_DIM
from .utils import compute_qk_topk_indices_batched
from .wrapper import BaseHeadwiseSparseAttentionWrapper, SelectionState, _get

NUM_SPECIAL_TOKENS = 5
NUM_GLOBAL_BLOCKS = 24
NUM_ATTENTION_HEADS = 16
PATCH_SIZE = 14


def _load_config(model_cfg):
    cfg = _get(model_cfg, "sparse_config")
    if cfg is None:
        path = _get(model_cfg, "sparse_config_path")
        if path is None:
            raise ValueError("headsparse patching needs sparse_config_path (or sparse_config)")
        with open(path, "r") as f:
            cfg = json.load(f)
    return cfg


def patch_model(model, model_cfg):
    pm = _get(model_cfg, "patch_module")
    ptype = _get(pm, "type")
    if ptype == "headprofile":  # offline profiler writing the head-profile JSON (profiler.py)
        from .profiler import patch_model_profile
        model = patch_model_profile(model, model_cfg, HeadwiseSparseAttentionWrapper, NUM_SPECIAL_TOKENS,
                                    model.aggregator.global_blocks[0].attn.num_heads,
                                    len(model.aggregator.global_blocks), SelectionState())
        install_feature_topk(model, model_cfg)
        return model
    if ptype != "headsparse":
        raise NotImplementedError(f"patch_module.type={ptype!r}: only 'headsparse' and 'headprofile' are built")
    config = _load_config(model_cfg)
    has_dino = any(g["mode"] == "dino_topk" for groups in config.values() for g in groups)
    lazy = bool(_get(pm, "lazy_dino_topk", False))
    if has_dino and _get(pm, "topk_mode", "token") != "token":
        raise AssertionError("dino_topk heads need patch_module.topk_mode == 'token'")
    state = SelectionState()
    blocks = model.aggregator.global_blocks
    for layer_key, layer_config in config.items():
        i = int(layer_key)
        if i >= len(blocks):
            raise ValueError(f"Failed to get module aggregator.global_blocks.{i}.attn from the model.")
        orig = blocks[i].attn
        blocks[i].attn = HeadwiseSparseAttentionWrapper(
            orig, layer_idx=i, dino_topk=_get(pm, "topk", 4), lazy_dino_topk=lazy, config=layer_config,
            block_topk=_get(pm, "block_topk", 4), topk_scope=_get(pm, "topk_scope", "frame"), shared=state)
    model.saf3r_selection_state = state
    if has_dino and not lazy:
        install_feature_topk(model, model_cfg)
    return model


def install_feature_topk(model, model_cfg):
    """Compute the non-lazy token top-k from the DINO patch tokens in every forward: a forward hook on
    ``model.aggregator.patch_embed`` passes its post-norm patch tokens (``x_norm_patchtokens`` of the
    DINOv2 output dict, or the token tensor of a plain patch embedding), [S, P, C] for the S frames of
    the batch-1 input, to ``set_dino_topk_from_features``. ref: saf3r/patch/patch_vggt.py:195-207 and
    :226-240 (the rebound aggregator forward of the non-lazy and profiling modes), :313-357 (its body).
    Returns the hook handle, or None for a host without a patch embedding (such a host calls
    ``set_dino_topk_from_features`` itself)."""
    agg = getattr(model, "aggregator", None)
    pe = getattr(agg, "patch_embed", None) if agg is not None else None
    if pe is None:
        return None
    old = getattr(model, "saf3r_feature_topk_hook", None)
    if old is not None:
        old.remove()

    def hook(module, inputs, output):
        tokens = output["x_norm_patchtokens"] if isinstance(output, dict) else output
        set_dino_topk_from_features(model, tokens, model_cfg)

    handle = pe.register_forward_hook(hook)
    model.saf3r_feature_topk_hook = handle
    return handle


def update_args_per_forward(model, img_h, img_w):
    patch_height = img_h // PATCH_SIZE
    patch_width = img_w // PATCH_SIZE
    state = getattr(model, "saf3r_selection_state", None)
    if state is not None:
        state.reset()
    from .profiler import SparseAttentionProfiler
    for block in model.aggregator.global_blocks:
        attn = block.attn
        if isinstance(attn, SparseAttentionProfiler):
            attn.patch_height = patch_height
            attn.patch_width = patch_width
            continue
        if not isinstance(attn, BaseHeadwiseSparseAttentionWrapper):
            continue
        attn.patch_height = patch_height
        attn.patch_width = patch_width
        attn.first_dino_flag = False


def set_dino_topk_from_features(model, patch_tokens: Tensor, model_cfg):
    """The selection step of the reference's non-lazy aggregator forward (``patch_vggt.py:313-357``):
    ``patch_tokens`` [S, P, C] are the DINO patch tokens (post-norm) of the S frames; their
    L2-normalised features give every image token its keys (``compute_qk_topk_indices_batched``),
    which every dino_topk head of every patched layer reads in this forward. Call it after
    ``update_args_per_forward``. Returns int32 [S*P, width]."""
    pm = _get(model_cfg, "patch_module")
    S, P, C = patch_tokens.shape
    feat = torch.nn.functional.normalize(patch_tokens.reshape(1, S * P, C), p=2, dim=-1)
    idx = compute_qk_topk_indices_batched(
        feat, feat, topk=_get(pm, "topk", 4), q_blocksize=4096, per_frame=bool(_get(pm, "per_frame_topk", True)),
        num_toks_per_img=P, max_topk=_get(pm, "max_topk", 2048),
        include_first_frame=bool(_get(pm, "include_first_frame", False)),
        first_frame_stride=_get(pm, "first_frame_stride", 4)).reshape(S * P, -1)
    state = getattr(model, "saf3r_selection_state", None)
    if state is not None:
        state.est_topk_idx = idx
    for block in model.aggregator.global_blocks:
        if isinstance(block.attn, BaseHeadwiseSparseAttentionWrapper):
            block.attn.est_topk_idx = idx
    return idx


class HeadwiseSparseAttentionWrapper(BaseHeadwiseSparseAttentionWrapper):
    def __init__(self, orig_module, **kwargs):
        super().__init__(orig_module, NUM_SPECIAL_TOKENS, orig_module.num_heads, **kwargs)
        if orig_module.head_dim != HEAD_DIM:
            raise NotImplementedError(f"head_dim {orig_module.head_dim}: the kernels are built for 64")

    def forward(self, x: Tensor, pos=None) -> Tensor:
        B, N, C = x.shape
        if B != 1:
            raise AssertionError("Currently only support batch size of 1 for simplicity")
        if not x.is_cuda:
            raise RuntimeError("HeadwiseSparseAttentionWrapper runs on the GPU kernels only")
        om = self.orig_module
        geom = self.geometry(N)
        qkv = om.qkv(x).reshape(N, 3 * C)
        if qkv.dtype != torch.bfloat16:
            qkv = qkv.to(torch.bfloat16)
        qkv = qkv.contiguous()
        out = self.compute_multihead_attention_packed(qkv, None if pos is None else pos[0], geom)
        y = out.reshape(B, N, C)
        if not torch.is_autocast_enabled("cuda") and y.dtype != om.proj.weight.dtype:
            y = y.to(om.proj.weight.dtype)
        y = om.proj(y)
        return om.proj_drop(y)
