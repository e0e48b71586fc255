"""Plugin surface of the reference (``saf3r/patch/__init__.py:12-33``): model-name dispatch of
``patch_model`` and ``update_args_per_forward``. VGGT is the model family of this package; other
names raise ``ValueError`` like the reference does for unknown models."""
from . import patch_vggt
from .patch_vggt import HeadwiseSparseAttentionWrapper, set_dino_topk_from_features  # noqa: F401
from .profiler import SparseAttentionProfiler, save_profile_results  # noqa: F401
from .wrapper import BaseHeadwiseSparseAttentionWrapper  # noqa: F401


def patch_model(model, model_name, cfg):
    if "vggt" in model_name.lower():
        return patch_vggt.patch_model(model, cfg)
    raise ValueError(f"Unsupported model name: {model_name}")


def update_args_per_forward(model, model_name, img_h, img_w):
    if "vggt" in model_name.lower():
        return patch_vggt.update_args_per_forward(model, img_h, img_w)
    raise ValueError(f"Unsupported model name: {model_name}")
