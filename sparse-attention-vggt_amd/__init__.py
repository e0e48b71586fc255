"""MI355X-native SAF3R head-wise sparse global attention for VGGT-style transformers.

Import name: ``sparse_attention_vggt_amd`` (the directory ``sparse-attention-vggt_amd`` is loaded by
path, see ``__graft_entry__.package()``).

Layers
------
``patch``   plugin surface of the reference (``patch_model``, ``update_args_per_forward``,
            ``HeadwiseSparseAttentionWrapper``), driving the kernels below.
``ops``     torch-facing wrappers of the C ABI in ``include/saf3r_hip.h``.
``csrc``    gfx950 HIP kernels (prologue, block pooling / selection, block-sparse MFMA attention,
            gather attention, per-frame token top-k) built into ``libsaf3r_hip.so``.
``synth``   seeded synthetic workloads of the benchmark configurations.
``vggt``    the VGGT global-attention module shape (``Attention`` with qkv / q_norm / k_norm /
            rope / proj) used when no host model is supplied.
"""
from . import layout, ops  # noqa: F401
from .layout import Geometry  # noqa: F401
