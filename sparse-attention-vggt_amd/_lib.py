"""ctypes binding of the gfx950 C-ABI library ``libsaf3r_hip.so`` (declared in ``include/saf3r_hip.h``).

The library must be built (``__graft_entry__.build()`` or ``make -C csrc``). There is no fallback:
if it is missing or fails to load, every op raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  -- loads the HIP runtime first so the library binds to the same one

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsaf3r_hip.so")

EXPORTS = (
    "saf3r_abi_version", "saf3r_last_error", "saf3r_packed_slots", "saf3r_pack_qkv", "saf3r_block_pool",
    "saf3r_topk_from_scores", "saf3r_block_select", "saf3r_sparse_attn_fwd", "saf3r_gather_attn_fwd",
    "saf3r_token_topk", "saf3r_probe_scores", "saf3r_keyset_build", "saf3r_keyset_gather",
    "saf3r_frame_topk_scores", "saf3r_probe_scores_noalloc", "saf3r_token_topk_workspace_bytes",
    "saf3r_pooled_prepare", "saf3r_block_select_pooled", "saf3r_block_select_pooled_workspace_bytes",
    "saf3r_gather_attn_fwd_sliced", "saf3r_gather_attn_workspace_bytes",
)
ABI_VERSION = 13
GATHER_QK_FP32, GATHER_V_FP32, GATHER_OUT_FP32 = 1, 2, 4  # enum saf3r_gather_dtype
SAF3R_OK, SAF3R_ERR_INVALID, SAF3R_ERR_UNSUPPORTED, SAF3R_ERR_LAUNCH, SAF3R_ERR_INJECTED = range(5)

_lib = None


class Rows(ctypes.Structure):
    """``saf3r_rows``: logical row r at ptr + (base_row + (r // rows_per_frame) * frame_row_stride
    + r % rows_per_frame) * row_stride elements."""
    _fields_ = [
        ("ptr", ctypes.c_void_p),
        ("row_stride", ctypes.c_int64),
        ("base_row", ctypes.c_int64),
        ("rows_per_frame", ctypes.c_int64),
        ("frame_row_stride", ctypes.c_int64),
    ]


class Saf3rError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"saf3r error {code}: {msg}")
        self.code = code


def load():
    """Load the library once and declare every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"HIP library not built: {LIB_PATH} is missing (run __graft_entry__.build())")
    lib = ctypes.CDLL(LIB_PATH)
    i32, i64, p, f32 = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_float
    rows = ctypes.POINTER(Rows)
    sig = {
        "saf3r_abi_version": ([], i32),
        "saf3r_last_error": ([], ctypes.c_char_p),
        "saf3r_packed_slots": ([i32, i32, i32], i64),
        "saf3r_pack_qkv": ([p, p, p, i64, i64, i32, i32, i32, i32, p, p, p, p, f32, i32, p, p, p, i32, p, p, p, p, p,
                            p, p, f32, p, p, p, p, p], i32),
        "saf3r_pooled_prepare": ([p, i64, p, p, p], i32),
        "saf3r_block_select_pooled": ([p, p, p, i32, i32, i32, i32, p, p, i64, p], i32),
        "saf3r_block_select_pooled_workspace_bytes": ([i32, i32, i32, i32], i64),
        "saf3r_block_pool": ([p, p, i32, i32, i32, i32, p, i32, p, p, p], i32),
        "saf3r_topk_from_scores": ([p, i32, i32, i32, i32, i32, p, p], i32),
        "saf3r_block_select": ([p, p, i32, i32, i32, i32, i32, i32, p, p], i32),
        "saf3r_sparse_attn_fwd": ([p, p, p, i32, i32, i32, i32, p, p, i32, f32, p, i64, p, p, p, i64, p, p, p, p, p,
                                   i32, p, ctypes.c_uint, p], i32),
        "saf3r_gather_attn_fwd": ([rows, rows, rows, p, i64, i32, i32, i64, f32, i32, rows, p], i32),
        "saf3r_gather_attn_fwd_sliced": ([rows, rows, rows, p, i64, i32, i32, i64, f32, i32, rows, p, i64, p], i32),
        "saf3r_gather_attn_workspace_bytes": ([i32, i32], i64),
        "saf3r_token_topk": ([rows, rows, i32, i32, i32, i32, p, p, i64, p], i32),
        "saf3r_token_topk_workspace_bytes": ([i32, i32, i32, i32], i64),
        "saf3r_probe_scores": ([p, p, i64, i32, p, i32, p, i32, f32, p, p, p, i64, p], i32),
        "saf3r_probe_scores_noalloc": ([p, p, i64, i32, p, i32, p, i32, f32, p, p, i64, p], i32),
        "saf3r_keyset_build": ([p, i64, i32, p, p, p, p, i32, i32, i32, p, i64, p, p], i32),
        "saf3r_keyset_gather": ([p, i32, i32, i32, p, i32, p, i64, i64, p, i64, p, i32, p, p, i64, p], i32),
        "saf3r_frame_topk_scores": ([p, i64, i32, i32, i32, i32, i32, i32, i32, i32, p, i64, p, p, p], i32),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    if lib.saf3r_abi_version() != ABI_VERSION:
        raise RuntimeError(f"libsaf3r_hip.so ABI {lib.saf3r_abi_version()} != expected {ABI_VERSION}")
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != 0:
        msg = load().saf3r_last_error().decode(errors="replace")
        raise Saf3rError(rc, msg)


def stream_ptr(device=None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
