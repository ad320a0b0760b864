"""ctypes binding of ``libfpv2_hip.so`` (C ABI declared in ``include/fpv2.h`` and
``include/fpv2_decoder.h``).

The library is built in-tree by ``flashprefillv2-mlx_amd/build.py``.  There is
no fallback: if the library is missing or a tensor is not on a ROCm device,
the call raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_NAME = "libfpv2_hip.so"
# The in-tree build; FPV2_LIBRARY may point at another build of the same ABI.
LIB_PATH = Path(os.environ.get("FPV2_LIBRARY") or Path(__file__).resolve().parent / LIB_NAME)
ABI_VERSION = 3

FPV2_OK = 0
FPV2_ERR_ARGUMENT = -1
FPV2_ERR_UNSUPPORTED = -2
FPV2_ERR_LAUNCH = -3

F32, F16, BF16 = 0, 1, 2
MAX_BLOCKS = 8192
SPLIT_SCRATCH_BYTES = 64 << 20  # FPV2_SPLIT_SCRATCH_BYTES

_DTYPE_CODES = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

EXPORTED_SYMBOLS = (
    "fpv2_abi_version",
    "fpv2_last_error",
    "fpv2_pool_blocks",
    "fpv2_pool_kv",
    "fpv2_score_select",
    "fpv2_compact_block_indices",
    "fpv2_sparse_attention",
    "fpv2_sparse_attention_split_workspace_bytes",
    "fpv2_sparse_attention_split",
    "fpv2_sparse_attention_split_static",
    # decoder-layer operations of the end-to-end harness (fpv2_decoder.h)
    "fpv2_add_rms_norm",
    "fpv2_qk_norm_rope",
    "fpv2_silu_mul",
)


class SelectParams(ctypes.Structure):
    """``fpv2_select_params`` (field order and types as in fpv2.h)."""

    _fields_ = [
        ("query_heads", ctypes.c_int64),
        ("kv_heads", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("padded_query_length", ctypes.c_int64),
        ("query_length", ctypes.c_int64),
        ("num_blocks", ctypes.c_int64),
        ("key_length", ctypes.c_int64),
        ("offset", ctypes.c_int64),
        ("block_k", ctypes.c_int64),
        ("tile_q", ctypes.c_int64),
        ("sink_tokens", ctypes.c_int64),
        ("window_tokens", ctypes.c_int64),
        ("last_n_blocks", ctypes.c_int64),
        ("scale", ctypes.c_float),
        ("alpha", ctypes.c_float),
        ("q_head_stride", ctypes.c_int64),
        ("q_row_stride", ctypes.c_int64),
        ("pooled_head_stride", ctypes.c_int64),
    ]


class AttnParams(ctypes.Structure):
    """``fpv2_attn_params`` (field order and types as in fpv2.h)."""

    _fields_ = [
        ("query_heads", ctypes.c_int64),
        ("kv_heads", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("padded_query_length", ctypes.c_int64),
        ("query_length", ctypes.c_int64),
        ("out_rows", ctypes.c_int64),
        ("key_length", ctypes.c_int64),
        ("num_blocks", ctypes.c_int64),
        ("offset", ctypes.c_int64),
        ("block_k", ctypes.c_int64),
        ("tile_q", ctypes.c_int64),
        ("mean_correction", ctypes.c_int32),
        ("scale", ctypes.c_double),
        ("q_head_stride", ctypes.c_int64),
        ("q_row_stride", ctypes.c_int64),
        ("k_head_stride", ctypes.c_int64),
        ("k_row_stride", ctypes.c_int64),
        ("v_head_stride", ctypes.c_int64),
        ("v_row_stride", ctypes.c_int64),
        ("o_head_stride", ctypes.c_int64),
        ("o_row_stride", ctypes.c_int64),
        ("pooled_head_stride", ctypes.c_int64),
    ]


_lib = None


def _declare(lib: ctypes.CDLL) -> None:
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    lib.fpv2_abi_version.restype = ctypes.c_int
    lib.fpv2_abi_version.argtypes = []
    lib.fpv2_last_error.restype = ctypes.c_char_p
    lib.fpv2_last_error.argtypes = []
    lib.fpv2_pool_blocks.restype = ctypes.c_int
    lib.fpv2_pool_blocks.argtypes = [vp, vp, i32, i64, i64, i64, i64, i64, i64, i64, i64, vp]
    lib.fpv2_pool_kv.restype = ctypes.c_int
    lib.fpv2_pool_kv.argtypes = [vp, vp, vp, vp, i32, i64, i64, i64, i64, i64, i64, i64, i64, vp]
    lib.fpv2_score_select.restype = ctypes.c_int
    lib.fpv2_score_select.argtypes = [vp, vp, i32, ctypes.POINTER(SelectParams), vp, vp,
                                      vp, vp, vp, vp, vp]
    lib.fpv2_compact_block_indices.restype = ctypes.c_int
    lib.fpv2_compact_block_indices.argtypes = [vp, i64, i64, i64, i64, i64, i64, i64,
                                               vp, vp, vp, vp, vp]
    lib.fpv2_sparse_attention.restype = ctypes.c_int
    lib.fpv2_sparse_attention.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32,
                                          ctypes.POINTER(AttnParams), vp]
    lib.fpv2_sparse_attention_split_workspace_bytes.restype = i64
    lib.fpv2_sparse_attention_split_workspace_bytes.argtypes = [ctypes.POINTER(AttnParams),
                                                                i64, i64]
    lib.fpv2_sparse_attention_split.restype = ctypes.c_int
    lib.fpv2_sparse_attention_split.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32,
                                                ctypes.POINTER(AttnParams), i64, i64, vp, i64,
                                                vp]
    lib.fpv2_sparse_attention_split_static.restype = ctypes.c_int
    lib.fpv2_sparse_attention_split_static.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp,
                                                       i32, ctypes.POINTER(AttnParams), i64, i64,
                                                       vp]
    f32 = ctypes.c_float
    lib.fpv2_add_rms_norm.restype = ctypes.c_int
    lib.fpv2_add_rms_norm.argtypes = [vp, vp, vp, vp, i32, i64, i64, i64, i64, i64, f32, vp]
    lib.fpv2_qk_norm_rope.restype = ctypes.c_int
    lib.fpv2_qk_norm_rope.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, i32, i64, i64, i64, i64,
                                      i64, i64, i64, i64, i64, f32, vp]
    lib.fpv2_silu_mul.restype = ctypes.c_int
    lib.fpv2_silu_mul.argtypes = [vp, vp, i32, i64, i64, i64, i64, vp]


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise if it is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    target = Path(path) if path is not None else LIB_PATH
    if not target.exists():
        raise RuntimeError(
            f"{target} is missing: build it with `python flashprefillv2-mlx_amd/build.py` "
            "(FPV2 has no non-HIP fallback)"
        )
    lib = ctypes.CDLL(str(target))
    _declare(lib)
    version = lib.fpv2_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"{target} has ABI version {version}, expected {ABI_VERSION}")
    if path is None:
        _lib = lib
    return lib


def check(status: int, what: str) -> None:
    """Raise for a non-zero status from the library."""
    if status == FPV2_OK:
        return
    message = (_lib.fpv2_last_error() or b"").decode(errors="replace")
    if status == FPV2_ERR_ARGUMENT:
        raise ValueError(f"{what}: {message}")
    raise RuntimeError(f"{what} failed ({status}): {message}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError as error:
        raise ValueError(f"unsupported dtype {dtype}") from error


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one ROCm device; returns it.  Raises otherwise."""
    device = tensors[0].device
    for t in tensors:
        if t.device.type != "cuda":
            raise RuntimeError(
                "FPV2 kernels run on ROCm devices only; got a tensor on "
                f"{t.device} (there is no CPU fallback)"
            )
        if t.device != device:
            raise ValueError("all tensors must be on the same device")
    return device


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
