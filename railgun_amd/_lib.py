"""ctypes binding of librailgun_hip.so, the C ABI declared in include/railgun_hip.h.

The library is built in-tree (``__graft_entry__.build()``) next to this file.  There is
no fallback: if it is missing or cannot be loaded, importing the ops raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_size_t, c_void_p

LIB_NAME = "librailgun_hip.so"
# RAILGUN_HIP_LIB selects another build of the same library (e.g. a tuning variant).
LIB_PATH = os.environ.get("RAILGUN_HIP_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

RG_OK = 0
RG_ERR_INVALID_ARGUMENT = 1
RG_ERR_NOT_SUPPORTED = 2
RG_ERR_HIP = 3
RG_ERR_WORKSPACE = 4

RG_DTYPE_F32 = 0
RG_DTYPE_BF16 = 1
RG_DTYPE_F16 = 2

_ERR_NAMES = {
    RG_ERR_INVALID_ARGUMENT: "InvalidArgument",
    RG_ERR_NOT_SUPPORTED: "NotSupported",
    RG_ERR_HIP: "Hip",
    RG_ERR_WORKSPACE: "Workspace",
}


class RailgunError(RuntimeError):
    """A non-zero status from the C ABI; ``code`` is the RG_ERR_* value."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{_ERR_NAMES.get(code, code)}] {message}")
        self.code = code
        self.message = message


i32p = POINTER(c_int32)
f32p = POINTER(c_float)

# name -> (restype, argtypes); mirrors include/railgun_hip.h one to one.
SIGNATURES = {
    "rg_last_error": (c_char_p, []),
    "rg_abi_version": (c_int, []),
    "rg_init": (c_int, [c_int]),
    "rg_rope": (c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p]),
    "rg_rope_cos_sin_table": (c_int, [f32p, c_int32, c_int32, c_double]),
    "rg_reshape_and_cache": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32,
         c_int64, c_void_p],
    ),
    "rg_reshape_and_cache_isoquant": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32,
         c_int32, c_int64, c_void_p],
    ),
    "rg_rope_reshape_and_cache": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32,
         c_int32, c_int32, c_int32, c_int32, c_int64, c_void_p],
    ),
    "rg_qkv_rope_reshape_and_cache": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32,
         c_int32, c_int32, c_int32, c_int32, c_int64, c_void_p],
    ),
    "rg_copy_blocks": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int64, c_int64, c_int64, c_int32, c_int64, c_int64, c_void_p],
    ),
    "rg_rms_norm": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_int32, c_int32, c_int32, c_void_p]),
    "rg_silu_and_mul": (c_int, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p]),
    "rg_linear": (c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int64, c_int64, c_int64, c_void_p,
                          c_size_t, c_int32, c_void_p]),
    "rg_linear_workspace_bytes": (c_size_t, [c_int32, c_int32, c_int32]),
    "rg_linear_silu_mul": (c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int64, c_int64, c_int64,
                                   c_int32, c_void_p]),
    "rg_linear_qkv_rope_reshape_and_cache": (c_int, [c_void_p] * 8 + [c_int32] * 6 + [c_int64] * 4 + [c_int32, c_void_p]),
    "rg_linear_residual": (c_int, [c_void_p] * 3 + [c_int32] * 3 + [c_int64] * 3 + [c_void_p, c_size_t, c_int32, c_void_p]),
    "rg_rms_norm_linear_silu_mul": (c_int, [c_void_p, c_void_p, c_float, c_void_p, c_void_p] + [c_int32] * 3
                                    + [c_int64] * 3 + [c_int32, c_void_p]),
    "rg_rms_norm_linear_qkv_rope_reshape_and_cache": (c_int, [c_void_p, c_void_p, c_float] + [c_void_p] * 7
                                                      + [c_int32] * 6 + [c_int64] * 4 + [c_int32, c_void_p]),
    "rg_validate_block_tables": (c_int, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p]),
    "rg_validate_slot_mapping": (c_int, [c_void_p, c_int32, c_int64, c_void_p]),
    "rg_paged_attention_v1_workspace_bytes": (c_size_t, [c_int32, c_int32, c_int32, c_int32, c_int32, c_int32]),
    "rg_paged_attention_v1": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_int32, c_int32, c_int32,
         c_int32, c_int32, c_int32, c_int32, c_int64, c_void_p, c_size_t, c_void_p],
    ),
    "rg_rope_reshape_and_cache_paged_attention_v1": (
        c_int,
        [c_void_p] * 11 + [c_float] + [c_int32] * 7 + [c_int64, c_void_p, c_size_t, c_void_p],
    ),
    "rg_paged_attention_v1_no_alloc": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_int32, c_int32, c_int32,
         c_int32, c_int32, c_int32, c_int32, c_int64, c_void_p],
    ),
    "rg_paged_attention_v1_plus": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_int32, c_int32,
         c_int32, c_int32, c_int32, c_int32, c_int32, c_int64, c_void_p, c_size_t, c_void_p],
    ),
    "rg_v2_workspace_bytes": (c_size_t, [c_int32, c_int32, c_int32, c_int32]),
    "rg_paged_attention_v2_partition": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_float,
         c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int64, c_void_p],
    ),
    "rg_paged_attention_v2_reduce": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32,
         c_int32, c_int32, c_void_p],
    ),
    "rg_paged_attention_v2": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_int32, c_int32, c_int32,
         c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int64, c_void_p, c_size_t, c_void_p],
    ),
    "rg_prefill_packed": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_int32, c_int32,
         c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int64, c_void_p],
    ),
}

_lib = None


def load_library(path: str | None = None) -> ctypes.CDLL:
    """Loads the HIP library once and attaches the C signatures; raises if absent."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise ImportError(f"{p} is not built: run `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = ctypes.CDLL(p)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def last_error() -> str:
    msg = load_library().rg_last_error()
    return msg.decode() if msg else ""


def check(status: int) -> None:
    """Raises RailgunError for a non-zero status, with the library's message."""
    if status != RG_OK:
        raise RailgunError(status, last_error())
