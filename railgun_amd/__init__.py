"""railgun_amd — MI355X (gfx950) attention hot path of the Railgun inference engine.

Hand-written HIP kernels (paged decode v1/v2, reshape_and_cache, packed RoPE, packed
causal prefill) behind the C ABI of ``include/railgun_hip.h``, plus the host-side mirror of
Railgun's ``PagedAttentionKernels`` / ``PagedAttentionOp`` in :mod:`railgun_amd.ops`.
"""
from ._lib import LIB_PATH, RailgunError, load_library

__all__ = ["LIB_PATH", "RailgunError", "load_library"]
