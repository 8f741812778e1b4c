"""ember_amd: the paged-KV hot path of YUStulinu/Ember, rebuilt for AMD MI355X (gfx950).

The product is native: HIP kernels for gfx950 and C++ host code behind the C
ABI of include/ember_hip.h, built into ember_amd/libember_hip.so. This package
binds that library for Python callers (tests, bench); it never computes
anything itself and has no fallback path.
"""
from ._lib import BLOCK_SIZE, DTYPE_F16, DTYPE_F32, MAX_RUN, PREFILL_TILE, EmberError, lib  # noqa: F401
from .block_manager import BlockManager  # noqa: F401

__all__ = ["lib", "EmberError", "BlockManager", "BLOCK_SIZE", "MAX_RUN", "PREFILL_TILE", "DTYPE_F16", "DTYPE_F32"]
