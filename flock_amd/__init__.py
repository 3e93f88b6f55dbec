"""flock_amd -- MI355X-native (gfx950) attention hot path of flock.

The product is libflock_attn.so (HIP kernels behind the C ABI in
include/flock_attn.h). This package is its Python host: ``ops`` wraps each
entry point, ``layer.Layer`` mirrors the attention slice of the reference's
kernels/layer.ts. Importing ``ops`` or ``layer`` loads the library and fails
loudly if it has not been built (``python -m flock_amd.build``).
"""
from ._lib import (CacheFullError, FlockError, UnsupportedError, WorkspaceError,  # noqa: F401
                   LIB_PATH, lib)

__all__ = ["lib", "LIB_PATH", "FlockError", "CacheFullError", "UnsupportedError",
           "WorkspaceError"]
