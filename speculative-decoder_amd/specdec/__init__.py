"""Native kernels of the speculative-decoding hot path (libspecdec.so, gfx950).

`specdec.ops` wraps each C-ABI entry point for torch tensors on the GPU.
The library is loaded on first use; a missing library is an error, never a
silent fallback.
"""
from specdec._lib import LIB_PATH, available, lib, spin_wait  # noqa: F401
