"""MI355X (gfx950) sparse 3D convolution path: voxel hash neighbour map,
MFMA gather-GEMM submanifold conv, C2S subdivision -- behind the C ABI of
include/sparseconv.h (libsparseconv.so, built in-tree)."""
from ._capi import SparseConvError  # noqa: F401

__all__ = ["SparseConvError"]
