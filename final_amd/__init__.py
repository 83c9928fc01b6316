"""final_amd: MI355X (gfx950) sparse-MoE block - router, dispatch, grouped
SwiGLU experts and combine as hand-written HIP kernels behind a C-ABI
(include/moe_capi.h), with the reference's C++ layer interface
(include/layer.h) and this Python mirror of it."""
from . import _native
from .moe import DenseMLP, SparseMoeBlock

__all__ = ["DenseMLP", "SparseMoeBlock", "_native"]
