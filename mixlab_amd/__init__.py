"""mixlab_amd -- MI355X-native executor of mixlab's MoE feed-forward op (IR op 74).

libmixmoe.so (HIP, gfx950) holds the kernels and the C ABI declared in
include/mixmoe.h; ``mixlab_amd.moe`` restates the reference's MoE config and
op-encoding surface; ``mixlab_amd.op.MoEFeedForward`` runs one op on the GPU.
"""
from . import moe  # noqa: F401
from ._lib import LIB_PATH, MixMoEError, load  # noqa: F401

__all__ = ["moe", "load", "LIB_PATH", "MixMoEError"]
