"""h3turbo_amd: MI355X-native W4A8 ConvRot quantised-linear path of the official H3 DiT.

Drop-in for the reference's h3turbo.h3 ops (qlinear), contracts (types), the DiT block (block), block storage
(blockstore), weight streaming (stream) and the engine façade (engine), computing on hand-written gfx950 HIP
kernels (libh3k.so, C ABI in include/h3k.h).
"""
from . import qlinear, types  # noqa: F401
from .types import BlockProvider, BlockWeights, W4A8Weight, Weight  # noqa: F401

__version__ = "0.2.0"
