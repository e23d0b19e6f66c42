"""pollux_amd: MI355X (gfx950) HIP implementation of Pollux's Leech-lattice quantization path.

Modules
-------
castor   castor.py-compatible API: codebook, 18-bit pack/unpack, row scale,
         nearest-neighbour quantizer, fused requantize
packed   PackedH24Linear with HIP dequantization
build    builds lib/libpollux_amd.so (hipcc, gfx950) in-tree
"""

from . import castor  # noqa: F401
from .packed import PackedH24Linear, dequant_linear, dequantize_h24  # noqa: F401

__all__ = ["castor", "PackedH24Linear", "dequant_linear", "dequantize_h24"]
