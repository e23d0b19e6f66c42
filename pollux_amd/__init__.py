"""pollux_amd: MI355X (gfx950) HIP implementation of Pollux's Leech-lattice quantization path.

Modules
-------
castor   castor.py-compatible API: codebook, 18-bit pack/unpack, row scale,
         nearest-neighbour quantizer (NN-B / NN-T / NN-P), fused requantize
packed   PackedH24Linear (HIP dequantization, fused dequant-GEMV/GEMM) and the
         INT8 periphery layers PackedInt8Embedding / PackedInt8Linear
pack     pack.py-compatible pack-time quantization (_quantize_h24_layer,
         _quantize_int8, the state-dict packing loop)
plx      the .plx container: byte-exact writer, reader, memory-mapped loader
optim    the fused optimiser step + requantize of an H24 parameter (pollux_step's H24 branch)
model    packed Pollux decoder for inference (.plx loading, fused packed layers, KV-cached decode)
build    builds lib/libpollux_amd.so (hipcc, gfx950) in-tree
"""

from . import castor, model, optim, pack, plx  # noqa: F401
from .packed import (  # noqa: F401
    PackedH24Linear,
    PackedInt8Embedding,
    PackedInt8Linear,
    dequant_linear,
    dequantize_h24,
    dequantize_int8_rows,
    h24_plane_layout,
)

__all__ = [
    "castor", "model", "optim", "pack", "plx", "PackedH24Linear", "PackedInt8Embedding", "PackedInt8Linear",
    "dequant_linear", "dequantize_h24", "dequantize_int8_rows", "h24_plane_layout",
]
