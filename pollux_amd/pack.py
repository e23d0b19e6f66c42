"""Pack-time quantization of H24 layers (mirrors the reference's pack.py).

``_quantize_h24_layer(weight, codebook)`` has the signature and results of
``pack._quantize_h24_layer`` (pack.py:139-180): NN-P indices of the raw fp32
atoms (first maximum of w . kp over the fp32 kissing points; origin iff
||atom||_2 < 1e-8), packed 18-bit, and fp16 row scales
fp16(max(row_rms(w) * sqrt(12), 1e-8)).  The search, the row scale and the
packing run in one C-ABI call (plx_quantize_layer_pack) on the weight's
device; like the reference it returns the two tensors on the CPU.
``quantize_h24_layer`` returns them on the device instead.
"""

from __future__ import annotations

import torch

from . import _lib
from .castor import BYTES_PER_CHUNK, H24_DIM, _check_codebook, _workspace, assert_row_aligned_in_features


def quantize_h24_layer(weight: torch.Tensor, *, return_indices: bool = False):
    """Device-resident pack of one H24 weight [out, in].

    Returns (packed uint8 [((N+3)//4)*9], sigma_rows fp16 [out]) on the
    weight's device, plus int32 indices [N] when ``return_indices``.
    """
    if weight.dim() != 2:
        raise ValueError(f"expected a 2D weight matrix, got {weight.dim()}D.")
    _lib.require_device(weight, "quantize_h24_layer input")
    rows, cols = weight.shape
    assert_row_aligned_in_features(cols)
    w = weight.detach().float().contiguous()
    dev = w.device
    n = rows * (cols // H24_DIM)
    packed = torch.empty(((n + 3) // 4) * BYTES_PER_CHUNK, dtype=torch.uint8, device=dev)
    sigma = torch.empty(rows, dtype=torch.float16, device=dev)
    idx = torch.empty(n, dtype=torch.int32, device=dev) if return_indices else None
    if rows:
        ws = _workspace(n, dev)
        with torch.cuda.device(dev):
            st = _lib.lib().plx_quantize_layer_pack(
                _lib.ptr(w), rows, cols, _lib.ptr(packed), _lib.ptr(sigma), _lib.ptr(idx),
                _lib.ptr(ws), ws.numel(), _lib.stream_of(dev),
            )
        _lib.check(st, "quantize_h24_layer")
    return (packed, sigma, idx) if return_indices else (packed, sigma)


def _quantize_h24_layer(weight: torch.Tensor, codebook: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """pack._quantize_h24_layer (pack.py:139-180): (packed uint8, sigma_rows fp16), both on the CPU.

    ``codebook`` must be the canonical table (get_h24_codebook, any dtype);
    the search always uses its fp32 values, as the reference does.
    """
    _lib.require_device(weight, "_quantize_h24_layer input")
    _check_codebook(codebook, weight.device)
    packed, sigma = quantize_h24_layer(weight)
    return packed.cpu(), sigma.cpu()
