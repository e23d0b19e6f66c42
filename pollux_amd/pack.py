"""Pack-time quantization of H24 layers (mirrors the reference's pack.py).

``_quantize_h24_layer(weight, codebook)`` has the signature and results of
``pack._quantize_h24_layer`` (pack.py:139-180): NN-P indices of the raw fp32
atoms (first maximum of w . kp over the fp32 kissing points; origin iff
||atom||_2 < 1e-8), packed 18-bit, and fp16 row scales
fp16(max(row_rms(w) * sqrt(12), 1e-8)).  The search, the row scale and the
packing run in one C-ABI call (plx_quantize_layer_pack) on the weight's
device; like the reference it returns the two tensors on the CPU.
``quantize_h24_layer`` returns them on the device instead.

``_quantize_int8`` / ``quantize_int8_rows`` are the per-row INT8 format of
the embeddings and LM head (pack.py:124-136), and ``pack_state_dict`` is the
tensor loop of ``pack_checkpoint`` (pack.py:254-286) over an in-memory state
dict (the reference's ``torch.load(..., weights_only=False)`` is not
repeated: callers load checkpoints with a safe loader).
"""

from __future__ import annotations

import torch

from . import _lib
from .castor import (
    BACKBONE_BITS_PER_PARAM,
    BYTES_PER_CHUNK,
    H24_DIM,
    _check_codebook,
    _workspace,
    get_h24_codebook,
    row_rms_from_matrix,
)


def quantize_h24_layer(weight: torch.Tensor, *, return_indices: bool = False):
    """Device-resident pack of one H24 weight [out, in].

    Returns (packed uint8 [((N+3)//4)*9], sigma_rows fp16 [out]) on the
    weight's device, plus int32 indices [N] when ``return_indices``.
    """
    if weight.dim() != 2:
        raise ValueError(f"expected a 2D weight matrix, got {weight.dim()}D.")
    _lib.require_device(weight, "quantize_h24_layer input")
    rows, cols = weight.shape
    if weight.numel() % H24_DIM:
        raise ValueError(f"H24 packing needs a multiple of {H24_DIM} elements; got shape {tuple(weight.shape)}")
    w = weight.detach().float().contiguous()
    dev = w.device
    n = w.numel() // H24_DIM
    packed = torch.empty(((n + 3) // 4) * BYTES_PER_CHUNK, dtype=torch.uint8, device=dev)
    sigma = torch.empty(rows, dtype=torch.float16, device=dev)
    if not return_indices and cols % H24_DIM == 0:
        idx = None
    else:
        idx = torch.empty(n, dtype=torch.int32, device=dev)
    if rows and cols:
        with torch.cuda.device(dev):
            lib = _lib.lib()
            if cols % H24_DIM == 0:
                ws = _workspace(n, dev)
                st = lib.plx_quantize_layer_pack(
                    _lib.ptr(w), rows, cols, _lib.ptr(packed), _lib.ptr(sigma), _lib.ptr(idx),
                    _lib.ptr(ws), ws.numel(), _lib.stream_of(dev),
                )
                _lib.check(st, "quantize_h24_layer")
            else:
                # atoms straddle rows (numel % 24 == 0 only, pack.py:161): three calls
                from .castor import quantize_indices, pack_indices, sigma16_pack

                idx.copy_(quantize_indices(w.reshape(-1, H24_DIM), mode="pack"))
                packed.copy_(pack_indices(idx))
                sigma.copy_(sigma16_pack(w))
    return (packed, sigma, idx) if return_indices else (packed, sigma)


def _quantize_h24_layer(weight: torch.Tensor, codebook: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """pack._quantize_h24_layer (pack.py:139-180): (packed uint8, sigma_rows fp16), both on the CPU.

    ``codebook`` must be the canonical table (get_h24_codebook) in fp32 or
    fp64, whose values the reference scores (``codebook[1:].to(fp32)``), or
    in fp16: the fp16 table is the raw integer codes times 0.353515625
    exactly, so its scores order the codes like the fp32 table's up to
    4.8e-8 * |x_pos| (fp32(3s) - 3s), inside the near-tie envelope, and the
    indices agree on every atom that is not a near-tie.  A bfloat16 table
    (3s rounded to 1.0625) scores type-3 codes differently and raises
    ValueError.
    """
    _lib.require_device(weight, "_quantize_h24_layer input")
    _check_codebook(codebook, "pack")
    packed, sigma = quantize_h24_layer(weight)
    return packed.cpu(), sigma.cpu()


def quantize_int8_rows(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Device-resident pack._quantize_int8: (int8 like weight, fp16 mu per row of the last dim)."""
    _lib.require_device(weight, "quantize_int8_rows input")
    if weight.dim() < 1 or weight.shape[-1] == 0:
        raise ValueError(f"INT8 packing needs a non-empty last dimension; got shape {tuple(weight.shape)}")
    w = weight.detach().float().contiguous()
    cols = w.shape[-1]
    rows = w.numel() // cols
    q = torch.empty(w.shape, dtype=torch.int8, device=w.device)
    mu = torch.empty(w.shape[:-1], dtype=torch.float16, device=w.device)
    if rows:
        with torch.cuda.device(w.device):
            st = _lib.lib().plx_quantize_int8_rows(
                _lib.ptr(w), rows, cols, _lib.ptr(q), _lib.ptr(mu), _lib.stream_of(w.device)
            )
        _lib.check(st, "quantize_int8_rows")
    return q, mu


def _quantize_int8(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """pack._quantize_int8 (pack.py:124-136): (int8 weight, fp16 mu_rows), both on the CPU."""
    q, mu = quantize_int8_rows(weight)
    return q.cpu(), mu.cpu()


def _is_packable_h24(name: str, tensor: torch.Tensor) -> bool:
    """pack._is_packable_h24 (pack.py:110-117) with pollux._is_h24_tensor (pollux.py:115-117)."""
    if not name.endswith(".weight") or name.startswith(("tok_emb.", "pos_emb.", "head.")):
        return False
    return tensor.dim() >= 2 and tensor.numel() > 0 and tensor.numel() % H24_DIM == 0


def pack_state_dict(state_in: dict[str, torch.Tensor], device: torch.device | str) -> tuple[dict, dict]:
    """The tensor loop of pack.pack_checkpoint (pack.py:254-286) on ``device``.

    Returns (state_out with CPU tensors in the reference's order and naming,
    stats dict with h24_atom_count / h24_scale_row_count).  Config keys the
    reference adds before writing: ``pack_config(cfg)``.
    """
    codebook = get_h24_codebook(device, torch.float32)
    out: dict[str, torch.Tensor] = {}
    atoms = scale_rows = 0
    for name, tensor in state_in.items():
        if name in ("tok_emb.weight", "head.weight"):
            q, mu = _quantize_int8(tensor.to(device))
            out[name.replace(".weight", ".weight_int8")] = q
            out[name.replace(".weight", ".mu_rows")] = mu
        elif _is_packable_h24(name, tensor):
            if tensor.dim() != 2:
                # the reference's row_rms_from_matrix rejects it the same way (castor.py:312)
                row_rms_from_matrix(tensor)
            pw, sigma = _quantize_h24_layer(tensor.to(device), codebook)
            out[name.replace(".weight", ".packed_weights")] = pw
            out[name.replace(".weight", ".sigma_rows")] = sigma
            atoms += tensor.numel() // H24_DIM
            scale_rows += int(sigma.numel())
        else:
            out[name] = tensor.detach().cpu()
    return out, {"h24_atom_count": atoms, "h24_scale_row_count": scale_rows}


def pack_config(cfg_dict: dict) -> dict:
    """The config keys pack_checkpoint adds before writing (pack.py:289-292)."""
    cfg = dict(cfg_dict)
    cfg["scales_per_row"] = 1
    cfg["scale_serialization"] = "row_wise"
    cfg["bits_per_param"] = BACKBONE_BITS_PER_PARAM
    return cfg
