"""ctypes binding of ``lib/libpollux_amd.so`` (the C ABI in include/pollux_amd.h).

The library is built in-tree by ``pollux_amd.build`` for gfx950.  Loading
fails loudly when it is missing: there is no CPU or PyTorch fallback for any
compute entry point.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libpollux_amd.so"

PLX_OK, PLX_EINVAL, PLX_EHIP, PLX_ENOMEM = 0, 1, 2, 3
NN_BF16_SCORES, NN_FP32_SCORES, NN_PACK_FP32 = 0, 1, 2
NN_DENSE_TYPE3 = 0x100  # flag on NN_BF16_SCORES: the dense sweep of every code instead of the structured scorers
NN_T3_ROWS_BY_SWEEP = 0x200  # flag on NN_BF16_SCORES (diagnostics): the structured scorers' overflow path
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
PROF_NN, PROF_PACK, PROF_UNPACK, PROF_DEQUANT, PROF_ADAM, PROF_T3, PROF_T12 = 0, 1, 2, 3, 4, 5, 6  # plx_profile_select

_vp, _i64, _int, _sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t

# name -> (restype, argtypes); every symbol declared in include/pollux_amd.h
SIGNATURES = {
    "plx_last_error": (ctypes.c_char_p, []),
    "plx_version": (_int, []),
    "plx_codebook_raw": (_int, [_vp, _i64]),
    "plx_codebook_f32": (_int, [_vp, _i64]),
    "plx_codebook_fingerprint": (_int, [_vp]),
    "plx_device_init": (_int, []),
    "plx_pack_indices": (_int, [_vp, _int, _i64, _vp, _vp]),
    "plx_unpack_indices": (_int, [_vp, _i64, _i64, _vp, _vp]),
    "plx_row_rms": (_int, [_vp, _i64, _i64, _vp, _vp]),
    "plx_sigma16_pack": (_int, [_vp, _i64, _i64, _vp, _vp]),
    "plx_quantize_workspace_bytes": (_sz, [_i64]),
    "plx_quantize": (_int, [_vp, _i64, _int, _vp, _vp, _sz, _vp]),
    "plx_gather_codebook": (_int, [_vp, _i64, _int, _vp, _vp]),
    "plx_requantize": (_int, [_vp, _i64, _i64, _int, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "plx_quantize_layer_pack": (_int, [_vp, _i64, _i64, _vp, _vp, _vp, _vp, _sz, _vp]),
    "plx_requantize_batch": (_int, [_vp, _int, _int, _vp, _sz, _vp]),
    "plx_requantize_noalloc": (_int, [_vp, _i64, _i64, _int, _vp, _vp, _vp, _vp, _vp]),
    "plx_pollux_step_workspace_bytes": (_sz, [_i64, _i64]),
    "plx_pollux_step_h24": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _vp, _int, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "plx_pollux_step_batch_workspace_bytes": (_sz, [_vp, _int]),
    "plx_pollux_step_h24_batch": (_int, [_vp, _int, _vp, _int, _vp, _sz, _vp]),
    "plx_quantize_int8_rows": (_int, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "plx_dequant_int8_rows": (_int, [_vp, _vp, _i64, _i64, _vp, _vp]),
    "plx_dequant_f16": (_int, [_vp, _i64, _vp, _i64, _i64, _vp, _vp]),
    "plx_dequant_linear_workspace_bytes": (_sz, [_i64, _i64, _i64, _int]),
    "plx_dequant_linear": (_int, [_vp, _i64, _vp, _i64, _i64, _vp, _int, _i64, _vp, _vp, _sz, _vp]),
    "plx_h24_plane_layout": (_int, [_vp, _i64, _i64, _vp, _vp]),
    "plx_plane_table": (_i64, [_vp, _i64]),
    "plx_dequant_linear_multi_workspace_bytes": (_sz, [_vp, _int, _i64, _i64, _int]),
    "plx_dequant_linear_multi": (_int, [_vp, _int, _i64, _vp, _int, _i64, _vp, ctypes.c_float, _vp, _sz, _vp]),
    "plx_int8_linear": (_int, [_vp, _vp, _i64, _i64, _vp, _i64, _vp, ctypes.c_float, _vp, _vp]),
    "plx_int8_linear_argmax_workspace_bytes": (ctypes.c_size_t, [_i64, _i64]),
    "plx_int8_linear_argmax": (_int, [_vp, _vp, _i64, _i64, _vp, _i64, _vp, ctypes.c_float, _vp, _vp, _vp, _i64,
                                      _vp, _vp, ctypes.c_size_t, _vp]),
    "plx_int8_embed": (_int, [_vp, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp]),
    "plx_argmax_rows": (_int, [_vp, _i64, _i64, _vp, _vp]),
    "plx_rms_norm": (_int, [_vp, _vp, _vp, _i64, _i64, ctypes.c_float, _vp]),
    "plx_decode_attention": (_int, [_vp, _vp, _vp, _i64, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _i64, _i64, _i64, _vp,
                                    _vp]),
    "plx_prefill_attention": (_int, [_vp, _vp, _vp, _i64, _vp, _vp, ctypes.c_float, _vp, _vp, _i64, _i64, _i64, _i64,
                                     _i64, _vp, _vp]),
    "plx_profile_select": (_int, [_int]),
    "plx_profile_begin": (_int, []),
    "plx_profile_end": (_int, [_vp, _vp]),
}

class PolluxStepItem(ctypes.Structure):
    """plx_pollux_step_item (include/pollux_amd.h)."""

    _fields_ = [
        ("grad", _vp), ("m", _vp), ("v", _vp), ("latent", _vp), ("rows", _i64), ("cols", _i64),
        ("sigma_out", _vp), ("idx_out", _vp), ("packed_out", _vp), ("weight_out", _vp), ("adam_norm_out", _vp),
    ]


class RequantizeItem(ctypes.Structure):
    """plx_requantize_item (include/pollux_amd.h)."""

    _fields_ = [
        ("latent", _vp), ("rows", _i64), ("cols", _i64), ("sigma_out", _vp),
        ("idx_out", _vp), ("packed_out", _vp), ("weight_out", _vp),
    ]


class DqlTarget(ctypes.Structure):
    """plx_dql_target (include/pollux_amd.h)."""

    _fields_ = [("packed", _vp), ("sigma16", _vp), ("rows", _i64), ("y", _vp), ("residual", _vp)]


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(
                        f"pollux_amd: HIP library {LIB_PATH} is missing; build it with "
                        "`python -m pollux_amd.build` (hipcc, gfx950)."
                    )
                handle = ctypes.CDLL(str(LIB_PATH))
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    """Map a PLX_* status to the reference's exception types."""
    if status == PLX_OK:
        return
    msg = lib().plx_last_error().decode(errors="replace")
    if status == PLX_EINVAL:
        raise ValueError(msg or f"{what}: invalid argument")
    raise RuntimeError(f"{what} failed ({status}): {msg}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_device(t: torch.Tensor, name: str) -> None:
    if t.device.type != "cuda":
        raise ValueError(
            f"pollux_amd: {name} must be on a ROCm device (torch 'cuda'); got {t.device}. "
            "This library has no CPU path."
        )
