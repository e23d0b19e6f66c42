"""castor-compatible API over the MI355X HIP library (drop-in for castor.py's hot path).

Same names, signatures, argument meaning and exception types as the
reference's ``castor`` module (alavicka/pollux castor.py), so callers such as
``pollux_step`` (pollux.py:874-884), ``pack._quantize_h24_layer``
(pack.py:139-180) and ``PackedH24Linear`` (pollux.py:461-507) can import from
here instead.  Tensors for the compute entry points must live on a ROCm device
(torch's "cuda"); there is no CPU path: a CPU tensor raises ValueError.

Differences from the reference, by design:
  * ``castor_quantize_leech`` runs the HIP MFMA quantizer for every device
    tensor.  Its default semantics are the reference's non-Triton path (NN-B:
    scores rounded to bf16, lowest index on ties, castor.py:544-557), the only
    path whose results can be reproduced bit-exactly off NVIDIA hardware.  The
    Triton kernel's fp32-score semantics (NN-T, castor.py:407-460) are
    available through ``set_nn_mode("fp32")`` or POLLUX_AMD_NN_MODE=fp32.
  * The quantizer always searches the canonical codebook; a ``codebook``
    argument must equal ``get_h24_codebook`` in its own dtype (checked once
    per tensor and version) -- the reference only ever passes that table.
    Its dtype keeps the reference's meaning (castor.py:521-522, 533, 559):
    the returned vectors are the passed table's values cast to the latent's
    dtype; under NN-B an fp16 or bf16 table gives the fp32 table's indices
    (their bf16 operands are identical and 2*M < c_sq of either table is the
    same test on bf16 scores M); NN-T, whose fp32 scores would meet the
    rounded table's c_sq = 3.99915, accepts fp32 / fp64 tables only.
  * ``chunk_size`` is accepted for signature compatibility; the kernel never
    materialises scores, so it has no memory-bounding role.
"""

from __future__ import annotations

import math
import os
import threading
import weakref
from functools import lru_cache

import numpy as np
import torch

from . import _lib

# =============================================================================
# Constants (castor.py:34-68)
# =============================================================================
friction_c: float = math.sqrt(2.0)
G24: float = 0.065771
gamma: float = G24
H24_DIM: int = 24
s_lattice: float = 1.0 / friction_c
NUMERICAL_EPSILON: float = 1e-8

H24_KISSING_COUNT = 196_560
H24_CODEBOOK_COUNT = H24_KISSING_COUNT + 1
H24_INDEX_BITS = 18
H24_INDEX_MASK = (1 << H24_INDEX_BITS) - 1
BACKBONE_BITS_PER_PARAM = 0.76
BITS_PER_PARAM_INDEX = 18 / H24_DIM
INDICES_PER_CHUNK = 4
BYTES_PER_CHUNK = 9
LEECH_SCALE: float = 1.0 / math.sqrt(8.0)

# "bf16-dense": NN-B with every code scored densely on MFMA (the sweep the structured scorers
# replace; same answers off near-ties), kept as the measured baseline
_MODES = {"bf16": _lib.NN_BF16_SCORES, "fp32": _lib.NN_FP32_SCORES,
          "bf16-dense": _lib.NN_BF16_SCORES | _lib.NN_DENSE_TYPE3}
# quantize_indices also takes "pack": the pack-time NN-P search (pack.py:167-177)
_INDEX_MODES = {**_MODES, "pack": _lib.NN_PACK_FP32,
                 # NN-B through the structured scorers' list-overflow path (their tests)
                 "bf16-rows-sweep": _lib.NN_BF16_SCORES | _lib.NN_T3_ROWS_BY_SWEEP}
_mode_lock = threading.Lock()
_nn_mode = os.environ.get("POLLUX_AMD_NN_MODE", "bf16")
if _nn_mode not in _MODES:
    raise ValueError(f"POLLUX_AMD_NN_MODE must be one of {sorted(_MODES)}, got {_nn_mode!r}")


def set_nn_mode(mode: str) -> None:
    """Select the quantizer semantics: "bf16" (NN-B, default), "fp32" (NN-T), or "bf16-dense" (NN-B with
    every code scored densely instead of by the structured scorers: the same answers off near-ties)."""
    global _nn_mode
    if mode not in _MODES:
        raise ValueError(f"nn mode must be one of {sorted(_MODES)}, got {mode!r}")
    with _mode_lock:
        _nn_mode = mode


def get_nn_mode() -> str:
    return _nn_mode


# =============================================================================
# Codebook (castor.py:146-199, 263-266)
# =============================================================================


@lru_cache(maxsize=1)
def _codebook_cpu() -> torch.Tensor:
    """fp32 [196561, 24]: the native generator's table (castor.py:146-190)."""
    out = np.empty((H24_CODEBOOK_COUNT, H24_DIM), np.float32)
    _lib.check(_lib.lib().plx_codebook_f32(out.ctypes.data, out.size), "plx_codebook_f32")
    t = torch.from_numpy(out)
    t.requires_grad_(False)
    return t


def get_h24_codebook(device: torch.device | str, dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """The 196,561-entry codebook on ``device`` (castor.py:193-199). Index 0 = origin."""
    return _codebook_cpu().to(device=device, dtype=dtype)


def codebook_fingerprint() -> tuple[float, ...]:
    """First 4x4 block of the fp32 codebook as 16 floats (castor.py:263-266)."""
    out = np.empty(16, np.float32)
    _lib.check(_lib.lib().plx_codebook_fingerprint(out.ctypes.data), "plx_codebook_fingerprint")
    return tuple(float(v) for v in out)


# =============================================================================
# Shape / rate helpers (castor.py:269-306)
# =============================================================================


def h24_linear_atom_count(out_features: int, in_features: int) -> int:
    total = int(out_features) * int(in_features)
    if total % H24_DIM != 0:
        raise ValueError(
            f"H24 weight shape ({out_features}, {in_features}) has {total} params, "
            f"not divisible by H24_DIM={H24_DIM}."
        )
    return total // H24_DIM


def assert_h24_divisible(n_features: int, *, name: str = "features") -> None:
    if int(n_features) % H24_DIM != 0:
        raise ValueError(f"Pollux requires {name} divisible by H24_DIM={H24_DIM}; got {n_features}.")


def assert_row_aligned_width(d_model: int) -> None:
    assert_h24_divisible(d_model, name="d_model")


def assert_row_aligned_in_features(in_features: int) -> None:
    assert_h24_divisible(in_features, name="in_features")


def scale_bits_per_param(in_features: int) -> float:
    assert_row_aligned_in_features(in_features)
    return 16.0 / float(in_features)


def h24_linear_scale_row_count(out_features: int) -> int:
    return int(out_features)


# =============================================================================
# 18-bit packing (castor.py:226-260)
# =============================================================================


def pack_indices(indices: torch.Tensor) -> torch.Tensor:
    """Pack 18-bit indices, 4 per 9-byte big-endian group (castor.py:226-246)."""
    _lib.require_device(indices, "pack_indices input")
    flat = indices.reshape(-1)
    n = flat.numel()
    if flat.dtype not in (torch.int64, torch.int32):
        flat = flat.to(torch.int64)
    flat = flat.contiguous()
    out = torch.empty(((n + 3) // 4) * BYTES_PER_CHUNK, dtype=torch.uint8, device=flat.device)
    with torch.cuda.device(flat.device):
        st = _lib.lib().plx_pack_indices(
            _lib.ptr(flat), int(flat.dtype == torch.int64), n, _lib.ptr(out), _lib.stream_of(flat.device)
        )
    _lib.check(st, "pack_indices")
    return out


def unpack_indices(packed: torch.Tensor, num_indices: int) -> torch.Tensor:
    """Inverse of pack_indices; returns int64 [num_indices] (castor.py:249-260)."""
    _lib.require_device(packed, "unpack_indices input")
    flat = packed.reshape(-1)
    if flat.dtype != torch.uint8:
        raise ValueError(f"unpack_indices expects uint8 bytes, got {flat.dtype}")
    flat = flat.contiguous()
    num_indices = int(num_indices)
    if flat.numel() % BYTES_PER_CHUNK != 0:
        raise RuntimeError(f"shape '[-1, 9]' is invalid for input of size {flat.numel()}")
    total = (flat.numel() // BYTES_PER_CHUNK) * INDICES_PER_CHUNK
    if num_indices < 0:  # Python slice semantics of ``indices[:num_indices]``
        num_indices = max(total + num_indices, 0)
    num_indices = min(num_indices, total)
    out = torch.empty(num_indices, dtype=torch.int64, device=flat.device)
    with torch.cuda.device(flat.device):
        st = _lib.lib().plx_unpack_indices(
            _lib.ptr(flat), flat.numel(), num_indices, _lib.ptr(out), _lib.stream_of(flat.device)
        )
    _lib.check(st, "unpack_indices")
    return out


# =============================================================================
# Row RMS normalisation (castor.py:309-339)
# =============================================================================


def row_rms_from_matrix(weight: torch.Tensor) -> torch.Tensor:
    """sqrt(mean(w^2) + 1e-8) per row, fp32 (castor.py:309-313)."""
    if weight.dim() != 2:
        raise ValueError(f"row_rms_from_matrix expects a 2D weight matrix, got {weight.dim()}D.")
    _lib.require_device(weight, "row_rms_from_matrix input")
    w = weight.detach().float().contiguous()
    out = torch.empty(w.shape[0], dtype=torch.float32, device=w.device)
    with torch.cuda.device(w.device):
        st = _lib.lib().plx_row_rms(_lib.ptr(w), w.shape[0], w.shape[1], _lib.ptr(out), _lib.stream_of(w.device))
    _lib.check(st, "row_rms_from_matrix")
    return out


def normalize_matrix_by_row_rms(
    weight: torch.Tensor,
    sigma_rows: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """(weight / sigma.clamp_min(eps), sigma) with sigma per row (castor.py:316-333)."""
    out_f, in_f = weight.shape
    assert_row_aligned_in_features(in_f)
    if sigma_rows is None:
        sigma_rows = row_rms_from_matrix(weight)
    sigma = sigma_rows.reshape(out_f, 1).clamp_min(NUMERICAL_EPSILON)
    return weight / sigma, sigma_rows.reshape(-1)


def scale_matrix_by_row_rms(weight: torch.Tensor, sigma_rows: torch.Tensor) -> torch.Tensor:
    """weight * sigma[:, None] (castor.py:336-339)."""
    out_f, _in_f = weight.shape
    return weight * sigma_rows.reshape(out_f, 1)


# =============================================================================
# Quantizer (castor.py:487-580)
# =============================================================================

_CODEBOOK_DTYPES = (torch.float32, torch.float64, torch.float16, torch.bfloat16)
# id(table) -> (weak reference, _version, equals the canonical table); entries
# leave with their tensor, so a new tensor at a reused address is checked anew
_checked_codebooks: dict[int, tuple] = {}


def _codebook_is_canonical(codebook: torch.Tensor) -> bool:
    if tuple(codebook.shape) != (H24_CODEBOOK_COUNT, H24_DIM):
        raise ValueError(
            f"codebook must have shape ({H24_CODEBOOK_COUNT}, {H24_DIM}); got {tuple(codebook.shape)}"
        )
    if codebook.dtype not in _CODEBOOK_DTYPES:
        raise ValueError(f"codebook dtype must be one of {_CODEBOOK_DTYPES}; got {codebook.dtype}")
    # inference tensors have no version counter: compare them on every call
    version = None if codebook.is_inference() else codebook._version
    key = id(codebook)
    ent = _checked_codebooks.get(key)
    if version is not None and ent is not None and ent[0]() is codebook and ent[1] == version:
        return ent[2]
    ok = bool(torch.equal(codebook, get_h24_codebook(codebook.device, codebook.dtype)))
    if version is not None:
        ref = weakref.ref(codebook, lambda _r, k=key: _checked_codebooks.pop(k, None))
        _checked_codebooks[key] = (ref, version, ok)
    return ok


def _check_codebook(codebook: torch.Tensor, semantics: str) -> None:
    """Refuse a codebook argument whose search semantics this library does not reproduce.

    semantics: "bf16" (NN-B), "fp32" (NN-T) or "pack" (NN-P, pack.py:167-177).
    """
    if not _codebook_is_canonical(codebook):
        raise ValueError(
            "pollux_amd quantizes against the canonical Leech codebook only; the codebook argument "
            "differs from get_h24_codebook()"
        )
    dt = codebook.dtype
    semantics = "bf16" if semantics == "bf16-dense" else semantics
    if semantics == "fp32" and dt in (torch.float16, torch.bfloat16):
        raise ValueError(
            f"NN-T (fp32 scores) against a {dt} codebook compares 2*max with |kp[0]|^2 of the rounded "
            "table (3.99915, castor.py:521-522), which this library does not reproduce; pass the "
            "fp32 table (get_h24_codebook(device, torch.float32)) or use NN-B"
        )
    if semantics == "pack" and dt == torch.bfloat16:
        raise ValueError(
            "the pack-time search (pack.py:167-177) against a bfloat16 codebook scores 3s rounded to "
            "1.0625, which this library does not reproduce; pass the fp32 table as pack.py:259 does"
        )


_GATHER_DTYPES = {torch.float32: _lib.DTYPE_F32, torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16}


def _workspace(n_atoms: int, device: torch.device) -> torch.Tensor:
    nbytes = int(_lib.lib().plx_quantize_workspace_bytes(n_atoms))
    return torch.empty(max(nbytes, 8), dtype=torch.uint8, device=device)


def quantize_indices(x: torch.Tensor, mode: str | None = None) -> torch.Tensor:
    """int32 codebook indices of the atoms of ``x`` ([..., 24], any float dtype).

    mode: "bf16" (NN-B), "bf16-dense" (NN-B, dense sweep), "fp32" (NN-T) or "pack" (NN-P);
    default: the module mode.  ("bf16-rows-sweep": NN-B through the structured scorers' overflow path.)
    """
    _lib.require_device(x, "quantize input")
    xf = x.reshape(-1, H24_DIM).float().contiguous()
    n = xf.shape[0]
    idx = torch.empty(n, dtype=torch.int32, device=xf.device)
    if n == 0:
        return idx
    m = mode or _nn_mode
    if m not in _INDEX_MODES:
        raise ValueError(f"nn mode must be one of {sorted(_INDEX_MODES)}, got {m!r}")
    code = _INDEX_MODES[m]
    ws = _workspace(n, xf.device)
    with torch.cuda.device(xf.device):
        st = _lib.lib().plx_quantize(
            _lib.ptr(xf), n, code, _lib.ptr(idx), _lib.ptr(ws), ws.numel(), _lib.stream_of(xf.device)
        )
    _lib.check(st, "quantize")
    return idx


def gather_codebook(idx: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """codebook.to(dtype).index_select(0, idx) for int32 ``idx`` (castor.py:533,559)."""
    _lib.require_device(idx, "gather_codebook input")
    idx = idx.to(torch.int32).contiguous()
    n = idx.numel()
    gdt = dtype if dtype in _GATHER_DTYPES else torch.float32
    out = torch.empty((n, H24_DIM), dtype=gdt, device=idx.device)
    if n:
        with torch.cuda.device(idx.device):
            st = _lib.lib().plx_gather_codebook(
                _lib.ptr(idx), n, _GATHER_DTYPES[gdt], _lib.ptr(out), _lib.stream_of(idx.device)
            )
        _lib.check(st, "gather_codebook")
    return out if gdt == dtype else out.to(dtype)


def castor_quantize_leech(
    latent: torch.Tensor,
    codebook: torch.Tensor,
    chunk_size: int = 4096,
) -> torch.Tensor:
    """Nearest codebook vector of every 24-d atom of ``latent`` (castor.py:487-560).

    Returns a tensor of ``latent``'s shape and dtype whose atoms are codebook
    rows (the origin where no kissing point is closer than it).
    """
    del chunk_size  # the fused kernel needs no chunking
    orig_shape = latent.shape
    x = latent.reshape(-1, H24_DIM)
    if x.shape[0] == 0:
        return latent.clone()
    _lib.require_device(latent, "castor_quantize_leech input")
    mode = _nn_mode
    _check_codebook(codebook, mode)
    idx = quantize_indices(x, mode=mode)
    # codebook.to(dtype=latent.dtype).index_select(...) of the passed table (castor.py:533, 559)
    out = gather_codebook(idx, codebook.dtype)
    if out.dtype != latent.dtype:
        out = out.to(latent.dtype)
    return out.view(orig_shape)


class CastorQuantizeLeech(torch.autograd.Function):
    """Straight-through estimator around castor_quantize_leech (castor.py:563-580)."""

    @staticmethod
    def forward(ctx, latent, codebook):  # type: ignore[override]
        ctx.mark_non_differentiable(codebook)
        return castor_quantize_leech(latent, codebook)

    @staticmethod
    def backward(ctx, grad_output):  # type: ignore[override]
        return grad_output, None


# =============================================================================
# Fused per-step requantize (pollux.py:874-884) and pack-time scale (pack.py:164)
# =============================================================================


def requantize_h24(latent: torch.Tensor, *, mode: str | None = None, pack: bool = True, weight: bool = True) -> dict:
    """One fused pass of pollux.py:876-884 (+ castor.pack_indices) over an fp32 latent [R, C].

    Returns dict(sigma fp32 [R], indices int32 [R*C/24], packed uint8 or None,
    weight fp32 [R, C] or None) where weight = (codebook[idx] * sigma) * s_lattice
    is what the reference copies into ``p.data``.
    """
    if latent.dim() != 2:
        raise ValueError(f"requantize_h24 expects a 2D latent, got {latent.dim()}D.")
    _lib.require_device(latent, "requantize_h24 input")
    rows, cols = latent.shape
    assert_row_aligned_in_features(cols)
    lat = latent.detach().float().contiguous()
    n = rows * (cols // H24_DIM)
    dev = lat.device
    sigma = torch.empty(rows, dtype=torch.float32, device=dev)
    idx = torch.empty(n, dtype=torch.int32, device=dev)
    packed = torch.empty(((n + 3) // 4) * BYTES_PER_CHUNK, dtype=torch.uint8, device=dev) if pack else None
    w = torch.empty_like(lat) if weight else None
    ws = _workspace(n, dev)
    with torch.cuda.device(dev):
        st = _lib.lib().plx_requantize(
            _lib.ptr(lat), rows, cols, _MODES[mode or _nn_mode], _lib.ptr(sigma), _lib.ptr(idx),
            _lib.ptr(packed), _lib.ptr(w), _lib.ptr(ws), ws.numel(), _lib.stream_of(dev),
        )
    _lib.check(st, "requantize_h24")
    return {"sigma": sigma, "indices": idx, "packed": packed, "weight": w}


def requantize_h24_many(
    latents: list[torch.Tensor], *, mode: str | None = None, pack: bool = True, weight: bool = True
) -> list[dict]:
    """requantize_h24 on several fp32 latents with one scoring sweep over all their atoms.

    The per-step requantize of pollux.py:828-884 for a group of parameters
    (e.g. a layer's matrices) on one device; returns one dict per latent, as
    requantize_h24 does.  Indices equal separate requantize_h24 calls except
    possibly on near-tie atoms.
    """
    if not latents:
        return []
    dev = latents[0].device
    lats, outs, items = [], [], []
    for t in latents:
        if t.dim() != 2:
            raise ValueError(f"requantize_h24_many expects 2D latents, got {t.dim()}D.")
        _lib.require_device(t, "requantize_h24_many input")
        if t.device != dev:
            raise ValueError("requantize_h24_many: all latents must be on one device")
        rows, cols = t.shape
        assert_row_aligned_in_features(cols)
        lat = t.detach().float().contiguous()
        n = rows * (cols // H24_DIM)
        o = {
            "sigma": torch.empty(rows, dtype=torch.float32, device=dev),
            "indices": torch.empty(n, dtype=torch.int32, device=dev),
            "packed": torch.empty(((n + 3) // 4) * BYTES_PER_CHUNK, dtype=torch.uint8, device=dev) if pack else None,
            "weight": torch.empty_like(lat) if weight else None,
        }
        lats.append(lat)
        outs.append(o)
        items.append(_lib.RequantizeItem(_lib.ptr(lat), rows, cols, _lib.ptr(o["sigma"]), _lib.ptr(o["indices"]),
                                         _lib.ptr(o["packed"]), _lib.ptr(o["weight"])))
    total = sum(o["indices"].numel() for o in outs)
    ws = _workspace(total, dev)
    arr = (_lib.RequantizeItem * len(items))(*items)
    with torch.cuda.device(dev):
        st = _lib.lib().plx_requantize_batch(arr, len(items), _MODES[mode or _nn_mode], _lib.ptr(ws), ws.numel(),
                                             _lib.stream_of(dev))
    _lib.check(st, "requantize_h24_many")
    return outs


def sigma16_pack(weight: torch.Tensor) -> torch.Tensor:
    """fp16(clamp(row_rms(w) * sqrt(12), 1e-8)) per row (pack.py:164)."""
    if weight.dim() != 2:
        raise ValueError(f"sigma16_pack expects a 2D weight matrix, got {weight.dim()}D.")
    _lib.require_device(weight, "sigma16_pack input")
    w = weight.detach().float().contiguous()
    out = torch.empty(w.shape[0], dtype=torch.float16, device=w.device)
    with torch.cuda.device(w.device):
        st = _lib.lib().plx_sigma16_pack(_lib.ptr(w), w.shape[0], w.shape[1], _lib.ptr(out), _lib.stream_of(w.device))
    _lib.check(st, "sigma16_pack")
    return out
