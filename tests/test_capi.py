"""The C-ABI library: loads, exports every symbol include/pollux_amd.h declares, host entry points agree
with the oracle, and argument validation fails before any device work (no GPU needed)."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from oracle import codebook as cb
from pollux_amd import _lib, castor

HEADER = Path(__file__).resolve().parents[1] / "include" / "pollux_amd.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(plx_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_symbols()
    assert len(names) >= 15
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES)


def test_version_and_error_string():
    lib = _lib.lib()
    assert lib.plx_version() >= 1
    assert isinstance(lib.plx_last_error(), bytes)


def test_native_codebook_matches_oracle():
    raw = np.empty((196561, 24), np.int8)
    _lib.check(_lib.lib().plx_codebook_raw(raw.ctypes.data, raw.size), "raw")
    assert np.array_equal(raw, cb.codebook_int8())
    assert np.array_equal(castor.get_h24_codebook("cpu", dtype=__import__("torch").float32).numpy(), cb.codebook_f32())
    assert castor.codebook_fingerprint() == cb.fingerprint()


def test_native_codebook_size_checks():
    buf = np.empty(10, np.float32)
    assert _lib.lib().plx_codebook_f32(buf.ctypes.data, buf.size) == _lib.PLX_EINVAL
    assert b"need" in _lib.lib().plx_last_error()
    with pytest.raises(ValueError):
        _lib.check(_lib.lib().plx_codebook_raw(None, 0), "raw")


def test_validation_happens_before_device_work():
    lib = _lib.lib()
    # packed length must be a multiple of 9
    assert lib.plx_unpack_indices(None, 10, 1, None, None) == _lib.PLX_EINVAL
    # num_indices larger than the packed stream holds
    assert lib.plx_unpack_indices(None, 9, 5, None, None) == _lib.PLX_EINVAL
    # unknown quantizer mode
    assert lib.plx_quantize(None, 5, 7, None, None, 0, None) == _lib.PLX_EINVAL
    # in_features not divisible by 24 (castor.py:293-295 message)
    assert lib.plx_requantize(None, 4, 25, 0, None, None, None, None, None, 0, None) == _lib.PLX_EINVAL
    assert b"divisible by H24_DIM=24" in lib.plx_last_error()
    # dequant: packed length inconsistent with the shape
    assert lib.plx_dequant_f16(None, 8, None, 2, 24, None, None) == _lib.PLX_EINVAL
    # gather: unknown dtype
    assert lib.plx_gather_codebook(None, 3, 9, None, None) == _lib.PLX_EINVAL
    # zero-sized work is a no-op success
    assert lib.plx_pack_indices(None, 1, 0, None, None) == _lib.PLX_OK
    assert lib.plx_quantize_workspace_bytes(1000) >= 8000
    # plane layout: the packed length must match the atom count; the flag's batch sizes
    assert lib.plx_h24_plane_layout(None, 18, 9, None, None) == _lib.PLX_EINVAL
    assert lib.plx_h24_plane_layout(None, 0, 0, None, None) == _lib.PLX_OK
    assert lib.plx_dequant_linear(None, 6 * 80, None, 40, 48, None, 16, 3, None, None, 0, None) == _lib.PLX_EINVAL
    assert b"plane layout" in lib.plx_last_error()


def test_composite_entry_points_refuse_before_their_first_launch():
    # non-null dummy addresses (never dereferenced): a too-small workspace or a misaligned latent must be
    # refused as PLX_EINVAL before row_rms / adam / any table build runs, not as a launch error (PLX_EHIP)
    lib = _lib.lib()
    a, b, c = 0x10000, 0x20000, 0x30000
    need = int(lib.plx_quantize_workspace_bytes(4 * 48))
    assert lib.plx_requantize(a, 4, 1152, 0, b, c, None, None, c, need - 1, None) == _lib.PLX_EINVAL
    assert b"workspace" in lib.plx_last_error()
    assert lib.plx_requantize(a + 4, 4, 1152, 0, b, c, None, None, c, need, None) == _lib.PLX_EINVAL
    assert b"aligned" in lib.plx_last_error()
    assert lib.plx_quantize_layer_pack(a, 4, 1152, b, c, None, c, need - 1, None) == _lib.PLX_EINVAL
    assert b"workspace" in lib.plx_last_error()
    step_need = int(lib.plx_pollux_step_workspace_bytes(4, 1152))
    assert step_need > need
    assert lib.plx_pollux_step_h24(a, a, a, a, 4, 1152, a, 0, b, c, None, None, None, c, step_need - 1,
                                   None) == _lib.PLX_EINVAL
    assert lib.plx_pollux_step_h24(a, a, a, a + 4, 4, 1152, a, 0, b, c, None, None, None, c, step_need,
                                   None) == _lib.PLX_EINVAL
    assert b"aligned" in lib.plx_last_error()
    # the batched step: too small a workspace, then a misaligned latent in its second item
    items = (_lib.PolluxStepItem * 2)(_lib.PolluxStepItem(a, a, a, a, 4, 1152, b, c, None, None, None),
                                     _lib.PolluxStepItem(a, a, a, a, 2, 48, b, c, None, None, None))
    bneed = int(lib.plx_pollux_step_batch_workspace_bytes(items, 2))
    assert bneed > int(lib.plx_quantize_workspace_bytes(4 * 48 + 4))
    assert lib.plx_pollux_step_h24_batch(items, 2, a, 0, c, bneed - 1, None) == _lib.PLX_EINVAL
    assert b"workspace" in lib.plx_last_error()
    items[1].latent = a + 4
    assert lib.plx_pollux_step_h24_batch(items, 2, a, 0, c, bneed, None) == _lib.PLX_EINVAL
    assert b"aligned" in lib.plx_last_error()


def test_host_helpers_mirror_reference():
    assert castor.h24_linear_atom_count(1152, 1152) == 55296
    with pytest.raises(ValueError):
        castor.h24_linear_atom_count(5, 5)
    with pytest.raises(ValueError):
        castor.assert_row_aligned_in_features(1000)
    assert castor.scale_bits_per_param(1152) == 16 / 1152
    assert castor.h24_linear_scale_row_count(7) == 7
    assert castor.BITS_PER_PARAM_INDEX == 0.75 and castor.H24_INDEX_MASK == 0x3FFFF


def test_cpu_tensors_are_rejected():
    import torch

    with pytest.raises(ValueError, match="ROCm device"):
        castor.pack_indices(torch.zeros(4, dtype=torch.int64))
    with pytest.raises(ValueError, match="ROCm device"):
        castor.castor_quantize_leech(torch.zeros(2, 24), castor.get_h24_codebook("cpu", torch.float32))
    # N == 0 keeps the reference's early return (castor.py:519-520)
    e = torch.zeros(0, 24)
    assert castor.castor_quantize_leech(e, None).shape == (0, 24)


def test_plane_table_is_the_set_of_codebook_planes():
    # the 8-coordinate planes of every codebook row, as value-id words (byte i = id(c_i) | id(c_{4+i}) << 4)
    lib = _lib.lib()
    n = int(lib.plx_plane_table(None, 0))
    ids = np.zeros(n, np.uint32)
    assert int(lib.plx_plane_table(ids.ctypes.data, n)) == n
    assert np.all(np.diff(ids.astype(np.int64)) > 0)  # ascending, distinct
    values = np.array([0, 1, 2, 4, -4, -3, -2, -1], np.int8)
    nib = (ids[:, None] >> (4 * np.arange(8, dtype=np.uint32))[None, :]) & 0xF
    assert nib.max() < 8
    # nibble 2i is coordinate i, nibble 2i+1 coordinate 4+i
    order = np.array([0, 2, 4, 6, 1, 3, 5, 7])
    planes = values[nib[:, order]]
    raw = cb.codebook_int8().reshape(-1, 3, 8).reshape(-1, 8)
    want = np.unique(raw, axis=0)
    got = np.unique(planes, axis=0)
    assert len(got) == n == len(want) == 4961
    assert np.array_equal(got, want)
