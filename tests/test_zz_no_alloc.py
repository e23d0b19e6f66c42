"""plx_requantize_noalloc (the allocation-free requantize) against plx_requantize, through the C ABI.

The allocation-free entry point shares plx_requantize's kernels and uses a
library-owned device array as their workspace; its outputs must equal the
workspace entry point's bit for bit (same kernels, same inputs).  Two calls
in a row, the second on a smaller matrix, so the second runs on what the
first left in the shared array.
"""

import ctypes

import pytest
import torch

from pollux_amd import _lib

pytestmark = pytest.mark.gpu


def _outputs(rows, cols, dev):
    n = rows * cols // 24
    return {
        "sigma": torch.empty(rows, dtype=torch.float32, device=dev),
        "indices": torch.empty(n, dtype=torch.int32, device=dev),
        "packed": torch.empty((n + 3) // 4 * 9, dtype=torch.uint8, device=dev),
        "weight": torch.empty(rows, cols, dtype=torch.float32, device=dev),
    }


def _requantize(lib, w, mode, noalloc):
    rows, cols = w.shape
    o = _outputs(rows, cols, w.device)
    stream = _lib.stream_of(w.device)
    args = (_lib.ptr(w), rows, cols, mode, _lib.ptr(o["sigma"]), _lib.ptr(o["indices"]), _lib.ptr(o["packed"]),
            _lib.ptr(o["weight"]))
    if noalloc:
        st = lib.plx_requantize_noalloc(*args, stream)
    else:
        nbytes = int(lib.plx_quantize_workspace_bytes(rows * cols // 24))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=w.device)
        st = lib.plx_requantize(*args, _lib.ptr(ws), ws.numel(), stream)
    _lib.check(st, "plx_requantize_noalloc" if noalloc else "plx_requantize")
    return o


@pytest.mark.parametrize("mode", [_lib.NN_BF16_SCORES, _lib.NN_FP32_SCORES])
def test_noalloc_equals_workspace_entry_point(dev, mode):
    lib = _lib.lib()
    with torch.cuda.device(dev):
        _lib.check(lib.plx_device_init(), "plx_device_init")
        g = torch.Generator().manual_seed(5150 + mode)
        # a Pollux-1920 up projection (614,400 atoms), then a smaller ragged matrix
        for shape in [(7680, 1920), (37, 1152)]:
            w = (torch.randn(*shape, generator=g) * 0.02).to(dev)
            got = _requantize(lib, w, mode, noalloc=True)
            want = _requantize(lib, w, mode, noalloc=False)
            torch.cuda.synchronize()
            print(f"[noalloc] mode {mode} {shape}: {got['indices'].numel()} atoms", flush=True)
            for k in ("sigma", "indices", "packed", "weight"):
                assert torch.equal(got[k], want[k]), (shape, k)


def test_noalloc_rejects_more_than_its_maximum(dev):
    lib = _lib.lib()
    max_atoms = 1048576  # PLX_NOALLOC_MAX_ATOMS
    with torch.cuda.device(dev):
        _lib.check(lib.plx_device_init(), "plx_device_init")
        w = torch.zeros(8, 24, device=dev)
        o = _outputs(8, 24, dev)
        # rows * cols / 24 = max + 1: refused before anything is read or launched
        st = lib.plx_requantize_noalloc(_lib.ptr(w), max_atoms + 1, 24, 0, _lib.ptr(o["sigma"]),
                                        _lib.ptr(o["indices"]), None, None, _lib.stream_of(dev))
        assert st == _lib.PLX_EINVAL
        assert "maximum" in lib.plx_last_error().decode()
        # exactly the maximum passes validation (checked without launching: a null latent is refused next)
        st = lib.plx_requantize_noalloc(None, max_atoms, 24, 0, None, None, None, None, _lib.stream_of(dev))
        assert st == _lib.PLX_EINVAL and "null pointer" in lib.plx_last_error().decode()
