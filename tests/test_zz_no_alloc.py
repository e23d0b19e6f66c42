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


def test_noalloc_call_captured_in_a_graph(dev):
    # torch.cuda.graph captures in the global mode, where a device allocation by any thread fails the
    # capture: the call records only kernels.  Each replay (eager work and a synchronisation between
    # replays, the latent rewritten in place) must equal an eager call on the same latent.
    lib = _lib.lib()
    with torch.cuda.device(dev):
        _lib.check(lib.plx_device_init(), "plx_device_init")
        g = torch.Generator().manual_seed(77)
        rows, cols = 384, 1152
        w = (torch.randn(rows, cols, generator=g) * 0.02).to(dev)
        o = _outputs(rows, cols, dev)
        args = (_lib.ptr(w), rows, cols, _lib.NN_BF16_SCORES, _lib.ptr(o["sigma"]), _lib.ptr(o["indices"]),
                _lib.ptr(o["packed"]), _lib.ptr(o["weight"]))
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # warm-up call outside capture (tables already built by init)
            _lib.check(lib.plx_requantize_noalloc(*args, _lib.stream_of(dev)), "warm-up")
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            st = lib.plx_requantize_noalloc(*args, _lib.stream_of(dev))
        _lib.check(st, "plx_requantize_noalloc under capture")
        for rep in range(3):
            w.copy_((torch.randn(rows, cols, generator=g) * 0.02).to(dev))
            graph.replay()
            torch.cuda.synchronize()
            got = {k: v.clone() for k, v in o.items()}
            want = _requantize(lib, w, _lib.NN_BF16_SCORES, noalloc=False)
            torch.cuda.synchronize()
            print(f"[noalloc] graph replay {rep}: {got['indices'].numel()} atoms", flush=True)
            for k in ("sigma", "indices", "packed", "weight"):
                assert torch.equal(got[k], want[k]), (rep, k)


def test_noalloc_refusal_writes_nothing(dev):
    # a latent that is not 16-byte aligned is refused before row_rms runs: sigma_out keeps its contents
    lib = _lib.lib()
    with torch.cuda.device(dev):
        _lib.check(lib.plx_device_init(), "plx_device_init")
        base = torch.randn(4 * 1152 + 1, device=dev) * 0.02
        w = base[1:]  # 4 bytes past an aligned allocation
        assert _lib.ptr(w) % 16 == 4
        o = _outputs(4, 1152, dev)
        o["sigma"].fill_(-7.0)
        st = lib.plx_requantize_noalloc(_lib.ptr(w), 4, 1152, _lib.NN_BF16_SCORES, _lib.ptr(o["sigma"]),
                                        _lib.ptr(o["indices"]), None, None, _lib.stream_of(dev))
        torch.cuda.synchronize()
        assert st == _lib.PLX_EINVAL and "aligned" in lib.plx_last_error().decode()
        assert torch.all(o["sigma"] == -7.0)
