"""The HIP path at BASELINE's full config sizes (configs 2, 3, 4).

The exact oracle (oracle/nn.py) needs ~1.5 ms per atom on the CPU, so at these
sizes each test checks a seeded random sample of atoms against it (indices
bit-exact on every non-near-tie atom) and the whole output through properties
that do not depend on size: every index lies in 0..196,560, unpack(pack(idx))
== idx over the full stream, the packed bytes equal the oracle packer's on the
full stream, and the reconstructed weights equal (c * sigma) * fp32(1/sqrt 2)
for every atom (pollux.py:883).
"""

import numpy as np
import pytest
import torch

from oracle import nn, packing, torch_ref
from pollux_amd import castor

import c3_stress  # tests/ is on sys.path (pytest's rootdir-relative import of this directory)

pytestmark = pytest.mark.gpu

SAMPLE = 1500


def _sample_check(x_cpu, got, mode, seed, label, max_near=0.02):
    rng = np.random.default_rng(seed)
    pick = np.sort(rng.choice(x_cpu.shape[0], size=min(SAMPLE, x_cpu.shape[0]), replace=False))
    r = nn.quantize(x_cpu[pick].numpy(), mode)
    near = r["near_tie"]
    bad = (got[pick] != r["idx"]) & ~near
    print(f"[{label}] sample={len(pick)} near_ties={int(near.sum())} mismatch_non_near={int(bad.sum())}", flush=True)
    assert near.mean() <= max_near
    assert not bad.any(), pick[np.nonzero(bad)[0][:10]]


def _stream_checks(dev, idx):
    """Full-stream properties of an int64 index vector on the device."""
    n = idx.numel()
    assert int(idx.min()) >= 0 and int(idx.max()) <= 196560
    packed = castor.pack_indices(idx)
    assert packed.numel() == (n + 3) // 4 * 9
    assert torch.equal(castor.unpack_indices(packed, n), idx)
    return packed


def test_config4_sweep_full_size(dev):
    # 16,777,200 atoms = 209,715 rows of 1920 (80 atoms per row); directions on
    # S^23, radius U(0, 2) * sqrt(32), fed directly as quantizer input.
    n = 209_715 * 80
    g = torch.Generator(device=dev).manual_seed(404)
    d = torch.randn(n, 24, generator=g, device=dev)
    x = d / d.norm(dim=1, keepdim=True) * (torch.rand(n, 1, generator=g, device=dev) * 2.0 * np.sqrt(32.0))
    del d
    got = castor.quantize_indices(x, mode="bf16").long()
    packed = _stream_checks(dev, got)
    got_cpu = got.cpu().numpy()
    # the packed stream equals the oracle packer's (castor.py:226-246) byte for byte
    assert np.array_equal(packed.cpu().numpy(), packing.pack(got_cpu))
    _sample_check(x.cpu(), got_cpu, "B", 4, "config4")
    # the origin snap fires only for small radii: an atom of norm > 8 has a
    # coordinate of magnitude >= 8/sqrt(24) = 1.63, so its best +-4 pair scores
    # >= 4 * 0.3535 * 1.63 = 2.31, above the 2.0 snap threshold
    big = (x.norm(dim=1) > 8.0).cpu().numpy()
    assert not np.any(got_cpu[big] == 0)


def test_config3_boundary_stress_full_size(dev):
    # Pollux-1920 layer, 1,843,200 atoms in lattice units; 5% of atoms replaced by
    # midpoints of code pairs at raw inner product 16 plus N(0, 1e-3) noise, 5%
    # by random directions at norm sqrt 2 (the origin boundary).
    x, mid_at, near_at = c3_stress.build(303)
    n = x.shape[0]
    got = castor.quantize_indices(x.to(dev), mode="bf16").long()
    _stream_checks(dev, got)
    got_cpu = got.cpu().numpy()
    # sample the stressed atoms and the ordinary ones separately
    _sample_check(x[torch.from_numpy(mid_at)], got_cpu[mid_at], "B", 31, "config3 midpoints", max_near=0.05)
    _sample_check(x[torch.from_numpy(near_at)], got_cpu[near_at], "B", 32, "config3 near-origin")
    rest = np.setdiff1d(np.arange(n), np.concatenate([mid_at, near_at]))
    _sample_check(x[torch.from_numpy(rest)], got_cpu[rest], "B", 33, "config3 unmodified")


def test_config2_requantize_full_size(dev):
    # The bench workload: fused sigma + NN-B + pack + reconstruction of the four
    # Pollux-1152 latents (bf16-rounded N(0, 0.02) master weights held as fp32).
    shapes = [(3456, 1152), (1152, 1152), (4608, 1152), (1152, 4608)]
    g = torch.Generator().manual_seed(2024)
    for k, (r, c) in enumerate(shapes):
        w = (torch.randn(r, c, generator=g) * 0.02).to(torch.bfloat16).float()
        out = castor.requantize_h24(w.to(dev))
        idx = out["indices"].long()
        packed = _stream_checks(dev, idx)
        assert torch.equal(packed, out["packed"])
        sigma = out["sigma"].cpu()
        x, _ = torch_ref.lattice_input(w, sigma)
        idx_cpu = idx.cpu().numpy()
        _sample_check(x.reshape(-1, 24), idx_cpu, "B", 20 + k, f"config2 {r}x{c}")
        # reconstruction of every atom: fp32((c * sigma) * fp32(1/sqrt 2))
        center = torch_ref.codebook_tensor()[torch.from_numpy(idx_cpu)].reshape(r, c)
        assert torch.equal(out["weight"].cpu(), torch_ref.reconstruct(center, sigma))
