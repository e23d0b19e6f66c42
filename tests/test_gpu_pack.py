"""HIP 18-bit pack / unpack (castor.py:226-260) against the oracle, bit-exact."""

import numpy as np
import pytest
import torch

from oracle import packing
from pollux_amd import castor

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 8, 1023, 1024, 1025, 4097, 65537, 1_000_003])
@pytest.mark.parametrize("dtype", [torch.int64, torch.int32])
def test_pack_matches_oracle(dev, n, dtype):
    g = torch.Generator().manual_seed(n)
    idx = torch.randint(0, 196561, (n,), generator=g, dtype=torch.int64)
    got = castor.pack_indices(idx.to(dtype).to(dev)).cpu().numpy()
    assert np.array_equal(got, packing.pack(idx.numpy()))


@pytest.mark.parametrize("lane", [0, 1, 2, 3])
def test_exhaustive_values_every_lane(dev, lane):
    v = torch.arange(1 << 18, dtype=torch.int64)
    idx = torch.zeros(v.numel(), 4, dtype=torch.int64)
    idx[:, lane] = v
    idx[:, (lane + 2) % 4] = v.flip(0)
    flat = idx.reshape(-1)
    p = castor.pack_indices(flat.to(dev))
    assert np.array_equal(p.cpu().numpy(), packing.pack(flat.numpy()))
    back = castor.unpack_indices(p, flat.numel()).cpu()
    assert torch.equal(back, flat)


@pytest.mark.parametrize("nbytes,num", [(9, 1), (9, 4), (18, 5), (9 * 1000, 3999), (9 * 257, 1028), (9 * 100_001, 400_001)])
def test_unpack_arbitrary_bytes(dev, nbytes, num):
    g = torch.Generator().manual_seed(nbytes + num)
    b = torch.randint(0, 256, (nbytes,), generator=g, dtype=torch.uint8)
    got = castor.unpack_indices(b.to(dev), num).cpu().numpy()
    assert got.dtype == np.int64
    assert np.array_equal(got, packing.unpack(b.numpy(), num))


def test_high_bits_and_negative_inputs(dev):
    idx = torch.tensor([(1 << 18) + 7, (5 << 18) + 3, -1, 2**31 + 9, 196560], dtype=torch.int64)
    got = castor.pack_indices(idx.to(dev)).cpu().numpy()
    assert np.array_equal(got, packing.pack(idx.numpy()))


def test_unaligned_views(dev):
    g = torch.Generator().manual_seed(3)
    base = torch.randint(0, 196561, (4099,), generator=g, dtype=torch.int64).to(dev)
    view = base[3:]  # 24-byte offset: not 16-byte aligned
    got = castor.pack_indices(view).cpu().numpy()
    assert np.array_equal(got, packing.pack(base[3:].cpu().numpy()))
    p = castor.pack_indices(base)
    buf = torch.zeros(p.numel() + 1, dtype=torch.uint8, device=dev)
    buf[1:] = p
    back = castor.unpack_indices(buf[1:], base.numel())
    assert torch.equal(back, base)


def test_empty(dev):
    assert castor.pack_indices(torch.zeros(0, dtype=torch.int64, device=dev)).numel() == 0
    assert castor.unpack_indices(torch.zeros(0, dtype=torch.uint8, device=dev), 0).numel() == 0


def test_sweep_scale_roundtrip(dev):
    # BASELINE config 4 size: 16,777,216 indices
    n = 16_777_216
    g = torch.Generator(device=dev).manual_seed(4)
    idx = torch.randint(0, 196561, (n,), generator=g, device=dev, dtype=torch.int64)
    p = castor.pack_indices(idx)
    assert p.numel() == n // 4 * 9 == 37_748_736
    assert torch.equal(castor.unpack_indices(p, n), idx)
    # spot-check bytes against the oracle on a slice of whole groups
    a, b = 4 * 123_457, 4 * 123_457 + 4 * 4096
    assert np.array_equal(p[a // 4 * 9 : b // 4 * 9].cpu().numpy(), packing.pack(idx[a:b].cpu().numpy()))
