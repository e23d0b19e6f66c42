"""Oracle 18-bit packing (castor.py:226-260) against hand vectors and an independent bit-string restatement."""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import packing

GOLDEN = json.loads((Path(__file__).parent / "golden" / "golden.json").read_text())


@pytest.mark.parametrize("vec", GOLDEN["pack_vectors"], ids=lambda v: str(v["indices"]))
def test_hand_vectors(vec):
    assert packing.pack(vec["indices"]).tobytes().hex() == vec["bytes"]
    assert packing.pack_bitstring(vec["indices"]).hex() == vec["bytes"]


def test_bitstring_agrees_random():
    rng = np.random.default_rng(1)
    for n in (1, 2, 3, 4, 5, 17, 64, 1001):
        idx = rng.integers(0, 1 << 18, n)
        assert packing.pack(idx).tobytes() == packing.pack_bitstring(idx)


@pytest.mark.parametrize("lane", [0, 1, 2, 3])
def test_exhaustive_roundtrip_each_lane(lane):
    v = np.arange(1 << 18, dtype=np.int64)
    idx = np.zeros((v.size, 4), np.int64)
    idx[:, lane] = v
    idx[:, (lane + 1) % 4] = v[::-1]  # a second, different value in a neighbouring lane
    flat = idx.reshape(-1)
    out = packing.unpack(packing.pack(flat), flat.size)
    assert np.array_equal(out, flat)


@pytest.mark.parametrize("n", [0, 1, 2, 3, 4, 5, 6, 7, 8, 9])
def test_padding_and_truncation(n):
    rng = np.random.default_rng(n)
    idx = rng.integers(0, 196561, n)
    p = packing.pack(idx)
    assert p.size == packing.packed_nbytes(n) == ((n + 3) // 4) * 9
    assert np.array_equal(packing.unpack(p, n), idx)
    # padded lanes are zero
    assert np.all(packing.unpack(p, ((n + 3) // 4) * 4)[n:] == 0)


def test_high_bits_are_dropped():
    # castor.py casts to int32 and masks each byte: only the low 18 bits survive
    idx = np.array([(1 << 18) + 7, (5 << 18) + 3, -1, 2**31 + 9], np.int64)
    out = packing.unpack(packing.pack(idx), 4)
    assert out.tolist() == [7, 3, (1 << 18) - 1, 9]
