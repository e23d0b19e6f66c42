"""Oracle: 18-bit index packing -- TEST INFRASTRUCTURE ONLY.

Restates castor.py:226-260.  Four 18-bit indices form one 9-byte group: the
72-bit big-endian concatenation i0|i1|i2|i3.  The index stream is zero-padded
to a multiple of four; unpack truncates back to ``num_indices`` and returns
int64.  Indices are taken modulo 2^18 bit-wise exactly as the reference's
shifts and masks do (the reference masks every byte with 0xFF after shifting
an int32; bits above 17 of i1..i3 are masked away, bits above 17 of i0 would
leak into nothing because b0 = (i0 >> 10) & 0xFF keeps bits 10..17 only).

Pinned by (tests/test_oracle_packing.py): hand-computed vectors, a
bit-string restatement (format each index as 18 binary digits, concatenate,
cut into bytes), exhaustive round trips over all 2^18 values in every lane
position, and the padding / truncation cases N % 4 in {1, 2, 3}.
"""

from __future__ import annotations

import numpy as np

INDEX_BITS = 18
INDICES_PER_GROUP = 4
BYTES_PER_GROUP = 9


def packed_nbytes(num_indices: int) -> int:
    return ((int(num_indices) + 3) // 4) * 9


def pack(indices: np.ndarray) -> np.ndarray:
    """castor.pack_indices: any-int [N] -> uint8 [ceil(N/4)*9]."""
    idx = np.asarray(indices).reshape(-1).astype(np.int64)
    pad = (-len(idx)) % 4
    if pad:
        idx = np.concatenate([idx, np.zeros(pad, np.int64)])
    g = idx.reshape(-1, 4).astype(np.int32).astype(np.int64)
    i0, i1, i2, i3 = g[:, 0], g[:, 1], g[:, 2], g[:, 3]
    out = np.empty((g.shape[0], 9), np.int64)
    out[:, 0] = i0 >> 10
    out[:, 1] = i0 >> 2
    out[:, 2] = ((i0 & 0x03) << 6) | ((i1 >> 12) & 0x3F)
    out[:, 3] = i1 >> 4
    out[:, 4] = ((i1 & 0x0F) << 4) | ((i2 >> 14) & 0x0F)
    out[:, 5] = i2 >> 6
    out[:, 6] = ((i2 & 0x3F) << 2) | ((i3 >> 16) & 0x03)
    out[:, 7] = i3 >> 8
    out[:, 8] = i3
    return (out & 0xFF).astype(np.uint8).reshape(-1)


def unpack(packed: np.ndarray, num_indices: int) -> np.ndarray:
    """castor.unpack_indices: uint8 [9k] -> int64 [num_indices]."""
    b = np.asarray(packed, dtype=np.uint8).reshape(-1, 9).astype(np.int64)
    i0 = (b[:, 0] << 10) | (b[:, 1] << 2) | (b[:, 2] >> 6)
    i1 = ((b[:, 2] & 0x3F) << 12) | (b[:, 3] << 4) | (b[:, 4] >> 4)
    i2 = ((b[:, 4] & 0x0F) << 14) | (b[:, 5] << 6) | (b[:, 6] >> 2)
    i3 = ((b[:, 6] & 0x03) << 16) | (b[:, 7] << 8) | b[:, 8]
    return np.stack([i0, i1, i2, i3], axis=1).reshape(-1)[: int(num_indices)].astype(np.int64)


def pack_bitstring(indices) -> bytes:
    """Independent restatement for small inputs: 18-digit binary strings, concatenated."""
    idx = [int(v) & 0x3FFFF for v in indices]
    idx += [0] * ((-len(idx)) % 4)
    bits = "".join(format(v, "018b") for v in idx)
    return bytes(int(bits[i : i + 8], 2) for i in range(0, len(bits), 8))
