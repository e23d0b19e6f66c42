"""Oracle: extended Golay code and the Leech codebook -- TEST INFRASTRUCTURE ONLY.

Restates castor.py:74-199 (codebook) and castor.py:263-266 (fingerprint) in
numpy.  The codebook is held as raw integer coordinates (int8, the reference's
un-scaled vectors) and as the reference's fp32 table ``raw * fp32(1/sqrt(8))``.

Pinned by (tests/test_oracle_codebook.py):
  * closed forms: 4,096 Golay words with weight distribution 1/759/2576/759/1;
    type counts 1,104 / 97,152 / 98,304; squared raw norm 32 for every row;
    196,561 distinct rows; coordinate alphabet {-4,-3,-2,-1,0,1,2,4};
  * the reference's documented quirk: exactly 49,152 type-3 rows fail
    Leech-lattice membership (those whose Golay bit at the -3 position is set);
  * order: rows 1..3 and the last row in closed form, and the 16-float
    fingerprint in closed form (castor.py:263-266);
  * an independent restatement: the product's C++ generator
    (pollux_amd/csrc/codebook.cpp) must produce the same bytes, and both must
    match the SHA-256 digests committed under tests/golden/.
"""

from __future__ import annotations

import functools

import numpy as np

H24_DIM = 24
KISSING_COUNT = 196_560
CODEBOOK_COUNT = KISSING_COUNT + 1
# fp32(1/sqrt(8)) -- castor.py:68 (LEECH_SCALE), applied as an fp32 multiply (castor.py:157)
LEECH_SCALE_F32 = np.float32(1.0 / np.sqrt(8.0))

# x^11 + x^9 + x^7 + x^6 + x^5 + x + 1  (castor.py:74)
GOLAY_POLY = 0xAE3


def golay_remainder(value: int) -> int:
    """Remainder of a GF(2) polynomial division by GOLAY_POLY (castor.py:77-82)."""
    while value.bit_length() > 11:
        value ^= GOLAY_POLY << (value.bit_length() - 12)
    return value


def extended_golay_words() -> np.ndarray:
    """The 4,096 extended Golay codewords in message order (castor.py:85-95).

    Word for message m: bits 22..11 = m, bits 10..0 = remainder of m*x^11,
    bit 23 = parity of the 23-bit word.
    """
    out = np.empty(4096, dtype=np.int64)
    for msg in range(4096):
        w23 = (msg << 11) | golay_remainder(msg << 11)
        out[msg] = w23 | ((bin(w23).count("1") & 1) << 23)
    return out


def _bits(words: np.ndarray) -> np.ndarray:
    """[n] words -> [n, 24] 0/1 matrix, column b = bit b (castor.py:119,136)."""
    return ((words[:, None] >> np.arange(24)[None, :]) & 1).astype(np.int8)


def raw_minimal_vectors() -> np.ndarray:
    """The reference's 196,560 raw vectors, unsorted, as int8 [196560, 24].

    castor.py:98-143.  Type 1: +-4 at two coordinates.  Type 2: +-2 on each
    weight-8 word (octad) with an even number of minus signs.  Type 3: for each
    position p and each word w, -1 where w has a 1, +1 elsewhere, then -3 at p
    (the reference does not flip the -3 by the word's bit at p).
    """
    words = extended_golay_words()
    bits = _bits(words)

    t1 = []
    for i in range(24):
        for j in range(i + 1, 24):
            for a in (-4, 4):
                for b in (-4, 4):
                    r = np.zeros(24, np.int8)
                    r[i], r[j] = a, b
                    t1.append(r)
    t1 = np.stack(t1)

    octads = bits[bits.sum(axis=1) == 8]
    masks = np.arange(256)
    sign_bits = ((masks[:, None] >> np.arange(8)[None, :]) & 1).astype(np.int8)  # 1 -> +
    even = ((8 - sign_bits.sum(axis=1)) % 2) == 0
    signs = (2 * sign_bits[even] - 1).astype(np.int8)  # [128, 8]
    t2 = np.zeros((octads.shape[0] * signs.shape[0], 24), np.int8)
    r = 0
    for o in octads:
        pos = np.nonzero(o)[0]
        blk = t2[r : r + signs.shape[0]]
        blk[:, pos] = 2 * signs
        r += signs.shape[0]

    base = (1 - 2 * bits).astype(np.int8)  # -1 where bit set, +1 elsewhere
    t3 = np.repeat(base[None, :, :], 24, axis=0).copy()  # [pos, word, 24]
    for p in range(24):
        t3[p, :, p] = -3
    t3 = t3.reshape(-1, 24)
    return np.concatenate([t1, t2, t3], axis=0)


@functools.lru_cache(maxsize=1)
def codebook_int8() -> np.ndarray:
    """Sorted raw codebook with the origin prepended: int8 [196561, 24].

    Sort: np.lexsort with keys col23..col0, i.e. col0 is the primary key,
    ascending (castor.py:168-171).  The fp32 scale is strictly monotone on the
    alphabet, so sorting raw integers gives the same order as sorting the fp32
    table.  Origin at index 0 (castor.py:177-178).
    """
    raw = raw_minimal_vectors()
    order = np.lexsort([raw[:, c] for c in range(23, -1, -1)])
    out = np.zeros((CODEBOOK_COUNT, 24), np.int8)
    out[1:] = raw[order]
    out.setflags(write=False)
    return out


def codebook_f32() -> np.ndarray:
    """The reference table ``_build_codebook_cpu()``: fp32 [196561, 24] (castor.py:146-190)."""
    return (codebook_int8().astype(np.float32) * LEECH_SCALE_F32).astype(np.float32)


def fingerprint() -> tuple[float, ...]:
    """First 4x4 block of the fp32 codebook as 16 Python floats (castor.py:263-266)."""
    return tuple(float(v) for v in codebook_f32()[:4, :4].reshape(-1))


def bf16_round_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit pattern, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def codebook_bf16_f32() -> np.ndarray:
    """The codebook after the reference's bf16 cast, as exact fp32 values."""
    return bf16_to_f32(bf16_round_bits(codebook_f32()))


def codebook_f16() -> np.ndarray:
    """``get_h24_codebook(device, torch.float16)``: RNE cast of the fp32 table (castor.py:193-199)."""
    return codebook_f32().astype(np.float16)
