"""Oracle codebook (castor.py:74-199, 263-266) against closed forms and golden digests."""

import hashlib
import json
from pathlib import Path

import numpy as np

from oracle import codebook as cb

GOLDEN = json.loads((Path(__file__).parent / "golden" / "golden.json").read_text())


def test_golay_weight_distribution():
    w = cb.extended_golay_words()
    assert len(w) == 4096 and len(set(w.tolist())) == 4096
    wt = [bin(int(x)).count("1") for x in w]
    got = {str(k): wt.count(k) for k in sorted(set(wt))}
    assert got == GOLDEN["golay_weight_distribution"]


def test_golay_is_linear_code():
    w = cb.extended_golay_words()
    s = set(w.tolist())
    rng = np.random.default_rng(0)
    for _ in range(200):
        a, b = rng.integers(0, 4096, 2)
        assert int(w[a]) ^ int(w[b]) in s
    # minimum distance 8: every nonzero word has weight >= 8
    assert min(bin(int(x)).count("1") for x in w if x) == 8


def test_type_counts_and_norms():
    raw = cb.raw_minimal_vectors().astype(np.int64)
    nz = (raw != 0).sum(1)
    t1 = (nz == 2).sum()
    t2 = ((nz == 8) & (np.abs(raw).max(1) == 2)).sum()
    t3 = (nz == 24).sum()
    assert {"type1": int(t1), "type2": int(t2), "type3": int(t3)} == GOLDEN["type_counts"]
    assert np.all((raw * raw).sum(1) == 32)


def test_table_shape_alphabet_uniqueness():
    c = cb.codebook_int8()
    assert c.shape == (196561, 24)
    assert np.all(c[0] == 0)
    assert set(np.unique(c).tolist()) == {-4, -3, -2, -1, 0, 1, 2, 4}
    assert len(np.unique(c, axis=0)) == 196561


def test_type3_off_lattice_count():
    # Leech lattice (raw coords): all-odd vectors need x_i = m (mod 4) with the
    # positions where x_i = m+2 (mod 4) ... equivalently sum(x) = 4*m (mod 8)
    # for the vectors of shape (-+3, +-1^23).  The reference puts -3 without
    # flipping by the codeword bit, so exactly half of the type-3 rows fail.
    c = cb.codebook_int8().astype(np.int64)
    odd = np.all(c % 2 != 0, axis=1)
    rows = c[odd]
    assert len(rows) == 98304
    # membership test for odd Leech vectors: x = 1 + 2*codeword-signs - 4*(...):
    # x_i mod 4 must be (1 everywhere except on a Golay codeword where it is 3),
    # up to the global shift; i.e. the set {i : x_i = 3 (mod 4)} is a codeword
    # when sum x = 4 (mod 8), or its complement when sum x = -4 (mod 8).
    words = set(cb.extended_golay_words().tolist())
    bad = 0
    for r in rows:
        m3 = sum(1 << i for i in range(24) if r[i] % 4 == 3)
        total = int(r.sum()) % 8
        ok = (m3 in words) and total in (4,)
        ok |= ((m3 ^ 0xFFFFFF) in words) and total in (4,)
        bad += not ok
    assert bad == GOLDEN["type3_off_lattice"]


def test_order_rows_and_fingerprint():
    c = cb.codebook_int8()
    for k, row in GOLDEN["codebook_rows"].items():
        assert c[int(k)].tolist() == row
    # ascending lexicographic order, coordinate 0 most significant
    a = c[1:].astype(np.int64)
    diff = a[1:] - a[:-1]
    first = np.argmax(diff != 0, axis=1)
    assert np.all(diff[np.arange(len(diff)), first] > 0)
    assert list(cb.fingerprint()) == GOLDEN["fingerprint"]


def test_fp32_values_and_digests():
    f = cb.codebook_f32()
    vals = {float(v) for v in np.unique(f)}
    s = np.float32(1 / np.sqrt(8))
    assert s.view(np.uint32) == int(GOLDEN["constants_f32_hex"]["leech_scale"], 16)
    assert vals == {float(np.float32(k) * s) for k in (-4, -3, -2, -1, 0, 1, 2, 4)}
    norms = (f.astype(np.float64) ** 2).sum(1)[1:]
    assert np.all(np.abs(norms - 4.0) < 1e-4)  # castor.py:159-166
    d = GOLDEN["codebook_sha256"]
    assert hashlib.sha256(cb.codebook_int8().tobytes()).hexdigest() == d["int8_raw"]
    assert hashlib.sha256(f.tobytes()).hexdigest() == d["fp32"]
    assert hashlib.sha256(cb.bf16_round_bits(f).tobytes()).hexdigest() == d["bf16_bits"]
    assert hashlib.sha256(cb.codebook_f16().tobytes()).hexdigest() == d["fp16"]


def test_bf16_fp16_casts_match_closed_form():
    # bf16(s,2s,3s,4s) = 0x3EB5, 0x3F35, 0x3F88, 0x3FB5; fp16 = 0x35A8, 0x39A8, 0x3C3E, 0x3DA8
    s = np.float32(1 / np.sqrt(8))
    v = np.array([np.float32(k) * s for k in (1, 2, 3, 4)], np.float32)
    assert [hex(x) for x in cb.bf16_round_bits(v)] == ["0x3eb5", "0x3f35", "0x3f88", "0x3fb5"]
    assert [hex(x) for x in v.astype(np.float16).view(np.uint16)] == ["0x35a8", "0x39a8", "0x3c3e", "0x3da8"]
