"""The structured type-1/2 scorer's mathematics against a brute force over all 98,256 type-1/2 codes.

t12_kernel (quantize.hip) never scores most codes: per octad it takes the best sign pattern from
the parity rule, and at the final bucket it enumerates only the flip sets whose positions each fit
in the room U - lo(M); type 1 from the atoms's largest coordinates.  This CPU test restates that
math in numpy, with exact scores (float64 sums of exact bf16 products, rounded once to fp32 as a
correctly rounded fp32 sum would be) on both sides, and requires the same best bf16 bucket
(round-half-up, castor.py:553-557 semantics as the kernels take them) and the same lowest codebook
row as scoring every code, on atoms built to have many exact ties: sums of two codes, small integer
vectors, scaled codes, spiky atoms, signed zeros, plus random bf16 atoms.  The row tables are built
here from the oracle codebook (oracle/codebook.py), independently of the library's tables.cpp.
"""

import itertools

import numpy as np
import pytest

from oracle import codebook as cb

C1 = np.float64(1.4140625)   # bf16(4 * fp32(1/sqrt 8))
C2 = np.float64(0.70703125)  # bf16(2 * fp32(1/sqrt 8))


def _bucket(v):
    """Round-half-up bf16 bucket of the fp32 rounding of v (v > 0)."""
    u = np.asarray(np.float32(v)).view(np.uint32).astype(np.int64)
    return int((u + 0x8000) >> 16)


@pytest.fixture(scope="module")
def tables():
    raw = cb.codebook_int8().astype(np.int64)
    nz = (raw != 0).sum(1)
    rows12 = np.nonzero((nz == 2) | (nz == 8))[0]
    octs = sorted({int(((raw[r] != 0) * (1 << np.arange(24))).sum()) for r in rows12 if nz[r] == 8})
    assert len(octs) == 759
    oid = {m: i for i, m in enumerate(octs)}
    opos = np.array([[c for c in range(24) if (m >> c) & 1] for m in octs])
    t2_rows = np.zeros((759, 128), np.int64)
    t1_rows = np.zeros((24, 24, 4), np.int64)
    for r in rows12:
        p = np.nonzero(raw[r])[0]
        minus = sum(1 << k for k, c in enumerate(p) if raw[r, c] < 0)
        if nz[r] == 8:
            assert bin(minus).count("1") % 2 == 0
            t2_rows[oid[int(((raw[r] != 0) * (1 << np.arange(24))).sum())], minus & 0x7F] = r
        else:
            t1_rows[p[0], p[1], minus] = r
    scale = np.where(np.abs(raw[rows12]) == 4, C1, np.where(raw[rows12] != 0, C2, 0.0)) * np.sign(raw[rows12])
    return {"raw": raw, "rows12": rows12, "codes": scale, "opos": opos, "t2_rows": t2_rows, "t1_rows": t1_rows}


def _brute(x, t):
    s = t["codes"] @ x  # exact: at most 8 nonzero exact products
    best, row = 0, None
    for r, v in zip(t["rows12"], s):
        if not v > 0:
            continue
        b = _bucket(v)
        if b > best:
            best, row = b, r
        elif b == best:
            row = min(row, r)
    return (best, row) if best >= 0x4000 else (0, None)


def _structured(x, t):
    ax = np.abs(x)
    top = np.sort(ax)[::-1]
    m1 = _bucket(C1 * top[0] + C1 * top[1]) if C1 * (top[0] + top[1]) > 0 else 0
    M = m1
    xo = x[t["opos"]]                      # [759, 8]
    ao = np.abs(xo)
    sg = (np.signbit(xo) * (1 << np.arange(8))).sum(1)
    odd = np.array([bin(int(v)).count("1") & 1 for v in sg])
    best_s = C2 * (ao.sum(1) - 2 * odd * ao.min(1))
    best_b = np.array([_bucket(v) if v > 0 else 0 for v in best_s])
    M = max(M, int(best_b.max()))
    if M < 0x4000:
        return (0, None)
    lo = np.float64(np.uint32((M << 16) - 0x8000).view(np.float32))
    rmin = None
    for o in np.nonzero(best_b == M)[0]:
        U = C2 * ao[o].sum()
        room = (U - lo) + U * 2.0 ** -14
        C = [k for k in range(8) if 2 * C2 * ao[o, k] <= room]
        for nf in range(len(C) + 1):
            for F in itertools.combinations(C, nf):
                if nf % 2 != odd[o]:
                    continue
                fm = sum(1 << k for k in F)
                v = C2 * (ao[o].sum() - 2 * sum(ao[o, k] for k in F))
                if v > 0 and _bucket(v) == M:
                    r = t["t2_rows"][o, (int(sg[o]) ^ fm) & 0x7F]
                    rmin = r if rmin is None else min(rmin, r)
    if m1 == M:
        need = lo - C1 * top[0] - C1 * top[0] * 2.0 ** -13
        C = [i for i in range(24) if C1 * ax[i] >= need]
        for i, j in itertools.combinations(C, 2):
            for e in range(4):
                v = C1 * (-x[i] if e & 1 else x[i]) + C1 * (-x[j] if e & 2 else x[j])
                if v > 0 and _bucket(v) == M:
                    r = t["t1_rows"][i, j, e]
                    rmin = r if rmin is None else min(rmin, r)
    return (M, rmin)


def _bf16(a):
    a = np.ascontiguousarray(a, np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


def _atoms(t):
    rng = np.random.default_rng(31)
    raw = t["raw"].astype(np.float64)
    a, b = rng.integers(1, 196561, 25), rng.integers(1, 196561, 25)
    d = rng.normal(size=(25, 24))
    sp = _bf16(rng.normal(size=(15, 24)) * 0.05)
    sp[np.arange(15), rng.integers(0, 24, 15)] = 4.0
    z = np.zeros((4, 24))
    z[1, 3], z[2, 5], z[3, [1, 7]] = -0.0, 3.0, [3.0, -3.0]
    z[0, :] = -0.0
    return np.concatenate([
        raw[a] + raw[b],                                                       # sums of two codes
        rng.integers(-4, 5, (20, 24)).astype(np.float64),                      # small integer vectors
        rng.integers(-1, 2, (20, 24)).astype(np.float64),
        2.0 * raw[rng.integers(1, 196561, 10)],                                # scaled codes
        sp,                                                                    # one dominant coordinate
        _bf16(d / np.linalg.norm(d, axis=1, keepdims=True) * rng.uniform(0, 16, (25, 1))),
        z])


def test_structured_pair_math_equals_brute_force(tables):
    xs = _atoms(tables)
    bad = [(k, _brute(x, tables), _structured(x, tables)) for k, x in enumerate(xs)]
    bad = [b for b in bad if b[1] != b[2]]
    assert not bad, bad[:5]


def test_every_octad_code_is_its_own_answer(tables):
    # a type-2 code as input: its own bucket is the best, and it is the lowest row there unless an exact tie
    # sits lower; brute force and the structured math must agree on it
    rng = np.random.default_rng(32)
    raw = tables["raw"].astype(np.float64)
    nz = (raw != 0).sum(1)
    picks = rng.choice(np.nonzero(nz == 8)[0], 40)
    for r in picks:
        x = _bf16(raw[r] / np.sqrt(8.0))
        assert _structured(x, tables) == _brute(x, tables)
