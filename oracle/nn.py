"""Oracle: exact nearest-neighbour search for the three reference semantics -- TEST INFRASTRUCTURE ONLY.

The reference has three numerically different quantizers:

NN-B  castor.py:544-557 (the CPU / non-Triton path).  Operands are rounded to
      bf16 (autocast), the contraction is accumulated in fp32 and the *score is
      rounded to bf16* (autocast matmul output dtype), ``.float().max(-1)`` takes
      the first (lowest-index) maximum, and the origin wins when
      ``2*max < c_sq_norm`` with c_sq_norm = fp32 |codebook[1]|^2 = 0x407FFFFF.
NN-T  castor.py:407-460 (the Triton kernel).  Same bf16 operands and fp32
      accumulation, no rounding of the score, lowest index among equal fp32
      maxima, same origin rule.
NN-P  pack.py:167-177 (pack time).  fp32 atoms against the fp32 codebook, fp32
      accumulation, first maximum, origin only when |atom|_2 < 1e-8.

Scores here are computed exactly (float64; every product of two bf16 or two
fp32 values is exact in float64) and then rounded the way each mode rounds.
An fp32 contraction of 24 terms -- whatever its summation order, on a CPU BLAS
or on MFMA, with exact (bf16 x bf16) or once-rounded (fp32 x fp32) products --
lands within ``DELTA_REL * sum_i |x_i c_i|`` of the exact value, with
DELTA_REL = 24 * 2^-24 = 2^-19.4: the worst-case bound of n * u for n = 24
terms and u = 2^-24 (each of at most 23 additions and the product rounds at
most once per term).  It is a bound, not a measurement: MFMA on MI355X was
measured at worst 2^-22.6.  An atom is a *near-tie* when perturbing its
candidate scores anywhere inside that envelope could change the selected
index; every other atom has one answer that any correct fp32 implementation
must reproduce bit-exactly.  Near-ties are counted and reported, never
silently excluded.

Pinned by (tests/test_oracle_nn.py): every codebook vector maps to its own
index in all three modes; x = 0 maps to 0; NN-P is invariant under positive
scaling; the snap boundary 2*M < 0x407FFFFF is exercised from both sides;
agreement with the torch-op restatement of NN-B (oracle/torch_ref.py, the
reference's own ops) on every non-near-tie atom; and, in all three modes on
2,000 atoms (row-scaled weights, sphere atoms, contact-pair midpoints),
agreement with an independent structured decoder that never reads the
sorted table: a +-1 transform over the 4,096 Golay words with the -3
correction for type 3, per-octad |x| sums with the sign-parity fix for type
2, the two largest |x_i| for type 1 (tests/test_oracle_nn.py).
"""

from __future__ import annotations

import numpy as np

from . import codebook as cbm

DELTA_REL = 24 * 2.0 ** -24  # n * u for n = 24 fp32 terms (any summation order)
C_SQ_NORM_F32 = np.uint32(0x407FFFFF).view(np.float32)  # fp32 |codebook[1]|^2 (castor.py:522)
NUMERICAL_EPSILON_F32 = np.float32(1e-8)
BF16_TWO = 0x4000  # bf16 bits of 2.0: NN-B snaps iff the bf16 max is below 2.0

MODE_B, MODE_T, MODE_P = "B", "T", "P"


def _bf16_f64(x: np.ndarray) -> np.ndarray:
    return cbm.bf16_to_f32(cbm.bf16_round_bits(np.asarray(x, np.float32))).astype(np.float64)


def _bf16_of_f64(v: np.ndarray) -> np.ndarray:
    """f64 -> fp32 (RNE) -> bf16 (RNE), returned as exact float64 values."""
    return _bf16_f64(v.astype(np.float32))


class _Tables:
    _cache: dict = {}

    @classmethod
    def get(cls, mode: str):
        if mode not in cls._cache:
            kp32 = cbm.codebook_f32()[1:]
            if mode == MODE_P:
                c64 = kp32.astype(np.float64)
            else:
                c64 = _bf16_f64(kp32)
            cls._cache[mode] = (c64, np.abs(c64), c64.astype(np.float32))
        return cls._cache[mode]


def quantize(x: np.ndarray, mode: str = MODE_B, chunk: int = 128) -> dict:
    """Exact NN search.  x: [N, 24] fp32 (lattice coordinates for B/T, raw atoms for P).

    Returns dict with
      idx       int64 [N]  codebook index (0 = origin), the nominal answer
      near_tie  bool  [N]  True when the answer is not determined within DELTA_REL
      top       float64 [N] nominal winning score (bf16 value for B, fp32 for T/P)
    """
    x = np.ascontiguousarray(np.asarray(x, np.float32).reshape(-1, 24))
    n = x.shape[0]
    c64, cabs, c32 = _Tables.get(mode)
    idx = np.zeros(n, np.int64)
    near = np.zeros(n, bool)
    top = np.zeros(n, np.float64)
    for a in range(0, n, chunk):
        xs = x[a : a + chunk]
        xq = xs.astype(np.float64) if mode == MODE_P else _bf16_f64(xs)
        i, nt, tp = _chunk(xq, mode, c64, cabs, c32)
        idx[a : a + chunk], near[a : a + chunk], top[a : a + chunk] = i, nt, tp
    return {"idx": idx, "near_tie": near, "top": top}


def _chunk(xq, mode, c64, cabs, c32):
    m = xq.shape[0]
    xabs = np.abs(xq)
    # Loose per-atom envelope: sum_i |x_i| * max|c| bounds every code's sum|x_i c_i|.
    dbound = DELTA_REL * xabs.sum(1) * np.abs(c64).max()
    # fp32 filter pass: candidates are codes within a generous margin of the max.
    s32 = xq.astype(np.float32) @ c32.T
    smax32 = s32.max(1).astype(np.float64)
    filt_err = 2.0 ** -16 * xabs.sum(1) * np.abs(c64).max()  # covers fp32 GEMM error
    mag = np.maximum(np.abs(smax32), 2.0 ** -60)
    ulp_bf16 = np.exp2(np.floor(np.log2(mag)) - 7)
    margin = (2 * ulp_bf16 if mode == MODE_B else 0.0) + 4 * dbound + 2 * filt_err
    thr = smax32 - margin
    rows, cols = np.nonzero(s32 >= thr[:, None].astype(np.float32))
    idx = np.zeros(m, np.int64)
    near = np.zeros(m, bool)
    top = np.zeros(m, np.float64)
    order = np.argsort(rows, kind="stable")
    rows, cols = rows[order], cols[order]
    bounds = np.searchsorted(rows, np.arange(m + 1))
    for r in range(m):
        ks = cols[bounds[r] : bounds[r + 1]]  # ascending code order (np.nonzero is row-major)
        S = c64[ks] @ xq[r]
        D = DELTA_REL * (cabs[ks] @ xabs[r])
        if mode == MODE_B:
            idx[r], near[r], top[r] = _decide_b(ks, S, D)
        elif mode == MODE_T:
            idx[r], near[r], top[r] = _decide_t(ks, S, D)
        else:
            idx[r], near[r], top[r] = _decide_p(ks, S, D, xq[r])
    return idx, near, top


def _decide_b(ks, S, D):
    nom = _bf16_of_f64(S)
    lo = _bf16_of_f64(S - D)
    hi = _bf16_of_f64(S + D)
    M = nom.max()
    k_nom = ks[np.argmax(nom == M)]
    near = lo.max() != hi.max()
    if not near:
        Mr = lo.max()
        # A robust snap makes the winner irrelevant; otherwise the lowest code
        # that could reach Mr must certainly reach it.
        if 2.0 * Mr >= float(C_SQ_NORM_F32):
            near = np.argmax(hi == Mr) != np.argmax(lo == Mr)
    snap = 2.0 * M < float(C_SQ_NORM_F32)
    return (0 if snap else int(k_nom) + 1), bool(near), float(M)


def _decide_t(ks, S, D):
    s32 = S.astype(np.float32).astype(np.float64)
    M = s32.max()
    j = int(np.argmax(s32 == M))
    others = np.ones(len(ks), bool)
    others[j] = False
    thr = float(C_SQ_NORM_F32) / 2.0
    if S.max() + D.max() < thr:  # every score certainly snaps to the origin
        near = False
    else:
        near = bool(np.any(S[others] + D[others] >= S[j] - D[j]))
        near |= bool((S[j] - D[j] < thr) != (S[j] + D[j] < thr))
    snap = 2.0 * np.float32(M) < C_SQ_NORM_F32
    return (0 if snap else int(ks[j]) + 1), near, float(M)


def _decide_p(ks, S, D, xr):
    s32 = S.astype(np.float32).astype(np.float64)
    M = s32.max()
    j = int(np.argmax(s32 == M))
    others = np.ones(len(ks), bool)
    others[j] = False
    nrm = float(np.sqrt(np.sum(xr * xr)))
    eps = float(NUMERICAL_EPSILON_F32)
    if nrm < eps * (1 - 1e-6):  # certainly the origin; the winner is irrelevant
        near = False
    else:
        near = bool(np.any(S[others] + D[others] >= S[j] - D[j]))
        near |= abs(nrm - eps) <= 1e-6 * eps
    snap = nrm < eps
    return (0 if snap else int(ks[j]) + 1), near, float(M)


def codebook_vectors(idx: np.ndarray, dtype=np.float32) -> np.ndarray:
    """index_select of the reference codebook (castor.py:533,559)."""
    return cbm.codebook_f32()[np.asarray(idx, np.int64)].astype(dtype)
