"""Pins of the oracle's row-scale and dequant functions (oracle/torch_ref.py) by closed forms.

oracle/torch_ref.py restates castor.py:309-339, pack.py:164 and
pollux.py:485-507 with the reference's torch ops.  A slip in that restatement
(eps outside the sqrt, the clamp before the multiply, one rounding where the
reference rounds twice, a multiply where it divides) would be shared by the
HIP kernels written against it, so each function here is checked against an
independent computation: float64 arithmetic rounded once to fp32 (a correctly
rounded result, since 53 >= 2*24 + 2), or numpy's own float16 / float32
conversions.  Each test also shows that the plausible slip fails the same
check, so the check has the power to catch it.
"""

import math

import numpy as np
import pytest
import torch

from oracle import codebook as cb
from oracle import torch_ref

F32_EPS = np.float32(1e-8)  # castor.py:50 as fp32 (0x322BCC77)
SQRT12_F32 = np.uint32(0x405DB3D7).view(np.float32)  # fp32(sqrt 12), pack.py:164
S_LATTICE_F32 = np.uint32(0x3F3504F3).view(np.float32)  # fp32(1/sqrt 2), castor.py:47


def _ulps(a, b):
    ai = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    bi = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(ai - bi)


def _f32(x64):
    return np.asarray(x64, np.float64).astype(np.float32)


# ---------------------------------------------------------------- row RMS ----


def _rms_closed_form(w32: np.ndarray) -> np.ndarray:
    """sqrt(mean(fp32(w^2)) + fp32(1e-8)), the mean and sqrt in float64, rounded once to fp32."""
    with np.errstate(over="ignore"):
        sq = (w32 * w32).astype(np.float64)  # the reference squares in fp32 (w.pow(2)), incl. overflow to inf
    return _f32(np.sqrt(sq.mean(axis=1) + np.float64(F32_EPS)))


def _rms_rows():
    g = torch.Generator().manual_seed(31)
    rows = [
        (torch.randn(64, 1152, generator=g) * 0.02).numpy(),
        (torch.randn(16, 4608, generator=g) * 0.02).numpy(),
        (torch.randn(8, 1920, generator=g) * 3.0).numpy(),
        np.zeros((2, 1152), np.float32),  # sigma = sqrt(1e-8) = 1e-4
    ]
    huge = np.zeros((2, 1152), np.float32)
    huge[0, 7] = 1e18  # one huge element: its square dominates
    huge[1, :] = 1e-3
    huge[1, 100] = 1e17
    sub = np.full((2, 1152), 1e-41, np.float32)  # subnormals: squares underflow to 0
    sub[1, ::2] = -3e-39
    rows += [huge, sub]
    return np.concatenate([r.reshape(-1, 1152) if r.shape[1] == 1152 else r[:, :1152] for r in rows]).astype(
        np.float32
    )


def test_row_rms_closed_form():
    w = _rms_rows()
    got = torch_ref.row_rms(torch.from_numpy(w)).numpy()
    want = _rms_closed_form(w)
    d = _ulps(got, want)
    assert d.max() <= 1, (d.max(), np.nonzero(d > 1)[0][:8])
    assert np.all(got[-4:-2] > 0) and got[-2] == np.float32(1e-4)  # subnormal rows: the eps alone
    # the slip "sqrt(mean) + eps" (eps outside the root) fails the same bound
    # on every N(0, 0.02) row (the training statistics) and on the zero rows
    slip = _f32(np.sqrt((w.astype(np.float64) ** 2).mean(axis=1)) + 1e-8)
    bad = _ulps(slip, want) > 1
    assert bad[:80].all() and bad[88:90].all()


def test_row_rms_overflowing_square():
    # fp32(w^2) overflows: the reference's sigma is +inf, and so is the closed form
    w = np.full((1, 48), 1e-2, np.float32)
    w[0, 3] = 3e19
    got = torch_ref.row_rms(torch.from_numpy(w)).numpy()
    assert np.isinf(got[0]) and np.isinf(_rms_closed_form(w)[0])


def test_row_rms_wide_rows_random_widths():
    rng = np.random.default_rng(5)
    for cols in (24, 72, 1920, 7680):
        w = (rng.standard_normal((32, cols)) * rng.uniform(1e-4, 10, (32, 1))).astype(np.float32)
        d = _ulps(torch_ref.row_rms(torch.from_numpy(w)).numpy(), _rms_closed_form(w))
        assert d.max() <= 1, (cols, d.max())


# ------------------------------------------------- normalise / lattice input ----


def _div_f32(a32, b32):
    """Correctly rounded fp32 quotient: the float64 quotient rounded once."""
    return _f32(np.asarray(a32, np.float64) / np.asarray(b32, np.float64))


def test_lattice_input_closed_form():
    g = torch.Generator().manual_seed(41)
    w = torch.randn(96, 1152, generator=g) * 0.02  # 110,592 elements
    x, sigma = torch_ref.lattice_input(w)
    w32, s32 = w.numpy(), sigma.numpy()
    normed = _div_f32(w32, np.maximum(s32, F32_EPS)[:, None])
    want = _div_f32(normed, S_LATTICE_F32)
    assert np.array_equal(x.numpy().view(np.uint32), want.view(np.uint32))
    # the slip "multiply by fp32(sqrt 2)" instead of dividing by fp32(1/sqrt 2) differs
    slip = _f32(normed.astype(np.float64) * np.float64(np.float32(math.sqrt(2.0))))
    assert np.mean(slip != want) > 0.05
    # and so does folding both divisions into one by sigma * s_lattice
    slip2 = _div_f32(w32, _f32(s32.astype(np.float64) * np.float64(S_LATTICE_F32))[:, None])
    assert np.mean(slip2 != want) > 0.05


def test_normalize_sigma_clamp():
    # castor.py:330-333: sigma.clamp_min(1e-8), then an IEEE division
    w = np.linspace(-1e-6, 1e-6, 4 * 48, dtype=np.float32).reshape(4, 48)
    sigma = np.array([0.0, 1e-9, np.float32(1e-8), 3e-8], np.float32)
    got, back = torch_ref.normalize(torch.from_numpy(w), torch.from_numpy(sigma))
    want = _div_f32(w, np.maximum(sigma, F32_EPS)[:, None])
    assert np.array_equal(got.numpy().view(np.uint32), want.view(np.uint32))
    assert np.array_equal(back.numpy(), sigma)  # the unclamped sigma is returned


# ------------------------------------------------------------------ sigma16 ----


def _sigma16_closed_form(s32: np.ndarray) -> np.ndarray:
    prod = _f32(s32.astype(np.float64) * np.float64(SQRT12_F32))  # exact product, rounded once
    with np.errstate(over="ignore"):
        return np.maximum(prod, F32_EPS).astype(np.float16)  # numpy's fp32 -> fp16 cast is RNE


def _sigma16_inputs():
    rng = np.random.default_rng(9)
    s = [np.exp(rng.uniform(np.log(1e-12), np.log(1e6), 20000)).astype(np.float32)]
    # sigma * sqrt12 on and next to fp16 rounding midpoints, across the normal range
    h = np.arange(0x0400, 0x7BFF, 37, dtype=np.uint16).view(np.float16).astype(np.float64)
    nxt = np.nextafter(h.astype(np.float16), np.float16(np.inf)).astype(np.float64)
    mids = (h + nxt) / 2
    for m in (mids, h):
        base = _f32(m / float(SQRT12_F32))
        s += [base, np.nextafter(base, np.float32(0)), np.nextafter(base, np.float32(np.inf))]
    # subnormal fp16 outputs, the clamp region, zero, overflow of fp16
    s.append(np.array([0.0, 1e-12, 2.8e-9, 2.9e-9, 1e-8, 1.7e-8, 5e-8, 1e-4, 18918.0, 18919.0, 3e4, 1e30],
                      np.float32))
    return np.concatenate(s).astype(np.float32)


def test_sigma16_from_sigma_closed_form():
    s = _sigma16_inputs()
    got = torch_ref.sigma16_from_sigma(torch.from_numpy(s)).numpy()
    want = _sigma16_closed_form(s)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    assert np.isinf(want[-1]) and want[-12] == 0  # overflow to inf; sigma 0 clamps to 1e-8, fp16 zero
    # the slip "clamp sigma first, then multiply" differs in the clamp region
    with np.errstate(over="ignore"):
        slip = _f32(np.maximum(s, F32_EPS).astype(np.float64) * np.float64(SQRT12_F32)).astype(np.float16)
        # a single rounding of the exact sigma * sqrt(12) to fp16 differs on some boundary inputs
        single = np.maximum(s.astype(np.float64) * math.sqrt(12.0), 1e-8).astype(np.float16)
    assert np.any(slip.view(np.uint16) != want.view(np.uint16))
    assert np.any(single.view(np.uint16) != want.view(np.uint16))


def test_sigma16_pack_composes_row_rms():
    g = torch.Generator().manual_seed(10)
    w = torch.randn(200, 1152, generator=g) * 0.02
    got = torch_ref.sigma16_pack(w).numpy()
    want = _sigma16_closed_form(_rms_closed_form(w.numpy()))
    # row_rms is within 1 ulp of its closed form; the fp16 result then within 1 fp16 ulp
    d = np.abs(got.view(np.int16).astype(np.int64) - want.view(np.int16).astype(np.int64))
    assert d.max() <= 1 and np.mean(d == 0) > 0.99


# -------------------------------------------------------------- reconstruct ----


def test_reconstruct_closed_form():
    rng = np.random.default_rng(12)
    idx = rng.integers(0, 196561, 40 * 48)
    c = cb.codebook_f32()[idx].reshape(40, 1152)
    sigma = (rng.uniform(1e-3, 0.1, 40)).astype(np.float32)
    got = torch_ref.reconstruct(torch.from_numpy(c), torch.from_numpy(sigma)).numpy()
    cs = _f32(c.astype(np.float64) * sigma[:, None].astype(np.float64))
    want = _f32(cs.astype(np.float64) * np.float64(S_LATTICE_F32))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # the other association, c * (sigma * s), differs on a fraction of the elements
    ss = _f32(sigma.astype(np.float64) * np.float64(S_LATTICE_F32))
    slip = _f32(c.astype(np.float64) * ss[:, None].astype(np.float64))
    assert np.sum((slip != want) & (c != 0)) > 100


# -------------------------------------------------------------- materialize ----


def _alphabet_codes():
    """Three codebook indices whose rows together hold all 8 raw values {-4,-3,-2,-1,0,1,2,4}."""
    raw = cb.codebook_int8()
    t1 = np.nonzero((raw == 4).any(1) & (raw == -4).any(1))[0][0]
    t2 = np.nonzero((raw == 2).any(1) & (raw == -2).any(1))[0][0]
    t3 = np.nonzero((raw == -3).any(1) & (raw == 1).any(1) & (raw == -1).any(1))[0][0]
    codes = np.array([t1, t2, t3])
    assert set(np.unique(raw[codes])) == {-4, -3, -2, -1, 0, 1, 2, 4}
    return codes


def test_materialize_exhaustive_fp16_sigma():
    # every finite fp16 sigma bit pattern (both signs) x every alphabet value
    bits = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)
    sig16 = bits.view(np.float16)
    sig16 = sig16[np.isfinite(sig16)]
    assert sig16.size == 63488
    codes = _alphabet_codes()
    rows = sig16.size
    idx = np.tile(codes, rows)
    got = torch_ref.materialize(torch.from_numpy(idx), torch.from_numpy(sig16), rows, 72).numpy()
    c16 = cb.codebook_f32()[codes].reshape(-1).astype(np.float16)  # fp16 table values (castor.py:193)
    with np.errstate(over="ignore"):
        p = (c16[None, :].astype(np.float32) * sig16[:, None].astype(np.float32)).astype(np.float16)
        want = (p.astype(np.float32) * S_LATTICE_F32).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    # one rounding of the exact c16 * sigma16 * s_lattice differs from the reference's two
    with np.errstate(over="ignore"):
        single = (c16[None, :].astype(np.float64) * sig16[:, None].astype(np.float64) * np.float64(S_LATTICE_F32))
        single = single.astype(np.float32).astype(np.float16)
    assert np.sum(single.view(np.uint16) != want.view(np.uint16)) > 1000


# ------------------------------------------------------------------ linear ----


def test_linear_fp32_error_bound():
    g = torch.Generator().manual_seed(13)
    k = 1920
    x = torch.randn(64, k, generator=g)
    w16 = (torch.randn(96, k, generator=g) * 0.03).to(torch.float16)
    got = torch_ref.linear_fp32(x, w16).numpy().astype(np.float64)
    x64, w64 = x.numpy().astype(np.float64), w16.numpy().astype(np.float64)
    exact = x64 @ w64.T
    bound = k * 2.0 ** -24 * (np.abs(x64) @ np.abs(w64).T)  # any fp32 summation order of k exact products
    assert np.all(np.abs(got - exact) <= bound)

    def rel_l2(y):
        return np.linalg.norm(y - exact) / np.linalg.norm(exact)

    assert rel_l2(got) < 1e-6
    # bf16-rounded weights (the literal F.linear(x_bf16, W.to(bf16)) rounding) are 1e-3 off
    wb = w16.to(torch.bfloat16).float().numpy().astype(np.float64)
    assert rel_l2(x64 @ wb.T) > 1e-4
    # and the transposed operand is not a small error
    assert np.abs(got - exact).max() < 1e-3 * np.abs(exact).max()


def test_linear_as_reference_rounds_weight_to_x_dtype():
    g = torch.Generator().manual_seed(14)
    x = torch.randn(3, 240, generator=g).to(torch.bfloat16)
    w16 = (torch.randn(8, 240, generator=g) * 0.03).to(torch.float16)
    got = torch_ref.linear_as_reference(x, w16).numpy().astype(np.float64)
    wb = w16.to(torch.bfloat16).float().numpy().astype(np.float64)
    exact = x.float().numpy().astype(np.float64) @ wb.T
    bound = 240 * 2.0 ** -24 * (np.abs(x.float().numpy().astype(np.float64)) @ np.abs(wb).T)
    assert np.all(np.abs(got - exact) <= bound)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_codebook_tensor_dtypes(dtype):
    t = torch_ref.codebook_tensor(dtype)
    assert t.shape == (196561, 24) and t.dtype == dtype
    assert np.array_equal(t.float().numpy(), cb.codebook_f32().astype(np.dtype(str(dtype).split(".")[1])).astype(
        np.float32))
