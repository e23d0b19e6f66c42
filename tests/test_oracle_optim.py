"""The optimiser-step oracle (oracle/optim.py) against the reference's torch ops on the CPU.

Each rounding rule the oracle states is pinned on its own against the torch op
it restates, then the whole H24 step (pollux.py:815-878) bit for bit, in
regimes with and without the per-atom speed cap.
"""

import math

import numpy as np
import pytest
import torch

from oracle import optim, torch_ref

F32 = np.float32


def _state(seed, rows, cols, gscale):
    g = torch.Generator().manual_seed(seed)
    grad = torch.randn(rows, cols, generator=g) * gscale
    m = torch.randn(rows, cols, generator=g) * gscale * 0.3
    v = torch.rand(rows, cols, generator=g) * gscale * gscale
    latent = torch.randn(rows, cols, generator=g) * 0.02
    return grad, m, v, latent


def test_add_alpha_is_fused():
    g = torch.randn(1 << 16) * 1e-3
    m = torch.randn(1 << 16) * 1e-3
    b1 = 1.0 - math.sqrt(optim.GAMMA)
    want = m.clone().mul_(b1).add_(g, alpha=1.0 - b1).numpy()
    got = optim.fma(g.numpy(), F32(1.0 - b1), (m.numpy() * F32(b1)).astype(F32))
    assert np.array_equal(want, got)


def test_addcmul_is_fused_after_the_scalar_product():
    g = torch.randn(1 << 16) * 1e-3
    v = torch.rand(1 << 16) * 1e-6
    b2 = 1.0 - optim.GAMMA
    want = v.clone().mul_(b2).addcmul_(g, g, value=1.0 - b2).numpy()
    got = optim.fma((F32(1.0 - b2) * g.numpy()).astype(F32), g.numpy(), (v.numpy() * F32(b2)).astype(F32))
    assert np.array_equal(want, got)


def test_vector_norm_order_of_24_element_rows():
    x = torch.randn(8192, 24) * 1e-3
    want = torch.linalg.vector_norm(x, dim=-1).numpy()
    assert np.array_equal(want, optim.atom_norm(x.numpy()))


def test_cpu_sqrt_is_faithful_not_correctly_rounded():
    # why the oracle states sqrt as correctly rounded (the GPU's sqrtf) and the
    # torch restatement computes it through float64
    x = torch.rand(1 << 18) * 1e-6
    want = np.sqrt(x.numpy().astype(np.float64)).astype(F32)
    assert np.array_equal(np.sqrt(x.numpy()), want)  # numpy's fp32 sqrt is correctly rounded
    got = torch.sqrt(x).numpy()
    ulps = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1


def test_float_over_tensor_is_a_reciprocal_product():
    t = torch.rand(1 << 16) * 1e-3 + 1e-7
    cap = optim.KINEMATIC_LIMIT * optim.S_LATTICE
    want = (cap / t).numpy()
    got = ((F32(1.0) / t.numpy()).astype(F32) * F32(cap)).astype(F32)
    assert np.array_equal(want, got)


@pytest.mark.parametrize("heat,step,d,gscale", [
    (0.065771, 0, 1152, 1e-3),   # minimum heat, first step (bias correction ~ 1 - beta)
    (0.5, 7, 1920, 1e-3),        # width inertia > 1
    (1.0, 0, 1152, 1e-2),        # maximum heat: most atoms hit the speed cap
    (0.8, 1000, 1152, 1e-4),     # late step, bias correction ~ 1
])
def test_h24_step_matches_torch_ops(heat, step, d, gscale):
    grad, m, v, latent = _state(step + 11, 96, 1152, gscale)
    inertia = 1.0 + math.sqrt(2.0) * math.log(d / ((24.0 * math.sqrt(2.0)) ** 2))
    sc = optim.scalars(heat, step, inertia)
    o_m, o_v, o_lat, o_step = optim.h24_update(grad.numpy(), m.numpy(), v.numpy(), latent.numpy(), sc)
    tm, tv, tl = m.clone(), v.clone(), latent.clone()
    t_step = torch_ref.pollux_h24_update(grad, tm, tv, tl, torch.tensor(heat, dtype=torch.float32), step, inertia)
    assert np.array_equal(o_m, tm.numpy())
    assert np.array_equal(o_v, tv.numpy())
    assert np.array_equal(o_step, t_step.numpy())
    assert np.array_equal(o_lat, tl.numpy())


def test_speed_cap_regimes_are_both_exercised():
    grad, m, v, latent = _state(3, 96, 1152, 1e-2)
    sc = optim.scalars(1.0, 0, 1.0)
    _, _, _, capped = optim.h24_update(grad.numpy(), m.numpy(), v.numpy(), latent.numpy(), sc)
    norms = optim.atom_norm(capped)
    cap = F32(sc[8])
    frac = np.mean(norms >= cap * F32(0.999))  # capped atoms sit at the cap
    assert 0.1 < frac < 0.9, frac  # both regimes in one call
    sc = optim.scalars(0.065771, 0, 1.0)
    _, _, _, free = optim.h24_update(grad.numpy(), m.numpy(), v.numpy(), latent.numpy(), sc)
    assert np.all(optim.atom_norm(free) < cap)


def test_step_scalars_of_the_package_match_the_oracle_on_cpu():
    from pollux_amd import optim as popt

    for heat, step, d in ((0.065771, 0, 1152), (0.5, 7, 1920), (1.0, 123, 768)):
        inertia = popt.width_inertia(d)
        got = popt.step_scalars(torch.tensor(heat), torch.tensor(step), inertia, torch.device("cpu")).numpy()
        assert np.array_equal(got, optim.scalars(heat, step, inertia))
