"""Oracle: the H24 branch of the reference optimiser step -- TEST INFRASTRUCTURE ONLY.

Restates pollux.py:836-878 (Adam moments, bias correction, heat-scaled step,
per-atom speed cap, weight decay of the latent) in numpy with the rounding of
each torch op made explicit, as torch evaluates them on fp32 CPU tensors:

  m.mul_(b1).add_(g, alpha=1-b1)          m = fma(g, 1-b1, m*b1)
  v.mul_(b2).addcmul_(g, g, value=1-b2)   v = fma((1-b2)*g, g, v*b2)
  m / clamp(bc1, 1e-8), v / clamp(bc2)     true divisions
  sqrt(v_unbiased) + 1e-8                  correctly rounded sqrt (sqrtf on the reference's
                                           GPU; torch's vectorised CPU sqrt is only
                                           faithful), then add
  neg_scale * (m_unbiased / denom)         neg_scale = -(heat*gamma/C / inertia), a 0-dim fp32 tensor
  vector_norm(step.reshape(-1, 24), dim=-1)
      8 accumulators (lane i: coordinates i, i+8, i+16, fused multiply-add),
      summed in lane order, sqrt
  cap / (norm + 1e-8)                      reciprocal(norm + 1e-8) * fp32(cap) (float / tensor)
  clamp(max=1.0), step * factor
  latent.mul_(wdf).add_(step)              two roundings, wdf = 1 - heat*gamma^2

Pinned by tests/test_oracle_optim.py against those torch ops run on the CPU
(bit-exact), including the pinning of each rounding rule on its own.
"""

from __future__ import annotations

import math

import numpy as np

GAMMA = 0.065771  # castor.py:39-40 (G24)
FRICTION_C = math.sqrt(2.0)  # castor.py:34
S_LATTICE = 1.0 / FRICTION_C  # castor.py:47
KINEMATIC_LIMIT = (FRICTION_C - 1.0) / 2.0  # pollux.py:59,62 (GEOMETRIC_SLACK / 2)
EPS = np.float32(1e-8)
F32 = np.float32


def fma(a, b, c) -> np.ndarray:
    """fp32 fused multiply-add (the float64 product of two fp32 values is exact)."""
    return (np.asarray(a, np.float64) * np.asarray(b, np.float64) + np.asarray(c, np.float64)).astype(F32)


def scalars(heat: float, step: int, width_inertia: float) -> np.ndarray:
    """The nine fp32 scalars of one step, evaluated like the reference's 0-dim fp32 tensor ops (CPU).

    heat: fp32 macro heat; step: the optimiser step counter before the update
    (pollux.py:817-820); width_inertia: 1 + C ln(d / (24 C)^2) for matrices.
    """
    import torch

    b1 = 1.0 - math.sqrt(GAMMA)
    b2 = 1.0 - GAMMA
    step_f = torch.tensor(float(step), dtype=torch.float32) + 1.0
    bc1 = 1.0 - (torch.as_tensor(b1, dtype=torch.float32) ** step_f)
    bc2 = 1.0 - (torch.as_tensor(b2, dtype=torch.float32) ** step_f)
    h = torch.tensor(heat, dtype=torch.float32)
    kinetic_scale = h * float(GAMMA) / float(FRICTION_C)
    neg_scale = -(kinetic_scale / width_inertia)
    wdf = 1.0 - (h * (float(GAMMA) ** 2))
    vals = [
        torch.tensor(b1, dtype=torch.float32), torch.tensor(1.0 - b1, dtype=torch.float32),
        torch.tensor(b2, dtype=torch.float32), torch.tensor(1.0 - b2, dtype=torch.float32),
        torch.clamp(bc1, min=1e-8), torch.clamp(bc2, min=1e-8), neg_scale, wdf,
        torch.tensor(float(KINEMATIC_LIMIT) * float(S_LATTICE), dtype=torch.float32),
    ]
    return np.array([float(t) for t in vals], dtype=F32)


def atom_norm(step: np.ndarray) -> np.ndarray:
    """|s|_2 per 24-element atom in the CPU reduction order (8 fused-multiply-add lanes, lane-order sum)."""
    s = step.reshape(-1, 24).astype(F32)
    acc = (s[:, 0:8] * s[:, 0:8]).astype(F32)
    acc = fma(s[:, 8:16], s[:, 8:16], acc)
    acc = fma(s[:, 16:24], s[:, 16:24], acc)
    tot = acc[:, 0]
    for i in range(1, 8):
        tot = (tot + acc[:, i]).astype(F32)
    return np.sqrt(tot).astype(F32)


def h24_update(grad, m, v, latent, sc: np.ndarray):
    """One H24 step: returns (m, v, latent, capped step) as new fp32 arrays of the input shape."""
    b1, omb1, b2, omb2, bc1, bc2, neg_scale, wdf, cap = [F32(x) for x in sc]
    g = np.asarray(grad, F32)
    m2 = fma(g, omb1, (np.asarray(m, F32) * b1).astype(F32))
    v2 = fma((omb2 * g).astype(F32), g, (np.asarray(v, F32) * b2).astype(F32))
    mu = (m2 / bc1).astype(F32)
    den = (np.sqrt((v2 / bc2).astype(F32)).astype(F32) + EPS).astype(F32)
    step = (neg_scale * (mu / den).astype(F32)).astype(F32)
    t = (atom_norm(step) + EPS).astype(F32)
    fac = np.minimum(((F32(1.0) / t).astype(F32) * cap).astype(F32), F32(1.0))
    capped = (step.reshape(-1, 24) * fac[:, None]).astype(F32).reshape(step.shape)
    lat = ((np.asarray(latent, F32) * wdf).astype(F32) + capped).astype(F32)
    return m2, v2, lat, capped
