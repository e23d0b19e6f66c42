"""Fused optimiser step + requantize (plx_pollux_step_h24) against the oracle.

Bar: m, v and the latent bit-exact against oracle/optim.py given the same fp32
step scalars (the elementwise chain is deterministic); the step norm within
1e-5 relative of its float64 value; then the requantize of the new latent to
the bar of the requantize tests: sigma within 2 fp32 ulp of the reference's
row RMS, indices bit-exact on every non-near-tie atom (sampled), the written
parameter equal to (codebook[idx] * sigma) * fp32(1/sqrt 2) for every atom.
"""

import math

import numpy as np
import pytest
import torch

from oracle import nn, optim, packing, torch_ref
from pollux_amd import optim as popt

pytestmark = pytest.mark.gpu


def _ulp_diff(a, b):
    ai = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    bi = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(ai - bi)


@pytest.mark.parametrize("shape,heat,d,gscale,seed", [
    ((96, 1152), 0.065771, 1152, 1e-3, 1),
    ((64, 1920), 1.0, 1152, 1e-2, 2),     # heat high enough that part of the atoms hit the speed cap
    ((1152, 4608), 1.0, 1152, 1e-2, 3),   # a full Pollux-1152 down projection
])
def test_fused_step_matches_oracle(dev, shape, heat, d, gscale, seed):
    rows, cols = shape
    g = torch.Generator().manual_seed(seed)
    grad = torch.randn(rows, cols, generator=g) * gscale
    m = torch.randn(rows, cols, generator=g) * gscale * 0.3
    v = torch.rand(rows, cols, generator=g) * gscale * gscale
    latent = torch.randn(rows, cols, generator=g) * 0.02
    inertia = popt.width_inertia(d)
    dm, dv, dl = m.to(dev), v.to(dev), latent.to(dev)
    p = torch.empty(rows, cols, device=dev)
    o_m, o_v, o_l = m.numpy(), v.numpy(), latent.numpy()
    for step in range(3):  # consecutive steps carry the state
        heat_t = torch.tensor(heat, device=dev)
        step_t = torch.tensor(step, device=dev)
        sc = popt.step_scalars(heat_t, step_t, inertia, dev).cpu().numpy()
        # the device-evaluated scalars agree with the CPU evaluation to 1 ulp (pow may differ)
        assert _ulp_diff(sc, optim.scalars(heat, step, inertia)).max() <= 1
        norm, codes = popt.pollux_h24_step_(p, grad.to(dev), dm, dv, dl, heat=heat_t, step=step_t,
                                           width_inertia=inertia, return_codes=True)
        o_m, o_v, o_l, o_step = optim.h24_update(grad.numpy(), o_m, o_v, o_l, sc)
        assert np.array_equal(dm.cpu().numpy(), o_m), f"m differs at step {step}"
        assert np.array_equal(dv.cpu().numpy(), o_v), f"v differs at step {step}"
        assert np.array_equal(dl.cpu().numpy(), o_l), f"latent differs at step {step}"
        want = float(np.sqrt((o_step.astype(np.float64) ** 2).sum()))
        assert abs(float(norm) - want) <= 1e-5 * want
    # the requantize of the final latent
    lat = torch.from_numpy(o_l)
    sigma = codes["sigma"].cpu()
    assert _ulp_diff(sigma.numpy(), torch_ref.row_rms(lat).numpy()).max() <= 2
    idx = codes["indices"].cpu().numpy().astype(np.int64)
    assert np.array_equal(codes["packed"].cpu().numpy(), packing.pack(idx))
    x, _ = torch_ref.lattice_input(lat, sigma)
    x = x.reshape(-1, 24)
    rng = np.random.default_rng(seed)
    pick = np.sort(rng.choice(x.shape[0], size=min(1500, x.shape[0]), replace=False))
    r = nn.quantize(x[pick].numpy(), "B")
    assert not np.any((idx[pick] != r["idx"]) & ~r["near_tie"])
    center = torch_ref.codebook_tensor()[torch.from_numpy(idx)].reshape(rows, cols)
    assert torch.equal(p.cpu(), torch_ref.reconstruct(center, sigma))


def test_speed_cap_is_active_in_the_high_heat_case(dev):
    # guards the parametrisation above: at heat 1.0 / grad scale 1e-2 part of the atoms are capped
    g = torch.Generator().manual_seed(2)
    grad = torch.randn(64, 1920, generator=g) * 1e-2
    m = torch.randn(64, 1920, generator=g) * 3e-3
    v = torch.rand(64, 1920, generator=g) * 1e-4
    sc = optim.scalars(1.0, 0, popt.width_inertia(1152))
    _, _, _, capped = optim.h24_update(grad.numpy(), m.numpy(), v.numpy(), np.zeros((64, 1920), np.float32), sc)
    frac = np.mean(optim.atom_norm(capped) >= sc[8] * np.float32(0.999))
    assert 0.05 < frac < 0.95, frac


def test_bad_arguments_raise(dev):
    p = torch.empty(4, 48, device=dev)
    z = torch.zeros(4, 48, device=dev)
    with pytest.raises(ValueError):
        popt.pollux_h24_step_(p, z, z.clone(), z.clone(), z[:, :24].clone(), heat=0.5, step=0, width_inertia=1.0)
    with pytest.raises(ValueError):
        q = torch.empty(4, 36, device=dev)
        y = torch.zeros(4, 36, device=dev)
        popt.pollux_h24_step_(q, y, y.clone(), y.clone(), y.clone(), heat=0.5, step=0, width_inertia=1.0)
    assert math.isfinite(popt.width_inertia(1152)) and popt.width_inertia(1152) == pytest.approx(1.0)


def test_batched_step_equals_separate_calls(dev):
    # plx_pollux_step_h24_batch over a Pollux-1152 layer's four matrices plus ragged small ones, two
    # consecutive steps: m, v, latents, norms bit-identical to per-parameter calls; indices equal them
    # except on near-tie atoms (checked against the oracle), and the written parameters follow the indices
    shapes = [(3456, 1152), (1152, 1152), (4608, 1152), (1152, 4608), (5, 24), (0, 48), (3, 72)]
    g = torch.Generator().manual_seed(31)
    base = []
    for r, c in shapes:
        base.append((torch.randn(r, c, generator=g) * 1e-2, torch.randn(r, c, generator=g) * 3e-3,
                     torch.rand(r, c, generator=g) * 1e-4, torch.randn(r, c, generator=g) * 0.02))
    inertia = popt.width_inertia(1920)
    state_a = [(torch.empty(r, c, device=dev), gr.to(dev), m.to(dev), v.to(dev), l.to(dev))
               for (r, c), (gr, m, v, l) in zip(shapes, base)]
    state_b = [(torch.empty(r, c, device=dev), gr.to(dev), m.to(dev), v.to(dev), l.to(dev))
               for (r, c), (gr, m, v, l) in zip(shapes, base)]
    for step in range(2):
        heat_t = torch.tensor(0.8, device=dev)
        step_t = torch.tensor(step, device=dev)
        sc = popt.step_scalars(heat_t, step_t, inertia, dev)
        one = [popt.pollux_h24_step_(*s, heat=heat_t, step=step_t, width_inertia=inertia, scalars=sc,
                                     return_codes=True) for s in state_a]
        norms, codes = popt.pollux_h24_step_many_(state_b, heat=heat_t, step=step_t, width_inertia=inertia,
                                                  scalars=sc, return_codes=True)
        torch.cuda.synchronize()
        near_total = 0
        for k, ((pa, _, ma, va, la), (pb, _, mb, vb, lb)) in enumerate(zip(state_a, state_b)):
            assert torch.equal(ma, mb) and torch.equal(va, vb) and torch.equal(la, lb), (step, k)
            na, ca = one[k]
            assert torch.equal(na, norms[k]), (step, k)
            assert torch.equal(ca["sigma"], codes[k]["sigma"])
            diff = (ca["indices"] != codes[k]["indices"]).nonzero().flatten().cpu().numpy()
            if len(diff):
                x, _ = torch_ref.lattice_input(la.cpu(), ca["sigma"].cpu())
                r = nn.quantize(x.reshape(-1, 24)[torch.from_numpy(diff)].numpy(), "B")
                assert r["near_tie"].all(), (step, k, diff[~r["near_tie"]][:10])
                near_total += len(diff)
            else:
                assert torch.equal(ca["packed"], codes[k]["packed"]) and torch.equal(pa, pb), (step, k)
            assert np.array_equal(codes[k]["packed"].cpu().numpy(),
                                  packing.pack(codes[k]["indices"].cpu().numpy().astype(np.int64)))
        print(f"[optim batch] step {step}: near-tie index differences {near_total}", flush=True)
        # the next step continues from the (identical) m, v, latents; parameters copied to keep them equal
        for (pa, *_), (pb, *_) in zip(state_a, state_b):
            pb.copy_(pa)
