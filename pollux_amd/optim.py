"""Fused optimiser step + requantize of an H24 parameter (the H24 branch of pollux_step, pollux.py:836-888).

The reference updates each quantizable matrix with ~15 separate tensor ops
(Adam moments, bias correction, heat-scaled step, per-atom speed cap, weight
decay) and then requantizes the latent (pollux.py:874-884).  Here one HIP
kernel reads grad, m, v and the latent once and writes m, v and the latent
once, reproducing each op's fp32 rounding; the requantize (row scale, NN
search, 18-bit pack, reconstructed weight) follows in the same call.

The step scalars are computed here with the reference's own 0-dim tensor
expressions on the parameter's device (pollux.py:815-820, 849-855, 870), so
nothing is synchronised with the host.  A caller replaces the body of the
reference's loop for an H24 tensor with::

    adam_norm = pollux_h24_step_(p, p.grad, m, v, latent, heat=heat_t,
                                 step=state.step, width_inertia=width_inertia)
    adam_energy_sum = adam_energy_sum + adam_norm
"""

from __future__ import annotations

import math

import torch

from . import _lib
from . import castor as _castor
from .castor import BYTES_PER_CHUNK, H24_DIM, NUMERICAL_EPSILON, assert_row_aligned_in_features

GAMMA = 0.065771  # castor.py:39-40 (G24)
FRICTION_C = math.sqrt(2.0)  # castor.py:34; pollux.py:50 (C)
S_LATTICE = 1.0 / FRICTION_C  # castor.py:47
GEOMETRIC_SLACK = FRICTION_C - 1.0  # pollux.py:59
KINEMATIC_LIMIT = GEOMETRIC_SLACK / 2.0  # pollux.py:62


def width_inertia(n_embd: float) -> float:
    """eta_d = 1 + C ln(d / (24 C)^2) (pollux.py:785), 1.0 at d = 1152."""
    return 1.0 + FRICTION_C * math.log(float(n_embd) / ((float(H24_DIM) * FRICTION_C) ** 2))


_CONSTS: dict[torch.device, torch.Tensor] = {}


def _consts(device: torch.device) -> torch.Tensor:
    """fp32 [b1, 1-b1, b2, 1-b2, cap] on ``device``, uploaded once per device."""
    c = _CONSTS.get(device)
    if c is None:
        beta_2 = 1.0 - float(GAMMA)  # pollux.py:815-816
        beta_1 = 1.0 - math.sqrt(float(GAMMA))
        cap = float(KINEMATIC_LIMIT) * float(S_LATTICE)  # pollux.py:862
        c = torch.tensor([beta_1, 1.0 - beta_1, beta_2, 1.0 - beta_2, cap], dtype=torch.float32).to(device)
        _CONSTS[device] = c
    return c


def step_scalars(heat: torch.Tensor, step: torch.Tensor | int, inertia: float, device: torch.device) -> torch.Tensor:
    """The nine fp32 scalars of plx_pollux_step_h24 as the reference evaluates them.

    heat: the 0-dim macro heat (``heat_t``, pollux.py:810); step: the step counter
    before this update (``state.step``); inertia: width_inertia for matrices.
    Device-resident inputs keep the whole computation on the device; it is the
    same for every parameter of one step and width, so callers compute it once.
    """
    f32 = torch.float32
    device = torch.device(device)
    if device.type == "cuda" and device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    c = _consts(device)
    step_f = torch.as_tensor(step).to(dtype=f32, device=device) + 1.0  # pollux.py:817-819
    bc1 = 1.0 - (c[0] ** step_f)  # torch.as_tensor(beta_1, fp32) ** step_f
    bc2 = 1.0 - (c[2] ** step_f)
    h = torch.as_tensor(heat).to(device=device, dtype=f32).reshape(())
    kinetic_scale = h * float(GAMMA) / float(FRICTION_C)  # pollux.py:851
    neg_scale = -(kinetic_scale / inertia)  # pollux.py:852
    wdf = 1.0 - (h * (float(GAMMA) ** 2))  # pollux.py:869
    return torch.cat([
        c[0:4],
        torch.clamp(bc1.reshape(1), min=NUMERICAL_EPSILON), torch.clamp(bc2.reshape(1), min=NUMERICAL_EPSILON),
        neg_scale.reshape(1), wdf.reshape(1), c[4:5],
    ])


def pollux_h24_step_(
    p: torch.Tensor,
    grad: torch.Tensor,
    m: torch.Tensor,
    v: torch.Tensor,
    latent: torch.Tensor,
    *,
    heat: torch.Tensor | float,
    step: torch.Tensor | int,
    width_inertia: float,
    mode: str | None = None,
    return_codes: bool = False,
    scalars: torch.Tensor | None = None,
):
    """pollux.py:836-884 for one H24 parameter: updates m, v, latent and p.data in place.

    All of p, grad, m, v, latent are fp32 tensors of one [R, C] shape (C % 24 ==
    0) on one ROCm device.  Returns the 0-dim fp32 norm of the capped step (the
    parameter's term of adam_energy_sum, pollux.py:886-888); with
    ``return_codes`` also a dict(sigma, indices, packed) of the requantize.
    ``scalars``: the output of step_scalars for this step (computed here if None).
    """
    if p.dim() != 2:
        raise ValueError(f"pollux_h24_step_ expects a 2D parameter, got {p.dim()}D.")
    rows, cols = p.shape
    assert_row_aligned_in_features(cols)
    for name, t in (("grad", grad), ("m", m), ("v", v), ("latent", latent), ("p", p)):
        _lib.require_device(t, f"pollux_h24_step_ {name}")
        if t.shape != p.shape or t.dtype != torch.float32:
            raise ValueError(f"pollux_h24_step_: {name} must be float32 of shape {tuple(p.shape)}")
    for name, t in (("m", m), ("v", v), ("latent", latent)):
        if not t.is_contiguous():
            raise ValueError(f"pollux_h24_step_: {name} is updated in place and must be contiguous")
    dev = p.device
    g = grad.detach().contiguous()
    scal = scalars if scalars is not None else step_scalars(heat, step, float(width_inertia), dev)
    if scal.dtype != torch.float32 or scal.numel() != 9 or scal.device != dev:
        raise ValueError("pollux_h24_step_: scalars must be the 9 float32 values of step_scalars on the device")
    scal = scal.contiguous()
    n = rows * (cols // H24_DIM)
    sigma = torch.empty(rows, dtype=torch.float32, device=dev)
    idx = torch.empty(n, dtype=torch.int32, device=dev)
    packed = torch.empty(((n + 3) // 4) * BYTES_PER_CHUNK, dtype=torch.uint8, device=dev) if return_codes else None
    w = p.data if p.data.is_contiguous() else torch.empty_like(p.data)
    norm = torch.zeros((), dtype=torch.float32, device=dev)  # an empty parameter's norm is 0 (not written)
    nws = int(_lib.lib().plx_pollux_step_workspace_bytes(rows, cols))
    ws = torch.empty(max(nws, 16), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        st = _lib.lib().plx_pollux_step_h24(
            _lib.ptr(g), _lib.ptr(m), _lib.ptr(v), _lib.ptr(latent), rows, cols, _lib.ptr(scal),
            _castor._MODES[mode or _castor._nn_mode], _lib.ptr(sigma), _lib.ptr(idx), _lib.ptr(packed), _lib.ptr(w),
            _lib.ptr(norm), _lib.ptr(ws), nws, _lib.stream_of(dev),
        )
    _lib.check(st, "pollux_h24_step_")
    if w is not p.data:
        p.data.copy_(w)
    if return_codes:
        return norm, {"sigma": sigma, "indices": idx, "packed": packed}
    return norm


def pollux_h24_step_many_(
    params: list[tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]],
    *,
    heat: torch.Tensor | float,
    step: torch.Tensor | int,
    width_inertia: float,
    mode: str | None = None,
    return_codes: bool = False,
    scalars: torch.Tensor | None = None,
):
    """pollux.py:828-888 for every H24 parameter of one step: pollux_h24_step_ on each (p, grad, m, v, latent).

    One update pass per parameter, then one scoring sweep over the atoms of all
    their new latents (plx_pollux_step_h24_batch): m, v, latents and the norms
    are bit-identical to separate pollux_h24_step_ calls, indices equal them up
    to near-ties.  All tensors on one device; the step scalars are shared (one
    heat, step counter and width_inertia per step, pollux.py:785, 815-820).
    Returns the list of 0-dim step norms (and, with ``return_codes``, the list
    of dict(sigma, indices, packed)).
    """
    if not params:
        return ([], []) if return_codes else []
    dev = params[0][0].device
    scal = scalars if scalars is not None else step_scalars(heat, step, float(width_inertia), dev)
    if scal.dtype != torch.float32 or scal.numel() != 9 or scal.device != dev:
        raise ValueError("pollux_h24_step_many_: scalars must be the 9 float32 values of step_scalars on the device")
    scal = scal.contiguous()
    items, keep, outs = [], [], []
    for k, (p, grad, m, v, latent) in enumerate(params):
        if p.dim() != 2:
            raise ValueError(f"pollux_h24_step_many_: parameter {k} is {p.dim()}D, expected 2D")
        rows, cols = p.shape
        assert_row_aligned_in_features(cols)
        for name, t in (("grad", grad), ("m", m), ("v", v), ("latent", latent), ("p", p)):
            _lib.require_device(t, f"pollux_h24_step_many_ {name}")
            if t.device != dev:
                raise ValueError("pollux_h24_step_many_: all tensors must be on one device")
            if t.shape != p.shape or t.dtype != torch.float32:
                raise ValueError(f"pollux_h24_step_many_: {name} of parameter {k} must be float32 {tuple(p.shape)}")
        for name, t in (("m", m), ("v", v), ("latent", latent)):
            if not t.is_contiguous():
                raise ValueError(f"pollux_h24_step_many_: {name} is updated in place and must be contiguous")
        n = rows * (cols // H24_DIM)
        g = grad.detach().contiguous()
        o = {
            "sigma": torch.empty(rows, dtype=torch.float32, device=dev),
            "indices": torch.empty(n, dtype=torch.int32, device=dev),
            "packed": torch.empty(((n + 3) // 4) * BYTES_PER_CHUNK, dtype=torch.uint8, device=dev)
            if return_codes else None,
            "norm": torch.zeros((), dtype=torch.float32, device=dev),  # stays 0 for an empty parameter
        }
        w = p.data if p.data.is_contiguous() else torch.empty_like(p.data)
        keep.append((g, w, p))
        outs.append(o)
        items.append(_lib.PolluxStepItem(_lib.ptr(g), _lib.ptr(m), _lib.ptr(v), _lib.ptr(latent), rows, cols,
                                         _lib.ptr(o["sigma"]), _lib.ptr(o["indices"]), _lib.ptr(o["packed"]),
                                         _lib.ptr(w), _lib.ptr(o["norm"])))
    arr = (_lib.PolluxStepItem * len(items))(*items)
    nws = int(_lib.lib().plx_pollux_step_batch_workspace_bytes(arr, len(items)))
    ws = torch.empty(max(nws, 16), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        st = _lib.lib().plx_pollux_step_h24_batch(arr, len(items), _lib.ptr(scal),
                                                  _castor._MODES[mode or _castor._nn_mode], _lib.ptr(ws), nws,
                                                  _lib.stream_of(dev))
    _lib.check(st, "pollux_h24_step_many_")
    for g, w, p in keep:
        if w is not p.data:
            p.data.copy_(w)
    norms = [o["norm"] for o in outs]
    if return_codes:
        return norms, [{"sigma": o["sigma"], "indices": o["indices"], "packed": o["packed"]} for o in outs]
    return norms
