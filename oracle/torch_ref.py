"""Oracle: the reference's non-Triton path restated with the same torch ops -- TEST INFRASTRUCTURE ONLY.

castor.py:544-557 (NN-B), pack.py:139-180 (NN-P + sigma16), castor.py:309-339
and pollux.py:874-884 (row scale and the per-step requantize composition),
pollux.py:485-507 (materialize + linear).  These call the same torch CPU ops
the reference calls (autocast-bf16 matmul, ``.float().max(-1)``, ``pow``,
``mean``, ``sqrt``, fp16 broadcast multiplies), so on the CPU they reproduce
the reference's results by construction.  bench.py times ``nn_b_indices`` on
the host cores as the CPU baseline ("kind": "port").

Pinned by (tests/test_oracle_nn.py, tests/test_oracle_rowscale.py): agreement
with the exact float64 oracle (oracle/nn.py) on every non-near-tie atom, and
float64 closed forms for the row scale (within 2 fp32 ulp).
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import codebook as cbm

S_LATTICE = 1.0 / math.sqrt(2.0)  # castor.py:47 (s_lattice = 1/friction_c)
NUMERICAL_EPSILON = 1e-8  # castor.py:50


def codebook_tensor(dtype=torch.float32) -> torch.Tensor:
    return torch.from_numpy(cbm.codebook_f32().copy()).to(dtype)


def nn_b_indices(x: torch.Tensor, chunk_size: int = 4096, kp: torch.Tensor | None = None) -> torch.Tensor:
    """castor.py:544-557: chunked autocast-bf16 matmul, first max, origin snap. int64 [N]."""
    x = x.reshape(-1, 24).float()
    if kp is None:
        kp = codebook_tensor()[1:]
    c_sq = float(kp[0].pow(2).sum().item())
    out = torch.empty(x.shape[0], dtype=torch.long)
    for i in range(0, x.shape[0], chunk_size):
        with torch.autocast(device_type="cpu", dtype=torch.bfloat16):
            scores = torch.matmul(x[i : i + chunk_size], kp.t())
        best_val, best = scores.float().max(dim=-1)
        snap = (2.0 * best_val) < c_sq
        out[i : i + chunk_size] = (best + 1).masked_fill(snap, 0)
    return out


def nn_p_indices(w: torch.Tensor, chunk_size: int = 4096, kp: torch.Tensor | None = None) -> torch.Tensor:
    """pack.py:167-177: fp32 matmul on raw atoms, first max, origin iff |atom| < 1e-8."""
    atoms = w.detach().float().reshape(-1, 24)
    if kp is None:
        kp = codebook_tensor()[1:]
    out = torch.zeros(atoms.shape[0], dtype=torch.long)
    for i in range(0, atoms.shape[0], chunk_size):
        s = atoms[i : i + chunk_size]
        _, best = torch.matmul(s, kp.t()).max(dim=-1)
        snap = s.norm(dim=-1) < NUMERICAL_EPSILON
        out[i : i + chunk_size] = (best + 1).masked_fill(snap, 0)
    return out


def row_rms(w: torch.Tensor) -> torch.Tensor:
    """castor.py:309-313."""
    return torch.sqrt(w.pow(2).mean(dim=-1) + NUMERICAL_EPSILON)


def normalize(w: torch.Tensor, sigma: torch.Tensor | None = None):
    """castor.py:316-333: (w / sigma.clamp_min(eps), sigma)."""
    if sigma is None:
        sigma = row_rms(w)
    return w / sigma.reshape(-1, 1).clamp_min(NUMERICAL_EPSILON), sigma.reshape(-1)


def lattice_input(w: torch.Tensor, sigma: torch.Tensor | None = None):
    """pollux.py:876-882: x = normalize(w)/fp32(s_lattice) (a true division); returns (x, sigma)."""
    normed, sigma = normalize(w, sigma)
    return normed / float(S_LATTICE), sigma


def reconstruct(center: torch.Tensor, sigma: torch.Tensor) -> torch.Tensor:
    """castor.py:336-339 then pollux.py:883: (center * sigma[:, None]) * fp32(s_lattice)."""
    return (center * sigma.reshape(-1, 1)) * float(S_LATTICE)


def requantize(latent: torch.Tensor, sigma: torch.Tensor | None = None):
    """pollux.py:874-884 on the CPU: returns (indices int64 [N], sigma fp32 [R], p fp32 [R, C])."""
    x, sigma = lattice_input(latent, sigma)
    idx = nn_b_indices(x)
    center = codebook_tensor()[idx].reshape(latent.shape)
    return idx, sigma, reconstruct(center, sigma)


def sigma16_pack(w: torch.Tensor) -> torch.Tensor:
    """pack.py:164: fp16(clamp(row_rms(w) * fp32(sqrt(12)), 1e-8))."""
    return (row_rms(w.detach().float()) * math.sqrt(12.0)).clamp_min(NUMERICAL_EPSILON).to(torch.float16)


def materialize(indices: torch.Tensor, sigma16: torch.Tensor, out_features: int, in_features: int) -> torch.Tensor:
    """pollux.py:485-504: fp16 codebook gather, * sigma16 per row, * s_lattice, all in fp16."""
    cb16 = codebook_tensor(torch.float16)
    atoms = cb16.index_select(0, indices.long()).view(out_features, in_features // 24, 24)
    return (atoms * sigma16.view(-1, 1, 1) * S_LATTICE).reshape(out_features, in_features)


def linear_fp32(x: torch.Tensor, w16: torch.Tensor) -> torch.Tensor:
    """The fp32 reference for the packed layer: F.linear(x.float(), W.float()) (pollux.py:507 with fp32 x)."""
    return torch.nn.functional.linear(x.float(), w16.float())
