"""Oracle: classification of index disagreements with the reference -- TEST INFRASTRUCTURE ONLY.

Used by the parity tests and bench.py's parity record to sort every index on
which the HIP path and the reference's own CPU ops (oracle/torch_ref.py)
disagree into one of three classes, by the exact oracle (oracle/nn.py):

  near_tie   the reference's answer is not determined within the fp32
             envelope 24 * 2^-24 * sum|x_i c_i| (oracle.nn.DELTA_REL) on the
             reference's own x;
  sigma_ulp  (requantize only) not a near-tie, but the row's sigma differs by
             an fp32 ulp between the two row reductions, and each side's index
             is the exact oracle's answer on the x built from its own sigma;
  real       anything else.  Every parity bar requires real == 0.

Sigma bar: the GPU's row RMS (an fp64 sum rounded once) within 2 fp32 ulp of
torch's CPU reduction (castor.py:309-313), whose fp32 summation order depends
on the host ISA.

Pinned by tests/test_oracle_parity.py: planted disagreements of each class
(an index moved on a non-near-tie atom is "real", a near-tie atom's alternate
answer is "near_tie", an index computed from a sigma one ulp away is
"sigma_ulp") land in their class, and agreement gives zero counts.
"""

from __future__ import annotations

import numpy as np
import torch

from . import nn, torch_ref

SIGMA_BAR_ULP = 2


def ulp_distance(a: torch.Tensor, b: torch.Tensor) -> np.ndarray:
    """|bits(a) - bits(b)| of two fp32 tensors of one shape (same-sign finite values)."""
    return np.abs(a.numpy().view(np.int32).astype(np.int64) - b.numpy().view(np.int32).astype(np.int64))


def classify_given_x(x: torch.Tensor, got: torch.Tensor, ref: torch.Tensor, mode: str) -> dict:
    """Disagreements of two index vectors on the same atoms x [N, 24]: near_tie or real (mode "B" / "T" / "P").

    Returns {"atoms_compared", "disagree", "near_tie", "real", "real_at"} (real_at: atom positions).
    """
    got = got.reshape(-1).long()
    ref = ref.reshape(-1).long()
    diff = (got != ref).nonzero().flatten()
    near = 0
    real_at: list[int] = []
    if len(diff):
        o = nn.quantize(x.reshape(-1, 24)[diff].numpy(), mode)
        near = int(o["near_tie"].sum())
        real_at = diff[torch.from_numpy(~o["near_tie"])].tolist()
    return {"atoms_compared": int(ref.numel()), "disagree": int(len(diff)), "near_tie": near,
            "real": len(real_at), "real_at": real_at}


def classify_requantize(w: torch.Tensor, idx_gpu: torch.Tensor, sigma_gpu: torch.Tensor,
                        idx_ref: torch.Tensor, sigma_ref: torch.Tensor) -> dict:
    """Disagreements of the fused requantize (NN-B) with the reference's CPU composition on latent w [R, C].

    idx_*: int [R * C / 24], sigma_*: fp32 [R], all on the CPU.  Returns the counts of the three classes,
    the atom positions of the real ones, and the sigma statistics (fraction of rows bit-equal, max ulp).
    """
    apr = w.shape[1] // 24
    idx_gpu = idx_gpu.reshape(-1).long()
    idx_ref = idx_ref.reshape(-1).long()
    d_sig = ulp_distance(sigma_gpu.reshape(-1).float(), sigma_ref.reshape(-1).float())
    diff = (idx_gpu != idx_ref).nonzero().flatten()
    counts = {"near_tie": 0, "sigma_ulp": 0, "real": 0}
    real_at: list[int] = []
    if len(diff):
        x_ref, _ = torch_ref.lattice_input(w, sigma_ref)
        x_gpu, _ = torch_ref.lattice_input(w, sigma_gpu)
        o_ref = nn.quantize(x_ref.reshape(-1, 24)[diff].numpy(), "B")
        o_gpu = nn.quantize(x_gpu.reshape(-1, 24)[diff].numpy(), "B")
        row_of = (diff // apr).numpy()
        for k in range(len(diff)):
            a = int(diff[k])
            if o_ref["near_tie"][k]:
                counts["near_tie"] += 1
            elif (d_sig[row_of[k]] != 0 and not o_gpu["near_tie"][k] and o_gpu["idx"][k] == int(idx_gpu[a])
                  and o_ref["idx"][k] == int(idx_ref[a])):
                counts["sigma_ulp"] += 1
            else:
                counts["real"] += 1
                real_at.append(a)
    return {"atoms_compared": int(idx_ref.numel()), "disagree": int(len(diff)), **counts, "real_at": real_at,
            "sigma_rows_exact": float(np.mean(d_sig == 0)), "sigma_max_ulp": int(d_sig.max()) if d_sig.size else 0,
            "sigma_bar_ulp": SIGMA_BAR_ULP}
