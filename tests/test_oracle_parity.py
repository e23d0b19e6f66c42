"""The disagreement classifier (oracle/parity.py) on planted disagreements of each class (CPU).

sigma_ulp: latent atoms whose lattice coordinates sit exactly on bf16
rounding midpoints next to contact-pair midpoints, so a one-ulp change of the
row scale flips the bf16 rounding of about half the coordinates and with it
the NN-B answer on many atoms, none of them near-ties; the same index pairs
with equal sigmas must count as real.  near_tie: exact midpoints of two
codes (equal exact scores under the fp32-score rule).  real: an index moved on a non-near-tie atom.
"""

import numpy as np
import torch

from oracle import codebook as cb
from oracle import nn, parity, torch_ref


def _contact_midpoints(n, noise, seed):
    rng = np.random.default_rng(seed)
    raw = cb.codebook_int8().astype(np.int64)
    c32 = cb.codebook_f32()
    pts = []
    while len(pts) < n:
        a = int(rng.integers(1, 196561))
        cand = rng.integers(1, 196561, 4000)
        hits = cand[(raw[cand] @ raw[a]) == 16]
        if len(hits):
            pts.append(0.5 * (c32[a] + c32[int(hits[0])]) + rng.normal(0, noise, 24).astype(np.float32))
    return np.stack(pts).astype(np.float32)


def _on_bf16_midpoints(x):
    m, e = np.frexp(x.astype(np.float64))
    q = np.floor(np.abs(m) * 512)
    q = q + (q % 2 == 0)  # 9 significant bits, the last one set: halfway between two bf16 values
    return (np.sign(m) * q / 512 * 2.0 ** e).astype(np.float32)


def _latent_row(xm):
    """A latent row w with fp32(w / 1.0 / fp32(1/sqrt 2)) == xm wherever one ulp of w reaches it."""
    s = np.float32(1 / np.sqrt(2))
    w = (xm * s).astype(np.float32)
    for _ in range(4):
        back = (w / s).astype(np.float32)
        bad = back != xm
        if not bad.any():
            break
        w[bad] = np.nextafter(w[bad], np.where(back[bad] < xm[bad], np.inf, -np.inf)).astype(np.float32)
    return torch.from_numpy(w.reshape(1, -1))


def test_sigma_ulp_class_and_its_slip():
    w = _latent_row(_on_bf16_midpoints(_contact_midpoints(400, 3e-3, 5)))
    s_ref = torch.tensor([1.0])
    s_gpu = torch.tensor([float(np.nextafter(np.float32(1.0), np.float32(2.0)))])
    x_ref, _ = torch_ref.lattice_input(w, s_ref)
    x_gpu, _ = torch_ref.lattice_input(w, s_gpu)
    i_ref, i_gpu = torch_ref.nn_b_indices(x_ref), torch_ref.nn_b_indices(x_gpu)
    r = parity.classify_requantize(w, i_gpu, s_gpu, i_ref, s_ref)
    assert r["disagree"] >= 20 and r["sigma_ulp"] == r["disagree"] and r["real"] == 0 and r["near_tie"] == 0
    assert r["sigma_max_ulp"] == 1 and r["sigma_rows_exact"] == 0.0
    # the same disagreements with one sigma on both sides cannot be blamed on sigma
    r2 = parity.classify_requantize(w, i_gpu, s_ref, i_ref, s_ref)
    assert r2["real"] == r["disagree"] and r2["sigma_ulp"] == 0 and r2["sigma_max_ulp"] == 0
    # an index that is nobody's answer is real even where the sigmas differ
    bad = i_gpu.clone()
    k = int(r["real_at"][0]) if r["real_at"] else int((i_gpu != i_ref).nonzero()[0])
    bad[k] = 1 if int(i_gpu[k]) != 1 else 2
    r3 = parity.classify_requantize(w, bad, s_gpu, i_ref, s_ref)
    assert r3["real"] == 1 and r3["real_at"] == [k]


def test_near_tie_and_real_on_given_x():
    # exact midpoints: two codes with equal exact scores, a near-tie for the fp32-score rule (NN-T)
    x = torch.from_numpy(_contact_midpoints(64, 0.0, 9))
    o = nn.quantize(x.numpy(), "T")
    ref = torch.from_numpy(o["idx"])
    assert o["near_tie"].mean() > 0.5
    agree = parity.classify_given_x(x, ref, ref, "T")
    assert agree["disagree"] == 0 and agree["near_tie"] == 0 and agree["real"] == 0
    g = torch.Generator().manual_seed(1)
    y = torch.randn(64, 24, generator=g)
    y_ref = torch_ref.nn_b_indices(y)
    far = int(np.nonzero(~nn.quantize(y.numpy(), "B")["near_tie"])[0][0])
    tie = int(np.nonzero(o["near_tie"])[0][0])
    got_x, got_y = ref.clone(), y_ref.clone()
    got_x[tie] = int(ref[tie]) + 1
    got_y[far] = int(y_ref[far]) + 1
    r = parity.classify_given_x(x, got_x, ref, "T")
    assert (r["disagree"], r["near_tie"], r["real"]) == (1, 1, 0)
    r = parity.classify_given_x(y, got_y, y_ref, "B")
    assert (r["disagree"], r["near_tie"], r["real"], r["real_at"]) == (1, 0, 1, [far])
