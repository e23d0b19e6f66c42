"""Full-coverage index parity against the reference's own CPU path.

The fused requantize (NN-B) is checked on every atom of configs 1, 2 and 3
(2,562,048 atoms).  The reference side is oracle/torch_ref.requantize: the
reference's torch ops on the host (castor.py:309-333 row scale and
normalisation, pollux.py:882 lattice input, castor.py:549-557 NN-B search), so
its sigma is the reference's own.  Config 3's boundary-stress atoms (92,160
contact-pair midpoints and 92,160 near-origin atoms, tests/c3_stress.py) go
through the quantizer alone and are compared, every one of them, with the
reference's NN-B torch ops (torch_ref.nn_b_indices).  The pack-time quantizer
(NN-P, pack.py:139-180) is compared on every atom of config 1's raw weights
and of its requantized weights (what pack.py reads from a trained
checkpoint) with the reference's fp32 torch ops (torch_ref.nn_p_indices).

Every index disagreement is classified by oracle/parity.py with the exact
oracle (oracle/nn.py) as near_tie, sigma_ulp (requantize only: the row's sigma
differs by an ulp between the two reductions and each side's index is the
oracle's answer on its own x) or real.
Bars: real == 0; sigma within 2 fp32 ulp of the reference's CPU reduction
(its fp64 row sum rounded once on the GPU against torch's host-ISA-dependent
fp32 order).  The counts go to the terminal summary and
gpurun_out/parity_report.json.
"""

import numpy as np
import pytest
import torch

from oracle import packing, parity, torch_ref
from pollux_amd import castor
from pollux_amd import pack as plx_pack

import c3_stress  # tests/ is on sys.path (pytest's rootdir-relative import of this directory)

pytestmark = pytest.mark.gpu

C1 = [(1152, 1152)]
C2 = [(3456, 1152), (1152, 1152), (4608, 1152), (1152, 4608)]
C3 = [(5760, 1920), (1920, 1920), (7680, 1920), (1920, 7680)]


def _check_matrix(dev, w, row_step, label, report):
    """Requantize w on the GPU; compare the rows w[::row_step] with the reference's CPU path."""
    got = castor.requantize_h24(w.to(dev))
    rows = torch.arange(0, w.shape[0], row_step)
    wr = w[rows]
    apr = w.shape[1] // 24
    idx_ref, sig_ref, p_ref = torch_ref.requantize(wr)
    sig_gpu = got["sigma"].cpu()[rows]
    atom_sel = (rows[:, None] * apr + torch.arange(apr)[None, :]).reshape(-1)
    idx_gpu = got["indices"].cpu().long()[atom_sel]
    c = parity.classify_requantize(wr, idx_gpu, sig_gpu, idx_ref, sig_ref)
    real_at = [int(atom_sel[a]) for a in c.pop("real_at")]
    rec = {"case": label, **c}
    report.append(rec)
    print(f"[parity] {rec}", flush=True)
    assert c["sigma_max_ulp"] <= parity.SIGMA_BAR_ULP
    assert c["real"] == 0, real_at[:10]
    # everything downstream of the indices is exact: packed bytes of the whole
    # matrix, and the reconstructed weight of the checked rows given each side's sigma
    assert np.array_equal(got["packed"].cpu().numpy(), packing.pack(got["indices"].cpu().numpy().astype(np.int64)))
    same = parity.ulp_distance(sig_gpu, sig_ref) == 0
    if same.any():
        keep = torch.from_numpy(np.repeat(same, w.shape[1]).reshape(len(rows), w.shape[1]))
        agree = (idx_gpu == idx_ref).reshape(len(rows), apr).repeat_interleave(24, dim=1)
        m = keep & agree
        assert torch.equal(got["weight"].cpu()[rows][m], p_ref[m])
    return rec


def _bf16_master(shapes, seed):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(r, c, generator=g) * 0.02).to(torch.bfloat16).float() for r, c in shapes]


def test_config1_every_atom(dev, parity_report):
    g = torch.Generator().manual_seed(1152)
    w = torch.randn(1152, 1152, generator=g) * 0.02  # fp32 N(0, 0.02)
    _check_matrix(dev, w, 1, "config1 1152x1152 (all 55,296 atoms)", parity_report)


@pytest.mark.timeout(600)
def test_config2_every_atom(dev, parity_report):
    total = 0
    for (r, c), w in zip(C2, _bf16_master(C2, 2024)):
        rec = _check_matrix(dev, w, 1, f"config2 {r}x{c} (all atoms)", parity_report)
        total += rec["atoms_compared"]
    assert total == 663_552


@pytest.mark.timeout(600)
@pytest.mark.parametrize("k", range(4))
def test_config3_requantize_every_atom(dev, parity_report, k):
    (r, c), w = C3[k], _bf16_master(C3, 1920)[k]
    rec = _check_matrix(dev, w, 1, f"config3 {r}x{c} (all atoms)", parity_report)
    assert rec["atoms_compared"] == r * c // 24


def _classify_given_x(x, got, ref, mode, label, report):
    """Disagreements between GPU and reference indices on the same x: near-tie (exact oracle) or real."""
    c = parity.classify_given_x(x, got, ref, mode)
    real_at = c.pop("real_at")
    rec = {"case": label, **c}
    report.append(rec)
    print(f"[parity] {rec}", flush=True)
    assert not real_at, real_at[:10]
    return rec


@pytest.mark.timeout(600)
def test_config3_boundary_stress_every_stressed_atom(dev, parity_report):
    x, mid_at, near_at = c3_stress.build(303)
    got = castor.quantize_indices(x.to(dev), mode="bf16").long().cpu()
    for name, at in (("contact-pair midpoints", mid_at), ("near-origin, norm sqrt 2", near_at)):
        sel = torch.from_numpy(np.sort(at))
        xs = x[sel]
        ref = torch_ref.nn_b_indices(xs)
        rec = _classify_given_x(xs, got[sel], ref, "B", f"config3 stress: all {len(at)} {name} (NN-B)",
                                parity_report)
        assert rec["atoms_compared"] == 92_160
        if name.startswith("near"):
            # both sides of the origin boundary occur: some atoms snap to the origin, most do not
            assert 0 < int((ref == 0).sum()) < len(at)


@pytest.mark.timeout(600)
def test_config1_pack_time_quantizer_every_atom(dev, parity_report):
    g = torch.Generator().manual_seed(1152)
    w = torch.randn(1152, 1152, generator=g) * 0.02  # fp32 N(0, 0.02)
    # the raw weights (pack.py:161-177 on any fp32 matrix) and the requantized ones (what pack.py reads from a
    # trained checkpoint: every atom a scaled codebook vector, so NN-P must return the requantize indices)
    rq = castor.requantize_h24(w.to(dev))
    p_data = rq["weight"].cpu()
    for name, m in (("raw weights", w), ("requantized weights", p_data)):
        packed, sig16, idx = plx_pack.quantize_h24_layer(m.to(dev), return_indices=True)
        got = idx.long().cpu()
        ref = torch_ref.nn_p_indices(m)
        _classify_given_x(m.reshape(-1, 24), got, ref, "P", f"config1 NN-P {name}: all 55296 atoms",
                          parity_report)
        # the .plx bytes: the oracle packer over the kernel's indices; sigma16 within 1 fp16 ulp
        assert np.array_equal(packed.cpu().numpy(), packing.pack(got.numpy()))
        want = torch_ref.sigma16_pack(m)
        assert (sig16.cpu().view(torch.int16).long() - want.view(torch.int16).long()).abs().max() <= 1
    assert torch.equal(got, rq["indices"].long().cpu())
