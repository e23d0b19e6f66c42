"""HIP nearest-neighbour quantizer (castor.py:487-560) against the exact oracle and the reference's torch ops.

Bar: indices bit-exact on every atom that is not a near-tie within the fp32
envelope DELTA_REL * sum|x_i c_i| (oracle/nn.py); near-ties are counted and
must stay rare.
"""

import numpy as np
import pytest
import torch

from oracle import codebook as cb
from oracle import nn, torch_ref
from pollux_amd import castor

pytestmark = pytest.mark.gpu

MODES = {"bf16": "B", "fp32": "T"}


def _check(dev, x, mode, max_near=0.01, label=""):
    got = castor.quantize_indices(x.to(dev), mode=mode).cpu().numpy().astype(np.int64)
    r = nn.quantize(x.reshape(-1, 24).numpy(), MODES[mode])
    near = r["near_tie"]
    bad = (got != r["idx"]) & ~near
    print(f"[{label} {mode}] atoms={len(got)} near_ties={int(near.sum())} "
          f"mismatch_on_near_ties={int(((got != r['idx']) & near).sum())} mismatch_non_near={int(bad.sum())}", flush=True)
    assert near.mean() <= max_near
    assert not bad.any(), np.nonzero(bad)[0][:10]
    return got, r


def _lattice_atoms(rows, cols, seed):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(rows, cols, generator=g) * 0.02
    x, _ = torch_ref.lattice_input(w)
    return x.reshape(-1, 24)


@pytest.mark.parametrize("mode", ["bf16", "fp32"])
def test_every_codebook_vector_is_a_fixed_point(dev, mode):
    c = torch.from_numpy(cb.codebook_f32()[1:].copy())  # all 196,560 kissing points
    got = castor.quantize_indices(c.to(dev), mode=mode).cpu()
    assert torch.equal(got.long(), torch.arange(1, 196561))


@pytest.mark.parametrize("n", [1, 5, 511, 512, 513, 2049])
def test_zero_atoms_and_ragged_tails(dev, n):
    got = castor.quantize_indices(torch.zeros(n, 24, device=dev))
    assert got.shape == (n,) and torch.all(got == 0)


@pytest.mark.parametrize("mode", ["bf16", "fp32"])
def test_config1_statistics_vs_oracle(dev, mode):
    x = _lattice_atoms(96, 1152, 21)  # 4,608 atoms, N(0, 0.02) rows normalised as in pollux.py:876-882
    _check(dev, x, mode, label="c1")


def test_nn_b_vs_reference_torch_ops(dev):
    x = _lattice_atoms(64, 1152, 22)
    got = castor.quantize_indices(x.to(dev), mode="bf16").cpu().numpy()
    ref = torch_ref.nn_b_indices(x).numpy()
    near = nn.quantize(x.numpy(), "B")["near_tie"]
    assert np.array_equal(got[~near], ref[~near])


@pytest.mark.parametrize("mode", ["bf16", "fp32"])
def test_boundary_stress_vs_oracle(dev, mode):
    # BASELINE config-3 stress in lattice units: midpoints of code pairs at raw
    # inner product 16 plus N(0, 1e-3) noise, and random directions at norm sqrt 2.
    rng = np.random.default_rng(31)
    c32 = cb.codebook_f32()
    raw = cb.codebook_int8().astype(np.int64)
    pts = []
    while len(pts) < 1500:
        a = int(rng.integers(1, 196561))
        cand = rng.integers(1, 196561, 4000)
        ip = raw[cand] @ raw[a]
        hits = cand[ip == 16]
        if len(hits):
            b = int(hits[0])
            pts.append(0.5 * (c32[a] + c32[b]) + rng.normal(0, 1e-3, 24).astype(np.float32))
    d = rng.normal(size=(1500, 24))
    d = d / np.linalg.norm(d, axis=1, keepdims=True) * np.sqrt(2.0)
    x = torch.from_numpy(np.concatenate([np.stack(pts), d]).astype(np.float32))
    # bf16 rounding of x erases much of the 1e-3 noise, so many midpoints are
    # exact mathematical ties between the two codes: NN-T flags ~10% of atoms
    # (all resolved to the lowest index); NN-B's bf16 buckets absorb them.
    _check(dev, x, mode, max_near=0.05 if mode == "bf16" else 0.25, label="stress")


def test_uniform_sphere_sweep_sample(dev):
    # BASELINE config-4 distribution: directions on S^23, radius U(0,2)*sqrt(32)
    g = torch.Generator().manual_seed(41)
    d = torch.randn(3000, 24, generator=g)
    d = d / d.norm(dim=1, keepdim=True)
    r = torch.rand(3000, 1, generator=g) * 2 * np.sqrt(32.0)
    _check(dev, (d * r).float(), "bf16", label="sweep")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_castor_quantize_leech_returns_codebook_vectors(dev, dtype):
    x = _lattice_atoms(8, 1152, 51).reshape(8, 1152).to(dtype)
    cbk = castor.get_h24_codebook(dev, torch.float32)
    out = castor.castor_quantize_leech(x.to(dev), cbk)
    assert out.shape == x.shape and out.dtype == dtype
    idx = castor.quantize_indices(x.to(dev)).long().cpu()
    want = castor.get_h24_codebook("cpu", dtype)[idx].reshape(x.shape)
    assert torch.equal(out.cpu(), want)
    # straight-through estimator keeps the gradient
    lat = x.to(dev).float().requires_grad_(True)
    y = castor.CastorQuantizeLeech.apply(lat, cbk)
    y.sum().backward()
    assert torch.equal(lat.grad, torch.ones_like(lat))


def test_non_canonical_codebook_is_rejected(dev):
    cbk = castor.get_h24_codebook(dev, torch.float32).clone()
    cbk[5, 0] += 1.0
    with pytest.raises(ValueError):
        castor.castor_quantize_leech(torch.zeros(4, 24, device=dev), cbk)


def test_codebook_checked_again_after_in_place_change_and_address_reuse(dev):
    x = torch.zeros(4, 24, device=dev)
    cbk = castor.get_h24_codebook(dev, torch.float32)
    castor.castor_quantize_leech(x, cbk)  # accepted and cached
    cbk[7, 3] = 0.5  # in place: a new version of the same tensor
    with pytest.raises(ValueError):
        castor.castor_quantize_leech(x, cbk)
    ok = castor.get_h24_codebook(dev, torch.float32)
    castor.castor_quantize_leech(x, ok)
    addr = ok.data_ptr()
    del ok
    bad = torch.empty(196561, 24, device=dev)  # the caching allocator usually hands back the same block
    bad.copy_(castor.get_h24_codebook(dev, torch.float32))
    bad[11, 0] = 9.0
    print(f"[codebook] reused address: {bad.data_ptr() == addr}", flush=True)
    with pytest.raises(ValueError):
        castor.castor_quantize_leech(x, bad)


def test_inference_mode_codebook(dev):
    # an inference tensor has no version counter; it is compared on every call
    x = _lattice_atoms(4, 1152, 52).to(dev)
    with torch.inference_mode():
        cbk = castor.get_h24_codebook(dev, torch.float32)
        a = castor.castor_quantize_leech(x, cbk)
    b = castor.castor_quantize_leech(x, cbk)
    assert torch.equal(a, b)
    with torch.inference_mode():
        bad = cbk.clone()
        bad[3, 3] = 1.0
        with pytest.raises(ValueError):
            castor.castor_quantize_leech(x, bad)


@pytest.mark.parametrize("table", [torch.float16, torch.bfloat16, torch.float64])
@pytest.mark.parametrize("out", [torch.float32, torch.float16, torch.bfloat16])
def test_codebook_dtype_semantics_nn_b(dev, table, out):
    # castor.py:521-559 with a rounded table: NN-B indices equal the fp32 table's
    # (identical bf16 operands; 2*M < c_sq is the same test on bf16 scores), and
    # the vectors are the passed table's values cast to the latent's dtype
    x = _lattice_atoms(8, 1152, 53).to(dev).to(out)
    cbk = castor.get_h24_codebook(dev, table)
    got = castor.castor_quantize_leech(x, cbk)
    idx = castor.quantize_indices(x, mode="bf16").long()
    want = cbk.to(out).index_select(0, idx).view(x.shape)
    assert got.dtype == out and torch.equal(got, want)


def test_codebook_dtype_nn_t_refuses_rounded_tables(dev):
    x = torch.zeros(4, 24, device=dev)
    castor.set_nn_mode("fp32")
    try:
        castor.castor_quantize_leech(x, castor.get_h24_codebook(dev, torch.float32))
        for dt in (torch.float16, torch.bfloat16):
            with pytest.raises(ValueError, match="NN-T"):
                castor.castor_quantize_leech(x, castor.get_h24_codebook(dev, dt))
    finally:
        castor.set_nn_mode("bf16")
