"""Fused requantize (pollux.py:874-884 + castor.pack_indices) against the reference's ops."""

import numpy as np
import pytest
import torch

from oracle import nn, packing, torch_ref
from pollux_amd import castor

pytestmark = pytest.mark.gpu


def _ulp_diff(a, b):
    ai = a.numpy().view(np.int32).astype(np.int64)
    bi = b.numpy().view(np.int32).astype(np.int64)
    return np.abs(ai - bi)


@pytest.mark.parametrize("shape,seed", [((1152, 1152), 1), ((96, 4608), 2), ((40, 1920), 3), ((3, 24), 4), ((5, 48), 5)])
def test_requantize_matches_reference(dev, shape, seed):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(*shape, generator=g) * 0.02
    r = castor.requantize_h24(w.to(dev))
    sig = r["sigma"].cpu()
    # sigma: the reference's CPU reduction order differs; allow 2 fp32 ulp
    d = _ulp_diff(sig, torch_ref.row_rms(w))
    print(f"[requant {shape}] sigma exact {np.mean(d == 0):.4f} max ulp {d.max()}", flush=True)
    assert d.max() <= 2
    # indices: NN-B on x = (w / sigma) / s_lattice with the kernel's sigma
    x, _ = torch_ref.lattice_input(w, sig)
    idx = r["indices"].cpu().numpy().astype(np.int64)
    sub = slice(0, min(len(idx), 4608))
    o = nn.quantize(x.reshape(-1, 24)[sub].numpy(), "B")
    bad = (idx[sub] != o["idx"]) & ~o["near_tie"]
    print(f"[requant {shape}] near_ties {int(o['near_tie'].sum())}/{len(o['idx'])}", flush=True)
    assert not bad.any()
    # packed bytes are the reference packing of the kernel's own indices (all atoms)
    assert np.array_equal(r["packed"].cpu().numpy(), packing.pack(idx))
    # weight = (codebook[idx] * sigma) * s_lattice, bit-exact (all atoms)
    center = torch_ref.codebook_tensor()[torch.from_numpy(idx)].reshape(shape)
    want = torch_ref.reconstruct(center, sig)
    assert torch.equal(r["weight"].cpu(), want)


def test_requantize_composition_equals_mirrored_api(dev):
    # the unfused castor-API composition of pollux.py:876-884 gives the same weight
    g = torch.Generator().manual_seed(8)
    w = (torch.randn(48, 1152, generator=g) * 0.02).to(dev)
    r = castor.requantize_h24(w)
    normed, sig = castor.normalize_matrix_by_row_rms(w)
    cbk = castor.get_h24_codebook(dev, torch.float32)
    center = castor.castor_quantize_leech(normed / float(castor.s_lattice), cbk)
    p = castor.scale_matrix_by_row_rms(center, sig) * float(castor.s_lattice)
    assert torch.equal(sig, r["sigma"])
    assert torch.equal(p, r["weight"])


def test_sigma16_pack(dev):
    g = torch.Generator().manual_seed(9)
    w = torch.randn(300, 1152, generator=g) * 0.02
    got = castor.sigma16_pack(w.to(dev)).cpu()
    want = torch_ref.sigma16_pack(w)
    d = (got.view(torch.int16).long() - want.view(torch.int16).long()).abs()
    assert d.max() <= 1
    print(f"[sigma16] exact {float((d == 0).float().mean()):.4f}", flush=True)


def test_batched_requantize_equals_separate_calls(dev):
    # plx_requantize_batch: one scoring sweep over the atoms of several latents
    # (BASELINE config-2 layer + a ragged small matrix); every output equals the
    # separate requantize_h24 calls, except indices that differ only on
    # near-tie atoms (checked against the oracle).
    g = torch.Generator().manual_seed(77)
    shapes = [(3456, 1152), (1152, 1152), (4608, 1152), (1152, 4608), (5, 24), (0, 48), (3, 72)]
    lats = [((torch.randn(r, c, generator=g) * 0.02).to(torch.bfloat16).float()).to(dev) for r, c in shapes]
    many = castor.requantize_h24_many(lats)
    for lat, got in zip(lats, many):
        one = castor.requantize_h24(lat)
        assert torch.equal(got["sigma"], one["sigma"])
        diff = (got["indices"] != one["indices"]).nonzero().flatten().cpu().numpy()
        if len(diff):
            x, _ = torch_ref.lattice_input(lat.cpu(), one["sigma"].cpu())
            r = nn.quantize(x.reshape(-1, 24)[torch.from_numpy(diff)].numpy(), "B")
            assert r["near_tie"].all(), diff[~r["near_tie"]][:10]
            assert len(diff) <= max(3, got["indices"].numel() // 1000)
        else:
            assert torch.equal(got["packed"], one["packed"])
            assert torch.equal(got["weight"], one["weight"])
        assert np.array_equal(got["packed"].cpu().numpy(), packing.pack(got["indices"].cpu().numpy().astype(np.int64)))
