"""HIP NN-P pack-time quantizer (pack.py:139-180) against the exact oracle and the reference's torch ops.

Bar: indices bit-exact on every atom that is not a near-tie within the fp32
envelope DELTA_REL * sum|x_i c_i| (oracle/nn.py, mode "P"); near-ties are
counted and must stay rare.  sigma_rows within 1 fp16 ulp of the torch
restatement (summation order of the row mean), packed bytes equal to
pack(indices).
"""

import numpy as np
import pytest
import torch

from oracle import codebook as cb
from oracle import nn, packing, torch_ref
from pollux_amd import castor
from pollux_amd import pack as plx_pack

pytestmark = pytest.mark.gpu


def _check_p(dev, w, max_near=0.01, label=""):
    x = w.reshape(-1, 24)
    got = castor.quantize_indices(x.to(dev), mode="pack").cpu().numpy().astype(np.int64)
    r = nn.quantize(x.numpy(), "P")
    near = r["near_tie"]
    bad = (got != r["idx"]) & ~near
    print(f"[{label} P] atoms={len(got)} near_ties={int(near.sum())} "
          f"mismatch_on_near_ties={int(((got != r['idx']) & near).sum())} mismatch_non_near={int(bad.sum())}",
          flush=True)
    assert near.mean() <= max_near
    assert not bad.any(), np.nonzero(bad)[0][:10]
    return got, r


@pytest.mark.parametrize("alpha", [1.0, 0.37, 5.0, 1e-3])
def test_scaled_codebook_vectors_are_fixed_points(dev, alpha):
    c = torch.from_numpy(cb.codebook_f32()[1:].copy()) * alpha
    got = castor.quantize_indices(c.to(dev), mode="pack").cpu()
    assert torch.equal(got.long(), torch.arange(1, 196561))


def test_origin_rule_is_the_atom_norm(dev):
    g = torch.Generator().manual_seed(3)
    d = torch.randn(600, 24, generator=g)
    d = d / d.norm(dim=1, keepdim=True)
    x = torch.cat([torch.zeros(8, 24), d[:200] * 1e-10, d[200:400] * 5e-9, d[400:] * 1e-7])
    got = castor.quantize_indices(x.to(dev), mode="pack").cpu()
    assert torch.all(got[:408] == 0)          # |x| < 1e-8: origin, whatever the scores
    assert torch.all(got[408:] > 0)           # |x| = 1e-7: a kissing point, never the origin
    r = nn.quantize(x.numpy(), "P")
    ok = ~r["near_tie"]
    assert np.array_equal(got.numpy()[ok], r["idx"][ok])


@pytest.mark.parametrize("n", [1, 5, 511, 513, 2049])
def test_ragged_sizes(dev, n):
    g = torch.Generator().manual_seed(100 + n)
    _check_p(dev, torch.randn(n, 24, generator=g), label=f"n={n}")


def test_config1_weights_vs_oracle(dev):
    g = torch.Generator().manual_seed(11)
    w = torch.randn(96, 1152, generator=g) * 0.02  # 4,608 raw atoms (pack.py quantizes p.data directly)
    _check_p(dev, w, label="c1")


def test_scale_invariance(dev):
    g = torch.Generator().manual_seed(12)
    w = torch.randn(2048, 24, generator=g)
    a = castor.quantize_indices(w.to(dev), mode="pack").cpu().numpy()
    b = castor.quantize_indices((w * 37.0).to(dev), mode="pack").cpu().numpy()
    near = nn.quantize(w.numpy(), "P")["near_tie"] | nn.quantize((w * 37.0).numpy(), "P")["near_tie"]
    assert np.array_equal(a[~near], b[~near])


def test_vs_reference_torch_ops(dev):
    g = torch.Generator().manual_seed(13)
    w = torch.randn(64, 1152, generator=g) * 0.02
    got = castor.quantize_indices(w.reshape(-1, 24).to(dev), mode="pack").cpu().numpy()
    ref = torch_ref.nn_p_indices(w).numpy()
    near = nn.quantize(w.reshape(-1, 24).numpy(), "P")["near_tie"]
    assert np.array_equal(got[~near], ref[~near])


def test_midpoint_stress_vs_oracle(dev):
    # midpoints of code pairs at raw inner product 16 with N(0, 1e-4) noise:
    # two codes nearly tie on every atom; only the fp32-exact order decides.
    rng = np.random.default_rng(14)
    c32 = cb.codebook_f32()
    raw = cb.codebook_int8().astype(np.int64)
    pts = []
    while len(pts) < 1500:
        a = int(rng.integers(1, 196561))
        cand = rng.integers(1, 196561, 4000)
        hits = cand[(raw[cand] @ raw[a]) == 16]
        if len(hits):
            pts.append(0.5 * (c32[a] + c32[int(hits[0])]) + rng.normal(0, 1e-4, 24).astype(np.float32))
    _check_p(dev, torch.from_numpy(np.stack(pts).astype(np.float32)), max_near=0.05, label="midpoints")


def test_quantize_h24_layer_matches_reference_composition(dev):
    g = torch.Generator().manual_seed(15)
    w = torch.randn(200, 480, generator=g) * 0.02
    w[3] = 0.0                                                # an all-zero row: sigma clamps to 1e-8
    cbk = castor.get_h24_codebook(dev, torch.float32)
    packed, sigma = plx_pack._quantize_h24_layer(w.to(dev), cbk)
    assert packed.device.type == "cpu" and sigma.device.type == "cpu"
    assert packed.dtype == torch.uint8 and sigma.dtype == torch.float16
    n = w.numel() // 24
    assert packed.numel() == ((n + 3) // 4) * 9 and sigma.shape == (200,)
    idx = packing.unpack(packed.numpy(), n)
    r = nn.quantize(w.reshape(-1, 24).numpy(), "P")
    ok = ~r["near_tie"]
    assert np.array_equal(idx[ok], r["idx"][ok])
    # bytes are the reference packing of the kernel's own indices
    assert np.array_equal(packed.numpy(), packing.pack(idx))
    want = torch_ref.sigma16_pack(w)
    d = (sigma.view(torch.int16).long() - want.view(torch.int16).long()).abs()
    assert d.max() <= 1 and sigma[3].item() == want[3].item()
    # device variant with indices agrees
    p2, s2, i2 = plx_pack.quantize_h24_layer(w.to(dev), return_indices=True)
    assert torch.equal(p2.cpu(), packed) and torch.equal(s2.cpu(), sigma)
    assert np.array_equal(i2.cpu().numpy().astype(np.int64), idx)


def test_quantize_h24_layer_codebook_dtypes(dev):
    # pack.py:167: the fp16 table is the raw codes times 0.353515625 exactly, so
    # its indices equal the fp32 table's off near-ties; a bf16 table is refused
    g = torch.Generator().manual_seed(16)
    w = (torch.randn(64, 480, generator=g) * 0.02).to(dev)
    p32, s32 = plx_pack._quantize_h24_layer(w, castor.get_h24_codebook(dev, torch.float32))
    p16, s16 = plx_pack._quantize_h24_layer(w, castor.get_h24_codebook(dev, torch.float16))
    assert torch.equal(s32, s16)
    n = w.numel() // 24
    i32, i16 = packing.unpack(p32.numpy(), n), packing.unpack(p16.numpy(), n)
    diff = np.nonzero(i32 != i16)[0]
    if len(diff):
        r = nn.quantize(w.reshape(-1, 24).cpu().numpy()[diff], "P")
        assert r["near_tie"].all()
    with pytest.raises(ValueError, match="bfloat16"):
        plx_pack._quantize_h24_layer(w, castor.get_h24_codebook(dev, torch.bfloat16))
