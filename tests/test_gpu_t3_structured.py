"""The structured type-3 scorer (t3_kernel, the NN-B default) against the dense type-3 sweep and the oracle.

Both compute NN-B (castor.py:544-557): indices must be equal on every atom that
is not a near-tie (oracle/nn.py classifies each disagreement).  Cases: the
config-4 distribution at every launch size the scorer distinguishes (1, 2 and
4 atom tiles per wave), atoms dominated by one coordinate (whose
candidate threshold falls to zero or below, so both signs of a word are
listed), near-origin and zero atoms, ragged small launches, atoms whose
best code sits in the type-3 family by construction (scaled type-3 codes plus
noise), and integer atoms, whose scores are exact in any summation order, so
both paths must agree on every atom through the exact ties between codes --
among them sums of a type-3 and a type-2 code that tie at the best bucket, so
that t12_kernel's type-3 floor meets its best pair bucket.
"""

import numpy as np
import pytest
import torch

from oracle import codebook as cb
from oracle import nn
from pollux_amd import castor

pytestmark = pytest.mark.gpu


def _c4_atoms(n, seed):
    g = torch.Generator().manual_seed(seed)
    d = torch.randn(n, 24, generator=g)
    return d / d.norm(dim=1, keepdim=True) * (torch.rand(n, 1, generator=g) * 2.0 * np.sqrt(32.0))


def _compare(dev, x, label, max_near=0.002):
    xs = x.to(dev)
    got = castor.quantize_indices(xs, mode="bf16").long().cpu()
    ref = castor.quantize_indices(xs, mode="bf16-dense").long().cpu()
    diff = (got != ref).nonzero().flatten()
    near = 0
    if len(diff):
        o = nn.quantize(x[diff].numpy(), "B")
        near = int(o["near_tie"].sum())
        bad = diff[torch.from_numpy(~o["near_tie"])]
        assert len(bad) == 0, (label, bad[:10].tolist(), got[bad[:10]].tolist(), ref[bad[:10]].tolist())
    print(f"[t3 {label}] atoms={len(x)} disagree={len(diff)} near_ties={near}", flush=True)
    assert len(diff) <= max(2, max_near * len(x))
    return got


# (the scorers take 1 atom tile per wave below 98,304 atoms, 2 below 131,072, else 4)
@pytest.mark.parametrize("n", [1000, 40_000, 98_304, 131_071, 140_000, 300_000])
def test_structured_equals_dense_c4(dev, n):
    _compare(dev, _c4_atoms(n, n), f"c4 n={n}")


@pytest.mark.parametrize("n", [1, 5, 63, 65, 513, 4097])
def test_ragged_small_launches(dev, n):
    x = _c4_atoms(n, 7 + n)
    got = _compare(dev, x, f"ragged n={n}")
    o = nn.quantize(x.numpy(), "B")
    ok = ~o["near_tie"]
    assert np.array_equal(got.numpy()[ok], o["idx"][ok])


def test_spiky_atoms(dev):
    # one coordinate far larger than the rest: the bound on the bonus spans the whole S range, so the
    # candidate threshold is <= 0 and both signs of words are listed (the slow but exact path)
    g = torch.Generator().manual_seed(11)
    n = 20_000
    x = torch.randn(n, 24, generator=g) * 0.05
    k = torch.randint(0, 24, (n,), generator=g)
    mag = torch.rand(n, generator=g) * 8.0 + 1.0
    sign = torch.where(torch.rand(n, generator=g) < 0.5, -1.0, 1.0)
    x[torch.arange(n), k] = mag * sign
    _compare(dev, x, "spiky")


def test_near_origin_and_zero_atoms(dev):
    g = torch.Generator().manual_seed(12)
    d = torch.randn(30_000, 24, generator=g)
    d = d / d.norm(dim=1, keepdim=True)
    r = torch.rand(30_000, 1, generator=g) * 2.5  # around the origin boundary (norm sqrt 2 in these units)
    x = torch.cat([torch.zeros(100, 24), d * r])
    got = _compare(dev, x, "near-origin")
    assert torch.all(got[:100] == 0)


def test_type3_winners(dev):
    # scaled type-3 codes plus noise: the type-3 family holds the answer, often with close runners-up
    rng = np.random.default_rng(13)
    c32 = cb.codebook_f32()
    raw = cb.codebook_int8()
    t3 = np.nonzero((raw == -3).any(1))[0]
    pick = rng.choice(t3, 20_000)
    x = c32[pick] * rng.uniform(0.6, 1.6, (20_000, 1)) + rng.normal(0, 0.08, (20_000, 24))
    got = _compare(dev, torch.from_numpy(x.astype(np.float32)), "type-3 winners")
    assert (got.numpy() == pick).mean() > 0.5


def test_fixed_points_of_every_type3_code(dev):
    c = torch.from_numpy(cb.codebook_f32()[1:].copy())
    got = castor.quantize_indices(c.to(dev), mode="bf16").long().cpu()
    assert torch.equal(got, torch.arange(1, 196561))


def test_row_sweep_path_equals_survivor_path(dev):
    # the lowest row at the best bucket comes from the per-wave survivor lists unless one overflows; the
    # overflow path (a second sweep over the patterns) must give the same indices on every atom
    g = torch.Generator().manual_seed(14)
    n = 60_000
    spiky = torch.randn(n // 4, 24, generator=g) * 0.05
    spiky[torch.arange(n // 4), torch.randint(0, 24, (n // 4,), generator=g)] = 4.0
    raw = torch.from_numpy(cb.codebook_f32())
    t3 = torch.nonzero(torch.from_numpy((cb.codebook_int8() == -3).any(1))).flatten()
    pick = t3[torch.randint(0, len(t3), (n // 4,), generator=g)]
    near_t3 = raw[pick] * 1.1 + torch.randn(n // 4, 24, generator=g) * 0.08
    x = torch.cat([_c4_atoms(n // 2, 15), spiky, near_t3]).to(dev)
    a = castor.quantize_indices(x, mode="bf16").cpu()
    b = castor.quantize_indices(x, mode="bf16-rows-sweep").cpu()
    assert torch.equal(a, b), int((a != b).sum())


def test_integer_atoms_exact_ties(dev):
    # integer coordinates: every score is an exact fp32 sum in any order (multiples of 2^-9 below 2^15),
    # so the structured and the dense path see the same bf16 buckets and must pick the same lowest row
    # on every atom -- including the many exact ties between codes -- and the oracle's answer wherever it
    # is determined (exact bf16 midpoints, where the reference rounds to even, are its near-ties)
    g = torch.Generator().manual_seed(16)
    raw = torch.from_numpy(cb.codebook_int8().astype(np.float32))
    n = 6_000
    a = torch.randint(1, 196561, (n,), generator=g)
    b = torch.randint(1, 196561, (n,), generator=g)
    x = torch.cat([raw[a] + raw[b],                                    # sums of two codes
                   torch.randint(-4, 5, (n, 24), generator=g).float(),  # small integer vectors
                   2.0 * raw[a[: n // 2]],                              # scaled codes
                   torch.randint(-1, 2, (n // 2, 24), generator=g).float()])
    xs = x.to(dev)
    s = castor.quantize_indices(xs, mode="bf16").long().cpu()
    d = castor.quantize_indices(xs, mode="bf16-dense").long().cpu()
    r = castor.quantize_indices(xs, mode="bf16-rows-sweep").long().cpu()
    assert torch.equal(s, d), int((s != d).sum())
    assert torch.equal(s, r), int((s != r).sum())
    sub = torch.cat([torch.arange(k, k + 375) for k in (0, n, 2 * n, 2 * n + n // 2)])  # 375 of each kind
    o = nn.quantize(x[sub].numpy(), "B")
    ok = ~o["near_tie"]
    print(f"[t3 integer atoms] {len(x)} atoms equal on both paths; oracle on {len(sub)}: "
          f"{int((~ok).sum())} near-ties", flush=True)
    assert np.array_equal(s[sub].numpy()[ok], o["idx"][ok])


def _contact_midpoints(n, seed):
    # midpoints of code pairs at raw inner product 16 (the contact pairs) plus tiny noise: many codes tie at
    # the best bucket there, so the scorers' per-wave survivor lists overflow for some atoms and not others
    rng = np.random.default_rng(seed)
    raw = cb.codebook_int8().astype(np.int64)
    c32 = cb.codebook_f32()
    a = rng.integers(1, 196561, 8 * n)
    b = rng.integers(1, 196561, (8 * n, 64))
    ip = (raw[b] * raw[a][:, None, :]).sum(-1)
    ok = (ip == 16).any(1)
    a, b, ip = a[ok][:n], b[ok][:n], ip[ok][:n]
    bb = b[np.arange(len(a)), (ip == 16).argmax(1)]
    return torch.from_numpy((0.5 * (c32[a] + c32[bb]) + rng.normal(0, 1e-3, (len(a), 24))).astype(np.float32))


def test_midpoints_among_ordinary_atoms(dev):
    # some waves lose survivors (their atoms' rows come from the second sweep), the rest keep theirs
    mid = _contact_midpoints(3000, 17)
    x = _c4_atoms(60_000, 18)
    pos = torch.randperm(len(x), generator=torch.Generator().manual_seed(19))[: len(mid)]
    x[pos] = mid
    got = _compare(dev, x, "midpoints among c4 atoms", max_near=0.01)
    r = castor.quantize_indices(x.to(dev), mode="bf16-rows-sweep").long().cpu()
    assert torch.equal(got, r), int((got != r).sum())


def test_non_finite_atoms_go_to_the_origin(dev):
    # a NaN or infinite coordinate: both NN-B paths give the origin (the reference's torch ops give the first
    # row whose score is NaN, outside any tested domain); the other atoms of the launch are unaffected
    x = _c4_atoms(5000, 20)
    ref = castor.quantize_indices(x.to(dev), mode="bf16").long().cpu()
    bad = torch.arange(0, 5000, 97)
    x[bad[0::3], 5] = float("nan")
    x[bad[1::3], 7] = float("inf")
    x[bad[2::3], 11] = -float("inf")
    x[bad[:5]] = float("nan")
    s = castor.quantize_indices(x.to(dev), mode="bf16").long().cpu()
    d = castor.quantize_indices(x.to(dev), mode="bf16-dense").long().cpu()
    assert torch.all(s[bad] == 0) and torch.all(d[bad] == 0)
    keep = torch.ones(5000, dtype=torch.bool)
    keep[bad] = False
    assert torch.equal(s[keep], ref[keep])


def test_pair_and_type3_ties(dev):
    # x = c2 + c3 for a type-3 code c3 and a type-2 code c2 of largest c2.c3 (integer units): both codes
    # score 32 + c2.c3, exactly in any summation order, so the best bucket usually holds both families and
    # the answer is the lower row.  t12_kernel's Chase-decoded type-3 floor then equals its best pair
    # bucket (the pair row must survive the tie) or exceeds it (the pair key carries the floor without a
    # row); every atom must match the dense path and, where determined, the oracle
    rng = np.random.default_rng(17)
    raw = cb.codebook_int8().astype(np.float32)
    nz = (raw != 0).sum(1)
    t2 = np.nonzero(nz == 8)[0]
    t3 = np.nonzero(nz == 24)[0]
    c3 = rng.choice(t3, 3000)
    c2 = np.empty_like(c3)
    for k in range(0, len(c3), 250):
        dots = raw[c3[k:k + 250]] @ raw[t2].T  # exact small integers
        best = dots.max(1, keepdims=True)
        for i, row in enumerate(dots == best):
            c2[k + i] = t2[rng.choice(np.nonzero(row)[0])]
    x = torch.from_numpy(raw[c2] + raw[c3])
    xs = x.to(dev)
    s = castor.quantize_indices(xs, mode="bf16").long().cpu()
    d = castor.quantize_indices(xs, mode="bf16-dense").long().cpu()
    assert torch.equal(s, d), int((s != d).sum())
    # (the oracle on a sample: every answer is the lower of the two rows, c2 and c3 about equally often;
    # a third code at the same bucket could take a few atoms)
    lower = (s.numpy() == np.minimum(c2, c3)).mean()
    print(f"[t3 pair/type-3 ties] {len(x)} atoms: answer is the lower of the two rows on {lower:.3f}", flush=True)
    assert lower >= 0.99 and 0.3 < (s.numpy() == c2).mean() < 0.7
    sub = np.arange(0, len(x), 5)
    o = nn.quantize(x[sub].numpy(), "B")
    ok = ~o["near_tie"]
    assert np.array_equal(s[sub].numpy()[ok], o["idx"][ok])
