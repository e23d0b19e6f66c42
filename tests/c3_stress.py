"""BASELINE config 3's boundary-stress atoms (shared by the full-size and the parity tests).

The four Pollux-1920 latents (QKV 5760x1920, O 1920x1920, up 7680x1920, down
1920x7680), seeded N(0, 0.02) fp32, in lattice units (pollux.py:876-882:
x = (w / row_rms) / fp32(1/sqrt 2)): 1,843,200 atoms.  5% of them (92,160) are
replaced by midpoints (a + b) / 2 of random code pairs at raw inner product 16
(the true-Leech contact) plus N(0, 1e-3^2) noise, another 5% by random
directions at norm sqrt 2 (where 2 x.c meets c_sq: the origin boundary).  The
replaced atoms are written into x directly, so the row scales are those of the
unmodified latents.
"""

import numpy as np
import torch

from oracle import codebook as cb
from oracle import torch_ref

SHAPES = [(5760, 1920), (1920, 1920), (7680, 1920), (1920, 7680)]
N_ATOMS = 1_843_200


def build(seed=303):
    """(x fp32 [1,843,200, 24] on the CPU, midpoint atom positions, near-origin atom positions)."""
    g = torch.Generator().manual_seed(seed)
    xs = []
    for r, c in SHAPES:
        w = torch.randn(r, c, generator=g) * 0.02
        x, _ = torch_ref.lattice_input(w)
        xs.append(x.reshape(-1, 24))
    x = torch.cat(xs)
    n = x.shape[0]
    assert n == N_ATOMS
    rng = np.random.default_rng(seed)
    perm = rng.permutation(n)
    mid_at, near_at = perm[: n // 20], perm[n // 20: n // 10]
    raw = cb.codebook_int8()
    c32 = cb.codebook_f32()
    a = rng.integers(1, 196561, len(mid_at))
    b = np.zeros_like(a)
    todo = np.arange(len(a))
    while len(todo):  # a partner at raw inner product 16
        for lo in range(0, len(todo), 4096):
            t = todo[lo: lo + 4096]
            cand = rng.integers(1, 196561, (len(t), 256))
            ip = np.einsum("nkd,nd->nk", raw[cand].astype(np.int32), raw[a[t]].astype(np.int32))
            hit = ip == 16
            ok = hit.any(axis=1)
            b[t[ok]] = cand[ok, hit[ok].argmax(axis=1)]
        todo = todo[b[todo] == 0]
    mids = 0.5 * (c32[a] + c32[b]) + rng.normal(0, 1e-3, (len(a), 24)).astype(np.float32)
    dirs = rng.normal(size=(len(near_at), 24))
    dirs = dirs / np.linalg.norm(dirs, axis=1, keepdims=True) * np.sqrt(2.0)
    x[torch.from_numpy(mid_at)] = torch.from_numpy(mids.astype(np.float32))
    x[torch.from_numpy(near_at)] = torch.from_numpy(dirs.astype(np.float32))
    return x, mid_at, near_at
