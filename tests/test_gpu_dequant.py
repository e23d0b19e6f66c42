"""HIP dequantization (pollux.py:485-504) against the reference's fp16 torch ops, bit-exact."""

import numpy as np
import pytest
import torch

from oracle import packing, torch_ref
from pollux_amd import PackedH24Linear, castor, dequantize_h24

pytestmark = pytest.mark.gpu


def _packed_layer(out_f, in_f, seed):
    g = torch.Generator().manual_seed(seed)
    n = out_f * in_f // 24
    idx = torch.randint(0, 196561, (n,), generator=g, dtype=torch.int64)
    sig = (torch.rand(out_f, generator=g) * 0.045 + 0.005).to(torch.float16)
    packed = torch.from_numpy(packing.pack(idx.numpy()))
    return idx, sig, packed


@pytest.mark.parametrize("shape", [(96, 1152), (48, 1920), (7, 24), (5, 48), (1920, 7680), (7680, 1920)])
def test_dequant_matches_reference_ops(dev, shape):
    out_f, in_f = shape
    idx, sig, packed = _packed_layer(out_f, in_f, out_f + in_f)
    want = torch_ref.materialize(idx, sig, out_f, in_f)
    got = dequantize_h24(packed.to(dev), sig.to(dev), out_f, in_f).cpu()
    assert got.dtype == torch.float16
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_every_fp16_sigma_and_alphabet_value(dev):
    # all 63,488 finite fp16 sigma (negative, zero, subnormal and huge ones included) x the 8 raw values
    # {0, +-1, +-2, -3, +-4} at several positions: per row one +-4 pair, one +-2 octad and one type-3 code,
    # against the oracle's materialize (pinned exhaustively against numpy's float16 emulation)
    from oracle import codebook as cb

    raw = cb.codebook_int8()
    pick = [int(np.nonzero((raw == 4).any(1) & (raw == -4).any(1))[0][0]),
            int(np.nonzero((raw == 2).any(1) & (raw == -2).any(1))[0][0]),
            int(np.nonzero((raw == -3).any(1) & (raw == 1).any(1) & (raw == -1).any(1))[0][0])]
    sig = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.float16)
    sig = sig[torch.isfinite(sig)]
    rows = sig.numel()
    idx = torch.tensor(pick, dtype=torch.int64).repeat(rows)
    packed = torch.from_numpy(packing.pack(idx.numpy()))
    want = torch_ref.materialize(idx, sig, rows, 72)
    got = dequantize_h24(packed.to(dev), sig.to(dev), rows, 72).cpu()
    bad = (got.view(torch.int16) != want.view(torch.int16)).nonzero()
    assert len(bad) == 0, (len(bad), bad[:5].tolist())


def test_sigma_edge_values(dev):
    out_f, in_f = 6, 48
    idx, _, packed = _packed_layer(out_f, in_f, 1)
    sig = torch.tensor([1e-8, 6.1e-5, 1.0, 65504.0, 0.0, 3.3e-3], dtype=torch.float16)
    want = torch_ref.materialize(idx, sig, out_f, in_f)
    got = dequantize_h24(packed.to(dev), sig.to(dev), out_f, in_f).cpu()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_invalid_indices_decode_as_origin(dev):
    idx = torch.tensor([196561, 262143, 5, 0], dtype=torch.int64)
    packed = torch.from_numpy(packing.pack(idx.numpy()))
    sig = torch.ones(4, dtype=torch.float16)
    got = dequantize_h24(packed.to(dev), sig.to(dev), 4, 24).cpu()
    assert torch.all(got[0] == 0) and torch.all(got[1] == 0)
    want = torch_ref.materialize(torch.tensor([5, 0]), sig[2:], 2, 24)
    assert torch.equal(got[2:], want)


def test_packed_linear_module(dev):
    out_f, in_f = 64, 1152
    idx, sig, packed = _packed_layer(out_f, in_f, 9)
    m = PackedH24Linear(in_f, out_f)
    m.load_state_dict({"packed_weights": packed, "sigma_rows": sig})
    m = m.to(dev)
    m.materialize()
    m.materialize()  # idempotent (pollux.py:486-487)
    assert not hasattr(m, "packed_weights") and not hasattr(m, "sigma_rows")
    want_w = torch_ref.materialize(idx, sig, out_f, in_f)
    assert torch.equal(m.weight.detach().cpu(), want_w)
    x = torch.randn(3, in_f, generator=torch.Generator().manual_seed(1))
    y = m(x.to(dev)).cpu()
    ref = torch_ref.linear_fp32(x, want_w)
    assert torch.allclose(y, ref, rtol=1e-5, atol=1e-6)


def test_roundtrip_through_castor_api(dev):
    g = torch.Generator().manual_seed(2)
    idx = torch.randint(0, 196561, (4 * 1000 + 3,), generator=g, dtype=torch.int64)
    p = castor.pack_indices(idx.to(dev))
    back = castor.unpack_indices(p, idx.numel()).cpu()
    assert torch.equal(back, idx)
    assert np.array_equal(p.cpu().numpy(), packing.pack(idx.numpy()))
