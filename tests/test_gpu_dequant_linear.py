"""Fused dequant-linear (PackedH24Linear.forward, pollux.py:485-507) against the reference's fp32 F.linear.

packed [7680, 1920] and [1920, 7680] (torch (out, in) layout),
indices uniform over 0..196560, sigma16 ~ U(0.005, 0.05), bf16 activations
N(0, 1) at batch 1 (GEMV) and 64 (GEMM), fp32 accumulation.
Tolerance (stated): relative L2 error <= 1e-5 against F.linear(x.float(),
W16.float()), and per element |dy| <= 1e-5 * sum_i |x_i W_i| (the products are
exact in fp32; only the summation order differs).
"""

import pytest
import torch

from oracle import packing, torch_ref
from pollux_amd import PackedH24Linear, dequant_linear

pytestmark = pytest.mark.gpu

REL_L2 = 1e-5
ELEM = 1e-5


def _layer(out_f, in_f, seed):
    g = torch.Generator().manual_seed(seed)
    n = out_f * in_f // 24
    idx = torch.randint(0, 196561, (n,), generator=g, dtype=torch.int64)
    sig = (torch.rand(out_f, generator=g) * 0.045 + 0.005).to(torch.float16)
    packed = torch.from_numpy(packing.pack(idx.numpy()))
    return idx, sig, packed, g


def _check(y, x, w16):
    ref = torch_ref.linear_fp32(x, w16)
    err = (y.double() - ref.double())
    rel = err.norm() / ref.double().norm()
    bound = ELEM * (x.double().abs() @ w16.double().abs().t())
    worst = (err.abs() / bound).max().item()
    print(f"[dql] rel_l2 {rel:.3e} worst elem/bound {worst:.3f}", flush=True)
    assert rel <= REL_L2
    assert worst <= 1.0


@pytest.mark.parametrize("shape", [(7680, 1920), (1920, 7680)])
@pytest.mark.parametrize("m", [1, 64])
def test_config5_bf16_activations(dev, shape, m):
    out_f, in_f = shape
    idx, sig, packed, g = _layer(out_f, in_f, out_f + m)
    x = torch.randn(m, in_f, generator=g).to(torch.bfloat16)
    w16 = torch_ref.materialize(idx, sig, out_f, in_f)
    y = dequant_linear(packed.to(dev), sig.to(dev), out_f, in_f, x.to(dev)).cpu()
    assert y.dtype == torch.float32 and y.shape == (m, out_f)
    _check(y, x.float(), w16)


@pytest.mark.parametrize("shape,m", [((1152, 1152), 17), ((37, 1920), 33), ((4608, 1152), 100), ((20, 240), 64)])
def test_mfma_gemm_batches_bf16(dev, shape, m):
    out_f, in_f = shape
    idx, sig, packed, g = _layer(out_f, in_f, 3 * out_f + m)
    x = (torch.randn(m, in_f, generator=g) * 2.0).to(torch.bfloat16)
    w16 = torch_ref.materialize(idx, sig, out_f, in_f)
    y = dequant_linear(packed.to(dev), sig.to(dev), out_f, in_f, x.to(dev)).cpu()
    _check(y, x.float(), w16)


@pytest.mark.parametrize("shape,m", [((37, 48), 3), ((1152, 1152), 5), ((100, 4608), 2), ((24, 24), 1)])
def test_ragged_shapes_fp32_activations(dev, shape, m):
    out_f, in_f = shape
    idx, sig, packed, g = _layer(out_f, in_f, 7 * out_f + m)
    x = torch.randn(m, in_f, generator=g) * 3.0
    w16 = torch_ref.materialize(idx, sig, out_f, in_f)
    y = dequant_linear(packed.to(dev), sig.to(dev), out_f, in_f, x.to(dev)).cpu()
    _check(y, x, w16)


def test_packed_layer_forward_without_materialize(dev):
    out_f, in_f = 96, 1152
    idx, sig, packed, g = _layer(out_f, in_f, 11)
    m = PackedH24Linear(in_f, out_f, bias=True)
    with torch.no_grad():
        m.bias.copy_(torch.randn(out_f, generator=g))
    m.load_state_dict({"packed_weights": packed, "sigma_rows": sig, "bias": m.bias.detach().clone()})
    m = m.to(dev)
    x = torch.randn(2, 3, in_f, generator=g)
    y_fused = m(x.to(dev)).cpu()
    m.materialize()
    y_dense = m(x.to(dev)).cpu()
    w16 = torch_ref.materialize(idx, sig, out_f, in_f)
    ref = torch_ref.linear_fp32(x.reshape(-1, in_f), w16).reshape(2, 3, out_f) + m.bias.detach().cpu()
    assert y_fused.shape == (2, 3, out_f)
    assert ((y_fused - ref).norm() / ref.norm()).item() <= REL_L2
    assert ((y_dense - ref).norm() / ref.norm()).item() <= 1e-5
