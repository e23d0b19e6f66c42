"""Fused dequant-linear (PackedH24Linear.forward, pollux.py:485-507) against the reference's F.linear.

packed [7680, 1920] and [1920, 7680] (torch (out, in) layout),
indices uniform over 0..196560, sigma16 ~ U(0.005, 0.05), bf16 activations
N(0, 1) at batch 1 (GEMV) and 64 (GEMM), fp32 accumulation.
Default mode ("exact"): the expected value is F.linear(x.float(), W16.float())
(oracle.torch_ref.linear_fp32), the fp32 numerics of pollux.py:507.
Mode "as_x": the reference's literal F.linear(x, W16.to(x.dtype)), which for
bf16 activations rounds the fp16 weight to bf16 first, evaluated in fp32
(oracle.torch_ref.linear_as_reference); its distance from the exact product
(~1.7e-3 relative at config 5) is printed as context.
Tolerance (stated), either mode: relative L2 error <= 1e-5, and per element
|dy| <= 1e-5 * sum_i |x_i W_i| (the products are exact in fp32; only the
summation order differs).  For bf16 activations each check also asserts that
the result is > 1e-4 away from the other mode's expected value, so the tests
tell the two roundings apart.
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


def _check(y, x, w16, mode="exact"):
    """y against the expected value of `mode` (x in its own dtype)."""
    exact = torch_ref.linear_fp32(x, w16).double()
    literal = torch_ref.linear_as_reference(x, w16).double()
    ref, other = (exact, literal) if mode == "exact" else (literal, exact)
    w = (w16 if mode == "exact" else w16.to(x.dtype)).double()
    err = y.double() - ref
    rel = err.norm() / ref.norm()
    bound = ELEM * (x.double().abs() @ w.abs().t())
    worst = (err.abs() / bound).max().item()
    ctx = ((literal - exact).norm() / exact.norm()).item()
    print(f"[dql] {mode}: rel_l2 {rel:.3e} worst elem/bound {worst:.3f}; literal-vs-exact {ctx:.2e}", flush=True)
    assert rel <= REL_L2
    assert worst <= 1.0
    if x.dtype == torch.bfloat16:
        assert (y.double() - other).norm() / other.norm() > 1e-4  # the two roundings are told apart


@pytest.mark.parametrize("shape", [(7680, 1920), (1920, 7680)])
@pytest.mark.parametrize("m", [1, 64])
def test_config5_bf16_activations(dev, shape, m):
    out_f, in_f = shape
    idx, sig, packed, g = _layer(out_f, in_f, out_f + m)
    x = torch.randn(m, in_f, generator=g).to(torch.bfloat16)
    w16 = torch_ref.materialize(idx, sig, out_f, in_f)
    y = dequant_linear(packed.to(dev), sig.to(dev), out_f, in_f, x.to(dev)).cpu()
    assert y.dtype == torch.float32 and y.shape == (m, out_f)
    _check(y, x, w16)


# cases: K split with partials (1152 x 1152), 2-tile token slab (m <= 32), rows % 4 != 0 (37),
# two token slabs (m = 100), rows of a non-multiple of 4 atoms in one block (1176 = 49 atoms)
# and over several blocks (240 = 10 atoms), one atom per row (24)
@pytest.mark.parametrize("shape,m", [((1152, 1152), 17), ((37, 1920), 33), ((4608, 1152), 100), ((20, 240), 64),
                                     ((64, 1176), 40), ((130, 24), 20)])
def test_mfma_gemm_batches_bf16(dev, shape, m):
    out_f, in_f = shape
    idx, sig, packed, g = _layer(out_f, in_f, 3 * out_f + m)
    x = (torch.randn(m, in_f, generator=g) * 2.0).to(torch.bfloat16)
    w16 = torch_ref.materialize(idx, sig, out_f, in_f)
    y = dequant_linear(packed.to(dev), sig.to(dev), out_f, in_f, x.to(dev)).cpu()
    _check(y, x, w16)


@pytest.mark.parametrize("shape,m", [((1152, 1152), 7), ((37, 48), 2), ((100, 4608), 16)])
def test_gemv_bf16_small_batches(dev, shape, m):
    # batches of up to 16 tokens take the GEMV kernel, which rounds the magnitudes to bf16
    out_f, in_f = shape
    idx, sig, packed, g = _layer(out_f, in_f, 5 * out_f + m)
    x = torch.randn(m, in_f, generator=g).to(torch.bfloat16)
    w16 = torch_ref.materialize(idx, sig, out_f, in_f)
    y = dequant_linear(packed.to(dev), sig.to(dev), out_f, in_f, x.to(dev)).cpu()
    _check(y, x, w16)


@pytest.mark.parametrize("shape,m", [((37, 48), 3), ((1152, 1152), 5), ((100, 4608), 2), ((24, 24), 1),
                                     ((7680, 1920), 64), ((1920, 7680), 64), ((37, 1920), 33), ((64, 1176), 40),
                                     ((4608, 1152), 100), ((130, 24), 20), ((5, 73728), 1), ((3, 73728), 20)])
def test_ragged_shapes_fp32_activations(dev, shape, m):
    # m > 16 runs the MFMA GEMM with each fp32 activation split into three bf16 parts
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


@pytest.mark.parametrize("shape,m", [((7680, 1920), 64), ((1920, 7680), 64), ((7680, 1920), 1), ((1152, 1152), 17),
                                     ((37, 1920), 5)])
def test_reference_literal_rounding(dev, shape, m):
    # weight_rounding="as_x": F.linear(x, W.to(x.dtype)) as the reference evaluates it with bf16 x
    out_f, in_f = shape
    idx, sig, packed, g = _layer(out_f, in_f, 13 * out_f + m)
    x = torch.randn(m, in_f, generator=g).to(torch.bfloat16)
    w16 = torch_ref.materialize(idx, sig, out_f, in_f)
    y = dequant_linear(packed.to(dev), sig.to(dev), out_f, in_f, x.to(dev), weight_rounding="as_x").cpu()
    _check(y, x, w16, mode="as_x")


# one token of bf16 x: rows of 1, 2, 10, 48 (16 lanes), 49 (groups straddle rows), 192 (64 lanes) atoms,
# row counts that leave the last block partly empty, and a row longer than the one-token kernel takes
@pytest.mark.parametrize("shape", [(24, 24), (37, 48), (33, 240), (1152, 1152), (7, 1176), (100, 4608), (130, 24),
                                   (5, 73728)])
@pytest.mark.parametrize("mode", ["exact", "as_x"])
def test_one_token_bf16_ragged(dev, shape, mode):
    out_f, in_f = shape
    idx, sig, packed, g = _layer(out_f, in_f, 17 * out_f + in_f)
    mag = torch.pow(2.0, torch.randint(-40, 41, (1, in_f), generator=g).float())
    x = (torch.randn(1, in_f, generator=g) * mag).to(torch.bfloat16)
    w16 = torch_ref.materialize(idx, sig, out_f, in_f)
    y = dequant_linear(packed.to(dev), sig.to(dev), out_f, in_f, x.to(dev), weight_rounding=mode).cpu()
    _check(y, x, w16, mode=mode)


def test_literal_rounding_is_exact_for_fp32_activations(dev):
    # W.to(fp32) is exact, so both modes agree bit for bit with fp32 x
    out_f, in_f = 64, 1152
    idx, sig, packed, g = _layer(out_f, in_f, 21)
    for m in (3, 40):
        x = torch.randn(m, in_f, generator=g).to(dev)
        a = dequant_linear(packed.to(dev), sig.to(dev), out_f, in_f, x)
        b = dequant_linear(packed.to(dev), sig.to(dev), out_f, in_f, x, weight_rounding="as_x")
        assert torch.equal(a, b)
    with pytest.raises(ValueError):
        dequant_linear(packed.to(dev), sig.to(dev), out_f, in_f, x, weight_rounding="bf16")


def test_fp32_activations_wide_dynamic_range(dev):
    # activations spanning 2^-60..2^60 (and exact zeros): the three-part split keeps every product
    out_f, in_f, m = 96, 1152, 24
    idx, sig, packed, g = _layer(out_f, in_f, 31)
    mag = torch.pow(2.0, torch.randint(-60, 61, (m, in_f), generator=g).float())
    x = torch.randn(m, in_f, generator=g) * mag
    x[:, ::7] = 0.0
    w16 = torch_ref.materialize(idx, sig, out_f, in_f)
    y = dequant_linear(packed.to(dev), sig.to(dev), out_f, in_f, x.to(dev)).cpu()
    _check(y, x, w16)


@pytest.mark.parametrize("m,dtype", [(1, torch.bfloat16), (5, torch.float32), (40, torch.bfloat16), (33, torch.float32)])
def test_multi_target_equals_separate_calls(dev, m, dtype):
    # q/k/v-style targets sharing x (plus one with other rows, a zero-row one, and more than four in all)
    from pollux_amd.packed import dequant_linear_multi

    in_f = 1152
    shapes = [1152, 1152, 1152, 96, 0, 600]
    layers = [_layer(max(o, 1), in_f, 40 + i) for i, o in enumerate(shapes)]
    g = torch.Generator().manual_seed(m)
    x = torch.randn(m, in_f, generator=g).to(dtype).to(dev)
    weights = [(pk.to(dev) if o else pk[:0].to(dev), sig.to(dev) if o else sig[:0].to(dev), o)
               for (idx, sig, pk, _), o in zip(layers, shapes)]
    ys = dequant_linear_multi(weights, in_f, x)
    for (pk, sg, o), y in zip(weights, ys):
        assert y.shape == (m, o)
        if o:
            assert torch.equal(y, dequant_linear(pk, sg, o, in_f, x))


@pytest.mark.parametrize("m", [1, 7, 64])
def test_multi_target_epilogues(dev, m):
    from pollux_amd.packed import dequant_linear_multi

    out_f, in_f = 1920, 1920
    idx, sig, packed, g = _layer(out_f, in_f, 77 + m)
    x = torch.randn(m, in_f, generator=g).to(dev)
    pk, sg = packed.to(dev), sig.to(dev)
    plain = dequant_linear(pk, sg, out_f, in_f, x)
    r = torch.randn(m, out_f, generator=g).to(dev)
    (with_res,) = dequant_linear_multi([(pk, sg, out_f)], in_f, x, residuals=[r])
    assert torch.equal(with_res, r + plain)  # the reference's x + linear(h)
    (act,) = dequant_linear_multi([(pk, sg, out_f)], in_f, x, gelu=True)
    want = torch.nn.functional.gelu(plain)
    ulp = (act.view(torch.int32).long() - want.view(torch.int32).long()).abs().max().item()
    print(f"[dql] gelu epilogue vs F.gelu: max {ulp} ulp", flush=True)
    assert ulp <= 2


def test_multi_target_bad_arguments(dev):
    from pollux_amd.packed import dequant_linear_multi

    idx, sig, packed, g = _layer(48, 48, 5)
    x = torch.randn(2, 48, device=dev)
    with pytest.raises(ValueError):
        dequant_linear_multi([(packed.to(dev), sig.to(dev), 48)] * 17, 48, x)
    with pytest.raises(ValueError):
        dequant_linear_multi([(packed.to(dev)[:-9], sig.to(dev), 48)], 48, x)
    with pytest.raises(ValueError):
        dequant_linear_multi([(packed.to(dev), sig.to(dev), 48)], 48, x, residuals=[torch.zeros(3, device=dev)])


# in-kernel norm of the GEMV path: m = 1, 3 (two token chunks of 2) at 1920 columns; the MFMA
# batch path, where the norm writes the fragment-order copy in one launch (normfrag_kernel): 7,
# 40 and 65 tokens (two slabs) at 1920 columns, 16 tokens at 1944 (81 atoms: the last quad of 4
# atoms is padded with zeros); rows too wide for it (5 x 3072, 20 x 2064: plx_rms_norm into the
# workspace, then the fragment-order copy)
@pytest.mark.parametrize(
    "m,in_f", [(1, 1920), (3, 1920), (7, 1920), (5, 3072), (40, 1920), (65, 1920), (16, 1944), (20, 2064)]
)
def test_multi_target_rms_norm_prologue(dev, m, in_f):
    from pollux_amd.model import rms_norm
    from pollux_amd.packed import dequant_linear_multi

    shapes = [1920, 96]
    layers = [_layer(o, in_f, 300 + i + m) for i, o in enumerate(shapes)]
    g = torch.Generator().manual_seed(m * 7 + in_f)
    x = (torch.randn(m, in_f, generator=g) * 3.0 + 0.5).to(dev)
    nw = (1.0 + 0.1 * torch.randn(in_f, generator=g)).to(dev)
    r = torch.randn(m, shapes[0], generator=g).to(dev)
    weights = [(pk.to(dev), sig.to(dev), o) for (idx, sig, pk, _), o in zip(layers, shapes)]
    ys = dequant_linear_multi(weights, in_f, x, residuals=[r, None], norm=(nw, 1e-8))
    xn = rms_norm(x, nw, 1e-8)
    in_lds = m <= 4 and in_f == 1920  # the GEMV path's norm; the MFMA path's equals plx_rms_norm's bit for bit
    for i, ((pk, sg, o), y) in enumerate(zip(weights, ys)):
        sep = dequant_linear(pk, sg, o, in_f, xn) + (r if i == 0 else 0.0)
        if in_lds:  # the sum of squares is taken in another order than plx_rms_norm's
            rel = ((y - sep).double().norm() / sep.double().norm()).item()
            print(f"[dql] norm prologue m={m} target {i}: rel vs rms_norm + dequant_linear {rel:.2e}", flush=True)
            assert rel <= 1e-6
        else:
            assert torch.equal(y, sep)
    # against the reference's expressions in fp64 (RMSNorm.forward, F.linear on the fp16 weight)
    idx, sig, _, _ = layers[1]
    w16 = torch_ref.materialize(idx, sig, shapes[1], in_f)
    xd = x.double().cpu()
    xn_ref = (xd * torch.rsqrt(xd.pow(2).mean(dim=-1, keepdim=True) + 1e-8) * nw.double().cpu()).float()
    _check(ys[1].cpu(), xn_ref, w16)


def test_rms_norm_flag_and_weight_go_together(dev):
    from pollux_amd import _lib
    from pollux_amd.packed import DQL_RMS_NORM, DQL_X_F32, dequant_linear_multi

    idx, sig, packed, g = _layer(48, 48, 6)
    pk, sg = packed.to(dev), sig.to(dev)
    x = torch.randn(2, 48, device=dev)
    with pytest.raises(ValueError):  # bf16 x
        dequant_linear_multi([(pk, sg, 48)], 48, x.bfloat16(), norm=(torch.ones(48, device=dev), 1e-8))
    with pytest.raises(ValueError):  # weight of the wrong length
        dequant_linear_multi([(pk, sg, 48)], 48, x, norm=(torch.ones(24, device=dev), 1e-8))
    y = torch.zeros(2, 48, device=dev)
    arr = (_lib.DqlTarget * 1)()
    arr[0] = _lib.DqlTarget(pk.data_ptr(), sg.data_ptr(), 48, y.data_ptr(), None)
    lib = _lib.lib()
    w = torch.ones(48, device=dev)
    s = _lib.stream_of(x.device)
    # flag without weight, weight without flag, flag with bf16 x: refused before any launch
    assert lib.plx_dequant_linear_multi(arr, 1, 48, x.data_ptr(), DQL_X_F32 | DQL_RMS_NORM, 2, None, 1e-8, None, 0, s) != 0
    assert lib.plx_dequant_linear_multi(arr, 1, 48, x.data_ptr(), DQL_X_F32, 2, w.data_ptr(), 1e-8, None, 0, s) != 0
    xb = x.bfloat16()
    assert lib.plx_dequant_linear_multi(arr, 1, 48, xb.data_ptr(), DQL_RMS_NORM, 2, w.data_ptr(), 1e-8, None, 0, s) != 0
    torch.cuda.synchronize()
    assert torch.equal(y, torch.zeros(2, 48, device=dev))


@pytest.mark.parametrize("m", [3, 8, 40])
def test_packed_linear_group_stacked_qkv(dev, m):
    # above 4 tokens q / k / v run as one stacked weight (one GEMM launch); at or below, as one GEMV launch
    from pollux_amd.packed import PackedH24Linear, packed_linear_group

    in_f = 1920
    layers = []
    for i in range(3):
        idx, sig, packed, g = _layer(1920, in_f, 500 + i)
        lyr = PackedH24Linear(in_f, 1920).to(dev)
        lyr.packed_weights.copy_(packed.to(dev))
        lyr.sigma_rows.copy_(sig.to(dev))
        layers.append(lyr)
    x = torch.randn(2, (m + 1) // 2, in_f, generator=torch.Generator().manual_seed(m)).to(dev)
    nw = (1.0 + 0.1 * torch.randn(in_f, generator=torch.Generator().manual_seed(m + 1))).to(dev)
    with torch.inference_mode():
        got = packed_linear_group(layers, x, norm=(nw, 1e-8))
        sep = [packed_linear_group([l], x, norm=(nw, 1e-8))[0] for l in layers]
        again = packed_linear_group(layers, x, norm=(nw, 1e-8))
    for a, b, c in zip(got, sep, again):
        assert a.shape == b.shape == (2, (m + 1) // 2, 1920)
        rel = ((a - b).double().norm() / b.double().norm()).item()
        assert rel <= 1e-6, rel
        assert torch.equal(a, c)
    stacked = x.shape[0] * x.shape[1] > 4
    assert ("_stacked" in layers[0].__dict__) == stacked
    if stacked:
        # an in-place update of one layer's weights rebuilds the stacked copy
        idx, sig, packed, _ = _layer(1920, in_f, 777)
        with torch.inference_mode():
            layers[1].packed_weights.copy_(packed.to(dev))
            layers[1].sigma_rows.copy_(sig.to(dev))
            new = packed_linear_group(layers, x, norm=(nw, 1e-8))[1]
            want = packed_linear_group([layers[1]], x, norm=(nw, 1e-8))[0]
        assert ((new - want).double().norm() / want.double().norm()).item() <= 1e-6
