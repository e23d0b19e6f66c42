"""The plane layout (plx_h24_plane_layout) and the dequant-linear kernels that read it.

Layout: every code 0..196,560 (and indices above it, which the packed kernels
read as the origin) is laid out and decoded back through the host plane table
(plx_plane_table); the decoded rows must equal the oracle's raw codebook rows,
and the extra bits the code's type (from its count of non-zero coordinates)
and the position of its -3, both taken from the oracle rows.
Dequant-linear from the layout: the same kernels as from the packed stream
after the decode, so the results must equal the packed path's bit for bit
where both run the same lane layout (rows of more than 80 atoms at one token
may take another, summing in another order), and both must meet the
tolerance of the fused dequant-linear against the oracle (relative L2 <=
1e-5, per element <= 1e-5 * sum_i |x_i W_i|).
"""

import numpy as np
import pytest
import torch

from oracle import codebook as cb
from oracle import packing, torch_ref
from pollux_amd import PackedH24Linear, _lib, dequant_linear, h24_plane_layout
from pollux_amd.packed import DQL_PLANES

pytestmark = pytest.mark.gpu

REL_L2 = 1e-5
ELEM = 1e-5
VALUES = np.array([0, 1, 2, 4, -4, -3, -2, -1], np.int8)


def _plane_table():
    lib = _lib.lib()
    n = int(lib.plx_plane_table(None, 0))
    ids = np.zeros(n, np.uint32)
    assert int(lib.plx_plane_table(ids.ctypes.data, n)) == n
    nib = (ids[:, None] >> (4 * np.arange(8, dtype=np.uint32))[None, :]) & 0xF
    return VALUES[nib[:, [0, 2, 4, 6, 1, 3, 5, 7]]]  # [n, 8] raw values


def test_layout_of_every_code(dev):
    idx = np.concatenate([np.arange(196561), [196561, 200000, 262143, 0, 196560]]).astype(np.int64)
    n = len(idx)
    packed = torch.from_numpy(packing.pack(idx)).to(dev)
    rec = h24_plane_layout(packed, n).cpu().numpy().view(np.uint16).reshape(n, 3).astype(np.int64)
    planes = _plane_table()
    decoded = planes[rec & 0x1FFF].reshape(n, 24)
    raw = cb.codebook_int8()
    want = raw[np.where(idx <= 196560, idx, 0)]
    assert np.array_equal(decoded, want)
    nz = np.count_nonzero(want, axis=1)
    want_type = np.select([nz == 0, nz == 2, nz == 8], [0, 1, 2], 3)
    assert np.array_equal(rec[:, 0] >> 13, want_type)
    assert set(np.unique(nz[want_type == 3])) == {24}
    pos = ((rec[:, 1] >> 13) & 7) | ((rec[:, 2] >> 13) & 3) << 3
    t3 = want_type == 3
    assert np.all(want[t3, pos[t3]] == -3)
    assert np.all(np.count_nonzero(want[t3] == -3, axis=1) == 1)
    assert np.all(pos[~t3] == 0)


def test_layout_argument_checks(dev):
    packed = torch.zeros(18, dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError):
        h24_plane_layout(packed, 9)  # 18 bytes hold 5..8 atoms
    lib = _lib.lib()
    assert lib.plx_h24_plane_layout(None, 0, -1, None, None) == _lib.PLX_EINVAL
    assert lib.plx_h24_plane_layout(None, 18, 9, None, None) == _lib.PLX_EINVAL  # 9 atoms take 27 bytes
    assert b"does not match" in lib.plx_last_error()
    assert h24_plane_layout(torch.zeros(0, dtype=torch.uint8, device=dev), 0).numel() == 0


def _layer(out_f, in_f, seed):
    g = torch.Generator().manual_seed(seed)
    n = out_f * in_f // 24
    idx = torch.randint(0, 196561, (n,), generator=g, dtype=torch.int64)
    sig = (torch.rand(out_f, generator=g) * 0.045 + 0.005).to(torch.float16)
    packed = torch.from_numpy(packing.pack(idx.numpy()))
    return idx, sig, packed, g


def _check(y, x, w16, mode):
    ref = (torch_ref.linear_fp32(x, w16) if mode == "exact" else torch_ref.linear_as_reference(x, w16)).double()
    w = (w16 if mode == "exact" else w16.to(x.dtype)).double()
    err = y.double() - ref
    assert (err.norm() / ref.norm()).item() <= REL_L2
    assert (err.abs() / (ELEM * (x.double().abs() @ w.abs().t()))).max().item() <= 1.0


# one token of bf16 x (the one-token GEMV) and batches above 4 tokens (the MFMA GEMM), ragged shapes and
# both weight roundings; the row of 320 atoms is the longest the one-token kernel takes from the layout;
# rows of 81-85 atoms in layers of more than 6,112 rows take 32 lanes (16 lanes hold at most 80 atoms)
@pytest.mark.parametrize("shape,m,dtype", [
    ((24, 24), 1, torch.bfloat16), ((37, 48), 1, torch.bfloat16), ((33, 240), 1, torch.bfloat16),
    ((1152, 1152), 1, torch.bfloat16), ((7, 1176), 1, torch.bfloat16), ((100, 4608), 1, torch.bfloat16),
    ((130, 7680), 1, torch.bfloat16), ((7680, 1920), 1, torch.bfloat16), ((6200, 2304), 1, torch.bfloat16),
    ((6200, 3816), 1, torch.bfloat16), ((6200, 2304), 1, torch.float32),
    ((6200, 1968), 1, torch.bfloat16), ((6200, 2040), 1, torch.bfloat16),
    ((1152, 1152), 17, torch.bfloat16), ((37, 1920), 33, torch.bfloat16), ((20, 240), 64, torch.bfloat16),
    ((7680, 1920), 64, torch.bfloat16), ((1920, 7680), 64, torch.bfloat16), ((100, 4608), 5, torch.float32),
    ((37, 48), 40, torch.float32), ((1152, 1152), 100, torch.float32),
])
@pytest.mark.parametrize("mode", ["exact", "as_x"])
def test_dequant_linear_from_layout(dev, shape, m, dtype, mode):
    out_f, in_f = shape
    if mode == "as_x" and dtype == torch.float32:
        pytest.skip("the two roundings are the same for fp32 activations")
    idx, sig, packed, g = _layer(out_f, in_f, 29 * out_f + 3 * in_f + m)
    mag = torch.pow(2.0, torch.randint(-30, 31, (1, in_f), generator=g).float())
    x = (torch.randn(m, in_f, generator=g) * mag).to(dtype)
    pk, sg, xd = packed.to(dev), sig.to(dev), x.to(dev)
    planes = h24_plane_layout(pk, out_f * in_f // 24)
    y_pl = dequant_linear(pk, sg, out_f, in_f, xd, weight_rounding=mode, planes=planes).cpu()
    y_pk = dequant_linear(pk, sg, out_f, in_f, xd, weight_rounding=mode).cpu()
    same = torch.equal(y_pl, y_pk)
    print(f"[planes] {shape} m={m} {dtype} {mode}: equal to the packed path: {same}", flush=True)
    w16 = torch_ref.materialize(idx, sig, out_f, in_f)
    _check(y_pl, x, w16, mode)
    if not same:
        # rows that the packed stream runs with another lane layout (e.g. more than 80 atoms at 16 lanes)
        # sum in another order: both must then meet the tolerance
        assert in_f // 24 > 80
        _check(y_pk, x, w16, mode)


def test_layout_refused_where_no_kernel_reads_it(dev):
    # 2..4 tokens, fp32 single tokens and rows above 320 atoms run from the packed stream; the C-ABI refuses
    # the flag there, and dequant_linear passes the layout only where it is read
    out_f, in_f = 40, 7704
    idx, sig, packed, g = _layer(out_f, in_f, 5)
    pk, sg = packed.to(dev), sig.to(dev)
    planes = h24_plane_layout(pk, out_f * in_f // 24)
    w16 = torch_ref.materialize(idx, sig, out_f, in_f)
    for m, dtype in ((1, torch.bfloat16), (3, torch.bfloat16), (1, torch.float32), (4, torch.float32)):
        x = torch.randn(m, in_f, generator=g).to(dtype)
        y = dequant_linear(pk, sg, out_f, in_f, x.to(dev), planes=planes).cpu()
        _check(y, x, w16, "exact")
    lib = _lib.lib()
    x = torch.randn(3, 48, generator=g).to(torch.bfloat16).to(dev)
    y = torch.empty(3, 40, device=dev)
    st = lib.plx_dequant_linear(_lib.ptr(planes), 6 * 80, _lib.ptr(sg), 40, 48, _lib.ptr(x), DQL_PLANES, 3,
                                _lib.ptr(y), None, 0, _lib.stream_of(dev))
    assert st == _lib.PLX_EINVAL
    with pytest.raises(ValueError):  # a layout of the wrong size
        dequant_linear(pk, sg, out_f, in_f, torch.randn(8, in_f, device=dev), planes=planes[:-3])


def test_packed_layer_keeps_its_layout_current(dev):
    out_f, in_f = 64, 1152
    idx, sig, packed, g = _layer(out_f, in_f, 31)
    layer = PackedH24Linear(in_f, out_f, bias=False)
    layer.load_state_dict({"packed_weights": packed, "sigma_rows": sig})
    layer = layer.to(dev)
    x = torch.randn(1, in_f, generator=g).to(torch.bfloat16)
    xb = torch.randn(9, in_f, generator=g).to(torch.bfloat16)
    for xx in (x, xb):
        y = layer(xx.to(dev)).float().cpu()
        ref = torch_ref.linear_fp32(xx, torch_ref.materialize(idx, sig, out_f, in_f)).to(torch.bfloat16).float()
        assert ((y - ref).norm() / ref.norm()).item() <= 1e-2  # bf16 output
    first = layer.plane_layout()
    assert layer.plane_layout() is first
    # a second state copied in place: the layout is rebuilt and the output follows
    idx2, sig2, packed2, _ = _layer(out_f, in_f, 32)
    layer.load_state_dict({"packed_weights": packed2, "sigma_rows": sig2})
    assert layer.plane_layout() is not first
    y2 = layer(xb.to(dev)).float().cpu()
    ref2 = torch_ref.linear_fp32(xb, torch_ref.materialize(idx2, sig2, out_f, in_f)).to(torch.bfloat16).float()
    assert ((y2 - ref2).norm() / ref2.norm()).item() <= 1e-2
    layer.use_plane_layout = False  # packed stream only: the same results
    assert torch.equal(layer(xb.to(dev)).float().cpu(), y2)


def test_graph_captured_before_any_eager_call(dev):
    # Derived buffers (plane layout, stacked q/k/v copy) built under capture hold nothing until a replay:
    # none is kept for eager calls, and the captured graph still computes the right result.
    from pollux_amd.packed import packed_linear_group

    with torch.cuda.device(dev):
        _lib.check(_lib.lib().plx_device_init(), "init")
    out_f, in_f = 96, 1152
    layers, w16s = [], []
    for i in range(3):
        idx, sig, packed, g = _layer(out_f, in_f, 40 + i)
        lyr = PackedH24Linear(in_f, out_f)
        lyr.load_state_dict({"packed_weights": packed, "sigma_rows": sig})
        layers.append(lyr.to(dev))
        w16s.append(torch_ref.materialize(idx, sig, out_f, in_f))
    xb = torch.randn(9, in_f, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    refs = [torch_ref.linear_fp32(xb, w).to(torch.bfloat16).float() for w in w16s]
    xd = xb.to(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_single = layers[0](xd)
        y_group = packed_linear_group(layers, xd.float())
    assert "_planes" not in layers[0].__dict__ and "_stacked" not in layers[0].__dict__

    def close(a, b):
        return ((a.float().cpu() - b).norm() / b.norm()).item() <= 1e-2  # bf16 rounding of the outputs

    assert close(layers[0](xd), refs[0])  # eager: builds the layout now
    eager_group = packed_linear_group(layers, xd.float())
    assert all(close(a, r) for a, r in zip(eager_group, refs))
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert close(y_single, refs[0])
        assert all(close(a, r) for a, r in zip(y_group, refs))
        assert close(layers[1](xd), refs[1])  # eager work between the replays


# one token through the multi-target kernel (q/k/v-style groups, the norm prologue, GELU and residual
# epilogues, fp32 and bf16 x) from the plane layouts: the same results as from the packed streams, bit
# for bit; rows of 2, 7, 48, 80 and 320 atoms (8, 16, 32 and 64 lanes per row), ragged row counts
@pytest.mark.parametrize("shapes,in_f", [([(96, 1152)] * 3, 1152), ([(37, 48), (5, 48)], 48), ([(130, 168)], 168),
                                         ([(1920, 1920)] * 3, 1920), ([(7680, 1920)], 1920), ([(1920, 7680)], 7680),
                                         ([(6200, 2304)], 2304), ([(3200, 3816)] * 2, 3816)])
@pytest.mark.parametrize("variant", ["fp32_norm", "fp32_gelu", "fp32_residual", "bf16_plain", "bf16_as_x"])
def test_multi_target_one_token_from_layout(dev, shapes, in_f, variant):
    from pollux_amd.packed import dequant_linear_multi

    g = torch.Generator().manual_seed(len(shapes) * 1000 + in_f)
    weights, planes, w16s = [], [], []
    for k, (out_f, _) in enumerate(shapes):
        idx, sig, packed, _ = _layer(out_f, in_f, 7 * k + in_f)
        pk, sg = packed.to(dev), sig.to(dev)
        weights.append((pk, sg, out_f))
        planes.append(h24_plane_layout(pk, out_f * in_f // 24))
        w16s.append(torch_ref.materialize(idx, sig, out_f, in_f))
    dtype = torch.bfloat16 if variant.startswith("bf16") else torch.float32
    x = (torch.randn(1, in_f, generator=g) * 2.0).to(dtype).to(dev)
    kw = {}
    if variant == "fp32_norm":
        kw["norm"] = ((1.0 + 0.1 * torch.randn(in_f, generator=g)).to(dev), 1e-5)
    elif variant == "fp32_gelu":
        kw["gelu"] = True
    elif variant == "fp32_residual":
        kw["residuals"] = [torch.randn(1, o, generator=g).to(dev) for o, _ in shapes]
    elif variant == "bf16_as_x":
        kw["weight_rounding"] = "as_x"
    y_pl = dequant_linear_multi(weights, in_f, x, planes=planes, **kw)
    y_pk = dequant_linear_multi(weights, in_f, x, **kw)
    same = all(torch.equal(a, b) for a, b in zip(y_pl, y_pk))
    print(f"[planes multi] {shapes[0]} x{len(shapes)} {variant}: equal to the packed path: {same}", flush=True)
    if not same:
        # another lane layout for these rows (more than 80 atoms at 16 lanes): another summation order, so
        # the two results differ by at most twice the per-element bound (GELU's slope is below 1.13)
        assert in_f // 24 > 80
        xn = x.float().cpu()
        if "norm" in kw:
            nw = kw["norm"][0].cpu()
            xn = xn * torch.rsqrt(xn.pow(2).mean(-1, keepdim=True) + kw["norm"][1]) * nw
        for a, b, w16 in zip(y_pl, y_pk, w16s):
            bound = 2.3 * ELEM * (xn.double().abs() @ w16.double().abs().t())
            assert ((a.cpu().double() - b.cpu().double()).abs() <= bound).all()
    if variant in ("bf16_plain", "bf16_as_x"):
        for y, w16 in zip(y_pl, w16s):
            _check(y.cpu(), x.cpu(), w16, "exact" if variant == "bf16_plain" else "as_x")


def test_multi_target_layout_refused_for_long_rows(dev):
    # rows of more than 320 atoms at one token read the packed stream: the C-ABI refuses the flag
    out_f, in_f = 8, 7704
    idx, sig, packed, g = _layer(out_f, in_f, 9)
    pk, sg = packed.to(dev), sig.to(dev)
    planes = h24_plane_layout(pk, out_f * in_f // 24)
    x = torch.randn(1, in_f, generator=g).to(dev)
    y = torch.empty(1, out_f, device=dev)
    arr = (_lib.DqlTarget * 1)()
    arr[0] = _lib.DqlTarget(planes.data_ptr(), sg.data_ptr(), out_f, y.data_ptr(), None)
    st = _lib.lib().plx_dequant_linear_multi(arr, 1, in_f, x.data_ptr(), 1 | DQL_PLANES, 1, None, 0.0, None, 0,
                                             _lib.stream_of(dev))
    assert st == _lib.PLX_EINVAL
    from pollux_amd.packed import dequant_linear_multi
    (y2,) = dequant_linear_multi([(pk, sg, out_f)], in_f, x, planes=[planes])  # falls back to the packed stream
    assert ((y2.cpu().double() - torch_ref.linear_fp32(x.cpu(), torch_ref.materialize(idx, sig, out_f, in_f)).double())
            .norm() / y2.cpu().double().norm()).item() <= REL_L2


def test_any_layout_content_stays_inside_the_tables(dev):
    # the kernels clamp plane indices to their staged table and the position bits stay inside the staged
    # x, so a buffer of arbitrary records (not made by h24_plane_layout) gives finite output, no error
    out_f, in_f = 96, 1920
    idx, sig, packed, g = _layer(out_f, in_f, 50)
    pk, sg = packed.to(dev), sig.to(dev)
    junk = torch.randint(-32768, 32768, (3 * out_f * in_f // 24,), generator=g, dtype=torch.int32)
    junk = junk.to(torch.int16).to(dev)
    for m, dtype in ((1, torch.bfloat16), (1, torch.float32), (8, torch.bfloat16), (8, torch.float32)):
        x = torch.randn(m, in_f, generator=g).to(dtype).to(dev)
        y = dequant_linear(pk, sg, out_f, in_f, x, planes=junk)
        torch.cuda.synchronize()
        assert torch.isfinite(y).all()
    from pollux_amd.packed import dequant_linear_multi
    x = torch.randn(1, in_f, generator=g).to(dev)
    ys = dequant_linear_multi([(pk, sg, out_f)] * 2, in_f, x, planes=[junk, junk], gelu=True)
    torch.cuda.synchronize()
    assert all(torch.isfinite(y).all() for y in ys)
