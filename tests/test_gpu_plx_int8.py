"""INT8 periphery kernels and the end-to-end .plx path on the GPU.

INT8 (pack.py:124-136, pollux.py:508-563): bit-exact against the reference's
own torch expressions evaluated on the same device.  End to end: a synthetic
Pollux-shaped state dict is packed on the GPU (pack_state_dict), written as
.plx, memory-mapped back onto the device and loaded into PackedH24Linear /
PackedInt8* layers, whose outputs match the oracle's materialisation.
"""

import numpy as np
import pytest
import torch

from oracle import nn, packing, torch_ref
from pollux_amd import pack as plx_pack
from pollux_amd import plx
from pollux_amd.packed import PackedH24Linear, PackedInt8Embedding, PackedInt8Linear, dequantize_int8_rows

pytestmark = pytest.mark.gpu


def _ref_int8(w):
    # pack.py:131-135, verbatim semantics, on w's device
    w = w.detach().float()
    mu = w.abs().amax(dim=-1, keepdim=True).clamp_min(1e-8)
    q = torch.round(w / mu * 127.0).clamp(-128, 127).to(torch.int8)
    return q, mu.squeeze(-1).to(torch.float16)


@pytest.mark.parametrize("shape", [(50, 1152), (7, 1000), (3, 5, 24), (1, 1), (64,)])
def test_quantize_int8_matches_reference_ops(dev, shape):
    g = torch.Generator().manual_seed(sum(shape))
    w = torch.randn(*shape, generator=g) * 0.05
    if len(shape) == 2 and shape[0] > 3:
        w[2] = 0.0  # all-zero row: mu clamps to 1e-8
    q, mu = plx_pack.quantize_int8_rows(w.to(dev))
    rq, rmu = _ref_int8(w.to(dev))
    assert q.dtype == torch.int8 and mu.dtype == torch.float16 and q.shape == w.shape and mu.shape == rmu.shape
    assert torch.equal(q, rq) and torch.equal(mu.view(torch.int16), rmu.view(torch.int16))
    cq, cmu = _ref_int8(w)  # the CPU evaluation of the same expression agrees too
    assert torch.equal(q.cpu(), cq) and torch.equal(mu.cpu(), cmu)


@pytest.mark.parametrize("shape", [(50, 1152), (7, 1001)])
def test_dequant_int8_matches_reference_ops(dev, shape):
    g = torch.Generator().manual_seed(7)
    q = torch.randint(-128, 128, shape, dtype=torch.int8, generator=g).to(dev)
    mu = (torch.rand(shape[0], generator=g) * 0.2 + 1e-3).to(torch.float16).to(dev)
    got = dequantize_int8_rows(q, mu)
    want = torch_ref.int8_materialize(q, mu)  # the reference's expression on the device
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert torch.equal(got.cpu().view(torch.int16), torch_ref.int8_materialize(q.cpu(), mu.cpu()).view(torch.int16))


def test_dequant_int8_every_fp16_scale(dev):
    # all 63,488 finite fp16 mu x all 256 int8 values against the oracle's CPU evaluation (itself pinned
    # exhaustively against numpy's float16 emulation in tests/test_oracle_forward.py)
    mu = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.float16)
    mu = mu[torch.isfinite(mu)]
    q = torch.arange(-128, 128, dtype=torch.int16).to(torch.int8).repeat(mu.numel(), 1)
    got = dequantize_int8_rows(q.to(dev), mu.to(dev)).cpu()
    want = torch_ref.int8_materialize(q, mu)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_packed_int8_layers(dev):
    g = torch.Generator().manual_seed(8)
    emb = PackedInt8Embedding(100, 48).to(dev)
    lin = PackedInt8Linear(48, 100).to(dev)
    w = torch.randn(100, 48, generator=g).to(dev)
    q, mu = plx_pack.quantize_int8_rows(w)
    for m in (emb, lin):
        m.weight_int8.copy_(q)
        m.mu_rows.copy_(mu)
    ids = torch.randint(0, 100, (3, 5), generator=g).to(dev)
    x = torch.randn(4, 48, generator=g).to(dev)
    wq = torch_ref.int8_materialize(q, mu)
    assert torch.equal(emb(ids), torch.nn.functional.embedding(ids, wq.float()))
    # fused INT8 kernels (4 tokens, 20 tokens: MFMA): exact products, another summation order than F.linear
    want = torch.nn.functional.linear(x, wq.float())
    _check_int8_linear(lin(x), x, wq)
    big = torch.randn(20, 48, generator=g).to(dev)
    _check_int8_linear(lin(big), big, wq)
    lin.gemv_max_tokens = 16  # beyond the kernels' token limit: the reference's F.linear
    assert torch.equal(lin(big), torch.nn.functional.linear(big, wq.float()))
    for m in (emb, lin):
        m.materialize()
    assert torch.equal(emb(ids), torch.nn.functional.embedding(ids, wq.float()))
    assert torch.equal(lin(x), want)


def test_packed_int8_linear_sees_new_weights(dev):
    # the cached cast of the head weight (token batches above the GEMV limit) is
    # rebuilt after load_state_dict copies new values into the buffers in place
    g = torch.Generator().manual_seed(81)
    lin = PackedInt8Linear(48, 100).to(dev)
    lin.gemv_max_tokens = 16  # 20 tokens take the F.linear path and its cached cast
    states = []
    for _ in range(2):
        q, mu = plx_pack.quantize_int8_rows(torch.randn(100, 48, generator=g).to(dev))
        states.append({"weight_int8": q, "mu_rows": mu})
    big = torch.randn(20, 48, generator=g).to(dev)
    for st in states + states[:1]:
        lin.load_state_dict(st)
        want = torch.nn.functional.linear(big, torch_ref.int8_materialize(st["weight_int8"], st["mu_rows"]).float())
        assert torch.equal(lin(big), want)
        assert torch.equal(lin(big.to(torch.bfloat16)),
                           torch.nn.functional.linear(big.to(torch.bfloat16),
                                                      torch_ref.int8_materialize(st["weight_int8"], st["mu_rows"])
                                                      .to(torch.bfloat16)))
    # replacing a buffer object is seen too
    lin.weight_int8 = states[1]["weight_int8"].clone()
    lin.mu_rows = states[1]["mu_rows"].clone()
    want = torch.nn.functional.linear(big, torch_ref.int8_materialize(states[1]["weight_int8"],
                                                                 states[1]["mu_rows"]).float())
    assert torch.equal(lin(big), want)


def test_packed_int8_linear_cast_not_kept_from_graph_capture(dev):
    # a cast made under graph capture is filled only on replay: it is not kept for eager calls
    g = torch.Generator().manual_seed(82)
    lin = PackedInt8Linear(48, 100).to(dev)
    lin.gemv_max_tokens = 16
    q, mu = plx_pack.quantize_int8_rows(torch.randn(100, 48, generator=g).to(dev))
    lin.load_state_dict({"weight_int8": q, "mu_rows": mu})
    big = torch.randn(20, 48, generator=g).to(dev)
    want = torch.nn.functional.linear(big, torch_ref.int8_materialize(q, mu).float())
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = lin(big)
    assert torch.float32 not in lin.__dict__.get("_cast", {})
    assert torch.equal(lin(big), want)
    for _ in range(2):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want)


def _check_int8_linear(y, x, w16, bound=1e-5):
    """y against fp64 x @ w16.T: |err| <= bound * sum |x||w| per element (fp32 accumulation)."""
    xd, wd = x.double().cpu(), w16.double().cpu()
    ref = xd @ wd.t()
    scale = xd.abs() @ wd.abs().t()
    err = (y.double().cpu() - ref).abs()
    worst = (err / scale.clamp_min(1e-300)).max().item()
    print(f"[int8] linear {tuple(y.shape)}: worst err / sum|x||w| {worst:.2e}", flush=True)
    assert worst <= bound


# rows % 4 != 0, 16 columns (one chunk), 1,040 columns (a second chunk on one lane only; K steps past the
# row), 1,920 (the Pollux head), 4,096 (four chunks per lane); one token (the GEMV), 2..16 tokens (MFMA, one
# token tile), 17..32 (two), 33 and more (four per 64-token slab; 65 and 100: a second, partial slab)
@pytest.mark.parametrize("rows,cols,m", [(4103, 1920, 1), (4103, 1920, 2), (4103, 1920, 7), (513, 16, 3),
                                         (999, 1040, 5), (257, 4096, 4), (130, 4096, 16), (61, 48, 1),
                                         (4103, 1920, 17), (1000, 1920, 33), (2049, 1920, 65), (77, 1040, 100)])
def test_int8_linear_matches_fp64(dev, rows, cols, m):
    from pollux_amd.packed import int8_linear

    g = torch.Generator().manual_seed(rows + cols + m)
    q = torch.randint(-128, 128, (rows, cols), dtype=torch.int8, generator=g)
    q[0, :] = -128  # the int8 range's end
    mu = (torch.rand(rows, generator=g) * 0.2 + 1e-3).to(torch.float16)
    mu[1] = 1.3e-4  # s16 ~ 1e-6 is an fp16 subnormal; the row's weights round on both sides of 2^-14
    x = (torch.randn(m, cols, generator=g) * 2.0).to(dev)
    qd, mud = q.to(dev), mu.to(dev)
    wq = torch_ref.int8_materialize(qd, mud)
    y = int8_linear(qd, mud, x)
    assert y.shape == (m, rows)
    _check_int8_linear(y, x, wq)
    assert torch.isfinite(y).all() and (wq[1] != 0).any() and (wq[1].abs() < 2.0 ** -14).any()
    nw = (1.0 + 0.1 * torch.randn(cols, generator=g)).to(dev)
    yn = int8_linear(qd, mud, x, norm=(nw, 1e-8))
    xd = x.double()
    xn = (xd * torch.rsqrt(xd.pow(2).mean(dim=-1, keepdim=True) + 1e-8) * nw.double()).float()
    _check_int8_linear(yn, xn, wq, bound=2e-5)  # + the norm's rounding (a few ulp of x)


# the head's shape at 1, 3 and 16 tokens (a pick block of 16, 4 and 1 waves per token), 20 tokens (two
# rounds of 16), few rows (one GEMV block), rows % 4 != 0
@pytest.mark.parametrize("rows,cols,m", [(50688, 1920, 1), (50688, 1920, 3), (50688, 1920, 16), (4103, 1920, 20),
                                         (5, 48, 2), (999, 1040, 5)])
def test_int8_linear_argmax_matches_torch(dev, rows, cols, m):
    """ids == torch.argmax(y, -1) of the same y (equal to int8_linear's), with ties, NaN rows, history and pos."""
    from pollux_amd.packed import int8_linear, int8_linear_argmax, int8_linear_argmax_workspace

    g = torch.Generator().manual_seed(rows + 7 * m)
    q = torch.randint(-128, 128, (rows, cols), dtype=torch.int8, generator=g)
    mu = (torch.rand(rows, generator=g) * 0.2 + 1e-3).to(torch.float16)
    xc = torch.randn(m, cols, generator=g)
    x = xc.to(dev)
    nw = (1.0 + 0.1 * torch.randn(cols, generator=g)).abs().to(dev)
    if rows > 8:
        # token 0's maximum three times (rows matched to its signs), at a lower row and two higher ones
        q[rows // 2] = q[rows - 2] = q[3] = (torch.sign(xc[0]) * 127).to(torch.int8)
        mu[rows // 2] = mu[rows - 2] = mu[3] = 0.5
    qd, mud = q.to(dev), mu.to(dev)
    hist = torch.full((m, 9), -1, dtype=torch.long, device=dev)
    pos = torch.tensor(4, dtype=torch.long, device=dev)
    ids = torch.empty(m, dtype=torch.long, device=dev)
    ws = int8_linear_argmax_workspace(rows, m, dev)
    y = int8_linear_argmax(qd, mud, x, ids, norm=(nw, 1e-5), history=hist, pos=pos, workspace=ws)
    assert torch.equal(y, int8_linear(qd, mud, x, norm=(nw, 1e-5)))
    want = torch.argmax(y, dim=-1)
    print(f"[int8] linear_argmax {rows}x{cols} m={m}: ids {ids[:4].tolist()}", flush=True)
    assert torch.equal(ids, want)
    if rows > 8:
        assert y[0, 3] == y[0, rows // 2] == y[0, rows - 2] == y[0].max() and int(ids[0]) == 3
    assert int(pos) == 5 and torch.equal(hist[:, 5], ids)
    assert (hist[:, :5] == -1).all() and (hist[:, 6:] == -1).all()
    # a NaN row beats every number (the lower of two NaN rows wins); a position past the history writes nothing
    if rows > 8:
        mu[rows - 1] = mu[rows // 3] = float("nan")
        mud = mu.to(dev)
        pos.fill_(8)
        y = int8_linear_argmax(qd, mud, x, ids, history=hist, pos=pos)  # workspace allocated per call
        assert torch.isnan(y[:, rows // 3]).all()
        assert torch.equal(ids, torch.full_like(ids, rows // 3)) and torch.equal(ids, torch.argmax(y, dim=-1))
        assert int(pos) == 9 and (hist[:, 6:] == -1).all()
    # no position: ids only; a workspace too small is refused
    y = int8_linear_argmax(qd, mud, x[:1], ids[:1], workspace=ws)
    assert torch.equal(ids[:1], torch.argmax(y, dim=-1))
    with pytest.raises(Exception, match="workspace"):
        int8_linear_argmax(qd, mud, x, ids, workspace=ws[:8])


def test_int8_embed_with_positions(dev):
    from pollux_amd.packed import int8_embed

    g = torch.Generator().manual_seed(21)
    q = torch.randint(-128, 128, (300, 72), dtype=torch.int8, generator=g).to(dev)
    mu = (torch.rand(300, generator=g) * 0.2 + 1e-3).to(torch.float16).to(dev)
    pos_w = torch.randn(40, 72, generator=g).to(dev)
    ids = torch.randint(0, 300, (3, 7), generator=g).to(dev)
    wq = torch_ref.int8_materialize(q, mu).float()
    p0 = torch.tensor(5, device=dev)
    got = int8_embed(q, mu, ids, pos_weight=pos_w, pos0=p0)
    want = torch.nn.functional.embedding(ids, wq) + pos_w[5:12].unsqueeze(0)
    assert torch.equal(got, want)
    assert torch.equal(int8_embed(q, mu, ids), torch.nn.functional.embedding(ids, wq))
    # an id out of range, then positions past the table: NaN rows, nothing else touched
    bad = ids.clone()
    bad[1, 2] = 300
    out = int8_embed(q, mu, bad, pos_weight=pos_w, pos0=p0)
    assert torch.isnan(out[1, 2]).all() and torch.equal(out[0], want[0])
    out = int8_embed(q, mu, ids, pos_weight=pos_w, pos0=torch.tensor(36, device=dev))
    assert torch.isnan(out[:, 4:]).all() and torch.isfinite(out[:, :4]).all()


def _state(g, d=96, hidden=384, vocab=200):
    s = {
        "tok_emb.weight": torch.randn(vocab, d, generator=g) * 0.02,
        "pos_emb.weight": torch.randn(16, d, generator=g) * 0.02,
        "blocks.0.ln_1.weight": torch.ones(d),
        "blocks.0.attn.q.weight": torch.randn(d, d, generator=g) * 0.02,
        "blocks.0.mlp.fc.weight": torch.randn(hidden, d, generator=g) * 0.02,
        "blocks.0.mlp.proj.weight": torch.randn(d, hidden, generator=g) * 0.02,
        "head.weight": torch.randn(vocab, d, generator=g) * 0.02,
    }
    s["blocks.0.attn.q.weight"][5] = 0.0  # a zero row: all-origin atoms, sigma 1e-8
    return s


def test_pack_write_load_forward(dev, tmp_path):
    g = torch.Generator().manual_seed(9)
    state = _state(g)
    out, stats = plx_pack.pack_state_dict(state, dev)
    assert list(out) == [
        "tok_emb.weight_int8", "tok_emb.mu_rows", "pos_emb.weight", "blocks.0.ln_1.weight",
        "blocks.0.attn.q.packed_weights", "blocks.0.attn.q.sigma_rows",
        "blocks.0.mlp.fc.packed_weights", "blocks.0.mlp.fc.sigma_rows",
        "blocks.0.mlp.proj.packed_weights", "blocks.0.mlp.proj.sigma_rows",
        "head.weight_int8", "head.mu_rows",
    ]
    assert stats["h24_atom_count"] == (96 * 96 + 2 * 384 * 96) // 24
    cfg = plx_pack.pack_config({"n_embd": 96})
    assert cfg["bits_per_param"] == 0.76 and cfg["scale_serialization"] == "row_wise"
    path = tmp_path / "tiny.plx"
    plx.write_plx(path, cfg, out)
    payload = plx.load_plx(path, dev)
    sd = payload["state_dict"]
    assert all(t.device.type == "cuda" for t in sd.values())
    for name in ("blocks.0.attn.q", "blocks.0.mlp.fc", "blocks.0.mlp.proj"):
        w = state[name + ".weight"]
        rows, cols = w.shape
        # indices: the oracle's NN-P on every non-near-tie atom; scales within 1 fp16 ulp
        idx = packing.unpack(sd[name + ".packed_weights"].cpu().numpy(), w.numel() // 24)
        r = nn.quantize(w.reshape(-1, 24).numpy(), "P")
        ok = ~r["near_tie"]
        assert np.array_equal(idx[ok], r["idx"][ok]), name
        ds = (sd[name + ".sigma_rows"].cpu().view(torch.int16).long()
              - torch_ref.sigma16_pack(w).view(torch.int16).long()).abs()
        assert ds.max() <= 1, name
        layer = PackedH24Linear(cols, rows).to(dev)
        layer.load_state_dict({"packed_weights": sd[name + ".packed_weights"],
                               "sigma_rows": sd[name + ".sigma_rows"]})
        x = torch.randn(3, cols, generator=g)
        w16 = torch_ref.materialize(torch.from_numpy(idx), sd[name + ".sigma_rows"].cpu(), rows, cols)
        want = x.double() @ w16.double().T
        y_fused = layer(x.to(dev)).cpu().double()
        assert torch.linalg.norm(y_fused - want) <= 1e-5 * torch.linalg.norm(want), name
        layer.materialize()
        assert torch.equal(layer.weight.detach().cpu().view(torch.int16), w16.view(torch.int16)), name
    q, mu = _ref_int8(state["head.weight"].to(dev))
    assert torch.equal(sd["head.weight_int8"], q) and torch.equal(sd["head.mu_rows"], mu)
