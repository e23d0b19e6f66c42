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


def _ref_int8_materialize(q, mu16):
    # pollux.py:526
    return q.to(torch.float16) * (mu16.unsqueeze(-1).to(torch.float16) / 127.0)


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
    want = _ref_int8_materialize(q, mu)
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
    wq = _ref_int8_materialize(q, mu)
    assert torch.equal(emb(ids), torch.nn.functional.embedding(ids, wq.float()))
    assert torch.equal(lin(x), torch.nn.functional.linear(x, wq.float()))


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
