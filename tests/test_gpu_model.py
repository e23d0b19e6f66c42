"""Packed Pollux decoder (pollux_amd.model) on the GPU.

Bars (stated):
* full-prefix logits of the packed model (fused dequant-linear kernels) against
  the reference's forward composed on the CPU from the materialised weights
  (oracle.torch_ref.pollux_packed_forward): relative L2 <= 1e-4 (fp32 on both
  sides, different summation orders), and <= 1e-5 against the same model with
  materialised fp16 weights on the GPU;
* KV-cached decode against the full-prefix forward of the same prefix:
  relative L2 <= 1e-5 per position;
* token-level generation with and without the cache, greedy and with a
  caller's seeded sampling step, past seq_len (where the reference's sliding
  window restarts the positions): identical token ids.
"""

import pytest
import torch

from oracle import torch_ref
from pollux_amd import pack, plx
from pollux_amd.model import PackedPolluxModel, PolluxConfig, generate

pytestmark = pytest.mark.gpu

CFG = {"n_layers": 2, "n_heads": 2, "d_head": 24, "n_embd": 48, "vocab_size": 96, "tokenizer_vocab_size": 90,
       "seq_len": 16}


def _dense_state(cfg, seed):
    """A full-precision training state dict with the reference's key names (pollux.py:566-702)."""
    g = torch.Generator().manual_seed(seed)
    d, v, s, n = cfg["n_embd"], cfg["vocab_size"], cfg["seq_len"], cfg["n_layers"]

    def w(*shape, scale=0.3):
        return torch.randn(*shape, generator=g) * scale

    st = {"tok_emb.weight": w(v, d, scale=1.0), "pos_emb.weight": w(s, d, scale=0.5)}
    for i in range(n):
        p = f"blocks.{i}."
        st[p + "ln1.weight"] = 1.0 + w(d, scale=0.1)
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            st[p + f"attn.{name}.weight"] = w(d, d)
        st[p + "attn.q_ln.weight"] = 1.0 + w(24, scale=0.1)
        st[p + "attn.k_ln.weight"] = 1.0 + w(24, scale=0.1)
        st[p + "ln2.weight"] = 1.0 + w(d, scale=0.1)
        st[p + "mlp.fc1.weight"] = w(4 * d, d)
        st[p + "mlp.fc2.weight"] = w(d, 4 * d)
    st["ln_f.weight"] = 1.0 + w(d, scale=0.1)
    st["head.weight"] = w(v, d)
    return st


@pytest.fixture(scope="module")
def packed(dev, tmp_path_factory):
    state, _ = pack.pack_state_dict(_dense_state(CFG, 5), dev)
    path = tmp_path_factory.mktemp("plx") / "tiny.plx"
    plx.write_plx(path, pack.pack_config(CFG), state)
    return path, state


def _rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


def test_forward_matches_reference_composition(dev, packed):
    path, state = packed
    model = PackedPolluxModel.from_packed_checkpoint(str(path), dev)
    dense = PackedPolluxModel.from_packed_checkpoint(str(path), dev, materialize=True)
    idx = torch.randint(0, 90, (2, 12), generator=torch.Generator().manual_seed(1))
    with torch.inference_mode():
        y = model(idx.to(dev)).cpu()
        y_dense = dense(idx.to(dev)).cpu()
    ref = torch_ref.pollux_packed_forward(state, CFG, idx)
    e_ref, e_dense = _rel(y, ref), _rel(y, y_dense)
    print(f"[model] rel vs CPU composition {e_ref:.2e}, vs materialised {e_dense:.2e}", flush=True)
    assert y.shape == (2, 12, 96)
    assert e_ref <= 1e-4 and e_dense <= 1e-5


def test_kv_cache_decode_matches_full_forward(dev, packed):
    model = PackedPolluxModel.from_packed_checkpoint(str(packed[0]), dev)
    idx = torch.randint(0, 90, (1, 14), generator=torch.Generator().manual_seed(2)).to(dev)
    with torch.inference_mode():
        cache = model.new_cache(1)
        pre = model.prefill(idx[:, :5], cache)
        assert _rel(pre, model(idx[:, :5])) <= 1e-5
        worst = 0.0
        for s in range(5, 14):
            step = model.decode(idx[:, s], cache)
            full = model(idx[:, :s + 1])[:, -1]
            worst = max(worst, _rel(step, full))
        assert cache.length == 14
    print(f"[model] decode vs full forward, worst rel {worst:.2e}", flush=True)
    assert worst <= 1e-5


def test_chunked_prefill_and_batch(dev, packed):
    model = PackedPolluxModel.from_packed_checkpoint(str(packed[0]), dev)
    idx = torch.randint(0, 90, (2, 9), generator=torch.Generator().manual_seed(3)).to(dev)
    with torch.inference_mode():
        cache = model.new_cache(2)
        model.prefill(idx[:, :4], cache)
        more = model.prefill(idx[:, 4:9], cache)  # 5 queries at positions 4..8 over a filled cache
        full = model(idx)
        assert _rel(more, full[:, 4:9]) <= 1e-5
        # each sequence of the batch decodes as it does alone
        nxt = torch.tensor([7, 11], device=dev)
        both = model.decode(nxt, cache)
        for b in range(2):
            c1 = model.new_cache(1)
            model.prefill(idx[b:b + 1], c1)
            assert _rel(both[b:b + 1], model.decode(nxt[b:b + 1], c1)) <= 1e-5


def _seeded_sampler(generator, temperature):
    """A caller's sampling step: softmax at a temperature and one multinomial draw."""
    def sample(logits, ids):
        probs = torch.softmax(logits / temperature, dim=-1)
        return int(torch.multinomial(probs, 1, generator=generator).item())
    return sample


@pytest.mark.parametrize("sampled", [False, True])
def test_generate_with_and_without_cache(dev, packed, sampled):
    model = PackedPolluxModel.from_packed_checkpoint(str(packed[0]), dev)
    prompt = [3, 14, 15, 9, 26]
    runs = []
    for use_cache, use_graph in ((True, False), (False, False), (True, True)):
        g = torch.Generator(device=dev).manual_seed(7)
        sample = _seeded_sampler(g, 0.9) if sampled else None
        runs.append(generate(model, prompt, max_new_tokens=20, sample=sample, eos_id=95, use_cache=use_cache,
                             use_graph=use_graph))
    print(f"[model] generated {runs[0]}", flush=True)
    assert runs[0] == runs[1] == runs[2]
    assert runs[0][:5] == prompt and len(runs[0]) > 16  # went past seq_len unless eos came first
    with pytest.raises(ValueError):
        generate(model, [96], max_new_tokens=1)
    with pytest.raises(ValueError):
        generate(model, prompt, max_new_tokens=1, sample=lambda logits, ids: 96)


def test_config_from_plx_payload(dev, packed):
    payload = plx.read_plx(packed[0])
    cfg = PolluxConfig.from_dict(payload["config"])
    assert (cfg.n_layers, cfg.n_embd, cfg.vocab_size, cfg.seq_len) == (2, 48, 96, 16)
    model = PackedPolluxModel.from_packed_checkpoint(payload, dev)  # an already loaded payload works too
    idx = torch.tensor([[1, 2, 3]], device=dev)
    with torch.inference_mode():
        a = model(idx)
        b = PackedPolluxModel.from_packed_checkpoint(str(packed[0]), dev)(idx)
    assert torch.equal(a, b)


def test_graph_decoder_matches_eager_decode(dev, packed):
    # every replay of the captured step against the eager decode, across two prompts
    from pollux_amd.model import GraphDecoder

    model = PackedPolluxModel.from_packed_checkpoint(str(packed[0]), dev)
    dec = GraphDecoder(model, batch=1)
    g = torch.Generator().manual_seed(4)
    worst = 0.0
    for prompt_len in (3, 6):
        idx = torch.randint(0, 90, (1, 16), generator=g).to(dev)
        with torch.inference_mode():
            first = dec.prefill(idx[:, :prompt_len])
            cache = model.new_cache(1)
            assert _rel(first, model.prefill(idx[:, :prompt_len], cache)[:, -1]) <= 1e-6
            for s in range(prompt_len, 16):
                got = dec.decode(idx[:, s]).clone()
                torch.cuda.synchronize()
                want = model.decode(idx[:, s], cache)
                worst = max(worst, _rel(got, want))
        with pytest.raises(ValueError):
            dec.decode(idx[:, 0])  # the cache is full
    print(f"[model] graph decode vs eager decode, worst rel {worst:.2e}", flush=True)
    assert worst <= 1e-5


@pytest.mark.parametrize("fused_head", [True, False])
def test_graph_greedy_decode_matches_eager_argmax(dev, packed, fused_head):
    # the captured step's own argmax and token feedback against an eager KV-cached greedy loop; with the
    # choice in the INT8 head GEMV's epilogue, and (head GEMV limited to 1 token) after the F.linear head
    from pollux_amd.model import GraphDecoder

    model = PackedPolluxModel.from_packed_checkpoint(str(packed[0]), dev)
    if not fused_head:
        model.head.gemv_max_tokens = 1
    dec = GraphDecoder(model, batch=2, greedy=True)
    assert (dec._head_ws is not None) == fused_head
    idx = torch.randint(0, 90, (2, 4), generator=torch.Generator().manual_seed(9)).to(dev)
    with torch.inference_mode():
        first = dec.prefill(idx).argmax(-1)
        got = dec.decode_greedy(first, 12)  # inputs at positions 4..15 fill the cache; choices for 5..16
        cache = model.new_cache(2)
        t = model.prefill(idx, cache)[:, -1].argmax(-1)
        want = []
        for _ in range(12):
            t = model.decode(t, cache).argmax(-1)
            want.append(t)
        want = torch.stack(want, dim=1)
        with pytest.raises(ValueError):
            dec.decode_greedy(first, 1)  # the cache is full
    print(f"[model] greedy graph tokens {got.tolist()}", flush=True)
    assert got.shape == (2, 12)
    assert torch.equal(got, want)


def test_last_only_logits(dev, packed):
    # the head on the last position only (INT8 GEMV) against the last row of the full logits (F.linear)
    model = PackedPolluxModel.from_packed_checkpoint(str(packed[0]), dev)
    idx = torch.randint(0, 90, (2, 10), generator=torch.Generator().manual_seed(6)).to(dev)
    with torch.inference_mode():
        full = model(idx)
        last = model(idx, last_only=True)
        cache = model.new_cache(2)
        pre = model.prefill(idx, cache, last_only=True)
    assert last.shape == (2, 1, 96) and pre.shape == (2, 1, 96)
    assert _rel(last[:, 0], full[:, -1]) <= 1e-5
    assert _rel(pre[:, 0], full[:, -1]) <= 1e-5


def test_graph_prefill_buckets_match_eager(dev, tmp_path):
    # prompts padded to 4 / 16 / 32 / 64 positions (graphs captured per bucket), on both sides of the
    # GEMV / GEMM switch at 4 tokens, against the eager prefill; decoding continues from the padded prefill
    from pollux_amd.model import GraphDecoder

    cfg = dict(CFG, seq_len=64)
    state, _ = pack.pack_state_dict(_dense_state(cfg, 11), dev)
    path = tmp_path / "s64.plx"
    plx.write_plx(path, pack.pack_config(cfg), state)
    model = PackedPolluxModel.from_packed_checkpoint(str(path), dev)
    dec = GraphDecoder(model, batch=1)
    g = torch.Generator().manual_seed(12)
    for t in (1, 4, 5, 16, 17, 33, 64):
        idx = torch.randint(0, 90, (1, t), generator=g).to(dev)
        with torch.inference_mode():
            got = dec.prefill(idx)
            cache = model.new_cache(1)
            want = model.prefill(idx, cache)[:, -1]
            assert _rel(got, want) <= 1e-5, t
            if t < 64:
                nxt = torch.tensor([5], device=dev)
                assert _rel(dec.decode(nxt), model.decode(nxt, cache)) <= 1e-5, t
    assert sorted(dec._prefills) == [4, 16, 32, 64]
    with pytest.raises(ValueError):
        dec.prefill(torch.zeros(1, 65, dtype=torch.long, device=dev))
