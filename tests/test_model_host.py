"""Host-side parts of the packed Pollux decoder: config rules, module tree (no GPU)."""

import pytest
import torch

from pollux_amd.model import PackedPolluxModel, PolluxConfig


def test_config_defaults_aliases_and_rules():
    cfg = PolluxConfig.from_dict({})
    assert (cfg.n_layers, cfg.n_heads, cfg.d_head, cfg.n_embd, cfg.vocab_size, cfg.seq_len) == (18, 80, 24, 1920, 50688, 1024)
    cfg = PolluxConfig.from_dict({"d_model": 48, "n_head": 2, "n_layer": 3, "vocab_size": 96,
                                  "tokenizer_vocab_size": 90, "unknown": 1})
    assert (cfg.n_embd, cfg.n_heads, cfg.n_layers) == (48, 2, 3)
    assert cfg.to_dict()["n_embd"] == 48 and "unknown" not in cfg.to_dict()
    bad = [
        {"d_head": 12, "n_heads": 4, "n_embd": 48},                       # d_head must be 24
        {"n_heads": 3, "n_embd": 48},                                      # n_embd = n_heads * d_head
        {"n_heads": 2, "n_embd": 48, "vocab_size": 100, "tokenizer_vocab_size": 90},  # vocab % 24
        {"n_heads": 2, "n_embd": 48, "vocab_size": 48, "tokenizer_vocab_size": 90},   # vocab covers tokenizer
    ]
    for raw in bad:
        with pytest.raises(ValueError):
            PolluxConfig.from_dict(raw)


def test_state_dict_keys_are_the_reference_packed_keys():
    cfg = PolluxConfig(n_layers=2, n_heads=2, n_embd=48, vocab_size=96, tokenizer_vocab_size=90, seq_len=16)
    keys = set(PackedPolluxModel(cfg).state_dict())
    want = {"tok_emb.weight_int8", "tok_emb.mu_rows", "pos_emb.weight", "ln_f.weight", "head.weight_int8",
            "head.mu_rows"}
    for i in range(2):
        p = f"blocks.{i}."
        want |= {p + "ln1.weight", p + "ln2.weight", p + "attn.q_ln.weight", p + "attn.k_ln.weight"}
        for name in ("attn.q_proj", "attn.k_proj", "attn.v_proj", "attn.o_proj", "mlp.fc1", "mlp.fc2"):
            want |= {p + name + ".packed_weights", p + name + ".sigma_rows"}
    assert keys == want
    sd = PackedPolluxModel(cfg).state_dict()
    assert sd["blocks.0.mlp.fc1.packed_weights"].numel() == (192 * 48 // 24 + 3) // 4 * 9
    assert sd["blocks.0.mlp.fc2.sigma_rows"].shape == (48,)
    assert sd["head.weight_int8"].shape == (96, 48) and sd["head.weight_int8"].dtype == torch.int8


def test_stacked_qkv_cache_follows_the_layers_buffers():
    """The stacked q/k/v copy is rebuilt when a layer's buffer is replaced or written in place."""
    from pollux_amd.packed import PackedH24Linear, _fused_group

    layers = [PackedH24Linear(48, 24), PackedH24Linear(48, 48)]
    for i, l in enumerate(layers):
        l.packed_weights.copy_(torch.randint(0, 256, l.packed_weights.shape, dtype=torch.uint8))
        l.sigma_rows.fill_(i + 1)
    a = _fused_group(layers)
    assert _fused_group(layers) is a and (a[2], a[3]) == (72, [0, 24])
    assert a[0].equal(torch.cat([l.packed_weights.reshape(-1) for l in layers]))
    layers[1].packed_weights.add_(1)                                   # in place
    b = _fused_group(layers)
    assert b is not a and b[0][layers[0].packed_weights.numel():].equal(layers[1].packed_weights.reshape(-1))
    layers[1].sigma_rows = torch.full_like(layers[1].sigma_rows, 7)    # replaced
    c = _fused_group(layers)
    assert c is not b and (c[1][24:] == 7).all() and (c[1][:24] == 1).all()
