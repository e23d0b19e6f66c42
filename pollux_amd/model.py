"""Packed Pollux decoder for inference, with a KV cache (pollux.py:566-758, generate.py:280-336).

The reference loads a .plx checkpoint into ``PolluxModel`` with packed layers
(``from_packed_checkpoint``, pollux.py:704-758), materialises every packed
weight to fp16 and then, for every generated token, recomputes the whole
prefix (``generate``, generate.py:313-327).  Here:

* ``PackedPolluxModel`` has the reference's module tree and state-dict keys
  (``tok_emb``, ``pos_emb``, ``blocks.{i}.{ln1,attn,ln2,mlp}``, ``ln_f``,
  ``head``), so a .plx state dict loads with ``strict=True``;
* the H24 projections stay packed (0.76 bits per weight) and run the fused
  dequant-GEMV/GEMM kernels (``PackedH24Linear.forward``); ``materialize=True``
  gives the reference's dense fp16 path instead;
* ``prefill`` / ``decode`` keep each layer's keys and values in a ``KVCache``,
  so a new token costs one position instead of the whole prefix.

Activations are fp32, as in the reference's packed inference (no autocast):
the INT8 embedding rows are cast to fp32 (pollux.py:532-533), the packed
linears see fp32 x (exact products with the fp16 weights), the head multiplies
by its fp16 weight cast to fp32 (pollux.py:562-563).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable

import torch
import torch.nn as nn

from . import _lib
from .castor import H24_DIM, assert_row_aligned_width
from .packed import (
    PackedH24Linear,
    PackedInt8Embedding,
    PackedInt8Linear,
    int8_embed,
    int8_linear_argmax,
    int8_linear_argmax_workspace,
    packed_linear_group,
)
from .plx import check_fingerprint, load_plx

# pollux.py:258-278: the config fields and their aliases
CONFIG_FIELDS = (
    "n_layers", "n_heads", "d_head", "n_embd", "tokenizer_vocab_size", "vocab_size", "batch_size",
    "seq_len", "grad_accum_steps", "use_compile", "use_gradient_checkpointing", "target_tokens",
    "tokenizer_dir",
)
CONFIG_ALIASES = {"d_model": "n_embd", "n_layer": "n_layers", "n_head": "n_heads"}
CONFIG_DEFAULTS = {  # pollux.py:283-295
    "n_layers": 18, "n_heads": 80, "d_head": 24, "n_embd": 1920, "tokenizer_vocab_size": 50257,
    "vocab_size": 50688, "batch_size": 2, "seq_len": 1024, "grad_accum_steps": 128, "use_compile": False,
    "use_gradient_checkpointing": False, "target_tokens": 9_953_989_333, "tokenizer_dir": "",
}


class PolluxConfig:
    """PolluxConfig (pollux.py:280-356): architecture fields, dict round trip, validation."""

    def __init__(self, **overrides: Any) -> None:
        for name in CONFIG_FIELDS:
            setattr(self, name, overrides.get(name, CONFIG_DEFAULTS[name]))

    @classmethod
    def from_dict(cls, raw: dict[str, Any] | None) -> PolluxConfig:
        values = {}
        for key, value in (raw or {}).items():
            target = CONFIG_ALIASES.get(str(key), str(key))
            if target in CONFIG_FIELDS:
                values[target] = value
        cfg = cls(**values)
        cfg.validate_instance()
        return cfg

    def to_dict(self) -> dict[str, Any]:
        return {name: getattr(self, name) for name in CONFIG_FIELDS}

    def validate_instance(self) -> None:
        """pollux.py:324-349."""
        d_head, n_heads, n_embd = int(self.d_head), int(self.n_heads), int(self.n_embd)
        if d_head != H24_DIM:
            raise ValueError(
                f"d_head must equal H24_DIM ({H24_DIM}): each attention head is one "
                "24-dimensional Leech lattice atom."
            )
        if n_embd != n_heads * d_head:
            raise ValueError(
                "n_embd must equal n_heads * d_head: embedding width is an integer "
                "multiple of the 24D packing unit."
            )
        assert_row_aligned_width(n_embd)
        vocab, tok_vocab = int(self.vocab_size), int(self.tokenizer_vocab_size)
        if vocab % H24_DIM != 0:
            raise ValueError(f"vocab_size ({vocab}) must be divisible by H24_DIM ({H24_DIM}).")
        if vocab < tok_vocab:
            raise ValueError(f"vocab_size ({vocab}) must cover tokenizer_vocab_size ({tok_vocab}).")


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """x * rsqrt(mean(x^2) + eps) * weight over the last dimension, one HIP kernel (plx_rms_norm)."""
    _lib.require_device(x, "rms_norm input")
    if x.dtype != torch.float32 or weight.dtype != torch.float32:
        raise ValueError("rms_norm runs on fp32 activations and weights")
    xx = x.contiguous()
    w = weight.detach().contiguous()
    y = torch.empty_like(xx)
    d = xx.shape[-1]
    with torch.cuda.device(xx.device):
        st = _lib.lib().plx_rms_norm(_lib.ptr(xx), _lib.ptr(w), _lib.ptr(y), xx.numel() // d if d else 0, d,
                                     float(eps), _lib.stream_of(xx.device))
    _lib.check(st, "rms_norm")
    return y


def argmax_rows(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """torch.argmax(x, dim=-1) for fp32 x, one HIP kernel (plx_argmax_rows): int64 [...] (into ``out`` if given)."""
    _lib.require_device(x, "argmax_rows input")
    if x.dtype != torch.float32:
        raise ValueError("argmax_rows runs on fp32 values")
    cols = x.shape[-1]
    if cols == 0:
        raise ValueError("argmax_rows of an empty dimension")
    xx = x.reshape(-1, cols).contiguous()
    if out is None:
        out = torch.empty(x.shape[:-1], dtype=torch.long, device=x.device)
    if out.dtype != torch.long or out.numel() != xx.shape[0] or not out.is_contiguous() or out.device != x.device:
        raise ValueError("argmax_rows: out must be a contiguous int64 tensor with one element per row")
    with torch.cuda.device(x.device):
        st = _lib.lib().plx_argmax_rows(_lib.ptr(xx), xx.shape[0], cols, _lib.ptr(out), _lib.stream_of(x.device))
    _lib.check(st, "argmax_rows")
    return out


def _qkv_rows(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
    """(q, k, v, row stride) for the attention kernels: [b, t, c] views whose token rows lie a common
    stride apart (column slices of one stacked projection) are passed as they are, anything else
    as contiguous copies (stride 0)."""
    b, t, c = q.shape

    def stride_of(x):
        if x.shape != q.shape or x.stride(2) != 1 or x.data_ptr() % 16:
            return None
        s = x.stride(1) if t > 1 else x.stride(0)
        if b > 1 and x.stride(0) != t * s:
            return None
        return s if s >= c and s % 4 == 0 else None

    strides = {stride_of(x) for x in (q, k, v)}
    if len(strides) == 1 and None not in strides:
        return q, k, v, strides.pop()

    def aligned(x):  # the kernels read rows in 8- and 16-byte pieces
        x = x.contiguous()
        return x if x.data_ptr() % 16 == 0 else x.clone()

    return aligned(q), aligned(k), aligned(v), 0


def decode_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_ln: RMSNorm, k_ln: RMSNorm,
                     k_cache: torch.Tensor, v_cache: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
    """Attention of one new token per sequence over the cache (plx_decode_attention).

    q, k, v: [b, 1, H*24] projections (contiguous, or column slices of one stacked projection);
    caches [b, H, max_len, 24]; pos: 0-dim int64 device tensor.  Writes k_ln(k) and v at ``pos``;
    returns [b, 1, H*24].
    """
    b, t, c = q.shape
    heads = c // H24_DIM
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    qq, kk, vv, stride = _qkv_rows(q, k, v)
    with torch.cuda.device(q.device):
        st = _lib.lib().plx_decode_attention(
            _lib.ptr(qq), _lib.ptr(kk), _lib.ptr(vv), stride, _lib.ptr(q_ln.weight.detach()),
            _lib.ptr(k_ln.weight.detach()), float(q_ln.eps), _lib.ptr(k_cache), _lib.ptr(v_cache), _lib.ptr(pos),
            b * heads, heads, k_cache.shape[2], _lib.ptr(out), _lib.stream_of(q.device))
    _lib.check(st, "decode_attention")
    return out


def prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_ln: RMSNorm, k_ln: RMSNorm,
                      k_cache: torch.Tensor, v_cache: torch.Tensor, p0: int) -> torch.Tensor:
    """Causal attention of t new positions p0 .. p0+t-1 per sequence (plx_prefill_attention).

    q, k, v: [b, t, H*24] projections; caches [b, H, max_len, 24]. Writes
    k_ln(k) and v at positions p0 .. p0+t-1 and returns [b, t, H*24]: each query
    attends to every position up to its own (the cached prefix included).
    """
    b, t, c = q.shape
    heads = c // H24_DIM
    out = torch.empty(b, t, c, dtype=torch.float32, device=q.device)
    qq, kk, vv, stride = _qkv_rows(q, k, v)
    with torch.cuda.device(q.device):
        st = _lib.lib().plx_prefill_attention(
            _lib.ptr(qq), _lib.ptr(kk), _lib.ptr(vv), stride, _lib.ptr(q_ln.weight.detach()),
            _lib.ptr(k_ln.weight.detach()), float(q_ln.eps), _lib.ptr(k_cache), _lib.ptr(v_cache), b, heads, t,
            int(p0), k_cache.shape[2], _lib.ptr(out), _lib.stream_of(q.device))
    _lib.check(st, "prefill_attention")
    return out


class RMSNorm(nn.Module):
    """x * rsqrt(mean(x^2) + eps) * weight over the last dimension (pollux.py:566-582), fused on the device."""

    def __init__(self, dim: int, eps: float = 1e-8) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return rms_norm(x, self.weight, self.eps)


@dataclass
class KVCache:
    """Keys and values of every layer, [batch, heads, max_len, d_head] fp32, filled up to ``length``."""

    k: list[torch.Tensor]
    v: list[torch.Tensor]
    length: int = 0

    @classmethod
    def allocate(cls, cfg: PolluxConfig, batch: int, max_len: int, device) -> KVCache:
        # uninitialised: positions are only ever read after they are written (positions < length)
        shape = (batch, int(cfg.n_heads), max_len, int(cfg.d_head))
        n = int(cfg.n_layers)
        return cls([torch.empty(shape, device=device) for _ in range(n)],
                   [torch.empty(shape, device=device) for _ in range(n)])

    @property
    def max_len(self) -> int:
        return self.k[0].shape[2]


class PackedCausalAttention(nn.Module):
    """PolluxCausalAttention (pollux.py:585-626) on packed projections, with an optional KV cache."""

    def __init__(self, cfg: PolluxConfig) -> None:
        super().__init__()
        self.n_heads, self.d_head, self.n_embd = int(cfg.n_heads), int(cfg.d_head), int(cfg.n_embd)
        self.q_proj = PackedH24Linear(self.n_embd, self.n_embd)
        self.k_proj = PackedH24Linear(self.n_embd, self.n_embd)
        self.v_proj = PackedH24Linear(self.n_embd, self.n_embd)
        self.o_proj = PackedH24Linear(self.n_embd, self.n_embd)
        self.q_ln = RMSNorm(self.d_head)  # per-head Q/K norms on the 24-d atom
        self.k_ln = RMSNorm(self.d_head)

    def forward(self, x: torch.Tensor, cache: KVCache | None = None, layer: int = 0,
                pos: torch.Tensor | None = None, residual: torch.Tensor | None = None,
                norm: RMSNorm | None = None) -> torch.Tensor:
        """[residual +] o_proj(attention(norm(x))); norm and the q, k, v projections share one dequant-linear call."""
        b, t, c = x.shape
        q, k, v = packed_linear_group([self.q_proj, self.k_proj, self.v_proj], x,
                                      norm=None if norm is None else (norm.weight, norm.eps))
        if cache is not None and t == 1:
            # one new token per sequence: norms, cache write and attention in one kernel at device position pos
            if pos is None:
                pos = torch.full((), cache.length, dtype=torch.long, device=x.device)
            o = decode_attention(q, k, v, self.q_ln, self.k_ln, cache.k[layer], cache.v[layer], pos)
            return packed_linear_group([self.o_proj], o, residuals=[residual])[0]
        # q / k norms, cache writes and the causal attention in one kernel; without
        # a cache the keys and values go to a scratch cache of the prompt's length
        if cache is None:
            kc = torch.empty(b, self.n_heads, t, self.d_head, dtype=torch.float32, device=x.device)
            vc = torch.empty_like(kc)
            p0 = 0
        else:
            kc, vc, p0 = cache.k[layer], cache.v[layer], cache.length
        attn = prefill_attention(q, k, v, self.q_ln, self.k_ln, kc, vc, p0)
        return packed_linear_group([self.o_proj], attn, residuals=[residual])[0]


class PackedMLP(nn.Module):
    """PolluxMLP (pollux.py:629-645): fc2(gelu(fc1(x))), 4x expansion."""

    def __init__(self, cfg: PolluxConfig) -> None:
        super().__init__()
        n_embd = int(cfg.n_embd)
        self.fc1 = PackedH24Linear(n_embd, 4 * n_embd)
        self.fc2 = PackedH24Linear(4 * n_embd, n_embd)

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None,
                norm: RMSNorm | None = None) -> torch.Tensor:
        """[residual +] fc2(gelu(fc1(norm(x)))): the norm is fc1's prologue, the GELU and the residual add epilogues."""
        h = packed_linear_group([self.fc1], x, gelu=True, norm=None if norm is None else (norm.weight, norm.eps))[0]
        return packed_linear_group([self.fc2], h, residuals=[residual])[0]


class PackedBlock(nn.Module):
    """PolluxBlock (pollux.py:648-662): pre-norm attention and MLP residuals."""

    def __init__(self, cfg: PolluxConfig) -> None:
        super().__init__()
        self.ln1 = RMSNorm(int(cfg.n_embd))
        self.attn = PackedCausalAttention(cfg)
        self.ln2 = RMSNorm(int(cfg.n_embd))
        self.mlp = PackedMLP(cfg)

    def forward(self, x: torch.Tensor, cache: KVCache | None = None, layer: int = 0,
                pos: torch.Tensor | None = None) -> torch.Tensor:
        x = self.attn(x, cache, layer, pos, residual=x, norm=self.ln1)  # x + attn(ln1(x))
        return self.mlp(x, residual=x, norm=self.ln2)                    # x + mlp(ln2(x))


class PackedPolluxModel(nn.Module):
    """PolluxModel with ``packed_inference`` (pollux.py:665-702): INT8 embedding / head, packed H24 blocks."""

    def __init__(self, cfg: PolluxConfig) -> None:
        super().__init__()
        cfg.validate_instance()
        self.cfg = cfg
        n_embd = int(cfg.n_embd)
        self.tok_emb = PackedInt8Embedding(int(cfg.vocab_size), n_embd)
        self.pos_emb = nn.Embedding(int(cfg.seq_len), n_embd)
        self.blocks = nn.ModuleList([PackedBlock(cfg) for _ in range(int(cfg.n_layers))])
        self.ln_f = RMSNorm(n_embd)
        self.head = PackedInt8Linear(n_embd, int(cfg.vocab_size), bias=False)

    def _run(self, idx: torch.Tensor, pos0: int, cache: KVCache | None, last_only: bool = False,
             pick: torch.Tensor | None = None) -> torch.Tensor:
        t = idx.shape[1]
        pos = torch.arange(pos0, pos0 + t, device=idx.device).unsqueeze(0)
        x = self.embed(idx, pos[:, 0])
        step_pos = pos.view(()) if (cache is not None and t == 1) else None
        for i, block in enumerate(self.blocks):
            x = block(x, cache, i, step_pos)
        if cache is not None:
            cache.length = pos0 + t
        if pick is not None:  # one position given by a device index (graph-captured prefill of a padded prompt)
            return self.logits(x.index_select(1, pick.view(1)))
        return self.logits(x[:, -1:] if last_only else x)

    def embed(self, idx: torch.Tensor, pos0: torch.Tensor) -> torch.Tensor:
        """tok_emb(idx) + pos_emb(positions pos0 .. pos0 + t - 1) (pollux.py:691-693); pos0 a device int64 tensor."""
        if not self.tok_emb._materialized:
            return int8_embed(self.tok_emb.weight_int8, self.tok_emb.mu_rows, idx, pos_weight=self.pos_emb.weight,
                              pos0=pos0)
        pos = pos0.reshape(1, 1) + torch.arange(idx.shape[1], device=idx.device).unsqueeze(0)
        return self.tok_emb(idx) + self.pos_emb(pos)

    def logits(self, x: torch.Tensor) -> torch.Tensor:
        """head(ln_f(x)) (pollux.py:699-700), the norm fused into the INT8 head where that runs."""
        return self.head(x, norm=(self.ln_f.weight, self.ln_f.eps))

    def forward(self, idx: torch.Tensor, last_only: bool = False) -> torch.Tensor:
        """Logits [b, t, vocab] of the full prefix, positions 0..t-1 (pollux.py:691-702).

        ``last_only``: logits [b, 1, vocab] of the last position only (the head,
        the largest layer, then runs on one row per sequence).
        """
        if idx.shape[1] > int(self.cfg.seq_len):
            raise ValueError(f"sequence of {idx.shape[1]} tokens exceeds seq_len {self.cfg.seq_len}")
        return self._run(idx, 0, None, last_only)

    def new_cache(self, batch: int = 1, max_len: int | None = None) -> KVCache:
        device = self.pos_emb.weight.device
        return KVCache.allocate(self.cfg, batch, int(max_len or self.cfg.seq_len), device)

    def prefill(self, idx: torch.Tensor, cache: KVCache, last_only: bool = False) -> torch.Tensor:
        """Logits of ``idx`` appended at the cache's current length (``last_only``: of its last position only).

        The cache then holds the new positions too.
        """
        if cache.length + idx.shape[1] > min(cache.max_len, int(self.cfg.seq_len)):
            raise ValueError("the cache (or seq_len) is too short for these tokens")
        return self._run(idx, cache.length, cache, last_only)

    def decode(self, next_ids: torch.Tensor, cache: KVCache) -> torch.Tensor:
        """Logits [b, vocab] of one new token per sequence (next_ids [b] or [b, 1])."""
        return self.prefill(next_ids.reshape(-1, 1), cache)[:, -1]

    @classmethod
    def from_packed_checkpoint(cls, source: str | dict, device: torch.device | str, *,
                               materialize: bool = False) -> PackedPolluxModel:
        """PolluxModel.from_packed_checkpoint (pollux.py:704-758) for a .plx path or a loaded payload.

        The fingerprint check and the per-key dtype normalisation are the
        reference's.  Unless ``materialize`` (the reference's expansion of every
        packed layer to fp16), the H24 layers stay packed and the INT8 periphery
        stays INT8 (fused gather and GEMV kernels).
        """
        if isinstance(source, dict):
            check_fingerprint(source)
            payload = source
            state = {}
            for key, t in payload["state_dict"].items():
                if key.endswith(".packed_weights"):
                    t = t.to(dtype=torch.uint8)
                elif key.endswith(".weight_int8"):
                    t = t.to(dtype=torch.int8)
                elif key.endswith(".sigma_rows") or key.endswith(".mu_rows"):
                    t = t.to(dtype=torch.float16)
                elif t.is_floating_point():
                    t = t.to(dtype=torch.float32)
                state[key] = t.to(device)
        else:
            payload = load_plx(source, device)
            state = payload["state_dict"]
        cfg = PolluxConfig.from_dict(payload.get("config"))
        with torch.device("meta"):
            model = cls(cfg)
        model = model.to_empty(device=device)
        model.load_state_dict(state, strict=True)
        model.eval()
        if materialize:
            for module in model.modules():
                if isinstance(module, (PackedInt8Embedding, PackedInt8Linear, PackedH24Linear)):
                    module.materialize()
        return model


class GraphDecoder:
    """One-token decode steps of ``model`` replayed from a captured HIP graph.

    Static buffers: the token ids [batch], the position (a 0-dim device
    tensor the graph advances itself), the KV cache at its full length, and
    the logits.  The step is the eager modules' one-token path (fused packed
    linears, RMS norms and attention kernels, which read the position from
    the device), captured once.
    Usage: ``dec.prefill(prompt_ids)`` then ``logits = dec.decode(next_ids)``
    per token; the returned logits tensor is reused by the next replay.
    With ``greedy=True`` the captured step also takes the argmax of its
    logits, records it at its position and feeds it to the next replay:
    ``dec.decode_greedy(first_ids, n)`` then decodes n tokens without the
    host in the loop.  This is a raw-argmax path for measuring decode
    throughput, not the reference's sampler: the argmax runs over all
    ``vocab_size`` rows of the head, including any padded rows past the
    tokenizer's vocabulary, and applies no repetition penalty
    (generate.py:286-336 defaults to 1.1), so its tokens can differ from
    generate.py's.  ``generate`` below applies the reference's sampling rules.
    """

    def __init__(self, model: PackedPolluxModel, batch: int = 1, max_len: int | None = None,
                 greedy: bool = False) -> None:
        self.model = model
        cfg = model.cfg
        self.max_len = int(min(max_len or cfg.seq_len, cfg.seq_len))
        device = model.pos_emb.weight.device
        self.cache = model.new_cache(batch, self.max_len)
        self.ids = torch.zeros(batch, dtype=torch.long, device=device)
        self.pos = torch.zeros((), dtype=torch.long, device=device)
        self.greedy = bool(greedy)
        # token chosen at each position (greedy); one slot past the cache for the last step's choice
        self.history = torch.zeros(batch, self.max_len + 1, dtype=torch.long, device=device) if greedy else None
        # greedy with the INT8 head's GEMV: the argmax, the history entry and the position advance run as the
        # head kernel's epilogue plus one small kernel
        head = model.head
        self._head_ws = None
        if greedy and isinstance(head, PackedInt8Linear) and head.gemv_runs(
                torch.empty(batch, head.in_features, device="meta")):
            self._head_ws = int8_linear_argmax_workspace(head.out_features, batch, device)
        self.length = 0
        self.graph = None
        self.logits = None
        self._prefills = {}  # padded prompt length -> (graph, ids [batch, T], last position, logits)

    def _step(self) -> torch.Tensor:
        m = self.model
        b = self.ids.shape[0]
        x = m.embed(self.ids.view(b, 1), self.pos)
        for i, blk in enumerate(m.blocks):
            x = blk(x, self.cache, i, self.pos)
        if self._head_ws is not None and x.dtype == torch.float32:
            return int8_linear_argmax(m.head.weight_int8, m.head.mu_rows, x[:, -1], self.ids,
                                      norm=(m.ln_f.weight, m.ln_f.eps), history=self.history, pos=self.pos,
                                      workspace=self._head_ws)
        self.pos += 1
        logits = m.logits(x)[:, -1]
        if self.greedy:
            argmax_rows(logits, out=self.ids)  # the next replay's input
            self.history.index_copy_(1, self.pos.view(1), self.ids.view(b, 1))  # at the new token's position
        return logits

    @torch.inference_mode()
    def prefill(self, idx: torch.Tensor) -> torch.Tensor:
        """Prefill of ``idx`` [batch, t] from position 0; returns the logits of its last position.

        Replayed from a graph captured per padded length (4, then powers of
        two from 16, at most the cache length; captured on first use): the prompt is
        padded at its end, which causal attention makes exact -- no real
        position sees the padding, the logits come from position t - 1, and
        the padding's cache rows are overwritten by the decode steps before
        they are read.
        """
        b, t = idx.shape
        if b != self.ids.shape[0]:
            raise ValueError(f"prefill of {b} sequences for a decoder of batch {self.ids.shape[0]}")
        if not 1 <= t <= self.max_len:
            raise ValueError(f"a prompt of {t} tokens does not fit the cache's {self.max_len} positions")
        # 4, then 16, 32, 64, ...: the edge at 4 is the dequant-linear's GEMV / GEMM switch, so the real
        # tokens take the same kernels as without padding
        T = min(4 if t <= 4 else max(16, 1 << (t - 1).bit_length()), self.max_len)
        entry = self._prefills.get(T)
        if entry is None:
            entry = self._prefills[T] = self._capture_prefill(T)
        graph, ids, last, logits = entry
        ids[:, :t].copy_(idx)
        ids[:, t:].zero_()
        last.fill_(t - 1)
        graph.replay()
        self.cache.length = t
        self.length = t
        self.pos.fill_(t)
        if self.graph is None:
            self._capture()
        return logits[:, 0].clone()

    def _capture_prefill(self, T: int):
        device = self.pos.device
        ids = torch.zeros(self.ids.shape[0], T, dtype=torch.long, device=device)
        last = torch.full((), T - 1, dtype=torch.long, device=device)

        def run():
            self.cache.length = 0
            return self.model._run(ids, 0, self.cache, pick=last)

        side = torch.cuda.Stream(device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            for _ in range(2):  # warm-up: lazy casts, allocator
                run()
        torch.cuda.current_stream(device).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            logits = run()
        return graph, ids, last, logits

    def _capture(self) -> None:
        saved = self.length
        side = torch.cuda.Stream(self.pos.device)
        side.wait_stream(torch.cuda.current_stream(self.pos.device))
        with torch.cuda.stream(side):
            for _ in range(2):  # warm-up (lazy casts, allocator); writes only positions >= length
                self.pos.fill_(saved)
                self._step()
        torch.cuda.current_stream(self.pos.device).wait_stream(side)
        self.pos.fill_(saved)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.logits = self._step()
        self.pos.fill_(saved)  # capture does not run the step

    @torch.inference_mode()
    def decode(self, next_ids: torch.Tensor) -> torch.Tensor:
        """Logits [batch, vocab] of one new token per sequence at the next position."""
        if self.graph is None:
            raise RuntimeError("GraphDecoder.decode before prefill")
        if self.length >= self.max_len:
            raise ValueError(f"the cache holds {self.max_len} positions")
        self.ids.copy_(next_ids.reshape(-1))
        self.graph.replay()
        self.length += 1
        return self.logits

    @torch.inference_mode()
    def decode_greedy(self, next_ids: torch.Tensor, n: int) -> torch.Tensor:
        """Token ids [batch, n]: n greedy steps from ``next_ids``, each replay feeding its argmax to the next."""
        if not self.greedy:
            raise RuntimeError("decode_greedy needs GraphDecoder(..., greedy=True)")
        if self.graph is None:
            raise RuntimeError("GraphDecoder.decode_greedy before prefill")
        if n < 0 or self.length + n > self.max_len:
            raise ValueError(f"{n} steps from position {self.length} exceed the cache's {self.max_len} positions")
        start = self.length + 1  # position of the first chosen token
        self.ids.copy_(next_ids.reshape(-1))
        for _ in range(n):
            self.graph.replay()
        self.length += n
        return self.history[:, start:start + n].clone()


@torch.inference_mode()
def generate(model: PackedPolluxModel, ids: list[int], *, max_new_tokens: int = 80,
             sample: Callable[[torch.Tensor, torch.Tensor], int] | None = None, eos_id: int = 50256,
             use_cache: bool = True, use_graph: bool = False) -> list[int]:
    """The model side of generate.generate's token loop (generate.py:286-336) on token ids.

    Each step's fp32 logits of the last position ([vocab]) go to
    ``sample(logits, ids)`` with the sequence so far (``ids`` [1, t] int64 on
    the device), which returns the next token id; the caller supplies the
    reference's own sampling there (vocabulary mask, repetition penalty,
    temperature, top-k / top-p, multinomial).  ``sample=None`` is greedy:
    the first index of the largest logit, as ``torch.argmax``.  With
    ``use_cache`` the prompt is prefilled once and each new token is one
    ``decode`` position; once the sequence is longer than seq_len the
    reference's window ``idx[:, -seq_len:]`` restarts the positions at 0, so
    from then on every step recomputes the window, exactly as the reference
    does.  ``use_graph`` (with ``use_cache``): the prefill and the decode
    steps are replayed from a ``GraphDecoder``'s graphs (captured once per
    call, worth it for long generations); ``sample`` runs on the host's stream
    between replays.  Prompt ids outside [0, vocab_size) are refused.
    """
    device = model.pos_emb.weight.device
    seq_len = int(model.cfg.seq_len)
    vocab = int(model.cfg.vocab_size)
    if not ids:
        raise ValueError("generate needs at least one prompt token")
    if any(t < 0 or t >= vocab for t in ids):
        raise ValueError(f"prompt token ids must lie in [0, {vocab})")
    idx = torch.tensor([ids], device=device, dtype=torch.long)
    dec = GraphDecoder(model, batch=1) if (use_cache and use_graph) else None
    cache = model.new_cache(1, seq_len) if (use_cache and dec is None) else None
    started = False
    for _ in range(max_new_tokens):
        if dec is not None and idx.shape[1] <= seq_len:
            logits = dec.decode(idx[:, -1]) if started else dec.prefill(idx)
            started = True
        elif cache is not None and idx.shape[1] <= seq_len:
            if cache.length == 0:
                logits = model.prefill(idx, cache, last_only=True)[:, -1]
            else:
                logits = model.decode(idx[:, -1], cache)
        else:
            logits = model(idx[:, -seq_len:], last_only=True)[:, -1]
        row = logits.float()[0]
        next_id = int(torch.argmax(row).item()) if sample is None else int(sample(row.clone(), idx))
        if not 0 <= next_id < vocab:
            raise ValueError(f"sample returned token id {next_id} outside [0, {vocab})")
        idx = torch.cat([idx, torch.tensor([[next_id]], device=device)], dim=1)
        if next_id == eos_id:
            break
    return idx[0].tolist()
