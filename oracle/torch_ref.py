"""Oracle: the reference's non-Triton path restated with the same torch ops -- TEST INFRASTRUCTURE ONLY.

castor.py:544-557 (NN-B), pack.py:139-180 (NN-P + sigma16), castor.py:309-339
and pollux.py:874-884 (row scale and the per-step requantize composition),
pollux.py:485-507 (materialize + linear).  These call the same torch CPU ops
the reference calls (autocast-bf16 matmul, ``.float().max(-1)``, ``pow``,
``mean``, ``sqrt``, fp16 broadcast multiplies), so on the CPU they reproduce
the reference's results by construction.  bench.py times ``nn_b_indices`` on
the host cores as the CPU baseline ("kind": "port").

Pinned by:
  nn_b_indices, nn_p_indices   agreement with the exact float64 oracle
                               (oracle/nn.py) on every non-near-tie atom
                               (tests/test_oracle_nn.py);
  row_rms                      float64 closed form over the fp32 squares,
                               within 1 fp32 ulp, on seeded rows, a zero row,
                               one huge element, subnormals, an overflowing
                               square (tests/test_oracle_rowscale.py);
  normalize, lattice_input     correctly rounded fp32 quotients computed in
                               float64, bit-exact, including the sigma clamp;
  sigma16_from_sigma           float64 product rounded to fp32, the clamp,
                               numpy's RNE cast to fp16, bit-exact over the
                               fp16 rounding boundaries, subnormals, overflow;
  reconstruct                  fp32(fp32(c * sigma) * 0x3F3504F3) from float64
                               products, bit-exact;
  materialize                  numpy float16 emulation of
                               fp16(fp32(fp16(c16 * sigma16)) * fp32(1/sqrt 2)),
                               exhaustive over every finite fp16 sigma and all
                               8 alphabet values;
  linear_fp32                  float64 matmul within K * 2^-24 * sum|x||w|;
  pollux_h24_update            rule by rule against oracle/optim.py
                               (tests/test_oracle_optim.py);
  int8_materialize             numpy float16 emulation of
                               fp16(fp32(q) * fp32(fp16(fp32(mu) / 127))),
                               exhaustive over every finite fp16 mu and all
                               256 int8 values (tests/test_oracle_forward.py);
  _rms_norm                    float64 closed form rounded once, within the
                               first-order bound (d + 5) * 2^-24 relative;
  pollux_packed_forward        an independent float64 numpy forward of the
                               same packed state (own dequant emulation,
                               explicit causal softmax, erf GELU), relative
                               L2 <= 2e-6.
Each of these tests also shows that a plausible slip (eps outside the sqrt,
the clamp before the multiply, one rounding instead of two, a multiply by
fp32(sqrt 2) instead of the division, bf16 weights, a missing q_ln, the tanh
GELU, no causal mask) fails the same check.  ``linear_as_reference`` composes
the pinned pieces with torch's own F.linear.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import codebook as cbm

S_LATTICE = 1.0 / math.sqrt(2.0)  # castor.py:47 (s_lattice = 1/friction_c)
NUMERICAL_EPSILON = 1e-8  # castor.py:50


def codebook_tensor(dtype=torch.float32) -> torch.Tensor:
    return torch.from_numpy(cbm.codebook_f32().copy()).to(dtype)


def nn_b_indices(x: torch.Tensor, chunk_size: int = 4096, kp: torch.Tensor | None = None) -> torch.Tensor:
    """castor.py:544-557: chunked autocast-bf16 matmul, first max, origin snap. int64 [N]."""
    x = x.reshape(-1, 24).float()
    if kp is None:
        kp = codebook_tensor()[1:]
    c_sq = float(kp[0].pow(2).sum().item())
    out = torch.empty(x.shape[0], dtype=torch.long)
    for i in range(0, x.shape[0], chunk_size):
        with torch.autocast(device_type="cpu", dtype=torch.bfloat16):
            scores = torch.matmul(x[i : i + chunk_size], kp.t())
        best_val, best = scores.float().max(dim=-1)
        snap = (2.0 * best_val) < c_sq
        out[i : i + chunk_size] = (best + 1).masked_fill(snap, 0)
    return out


def nn_p_indices(w: torch.Tensor, chunk_size: int = 4096, kp: torch.Tensor | None = None) -> torch.Tensor:
    """pack.py:167-177: fp32 matmul on raw atoms, first max, origin iff |atom| < 1e-8."""
    atoms = w.detach().float().reshape(-1, 24)
    if kp is None:
        kp = codebook_tensor()[1:]
    out = torch.zeros(atoms.shape[0], dtype=torch.long)
    for i in range(0, atoms.shape[0], chunk_size):
        s = atoms[i : i + chunk_size]
        _, best = torch.matmul(s, kp.t()).max(dim=-1)
        snap = s.norm(dim=-1) < NUMERICAL_EPSILON
        out[i : i + chunk_size] = (best + 1).masked_fill(snap, 0)
    return out


def row_rms(w: torch.Tensor) -> torch.Tensor:
    """castor.py:309-313."""
    return torch.sqrt(w.pow(2).mean(dim=-1) + NUMERICAL_EPSILON)


def normalize(w: torch.Tensor, sigma: torch.Tensor | None = None):
    """castor.py:316-333: (w / sigma.clamp_min(eps), sigma)."""
    if sigma is None:
        sigma = row_rms(w)
    return w / sigma.reshape(-1, 1).clamp_min(NUMERICAL_EPSILON), sigma.reshape(-1)


def lattice_input(w: torch.Tensor, sigma: torch.Tensor | None = None):
    """pollux.py:876-882: x = normalize(w)/fp32(s_lattice) (a true division); returns (x, sigma)."""
    normed, sigma = normalize(w, sigma)
    return normed / float(S_LATTICE), sigma


def reconstruct(center: torch.Tensor, sigma: torch.Tensor) -> torch.Tensor:
    """castor.py:336-339 then pollux.py:883: (center * sigma[:, None]) * fp32(s_lattice)."""
    return (center * sigma.reshape(-1, 1)) * float(S_LATTICE)


def requantize(latent: torch.Tensor, sigma: torch.Tensor | None = None):
    """pollux.py:874-884 on the CPU: returns (indices int64 [N], sigma fp32 [R], p fp32 [R, C])."""
    x, sigma = lattice_input(latent, sigma)
    idx = nn_b_indices(x)
    center = codebook_tensor()[idx].reshape(latent.shape)
    return idx, sigma, reconstruct(center, sigma)


def sigma16_from_sigma(sigma: torch.Tensor) -> torch.Tensor:
    """The scale step of pack.py:164 on a given fp32 row RMS: fp16(clamp(sigma * fp32(sqrt(12)), 1e-8))."""
    return (sigma.float() * math.sqrt(12.0)).clamp_min(NUMERICAL_EPSILON).to(torch.float16)


def sigma16_pack(w: torch.Tensor) -> torch.Tensor:
    """pack.py:164: fp16(clamp(row_rms(w) * fp32(sqrt(12)), 1e-8))."""
    return sigma16_from_sigma(row_rms(w.detach().float()))


def materialize(indices: torch.Tensor, sigma16: torch.Tensor, out_features: int, in_features: int) -> torch.Tensor:
    """pollux.py:485-504: fp16 codebook gather, * sigma16 per row, * s_lattice, all in fp16."""
    cb16 = codebook_tensor(torch.float16)
    atoms = cb16.index_select(0, indices.long()).view(out_features, in_features // 24, 24)
    return (atoms * sigma16.view(-1, 1, 1) * S_LATTICE).reshape(out_features, in_features)


def linear_fp32(x: torch.Tensor, w16: torch.Tensor) -> torch.Tensor:
    """The fp32 reference for the packed layer: F.linear(x.float(), W.float()) (pollux.py:507 with fp32 x)."""
    return torch.nn.functional.linear(x.float(), w16.float())


def linear_as_reference(x: torch.Tensor, w16: torch.Tensor) -> torch.Tensor:
    """pollux.py:507, F.linear(x, W.to(x.dtype)), evaluated in fp32 on the CPU.

    The weight is first rounded to x's dtype as the reference does (bf16 RNE for
    bf16 activations, exact for fp32); the products of two bf16 values are
    exact in fp32, so this differs from the reference's GEMM only in the
    summation order (and in not rounding the output back to x's dtype).
    """
    return torch.nn.functional.linear(x.float(), w16.to(x.dtype).float())


def pollux_h24_update(grad, m, v, latent, heat, step, width_inertia):
    """pollux.py:815-878 for one H24 parameter with the reference's torch ops on the CPU (sqrt correctly rounded).

    m, v, latent are updated in place (as the reference does); returns the capped step.
    heat: 0-dim fp32 tensor; step: the step counter before the update (int).
    """
    gamma = 0.065771
    c_f = math.sqrt(2.0)
    kinematic_limit = (c_f - 1.0) / 2.0
    beta_2 = 1.0 - float(gamma)
    beta_1 = 1.0 - math.sqrt(float(gamma))
    step_f = torch.tensor(float(step), dtype=torch.float32) + 1.0
    bc1 = 1.0 - (torch.as_tensor(beta_1, dtype=torch.float32) ** step_f)
    bc2 = 1.0 - (torch.as_tensor(beta_2, dtype=torch.float32) ** step_f)
    m.mul_(beta_1).add_(grad, alpha=1.0 - beta_1)
    v.mul_(beta_2).addcmul_(grad, grad, value=1.0 - beta_2)
    m_unbiased = m / torch.clamp(bc1, min=NUMERICAL_EPSILON)
    v_unbiased = v / torch.clamp(bc2, min=NUMERICAL_EPSILON)
    # torch's vectorised CPU sqrt is faithful, not correctly rounded (1 ulp off on
    # ~0.7% of fp32 inputs); the reference runs this step on its GPU, where sqrtf
    # is correctly rounded.  sqrt in float64 then rounded to fp32 is the
    # correctly rounded fp32 sqrt (53 >= 2*24 + 2 bits).
    denom = torch.sqrt(v_unbiased.double()).float() + NUMERICAL_EPSILON
    kinetic_scale = heat * float(gamma) / float(c_f)
    adam_step = -(kinetic_scale / width_inertia) * (m_unbiased / denom)
    adam_h24 = adam_step.reshape(-1, 24)
    step_norm = torch.linalg.vector_norm(adam_h24, dim=-1, keepdim=True)
    speed_cap = float(kinematic_limit) * float(S_LATTICE)
    adam_step = (adam_h24 * torch.clamp(speed_cap / (step_norm + NUMERICAL_EPSILON), max=1.0)).reshape_as(adam_step)
    weight_decay_factor = 1.0 - (heat * (float(gamma) ** 2))
    latent.mul_(weight_decay_factor)
    latent.add_(adam_step)
    return adam_step


def int8_materialize(q: torch.Tensor, mu16: torch.Tensor) -> torch.Tensor:
    """PackedInt8Embedding/Linear.materialize (pollux.py:521-530): int8 * (mu / 127.0) in fp16."""
    return q.to(torch.float16) * (mu16.unsqueeze(-1).to(torch.float16) / 127.0)


def _rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-8) -> torch.Tensor:
    """RMSNorm.forward (pollux.py:580-582)."""
    return x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps) * w


def pollux_packed_forward(state: dict, cfg: dict, idx: torch.Tensor) -> torch.Tensor:
    """PolluxModel.forward with packed_inference after from_packed_checkpoint (pollux.py:566-702, 704-758).

    ``state``: a packed state dict (the .plx tensors); every packed weight is
    materialised the reference's way (unpack, fp16 codebook gather, * sigma16,
    * s_lattice; int8 * (mu / 127)) and the forward runs in fp32 on the CPU:
    embeddings, pre-norm blocks with per-head Q/K RMS norms, causal SDPA, GELU
    MLP, final norm, head.  Returns logits [b, t, vocab] (fp32).
    """
    from . import packing

    n_layers, n_heads, d_head = int(cfg["n_layers"]), int(cfg["n_heads"]), int(cfg["d_head"])
    f = torch.nn.functional

    n_embd = int(cfg["n_embd"])
    in_features = {"q_proj": n_embd, "k_proj": n_embd, "v_proj": n_embd, "o_proj": n_embd,
                   "fc1": n_embd, "fc2": 4 * n_embd}

    def h24(name: str) -> torch.Tensor:
        sig = state[name + ".sigma_rows"]
        out_f, in_f = sig.numel(), in_features[name.rsplit(".", 1)[1]]
        ids = packing.unpack(state[name + ".packed_weights"].numpy(), out_f * in_f // 24)
        return materialize(torch.from_numpy(ids.astype(np.int64)), sig, out_f, in_f).float()

    emb = int8_materialize(state["tok_emb.weight_int8"], state["tok_emb.mu_rows"])
    head = int8_materialize(state["head.weight_int8"], state["head.mu_rows"]).float()
    b, t = idx.shape
    x = f.embedding(idx, emb.float()) + state["pos_emb.weight"].float()[:t].unsqueeze(0)
    for i in range(n_layers):
        p = f"blocks.{i}."
        h = _rms_norm(x, state[p + "ln1.weight"].float())
        q = f.linear(h, h24(p + "attn.q_proj")).view(b, t, n_heads, d_head)
        k = f.linear(h, h24(p + "attn.k_proj")).view(b, t, n_heads, d_head)
        v = f.linear(h, h24(p + "attn.v_proj")).view(b, t, n_heads, d_head).transpose(1, 2)
        q = _rms_norm(q, state[p + "attn.q_ln.weight"].float()).transpose(1, 2)
        k = _rms_norm(k, state[p + "attn.k_ln.weight"].float()).transpose(1, 2)
        a = f.scaled_dot_product_attention(q, k, v, is_causal=True)
        x = x + f.linear(a.transpose(1, 2).contiguous().view(b, t, n_heads * d_head), h24(p + "attn.o_proj"))
        h = _rms_norm(x, state[p + "ln2.weight"].float())
        x = x + f.linear(f.gelu(f.linear(h, h24(p + "mlp.fc1"))), h24(p + "mlp.fc2"))
    return f.linear(_rms_norm(x, state["ln_f.weight"].float()), head)
