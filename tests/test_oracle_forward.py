"""Pins of the oracle's INT8 and packed-forward compositions (oracle/torch_ref.py), CPU only.

int8_materialize (pollux.py:521-530, w = int8 * (mu / 127) in fp16): exhaustive
over every finite fp16 mu and all 256 int8 values against numpy's float16
emulation of the two roundings torch makes (fp16(fp32(mu) / 127), then
fp16(fp32(q) * fp32(that)); the product is exact in fp32); one rounding of
the exact value instead differs on millions of pairs.
_rms_norm (pollux.py:580-582): against float64 x / sqrt(mean(x^2) + eps) * w
rounded once, within the first-order bound of the fp32 chain (d + 5) * 2^-24
relative (square, d-term mean, + eps, rsqrt as sqrt and reciprocal, two
products); eps outside the sqrt, a missing gain and sum-for-mean fail it.
pollux_packed_forward (pollux.py:566-702 on the materialised packed state):
against an independent float64 numpy forward (own unpack (oracle.packing),
own fp16 dequant emulation, explicit causal softmax, erf GELU from
math.erf) on a 2-layer toy: relative L2 <= 2e-6 (fp32 against float64;
measured 1.6e-7);
dropping q_ln, the tanh GELU or a missing causal mask exceed it.
"""

import math

import numpy as np
import torch

from oracle import codebook as cb
from oracle import packing, torch_ref

U = 2.0 ** -24


# ---------------------------------------------------------------- INT8 ----


def test_int8_materialize_exhaustive():
    mu = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    mu = mu[np.isfinite(mu)]
    assert len(mu) == 63488
    q = np.arange(-128, 128, dtype=np.int8)
    got = torch_ref.int8_materialize(torch.from_numpy(np.broadcast_to(q, (len(mu), 256)).copy()),
                                     torch.from_numpy(mu)).numpy()
    with np.errstate(over="ignore"):
        scale = (mu.astype(np.float32) / np.float32(127.0)).astype(np.float16)
        want = (q[None, :].astype(np.float32) * scale[:, None].astype(np.float32)).astype(np.float16)
        one = (q[None, :].astype(np.float64) * mu[:, None].astype(np.float64) / 127.0).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    assert int((one.view(np.uint16) != want.view(np.uint16)).sum()) > 1_000_000  # one rounding is a slip


# ------------------------------------------------------------- RMS norm ----


def _rms64(x, w, eps=1e-8, where="inside", gain=True, mean=True):
    x64 = x.astype(np.float64)
    ms = (x64 * x64).mean(-1, keepdims=True) if mean else (x64 * x64).sum(-1, keepdims=True)
    r = 1.0 / np.sqrt(ms + eps) if where == "inside" else 1.0 / np.sqrt(ms) + eps
    return x64 * r * (w.astype(np.float64) if gain else 1.0)


def test_rms_norm_float64_bound_and_slips():
    g = torch.Generator().manual_seed(5)
    cases = []
    for d in (24, 48, 1920):
        w = 1.0 + torch.randn(d, generator=g) * 0.1
        cases += [(torch.randn(8, d, generator=g) * s, w) for s in (1.0, 3e-2, 1e-5)]  # 1e-5: eps dominates
    for x, w in cases:
        d = x.shape[-1]
        got = torch_ref._rms_norm(x, w).numpy().astype(np.float64)
        ref = _rms64(x.numpy(), w.numpy())
        bound = (d + 5) * U * np.abs(ref) + 1e-45
        err = np.abs(got - ref)
        assert np.all(err <= bound), (d, float((err / bound).max()))
        ulp = np.abs(got.astype(np.float32).view(np.int32).astype(np.int64) -
                     ref.astype(np.float32).view(np.int32).astype(np.int64))
        print(f"[rms_norm] d={d} |x|~{float(x.abs().mean()):.1e}: max {int(ulp.max())} ulp of float64", flush=True)
        small = float(x.abs().max()) < 1e-4
        slips = [_rms64(x.numpy(), w.numpy(), gain=False), _rms64(x.numpy(), w.numpy(), mean=False)]
        if small:
            slips.append(_rms64(x.numpy(), w.numpy(), where="outside"))
        for bad in slips:
            assert np.any(np.abs(got - bad) > (d + 5) * U * np.abs(bad) + 1e-45)


# ------------------------------------------------------- packed forward ----

CFG = {"n_layers": 2, "n_heads": 2, "d_head": 24, "n_embd": 48, "vocab_size": 96, "seq_len": 16}


def _packed_state(seed):
    rng = np.random.default_rng(seed)
    d, v, s = CFG["n_embd"], CFG["vocab_size"], CFG["seq_len"]
    st = {}

    def h24(name, out_f, in_f, lo=0.005, hi=0.05):
        n = out_f * in_f // 24
        st[name + ".packed_weights"] = torch.from_numpy(packing.pack(rng.integers(0, 196561, n)))
        st[name + ".sigma_rows"] = torch.from_numpy(rng.uniform(lo, hi, out_f).astype(np.float16))

    def int8(name, rows, cols):
        st[name + ".weight_int8"] = torch.from_numpy(rng.integers(-127, 128, (rows, cols)).astype(np.int8))
        st[name + ".mu_rows"] = torch.from_numpy(rng.uniform(0.02, 0.08, rows).astype(np.float16))

    int8("tok_emb", v, d)
    int8("head", v, d)
    st["pos_emb.weight"] = torch.from_numpy((rng.normal(0, 0.02, (s, d))).astype(np.float32))
    st["ln_f.weight"] = torch.from_numpy((1 + rng.normal(0, 0.1, d)).astype(np.float32))
    for i in range(CFG["n_layers"]):
        p = f"blocks.{i}."
        for name in ("ln1", "ln2"):
            st[p + name + ".weight"] = torch.from_numpy((1 + rng.normal(0, 0.1, d)).astype(np.float32))
        for name in ("q_ln", "k_ln"):
            st[p + "attn." + name + ".weight"] = torch.from_numpy((1 + rng.normal(0, 0.1, 24)).astype(np.float32))
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            h24(p + "attn." + name, d, d)
        h24(p + "mlp.fc1", 4 * d, d, 0.3, 0.8)  # pre-activations of order 1, where the GELU forms differ
        h24(p + "mlp.fc2", d, 4 * d)
    return st


_SL = float(np.float32(1 / math.sqrt(2)))


def _f64_forward(st, idx, *, q_norm=True, gelu="erf", causal=True):
    """The packed model's forward in float64 numpy from the packed state (no torch ops)."""
    cb16 = cb.codebook_f32().astype(np.float16)
    d, nh, dh = CFG["n_embd"], CFG["n_heads"], CFG["d_head"]
    in_of = {"q_proj": d, "k_proj": d, "v_proj": d, "o_proj": d, "fc1": d, "fc2": 4 * d}

    def w_h24(name):
        sig = st[name + ".sigma_rows"].numpy()
        out_f, in_f = len(sig), in_of[name.rsplit(".", 1)[1]]
        ids = packing.unpack(st[name + ".packed_weights"].numpy(), out_f * in_f // 24)
        c = cb16[ids].reshape(out_f, in_f).astype(np.float32)
        w = (c * sig.astype(np.float32)[:, None]).astype(np.float16)          # fp16(c16 * sigma16)
        return (w.astype(np.float32) * np.float32(_SL)).astype(np.float16).astype(np.float64)  # * s_lattice

    def w_int8(name):
        mu = st[name + ".mu_rows"].numpy()
        sc = (mu.astype(np.float32) / np.float32(127.0)).astype(np.float16)
        q = st[name + ".weight_int8"].numpy()
        return (q.astype(np.float32) * sc.astype(np.float32)[:, None]).astype(np.float16).astype(np.float64)

    def rms(x, w):
        return x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-8) * w

    def act(h):
        if gelu == "erf":
            return 0.5 * h * (1.0 + np.vectorize(math.erf)(h / math.sqrt(2.0)))
        return 0.5 * h * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (h + 0.044715 * h ** 3)))

    b, t = idx.shape
    x = w_int8("tok_emb")[idx] + st["pos_emb.weight"].numpy().astype(np.float64)[:t][None]
    for i in range(CFG["n_layers"]):
        p = f"blocks.{i}."
        f64 = lambda k: st[p + k].numpy().astype(np.float64)  # noqa: E731
        h = rms(x, f64("ln1.weight"))
        q = (h @ w_h24(p + "attn.q_proj").T).reshape(b, t, nh, dh)
        k = (h @ w_h24(p + "attn.k_proj").T).reshape(b, t, nh, dh)
        v = (h @ w_h24(p + "attn.v_proj").T).reshape(b, t, nh, dh)
        if q_norm:
            q = rms(q, f64("attn.q_ln.weight"))
        k = rms(k, f64("attn.k_ln.weight"))
        s = np.einsum("bihd,bjhd->bhij", q, k) / math.sqrt(dh)
        if causal:
            s = np.where(np.tril(np.ones((t, t), bool))[None, None], s, -np.inf)
        s = np.exp(s - s.max(-1, keepdims=True))
        a = np.einsum("bhij,bjhd->bihd", s / s.sum(-1, keepdims=True), v).reshape(b, t, d)
        x = x + a @ w_h24(p + "attn.o_proj").T
        h = rms(x, f64("ln2.weight"))
        x = x + act(h @ w_h24(p + "mlp.fc1").T) @ w_h24(p + "mlp.fc2").T
    return rms(x, st["ln_f.weight"].numpy().astype(np.float64)) @ w_int8("head").T


def test_packed_forward_against_float64():
    st = _packed_state(7)
    idx = torch.from_numpy(np.random.default_rng(8).integers(0, 96, (2, 12)))
    got = torch_ref.pollux_packed_forward(st, CFG, idx).numpy().astype(np.float64)
    ref = _f64_forward(st, idx.numpy())

    def rel(a):
        return float(np.linalg.norm(a - ref) / np.linalg.norm(ref))

    e = rel(got)
    print(f"[packed forward] fp32 oracle vs float64: rel L2 {e:.2e}", flush=True)
    assert e <= 2e-6
    for kw in ({"q_norm": False}, {"gelu": "tanh"}, {"causal": False}):
        e_slip = float(np.linalg.norm(got - _f64_forward(st, idx.numpy(), **kw)) / np.linalg.norm(ref))
        print(f"[packed forward] slip {kw}: rel L2 {e_slip:.2e}", flush=True)
        assert e_slip > 2e-6, kw
