"""plx_rms_norm, plx_decode_attention and plx_prefill_attention (the packed decoder's fused steps)
against torch references.

Bars (stated): RMS norm within 2e-6 relative per element of the torch
expression x * rsqrt(mean(x^2) + eps) * w (pollux.py:580-582); decode
attention within 1e-5 relative (L2) of scaled_dot_product_attention over the
cache with the new row appended, the written cache row within 2e-6 of the
normalised k and v bit-exact, every other cache row untouched; a position
outside the cache writes nothing and returns NaN.  Prefill attention: within
1e-5 relative (L2) of the causal attention computed in fp64 on the CPU over
the cached prefix and the new rows, written rows as for decode, every other
cache row untouched, positions past the cache refused.
"""

import math

import pytest
import torch

from pollux_amd.model import RMSNorm, decode_attention, prefill_attention, rms_norm

pytestmark = pytest.mark.gpu


def _ref_norm(x, w, eps=1e-8):
    return x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps) * w


@pytest.mark.parametrize("rows,d", [(37, 1920), (80, 24), (1, 7680), (513, 48)])
def test_rms_norm(dev, rows, d):
    g = torch.Generator().manual_seed(rows + d)
    x = (torch.randn(rows, d, generator=g) * 3.0).to(dev)
    w = (1.0 + 0.1 * torch.randn(d, generator=g)).to(dev)
    y = rms_norm(x, w, 1e-8)
    ref = _ref_norm(x.double(), w.double())
    err = ((y.double() - ref).abs() / ref.abs().clamp_min(1e-30)).max().item()
    print(f"[dec] rms_norm {rows}x{d}: max rel {err:.2e}", flush=True)
    assert err <= 2e-6
    with pytest.raises(ValueError):
        rms_norm(x.double(), w.double(), 1e-8)


def test_rms_norm_zero_row_and_module(dev):
    x = torch.zeros(2, 48, device=dev)
    x[1] = 1.0
    m = RMSNorm(48).to(dev)
    y = m(x)
    assert torch.equal(y[0], torch.zeros(48, device=dev))  # eps keeps the zero row finite
    assert torch.allclose(y[1], torch.ones(48, device=dev), rtol=1e-6)


# positions below one round of 64 (5 in a cache of 8 rows), at and across the round edges (63, 64)
# and the trip edges (191, 192: a block loads 3 rounds per trip; 255, 256), several trips (299,
# 1500), the first position (0), a batch of 16 sequences x 80 heads (the batched decode step)
@pytest.mark.parametrize("b,heads,max_len,pos", [(1, 80, 1024, 64), (2, 3, 16, 0), (1, 5, 300, 299), (3, 2, 8, 5),
                                                 (1, 4, 2048, 1500), (2, 3, 64, 63), (1, 2, 600, 191),
                                                 (1, 2, 600, 192), (1, 2, 600, 255), (1, 2, 600, 256),
                                                 (16, 80, 256, 100)])
def test_decode_attention(dev, b, heads, max_len, pos):
    g = torch.Generator().manual_seed(b * 1000 + heads + pos)
    c = heads * 24
    q = torch.randn(b, 1, c, generator=g).to(dev)
    k = torch.randn(b, 1, c, generator=g).to(dev)
    v = torch.randn(b, 1, c, generator=g).to(dev)
    q_ln, k_ln = RMSNorm(24).to(dev), RMSNorm(24).to(dev)
    with torch.no_grad():
        q_ln.weight.copy_(1.0 + 0.1 * torch.randn(24, generator=g))
        k_ln.weight.copy_(1.0 + 0.1 * torch.randn(24, generator=g))
    kc = torch.randn(b, heads, max_len, 24, generator=g).to(dev)
    vc = torch.randn(b, heads, max_len, 24, generator=g).to(dev)
    kc0, vc0 = kc.clone(), vc.clone()
    p = torch.tensor(pos, dtype=torch.long, device=dev)
    with torch.no_grad():
        out = decode_attention(q, k, v, q_ln, k_ln, kc, vc, p)
    # reference: the new row appended at pos, causal attention of the last query
    qn = _ref_norm(q.view(b, heads, 24).double(), q_ln.weight.detach().double())
    kn = _ref_norm(k.view(b, heads, 24).double(), k_ln.weight.detach().double())
    keys = kc0.double().clone()
    vals = vc0.double().clone()
    keys[:, :, pos] = kn
    vals[:, :, pos] = v.view(b, heads, 24).double()
    s = torch.einsum("bhc,bhjc->bhj", qn, keys[:, :, :pos + 1]) / math.sqrt(24)
    ref = torch.einsum("bhj,bhjc->bhc", torch.softmax(s, dim=-1), vals[:, :, :pos + 1]).reshape(b, 1, c)
    rel = ((out.double() - ref).norm() / ref.norm()).item()
    print(f"[dec] decode_attention b={b} H={heads} L={max_len} pos={pos}: rel {rel:.2e}", flush=True)
    assert rel <= 1e-5
    assert ((kc[:, :, pos].double() - kn).abs() / kn.abs().clamp_min(1e-30)).max().item() <= 2e-6
    assert torch.equal(vc[:, :, pos], v.view(b, heads, 24))
    rest = [j for j in range(max_len) if j != pos]
    assert torch.equal(kc[:, :, rest], kc0[:, :, rest]) and torch.equal(vc[:, :, rest], vc0[:, :, rest])


def test_decode_attention_alignment(dev):
    # a contiguous q that starts 4 bytes past a 16-byte boundary is copied to an aligned buffer by the
    # wrapper (same result); the C ABI refuses a q that is not 8-byte aligned and an odd row stride
    from pollux_amd import _lib

    b, heads, max_len, pos = 2, 3, 32, 9
    g = torch.Generator().manual_seed(77)
    base = torch.randn(b * heads * 24 + 1, generator=g).to(dev)
    q_off = base[1:].view(b, 1, heads * 24)
    assert q_off.data_ptr() % 16 == 4
    k = torch.randn(b, 1, heads * 24, generator=g).to(dev)
    v = torch.randn(b, 1, heads * 24, generator=g).to(dev)
    ln = RMSNorm(24).to(dev)
    kc = torch.randn(b, heads, max_len, 24, generator=g).to(dev)
    vc = torch.randn(b, heads, max_len, 24, generator=g).to(dev)
    kc2, vc2 = kc.clone(), vc.clone()
    p = torch.tensor(pos, dtype=torch.long, device=dev)
    with torch.no_grad():
        out = decode_attention(q_off, k, v, ln, ln, kc, vc, p)
        ref = decode_attention(q_off.clone(), k, v, ln, ln, kc2, vc2, p)
    assert torch.equal(out, ref) and torch.equal(kc, kc2)
    lib = _lib.lib()
    w = ln.weight.detach()
    o = torch.empty(b * heads, 24, device=dev)
    s = _lib.stream_of(dev)
    for qp, stride in ((q_off.data_ptr(), 0), (ref.data_ptr(), 0), (ref.data_ptr(), 73)):
        st = lib.plx_decode_attention(qp, k.data_ptr(), v.data_ptr(), stride, w.data_ptr(), w.data_ptr(), 1e-8,
                                      kc.data_ptr(), vc.data_ptr(), p.data_ptr(), b * heads, heads, max_len,
                                      o.data_ptr(), s)
        assert (st != 0) == (qp % 8 != 0 or stride % 2 != 0)
    torch.cuda.synchronize()


def test_decode_attention_position_outside_cache(dev):
    b, heads, max_len = 1, 2, 8
    q = torch.randn(b, 1, 48, device=dev)
    kc = torch.randn(b, heads, max_len, 24, device=dev)
    vc = torch.randn(b, heads, max_len, 24, device=dev)
    kc0, vc0 = kc.clone(), vc.clone()
    ln = RMSNorm(24).to(dev)
    for bad in (max_len, -1):
        with torch.no_grad():
            out = decode_attention(q, q, q, ln, ln, kc, vc, torch.tensor(bad, dtype=torch.long, device=dev))
        assert torch.isnan(out).all()
        assert torch.equal(kc, kc0) and torch.equal(vc, vc0)


@pytest.mark.parametrize("rows,cols", [(1, 50688), (3, 1000), (2, 7), (5, 4096), (1, 1)])
def test_argmax_rows_matches_torch(dev, rows, cols):
    from pollux_amd.model import argmax_rows

    g = torch.Generator().manual_seed(rows * 31 + cols)
    x = torch.randn(rows, cols, generator=g)
    if cols > 10:
        x[0, cols // 3] = x[0].max() + 1.0
        x[0, cols // 2] = x[0, cols // 3]  # a tie: the lower index wins
    x = x.to(dev)
    assert torch.equal(argmax_rows(x), torch.argmax(x, dim=-1))
    if cols > 10:
        y = x.clone()
        y[-1, 5] = float("nan")
        y[-1, 9] = float("nan")  # NaN counts as the maximum; the first NaN wins
        y[0] = float("-inf")      # all -inf: index 0
        assert torch.equal(argmax_rows(y), torch.argmax(y, dim=-1))
        # a row start that is not 16-byte aligned (element-wise loads)
        z = x.reshape(-1)[1:1 + (rows * cols - 1) // (cols - 1) * (cols - 1)].reshape(-1, cols - 1)
        assert torch.equal(argmax_rows(z), torch.argmax(z, dim=-1))


def test_argmax_rows_long_rows_and_out(dev):
    # rows past the register path (> 65,536 values) and the out= form
    from pollux_amd.model import argmax_rows

    x = torch.randn(2, 70_000, generator=torch.Generator().manual_seed(5)).to(dev)
    x[1, 69_999] = 100.0
    out = torch.full((2,), -1, dtype=torch.long, device=dev)
    assert argmax_rows(x, out=out) is out
    assert torch.equal(out, torch.argmax(x, dim=-1))
    with pytest.raises(ValueError):
        argmax_rows(x, out=torch.empty(3, dtype=torch.long, device=dev))


# (b, heads, t, p0, max_len): a Pollux-1920 prompt, two chunks of 256, a cached
# prefix, one token, a prefix plus more than a chunk
@pytest.mark.parametrize("b,heads,t,p0,max_len", [(1, 80, 64, 0, 128), (2, 3, 300, 0, 300), (2, 5, 17, 40, 64),
                                                  (1, 2, 1, 0, 4), (1, 4, 257, 7, 300)])
def test_prefill_attention(dev, b, heads, t, p0, max_len):
    g = torch.Generator().manual_seed(b * 7919 + heads * 31 + t + p0)
    c = heads * 24
    q = torch.randn(b, t, c, generator=g)
    k = torch.randn(b, t, c, generator=g)
    v = torch.randn(b, t, c, generator=g)
    qw = 1.0 + 0.1 * torch.randn(24, generator=g)
    kw = 1.0 + 0.1 * torch.randn(24, generator=g)
    kc0 = torch.randn(b, heads, max_len, 24, generator=g)
    vc0 = torch.randn(b, heads, max_len, 24, generator=g)
    q_ln, k_ln = RMSNorm(24).to(dev), RMSNorm(24).to(dev)
    with torch.no_grad():
        q_ln.weight.copy_(qw)
        k_ln.weight.copy_(kw)
    kc, vc = kc0.to(dev), vc0.to(dev)
    with torch.no_grad():
        out = prefill_attention(q.to(dev), k.to(dev), v.to(dev), q_ln, k_ln, kc, vc, p0)
    # reference (fp64, CPU): new rows at p0 .. p0+t-1, query i sees positions <= p0 + i
    qn = _ref_norm(q.view(b, t, heads, 24).double(), qw.double()).transpose(1, 2).contiguous()
    kn = _ref_norm(k.view(b, t, heads, 24).double(), kw.double()).transpose(1, 2).contiguous()
    vn = v.view(b, t, heads, 24).double().transpose(1, 2).contiguous()
    keys, vals = kc0.double().clone(), vc0.double().clone()
    keys[:, :, p0:p0 + t] = kn
    vals[:, :, p0:p0 + t] = vn
    keys, vals = keys[:, :, :p0 + t].contiguous(), vals[:, :, :p0 + t].contiguous()
    s = torch.matmul(qn, keys.transpose(-1, -2).contiguous()) / math.sqrt(24)
    allowed = torch.ones(t, p0 + t, dtype=torch.bool).tril(diagonal=p0)
    s = s.masked_fill(~allowed, float("-inf"))
    ref = torch.matmul(torch.softmax(s, dim=-1), vals).transpose(1, 2).reshape(b, t, c)
    rel = ((out.cpu().double() - ref).norm() / ref.norm()).item()
    print(f"[dec] prefill_attention b={b} H={heads} t={t} p0={p0}: rel {rel:.2e}", flush=True)
    assert rel <= 1e-5
    kcc, vcc = kc.cpu(), vc.cpu()
    assert ((kcc[:, :, p0:p0 + t].double() - kn).abs() / kn.abs().clamp_min(1e-30)).max().item() <= 2e-6
    assert torch.equal(vcc[:, :, p0:p0 + t], v.view(b, t, heads, 24).transpose(1, 2))
    rest = [j for j in range(max_len) if not p0 <= j < p0 + t]
    assert torch.equal(kcc[:, :, rest], kc0[:, :, rest]) and torch.equal(vcc[:, :, rest], vc0[:, :, rest])


def test_prefill_attention_refuses_positions_past_the_cache(dev):
    b, heads, max_len = 1, 2, 8
    x = torch.randn(b, 5, 48, device=dev)
    kc = torch.zeros(b, heads, max_len, 24, device=dev)
    ln = RMSNorm(24).to(dev)
    with pytest.raises(ValueError):
        prefill_attention(x, x, x, ln, ln, kc, kc.clone(), 4)
    assert torch.equal(kc, torch.zeros_like(kc))


@pytest.mark.parametrize("b,t", [(3, 1), (16, 1), (2, 5), (1, 9)])
def test_attention_reads_column_slices_of_a_stacked_projection(dev, b, t):
    # q, k, v as column slices of one [b, t, 3c] projection (the stacked q/k/v GEMM's output) are read
    # in place, rows 3c floats apart: the same results and cache writes as from contiguous copies
    heads, max_len = 4, 32
    c = heads * 24
    g = torch.Generator().manual_seed(b * 10 + t)
    qkv = torch.randn(b, t, 3 * c, generator=g).to(dev)
    q, k, v = qkv[..., :c], qkv[..., c:2 * c], qkv[..., 2 * c:]
    assert not q.is_contiguous()
    q_ln, k_ln = RMSNorm(24).to(dev), RMSNorm(24).to(dev)
    with torch.no_grad():
        q_ln.weight.copy_(1.0 + 0.1 * torch.randn(24, generator=g))
        k_ln.weight.copy_(1.0 + 0.1 * torch.randn(24, generator=g))
    kc = torch.randn(b, heads, max_len, 24, generator=g).to(dev)
    vc = torch.randn(b, heads, max_len, 24, generator=g).to(dev)
    kc2, vc2 = kc.clone(), vc.clone()
    with torch.no_grad():
        if t == 1:
            p = torch.tensor(7, dtype=torch.long, device=dev)
            a = decode_attention(q, k, v, q_ln, k_ln, kc, vc, p)
            r = decode_attention(q.contiguous(), k.contiguous(), v.contiguous(), q_ln, k_ln, kc2, vc2, p)
        else:
            a = prefill_attention(q, k, v, q_ln, k_ln, kc, vc, 3)
            r = prefill_attention(q.contiguous(), k.contiguous(), v.contiguous(), q_ln, k_ln, kc2, vc2, 3)
    assert torch.equal(a, r)
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
