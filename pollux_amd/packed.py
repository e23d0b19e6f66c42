"""Packed inference layer: PackedH24Linear with HIP dequantization (pollux.py:461-507).

Same constructor, buffers (``packed_weights`` uint8, ``sigma_rows`` fp16),
state-dict keys, ``materialize()`` and ``forward()`` as the reference, so
``PolluxModel.from_packed_checkpoint`` (pollux.py:704-752) can build it
unchanged.  ``materialize`` runs the fused unpack + LUT-gather + row-scale
kernel (plx_dequant_f16) instead of unpack_indices -> index_select -> two
broadcast multiplies.  Before ``materialize`` (or without it), ``forward``
runs the fused dequant-linear kernel on the packed weights directly.
"""

from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from .castor import assert_row_aligned_in_features, h24_linear_atom_count, h24_linear_scale_row_count


def dequantize_h24(packed: torch.Tensor, sigma16: torch.Tensor, out_features: int, in_features: int) -> torch.Tensor:
    """fp16 [out, in] = fp16(fp16(cb16[unpack(packed)] * sigma16[row]) * s_lattice) (pollux.py:491-499)."""
    _lib.require_device(packed, "dequantize_h24 packed input")
    if packed.dtype != torch.uint8:
        raise ValueError(f"packed weights must be uint8, got {packed.dtype}")
    if sigma16.dtype != torch.float16:
        raise ValueError(f"sigma rows must be float16, got {sigma16.dtype}")
    assert_row_aligned_in_features(in_features)
    pk = packed.reshape(-1).contiguous()
    sg = sigma16.reshape(-1).contiguous()
    if sg.numel() != out_features:
        raise ValueError(f"expected {out_features} sigma rows, got {sg.numel()}")
    out = torch.empty((out_features, in_features), dtype=torch.float16, device=pk.device)
    with torch.cuda.device(pk.device):
        st = _lib.lib().plx_dequant_f16(
            _lib.ptr(pk), pk.numel(), _lib.ptr(sg), out_features, in_features, _lib.ptr(out), _lib.stream_of(pk.device)
        )
    _lib.check(st, "dequantize_h24")
    return out


DQL_X_F32, DQL_W_AS_X, DQL_GELU, DQL_RMS_NORM, DQL_PLANES = 1, 2, 4, 8, 16  # plx_dequant_linear flags (include/pollux_amd.h)


def h24_plane_layout(packed: torch.Tensor, n_atoms: int) -> torch.Tensor:
    """The plane layout of a packed weight (plx_h24_plane_layout): int16 [3 * n_atoms], 6 bytes per atom.

    Per atom 3 records naming its three 8-coordinate planes in the table of the
    codebook's 4,961 distinct planes, so the dequant-linear kernels decode codes
    from a table in LDS instead of gathering from the 3 MB per-code tables.  A
    derived buffer: the packed stream stays the weight's state.
    """
    _lib.require_device(packed, "h24_plane_layout input")
    if packed.dtype != torch.uint8:
        raise ValueError("packed weights must be uint8")
    if packed.numel() != ((n_atoms + 3) // 4) * 9:
        raise ValueError(f"packed length {packed.numel()} does not match {n_atoms} atoms")
    pk = packed.reshape(-1).contiguous()
    out = torch.empty(3 * n_atoms, dtype=torch.int16, device=pk.device)
    if n_atoms:
        with torch.cuda.device(pk.device):
            st = _lib.lib().plx_h24_plane_layout(_lib.ptr(pk), pk.numel(), n_atoms, _lib.ptr(out),
                                                 _lib.stream_of(pk.device))
        _lib.check(st, "h24_plane_layout")
    return out


def plane_layout_takes(m: int, in_features: int) -> bool:
    """Whether the dequant-linear kernels run a batch of m tokens from the plane layout: one token
    with rows of at most 320 atoms (the GEMVs), or more than 4 tokens (the GEMM); layouts of 2^30
    bytes or more are not read (their kernels index them with 32-bit offsets)."""
    return m > 4 or (m == 1 and in_features // 24 <= 320)


def dequant_linear(
    packed: torch.Tensor, sigma16: torch.Tensor, out_features: int, in_features: int, x: torch.Tensor,
    weight_rounding: str = "exact", planes: torch.Tensor | None = None,
) -> torch.Tensor:
    """y = x @ W.T in fp32 without materialising W (pollux.py:491-507).

    weight_rounding="exact": products with the fp16 weights, exact, accumulated
    in fp32 -- the numerics of F.linear(x.float(), materialize(W).float()).
    weight_rounding="as_x": the reference's literal F.linear(x, W.to(x.dtype)),
    i.e. with bf16 activations the fp16 weight is rounded to bf16 first (for
    fp32 activations the two are the same).
    x: [..., in] bf16 or fp32 (other float dtypes are cast to fp32); returns fp32 [..., out].
    planes: the weight's h24_plane_layout, used for the batches plane_layout_takes
    names (same results, no per-atom table gathers); else the packed stream.
    """
    _lib.require_device(packed, "dequant_linear packed input")
    if packed.dtype != torch.uint8 or sigma16.dtype != torch.float16:
        raise ValueError("packed weights must be uint8 and sigma rows float16")
    if weight_rounding not in ("exact", "as_x"):
        raise ValueError(f"weight_rounding must be 'exact' or 'as_x', got {weight_rounding!r}")
    assert_row_aligned_in_features(in_features)
    if x.shape[-1] != in_features:
        raise ValueError(f"x has {x.shape[-1]} features, layer expects {in_features}")
    lead = x.shape[:-1]
    xx = x.reshape(-1, in_features)
    if xx.dtype not in (torch.bfloat16, torch.float32):
        xx = xx.float()
    xx = xx.contiguous()
    pk = packed.reshape(-1).contiguous()
    if pk.data_ptr() % 16:
        pk = pk.clone()  # the kernel streams the packed bytes as aligned 16-byte vectors
    if xx.data_ptr() % 16:
        xx = xx.clone()
    sg = sigma16.reshape(-1).contiguous()
    y = torch.empty((xx.shape[0], out_features), dtype=torch.float32, device=pk.device)
    flags = (DQL_X_F32 if xx.dtype == torch.float32 else 0) | (DQL_W_AS_X if weight_rounding == "as_x" else 0)
    src, nsrc = pk, pk.numel()
    n_atoms = out_features * (in_features // 24)
    if planes is not None and plane_layout_takes(xx.shape[0], in_features) and 6 * n_atoms < 1 << 30:
        if planes.dtype != torch.int16 or planes.numel() != 3 * n_atoms or planes.device != pk.device:
            raise ValueError("planes must be the weight's int16 plane layout (h24_plane_layout) on its device")
        src = planes.contiguous()
        if src.data_ptr() % 16:
            src = src.clone()
        nsrc = 6 * n_atoms
        flags |= DQL_PLANES
    lib = _lib.lib()
    nws = int(lib.plx_dequant_linear_workspace_bytes(out_features, in_features, xx.shape[0], flags))
    ws = torch.empty(max(nws, 16), dtype=torch.uint8, device=pk.device) if nws else None
    with torch.cuda.device(pk.device):
        st = lib.plx_dequant_linear(
            _lib.ptr(src), nsrc, _lib.ptr(sg), out_features, in_features, _lib.ptr(xx),
            flags, xx.shape[0], _lib.ptr(y), _lib.ptr(ws), nws, _lib.stream_of(pk.device),
        )
    _lib.check(st, "dequant_linear")
    return y.reshape(*lead, out_features)


def dequant_linear_multi(
    weights: list[tuple[torch.Tensor, torch.Tensor, int]], in_features: int, x: torch.Tensor, *,
    residuals: list[torch.Tensor | None] | None = None, gelu: bool = False, weight_rounding: str = "exact",
    norm: tuple[torch.Tensor, float] | None = None, planes: list[torch.Tensor] | None = None,
) -> list[torch.Tensor]:
    """Several packed weights sharing x in one call: [residual_i +] act(n(x) @ W_i.T), fp32 [..., out_i] each.

    ``weights``: (packed, sigma16, out_features) per target; act = GELU (erf
    form, as F.gelu) when ``gelu``; ``residuals``: fp32 [..., out_i] tensors
    added after the activation (or None); ``norm``: (weight, eps) of an
    RMSNorm applied to x first (fp32 x; n = identity when None).  At up to 4
    tokens, four targets share one GEMV launch, which also normalises x.
    Results equal separate dequant_linear calls followed by the same epilogue.
    ``planes``: each weight's h24_plane_layout, read for the batches
    plane_layout_takes names (same results), else the packed streams.
    """
    if weight_rounding not in ("exact", "as_x"):
        raise ValueError(f"weight_rounding must be 'exact' or 'as_x', got {weight_rounding!r}")
    if not 1 <= len(weights) <= 16:
        raise ValueError("dequant_linear_multi takes 1..16 weights")
    if planes is not None and len(planes) != len(weights):
        raise ValueError("planes: one plane layout per weight")
    assert_row_aligned_in_features(in_features)
    if x.shape[-1] != in_features:
        raise ValueError(f"x has {x.shape[-1]} features, layer expects {in_features}")
    lead = x.shape[:-1]
    xx = x.reshape(-1, in_features)
    if xx.dtype not in (torch.bfloat16, torch.float32):
        xx = xx.float()
    xx = xx.contiguous()
    if xx.data_ptr() % 16:
        xx = xx.clone()
    _lib.require_device(xx, "dequant_linear_multi x")
    m = xx.shape[0]
    use_planes = (planes is not None and plane_layout_takes(m, in_features)
                  and all(6 * out_f * (in_features // 24) < 1 << 30 for _, _, out_f in weights))
    residuals = residuals or [None] * len(weights)
    arr = (_lib.DqlTarget * len(weights))()
    ys, keep = [], []
    for i, (pk, sg, out_f) in enumerate(weights):
        _lib.require_device(pk, "dequant_linear_multi packed input")
        if pk.dtype != torch.uint8 or sg.dtype != torch.float16:
            raise ValueError("packed weights must be uint8 and sigma rows float16")
        pk = pk.reshape(-1).contiguous()
        if pk.data_ptr() % 16:
            pk = pk.clone()
        sg = sg.reshape(-1).contiguous()
        if sg.numel() != out_f or pk.numel() != ((out_f * in_features // 24 + 3) // 4) * 9:
            raise ValueError(f"target {i}: packed / sigma sizes do not match [{out_f}, {in_features}]")
        if use_planes:
            pl = planes[i]
            if pl.dtype != torch.int16 or pl.numel() != 3 * out_f * (in_features // 24) or pl.device != pk.device:
                raise ValueError(f"target {i}: planes must be the weight's int16 plane layout on its device")
            pk = pl.reshape(-1).contiguous()
            if pk.data_ptr() % 16:
                pk = pk.clone()
        y = torch.empty((m, out_f), dtype=torch.float32, device=xx.device)
        r = residuals[i]
        if r is not None:
            if r.dtype != torch.float32 or r.numel() != m * out_f:
                raise ValueError(f"target {i}: residual must be float32 with {m * out_f} elements")
            r = r.reshape(m, out_f).contiguous()
        arr[i] = _lib.DqlTarget(pk.data_ptr(), sg.data_ptr(), out_f, y.data_ptr(), _lib.ptr(r))
        keep += [pk, sg, r]
        ys.append(y)
    flags = (DQL_X_F32 if xx.dtype == torch.float32 else 0) | (DQL_W_AS_X if weight_rounding == "as_x" else 0) | (
        DQL_GELU if gelu else 0) | (DQL_PLANES if use_planes else 0)
    nw, eps = None, 0.0
    if norm is not None:
        nw, eps = norm[0].detach(), float(norm[1])
        if xx.dtype != torch.float32 or nw.dtype != torch.float32 or nw.numel() != in_features:
            raise ValueError(f"norm: fp32 x and an fp32 weight of {in_features} values")
        _lib.require_device(nw, "dequant_linear_multi norm weight")
        nw = nw.reshape(-1).contiguous()
        if nw.data_ptr() % 16:
            nw = nw.clone()
        flags |= DQL_RMS_NORM
    lib = _lib.lib()
    nws = int(lib.plx_dequant_linear_multi_workspace_bytes(arr, len(weights), in_features, m, flags))
    ws = torch.empty(max(nws, 16), dtype=torch.uint8, device=xx.device) if nws else None
    with torch.cuda.device(xx.device):
        st = lib.plx_dequant_linear_multi(arr, len(weights), in_features, _lib.ptr(xx), flags, m, _lib.ptr(nw), eps,
                                          _lib.ptr(ws), nws, _lib.stream_of(xx.device))
    _lib.check(st, "dequant_linear_multi")
    return [y.reshape(*lead, y.shape[1]) for y in ys]


def _capturing() -> bool:
    """Whether the current stream is capturing a HIP graph (False on a host without a device)."""
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def _fused_group(layers: list) -> tuple[torch.Tensor, torch.Tensor, int, list[int]]:
    """(packed, sigma16, rows, row offsets) of ``layers`` stacked along their output rows.

    Valid when every layer holds a whole number of 9-byte groups (rows * in_features / 24 % 4 == 0):
    the streams then concatenate byte for byte.  Kept on the first layer; rebuilt when any layer's
    buffers are replaced (the entry holds the tensors themselves, compared by identity) or
    modified in place (their version counters; tensors created under ``torch.inference_mode``
    keep none, so an in-place write to those is not seen: replace such buffers instead).
    """
    bufs = tuple(t for l in layers for t in (l.packed_weights, l.sigma_rows))
    versions = tuple(None if t.is_inference() else t._version for t in bufs)
    hit = layers[0].__dict__.get("_stacked")
    if hit is not None and len(hit[0]) == len(bufs) and all(a is b for a, b in zip(hit[0], bufs)) \
            and hit[1] == versions:
        return hit[2]
    offs, r = [], 0
    for l in layers:
        offs.append(r)
        r += l.out_features
    fused = (torch.cat([l.packed_weights.reshape(-1) for l in layers]),
             torch.cat([l.sigma_rows.reshape(-1) for l in layers]), r, offs)
    if not _capturing():
        # under graph capture the copies run only on replay: the captured graph makes its own, and
        # nothing is kept for eager calls that may come before a replay
        layers[0].__dict__["_stacked"] = (bufs, versions, fused)
    return fused


def _stacked_planes(layers: list, planes: list[torch.Tensor]) -> torch.Tensor:
    """The layers' plane layouts stacked along their output rows (records concatenate atom for atom),
    kept on the first layer while the same layout tensors are passed (each layer rebuilds its own
    layout when its packed buffer changes, which gives a new tensor here)."""
    hit = layers[0].__dict__.get("_stacked_planes")
    if hit is not None and len(hit[0]) == len(planes) and all(a is b for a, b in zip(hit[0], planes)):
        return hit[1]
    stacked = torch.cat([p.reshape(-1) for p in planes])
    if not _capturing():
        layers[0].__dict__["_stacked_planes"] = (tuple(planes), stacked)
    return stacked


def packed_linear_group(layers: list, x: torch.Tensor, *, residuals: list | None = None,
                        gelu: bool = False, norm: tuple[torch.Tensor, float] | None = None) -> list[torch.Tensor]:
    """[residual +] act(layer(n(x))) for PackedH24Linear layers sharing x, fused when they are all packed.

    ``norm``: (weight, eps) of an RMSNorm applied to x first (fp32 x), or None.
    Materialised layers take the reference's ops instead (the RMSNorm
    expression of pollux.py:580-582, F.linear on the weight cast to x's dtype,
    F.gelu, then the residual add).
    """
    residuals = residuals or [None] * len(layers)
    if all(isinstance(l, PackedH24Linear) and not l._materialized and l.bias is None for l in layers):
        in_f = layers[0].in_features
        m = x.numel() // max(in_f, 1)
        planes = None
        if all(l.use_plane_layout and l.in_features == in_f for l in layers) and plane_layout_takes(m, in_f):
            planes = [l.plane_layout() for l in layers]
            if any(p is None for p in planes):  # under graph capture without built layouts
                planes = None
        if (len(layers) > 1 and m > 4 and all(r is None for r in residuals)
                and all(l.in_features == in_f and (l.out_features * in_f // 24) % 4 == 0 for l in layers)
                and len({l.weight_rounding for l in layers}) == 1):
            # above 4 tokens the weights run as separate GEMM launches: one stacked weight takes one
            packed, sigma, rows, offs = _fused_group(layers)
            stacked_planes = None if planes is None else [_stacked_planes(layers, planes)]
            (y,) = dequant_linear_multi([(packed, sigma, rows)], in_f, x, gelu=gelu,
                                        weight_rounding=layers[0].weight_rounding, norm=norm, planes=stacked_planes)
            y = y.to(x.dtype)
            return [y[..., o:o + l.out_features] for l, o in zip(layers, offs)]
        ys = dequant_linear_multi([(l.packed_weights, l.sigma_rows, l.out_features) for l in layers],
                                  layers[0].in_features, x, residuals=residuals, gelu=gelu,
                                  weight_rounding=layers[0].weight_rounding, norm=norm, planes=planes)
        return [y.to(x.dtype) for y in ys]
    if norm is not None:
        x = x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + norm[1]) * norm[0]
    outs = []
    for layer, r in zip(layers, residuals):
        y = layer(x)
        if gelu:
            y = F.gelu(y)
        outs.append(y if r is None else r + y)
    return outs


class PackedH24Linear(nn.Module):
    """uint8 packed 18-bit indices + fp16 row scale; dense fp16 weight after materialize().

    Before materialize, forward runs dequant_linear with ``weight_rounding``
    (class default "exact"; "as_x" reproduces the reference's rounding of W to
    x's dtype).  With ``use_plane_layout`` (class default True) the batches
    plane_layout_takes names read a plane layout of the weight kept beside the
    packed buffer (6 B per atom, built on first use; same results, no per-atom
    table gathers); False keeps only the packed stream resident.
    Resident weight memory before materialize: 0.76 bits/param with the packed
    stream alone (18-bit indices + fp16 row scales), 2.76 bits/param once the
    plane layout is built (2 bits/param more) -- set use_plane_layout = False
    where memory, not the one-token latency, is the limit.
    """

    weight_rounding = "exact"
    use_plane_layout = True

    def __init__(self, in_features: int, out_features: int, bias: bool = False) -> None:
        super().__init__()
        assert_row_aligned_in_features(in_features)
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self.num_atoms = h24_linear_atom_count(self.out_features, self.in_features)
        self.num_sigma_rows = h24_linear_scale_row_count(self.out_features)
        packed_len = ((self.num_atoms + 3) // 4) * 9
        self.register_buffer("packed_weights", torch.zeros(packed_len, dtype=torch.uint8))
        self.register_buffer("sigma_rows", torch.ones(self.num_sigma_rows, dtype=torch.float16))
        self._materialized = False
        if bias:
            self.bias = nn.Parameter(torch.zeros(self.out_features))
        else:
            self.register_parameter("bias", None)

    def materialize(self) -> None:
        if self._materialized:
            return
        weight = dequantize_h24(self.packed_weights, self.sigma_rows.to(torch.float16), self.out_features, self.in_features)
        self.weight = nn.Parameter(weight, requires_grad=False)
        del self.packed_weights
        del self.sigma_rows
        self._materialized = True

    def plane_layout(self) -> torch.Tensor | None:
        """The packed weight's h24_plane_layout, built on first use and kept beside it (not part of the state).

        Rebuilt when packed_weights is replaced (compared by identity) or modified in place (its version
        counter; a tensor created under ``torch.inference_mode`` keeps none, so replace such a buffer instead).
        """
        pk = self.packed_weights
        ver = None if pk.is_inference() else pk._version
        hit = self.__dict__.get("_planes")
        if hit is not None and hit[0] is pk and hit[1] == ver:
            return hit[2]
        if _capturing():
            # a layout built under graph capture holds nothing until the graph is replayed: callers
            # then read the packed stream (build the layout with an eager call before capturing)
            return None
        planes = h24_plane_layout(pk, self.num_atoms)
        self.__dict__["_planes"] = (pk, ver, planes)
        return planes

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not self._materialized:
            # fused path: weights stay packed (0.76 bits/param); fp32 result cast to x's dtype.  The batches
            # plane_layout_takes names run from the plane layout (6 B per atom, built once and kept:
            # 2.76 bits/param resident with it).
            m = x.numel() // self.in_features if self.in_features else 0
            takes = self.use_plane_layout and plane_layout_takes(m, self.in_features)
            planes = self.plane_layout() if takes else None
            y = dequant_linear(self.packed_weights, self.sigma_rows, self.out_features, self.in_features, x,
                               weight_rounding=self.weight_rounding, planes=planes).to(x.dtype)
            return y if self.bias is None else y + self.bias.to(x.dtype)
        return F.linear(x, self.weight.to(dtype=x.dtype), self.bias)


def dequantize_int8_rows(q: torch.Tensor, mu16: torch.Tensor) -> torch.Tensor:
    """fp16 weight = q * (mu / 127) per row, as torch evaluates it on fp16 device tensors (pollux.py:526)."""
    _lib.require_device(q, "dequantize_int8_rows input")
    if q.dtype != torch.int8 or mu16.dtype != torch.float16:
        raise ValueError("INT8 rows need int8 values and float16 mu_rows")
    if q.dim() < 1:
        raise ValueError("INT8 rows need at least one dimension")
    cols = q.shape[-1]
    rows = q.numel() // cols if cols else 0
    if mu16.numel() != rows:
        raise ValueError(f"expected {rows} mu rows, got {mu16.numel()}")
    qq = q.contiguous()
    mu = mu16.reshape(-1).contiguous()
    out = torch.empty(q.shape, dtype=torch.float16, device=q.device)
    if rows and cols:
        with torch.cuda.device(q.device):
            st = _lib.lib().plx_dequant_int8_rows(
                _lib.ptr(qq), _lib.ptr(mu), rows, cols, _lib.ptr(out), _lib.stream_of(q.device)
            )
        _lib.check(st, "dequantize_int8_rows")
    return out


def int8_linear(q: torch.Tensor, mu16: torch.Tensor, x: torch.Tensor, *,
                norm: tuple[torch.Tensor, float] | None = None) -> torch.Tensor:
    """fp32 [..., rows] = n(x) @ W.T with W = q * (mu / 127) in fp16 (never stored), one HIP kernel (plx_int8_linear).

    Exact products, fp32 sums: F.linear(x, W.float()) up to summation order
    (PackedInt8Linear.forward, pollux.py:562-563).  ``norm``: (weight, eps) of
    an RMSNorm applied to x first, or None.  x fp32 with a multiple of 16 up to
    4,096 features.
    """
    _lib.require_device(x, "int8_linear input")
    if q.dtype != torch.int8 or mu16.dtype != torch.float16 or x.dtype != torch.float32:
        raise ValueError("int8_linear: int8 q, float16 mu and float32 x")
    rows, cols = q.shape
    if x.shape[-1] != cols or mu16.numel() != rows:
        raise ValueError(f"int8_linear: x has {x.shape[-1]} features, weight [{rows}, {cols}], {mu16.numel()} mu rows")
    xx = x.reshape(-1, cols).contiguous()
    if xx.data_ptr() % 16:
        xx = xx.clone()
    qq = q.contiguous()
    nw, eps = None, 0.0
    if norm is not None:
        nw, eps = norm[0].detach().reshape(-1).contiguous(), float(norm[1])
        if nw.dtype != torch.float32 or nw.numel() != cols:
            raise ValueError(f"int8_linear: the norm weight must be fp32 with {cols} values")
        if nw.data_ptr() % 16:
            nw = nw.clone()
    y = torch.empty((xx.shape[0], rows), dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        st = _lib.lib().plx_int8_linear(_lib.ptr(qq), _lib.ptr(mu16.contiguous()), rows, cols, _lib.ptr(xx),
                                        xx.shape[0], _lib.ptr(nw), eps, _lib.ptr(y), _lib.stream_of(x.device))
    _lib.check(st, "int8_linear")
    return y.reshape(*x.shape[:-1], rows)


def int8_linear_argmax_workspace(rows: int, tokens: int, device) -> torch.Tensor:
    """The workspace int8_linear_argmax needs for ``rows`` output rows and ``tokens`` tokens (uint8)."""
    n = int(_lib.lib().plx_int8_linear_argmax_workspace_bytes(int(rows), int(tokens)))
    return torch.empty(max(n, 8), dtype=torch.uint8, device=device)


def int8_linear_argmax(q: torch.Tensor, mu16: torch.Tensor, x: torch.Tensor, ids: torch.Tensor, *,
                       norm: tuple[torch.Tensor, float] | None = None, history: torch.Tensor | None = None,
                       pos: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """int8_linear with the argmax of each token's outputs into ``ids`` (plx_int8_linear_argmax).

    ids int64 [tokens]: torch.argmax(y, -1) of the returned y (greedy decoding,
    generate.py:313-320 with top_k = 1).  ``pos`` (0-dim int64 device
    tensor): the kernel then writes ids into ``history`` [tokens, L] (or None)
    at column pos + 1 and advances pos by one.  ``workspace``: from
    int8_linear_argmax_workspace (allocated per call when None).
    """
    _lib.require_device(x, "int8_linear_argmax input")
    if q.dtype != torch.int8 or mu16.dtype != torch.float16 or x.dtype != torch.float32:
        raise ValueError("int8_linear_argmax: int8 q, float16 mu and float32 x")
    rows, cols = q.shape
    if x.shape[-1] != cols or mu16.numel() != rows:
        raise ValueError(f"int8_linear_argmax: x has {x.shape[-1]} features, weight [{rows}, {cols}]")
    xx = x.reshape(-1, cols).contiguous()
    if xx.data_ptr() % 16:
        xx = xx.clone()
    m = xx.shape[0]
    if ids.dtype != torch.long or ids.numel() != m or not ids.is_contiguous():
        raise ValueError(f"int8_linear_argmax: ids must be contiguous int64 with {m} values")
    if history is not None:
        if pos is None or history.dtype != torch.long or history.dim() != 2 or history.shape[0] != m \
                or not history.is_contiguous():
            raise ValueError("int8_linear_argmax: history must be contiguous int64 [tokens, L], with pos")
    if pos is not None and (pos.dtype != torch.long or pos.numel() != 1):
        raise ValueError("int8_linear_argmax: pos must be one int64 value")
    nw, eps = None, 0.0
    if norm is not None:
        nw, eps = norm[0].detach().reshape(-1).contiguous(), float(norm[1])
        if nw.dtype != torch.float32 or nw.numel() != cols:
            raise ValueError(f"int8_linear_argmax: the norm weight must be fp32 with {cols} values")
        if nw.data_ptr() % 16:
            nw = nw.clone()
    if workspace is None:
        workspace = int8_linear_argmax_workspace(rows, m, x.device)
    y = torch.empty((m, rows), dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        st = _lib.lib().plx_int8_linear_argmax(
            _lib.ptr(q.contiguous()), _lib.ptr(mu16.contiguous()), rows, cols, _lib.ptr(xx), m, _lib.ptr(nw), eps,
            _lib.ptr(y), _lib.ptr(ids), _lib.ptr(history), 0 if history is None else history.shape[1], _lib.ptr(pos),
            _lib.ptr(workspace), workspace.numel(), _lib.stream_of(x.device))
    _lib.check(st, "int8_linear_argmax")
    return y.reshape(*x.shape[:-1], rows)


def int8_embed(q: torch.Tensor, mu16: torch.Tensor, ids: torch.Tensor, *, pos_weight: torch.Tensor | None = None,
               pos0: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 [b, t, cols] = W[ids] (+ pos_weight[p0 + i] at step i), one HIP kernel (plx_int8_embed).

    W = q * (mu / 127) in fp16 (PackedInt8Embedding.forward, pollux.py:532-533);
    the position term is the model's pos_emb (pollux.py:691-693), p0 a 0-dim
    int64 device tensor (0 when None).  Ids or positions out of range give NaN rows.
    """
    _lib.require_device(ids, "int8_embed ids")
    if q.dtype != torch.int8 or mu16.dtype != torch.float16:
        raise ValueError("int8_embed: int8 q and float16 mu")
    ii = ids.reshape(ids.shape[0] if ids.dim() > 1 else 1, -1).to(torch.int64).contiguous()
    vocab, cols = q.shape
    pw = None
    if pos_weight is not None:
        pw = pos_weight.detach().contiguous()
        if pw.dtype != torch.float32 or pw.shape[-1] != cols:
            raise ValueError("int8_embed: the position table must be fp32 [positions, cols]")
    p0 = None
    if pos0 is not None:
        p0 = pos0.reshape(()).to(torch.int64)
    out = torch.empty((*ii.shape, cols), dtype=torch.float32, device=ids.device)
    with torch.cuda.device(ids.device):
        st = _lib.lib().plx_int8_embed(_lib.ptr(q.contiguous()), _lib.ptr(mu16.contiguous()), vocab, cols, _lib.ptr(ii),
                                       ii.shape[0], ii.shape[1], _lib.ptr(pw), 0 if pw is None else pw.shape[0],
                                       _lib.ptr(p0), _lib.ptr(out), _lib.stream_of(ids.device))
    _lib.check(st, "int8_embed")
    return out.reshape(*ids.shape, cols)


class _PackedInt8Rows(nn.Module):
    """Shared buffers / materialize of the INT8 periphery layers (pollux.py:508-563)."""

    def _init_rows(self, rows: int, cols: int) -> None:
        self.register_buffer("weight_int8", torch.zeros(rows, cols, dtype=torch.int8))
        self.register_buffer("mu_rows", torch.ones(rows, dtype=torch.float16))
        self._materialized = False

    def materialize(self) -> None:
        if self._materialized:
            return
        weight = dequantize_int8_rows(self.weight_int8, self.mu_rows.to(torch.float16))
        self.weight = nn.Parameter(weight, requires_grad=False)
        del self.weight_int8
        del self.mu_rows
        self._materialized = True


class PackedInt8Embedding(_PackedInt8Rows):
    """Token embedding with INT8 weights and per-row fp16 scales (pollux.py:508-532)."""

    def __init__(self, num_embeddings: int, embedding_dim: int) -> None:
        super().__init__()
        self.num_embeddings = int(num_embeddings)
        self.embedding_dim = int(embedding_dim)
        self._init_rows(self.num_embeddings, self.embedding_dim)

    def forward(self, idx: torch.Tensor) -> torch.Tensor:
        if not self._materialized:
            # gathered and dequantised in one kernel: the values of F.embedding(idx, weight.float())
            return int8_embed(self.weight_int8, self.mu_rows, idx)
        # rows gathered, then cast: the same values as F.embedding(idx, weight.float())
        # (pollux.py:532-533) without casting the whole table per call
        return F.embedding(idx, self.weight).to(dtype=torch.float32)


class PackedInt8Linear(_PackedInt8Rows):
    """Output projection with INT8 weights and per-row fp16 scales (pollux.py:535-563)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = False) -> None:
        super().__init__()
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self._init_rows(self.out_features, self.in_features)
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features))
        else:
            self.register_parameter("bias", None)

    # token counts up to which the INT8 kernels run (plx_int8_linear: the GEMV at one
    # token, the MFMA kernel above); larger batches take the reference's F.linear
    gemv_max_tokens = 1 << 20

    def forward(self, x: torch.Tensor, norm: tuple[torch.Tensor, float] | None = None) -> torch.Tensor:
        """F.linear(n(x), W.to(x.dtype), bias) (pollux.py:562-563); ``norm``: (weight, eps) of an RMSNorm on x, or None.

        Until materialize(), fp32 batches of up to ``gemv_max_tokens`` tokens
        run the INT8 kernels (norm fused in); others take the reference's
        F.linear on the fp16 weight cast to x's dtype (kept for reuse).
        """
        if self.gemv_runs(x):
            return int8_linear(self.weight_int8, self.mu_rows, x, norm=norm)
        if norm is not None:
            x = x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + norm[1]) * norm[0]
        return F.linear(x, self._weight_as(x.dtype), self.bias)

    def gemv_runs(self, x: torch.Tensor) -> bool:
        """Whether forward(x) runs the INT8 kernels (packed, no bias, fp32 x of at most gemv_max_tokens tokens)."""
        return (not self._materialized and self.bias is None and x.dtype == torch.float32
                and x.numel() // max(self.in_features, 1) <= self.gemv_max_tokens
                and self.in_features % 16 == 0 and self.in_features <= 4096)

    def _weight_as(self, dtype: torch.dtype) -> torch.Tensor:
        """weight.to(dtype) (pollux.py:562-563), cast once per dtype and source state, then reused.

        The entry holds the source tensors themselves (compared by identity) and
        their version counters, so replacing the buffers (``load_state_dict``
        on a materialised layer, ``materialize``) or writing them in place
        (``load_state_dict`` on a packed layer copies into the buffers) makes
        the next call cast again.  Tensors made under ``torch.inference_mode``
        keep no version counter: for those an in-place write is not seen, so
        replace such buffers instead.
        """
        if self._materialized and self.weight.dtype == dtype:
            return self.weight
        src = (self.weight,) if self._materialized else (self.weight_int8, self.mu_rows)
        versions = tuple(None if t.is_inference() else t._version for t in src)
        cache = self.__dict__.setdefault("_cast", {})
        hit = cache.get(dtype)
        if hit is not None and len(hit[0]) == len(src) and all(a is b for a, b in zip(hit[0], src)) \
                and hit[1] == versions:
            return hit[2]
        w16 = self.weight if self._materialized else dequantize_int8_rows(self.weight_int8, self.mu_rows)
        w = w16.detach().to(dtype=dtype)
        if not _capturing():  # a cast made under capture is filled only on replay
            cache[dtype] = (src, versions, w)
        return w
