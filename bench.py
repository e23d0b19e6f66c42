#!/usr/bin/env python3
"""Benchmark of the Leech-lattice quantization hot path on one MI355X.

Headline (BASELINE.json metric, config 4): atoms/s of the bulk NN-B quantizer
(castor.py:544-557 semantics: bf16 operands, bf16 scores, lowest index) on
16,777,200 24-d fp32 atoms (209,715 rows of 1920 = 80 atoms per row, the
config's 16,777,216 rounded down to whole rows) whose directions are uniform
on S^23 and whose radius is U(0, 2) * sqrt(32), fed directly as quantizer
input.  One step = ``castor.quantize_indices`` over all of them (fp32 atoms
resident in HBM -> int32 codebook indices).

The JSON line also carries
  roofline      the dominant kernel of that launch, t3_kernel (the structured
                type-3 scorer), against the dense bf16 MFMA peak: its
                algorithmic MFMA flops 2*24*2,048 per atom (the representative
                Golay sign-pattern sums) over its HIP-event kernel time inside
                the timed region (events recorded on the launch stream); the
                VALU issue fraction that binds it (rocprofv3 counters) and its
                HBM traffic from profiles/; beside it t12_kernel's time (the
                structured type-1/2 scorer);
  dense_sweep_baseline  the same quantize with every code swept densely on
                MFMA (nn_kernel: 2*24*196,560 flops per atom);
  dequant_gemv  the metric's second half: the fused dequant-GEMV at d=1920
                (config 5, batch 1) in compressed-stream GB/s and as a fraction
                of HBM peak;
  cpu_baseline  the reference's own CPU path (autocast-bf16 matmul + max in
                chunks of 4096, castor.py:549-557) restated with the same torch
                ops (oracle/torch_ref.py) on a bounded prefix of the same atoms,
                on this host's physical cores;
  parity        that prefix's CPU indices against the GPU's, each disagreement
                classified by the exact oracle (near-tie or not);
  extras        config 2 / 3 requantize steps, pack / unpack / dequant HBM GB/s,
                dequant-GEMM, the fused optimiser step, pack-time NN-P, decode.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "atoms/sec Leech NN quantize (+MFMA util %); dequant-GEMV GB/s at d=1920"
# The dense sweep (NN-T, NN-P, and NN-B with the dense type-3 sweep): every code scored,
# 2 * 24 * 196,560 = 9,434,880 flops per atom (origin free, K padding not counted).
FLOP_PER_ATOM = 2 * 24 * 196_560
# MFMA flops the dense sweep issues per atom: 9,216 tiles of 16 codes (the 98,304
# type-3 codes, one representative per antipodal pair of the others, padding)
# at K = 32 (24 coordinates + 8 zeros) -- 9,437,184.
MFMA_FLOP_ISSUED_PER_ATOM = 2 * 32 * 9216 * 16
# NN-B's default path, the structured scorers: t12_kernel scores the 98,256 type-1 / type-2
# codes from the 759 octad sums of |x| (2 * 24 * 759 = 36,432 algorithmic MFMA flops per
# atom, issued as 48 tiles at K = 32: 49,152) and t3_kernel the 98,304 type-3 codes from
# the 2,048 representative Golay sign-pattern sums (2 * 24 * 2,048 = 98,304 flops per atom,
# issued as 128 tiles: 131,072); both evaluate their few candidate codes exactly on the VALU,
# and that VALU work, not the MFMA, bounds them.
T12_FLOP_PER_ATOM = 2 * 24 * 759
T12_MFMA_ISSUED_PER_ATOM = 2 * 32 * 48 * 16
T3_FLOP_PER_ATOM = 2 * 24 * 2048
T3_MFMA_ISSUED_PER_ATOM = 2 * 32 * 128 * 16
PEAK_BF16_FLOPS = 2.5e15  # MI355X dense bf16 MFMA
PEAK_HBM_BPS = 8.0e12  # MI355X HBM3E
C2_SHAPES = [(3456, 1152), (1152, 1152), (4608, 1152), (1152, 4608)]
C4_ROWS, C4_ATOMS_PER_ROW = 209_715, 80  # 16,777,200 atoms as rows of 1920


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_c2(device, seed=2024):
    import torch

    g = torch.Generator().manual_seed(seed)
    mats = []
    for r, c in C2_SHAPES:
        w = (torch.randn(r, c, generator=g) * 0.02).to(torch.bfloat16).float()
        mats.append(w.to(device))
    return mats


def time_gpu(fn, iters, warmup, rounds=1, warm_s=0.0):
    """Seconds per call: median over `rounds` of the mean over `iters` back-to-back calls.

    Warmup: `warmup` calls, continued until `warm_s` seconds have passed (an
    HBM-bound kernel reaches its steady memory clock only after a sustained load).
    """
    import torch

    t_end = time.perf_counter() + warm_s
    k = 0
    while k < warmup or time.perf_counter() < t_end:
        fn()
        k += 1
        if k % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    if iters <= 0:
        return 0.0
    per = []
    for _ in range(rounds):
        t0 = time.perf_counter()
        for _ in range(iters):
            fn()
        torch.cuda.synchronize()
        per.append((time.perf_counter() - t0) / iters)
    return sorted(per)[len(per) // 2]


def host_cpu():
    """(physical cores this process may run on, CPU model name) from /sys and /proc (lscpu's sources)."""
    cpus = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else list(range(os.cpu_count() or 1))
    cores = set()
    for c in cpus:
        base = Path(f"/sys/devices/system/cpu/cpu{c}/topology")
        try:
            cores.add(((base / "physical_package_id").read_text().strip(), (base / "core_id").read_text().strip()))
        except OSError:
            cores.add(("?", str(c)))
    # lscpu's "Model name" plus the family / model / stepping numbers, which
    # identify the core generation where a virtualised host reports a bare
    # vendor name
    fields = {}
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if ":" not in line:
                if fields:
                    break  # first processor's block only
                continue
            k, v = (t.strip() for t in line.split(":", 1))
            fields.setdefault(k.lower(), v)
    except OSError:
        pass
    model = fields.get("model name", "unknown")
    ids = [f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields]
    if ids:
        model += " (" + ", ".join(ids) + ")"
    return max(1, len(cores)), len(cpus), model


def cpu_baseline(x_gpu, idx_gpu, target_atoms):
    """The reference's CPU path (castor.py:549-557) on the first atoms of the headline input, plus parity.

    Returns (cpu_baseline record, parity record): the same torch ops on the
    host's physical cores, timed; their indices against the GPU's for the same
    atoms, each disagreement classified by the exact oracle (oracle/nn.py).
    """
    import numpy as np
    import torch

    from oracle import nn, torch_ref

    phys, logical, model = host_cpu()
    torch.set_num_threads(phys)
    n = min(int(target_atoms), x_gpu.shape[0])
    x = x_gpu[:n].cpu()
    kp = torch_ref.codebook_tensor()[1:]
    torch_ref.nn_b_indices(x[:4096], kp=kp)  # untimed: first-call setup of the bf16 matmul
    t0 = time.perf_counter()
    idx_cpu = torch_ref.nn_b_indices(x, kp=kp)
    dt = time.perf_counter() - t0
    got = idx_gpu[:n].long().cpu()
    diff = (got != idx_cpu).nonzero().flatten().numpy()
    near = 0
    if len(diff):
        r = nn.quantize(x[torch.from_numpy(diff)].numpy(), "B")
        near = int(r["near_tie"].sum())
    base = {
        "value": n / dt,
        "unit": "atoms/s",
        "cores": phys,
        "kind": "port",
        "sample": f"first {n} atoms of the headline input (config 4): the reference's NN-B CPU path "
        f"(autocast-bf16 matmul + max, chunk 4096, castor.py:549-557) restated with the same torch ops, "
        f"{dt:.1f} s on {phys} threads",
        "cpu_model": model,
        "logical_cpus_available": logical,
    }
    parity = {
        "atoms_compared": n,
        "against": "the reference's NN-B torch ops on the host (oracle/torch_ref.nn_b_indices)",
        "disagree": int(len(diff)),
        "near_tie": near,
        "not_near_tie": int(len(diff)) - near,
        "near_tie_envelope": "24 * 2^-24 * sum|x_i c_i| (any fp32 summation order)",
        "requantize_config1": requantize_parity(x_gpu.device),
    }
    return base, parity


def requantize_parity(device):
    """Config 1 through the fused requantize (row scale + NN-B) against the reference's CPU composition.

    Every atom of the seeded 1152x1152 fp32 N(0, 0.02) weight; disagreements
    classified as near_tie / sigma_ulp / real (oracle/parity.py), with the
    sigma statistics against the stated bar (within 2 fp32 ulp).
    """
    import torch

    from oracle import parity, torch_ref
    from pollux_amd import castor

    g = torch.Generator().manual_seed(1152)
    w = torch.randn(1152, 1152, generator=g) * 0.02
    got = castor.requantize_h24(w.to(device))
    idx_ref, sig_ref, _ = torch_ref.requantize(w)
    c = parity.classify_requantize(w, got["indices"].cpu(), got["sigma"].cpu(), idx_ref, sig_ref)
    c.pop("real_at")
    c["sigma_bar"] = f"row RMS within {parity.SIGMA_BAR_ULP} fp32 ulp of torch's CPU reduction"
    c["case"] = "config 1 (1152x1152 fp32 N(0, 0.02)), every atom, fused requantize vs oracle/torch_ref.requantize"
    return c


def extras(device, iters=24, sets=4):
    """Pack / unpack / dequant at config-4 size, each call on the next of `sets` distinct buffer sets.

    One set is 16,777,200 int64 indices (134 MB) + their packed bytes (37.7 MB);
    4 sets (688 MB) cycle so that a set's buffers were last touched 516 MB of
    traffic earlier, twice the 256 MB Infinity Cache: each call streams from
    HBM.  Dequant writes 805 MB of fp16 per call.  Rates: per Python call
    (median of 5 rounds of `iters` calls, after >= 0.3 s of warmup calls) and
    per kernel (HIP events on the launch stream around every launch).
    """
    import torch

    from pollux_amd import _lib, castor, dequantize_h24

    out = {}
    n = 16_777_200  # config 4: 209,715 rows of 1920 = 80 atoms/row
    rows, cols = 209_715, 1920
    g = torch.Generator(device=device).manual_seed(7)
    idx = [torch.randint(0, 196561, (n,), generator=g, device=device, dtype=torch.int64) for _ in range(sets)]
    packed = [castor.pack_indices(i) for i in idx]
    sig = (torch.rand(rows, generator=g, device=device) * 0.045 + 0.005).half()
    cyc = {"k": 0}

    def rot(fn):
        def call():
            k = cyc["k"] = (cyc["k"] + 1) % sets
            return fn(k)
        return call

    unit = {"pack": (8 + 2.25) * n, "unpack": (2.25 + 8) * n, "dequant": 2.25 * n + 48 * n + 2 * rows}
    calls = {
        "pack": (rot(lambda k: castor.pack_indices(idx[k])), _lib.PROF_PACK),
        "unpack": (rot(lambda k: castor.unpack_indices(packed[k], n)), _lib.PROF_UNPACK),
        "dequant": (rot(lambda k: dequantize_h24(packed[k], sig, rows, cols)), _lib.PROF_DEQUANT),
    }
    for name, (fn, kid) in calls.items():
        t, k_ms = _profiled(fn, iters, kid, warmup=10, rounds=5, warm_s=0.3)
        out[f"{name}_GBps"] = unit[name] / t / 1e9
        out[f"{name}_hbm_frac"] = unit[name] / t / PEAK_HBM_BPS
        out[f"{name}_kernel_us"] = k_ms * 1e3
        out[f"{name}_kernel_GBps"] = unit[name] / (k_ms / 1e3) / 1e9
        out[f"{name}_kernel_hbm_frac"] = unit[name] / (k_ms / 1e3) / PEAK_HBM_BPS
    out["hbm_peak_GBps"] = PEAK_HBM_BPS / 1e9
    out["bytes_per_call"] = {k: int(v) for k, v in unit.items()}
    out["scale"] = (f"16,777,200 indices / atoms (BASELINE config 4 size), rows of 1920; each call on the next of "
                    f"{sets} distinct buffer sets ({sets} x 172 MB, twice the 256 MB Infinity Cache between two "
                    f"touches of a set); per call: median of 5 rounds of {iters} back-to-back calls after >= 0.3 s "
                    "of warmup calls; per kernel: HIP events around every launch on its stream")
    del idx, packed
    return out


def hbm_workload(device, calls):
    """The HBM-bound kernels on rotating buffers, for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs."""
    import torch

    from pollux_amd import castor, dequantize_h24, optim

    n, rows, cols, sets = 16_777_200, 209_715, 1920, 4
    g = torch.Generator(device=device).manual_seed(7)
    idx = [torch.randint(0, 196561, (n,), generator=g, device=device, dtype=torch.int64) for _ in range(sets)]
    packed = [castor.pack_indices(i) for i in idx]
    sig = (torch.rand(rows, generator=g, device=device) * 0.045 + 0.005).half()
    for k in range(calls):
        castor.pack_indices(idx[k % sets])
    for k in range(calls):
        castor.unpack_indices(packed[k % sets], n)
    for k in range(calls):
        dequantize_h24(packed[k % sets], sig, rows, cols)
    torch.cuda.synchronize()
    del idx, packed
    shapes = [(r, c) for r, c in C2_SHAPES]
    states = [_optim_state(device, shapes, g) for _ in range(3)]
    heat = torch.tensor(0.5, device=device)
    for k in range(calls):
        sc = optim.step_scalars(heat, k, optim.width_inertia(1152), device)
        for st in states[k % 3]:
            optim.pollux_h24_step_(*st, heat=heat, step=k, width_inertia=1.0, scalars=sc)
    torch.cuda.synchronize()


def gemv_extras(device, copies=400, m_gemm=64, replays=5):
    """Config 5: fused dequant-GEMV (M=1) and dequant-GEMM (M=64) on [7680,1920] and [1920,7680].

    `copies` calls, each on a distinct packed weight (400 x 1.38 MB = 553 MB,
    more than twice the 256 MB Infinity Cache, so the compressed stream is read
    from HBM), are
    captured in one HIP graph; the graph is replayed and HIP events on the
    replay stream give the device time per call (kernel plus graph dispatch,
    without the Python call overhead).  Replay outputs are checked against an
    eager call.
    """
    import torch

    from pollux_amd import castor, dequant_linear, h24_plane_layout

    out = {}
    for name, (of, inf) in (("up_7680x1920", (7680, 1920)), ("down_1920x7680", (1920, 7680))):
        g = torch.Generator(device=device).manual_seed(of)
        n_atoms = of * inf // 24
        nbytes = (n_atoms + 3) // 4 * 9
        # indices uniform over 0..196,560 (config 5), packed per copy; each copy's plane layout beside it
        pk = torch.empty(copies, nbytes, dtype=torch.uint8, device=device)
        pl = torch.empty(copies, 3 * n_atoms, dtype=torch.int16, device=device)
        for i in range(copies):
            pk[i] = castor.pack_indices(torch.randint(0, 196561, (n_atoms,), generator=g, device=device))
            pl[i] = h24_plane_layout(pk[i], n_atoms)
        sg = (torch.rand(copies, of, generator=g, device=device) * 0.045 + 0.005).half()
        for m, mode, planes in ((1, "exact", False), (m_gemm, "exact", False), (m_gemm, "as_x", False),
                                (1, "exact", True), (m_gemm, "exact", True)):
            x = torch.randn(m, inf, generator=g, device=device).to(torch.bfloat16)

            def call(i):
                return dequant_linear(pk[i], sg[i], of, inf, x, weight_rounding=mode, planes=pl[i] if planes else None)

            eager = [call(i) for i in (0, copies - 1)]
            side = torch.cuda.Stream(device)
            side.wait_stream(torch.cuda.current_stream(device))
            with torch.cuda.stream(side):
                for i in range(3):
                    call(i)
            torch.cuda.current_stream(device).wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                ys = [call(i) for i in range(copies)]
            graph.replay()
            torch.cuda.synchronize()
            if not (torch.equal(ys[0], eager[0]) and torch.equal(ys[-1], eager[1])):
                raise RuntimeError(f"dequant_linear graph replay differs from the eager call ({name}, M={m})")
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(replays):
                graph.replay()
            e1.record()
            e1.synchronize()
            t = e0.elapsed_time(e1) / 1e3 / (replays * copies)
            del graph, ys
            comp = nbytes + 2 * of + 2 * m * inf + 4 * m * of
            key = f"{name}_M{m}" + ("" if mode == "exact" else f"_{mode}") + ("_planes" if planes else "")
            out[f"{key}_us"] = t * 1e6
            out[f"{key}_compressed_GBps"] = comp / t / 1e9
            if planes:  # bytes the call reads from the plane layout (6 B per atom instead of 2.25)
                out[f"{key}_layout_GBps"] = (6 * n_atoms + 2 * of + 2 * m * inf + 4 * m * of) / t / 1e9
            out[f"{key}_dense_equiv_GBps"] = (2 * of * inf) / t / 1e9
            out[f"{key}_TFLOPs"] = 2 * m * of * inf / t / 1e12
        if name == "up_7680x1920":
            out.update(latency_floor(pk, copies, replays))
        del pk, pl
    out["note"] = (f"HIP graph of {copies} calls on distinct packed copies ({copies} x 1.38 MB), replayed {replays}x; "
                   "compressed bytes = packed + sigma16 + x bf16 + y fp32; dense-equivalent = fp16 weight bytes; "
                   "default: exact products with the fp16 weights; _as_x: weights rounded to bf16 first, as the "
                   "reference's literal F.linear(x, W.to(x.dtype)); _planes: the same calls reading each copy's "
                   "plane layout (h24_plane_layout, 6 B per atom, built beforehand), compressed_GBps still on the "
                   "packed stream's bytes, layout_GBps on the bytes actually read")
    return out


POLLUX1920_H24 = (
    [("tok_emb", 50688, 1920), ("pos_emb", 1024, 1920), ("head", 50688, 1920)]
    + [(f"blocks.{i}.{n}", r, c) for i in range(18) for n, r, c in (
        ("attn.q_proj", 1920, 1920), ("attn.k_proj", 1920, 1920), ("attn.v_proj", 1920, 1920),
        ("attn.o_proj", 1920, 1920), ("mlp.fc1", 7680, 1920), ("mlp.fc2", 1920, 7680))]
)  # every >= 2-D H24 tensor pollux_step updates (pollux.py:828-888): 41,369,600 atoms


def _optim_state(device, shapes, g):
    """(p, grad, m, v, latent) per shape: grad N(0, 1e-3), m N(0, 3e-4), v U(0, 1e-6), latent N(0, 0.02)."""
    import torch

    out = []
    for r, c in shapes:
        out.append((torch.empty(r, c, device=device), torch.randn(r, c, generator=g, device=device) * 1e-3,
                    torch.randn(r, c, generator=g, device=device) * 3e-4,
                    torch.rand(r, c, generator=g, device=device) * 1e-6,
                    torch.randn(r, c, generator=g, device=device) * 0.02))
    return out


def optim_extras(device, mats, iters=9, sets=3):
    """Fused optimiser step + requantize (pollux.py:828-888).

    config 2: one step = the four Pollux-1152 latents, per parameter
    (plx_pollux_step_h24, four calls) and batched (plx_pollux_step_h24_batch:
    four update passes, one scoring sweep); each step on the next of `sets`
    distinct optimiser states (3 x 318 MB), so the update streams from HBM.
    The update kernel alone (28 B per element: grad, m, v, latent read; m, v,
    latent written) is timed by HIP events around every launch.
    Pollux-1920: one batched step over every H24 tensor of the model (18
    layers' q/k/v/o/fc1/fc2, tok_emb, pos_emb, head: 41.4 M atoms).
    """
    import torch

    from pollux_amd import _lib, optim

    g = torch.Generator(device=device).manual_seed(11)
    shapes = [tuple(w.shape) for w in mats]
    states = [_optim_state(device, shapes, g) for _ in range(sets)]
    heat = torch.tensor(0.5, device=device)
    inertia = optim.width_inertia(1152)
    counter = torch.zeros((), dtype=torch.int64, device=device)  # the optimiser's device-resident step counter
    cyc = {"k": 0}

    def step():
        cyc["k"] = (cyc["k"] + 1) % sets
        sc = optim.step_scalars(heat, counter, inertia, device)  # once per step, as pollux.py:815-820
        for st in states[cyc["k"]]:
            optim.pollux_h24_step_(*st, heat=heat, step=counter, width_inertia=inertia, scalars=sc)
        counter.add_(1)

    def step_batched():
        cyc["k"] = (cyc["k"] + 1) % sets
        sc = optim.step_scalars(heat, counter, inertia, device)
        optim.pollux_h24_step_many_(states[cyc["k"]], heat=heat, step=counter, width_inertia=inertia, scalars=sc)
        counter.add_(1)

    n_el = sum(r * c for r, c in shapes)
    t, adam_ms = _profiled(step, iters, _lib.PROF_ADAM, warmup=3)
    t_b, _ = _profiled(step_batched, iters, _lib.PROF_ADAM, warmup=3)
    adam_bytes = 28 * n_el / len(shapes)  # per launch, averaged over the four matrices
    out = {
        "step_ms": t * 1e3,
        "atoms_per_s": n_el / 24 / t,
        "batched_step_ms": t_b * 1e3,
        "batched_atoms_per_s": n_el / 24 / t_b,
        "update_kernel_us_avg": adam_ms * 1e3,
        "update_kernel_GBps": adam_bytes / (adam_ms / 1e3) / 1e9,
        "update_kernel_hbm_frac": adam_bytes / (adam_ms / 1e3) / PEAK_HBM_BPS,
        "update_bytes_per_element": 28,
        "note": f"config-2 latents; step_ms: 4 x plx_pollux_step_h24 (fused Adam/speed-cap/decay update + "
                f"requantize); batched: plx_pollux_step_h24_batch; each step on the next of {sets} distinct "
                "optimiser states (318 MB each); update kernel timed by HIP events on its stream",
    }
    del states
    torch.cuda.empty_cache()
    # a whole Pollux-1920 step's H24 tensors
    shapes = [(r, c) for _, r, c in POLLUX1920_H24]
    state = _optim_state(device, shapes, g)
    inertia = optim.width_inertia(1920)
    atoms = sum(r * c for r, c in shapes) // 24

    def full_step():
        sc = optim.step_scalars(heat, counter, inertia, device)
        optim.pollux_h24_step_many_(state, heat=heat, step=counter, width_inertia=inertia, scalars=sc)
        counter.add_(1)

    t_f, kms = _scorer_profiled(full_step, 3, warmup=1)
    out["pollux1920_step"] = {
        "atoms": atoms, "step_ms": t_f * 1e3, "atoms_per_s": atoms / t_f, **kms,
        "note": "plx_pollux_step_h24_batch over all 111 H24 tensors of Pollux-1920 (18 x q/k/v/o 1920x1920, "
                "fc1 7680x1920, fc2 1920x7680; tok_emb and head 50688x1920; pos_emb 1024x1920): 111 update "
                "passes and one pass of the structured scorers; synthetic state (latent N(0, 0.02))"}
    del state
    torch.cuda.empty_cache()
    return out


def pack_time_extras(mats, iters=5):
    """Pack-time NN-P quantizer (pack.py:139-180) on the config-2 weights: atoms/s.

    NN-P scores fp32 atoms exactly (three bf16 MFMA parts per tile) and
    rescans its candidates in fp64, so it does ~3x the MFMA work of NN-B.
    """
    from pollux_amd import pack

    t = time_gpu(lambda: [pack.quantize_h24_layer(w) for w in mats], iters, 2)
    n = sum(w.numel() for w in mats) // 24
    return {"atoms_per_s": n / t, "ms_per_layer": t * 1e3,
            "mfma_issue_frac_of_bf16_peak": 3 * MFMA_FLOP_ISSUED_PER_ATOM * n / t / PEAK_BF16_FLOPS,
            "note": "quantize_h24_layer (NN-P + sigma16 + 18-bit pack) on the four config-2 weights"}


def json_from_profiles(name):
    """A JSON summary committed under profiles/ (rocprofv3 counter runs), or {} when absent or unreadable."""
    p = ROOT / "profiles" / name
    if p.exists():
        try:
            return json.loads(p.read_text())
        except (ValueError, OSError):
            return {}
    return {}


def traffic_from_profiles(name):
    """HBM bytes per launch of a kernel measured by two rocprofv3 --pmc runs (committed under profiles/)."""
    return json_from_profiles(name).get("hbm_bytes_per_launch")


def make_c4(device, seed=404):
    """16,777,200 atoms, directions uniform on S^23, radius U(0, 2) * sqrt(32)."""
    import numpy as np
    import torch

    n = C4_ROWS * C4_ATOMS_PER_ROW
    g = torch.Generator(device=device).manual_seed(seed)
    d = torch.randn(n, 24, generator=g, device=device)
    x = d / d.norm(dim=1, keepdim=True) * (torch.rand(n, 1, generator=g, device=device) * 2.0 * np.sqrt(32.0))
    del d
    return x


def _profiled(fn, iters, kernel=0, warmup=0, rounds=1, warm_s=0.0):
    """(seconds per call, selected kernel's ms per launch) of fn, the kernel timed by HIP events.

    kernel: a PLX_PROF_* id (0 = nn_kernel, 1 pack, 2 unpack, 3 dequant, 4 the optimiser update, 5 t3_kernel,
    6 t12_kernel); the
    events are recorded on the kernel's launch stream around every launch of the timed calls.
    """
    import ctypes

    import torch

    from pollux_amd import _lib

    lib = _lib.lib()
    if warmup or warm_s:
        time_gpu(fn, 0, warmup, 1, warm_s)
    torch.cuda.synchronize()
    _lib.check(lib.plx_profile_select(kernel), "plx_profile_select")
    _lib.check(lib.plx_profile_begin(), "plx_profile_begin")
    t = time_gpu(fn, iters, 0, rounds)
    tot_ms, launches = ctypes.c_double(), ctypes.c_int64()
    _lib.check(lib.plx_profile_end(ctypes.byref(tot_ms), ctypes.byref(launches)), "plx_profile_end")
    _lib.check(lib.plx_profile_select(0), "plx_profile_select")
    return t, tot_ms.value / max(1, launches.value)


def _scorer_profiled(fn, iters, mode="bf16", warmup=0):
    """(seconds per call, {kernel: ms per launch}) of fn over iters calls, the scoring kernels timed by HIP events:
    NN-B's structured scorers (t3_kernel, t12_kernel), or nn_kernel (the dense sweep of the other modes)."""
    from pollux_amd import _lib

    if mode == "bf16":
        t, t3 = _profiled(fn, iters, _lib.PROF_T3, warmup=warmup)
        _, t12 = _profiled(fn, iters, _lib.PROF_T12)
        return t, {"t3_kernel_ms_avg": t3, "t12_kernel_ms_avg": t12}
    t, nn = _profiled(fn, iters, _lib.PROF_NN, warmup=warmup)
    return t, {"nn_kernel_ms_avg": nn}


def sweep_extras(device, mode="bf16", steps=10):
    """The other BASELINE quantizer configs: the config-2 and config-3 requantize steps.

    config 2: the fused requantize (row scale, NN-B, pack, reconstructed
    weight) of the four Pollux-1152 latents, per latent (the reference's
    per-parameter loop) and as one batched sweep.  config 3: the same step on
    the four Pollux-1920 latents, then quantize_indices on their lattice-unit
    atoms with 5% replaced by midpoints of code pairs at raw inner product 16
    (+ N(0, 1e-3) noise) and 5% by random directions at norm sqrt 2 (the
    origin boundary).
    """
    import numpy as np
    import torch

    from pollux_amd import castor

    out = {}
    mats2 = make_c2(device)
    atoms2 = sum(r * c // 24 for r, c in C2_SHAPES)

    def step2():
        for w in mats2:
            castor.requantize_h24(w, mode=mode)

    step2()
    t, kms = _scorer_profiled(step2, steps, mode)
    out["config2_requantize"] = {
        "atoms": atoms2, "ms_per_step": t * 1e3, "atoms_per_s": atoms2 / t, **kms,
        "note": "fused row scale + NN-B + pack + reconstructed weight of QKV 3456x1152, O 1152x1152, up 4608x1152, "
                "down 1152x4608 (bf16-rounded N(0, 0.02) master weights), one requantize_h24 call per latent "
                "(pollux.py:828-884); kernel times: the average over the four launches"}
    t_b = time_gpu(lambda: castor.requantize_h24_many(mats2, mode=mode), steps, 2)
    out["config2_requantize_batched"] = {
        "ms_per_step": t_b * 1e3, "atoms_per_s": atoms2 / t_b,
        "note": "the same step as one requantize_h24_many call (plx_requantize_batch, one sweep for all four)"}
    del mats2

    shapes = [(5760, 1920), (1920, 1920), (7680, 1920), (1920, 7680)]
    g = torch.Generator(device=device).manual_seed(303)
    mats = [(torch.randn(r, c, generator=g, device=device) * 0.02).to(torch.bfloat16).float() for r, c in shapes]
    atoms = sum(r * c // 24 for r, c in shapes)

    def step():
        for w in mats:
            castor.requantize_h24(w, mode="bf16")

    step()
    t, kms = _scorer_profiled(step, 5)
    out["config3_requantize"] = {
        "atoms": atoms, "ms_per_step": t * 1e3, "atoms_per_s": atoms / t, **kms,
        "note": "fused row scale + NN-B + pack + reconstructed weight of QKV 5760x1920, O 1920x1920, up 7680x1920, "
                "down 1920x7680 (bf16-rounded N(0, 0.02) master weights)"}

    # lattice-unit atoms (pollux.py:876-882) with the boundary stress
    xs = []
    for w in mats:
        sigma = castor.row_rms_from_matrix(w)
        xs.append((w / sigma.unsqueeze(1) / castor.s_lattice).reshape(-1, 24))
    x = torch.cat(xs)
    rng = torch.Generator(device=device).manual_seed(304)
    perm = torch.randperm(atoms, generator=rng, device=device)
    mid_at, near_at = perm[: atoms // 20], perm[atoms // 20: atoms // 10]
    cb = castor.get_h24_codebook(device, torch.float32)
    raw = torch.round(cb * np.sqrt(8.0)).to(torch.int32)
    a = torch.randint(1, 196561, (mid_at.numel(),), generator=rng, device=device)
    b = torch.zeros_like(a)
    todo = torch.arange(a.numel(), device=device)
    while todo.numel():  # a partner at raw inner product 16 (the true-Leech contact)
        cand = torch.randint(1, 196561, (todo.numel(), 64), generator=rng, device=device)
        ip = (raw[cand] * raw[a[todo]].unsqueeze(1)).sum(-1)
        hit = ip == 16
        ok = hit.any(dim=1)
        b[todo[ok]] = cand[ok].gather(1, hit[ok].int().argmax(dim=1, keepdim=True)).squeeze(1)
        todo = todo[~ok]
    x[mid_at] = 0.5 * (cb[a] + cb[b]) + torch.randn(a.numel(), 24, generator=rng, device=device) * 1e-3
    dirs = torch.randn(near_at.numel(), 24, generator=rng, device=device)
    x[near_at] = dirs / dirs.norm(dim=1, keepdim=True) * np.sqrt(2.0)
    castor.quantize_indices(x, mode="bf16")
    t, kms = _scorer_profiled(lambda: castor.quantize_indices(x, mode="bf16"), 5)
    out["config3_stress_quantize"] = {
        "atoms": atoms, "ms": t * 1e3, "atoms_per_s": atoms / t, **kms,
        "note": "quantize_indices (NN-B) on the config-3 lattice atoms with 5% contact-pair midpoints and 5% "
                "near-origin atoms (more near-ties for the exact rescoring pass)"}
    return out


def random_packed_pollux(device):
    """(model, generator, payload): packed Pollux-1920 (18 layers, d 1920, vocab 50,688), random packed weights."""
    import torch

    from pollux_amd import castor
    from pollux_amd.model import PackedPolluxModel
    from pollux_amd.plx import PLX_FORMAT

    cfg = {"n_layers": 18, "n_heads": 80, "d_head": 24, "n_embd": 1920, "vocab_size": 50688,
           "tokenizer_vocab_size": 50257, "seq_len": 1024}
    g = torch.Generator(device=device).manual_seed(1920)
    d, v = cfg["n_embd"], cfg["vocab_size"]
    state = {"pos_emb.weight": torch.randn(cfg["seq_len"], d, generator=g, device=device) * 0.02,
             "ln_f.weight": torch.ones(d, device=device)}
    for name, rows in (("tok_emb", v), ("head", v)):
        state[name + ".weight_int8"] = torch.randint(-127, 128, (rows, d), generator=g, device=device,
                                                     dtype=torch.int8)
        state[name + ".mu_rows"] = (torch.rand(rows, generator=g, device=device) * 0.1 + 0.01).half()
    shapes = {"attn.q_proj": (d, d), "attn.k_proj": (d, d), "attn.v_proj": (d, d), "attn.o_proj": (d, d),
              "mlp.fc1": (4 * d, d), "mlp.fc2": (d, 4 * d)}
    for i in range(cfg["n_layers"]):
        p = f"blocks.{i}."
        for k in ("ln1.weight", "ln2.weight"):
            state[p + k] = torch.ones(d, device=device)
        state[p + "attn.q_ln.weight"] = torch.ones(24, device=device)
        state[p + "attn.k_ln.weight"] = torch.ones(24, device=device)
        for name, (o, i_) in shapes.items():
            idx = torch.randint(0, 196561, (o * i_ // 24,), generator=g, device=device)
            state[p + name + ".packed_weights"] = castor.pack_indices(idx)
            state[p + name + ".sigma_rows"] = (torch.rand(o, generator=g, device=device) * 0.045 + 0.005).half()
    payload = {"format": PLX_FORMAT, "config": cfg, "codebook_fingerprint": castor.codebook_fingerprint(),
               "state_dict": state}
    return PackedPolluxModel.from_packed_checkpoint(payload, device), g, payload


def decode_workload(device, n_tokens, prompt_len=64, batch=1):
    """Greedy graph decode of n_tokens after a prompt per sequence (random packed Pollux-1920, `batch`
    sequences per step); returns a summary line."""
    import torch

    from pollux_amd.model import GraphDecoder

    model, g, _ = random_packed_pollux(device)
    prompt = torch.randint(0, 50257, (batch, prompt_len), generator=g, device=device)
    with torch.inference_mode():
        dec = GraphDecoder(model, batch=batch, greedy=True)
        first = dec.prefill(prompt).argmax(-1)
        t = dec.decode_greedy(first, 8)[:, -1]
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        dec.decode_greedy(t, n_tokens)
        e1.record()
        e1.synchronize()
    ms = e0.elapsed_time(e1) / n_tokens
    return (f"packed decode (graph with the argmax inside, batch {batch}, prompt {prompt_len}): {ms:.4f} ms per step "
            f"over {n_tokens} steps ({batch * 1e3 / ms:.0f} tokens/s)")


def decode_extras(device, prompt_len=64, new_tokens=128):
    """Packed Pollux-1920 decoder (18 layers, d 1920, vocab 50,688; random packed weights): tokens/s at batch 1.

    graph: GraphDecoder (KV cache, one HIP graph replay per token, greedy
    argmax on the device); eager: the same cached decode as plain module
    calls; recompute: the reference's loop (generate.py:313-315), the full
    prefix per token, once with the packed layers fused and once the
    reference's way (materialised fp16 weights cast to fp32 by every
    F.linear call, pollux.py:507).
    """
    import torch

    from pollux_amd.model import GraphDecoder, PackedPolluxModel

    model, g, payload = random_packed_pollux(device)
    prompt = torch.randint(0, 50257, (1, prompt_len), generator=g, device=device)

    def timed(fn, n):
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        fn(n)
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) / 1e3 / n

    out = {}
    with torch.inference_mode():
        dec = GraphDecoder(model, batch=1)
        nxt = dec.prefill(prompt).argmax(-1)

        def run_graph(n):
            t = nxt
            for _ in range(n):
                t = dec.decode(t).argmax(-1)

        run_graph(4)
        dec.prefill(prompt)
        t_graph = timed(run_graph, new_tokens)
        del dec
        gdec = GraphDecoder(model, batch=1, greedy=True)
        g_first = gdec.prefill(prompt).argmax(-1)
        gdec.decode_greedy(g_first, 4)
        gdec.prefill(prompt)
        t_greedy = timed(lambda n: gdec.decode_greedy(g_first, n), new_tokens)
        del gdec
        cache = model.new_cache(1)
        first = model.prefill(prompt, cache)[:, -1].argmax(-1)

        def run_eager(n):
            t = first
            for _ in range(n):
                t = model.decode(t, cache).argmax(-1)

        t_eager = timed(run_eager, 32)

        def run_prefill(n):
            for _ in range(n):
                c = model.new_cache(1)
                model.prefill(prompt, c, last_only=True)

        run_prefill(1)  # untimed: the first new cache (283 MB) may need a fresh device allocation
        t_prefill = timed(run_prefill, 8)
        pdec = GraphDecoder(model, batch=1)
        pdec.prefill(prompt)  # captures the 64-position prefill graph (and the step graph)
        t_prefill_graph = timed(lambda n: [pdec.prefill(prompt) for _ in range(n)], 8)
        del pdec
        seq = torch.cat([prompt, prompt[:, :1]], dim=1)
        model(seq)  # untimed: first use of each shape (library kernels load their code on first use)
        t_recompute = timed(lambda n: [model(seq)[:, -1].argmax(-1) for _ in range(n)], 4)
        del cache
        dense = PackedPolluxModel.from_packed_checkpoint(payload, device, materialize=True)
        dense(seq)  # untimed, as above (hipBLASLt's first call per GEMM shape)
        t_dense = timed(lambda n: [dense(seq)[:, -1].argmax(-1) for _ in range(n)], 4)
        del dense
        # last: the batch-16 decoder's cache (4.5 GB) and graph pools stay with the allocator afterwards
        prompts16 = torch.randint(0, 50257, (16, prompt_len), generator=g, device=device)
        bdec = GraphDecoder(model, batch=16, greedy=True)
        b_first = bdec.prefill(prompts16).argmax(-1)
        bdec.decode_greedy(b_first, 4)
        bdec.prefill(prompts16)
        t_batch16 = timed(lambda n: bdec.decode_greedy(b_first, n), new_tokens)
        del bdec
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    out["graph_cached_tokens_per_s"] = 1.0 / t_graph
    out["graph_cached_ms_per_token"] = t_graph * 1e3
    out["graph_greedy_tokens_per_s"] = 1.0 / t_greedy
    out["graph_greedy_ms_per_token"] = t_greedy * 1e3
    out["graph_greedy_batch16_tokens_per_s"] = 16.0 / t_batch16
    out["graph_greedy_batch16_ms_per_step"] = t_batch16 * 1e3
    out["eager_cached_tokens_per_s"] = 1.0 / t_eager
    out["prefill_graph_ms"] = t_prefill_graph * 1e3
    out["prefill_eager_ms"] = t_prefill * 1e3
    out["recompute_fused_tokens_per_s"] = 1.0 / t_recompute
    out["recompute_reference_dense_tokens_per_s"] = 1.0 / t_dense
    out["note"] = (f"batch 1, prompt {prompt_len} tokens, {new_tokens} greedy tokens (graph: one replay per token, "
                   f"torch argmax on the host's stream between replays; graph_greedy: the argmax and the token "
                   f"feedback inside the captured step, no host work per token; batch16: 16 sequences per "
                   f"step); prefill: the prompt into the "
                   f"cache with the last position's logits (time to first token), replayed from GraphDecoder's "
                   f"graph for the padded length or run eagerly into a new cache; recompute rows at a "
                   f"{prompt_len + 1}-token prefix; random packed weights (valid indices), fp32 activations")
    return out


def gemv_workload(device, replays, copies=400, m=1):
    """The config-5 calls of gemv_extras (one token, or m tokens) as graphs of `copies` calls, each replayed
    `replays` times (for rocprofv3 counter runs: up then down, packed stream then plane layout)."""
    import torch

    from pollux_amd import castor, dequant_linear, h24_plane_layout

    for of, inf in ((7680, 1920), (1920, 7680)):
        g = torch.Generator(device=device).manual_seed(of)
        n_atoms = of * inf // 24
        pk = torch.empty(copies, (n_atoms + 3) // 4 * 9, dtype=torch.uint8, device=device)
        pl = torch.empty(copies, 3 * n_atoms, dtype=torch.int16, device=device)
        for i in range(copies):
            pk[i] = castor.pack_indices(torch.randint(0, 196561, (n_atoms,), generator=g, device=device))
            pl[i] = h24_plane_layout(pk[i], n_atoms)
        sg = (torch.rand(copies, of, generator=g, device=device) * 0.045 + 0.005).half()
        x = torch.randn(m, inf, generator=g, device=device).to(torch.bfloat16)
        for planes in (False, True):
            def call(i):
                return dequant_linear(pk[i], sg[i], of, inf, x, planes=pl[i] if planes else None)

            side = torch.cuda.Stream(device)
            side.wait_stream(torch.cuda.current_stream(device))
            with torch.cuda.stream(side):
                for i in range(3):
                    call(i)
            torch.cuda.current_stream(device).wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                ys = [call(i) for i in range(copies)]
            for _ in range(replays):
                graph.replay()
            torch.cuda.synchronize()
            del graph, ys
        del pk, pl


def latency_floor(pk, copies, replays):
    """What one graph-replayed call costs at least: a node, and a node plus one HBM round trip.

    The same graph timing as gemv_extras on the smallest kernel of the library
    (plx_unpack_indices on one 9-byte group: one load, one 32-byte store):
    node_us with every call reading the same group (an L2 hit), latency_floor_us
    with call i reading the first group of packed copy i (copies of 1.38 MB
    apart), each replay timed alone right after 640 MB of writes to another
    buffer have evicted those groups from the L2s and the 256 MB MALL, so every
    call's load goes to HBM.
    """
    import torch

    from pollux_amd import castor

    res = {}
    flush = torch.empty(160 * 1024 * 1024, dtype=torch.float32, device=pk.device)
    for key, rot in (("node_us", False), ("latency_floor_us", True)):
        src = [pk[i if rot else 0][:9] for i in range(copies)]
        side = torch.cuda.Stream(pk.device)
        side.wait_stream(torch.cuda.current_stream(pk.device))
        with torch.cuda.stream(side):
            for i in range(3):
                castor.unpack_indices(src[i], 4)
        torch.cuda.current_stream(pk.device).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            ys = [castor.unpack_indices(src[i], 4) for i in range(copies)]
        graph.replay()
        torch.cuda.synchronize()
        if not torch.equal(ys[-1], castor.unpack_indices(src[-1], 4)):
            raise RuntimeError("unpack graph replay differs from the eager call")
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        tot = 0.0
        for _ in range(replays):
            if rot:
                flush.fill_(1.0)
            e0.record()
            graph.replay()
            e1.record()
            e1.synchronize()
            tot += e0.elapsed_time(e1)
        res[key] = tot * 1e3 / (replays * copies)
        del graph, ys
    del flush
    return res


def gemv_headline(gemv):
    """The metric's "dequant-GEMV GB/s at d=1920" from the config-5 batch-1 rows of gemv_extras."""
    rows = {}
    tot_bytes = tot_s = 0.0
    for name, (of, inf) in (("up_7680x1920", (7680, 1920)), ("down_1920x7680", (1920, 7680))):
        us = gemv[f"{name}_M1_us"]
        nbytes = (of * inf // 24 + 3) // 4 * 9 + 2 * of + 2 * inf + 4 * of
        rows[name] = {"us_per_call": us, "compressed_bytes": nbytes, "GBps": nbytes / (us * 1e-6) / 1e9,
                      "hbm_frac": nbytes / (us * 1e-6) / PEAK_HBM_BPS}
        tot_bytes += nbytes
        tot_s += us * 1e-6
    pl_us = {name: gemv.get(f"{name}_M1_planes_us") for name in rows}
    plane = None
    if all(v is not None for v in pl_us.values()):
        params = sum(of * inf for of, inf in ((7680, 1920), (1920, 7680)))
        packed_bits = sum(((of * inf // 24 + 3) // 4 * 9) * 8 + 16 * of for of, inf in ((7680, 1920), (1920, 7680)))
        plane = {
            "us_per_call": pl_us,
            "GBps_on_packed_stream": tot_bytes / (sum(pl_us.values()) * 1e-6) / 1e9,
            "resident_bits_per_param": {"packed": packed_bits / params,
                                        "packed_plus_plane_layout": (packed_bits + 48 * params // 24) / params},
            "note": "the same calls reading the plane layout (h24_plane_layout: 6 B per atom built once beside "
                    "the 2.25 B packed stream), which removes the per-atom codebook-table gathers",
        }
    floor = gemv.get("latency_floor_us")
    if floor:
        for r in rows.values():
            r["latency_floor_frac"] = floor / r["us_per_call"]
    return {
        "GBps": tot_bytes / tot_s / 1e9,
        "unit": "GB/s",
        "hbm_frac": tot_bytes / tot_s / PEAK_HBM_BPS,
        "peak": PEAK_HBM_BPS / 1e9,
        "latency_floor_us": floor,
        "node_us": gemv.get("node_us"),
        "latency_floor_note": "one graph node plus one HBM round trip, measured in the same run (plx_unpack_indices "
        "on one 9-byte group of a distinct packed copy per call); node_us: the same with an L2-resident group. "
        "At one token the call is latency-bound: hbm_frac is far from 1 by construction, latency_floor_frac is "
        "what one call can reach",
        "per_matrix": rows,
        "plane_layout": plane,
        "workload": "BASELINE config 5 at batch 1: y = x W^T with W the packed 18-bit indices + fp16 row scales "
        "of a 7680x1920 and a 1920x7680 weight (never materialised), bf16 x, fp32 accumulation and output",
        "bytes": "compressed stream: packed indices + sigma16 + x (bf16) + y (fp32) per call",
        "timing": "HIP graph of 400 calls on distinct packed copies (553 MB, twice the 256 MB MALL), replayed 5x",
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-atoms", type=int, default=262_144, help="CPU baseline sample size (atoms)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--mode", default="bf16", choices=["bf16", "bf16-dense", "fp32"])
    ap.add_argument(
        "--pmc-workload",
        choices=["c4", "c2", "hbm", "gemv", "gemm"],
        default=None,
        help="for rocprofv3 --pmc runs: 5 copies of a 256 MiB fp32 tensor (HBM-counter calibration), then "
        "--steps headline (c4) steps, config-2 requantize steps (c2), or (hbm) --steps calls each of pack, "
        "unpack and dequant at config-4 size on 4 rotating buffer sets and of the config-2 optimiser step on "
        "3 rotating states, or (gemv) --steps replays of the config-5 one-token graphs (400 calls each on "
        "distinct packed copies: up and down, packed stream then plane layout; gemm: the same at 64 tokens); "
        "prints nothing",
    )
    ap.add_argument(
        "--decode-workload",
        type=int,
        default=0,
        metavar="N",
        help="for rocprofv3 runs: the packed Pollux-1920 decoder only (prefill 64 tokens, then N greedy tokens "
        "replayed from its HIP graph); prints one line with ms/token",
    )
    ap.add_argument("--decode-batch", type=int, default=1, metavar="B",
                    help="with --decode-workload: B sequences per decode step")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py measures one GPU only: this build's hot path (Leech quantize / pack / dequant) is "
            "benchmarked per device (atoms and rows shard with no exchange; the packed indices are what "
            "ranks would all-gather), and no multi-GPU run is made.",
            file=sys.stderr,
        )
        return 2

    import torch

    from pollux_amd import _lib, castor

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm device", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    lib = _lib.lib()
    with torch.cuda.device(dev):
        _lib.check(lib.plx_device_init(), "plx_device_init")

    if args.decode_workload:
        print(decode_workload(dev, args.decode_workload, batch=args.decode_batch), flush=True)
        return 0

    if args.pmc_workload:
        src = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device=dev)  # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        del src, dst
        if args.pmc_workload in ("gemv", "gemm"):
            gemv_workload(dev, args.steps, m=1 if args.pmc_workload == "gemv" else 64)
        elif args.pmc_workload == "hbm":
            hbm_workload(dev, args.steps)
        elif args.pmc_workload == "c2":
            mats = make_c2(dev)
            for _ in range(args.steps):
                for w in mats:
                    castor.requantize_h24(w, mode=args.mode)
        else:
            x = make_c4(dev)
            for _ in range(args.steps):
                castor.quantize_indices(x, mode=args.mode)
        torch.cuda.synchronize()
        return 0

    x = make_c4(dev)
    atoms = x.shape[0]

    def step():
        return castor.quantize_indices(x, mode=args.mode)

    log(f"[bench] warmup {args.warmup} steps, workload config 4 ({atoms} atoms/step)")
    for _ in range(args.warmup):
        idx = step()
    torch.cuda.synchronize()
    structured = args.mode == "bf16"
    # the dominant kernel's launches are timed by HIP events on their stream inside the timed region
    _lib.check(lib.plx_profile_select(_lib.PROF_T3 if structured else _lib.PROF_NN), "plx_profile_select")
    _lib.check(lib.plx_profile_begin(), "plx_profile_begin")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        idx = step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    import ctypes

    tot_ms, launches = ctypes.c_double(), ctypes.c_int64()
    _lib.check(lib.plx_profile_end(ctypes.byref(tot_ms), ctypes.byref(launches)), "plx_profile_end")
    _lib.check(lib.plx_profile_select(_lib.PROF_NN), "plx_profile_select")
    ms_per_step = elapsed / args.steps * 1e3
    value = atoms * args.steps / elapsed
    log(f"[bench] timed {args.steps} steps: {ms_per_step:.3f} ms/step, {value:.4g} atoms/s")

    kernel_s = tot_ms.value / 1e3
    kernel_avg_ms = tot_ms.value / max(1, launches.value)
    fpa = T3_FLOP_PER_ATOM if structured else FLOP_PER_ATOM
    issued = T3_MFMA_ISSUED_PER_ATOM if structured else MFMA_FLOP_ISSUED_PER_ATOM
    achieved = fpa * atoms * args.steps / kernel_s if kernel_s > 0 else 0.0
    counters = json_from_profiles("quantize_c4_counters.json") if structured else {}
    roofline = {
        "bound": "mfma",
        "achieved": achieved / 1e12,
        "peak": PEAK_BF16_FLOPS / 1e12,
        "unit": "TFLOP/s",
        "frac": achieved / PEAK_BF16_FLOPS,
        "traffic": traffic_from_profiles("t3_kernel_c4_traffic.json" if structured else "nn_kernel_c4_dense_traffic.json"),
        "kernel": "t3_kernel (structured type-3 scorer: 128 Golay sign-pattern tiles on bf16 16x16x32 MFMA, the "
        "candidate words' 24 positions on the VALU)" if structured else
        "nn_kernel (bf16 16x16x32 MFMA scoring + running max over 9,216 tiles)",
        "kernel_launches": int(launches.value),
        "kernel_avg_ms": kernel_avg_ms,
        "flop_per_atom": fpa,
        "flop_per_launch": fpa * atoms,
        "mfma_issue_frac": issued * atoms * args.steps / kernel_s / PEAK_BF16_FLOPS if kernel_s > 0 else 0.0,
    }
    if structured:
        # the type-1/2 scorer, and the dense sweep the two structured scorers replace
        _, t12_ms = _profiled(step, 3, _lib.PROF_T12)
        t_d, nn_d = _profiled(lambda: castor.quantize_indices(x, mode="bf16-dense"), 3, _lib.PROF_NN, warmup=1)
        roofline["flop_per_atom_note"] = (
            "2 * 24 flops per representative Golay sign pattern (2,048 per atom; each also scores its "
            "complement); the candidates' exact evaluation is VALU work, which binds the kernel: valu_issue_frac")
        t3c = counters.get("t3_kernel", {})
        if t3c:
            roofline["valu_issue_frac"] = t3c.get("valu_issue_frac")
            roofline["valu_note"] = counters.get("valu_note")
        roofline["kernel_step_share"] = kernel_avg_ms / ms_per_step
        # the whole step priced on the dense contraction's work (2 * 24 * 196,560 flops per atom, the
        # figure the dense sweep's roofline uses): above 1 means the step beats the dense MFMA roofline
        roofline["dense_equivalent_frac"] = FLOP_PER_ATOM * atoms / (ms_per_step / 1e3) / PEAK_BF16_FLOPS
        roofline["dense_equivalent_note"] = (
            "the step's atoms/s x 9,434,880 flops per atom (every code's 24-term dot product) over the 2.5 PF "
            "dense bf16 peak: the dense sweep's ceiling is 2.65e8 atoms/s, which the structured scorers exceed "
            "because they skip ~99% of the codes exactly, not by computing faster")
        roofline["t12_kernel_avg_ms"] = t12_ms
        roofline["t12_kernel_step_share"] = t12_ms / ms_per_step
        roofline["t12_kernel_mfma_frac"] = T12_FLOP_PER_ATOM * atoms / (t12_ms / 1e3) / PEAK_BF16_FLOPS
        if counters.get("t12_kernel"):
            roofline["t12_kernel_valu_issue_frac"] = counters["t12_kernel"].get("valu_issue_frac")
        result_dense = {
            "ms_per_step": t_d * 1e3, "atoms_per_s": atoms / t_d, "nn_kernel_avg_ms": nn_d,
            "nn_kernel_frac": FLOP_PER_ATOM * atoms / (nn_d / 1e3) / PEAK_BF16_FLOPS,
            "nn_kernel_mfma_issue_frac": MFMA_FLOP_ISSUED_PER_ATOM * atoms / (nn_d / 1e3) / PEAK_BF16_FLOPS,
            "note": "the same workload with every code swept densely (9,216 tiles, 2 * 24 * 196,560 flops per "
                    "atom; castor mode 'bf16-dense', PLX_NN_DENSE_TYPE3): the baseline the structured scorers "
                    "are measured against; identical indices off near-ties"}

    result = {
        "metric": METRIC,
        "value": value,
        "unit": "atoms/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "BASELINE config 4: bulk NN-B quantize of 16,777,200 24-d fp32 atoms (209,715 rows of "
            "1920, the config's 16,777,216 rounded down to whole rows), directions uniform on S^23, radius "
            "U(0, 2) * sqrt(32), fed directly as quantizer input; fp32 atoms in HBM -> int32 indices",
            "atoms_per_step": atoms,
            "call": "castor.quantize_indices (plx_quantize: operand prep, t12_kernel structured type-1/2 scorer, "
            "t3_kernel structured type-3 scorer, pick)" if structured else
            "castor.quantize_indices (plx_quantize: operand prep, nn_kernel scoring sweep, resolve)",
            "nn_mode": "NN-T (fp32 scores)" if args.mode == "fp32" else "NN-B (bf16 scores)",
            "seed": 404,
        },
        "roofline": roofline,
    }
    if structured:
        result["dense_sweep_baseline"] = result_dense
    log("[bench] dequant-GEMV / GEMM at config 5")
    gemv = gemv_extras(dev)
    result["dequant_gemv"] = gemv_headline(gemv)
    if not args.no_cpu_baseline:
        log(f"[bench] CPU baseline + parity on {args.cpu_atoms} atoms")
        result["cpu_baseline"], result["parity"] = cpu_baseline(x, idx, args.cpu_atoms)
    del x, idx
    torch.cuda.empty_cache()
    if not args.no_extras:
        log("[bench] extras: config 2 / 3 steps, pack / unpack / dequant at config-4 scale, optimiser, decode")
        result["extras"] = extras(dev)
        result["extras"]["dequant_linear"] = gemv
        result["extras"]["quantizer_sweeps"] = sweep_extras(dev, args.mode)
        mats = make_c2(dev)
        result["extras"]["optimizer_step"] = optim_extras(dev, mats)
        result["extras"]["pack_time_nn_p"] = pack_time_extras(mats)
        del mats
        result["extras"]["packed_decode"] = decode_extras(dev)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
