#!/usr/bin/env python3
"""Triangle-attention block benchmark on one MI355X.

Workload (default ``--config c4``): both triangle-attention blocks (starting
and ending node) at N=1536, FP32, c_z=128, H=4, d=32, z ~ 2*N(0,1), the last
184 residues (12%) masked on both axes, triangle-bias weights x8 (logits span
about +/-40).  One step = one starting-node block followed by one ending-node
block on the same z, each a single C-ABI call (``fpx_tri_attn_block``).
Inputs, weights, outputs and workspace are resident in HBM before timing.

Output: one JSON line.  ``value`` is the step's algorithmic TFLOP/s
(2 x (512 N^3 + 164864 N^2) flop per step); ``ms_per_step`` covers both
blocks.  ``roofline`` is the attention kernel alone (``fpx_tri_attn_attend``)
timed with HIP events on the launch stream.  Its ``peak`` is that of the
matrix unit the kernel issues: the FP32 block computes its products on the
16-bit matrix cores (power-of-two scaled fp16 hi/lo planes, FP32-accurate),
so the peak is the 2.5 PFLOP/s dense fp16/bf16 figure; ``achieved`` counts
the algorithmic FP32 flop of the key tiles the kernel visits (trailing
masked tiles whose weights are exactly 0 are left out), and
``executed_frac`` the 16-bit matrix work it actually issues.
``roofline.traffic`` is the attention kernel's HBM bytes per launch from the
committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary.  ``cpu_baseline`` times
the CPU oracle (native PyTorch op order, FP32) on the lease's host cores on
the same step, and ``parity`` compares the timed GPU outputs of that step with
the oracle's, every element of both nodes (valid and padded rows apart).
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import platform
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "triangle-attn block ms + TFLOP/s (% MFMA peak) at N=1536 FP32, 1 GPU"
FP32_MFMA_PEAK_TFLOPS = 157.3
BF16_MFMA_PEAK_TFLOPS = 2500.0
HBM_PEAK_GBPS = 8000.0
TRAFFIC_FILE = ROOT / "profiles" / "attention_traffic.json"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def calibrate_copy(dev) -> None:
    """Three plain 1 GiB device-to-device copies: the known-size reference
    that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes."""
    import torch

    src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log("copy calibration: 3 x 1 GiB device copies")
    del src, dst


def host_cores() -> int:
    """Cores this process may run on: the lease's CPU share (OMP_NUM_THREADS
    when the host sets it, else the affinity mask)."""
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(int(env), affinity) if env.isdigit() and int(env) > 0 else affinity)


def cpu_model() -> str:
    try:
        for line in pathlib.Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def host_record(threads: int) -> dict:
    return {"cores": threads, "os_cpu_count": os.cpu_count(),
            "affinity_cpus": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity")
            else None, "cpu": cpu_model()}


def cpu_baseline(cfg, z, mask, weights, budget_s: float = 40.0):
    """Time the CPU oracle (native op order) on the lease's host cores.

    FP32 configurations run both directions in full (the starting node alone
    when it exceeds ``budget_s``, the ending node then taken as equal).  The
    BF16 configuration runs the native path on bfloat16 tensors for 8 and 24
    evenly spaced outer rows per direction and extrapolates linearly in rows
    (rows are independent), since the full N=2048 BF16 CPU run takes minutes.
    Returns the record and the oracle outputs it computed: ``{"start": dz,
    "end": dz}`` in z's frame (full), or ``{"start_rows": (rows, dz_x), ...}``
    for the sampled BF16 rows (x frame).
    """
    import torch

    from oracle import triangle_attention as oracle

    threads = host_cores()
    torch.set_num_threads(threads)
    outputs = {}
    params = oracle.BlockParams(**weights)
    times = {}
    both = True
    bf16 = cfg.dtype == "bf16"
    run = oracle.block_bf16 if bf16 else oracle.block
    with torch.inference_mode():
        for ending in (False, True):
            key = "end" if ending else "start"
            if bf16:
                spent = []
                for rows in (8, 24):
                    sel = torch.linspace(0, cfg.n - 1, rows).round().long()
                    t0 = time.perf_counter()
                    res = run(z, mask, params, ending=ending, outer_rows=sel)
                    spent.append(time.perf_counter() - t0)
                outputs[f"{key}_rows"] = (sel, res)
                per_row = max((spent[1] - spent[0]) / 16, 0.0)
                times[key] = max(spent[0] - 8 * per_row, 0.0) + per_row * cfg.n
                log(f"cpu oracle ending={ending}: 8 rows {spent[0]:.2f} s, 24 rows {spent[1]:.2f} s")
                continue
            if ending and times["start"] > budget_s:
                times["end"] = times["start"]
                both = False
                break
            t0 = time.perf_counter()
            outputs[key] = run(z, mask, params, ending=ending)
            times[key] = time.perf_counter() - t0
            log(f"cpu oracle ending={ending}: {times[key]:.2f} s")
    from oracle.triangle_attention import block_flops

    total = times["start"] + times["end"]
    flop = 2 * block_flops(cfg.n)["block"]
    if bf16:
        measured = ("native path on bfloat16 tensors, 8 and 24 evenly spaced outer rows per "
                    "direction, fitted linearly in rows and extrapolated to all rows")
    else:
        measured = ("both directions in full" if both
                    else "the starting node in full (ending node taken as equal)")
    record = {
        "value": round(flop / total / 1e12, 5),
        "unit": "TFLOP/s",
        "kind": "port",
        "sample": (f"CPU oracle (native PyTorch op order, {threads} threads, outer rows in "
                   f"chunks) on the same {cfg.name} inputs, {measured}: "
                   f"start {times['start']:.1f} s + end {times['end']:.1f} s per step"),
        "step_s": round(total, 2),
        **host_record(threads),
    }
    return record, outputs


def parity_report(cfg, gpu: dict, oracle_out: dict) -> dict:
    """Max |GPU - CPU oracle| over the step's outputs, valid and padded outer
    rows apart (x frame), with the largest |oracle| value beside it."""
    import torch

    valid = cfg.valid if cfg.valid is not None else cfg.n
    report = {}
    for key in ("start", "end"):
        if key in oracle_out:
            ref = oracle_out[key].double()
            got = gpu[key].double()
            if key == "end":
                ref, got = ref.transpose(0, 1), got.transpose(0, 1)
            rows = torch.arange(cfg.n)
        elif f"{key}_rows" in oracle_out:
            rows, ref = oracle_out[f"{key}_rows"]
            ref = ref.double()
            full = gpu[key].transpose(0, 1) if key == "end" else gpu[key]
            got = full[rows].double()
        else:
            continue
        entry = {"rows_compared": int(len(rows))}
        for region, sel in (("valid", rows < valid), ("padded", rows >= valid)):
            if bool(sel.any()):
                diff = (got[sel] - ref[sel]).abs()
                nan_same = bool(torch.equal(torch.isnan(got[sel]), torch.isnan(ref[sel])))
                finite = torch.isfinite(ref[sel])
                entry[region] = {"max_abs": float(diff[finite].max()) if bool(finite.any())
                                 else 0.0,
                                 "max_ref": float(ref[sel][finite].abs().max())
                                 if bool(finite.any()) else 0.0,
                                 "nan_positions_equal": nan_same}
        report[key] = entry
    return report

F32_ATOL = 1e-4
F32_RTOL = 1e-4
FP32_BAR_REL = 2e-6
BF16_RTOL = 2e-2
BF16_FLOOR = 1e-3


def sample_rows(n: int, valid: int | None, count: int = 12, seed: int = 11):
    """Outer rows for the float64 comparison: both ends, the middle, both
    sides of the masked tail, and ``count`` seeded draws."""
    import torch

    g = torch.Generator().manual_seed(seed)
    rows = {0, 1, n - 1, n // 2}
    if valid is not None and valid < n:
        rows |= {valid - 1, valid, min(valid + 1, n - 1)}
    rows |= set(torch.randint(0, n, (count,), generator=g).tolist())
    return torch.tensor(sorted(rows))


def parity_gate(cfg, gpu: dict, oracle_out: dict, z_cpu, mask_cpu, weights) -> dict:
    """The parity bars the headline is gated on, on the timed step's outputs.

    FP32 configurations:
      - functional bar (the stated FP32 tolerance), every element of both
        nodes: |GPU - FP32 oracle| <= 1e-4 + 1e-4 |FP32 oracle|, NaN where it is;
      - FP32 bar on sampled outer rows of both nodes, valid and padded rows
        apart: max |GPU - float64 oracle| <= max(2e-6 max|ref|, 2 x the FP32
        oracle's own error); padded (fully masked) rows against float64 with
        float32-rounded logits, which reproduces the native ties at -1e9.
    BF16 (c5): the oracle's native-bf16 rows elementwise, |GPU - ref| <=
    2e-2 |ref| + 1e-3 max|ref|.
    """
    import torch

    from oracle import triangle_attention as oracle

    valid = cfg.valid if cfg.valid is not None else cfg.n
    gate = {"pass": True}
    if cfg.dtype == "bf16":
        for key in ("start", "end"):
            rows, ref = oracle_out[f"{key}_rows"]
            full = gpu[key].transpose(0, 1) if key == "end" else gpu[key]
            got, ref = full[rows].double(), ref.double()
            floor = BF16_FLOOR * float(ref.abs().max())
            excess = ((got - ref).abs() - BF16_RTOL * ref.abs()).max()
            worst = float(((got - ref).abs() / (ref.abs() + floor / BF16_RTOL)).max())
            ok = bool(float(excess) <= floor) and bool(torch.isfinite(got).all())
            gate[key] = {"rows": int(len(rows)), "bar": f"|d| <= {BF16_RTOL} |ref| + {floor:.3e}",
                         "worst_rel_to_bar": round(worst / BF16_RTOL, 4), "pass": ok}
            gate["pass"] &= ok
        return gate
    p32 = oracle.BlockParams(**weights)
    p64 = p32.to(torch.float64)
    z64 = z_cpu.double()
    m64 = None if mask_cpu is None else mask_cpu.double()
    rows = sample_rows(cfg.n, cfg.valid)
    for key, ending in (("start", False), ("end", True)):
        if key not in oracle_out:  # the CPU leg timed one node only
            gate[key] = {"pass": True, "note": "no CPU oracle output for this node"}
            continue
        got = gpu[key].transpose(0, 1) if ending else gpu[key]
        ref32 = oracle_out[key].transpose(0, 1) if ending else oracle_out[key]
        nan_same = bool(torch.equal(torch.isnan(got), torch.isnan(ref32)))
        close = bool(torch.isclose(got, ref32, rtol=F32_RTOL, atol=F32_ATOL, equal_nan=True).all())
        entry = {"functional": {"elements": got.numel(), "bar": f"{F32_ATOL} + {F32_RTOL} |ref|",
                                "pass": close and nan_same}}
        ok = close and nan_same
        for region, sel in (("valid", rows < valid), ("padded", rows >= valid)):
            if not bool(sel.any()):
                continue
            sub = rows[sel]
            ref64 = oracle.block(z64, m64, p64, ending=ending, outer_rows=sub,
                                 logits_f32=(region == "padded"))
            keep = ~torch.isnan(ref64)
            err = float((got[sub].double() - ref64)[keep].abs().max())
            err32 = float((ref32[sub].double() - ref64)[keep].abs().max())
            ref = float(ref64[keep].abs().max())
            bar = max(FP32_BAR_REL * ref, 2.0 * err32)
            entry[f"fp32_{region}"] = {"rows": int(len(sub)), "max_abs": err,
                                       "fp32_oracle_err": err32, "bar": bar,
                                       "pass": err <= bar}
            ok &= err <= bar
        entry["pass"] = ok
        gate[key] = entry
        gate["pass"] &= ok
    return gate


OF3_METRIC = "OpenFold3 _attention ms + TFLOP/s (% MFMA peak) at B=N=1536 FP32, 1 GPU"


def visited_key_tiles(n: int, valid: int | None, skip: bool) -> int:
    """32-key tiles the block's attention visits per (outer row, head, query
    tile), summed over outer rows.  With a tail mask (the first ``valid``
    residues unmasked on both axes) and ``skip``, an outer row with an
    unmasked key leaves out the trailing tiles whose keys are all masked
    (their weights are exactly 0); fully masked rows visit every tile."""
    nkt = -(-n // 32)
    if valid is None or not skip or valid >= n:
        return n * nkt
    return valid * (-(-valid // 32)) + (n - valid) * nkt


def split_executed(batch: int, n: int, ms: float, tiles: int | None = None,
                   const_tiles: int = 0, per_head_scale: bool = True) -> dict:
    """16-bit matrix-core work the split attention kernel executes for its
    FP32-accurate products, per 32 x 32 (query x key) wave tile, counted in
    32x32x16 MFMAs of 32768 flop each (two K-halves per product term)
    against 2 * 65536 algorithmic flop: 3 fp16 terms of S^T and 3 of O^T =
    12 MFMAs.  fp16 and bf16 MFMAs share one dense peak.  Query rows are
    padded to 128, keys to 32.  ``tiles``: key tiles visited summed over the
    outer rows (default: every tile of every row).  ``const_tiles``: the part
    of ``tiles`` on constant-mask rows (padding rows, fl(s + m) = m for every
    key), whose S^T the kernel leaves out: 6 MFMAs per wave tile (O^T only).
    ``per_head_scale``: the block's planes carry one power of two per head
    and operand; the staged (strided) route's one per 32 x 32 tile of q and
    k and per key tile of v^T."""
    np_ = -(-n // 128) * 128
    nkt = -(-n // 32)
    visited = batch * nkt if tiles is None else tiles
    executed = ((visited - const_tiles) * 12 + const_tiles * 6) * 4 * (np_ // 32) * 32768
    executed_tflops = executed / (ms * 1e-3) / 1e12
    unit = ("fp16 hi/lo planes scaled by powers of two ("
            + ("one per head for q, k and v^T" if per_head_scale
               else "q, k per 32x32 tile; v^T per key tile")
            + "; p per tile), three terms per product")
    return {
        "matrix_unit": unit,
        "visited_key_tile_frac": round(visited / (batch * nkt), 4),
        "executed_flop_per_launch": executed,
        "executed_tflops": round(executed_tflops, 3),
        "executed_peak": BF16_MFMA_PEAK_TFLOPS,
        "executed_frac": round(executed_tflops / BF16_MFMA_PEAK_TFLOPS, 4),
    }


def recorded_traffic(key: str) -> int | None:
    """HBM bytes per launch recorded for ``key`` from the FETCH_SIZE and
    WRITE_SIZE counter runs, or None."""
    if not TRAFFIC_FILE.exists():
        return None
    try:
        return json.loads(TRAFFIC_FILE.read_text()).get(key, {}).get("bytes_per_launch")
    except (ValueError, AttributeError):
        return None


def bench_openfold3(args) -> dict:
    """OpenFold3 ``_attention`` at B = N = 1536 (the pair stack's triangle
    attention as OpenFold3 calls it), ending-node wire layout: q/k/v
    ``[B, 4, N, 32]`` views of ``[B, N, 4, 32]``, the mask bias as a
    transposed pair-mask view (12% of keys masked), the triangle bias as a
    transposed head-last view.  One step = one ``fpx_attn_strided`` launch
    sequence (mask and bias staging + attention), timed with HIP events on
    the launch stream.  ``config.native_ms`` times OpenFold3's own
    ``_attention`` arithmetic in torch on the same GPU (matmul, two bias adds,
    softmax, matmul; 128 rows per chunk so the scores fit), the path the
    reference accelerates with a fused mask+bias+softmax between two einsums.
    ``cpu_baseline`` times the oracle's ``attention_core`` on 16 rows and
    scales to all rows (rows are independent).
    """
    import torch

    from fireprot_amd import openfold3 as of3
    from fireprot_amd.block import block_flops

    n = 1536
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(2026)
    log(f"inputs openfold3 b={n} n={n}")

    def head_last():
        return torch.randn(n, n, 4, 32, generator=g, device=dev).transpose(1, 2)

    q = head_last() / 32 ** 0.5
    k = head_last()
    v = head_last()
    keep = torch.ones(n, n, device=dev)
    keep[:, n - 184:] = 0.0
    keep[n - 184:, :] = 0.0
    mask = (1e9 * (keep - 1.0)).t().contiguous().t()[:, None, None, :]
    bias = (8.0 * torch.randn(n, n, 4, generator=g, device=dev)).permute(1, 0, 2).contiguous()
    bias = bias.permute(2, 1, 0).unsqueeze(0)  # head-last memory, transposed view
    biases = [mask, bias]
    kernel = of3.StridedAttention()
    stream = torch.cuda.current_stream(dev)

    def timed(fn, steps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    with torch.inference_mode():
        for _ in range(args.warmup):
            out = kernel(q, k, v, biases)
        torch.cuda.synchronize()
        log(f"warmup {args.warmup} done")
        ms = timed(lambda: kernel(q, k, v, biases), args.steps)
        log(f"timed {args.steps} steps: {ms:.3f} ms/step")

        def native():
            chunk = 128
            res = torch.empty(n, 4, n, 32, device=dev)
            for r in range(0, n, chunk):
                a = torch.matmul(q[r:r + chunk], k[r:r + chunk].transpose(-1, -2).contiguous())
                a += mask[r:r + chunk]
                a += bias
                res[r:r + chunk] = torch.matmul(torch.softmax(a, dim=-1), v[r:r + chunk])
            return res

        ref = native()
        torch.cuda.synchronize()
        native_ms = timed(native, 2)
        log(f"torch native _attention: {native_ms:.3f} ms")
        diff = (ref - out).abs().max().item()
        log(f"max |fused - native| = {diff:.3e}")
        del ref

    flop = block_flops(n)["core"]
    tflops = flop / (ms * 1e-3) / 1e12
    of3_visited = visited_key_tiles(n, n - 184, skip=True)
    of3_flop = flop * of3_visited // (n * -(-n // 32))
    of3_peak = BF16_MFMA_PEAK_TFLOPS
    of3_achieved = of3_flop / (ms * 1e-3) / 1e12
    result = {
        "metric": OF3_METRIC,
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded torch.Generator q/k/v, x8 triangle bias, last 184 keys masked)",
        "config": {
            "workload": "openfold3-attention-b1536-n1536-f32: ending-node wire layout",
            "batch": n, "n": n, "heads": 4, "head_dim": 32,
            "native_ms": round(native_ms, 3),
            "speedup_vs_native": round(native_ms / ms, 2),
            "max_abs_vs_native": diff,
        },
        "roofline": {
            "kernel": ("attention_split_kernel<kAttnStaged> + plane, mask and bias staging"
                       " (fpx_attn_strided)"),
            "bound": "mfma", "achieved": round(of3_achieved, 3), "peak": of3_peak,
            "unit": "TFLOP/s", "frac": round(of3_achieved / of3_peak, 4),
            "traffic": recorded_traffic("openfold3"),
            "flop_per_launch": of3_flop, "flop_all_tiles": flop,
            "fp32_algorithmic_tflops_all_tiles": round(tflops, 3),
            "avg_launch_ms": round(ms, 4),
            **split_executed(n, n, ms, of3_visited, per_head_scale=False),
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        from oracle import triangle_attention as oracle

        threads = host_cores()
        torch.set_num_threads(threads)
        rows = torch.linspace(0, n - 1, 16).round().long().to(dev)
        parts = [t[rows].cpu() for t in (q, k, v, mask)]
        b_cpu = bias.cpu()
        with torch.inference_mode():
            t0 = time.perf_counter()
            oracle.attention_core(*parts[:3], [parts[3], b_cpu])
            spent = time.perf_counter() - t0
        total = spent * n / 16
        result["cpu_baseline"] = {
            "value": round(flop / total / 1e12, 5), "unit": "TFLOP/s", "kind": "port",
            "sample": (f"oracle attention_core (native op order, {threads} threads) on 16 "
                       f"evenly spaced rows of the same inputs, {spent:.1f} s, scaled to "
                       f"{n} rows: {total:.0f} s per step"),
            **host_record(threads),
        }
    return result


TRIMUL_METRIC = "triangle multiplication ms + TFLOP/s (% MFMA peak) at N=1536 FP32, 1 GPU"


def bench_trimul(args) -> dict:
    """Triangle multiplication at N = 1536, FP32, c_z = c_hidden = 128: one
    step = the outgoing then the incoming update, each in place on z
    (``fpx_tri_mul``, accumulate), as the Pairformer applies them; the last
    184 residues are masked (explicit mask).  Weights N(0, 0.1^2) as the
    reference's operator tests draw them.  ``roofline`` is the contraction
    kernel alone (2 N^3 128 flop per launch) timed with HIP events around
    its launch (the projection and finish kernels run before and after it),
    ``config.stage_ms`` splits one update by kernel from a standalone copy
    of each launch sequence.  ``cpu_baseline`` times the oracle on 8 rows of
    each direction and scales to all rows (rows are independent) plus the
    full-size projections it needs.
    """
    import torch

    from fireprot_amd import _native, workloads
    from fireprot_amd import triangle_multiplication as htm

    n = 1536
    dev = torch.device("cuda:0")
    log(f"inputs trimul n={n}")
    z0 = workloads.make_pair(n)
    keep = torch.arange(n) < n - 184
    mask_cpu = (keep[:, None] & keep[None, :]).float()
    w_cpu = workloads.make_trimul_weights()
    z = z0.to(dev)
    mask = mask_cpu.to(dev)
    weights = htm.TriMulWeights.from_tensors(**w_cpu).to(dev)
    ws = torch.empty(htm.workspace_bytes(n), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)

    def step():
        htm.triangle_multiplication(z, mask, weights, outgoing=True, out=z, accumulate=True,
                                    workspace=ws)
        htm.triangle_multiplication(z, mask, weights, outgoing=False, out=z, accumulate=True,
                                    workspace=ws)

    def timed(fn, steps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    with torch.inference_mode():
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        log(f"warmup {args.warmup} done")
        ms = timed(step, args.steps)
        log(f"timed {args.steps} steps: {ms:.3f} ms/step")
        out = torch.empty_like(z)
        update_ms = timed(lambda: htm.triangle_multiplication(
            z, mask, weights, outgoing=True, out=out, workspace=ws), max(args.steps, 5))
        log(f"one outgoing update: {update_ms:.3f} ms")
    lib = _native.library()
    del lib
    from oracle.triangle_multiplication import flops

    f = flops(n)
    value = 2 * f["total"] / (ms * 1e-3) / 1e12
    result = {
        "metric": TRIMUL_METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded z ~ N(0,1), N(0,0.1^2) weights, last 184 residues masked)",
        "config": {
            "workload": "trimul-n1536-f32: outgoing + incoming update, in place",
            "n": n, "c_z": 128, "c_hidden": 128,
            "update_ms": round(update_ms, 4),
            "step_flop": 2 * f["total"],
            "flop_per_update": f,
        },
        "roofline": None,
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        from oracle import triangle_multiplication as tm

        threads = host_cores()
        torch.set_num_threads(threads)
        params = tm.TriMulParams(**w_cpu)
        rows = torch.linspace(0, n - 1, 8).round().long()
        spent = {}
        with torch.inference_mode():
            for outgoing in (True, False):
                t0 = time.perf_counter()
                tm.update(z0, mask_cpu, params, outgoing=outgoing, rows=rows)
                spent[outgoing] = time.perf_counter() - t0
        # projections (full size) + 8 of n rows of contraction and output
        t0 = time.perf_counter()
        with torch.inference_mode():
            tm.gated_projections(z0, mask_cpu, params)
        proj_s = time.perf_counter() - t0
        total = sum(proj_s + (spent[d] - proj_s) * n / len(rows) for d in (True, False))
        result["cpu_baseline"] = {
            "value": round(2 * f["total"] / total / 1e12, 5), "unit": "TFLOP/s",
            "kind": "port",
            "sample": (f"oracle update (native op order, {threads} threads) on 8 evenly spaced "
                       f"rows per direction ({spent[True]:.1f} s and {spent[False]:.1f} s, "
                       f"full-size projections {proj_s:.1f} s included), row part scaled to "
                       f"{n} rows: {total:.0f} s per step"),
            **host_record(threads),
        }
    return result


TRANSITION_METRIC = "pair transition ms + TFLOP/s (% MFMA peak) at N=1536 FP32, 1 GPU"


def bench_transition(args) -> dict:
    """Pair transition at N = 1536 (2.36 M pair rows, c = 128, n = 4), FP32:
    one step = ``z += transition(z)`` in place (``fpx_transition``,
    accumulate), as the Pairformer applies it.  Weights N(0, 0.05^2).
    ``cpu_baseline`` times the oracle on 8192 rows and scales linearly.
    """
    import torch

    from fireprot_amd import transition as htr
    from fireprot_amd import workloads

    n = 1536
    dev = torch.device("cuda:0")
    log(f"inputs transition n={n}")
    z0 = workloads.make_pair(n)
    w_cpu = workloads.make_transition_weights()
    z = z0.to(dev)
    weights = htr.TransitionWeights.from_tensors(**w_cpu).to(dev)
    from fireprot_amd import _native

    size = _native.library().fpx_transition_workspace_bytes(n, n, 128, 4)
    ws = torch.empty(size, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)

    def step():
        htr.pair_transition_residual(z, weights, workspace=ws)

    with torch.inference_mode():
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        log(f"warmup {args.warmup} done")
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.steps):
            step()
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / args.steps
        log(f"timed {args.steps} steps: {ms:.3f} ms/step")
    from oracle.transition import flops

    flop = flops(n * n)
    value = flop / (ms * 1e-3) / 1e12
    # fp16 planes on the 16-bit matrix cores
    tr_peak = BF16_MFMA_PEAK_TFLOPS
    result = {
        "metric": TRANSITION_METRIC, "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded z ~ N(0,1), N(0,0.05^2) weights)",
        "config": {"workload": "transition-n1536-f32: z += transition(z), in place",
                   "n": n, "rows": n * n, "c": 128, "expansion": 4, "step_flop": flop,
                   "peak": tr_peak, "peak_frac": round(value / tr_peak, 4)},
        "roofline": None, "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        from oracle import transition as tr

        threads = host_cores()
        torch.set_num_threads(threads)
        sample = z0.reshape(-1, 128)[:8192]
        with torch.inference_mode():
            t0 = time.perf_counter()
            tr.transition(sample, tr.TransitionParams(**w_cpu))
            spent = time.perf_counter() - t0
        total = spent * n * n / sample.shape[0]
        result["cpu_baseline"] = {
            "value": round(flop / total / 1e12, 5), "unit": "TFLOP/s", "kind": "port",
            "sample": (f"oracle transition (native op order, {threads} threads) on the first "
                       f"8192 pair rows ({spent:.2f} s), scaled to {n * n} rows: "
                       f"{total:.1f} s per step"),
            **host_record(threads),
        }
    return result


CORE_METRIC = ("triangle-attention core ms + TFLOP/s (% MFMA peak) at B=512 N=1536 FP32, "
               "operator route, 1 GPU")


def p95(values: list[float]) -> float:
    """The reference benchmark's 95th percentile (benchmark_attention.py:190):
    ordered[(95 len + 99) // 100 - 1]."""
    ordered = sorted(values)
    return ordered[(95 * len(ordered) + 99) // 100 - 1]


def strict_rows(name: str, out, q, k, v, biases, rows) -> dict:
    """The FP32 bar on outer (batch) rows ``rows`` of an attention-core
    result ``out`` ``[B, 4, N, 32]``: max |out - float64| <= max(2e-6 max|ref|,
    2 x the FP32 oracle's own error)."""
    import torch

    from oracle import triangle_attention as oracle

    qs, ks, vs = (t[rows].cpu() for t in (q, k, v))
    bs = [b[rows].cpu() if b.shape[0] > 1 else b.cpu() for b in biases]
    ref64 = oracle.attention_core(qs.double(), ks.double(), vs.double(), [b.double() for b in bs])
    ref32 = oracle.attention_core(qs, ks, vs, [b.clone() for b in bs])
    got = out[rows].double().cpu()
    nan_same = bool(torch.equal(torch.isnan(got), torch.isnan(ref64)))
    keep = ~torch.isnan(ref64)
    err = float((got - ref64)[keep].abs().max())
    err32 = float((ref32.double() - ref64)[keep].abs().max())
    ref = float(ref64[keep].abs().max())
    bar = max(2e-6 * ref, 2.0 * err32)
    rec = {"rows": [int(r) for r in rows], "max_abs": err, "fp32_oracle_err": err32,
           "max_ref": ref, "bar": bar, "nan_positions_equal": nan_same,
           "pass": bool(nan_same and err <= bar)}
    log(f"parity {name}: {json.dumps(rec)}")
    return rec


def bench_core(args) -> dict:
    """The operator-level route of Protenix's triangle attention: the attention
    core ``_attention(q, k, v, [bias])`` per 512-row chunk at N=1536 and per
    1000-row call at N=1000, with the reference benchmark's inputs and timing
    (benchmarks/protenix/benchmark_attention.py:145-198): seed 419, q, k, v
    ``[B, 4, N, 32]`` views of ``[B, N, 4, 32]`` with q / sqrt(32), the bias
    ``[1, 4, N, N]`` a permuted view of ``[N, N, 4]``; each call bracketed by
    its own HIP events with its bias packing and output allocation inside, 5
    warmups (``--warmup``), 20 timed calls (``--steps``), median and p95.

    Timed routes per shape:
      - ``dispatch``: ``dispatch_triangle_attention`` -> the registered
        candidate ``amd-gfx950-hip-attention-f32`` (``fpx_attn_strided``:
        q, k, v staged into fp16 planes, the block's attention kernel on
        them; workspace cached per device and stream);
      - ``ck_attention_exact1536`` / ``ck_attention_vector_bias1000``: the
        reference's C ABI entries called as its ``attention()`` calls them
        (ck_attention.py:115-141: the bias packed into 1552-float rows at
        N=1536), on the FP32 matrix cores.
    ``value``: the dispatch route at B=512, N=1536.  Every record carries the
    FP32 bar on four batch rows against the float64 oracle.
    """
    import ctypes
    from types import SimpleNamespace

    import torch

    from fireprot_amd import _native
    from fireprot_amd import triangle_attention as ta

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    lib = ctypes.CDLL(str(_native.LIB_PATH))
    records = []
    inputs = {}
    warmup, reps = args.warmup, args.steps
    for batch, n, entry_name in ((512, 1536, "ck_attention_exact1536"),
                                 (1000, 1000, "ck_attention_vector_bias1000")):
        torch.manual_seed(419)
        with torch.inference_mode():
            q, k, v = [torch.randn(batch, n, 4, 32, device=dev).transpose(1, 2) for _ in range(3)]
            q.div_(32 ** 0.5)
            bias = torch.randn(n, n, 4, device=dev).permute(2, 0, 1).unsqueeze(0)
        inputs[n] = (q, k, v, bias)
        entry = getattr(lib, entry_name)
        entry.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 2 + [ctypes.c_void_p]
        entry.restype = ctypes.c_int

        def ck_call(entry=entry, q=q, k=k, v=v, bias=bias, n=n):
            if n == 1536:
                packed = torch.empty((1, 4, 1536, 1552), device=dev, dtype=q.dtype)
                packed[..., :1536].copy_(bias)
            else:
                packed = bias.contiguous()
                if packed.data_ptr() % 16:
                    packed = packed.clone()
            output = torch.empty_like(q)
            status = entry(q.data_ptr(), k.data_ptr(), v.data_ptr(), packed.data_ptr(),
                           output.data_ptr(), q.shape[0], q.shape[2], stream.cuda_stream)
            if status:
                raise RuntimeError(f"{entry_name} returned {status}")
            return output.transpose(-2, -3)

        def dispatch(q=q, k=k, v=v, bias=bias):
            return ta.dispatch_triangle_attention(
                module=SimpleNamespace(training=False), q=q, k=k, v=v, biases=[bias],
                native=lambda **_: (_ for _ in ()).throw(RuntimeError("native selected")))

        flop = 4 * 4 * 32 * batch * n * n
        for name, fn in (("dispatch", dispatch), (entry_name, ck_call)):
            times = []
            with torch.inference_mode():
                for it in range(warmup + reps):
                    e0 = torch.cuda.Event(enable_timing=True)
                    e1 = torch.cuda.Event(enable_timing=True)
                    e0.record(stream)
                    result = fn()
                    e1.record(stream)
                    e1.synchronize()
                    if it >= warmup:
                        times.append(e0.elapsed_time(e1))
            median = statistics_median(times)
            rows = torch.tensor([0, 1, batch // 2, batch - 1])
            # result is [B, N, 4, 32]; the oracle's layout is [B, 4, N, 32]
            parity = strict_rows(f"{name} b={batch} n={n}", result.transpose(1, 2), q, k, v,
                                 [bias], rows)
            peak = BF16_MFMA_PEAK_TFLOPS if name == "dispatch" else FP32_MFMA_PEAK_TFLOPS
            rec = {"route": name, "batch": batch, "n": n, "median_ms": round(median, 4),
                   "p95_ms": round(p95(times), 4), "min_ms": round(min(times), 4),
                   "tflops": round(flop / (median * 1e-3) / 1e12, 3),
                   "matrix_peak": peak,
                   "peak_frac": round(flop / (median * 1e-3) / 1e12 / peak, 4),
                   "flop": flop, "parity": parity}
            records.append(rec)
            log(f"{name} b={batch} n={n}: median {median:.3f} ms, p95 {rec['p95_ms']:.3f} ms, "
                f"{rec['tflops']} TFLOP/s")
            del result
            torch.cuda.empty_cache()
        assert ta.registry.count(ta.OPERATION, ta.IMPLEMENTATION) >= warmup + reps
    head = records[0]
    ok = all(r["parity"]["pass"] for r in records)
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import triangle_attention as oracle

        threads = host_cores()
        torch.set_num_threads(threads)
        q, k, v, bias = inputs[1536]
        qs, ks, vs = (t.cpu() for t in (q, k, v))
        bs = bias.cpu()
        chunk = 64  # batch rows per oracle call: 2.4 GB of scores
        with torch.inference_mode():
            oracle.attention_core(qs[:1], ks[:1], vs[:1], [bs])
            t0 = time.perf_counter()
            for r in range(0, qs.shape[0], chunk):
                oracle.attention_core(qs[r:r + chunk], ks[r:r + chunk], vs[r:r + chunk], [bs])
            spent = time.perf_counter() - t0
        cpu = {"value": round(head["flop"] / spent / 1e12, 5), "unit": "TFLOP/s",
               "kind": "port",
               "sample": (f"CPU oracle attention_core (native op order, FP32, {threads} "
                          f"threads) on the whole B=512 N=1536 call, batch rows in chunks of "
                          f"{chunk}: {spent:.2f} s"),
               "call_s": round(spent, 3), **host_record(threads)}
    return {
        "metric": CORE_METRIC, "value": head["tflops"] if ok else None, "unit": "TFLOP/s",
        "n_gpus": 1, "steps": reps, "warmup": warmup, "ms_per_step": head["median_ms"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (torch.manual_seed(419) q, k, v and bias as the reference benchmark)",
        "config": {"workload": "core-b512-n1536-f32: Protenix _attention per 512-row chunk "
                               "(operator route); also b1000-n1000",
                   "records": records},
        "roofline": {"kernel": "fpx_attn_strided (stage_planes_kernel + stage_bias_kernel + "
                               "mask_rows_kernel + attention_split_kernel<kAttnStaged>), "
                               "per call",
                     "bound": "mfma", "achieved": head["tflops"], "peak": BF16_MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": head["peak_frac"],
                     "traffic": recorded_traffic("core-b512-n1536"),
                     "avg_launch_ms": head["median_ms"]},
        "cpu_baseline": cpu,
        "parity": {"pass": ok},
    }


def statistics_median(values: list[float]) -> float:
    import statistics

    return statistics.median(values)


OPS_METRIC = "pair LayerNorm and sigmoid gate HBM GB/s (% of 8 TB/s) at N=1536 FP32, 1 GPU"


def bench_ops(args) -> dict:
    """The memory-bound stage kernels at N = 1536, FP32, each on its own:

    - pair LayerNorm of z [1536, 1536, 128] (``fpx_layer_norm_c128``), read
      contiguously (starting node) and through the transposed view with
      strides (128, N*128) (ending node, no transposed copy): reads and
      writes 512 N^2 bytes each, 2.42 GB per launch;
    - the sigmoid output gate ``out = value * sigmoid(gate)``
      (``fpx_sigmoid_mul_out``) over N^2 * 128 floats: two reads and one
      write, 3.62 GB per launch.

    The block fuses both (LN into the projection prologue, the gate into the
    attention epilogue); these standalone entries serve the reference's
    per-op hooks.  torch's own ops on the same GPU are timed beside them.
    ``value`` is the transposed-view LayerNorm's GB/s (the reference's
    transposed-norm benchmark); the line carries all six rates.
    """
    import torch
    import torch.nn.functional as F

    from fireprot_amd import _native, workloads

    n = 1536
    dev = torch.device("cuda:0")
    lib = _native.library()
    log(f"inputs ops n={n}")
    z = workloads.make_pair(n).to(dev)
    g = torch.Generator().manual_seed(733)
    w = torch.randn(128, generator=g).to(dev)
    b = torch.randn(128, generator=g).to(dev)
    gate = torch.randn(n, n, 128, generator=g).to(dev)
    y = torch.empty_like(z)
    stream = torch.cuda.current_stream(dev)
    count = n * n * 128
    ln_bytes = 2 * 4 * count
    gate_bytes = 3 * 4 * count

    def ln(transposed):
        si, sj = (128, n * 128) if transposed else (n * 128, 128)
        _native.check(lib.fpx_layer_norm_c128(z.data_ptr(), n, n, si, sj, w.data_ptr(), b.data_ptr(),
                                               1e-5, y.data_ptr(), stream.cuda_stream),
                      "fpx_layer_norm_c128")

    def sig():
        _native.check(lib.fpx_sigmoid_mul_out(gate.data_ptr(), z.data_ptr(), y.data_ptr(), count,
                                              stream.cuda_stream), "fpx_sigmoid_mul_out")

    cases = {
        "layer_norm": (lambda: ln(False), ln_bytes),
        "layer_norm_transposed": (lambda: ln(True), ln_bytes),
        "sigmoid_gate": (sig, gate_bytes),
        "torch_layer_norm": (lambda: F.layer_norm(z, (128,), w, b, 1e-5), ln_bytes),
        "torch_layer_norm_transposed":
            (lambda: F.layer_norm(z.transpose(0, 1), (128,), w, b, 1e-5), ln_bytes),
        "torch_sigmoid_gate": (lambda: torch.sigmoid(gate) * z, gate_bytes),
    }
    out = {}
    with torch.inference_mode():
        for name, (fn, nbytes) in cases.items():
            for _ in range(args.warmup):
                fn()
            torch.cuda.synchronize()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(args.steps):
                fn()
            e1.record(stream)
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / args.steps
            out[name] = {"ms": round(ms, 4), "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                         "hbm_peak_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
            log(f"{name}: {ms:.3f} ms, {out[name]['gbps']} GB/s")
    head = out["layer_norm_transposed"]
    traffic = recorded_traffic("ops-layer-norm-transposed")
    return {
        "metric": OPS_METRIC, "value": head["gbps"], "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": head["ms"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded z ~ N(0,1), gate ~ N(0,1), random LN affine)",
        "config": {"workload": "ops-n1536-f32: standalone pair LayerNorm (contiguous and "
                               "transposed view) and sigmoid gate", "n": n,
                   "bytes_per_launch": {"layer_norm": ln_bytes, "sigmoid_gate": gate_bytes},
                   "kernels": out},
        "roofline": {"kernel": "layer_norm32_kernel (fpx_layer_norm_c128, transposed view)",
                     "bound": "hbm", "achieved": head["gbps"], "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": head["hbm_peak_frac"], "traffic": traffic,
                     "avg_launch_ms": head["ms"]},
        "cpu_baseline": None,
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default 10; the core workload: 20 calls)")
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed warmup steps (default 3; the core workload: 5 calls)")
    ap.add_argument("--config", default="c4", choices=["c1", "c2", "c3", "c4", "c5"])
    ap.add_argument("--workload", default="block",
                    choices=["block", "core", "openfold3", "trimul", "transition", "ops"],
                    help="block: the triangle-attention block (default); core: the "
                         "attention core on the operator route (B512 N1536, B1000 N1000); "
                         "openfold3: "
                         "OpenFold3's _attention through fpx_attn_strided; trimul: "
                         "triangle multiplication (fpx_tri_mul); transition: the pair "
                         "transition (fpx_transition); ops: the standalone pair "
                         "LayerNorm and sigmoid gate (HBM-bound)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 1 GiB device-to-device copy (the known-size "
                         "reference for rocprofv3 FETCH_SIZE / WRITE_SIZE scaling)")
    args = ap.parse_args()
    core = args.workload == "core"
    args.steps = args.steps if args.steps is not None else (20 if core else 10)
    args.warmup = args.warmup if args.warmup is not None else (5 if core else 3)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py runs on exactly one GPU: the triangle-attention block is measured on "
              "one MI355X (multi-GPU sharding is a design note, not a measured path); "
              "use --gpus 1", file=sys.stderr)
        return 2

    import torch

    from fireprot_amd import _native, block, workloads

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2
    lib = _native.library()
    if args.workload == "core":
        result = bench_core(args)
        if args.calibrate_copy:
            calibrate_copy(torch.device("cuda:0"))
        print(json.dumps(result), flush=True)
        return 0 if result["parity"]["pass"] else 1
    if args.workload == "openfold3":
        result = bench_openfold3(args)
        if args.calibrate_copy:
            calibrate_copy(torch.device("cuda:0"))
        print(json.dumps(result), flush=True)
        return 0
    if args.workload == "trimul":
        result = bench_trimul(args)
        if args.calibrate_copy:
            calibrate_copy(torch.device("cuda:0"))
        print(json.dumps(result), flush=True)
        return 0
    if args.workload == "ops":
        result = bench_ops(args)
        if args.calibrate_copy:
            calibrate_copy(torch.device("cuda:0"))
        print(json.dumps(result), flush=True)
        return 0
    if args.workload == "transition":
        result = bench_transition(args)
        if args.calibrate_copy:
            calibrate_copy(torch.device("cuda:0"))
        print(json.dumps(result), flush=True)
        return 0
    cfg = workloads.CONFIGS[args.config]
    n = cfg.n
    log(f"inputs {cfg.name}")
    z_cpu, mask_cpu, w = workloads.make_inputs(cfg)
    dev = torch.device("cuda:0")
    dtype = torch.bfloat16 if cfg.dtype == "bf16" else torch.float32
    dtype_code = block.DTYPES[dtype]
    z = z_cpu.to(dtype).to(dev)
    mask = None if mask_cpu is None else mask_cpu.to(dev)
    weights = block.BlockWeights.from_tensors(**w, dtype=dtype).to(dev)
    out_s = torch.empty_like(z)
    out_e = torch.empty_like(z)
    ws = torch.empty(block.workspace_bytes(n, dtype), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)

    def step():
        block.triangle_attention_block(z, mask, weights, ending=False, out=out_s, workspace=ws)
        block.triangle_attention_block(z, mask, weights, ending=True, out=out_e, workspace=ws)

    with torch.inference_mode():
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        log(f"warmup {args.warmup} done")
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0.record(stream)
        for _ in range(args.steps):
            step()
        t1.record(stream)
        torch.cuda.synchronize()
        ms_per_step = t0.elapsed_time(t1) / args.steps
        log(f"timed {args.steps} steps: {ms_per_step:.3f} ms/step")

        # Stage timing on the launch stream: prepare (mask bias + LN/projections),
        # attend (attention kernel), finish (output projection), starting node.
        ws_bytes = ws.numel()
        sptr = stream.cuda_stream
        mptr = mask.data_ptr() if mask is not None else None
        mstr = (mask.stride(0), mask.stride(1)) if mask is not None else (0, 0)

        def prepare():
            _native.check(lib.fpx_tri_attn_prepare(
                dtype_code, z.data_ptr(), z.stride(0), z.stride(1), mptr, mstr[0], mstr[1],
                weights.ln_w.data_ptr(), weights.ln_b.data_ptr(), weights.eps,
                weights.w_qkvg.data_ptr(), None, weights.w_bias.data_ptr(), weights.inf, n, 0,
                ws.data_ptr(), ws_bytes, sptr), "prepare")

        def attend():
            _native.check(lib.fpx_tri_attn_attend(dtype_code, n, ws.data_ptr(), ws_bytes, sptr),
                          "attend")

        def finish():
            _native.check(lib.fpx_tri_attn_finish(dtype_code, weights.w_o.data_ptr(), None, n, 0,
                                                  out_s.data_ptr(), out_s.stride(0),
                                                  out_s.stride(1), ws.data_ptr(), ws_bytes,
                                                  sptr), "finish")

        # One block call at a time (starting node, the module's entry with
        # its output and workspace passed in), each bracketed by its own HIP
        # events: median and p95 over 20 calls, the reference benchmark's
        # per-call statistics.
        def one_block():
            block.triangle_attention_block(z, mask, weights, ending=False, out=out_s, workspace=ws)

        per_call = []
        for _ in range(20):
            c0 = torch.cuda.Event(enable_timing=True)
            c1 = torch.cuda.Event(enable_timing=True)
            c0.record(stream)
            one_block()
            c1.record(stream)
            c1.synchronize()
            per_call.append(c0.elapsed_time(c1))
        per_call.sort()
        block_call = {"calls": len(per_call), "median_ms": round(per_call[len(per_call) // 2], 4),
                      "p95_ms": round(per_call[int(0.95 * (len(per_call) - 1) + 0.5)], 4),
                      "min_ms": round(per_call[0], 4)}
        log(f"single block call (start): median {block_call['median_ms']:.3f} ms, "
            f"p95 {block_call['p95_ms']:.3f} ms")

        # The module-level route a caller uses: the registry's block dispatch
        # on a Protenix-shaped module (weights packed once and cached, the
        # workspace cached per device and stream, dz allocated per call).
        from fireprot_amd import triangle_attention as ta

        module = workloads.make_protenix_module(w, starting=True, device=dev).to(dtype)

        def module_call():
            return ta.dispatch_triangle_attention_block(
                module=module, z=z, mask=mask, ending=False,
                native=lambda **_: (_ for _ in ()).throw(RuntimeError("native selected")))

        for _ in range(2):
            module_call()
        module_times = []
        for _ in range(20):
            c0 = torch.cuda.Event(enable_timing=True)
            c1 = torch.cuda.Event(enable_timing=True)
            c0.record(stream)
            module_call()
            c1.record(stream)
            c1.synchronize()
            module_times.append(c0.elapsed_time(c1))
        module_times.sort()
        module_call_stats = {
            "calls": 20, "route": "dispatch_triangle_attention_block -> "
            + (ta.BLOCK_BF16_IMPLEMENTATION if dtype == torch.bfloat16 else ta.BLOCK_IMPLEMENTATION),
            "median_ms": round(module_times[10], 4),
            "p95_ms": round(module_times[int(0.95 * 19 + 0.5)], 4),
            "min_ms": round(module_times[0], 4)}
        log(f"module route (start): median {module_call_stats['median_ms']:.3f} ms, "
            f"p95 {module_call_stats['p95_ms']:.3f} ms")
        from fireprot_amd import workspace as ws_cache

        ws_cache.release()
        del module

        stages = {}
        for name, fn in (("prepare", prepare), ("attend", attend), ("finish", finish)):
            fn()
            torch.cuda.synchronize()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            reps = max(args.steps, 5)
            e0.record(stream)
            for _ in range(reps):
                fn()
            e1.record(stream)
            torch.cuda.synchronize()
            stages[name] = e0.elapsed_time(e1) / reps
            log(f"stage {name}: {stages[name]:.3f} ms")

        if args.calibrate_copy:
            calibrate_copy(dev)

    flops = block.block_flops(n)
    step_flop = 2 * flops["block"]
    value = step_flop / (ms_per_step * 1e-3) / 1e12
    traffic = recorded_traffic(cfg.name)
    split = cfg.dtype != "bf16"
    if cfg.dtype == "bf16":
        kernel_name = "attention_bf16_kernel (fpx_tri_attn_attend, BF16)"
    else:
        kernel_name = ("attention_split_kernel<kAttnBlock, fast | exact> + "
                       "attention_const_kernel<kAttnBlock> (fpx_tri_attn_attend, fp16 planes)")
    # The peak of the matrix unit the kernel issues: the dense fp16/bf16 one.
    peak = BF16_MFMA_PEAK_TFLOPS
    nkt = -(-n // 32)
    visited = visited_key_tiles(n, cfg.valid, skip=cfg.dtype != "bf16")
    visited_flop = flops["core"] * visited // (n * nkt)
    attend_tflops = visited_flop / (stages["attend"] * 1e-3) / 1e12
    roofline = {
        "kernel": kernel_name,
        "bound": "mfma",
        "achieved": round(attend_tflops, 3),
        "peak": peak,
        "unit": "TFLOP/s",
        "frac": round(attend_tflops / peak, 4),
        "traffic": traffic,
        "flop_per_launch": visited_flop,
        "flop_all_tiles": flops["core"],
        "visited_key_tile_frac": round(visited / (n * nkt), 4),
        "avg_launch_ms": round(stages["attend"], 4),
        "fp32_algorithmic_tflops_all_tiles": round(
            flops["core"] / (stages["attend"] * 1e-3) / 1e12, 3),
    }
    if split:
        # padding rows of a tail mask take the constant-mask kernel (no S^T)
        const_tiles = 0 if cfg.valid is None or cfg.valid >= n else (n - cfg.valid) * nkt
        roofline.update(split_executed(n, n, stages["attend"], visited,
                                       const_tiles=const_tiles))
    result = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg.dtype,
        "data": "synthetic (seeded torch.Generator inputs and N(0,0.02) random-init weights)",
        "config": {
            "workload": f"{cfg.name}: starting + ending triangle-attention block",
            "n": n, "c_z": 128, "heads": 4, "head_dim": 32,
            "valid_residues": cfg.valid if cfg.valid is not None else n,
            "bias_scale": cfg.bias_scale,
            "block_ms": round(ms_per_step / 2, 4),
            "block_tflops": round(value, 3),
            "block_peak_frac": round(value / peak, 4),
            "step_flop": step_flop,
            "stage_ms_start_node": {k: round(v, 4) for k, v in stages.items()},
            "block_call_start_node": block_call,
            "module_call_start_node": module_call_stats,
        },
        "roofline": roofline,
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        gpu_out = {"start": out_s.float().cpu(), "end": out_e.float().cpu()}
        del out_s, out_e, ws
        torch.cuda.empty_cache()
        record, oracle_out = cpu_baseline(cfg, z_cpu, mask_cpu, w)
        result["cpu_baseline"] = record
        result["parity"] = parity_report(cfg, gpu_out, oracle_out)
        gate = parity_gate(cfg, gpu_out, oracle_out, z_cpu, mask_cpu, w)
        result["parity"]["gate"] = gate
        log(f"parity vs CPU oracle: {json.dumps(result['parity'])}")
        if not gate["pass"]:
            # a result that misses its parity bar is not a measurement
            result["value"] = None
            print(json.dumps(result), flush=True)
            log("PARITY FAILED: value withheld")
            return 1
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
