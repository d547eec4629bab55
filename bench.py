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
``executed_frac`` the 16-bit matrix work it actually issues.  Under
``FPX_ATTENTION_MFMA=f32`` the peak is the 157.3 TFLOP/s FP32 matrix peak.
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
                   fp16_planes: bool = False, const_tiles: int = 0) -> dict:
    """16-bit matrix-core work the split attention kernel executes for its
    FP32-accurate products, per 32 x 32 (query x key) wave tile, counted in
    32x32x16 MFMAs of 32768 flop each (two K-halves per product term)
    against 2 * 65536 algorithmic flop:
      - caller-supplied q/k/v (strided layout): 6 bf16 terms of S^T and 3 of
        O^T = 18 MFMAs;
      - fp16 planes (the block's, and the staged strided operands): 3 fp16
        terms of S^T and 3 of O^T = 12.
    fp16 and bf16 MFMAs share one dense peak.  Query rows are padded to 128,
    keys to 32.  ``tiles``: key tiles visited summed over the outer rows
    (default: every tile of every row).  ``const_tiles``: the part of
    ``tiles`` on constant-mask rows (padding rows, fl(s + m) = m for every
    key), whose S^T the kernel leaves out: 6 MFMAs per wave tile (O^T only)."""
    np_ = -(-n // 128) * 128
    nkt = -(-n // 32)
    visited = batch * nkt if tiles is None else tiles
    per_tile = 12 if fp16_planes else 18
    executed = ((visited - const_tiles) * per_tile + const_tiles * 6) * 4 * (np_ // 32) * 32768
    executed_tflops = executed / (ms * 1e-3) / 1e12
    unit = ("fp16 hi/lo planes scaled by powers of two (q, k per 32x32 tile; v^T per key "
            "tile; p per tile), three terms per product" if fp16_planes
            else "bf16 (exact 3-plane split of K and Q, 2-plane V and P)")
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
    fp32_mfma = os.environ.get("FPX_ATTENTION_MFMA") == "f32"
    of3_visited = visited_key_tiles(n, n - 184, skip=not fp32_mfma)
    of3_flop = flop * of3_visited // (n * -(-n // 32))
    of3_peak = FP32_MFMA_PEAK_TFLOPS if fp32_mfma else BF16_MFMA_PEAK_TFLOPS
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
            "kernel": ("attention_kernel<kAttnStrided> + staging (fpx_attn_strided)" if fp32_mfma
                       else "attention_split_kernel<kAttnStaged> + plane, mask and bias staging"
                            " (fpx_attn_strided)"),
            "bound": "mfma", "achieved": round(of3_achieved, 3), "peak": of3_peak,
            "unit": "TFLOP/s", "frac": round(of3_achieved / of3_peak, 4),
            "traffic": recorded_traffic("openfold3/fp32-mfma" if fp32_mfma else "openfold3"),
            "flop_per_launch": of3_flop, "flop_all_tiles": flop,
            "fp32_algorithmic_tflops_all_tiles": round(tflops, 3),
            "avg_launch_ms": round(ms, 4),
            **({} if fp32_mfma else split_executed(n, n, ms, of3_visited, fp16_planes=True)),
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
    # fp16 planes on the 16-bit matrix cores unless the FP32 ones are selected
    tr_peak = (FP32_MFMA_PEAK_TFLOPS if os.environ.get("FPX_ATTENTION_MFMA") == "f32"
               else BF16_MFMA_PEAK_TFLOPS)
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
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c4", choices=["c1", "c2", "c3", "c4", "c5"])
    ap.add_argument("--workload", default="block",
                    choices=["block", "openfold3", "trimul", "transition", "ops"],
                    help="block: the triangle-attention block (default); openfold3: "
                         "OpenFold3's _attention through fpx_attn_strided; trimul: "
                         "triangle multiplication (fpx_tri_mul); transition: the pair "
                         "transition (fpx_transition); ops: the standalone pair "
                         "LayerNorm and sigmoid gate (HBM-bound)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 1 GiB device-to-device copy (the known-size "
                         "reference for rocprofv3 FETCH_SIZE / WRITE_SIZE scaling)")
    args = ap.parse_args()
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
    fp32_mfma = os.environ.get("FPX_ATTENTION_MFMA") == "f32"
    traffic = recorded_traffic(f"{cfg.name}/fp32-mfma" if fp32_mfma else cfg.name)
    split = cfg.dtype != "bf16" and not fp32_mfma
    if cfg.dtype == "bf16":
        kernel_name = "attention_bf16_kernel (fpx_tri_attn_attend, BF16)"
    elif split:
        kernel_name = ("attention_split_kernel<kAttnBlock, fast | exact> + "
                       "attention_const_kernel<kAttnBlock> (fpx_tri_attn_attend, fp16 planes)")
    else:
        kernel_name = "attention_kernel<kAttnBlock> (fpx_tri_attn_attend, FP32 matrix cores)"
    # The peak of the matrix unit the kernel issues: fp16/bf16 unless the FP32
    # matrix cores are selected.
    peak = FP32_MFMA_PEAK_TFLOPS if fp32_mfma and cfg.dtype != "bf16" else BF16_MFMA_PEAK_TFLOPS
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
        roofline.update(split_executed(n, n, stages["attend"], visited, fp16_planes=True,
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
        log(f"parity vs CPU oracle: {json.dumps(result['parity'])}")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
