"""Benchmark of the MI355X SpMM hot path (one JSON line on stdout).

Default workload: BASELINE config 2 (power-law CSR 100000x100000, ~1.9M nnz,
N=128 fp16, fp32 accumulate) — the configuration the headline metric
"SpMM GFLOP/s (2*nnz*N/t) and HBM GB/s % of peak, N=128 fp16" is quoted on.
A step is one SpMM call over resident device inputs.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2] [--width N]
                       [--op csr|mixed-empty] [--no-cpu]

Only one GPU is used; --gpus > 1 exits with a message.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

REPO = os.path.dirname(os.path.abspath(__file__))
for sub in ("ascend-spmm_amd", "tests"):
    sys.path.insert(0, os.path.join(REPO, sub))

import workloads  # noqa: E402

METRIC = "SpMM GFLOP/s (2·nnz·N/t) and HBM GB/s % of peak, N=128 fp16, 1 MI355X"
HBM_PEAK_GBPS = 8000.0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def cpu_baseline(w, B: np.ndarray, budget_s: float) -> dict:
    """The reference's CPU path (cpu_reference: torch CSR sparse.mm in fp32,
    tests/aic_aiv_ablation/common.py:173-177) on the host cores, same matrix."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle  # checker-only import: the CPU baseline leg

    threads = torch.get_num_threads()
    oracle.cpu_reference(w.rows, w.cols, w.crow, w.col, w.values, B)  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - t_start < budget_s and len(times) < 50):
        t0 = time.perf_counter()
        oracle.cpu_reference(w.rows, w.cols, w.crow, w.col, w.values, B)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s and len(times) >= 3:
            break
    t = float(np.median(times))
    width = B.shape[1]
    return {
        "value": round(2.0 * w.nnz * width / t / 1e9, 3),
        "unit": "GFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"full {w.name} matrix ({w.nnz} nnz) x N={width}, torch.sparse.mm fp32 "
                   f"(the reference's cpu_reference), median of {len(times)} reps, "
                   f"{t * 1e3:.1f} ms/rep, os.cpu_count()={os.cpu_count()}"),
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--width", type=int, default=None)
    ap.add_argument("--op", choices=["csr", "mixed-empty"], default="csr")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no "
              "multi-GPU path: the SpMM shards by row windows with no exchange when the dense "
              "operand is replicated, so N GPUs is N independent runs of this benchmark.",
              file=sys.stderr)
        return 2

    import spmm_npu

    w = workloads.make(args.config)
    width = args.width or w.widths[0]
    B = w.dense(width)
    log(f"[bench] workload {w.name}: {w.rows}x{w.cols}, nnz={w.nnz}, N={width}, {w.dtype}")

    dev = torch.device("cuda:0")
    crow = torch.from_numpy(w.crow.astype(np.int32)).to(dev)
    col = torch.from_numpy(w.col.astype(np.int32)).to(dev)
    val = torch.from_numpy(w.values).to(dev)
    dense = torch.from_numpy(B).to(dev)
    start = torch.zeros(40, dtype=torch.int32, device=dev)
    if args.op == "csr":
        def step():
            return spmm_npu.spmm_csr(crow, col, val, dense, start)
        op_name = "spmm_csr"
    else:
        e_i = torch.zeros(0, dtype=torch.int32, device=dev)
        e_v = torch.zeros(0, dtype=val.dtype, device=dev)
        z1 = torch.zeros(1, dtype=torch.int32, device=dev)
        z20 = torch.zeros(20, dtype=torch.int32, device=dev)

        def step():
            return spmm_npu.spmm_ascend_cube(z1, e_i, e_v, crow, col, val, dense, z20, start)
        op_name = "spmm_ascend_cube(vector part only)"

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"[bench] warmup {args.warmup} done")

    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        ev[i][0].record(stream)
        step()
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    wall_ms = (t1 - t0) * 1e3 / args.steps
    launch_ms = float(np.mean([a.elapsed_time(b) for a, b in ev]))
    log(f"[bench] timed {args.steps} steps: wall {wall_ms:.4f} ms/step, events {launch_ms:.4f} ms/call")

    flops = 2.0 * w.nnz * width
    alg_bytes = workloads.algorithmic_bytes(w, width)
    t_s = wall_ms / 1e3
    achieved = alg_bytes / (launch_ms / 1e3) / 1e9
    result = {
        "metric": METRIC,
        "value": round(flops / t_s / 1e9, 3),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16" if w.dtype == "fp16" else "fp32",
        "data": "synthetic (seeded generator of BASELINE config %d)" % args.config,
        "config": {
            "workload": f"{w.name} {w.rows}x{w.cols} nnz={w.nnz} N={width} {w.dtype}",
            "op": op_name,
            "accumulate": "fp32",
            "index": "int32",
        },
        "hbm_gbps_algorithmic": round(alg_bytes / t_s / 1e9, 1),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": None,
            "algorithmic_bytes_per_launch": alg_bytes,
            "launch_ms": round(launch_ms, 5),
        },
    }
    if not args.no_cpu:
        log("[bench] CPU baseline ...")
        result["cpu_baseline"] = cpu_baseline(w, B, args.cpu_budget)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
