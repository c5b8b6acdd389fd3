#!/usr/bin/env python3
"""Correctness checks of Ascend-SpMM's test harness, run on the MI355X build.

    python ascend-spmm_amd/checks.py task-mapping [options]   # partitions vs spmm_csr
    python ascend-spmm_amd/checks.py aic-aiv [options]        # operator aliases vs base ops
    python ascend-spmm_amd/checks.py aiv-bitwise [options]    # pure vector part vs spmm_csr, exact

The same modes, options, seeds and JSON report schema as the reference's
``scripts/run_tests.sh`` and its three scripts (tests/task_mapping/
correctness.py, tests/aic_aiv_ablation/correctness.py,
tests/aic_aiv_ablation/bitwise_correctness.py), so a dataset directory
prepared for the reference (``.pt`` payloads) is checked unchanged and the
reports line up field by field.  Differences: tensors live on the GPU
(``cuda``), and task-mapping restores the original row order of the
``ours`` partition before comparing (the reference compares the packed
rows directly).  No timing is collected.
"""

from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path
from typing import Dict, List, Optional, Sequence

import torch

import payloads as D
import partition as PT
import spmm_npu

ROOT = Path(__file__).resolve().parents[1]
MODES = ("aic-aiv", "aiv-bitwise", "task-mapping")


def require_gpu() -> None:
    if not torch.cuda.is_available():
        raise SystemExit("An available GPU (torch.cuda on ROCm) is required")


def compare(actual: torch.Tensor, expected: torch.Tensor, atol: float, rtol: float, what: str,
            names=("actual_value", "reference_value"), first_mismatch: bool = True) -> Dict:
    """isclose comparison in fp32 (task-mapping correctness.py:34-64)."""
    a = actual.detach().float().cpu()
    e = expected.detach().float().cpu()
    if a.shape != e.shape:
        raise RuntimeError(f"shape mismatch: {tuple(a.shape)} != {tuple(e.shape)}")
    if not bool(torch.isfinite(a).all()):
        raise RuntimeError(f"{what} output contains NaN or Inf")
    if not bool(torch.isfinite(e).all()):
        raise RuntimeError("CSR reference contains NaN or Inf")
    diff = (a - e).abs()
    close = torch.isclose(a, e, atol=atol, rtol=rtol)
    bad = int((~close).sum())
    result = {
        "bitwise_equal": bool(torch.equal(a, e)),
        "mismatch_count": bad,
        "max_abs_error": float(diff.max()) if diff.numel() else 0.0,
        "mean_abs_error": float(diff.mean()) if diff.numel() else 0.0,
        "passed": bad == 0,
    }
    if bad and first_mismatch:
        row, column = (int(x) for x in torch.nonzero(~close)[0].tolist())
        result.update(first_mismatch_row=row, first_mismatch_column=column,
                      **{names[0]: float(a[row, column]), names[1]: float(e[row, column])})
    return result


def check_dims(parser: argparse.ArgumentParser, dims: List[int], dtype: str) -> None:
    max_dim = 1024 if dtype == "fp16" else 512
    if any(d <= 0 or d > max_dim or d % 16 for d in dims):
        parser.error(f"every --dim must be a positive multiple of 16 no greater than {max_dim} for {dtype}")
    if len(dims) != len(set(dims)):
        parser.error("feature widths must not contain duplicates")


def add_selection(parser: argparse.ArgumentParser, single: bool = False) -> None:
    parser.add_argument("--dataset-dir", type=Path, default=ROOT / "datasets_pt",
                        help="CSR .pt directory (see payloads.convert_matrix_market).")
    parser.add_argument("--name", default="", help="Filter by parent or filename.")
    if single:
        parser.add_argument("--index", type=int, default=0, help="Dataset index when --name is absent.")
        return
    parser.add_argument("--index", type=int, help="Select one filtered dataset index.")
    parser.add_argument("--start", type=int, default=0, help="Inclusive filtered index.")
    parser.add_argument("--stop", type=int, help="Exclusive filtered index.")
    parser.add_argument("--limit", type=int, help="Maximum selected datasets.")


def dataset_dir_of(args) -> Path:
    d = args.dataset_dir.expanduser().resolve()
    if not d.is_dir():
        raise SystemExit(f"Dataset directory does not exist: {d}")
    return d


def discover(args, dataset_dir: Path):
    try:
        return D.discover_datasets(dataset_dir, args.name, args.index, args.start, args.stop, args.limit)
    except ValueError as exc:
        raise SystemExit(str(exc)) from exc


def write_report(report: Dict, output: Path) -> Path:
    output = output.expanduser().resolve()
    output.parent.mkdir(parents=True, exist_ok=True)
    output.write_text(json.dumps(report, indent=2) + "\n", encoding="utf-8")
    print(f"Result: {output}")
    return output


# ---------------------------------------------------------------- task-mapping

def task_mapping_args(argv: Sequence[str]):
    p = argparse.ArgumentParser(
        prog="checks.py task-mapping",
        description="Compare the task mapping and the three partition baselines with the "
                    "standalone CSR kernel. No timing is collected.")
    add_selection(p)
    p.add_argument("--method", action="append", choices=PT.METHODS,
                   help="Partition method; repeat to select several (default: all).")
    p.add_argument("--dim", dest="dims", action="append", type=int,
                   help="Feature width; repeat to test several widths (default: 128).")
    p.add_argument("--dtype", choices=("fp16", "fp32"), default="fp16")
    p.add_argument("--seed", type=int, default=2027)
    p.add_argument("--atol", type=float)
    p.add_argument("--rtol", type=float)
    p.add_argument("--block-ratio", type=float, default=PT.DEFAULT_BLOCK_RATIO,
                   help="Target block/vector ratio used by block_level_split.")
    p.add_argument("--naive-fraction", type=float, default=PT.DEFAULT_NAIVE_FRACTION,
                   help="Leading nonzero fraction assigned to the block part by the naive strategy.")
    p.add_argument("--neutronsparse-assume-symmetric", action="store_true",
                   help="Use row degree as column degree on square matrices.")
    p.add_argument("--output", type=Path,
                   help="JSON output (default: results/table6_correctness_<method|all>_<dtype>.json).")
    args = p.parse_args(argv)
    if args.index is not None and (args.start != 0 or args.stop is not None or args.limit is not None):
        p.error("--index cannot be combined with --start, --stop, or --limit")
    args.methods = args.method or list(PT.METHODS)
    if len(args.methods) != len(set(args.methods)):
        p.error("Table 6 methods must not contain duplicates")
    args.dims = args.dims or [128]
    check_dims(p, args.dims, args.dtype)
    if args.block_ratio <= 0:
        p.error("--block-ratio must be positive")
    if not 0.0 <= args.naive_fraction <= 1.0:
        p.error("--naive-fraction must be in [0, 1]")
    tol = 2e-2 if args.dtype == "fp16" else 1e-4
    args.atol = tol if args.atol is None else args.atol
    args.rtol = tol if args.rtol is None else args.rtol
    if args.atol < 0 or args.rtol < 0:
        p.error("--atol and --rtol must be non-negative")
    return args


def task_mapping_dataset(path: Path, dataset_dir: Path, args, dtype) -> Dict:
    name, rows, cols, crow, col = D.load_payload(path)
    relative = path.relative_to(dataset_dir).as_posix()
    seed = D.stable_seed(args.seed, relative)
    values = D.make_values(col.numel(), dtype, seed)
    cases, partitions = [], {}
    for method in args.methods:
        mapping, meta = PT.prepare_partition(method, rows, cols, crow, col, values,
                                             block_ratio=args.block_ratio,
                                             naive_fraction=args.naive_fraction,
                                             assume_symmetric=args.neutronsparse_assume_symmetric)
        partitions[method] = meta
        print(f"partition={method}, aic_nnz={meta['aic_nnz']}, aiv_nnz={meta['aiv_nnz']}")
        for dim in args.dims:
            dense = D.make_dense(cols, dim, dtype, seed + dim).cuda()
            reference = PT.run_reference(crow, col, values, dense)[:rows]
            output = PT.run_mapping(mapping, dense, rows)
            metrics = compare(output, reference, args.atol, args.rtol, "task-mapping")
            record = {"dataset": name, "path": relative, "rows": rows, "cols": cols, "nnz": col.numel(),
                      "method": method, "label": PT.METHOD_LABELS[method], "reference": "spmm_csr",
                      "feature_width": dim, "dtype": args.dtype, "atol": args.atol, "rtol": args.rtol,
                      **meta, **metrics}
            cases.append(record)
            print(f"{'PASS' if record['passed'] else 'FAIL'}: dataset={name}, method={method}, N={dim}, "
                  f"mismatches={record['mismatch_count']}, max_abs_error={record['max_abs_error']:.8g}")
    return {"dataset": name, "path": relative, "rows": rows, "cols": cols, "nnz": col.numel(),
            "dataset_seed": seed, "partitions": partitions, "cases": cases}


def task_mapping(argv: Sequence[str]) -> int:
    args = task_mapping_args(argv)
    require_gpu()
    dataset_dir = dataset_dir_of(args)
    paths = discover(args, dataset_dir)
    dtype = torch.float16 if args.dtype == "fp16" else torch.float32
    datasets, cases = [], []
    for i, path in enumerate(paths, start=1):
        print(f"[{i}/{len(paths)}] validating {path.relative_to(dataset_dir)}")
        result = task_mapping_dataset(path, dataset_dir, args, dtype)
        datasets.append({k: v for k, v in result.items() if k != "cases"})
        cases.extend(result["cases"])
    failures = sum(not c["passed"] for c in cases)
    report = {
        "schema_version": 1,
        "experiment": "Table 6 task-mapping correctness",
        "timing_collected": False,
        "reference": "spmm_csr on the original CSR",
        "dataset_dir": str(dataset_dir),
        "selected_datasets": len(paths),
        "methods": args.methods,
        "dtype": args.dtype,
        "feature_widths": args.dims,
        "seed": args.seed,
        "atol": args.atol,
        "rtol": args.rtol,
        "block_ratio": args.block_ratio,
        "naive_fraction": args.naive_fraction,
        "neutronsparse_assume_symmetric": args.neutronsparse_assume_symmetric,
        "comparisons": len(cases),
        "passed": failures == 0,
        "failed": failures,
        "datasets": datasets,
        "cases": cases,
    }
    suffix = args.methods[0] if len(args.methods) == 1 else "all"
    write_report(report, args.output or ROOT / "results" / f"table6_correctness_{suffix}_{args.dtype}.json")
    if failures:
        raise SystemExit(f"FAIL: {failures}/{len(cases)} comparisons failed")
    print(f"PASS: all {len(cases)} Table 6 comparisons passed; no timing collected")
    return 0


# ---------------------------------------------------------------- aic-aiv

ABLATION_METHODS = ("aic-pipeline", "aic-without-pipeline", "aiv-naive", "aiv-mb", "aiv-mb-batch",
                    "aiv-round-robin")
AIC_METHODS = ABLATION_METHODS[:2]
AIV_METHODS = ABLATION_METHODS[2:]
ABLATION_LABELS = {
    "aic-pipeline": "AIC hierarchy-aware pipeline (g=6)",
    "aic-without-pipeline": "AIC without hierarchy-aware pipeline (g=1)",
    "aiv-naive": "AIV Naive CSR",
    "aiv-mb": "AIV Multiple Buffer",
    "aiv-mb-batch": "AIV Multiple Buffer + Batched Process (batch=8, buffers=64)",
    "aiv-round-robin": "AIV Round-Robin Ring Buffer (L=64)",
}


def ablation_inputs(nnz: int, cols: int, dim: int, dtype, seed: int):
    """Values U(0, 1) then dense U(0, 1) from one seeded generator
    (aic_aiv_ablation/common.py:106-110)."""
    g = torch.Generator().manual_seed(seed)
    values = torch.rand(nnz, generator=g).to(dtype).contiguous()
    dense = torch.rand((cols, dim), generator=g).to(dtype).contiguous()
    return values, dense


def run_ablation(method: str, rows: int, cols: int, crow, col, values, dense) -> torch.Tensor:
    """One ablation operator on the GPU; the first ``rows`` output rows
    (aic_aiv_ablation/common.py:113-170).  aic-*: csr_to_bcsr, empty vector
    part; aiv-*: the CSR as the vector part (or spmm_csr itself)."""
    if method not in ABLATION_METHODS:
        raise ValueError(f"unknown ablation method: {method}")
    i32 = torch.int32
    d = dense.cuda()
    empty_ptr = torch.zeros(1, dtype=i32, device="cuda")
    empty_col = torch.empty(0, dtype=i32, device="cuda")
    empty_val = torch.empty(0, dtype=values.dtype, device="cuda")
    if method.startswith("aic-"):
        b = spmm_npu.csr_to_bcsr(crow.cuda(), col.cuda(), values.cuda(), rows, cols, 16)
        op = spmm_npu.spmm_ascend_cube if method == "aic-pipeline" else spmm_npu.spmm_ascend_cube_aic_without_pipeline
        cptr = b["crow_window_ptr"].to(i32)
        return op(cptr, b["unique_col_ids"].to(i32), b["value"], empty_ptr, empty_col, empty_val, d,
                  spmm_npu.make_start(cptr, PT.AIC_CORES).cuda(),
                  torch.zeros(PT.AIV_CORES, dtype=i32, device="cuda"))[:rows]
    rp, c, v = crow.to("cuda", i32), col.to("cuda", i32), values.cuda()
    vstart = spmm_npu.make_start(rp, PT.AIV_CORES).cuda()
    if method in ("aiv-naive", "aiv-mb-batch"):
        op = spmm_npu.spmm_csr if method == "aiv-naive" else spmm_npu.spmm_csr_aiv_mb_batch
        return op(rp, c, v, d, vstart)[:rows]
    op = spmm_npu.spmm_ascend_cube_aiv_mb if method == "aiv-mb" else spmm_npu.spmm_ascend_cube
    return op(empty_ptr, empty_col, empty_val, rp, c, v, d,
              torch.zeros(PT.AIC_CORES, dtype=i32, device="cuda"), vstart)[:rows]


def aic_aiv_args(argv: Sequence[str]):
    p = argparse.ArgumentParser(prog="checks.py aic-aiv",
                                description="Validate the AIC and AIV ablation operators.")
    add_selection(p, single=True)
    p.add_argument("--dim", dest="dims", action="append", type=int,
                   help="Feature width; repeat to test several widths (default: 128).")
    p.add_argument("--dtype", choices=("fp16", "fp32"), default="fp16")
    p.add_argument("--seed", type=int, default=2027)
    p.add_argument("--aic-atol", type=float)
    p.add_argument("--aic-rtol", type=float)
    p.add_argument("--aiv-atol", type=float, default=0.0)
    p.add_argument("--aiv-rtol", type=float, default=0.0)
    p.add_argument("--output", type=Path, help="JSON output (default: results/aic_aiv_correctness_<dtype>.json).")
    args = p.parse_args(argv)
    args.dims = args.dims or [128]
    check_dims(p, args.dims, args.dtype)
    if any(t is not None and t < 0 for t in (args.aic_atol, args.aic_rtol, args.aiv_atol, args.aiv_rtol)):
        p.error("all tolerances must be non-negative")
    tol = 2e-2 if args.dtype == "fp16" else 1e-4
    args.aic_atol = tol if args.aic_atol is None else args.aic_atol
    args.aic_rtol = tol if args.aic_rtol is None else args.aic_rtol
    return args


def aic_aiv(argv: Sequence[str]) -> int:
    args = aic_aiv_args(argv)
    require_gpu()
    dataset_dir = dataset_dir_of(args)
    try:
        path = D.select_dataset(dataset_dir, args.name, args.index)
        name, rows, cols, crow, col = D.load_payload(path)
    except ValueError as exc:
        raise SystemExit(str(exc)) from exc
    relative = path.relative_to(dataset_dir).as_posix()
    seed = D.stable_seed(args.seed, relative)
    dtype = torch.float16 if args.dtype == "fp16" else torch.float32
    cases = []
    for dim in args.dims:
        values, dense = ablation_inputs(col.numel(), cols, dim, dtype, seed + dim)
        for group, base, atol, rtol in ((AIC_METHODS, "aic-pipeline", args.aic_atol, args.aic_rtol),
                                        (AIV_METHODS, "aiv-naive", args.aiv_atol, args.aiv_rtol)):
            reference = run_ablation(base, rows, cols, crow, col, values, dense)
            for method in group:
                output = reference if method == base else run_ablation(method, rows, cols, crow, col, values, dense)
                record = {"method": method, "label": ABLATION_LABELS[method], "reference": base,
                          "feature_width": dim, "atol": atol, "rtol": rtol,
                          **compare(output, reference, atol, rtol, "ablation", first_mismatch=False)}
                cases.append(record)
                bitwise = f"bitwise={record['bitwise_equal']}, " if group is AIV_METHODS else ""
                print(f"{'PASS' if record['passed'] else 'FAIL'}: {method}, N={dim}, {bitwise}"
                      f"mismatches={record['mismatch_count']}, max_abs_error={record['max_abs_error']:.8g}")
    failed = sum(not c["passed"] for c in cases)
    report = {
        "schema_version": 1,
        "experiment": "Figure 10/11 kernel ablations",
        "timing_collected": False,
        "dataset": name,
        "path": relative,
        "rows": rows,
        "cols": cols,
        "nnz": col.numel(),
        "dtype": args.dtype,
        "feature_widths": args.dims,
        "seed": seed,
        "aic_reference": "hierarchy-aware pipeline with SPTILE=96 (g=6)",
        "aic_ablation": "without hierarchy-aware pipeline, SPTILE=16 (g=1)",
        "aiv_reference": "Naive CSR",
        "aiv_variants": ["Multiple Buffer", "Multiple Buffer + Batched Process (batch=8, buffers=64)",
                         "Round-Robin Ring Buffer"],
        "comparisons": len(cases),
        "passed": failed == 0,
        "failed": failed,
        "cases": cases,
    }
    write_report(report, args.output or ROOT / "results" / f"aic_aiv_correctness_{args.dtype}.json")
    if failed:
        raise SystemExit(f"FAIL: {failed}/{len(cases)} comparisons failed")
    print(f"PASS: all {len(cases)} ablation comparisons passed; no timing collected")
    return 0


# ---------------------------------------------------------------- aiv-bitwise

def aiv_bitwise_args(argv: Sequence[str]):
    p = argparse.ArgumentParser(prog="checks.py aiv-bitwise",
                                description="Compare the pure vector branch of spmm_ascend_cube with "
                                            "spmm_csr. No timing is collected.")
    add_selection(p)
    p.add_argument("--dim", dest="dims", action="append", type=int,
                   help="Feature width; repeat to test several widths.")
    p.add_argument("--dims", dest="dims_many", nargs="+", type=int,
                   help="Several feature widths at once.")
    p.add_argument("--dtype", choices=("fp16", "fp32"), default="fp16")
    p.add_argument("--seed", type=int, default=2027)
    p.add_argument("--atol", type=float, default=0.0)
    p.add_argument("--rtol", type=float, default=0.0)
    p.add_argument("--output", type=Path,
                   help="JSON output (default: results/aiv_bitwise_correctness_<dtype>.json).")
    args = p.parse_args(argv)
    if args.index is not None and (args.start != 0 or args.stop is not None or args.limit is not None):
        p.error("--index cannot be combined with --start, --stop, or --limit")
    if args.dims is not None and args.dims_many is not None:
        p.error("use either repeated --dim or --dims, not both")
    if args.dims_many is not None:
        args.dims = args.dims_many
    elif args.dims is None:
        args.dims = [16, 32, 64, 128, 256]
    check_dims(p, args.dims, args.dtype)
    if args.atol < 0 or args.rtol < 0:
        p.error("--atol and --rtol must be non-negative")
    return args


def aiv_bitwise_dataset(path: Path, dataset_dir: Path, args, dtype) -> List[Dict]:
    name, rows, cols, crow, col = D.load_payload(path)
    relative = path.relative_to(dataset_dir).as_posix()
    seed = D.stable_seed(args.seed, relative)
    g = torch.Generator().manual_seed(seed)
    values = (torch.rand(col.numel(), generator=g) * 2 - 1).to(dtype)
    cases = []
    for dim in args.dims:
        dense = (torch.rand((cols, dim), generator=g) * 2 - 1).to(dtype)
        vector = run_ablation("aiv-round-robin", rows, cols, crow, col, values, dense)
        reference = run_ablation("aiv-naive", rows, cols, crow, col, values, dense)
        m = compare(vector, reference, args.atol, args.rtol, "pure-AIV",
                    names=("aiv_value", "reference_value"))
        m.pop("bitwise_equal")
        record = {"dataset": name, "path": relative, "rows": rows, "cols": cols, "nnz": col.numel(),
                  "feature_width": dim, "dtype": args.dtype, "dataset_seed": seed, **m}
        cases.append(record)
        print(f"{'PASS' if record['passed'] else 'FAIL'}: dataset={name}, width={dim}, dtype={args.dtype}, "
              f"mismatches={record['mismatch_count']}, max_abs_error={record['max_abs_error']:.8g}")
    return cases


def aiv_bitwise(argv: Sequence[str]) -> int:
    args = aiv_bitwise_args(argv)
    require_gpu()
    dataset_dir = dataset_dir_of(args)
    paths = discover(args, dataset_dir)
    dtype = torch.float16 if args.dtype == "fp16" else torch.float32
    cases = []
    for i, path in enumerate(paths, start=1):
        print(f"[{i}/{len(paths)}] validating {path.relative_to(dataset_dir)}")
        cases.extend(aiv_bitwise_dataset(path, dataset_dir, args, dtype))
    failed = sum(not c["passed"] for c in cases)
    report = {
        "schema_version": 1,
        "check": "pure AIV spmm_ascend_cube versus spmm_csr",
        "timing_collected": False,
        "dataset_dir": str(dataset_dir),
        "dtype": args.dtype,
        "feature_widths": args.dims,
        "seed": args.seed,
        "atol": args.atol,
        "rtol": args.rtol,
        "selected_datasets": len(paths),
        "comparisons": len(cases),
        "passed": len(cases) - failed,
        "failed": failed,
        "cases": cases,
    }
    write_report(report, args.output or ROOT / "results" / f"aiv_bitwise_correctness_{args.dtype}.json")
    if failed:
        raise SystemExit(f"FAIL: {failed}/{len(cases)} AIV comparisons did not match")
    print(f"PASS: {len(cases)} AIV comparisons matched spmm_csr; no timing was collected")
    return 0


def main(argv: Optional[Sequence[str]] = None) -> int:
    argv = list(sys.argv[1:] if argv is None else argv)
    if not argv or argv[0] not in MODES:
        sys.stderr.write("Usage: python checks.py {aic-aiv|aiv-bitwise|task-mapping} [arguments]\n")
        return 2
    return {"task-mapping": task_mapping, "aic-aiv": aic_aiv, "aiv-bitwise": aiv_bitwise}[argv[0]](argv[1:])


if __name__ == "__main__":
    sys.exit(main())
