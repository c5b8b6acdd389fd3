"""Benchmark of the MI355X SpMM hot path (one JSON line on stdout).

Default workload: benchmark configuration 2 (power-law CSR 100000x100000, ~2.0M nnz,
N=128 fp16, fp32 accumulate) — the configuration the headline metric
"SpMM GFLOP/s (2*nnz*N/t) and HBM GB/s % of peak, N=128 fp16" is quoted on.
A step is one SpMM call over resident device inputs.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2] [--width N]
                       [--op csr|mixed|mixed-empty|bcsr|graph|preprocess] [--no-cpu] [--no-block-path] [--no-cold]
       python bench.py --copy-calibration

``--op mixed`` times ``spmm_ascend_cube`` on the output of the GPU
``preprocess`` (block windows on MFMA, the rest on the gather path); ``--op
bcsr`` on the output of ``csr_to_bcsr`` (every window on MFMA); ``--op
graph`` times pack_node_tensor -> spmm_ascend_cube on P A P^T ->
restore_node_tensor (``preprocess(graph_layout=True)``).  ``--op preprocess``
times the GPU preprocessing pipelines themselves (csr_to_bcsr,
block_level_split, preprocess) against the oracle's C restatement of the
reference's host routines.  Unless
``--no-block-path`` is given, the line also carries ``block_path``: config 3
(block-banded) at N=128 fp16, ``spmm_ascend_cube`` against ``spmm_csr`` on the
same matrix.  ``--copy-calibration`` runs a plain 256 MiB device copy five
times, the reference kernel for scaling the FETCH_SIZE / WRITE_SIZE counters,
and prints the copy bandwidth.

Only one GPU is used; --gpus > 1 exits with a message.
"""

from __future__ import annotations

import argparse
import ctypes
import glob
import hashlib
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
MFMA_PEAK_TFLOPS = {"fp16": 2500.0, "fp32": 157.3}

# HBM-side traffic per call of the op, from rocprofv3 --pmc runs of this
# script (FETCH_SIZE and WRITE_SIZE, KiB per dispatch, summed over the op's
# kernels, warm calls only: --no-cold), scaled by what the same counters read
# for a plain 256 MiB device copy (--copy-calibration: FETCH_SIZE reads 0.5 x
# the bytes copied, WRITE_SIZE 1.0 x).  The counters see L2-to-fabric
# traffic, Infinity Cache hits included.  Keyed by (config, op, width); the
# runs are summarised in profiles/*_traffic.md.  Each entry records the hash
# of the kernel sources it was measured on (kernel_sources_hash); when the
# sources differ, the line reports traffic null with the reason.
# The kernels one timed call launches (the roofline's event time covers all
# of them, in launch order on one stream).
OP_KERNELS = {
    "csr": ("segment_classify + gather_tiles + gather_post (one spmm_csr call; segment_classify and "
            "gather_tiles' segment work-groups only for inputs of at least 2^20 nonzeros and a dense "
            "operand of at most 128 MiB)"),
    "mixed-empty": "gather_tiles + gather_post (spmm_ascend_cube, empty block part)",
    "bcsr": "block_windows",
    "mixed": "gather_tiles + gather_post + block_windows",
    "graph": ("fill_minus_one + scatter_inverse + gather_rows (pack) + gather_tiles + gather_post + "
              "block_windows + gather_rows (restore)"),
}
FETCH_SCALE = 2.0
WRITE_SCALE = 1.0
PMC_KIB = {
    (2, "csr", 128): {"fetch_kib": 151664.0, "write_kib": 32708.3, "sources": "113fc3377585db2c",
                      "profile": "profiles/gather_c2_csr_n128_traffic.md"},
    (3, "mixed", 128): {"fetch_kib": 95199.2, "write_kib": 28595.1, "sources": "113fc3377585db2c",
                        "profile": "profiles/mixed_c3_n128_traffic.md"},
    (3, "bcsr", 128): {"fetch_kib": 35790.3, "write_kib": 16384.0, "sources": "113fc3377585db2c",
                       "profile": "profiles/block_c3_bcsr_n128_traffic.md"},
    (3, "bcsr", 256): {"fetch_kib": 47033.9, "write_kib": 32768.0, "sources": "113fc3377585db2c",
                       "profile": "profiles/block_c3_bcsr_n256_traffic.md"},
    (4, "mixed", 512): {"fetch_kib": 409029.1, "write_kib": 209044.9, "sources": "113fc3377585db2c",
                        "profile": "profiles/mixed_c4_n512_traffic.md"},
    (1, "csr", 128): {"fetch_kib": 15795.3, "write_kib": 8256.0, "sources": "113fc3377585db2c",
                      "profile": "profiles/gather_c1_csr_n128_traffic.md"},
    (3, "csr", 128): {"fetch_kib": 98295.3, "write_kib": 73071.9, "sources": "113fc3377585db2c",
                      "profile": "profiles/gather_c3_csr_n128_traffic.md"},
    (3, "mixed", 256): {"fetch_kib": 165836.2, "write_kib": 56965.8, "sources": "113fc3377585db2c",
                        "profile": "profiles/mixed_c3_n256_traffic.md"},
    (4, "mixed", 64): {"fetch_kib": 56335.0, "write_kib": 26255.0, "sources": "113fc3377585db2c",
                       "profile": "profiles/mixed_c4_n64_traffic.md"},
    # Per call: the op's kernels times their dispatches per call (four column
    # passes of gather_tiles, gather_post and block_windows; gather_rows for P
    # and for P^T; scatter_inverse and fill_minus_one once).
    (5, "graph", 512): {"fetch_kib": 36690259.8, "write_kib": 7052596.5, "sources": "113fc3377585db2c",
                        "profile": "profiles/graph_c5_n512_traffic.md"},
}


def kernel_sources_hash() -> str:
    """sha256 (first 16 hex digits) of the library's kernel sources: the
    HIP files and headers under ascend-spmm_amd/csrc, by name and content."""
    h = hashlib.sha256()
    csrc = os.path.join(REPO, "ascend-spmm_amd", "csrc")
    for path in sorted(glob.glob(os.path.join(csrc, "*.hip")) + glob.glob(os.path.join(csrc, "*.h"))):
        h.update(os.path.basename(path).encode())
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def measured_traffic(config: int, op: str, width: int):
    """(bytes per call, note): the PMC table's traffic when it was measured on
    the current kernel sources, else (None, the reason)."""
    pmc = PMC_KIB.get((config, op, width))
    if pmc is None:
        return None, "no counter run for this configuration"
    if pmc["sources"] != kernel_sources_hash():
        return None, f"stale: kernel sources changed since the counter run ({pmc['profile']})"
    return int(1024 * (pmc["fetch_kib"] * FETCH_SCALE + pmc["write_kib"] * WRITE_SCALE)), pmc["profile"]


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def host_cpu() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


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
                   f"{t * 1e3:.1f} ms/rep, torch threads {threads}, os.cpu_count()={os.cpu_count()}, "
                   f"{host_cpu()}"),
    }


def time_calls(step, steps: int, warmup: int, cold: bool = False):
    """Wall ms per step over `steps` back-to-back calls (synchronised on both
    sides) and the HIP-event ms per call, events recorded on the stream the
    ops launch on (torch's current stream).  Warm: one event pair brackets
    the whole loop, so no timing marker sits between calls.  With cold=True,
    a 512 MiB scratch write runs before every call to evict L2 and the
    Infinity Cache, and each call is bracketed by its own event pair."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    if not cold:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(steps):
            step()
        e1.record(stream)
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3 / steps
        return wall_ms, e0.elapsed_time(e1) / steps
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    scratch = torch.empty(512 * 1024 * 1024, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        scratch.fill_(i & 0xFF)
        ev[i][0].record(stream)
        step()
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    return wall_ms, float(np.mean([a.elapsed_time(b) for a, b in ev]))


def graph_ms(step, calls: int = 10, replays: int = 20) -> float:
    """HIP-event ms per call when `calls` back-to-back calls are captured in
    one HIP graph (torch.cuda.graph) and the graph is replayed `replays`
    times: the per-call time without host launch overhead."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls):
            step()
    graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(replays):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / (replays * calls)
    del graph
    torch.cuda.synchronize()
    return ms


def device_csr(w, dev):
    return (torch.from_numpy(w.crow.astype(np.int32)).to(dev),
            torch.from_numpy(w.col.astype(np.int32)).to(dev),
            torch.from_numpy(w.values).to(dev))


def mixed_operands(spmm_npu, w, dev, graph_layout: bool):
    """GPU preprocess of the workload; returns the spmm_ascend_cube operands
    (without dense) and the preprocessing dict.  Not timed."""
    crow, col, val = device_csr(w, dev)
    p = spmm_npu.preprocess(crow, col, val, w.rows, w.cols, 16, graph_layout)
    i32 = torch.int32
    ccol = p["renumbered_unique_col_ids"] if graph_layout else p["unique_col_ids"]
    vcol = p["renumbered_vcol_indices"] if graph_layout else p["vcol_indices"]
    cstart = spmm_npu.make_start(p["crow_window_ptr"], 20).to(dev)
    vstart = spmm_npu.make_start(p["vrow_window_ptr"], 40).to(dev)
    ops = (p["crow_window_ptr"].to(i32), ccol.to(i32), p["value"],
           p["vrow_window_ptr"].to(i32), vcol.to(i32), p["vvalue"])
    return ops, cstart, vstart, p


class _CsrDesc(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_int64), ("nnz", ctypes.c_int64), ("dense_rows", ctypes.c_int64),
                ("width", ctypes.c_int64), ("index_type", ctypes.c_int32), ("value_type", ctypes.c_int32)]


LIBRARY = os.path.join(REPO, "ascend-spmm_amd", "libspmm_mi355x.so")


def probe_limits_note(w, width: int, elem: int):
    """Why the position-order probe cannot run on this workload, or None.
    spmm_gather_probe takes int32 column ids, rows of at most 64 lanes of 16
    bytes (fp16 N <= 512, fp32 N <= 256) and a dense operand within 4 GB."""
    if width * elem > 1024:
        return f"rows of {width * elem} bytes exceed the probe's 64 lanes of 16 bytes"
    if w.cols * width * elem > 0xFFFFF000:
        return "dense operand beyond the probe's 4 GB buffer extent"
    return None


def position_order_probe_ms(col, val, dense, w, steps: int, warmup: int) -> float:
    """HIP-event ms per call of the gather-rate probe (spmm_gather_probe of
    the C ABI): the gather path's dense-row loads over the same nonzeros and
    ranges, in position order, without rows, partial sums or output rows.
    spmm_csr deals long rows' segments to the XCDs by column slab, so it can
    run faster than this probe: the probe is a reference rate for the
    position-order gather, not a ceiling of spmm_csr."""
    lib = ctypes.CDLL(LIBRARY)
    lib.spmm_last_error.restype = ctypes.c_char_p
    lib.spmm_gather_probe_sink.restype = ctypes.c_size_t
    d = _CsrDesc(w.rows, w.nnz, w.cols, dense.shape[1], 0, 0 if dense.dtype == torch.float16 else 1)
    sink = torch.empty(max(int(lib.spmm_gather_probe_sink(ctypes.byref(d))), 4), dtype=torch.float32,
                       device=dense.device)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def step():
        rc = lib.spmm_gather_probe(ctypes.byref(d), p(col), p(val), p(dense), p(sink), stream)
        if rc != 0:
            raise RuntimeError(lib.spmm_last_error().decode())

    return time_calls(step, steps, warmup)[1]


def rowscalar_ms(crow, col, val, dense, w) -> float:
    """HIP-event ms per call of the thread-per-row scalar CSR baseline
    (spmm_csr_rowscalar_run of the C ABI; one thread per output row), 1
    warm-up and 3 timed calls."""
    lib = ctypes.CDLL(LIBRARY)
    lib.spmm_last_error.restype = ctypes.c_char_p
    out = torch.empty(w.rows, dense.shape[1], dtype=dense.dtype, device=dense.device)
    d = _CsrDesc(w.rows, w.nnz, w.cols, dense.shape[1], 0, 0 if dense.dtype == torch.float16 else 1)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def step():
        rc = lib.spmm_csr_rowscalar_run(ctypes.byref(d), p(crow), p(col), p(val), p(dense), p(out), stream)
        if rc != 0:
            raise RuntimeError(lib.spmm_last_error().decode())

    return time_calls(step, 3, 1)[1]


def block_path(spmm_npu, dev, steps: int, warmup: int) -> dict:
    """Config 3 (block-banded) at N=128 fp16: spmm_ascend_cube on the output
    of the GPU preprocess (the reference's headline pipeline) and on the
    output of csr_to_bcsr (every window on MFMA, the reference's AIC-only
    configuration), each against spmm_csr on the same matrix."""
    w = workloads.make(3)
    width = 128
    dense = torch.from_numpy(w.dense(width)).to(dev)
    crow, col, val = device_csr(w, dev)
    start = spmm_npu.make_start(crow, 40).to(dev)
    ops, cstart, vstart, p = mixed_operands(spmm_npu, w, dev, False)
    i32 = torch.int32
    b = spmm_npu.csr_to_bcsr(crow, col, val, w.rows, w.cols, 16)
    bops = (b["crow_window_ptr"].to(i32), b["unique_col_ids"].to(i32), b["value"],
            torch.zeros(1, dtype=i32, device=dev), torch.zeros(0, dtype=i32, device=dev),
            torch.zeros(0, dtype=val.dtype, device=dev))
    bstart = spmm_npu.make_start(b["crow_window_ptr"], 20).to(dev)
    _, csr_ms = time_calls(lambda: spmm_npu.spmm_csr(crow, col, val, dense, start), steps, warmup)
    scalar_ms = rowscalar_ms(crow, col, val, dense, w)
    _, mixed_ms = time_calls(lambda: spmm_npu.spmm_ascend_cube(*ops, dense, cstart, vstart), steps, warmup)
    _, bcsr_ms = time_calls(lambda: spmm_npu.spmm_ascend_cube(*bops, dense, bstart, start), steps, warmup)
    nblk = int(p["crow_window_ptr"][-1].item())
    nblk_all = int(b["crow_window_ptr"][-1].item())
    mfma_tflops = 2.0 * 16 * nblk_all * width / (bcsr_ms / 1e3) / 1e12
    return {
        "workload": f"{w.name} {w.rows}x{w.cols} nnz={w.nnz} N={width} fp16",
        "spmm_csr_ms": round(csr_ms, 5),
        "preprocess_spmm_ascend_cube_ms": round(mixed_ms, 5),
        "speedup_preprocess_vs_spmm_csr": round(csr_ms / mixed_ms, 3),
        "bcsr_spmm_ascend_cube_ms": round(bcsr_ms, 5),
        "speedup_bcsr_vs_spmm_csr": round(csr_ms / bcsr_ms, 3),
        "gflops_bcsr": round(2.0 * w.nnz * width / (bcsr_ms / 1e3) / 1e9, 1),
        "preprocess_aic_windows": int(p["crow_window_ptr"].numel() - 1),
        "preprocess_aic_blocks_16x1": nblk,
        "preprocess_vector_nnz": int(p["vvalue"].numel()),
        "bcsr_blocks_16x1": nblk_all,
        "rowscalar_csr_ms": round(scalar_ms, 5),
        "speedup_preprocess_vs_rowscalar": round(scalar_ms / mixed_ms, 2),
        "speedup_bcsr_vs_rowscalar": round(scalar_ms / bcsr_ms, 2),
        "bcsr_mfma_executed_tflops": round(mfma_tflops, 2),
        "bcsr_mfma_utilisation": round(mfma_tflops / MFMA_PEAK_TFLOPS["fp16"], 4),
    }


def preprocessing(spmm_npu, w, steps: int, warmup: int, cpu: bool) -> int:
    """--op preprocess: the GPU preprocessing pipelines (csr_to_bcsr,
    csr_to_ascend_cube, block_level_split with the harness ratio (222/190)/2, preprocess; the
    graph layout for config 5) on device-resident CSR, wall time per call
    (each pipeline synchronises once to size its outputs), against the
    oracle's single-threaded C restatement of the reference's host routines
    on the same matrix (extension/custom_op.cpp:594-746, 429-592, 1146-1348,
    765-1110).
    Bytes per call: the CSR read (int32 indices) plus every output written."""
    dev = torch.device("cuda:0")
    crow, col, val = device_csr(w, dev)
    graph = w.name.startswith("C5")
    ratio = (222.0 / 190.0) * 0.5
    pipelines = {
        "csr_to_bcsr": lambda: spmm_npu.csr_to_bcsr(crow, col, val, w.rows, w.cols, 16),
        "csr_to_ascend_cube": lambda: spmm_npu.csr_to_ascend_cube(crow, col, val, w.rows, w.cols, 16),
        "block_level_split": lambda: spmm_npu.block_level_split(crow, col, val, w.rows, w.cols, ratio, 16),
        "preprocess": lambda: spmm_npu.preprocess(crow, col, val, w.rows, w.cols, 16, graph),
    }
    in_bytes = 4 * (w.rows + 1) + (4 + w.values.itemsize) * w.nnz
    out = {}
    for name, fn in pipelines.items():
        res = fn()
        torch.cuda.synchronize()
        out_bytes = sum(t.numel() * t.element_size() for t in res.values() if torch.is_tensor(t))
        del res
        wall_ms, _ = time_calls(fn, steps, warmup)
        out[name] = {"ms": round(wall_ms, 3), "bytes": int(in_bytes + out_bytes),
                     "gbps": round((in_bytes + out_bytes) / (wall_ms / 1e3) / 1e9, 1)}
        log(f"[bench] {name}: {wall_ms:.3f} ms")
    cpu_out = None
    if cpu:
        sys.path.insert(0, os.path.join(REPO, "oracle"))
        import oracle  # checker-only import: the CPU baseline leg

        c32, k32 = w.crow.astype(np.int32), w.col.astype(np.int32)
        cpu_fns = {
            "csr_to_bcsr": lambda: oracle.csr_to_bcsr(c32, k32, w.values, w.rows, w.cols, 16),
            "csr_to_ascend_cube": lambda: oracle.csr_to_ascend_cube(c32, k32, w.values, w.rows, w.cols, 16),
            "block_level_split": lambda: oracle.block_level_split(c32, k32, w.values, w.rows, w.cols, ratio, 16),
            "preprocess": lambda: oracle.preprocess(c32, k32, w.values, w.rows, w.cols, 16, graph),
        }
        cpu_out = {}
        for name, fn in cpu_fns.items():
            t0 = time.perf_counter()
            fn()
            cpu_out[name] = round((time.perf_counter() - t0) * 1e3, 1)
            out[name]["cpu_ms"] = cpu_out[name]
            out[name]["speedup_vs_cpu"] = round(cpu_out[name] / out[name]["ms"], 1)
            log(f"[bench] oracle {name}: {cpu_out[name]:.1f} ms")
    pre = out["preprocess"]
    result = {
        "metric": "GPU preprocessing throughput (nnz per second of preprocess)",
        "value": round(w.nnz / (pre["ms"] / 1e3) / 1e6, 2),
        "unit": "Mnnz/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": pre["ms"],
        "higher_is_better": True,
        "data": "synthetic (seeded generator of benchmark configuration %s)" % w.name[1],
        "config": {"workload": f"{w.name} {w.rows}x{w.cols} nnz={w.nnz} {w.dtype}",
                   "op": "preprocess" + (" (graph layout)" if graph else ""), "index": "int32"},
        "roofline": {"bound": "hbm", "achieved": pre["gbps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(pre["gbps"] / HBM_PEAK_GBPS, 4), "traffic": None,
                     "bytes_per_call": pre["bytes"]},
        "pipelines": out,
        "cpu_baseline": None if cpu_out is None else {
            "value": round(w.nnz / (cpu_out["preprocess"] / 1e3) / 1e6, 2), "unit": "Mnnz/s", "cores": 1,
            "kind": "port",
            "sample": "full matrix, one call of the oracle's C restatement of the reference's "
                      "single-threaded host routine"},
    }
    print(json.dumps(result), flush=True)
    return 0


def copy_gbps(n: int, copies: int, warmup: int) -> tuple:
    """A plain device copy of n bytes (torch's copy kernel): (ms per copy,
    read + write GB/s).  At 1 GiB the source and destination (2 GiB) are far
    past the 256 MB Infinity Cache, so this is the achievable HBM rate."""
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    _, ms = time_calls(lambda: dst.copy_(src), copies, warmup)
    del src, dst
    return ms, 2 * n / (ms / 1e3) / 1e9


def copy_calibration() -> int:
    n = 256 * 1024 * 1024
    ms, gbps = copy_gbps(n, 5, 0)
    print(json.dumps({"copy_bytes": n, "copies": 5, "ms_per_copy": round(ms, 4),
                      "copy_gbps_read_plus_write": round(gbps, 1)}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--width", type=int, default=None)
    ap.add_argument("--op", choices=["csr", "mixed", "mixed-empty", "bcsr", "graph", "preprocess"], default="csr")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-block-path", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--no-cold", action="store_true", help="skip the cold-cache timing (counter runs)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no "
              "multi-GPU path: the SpMM shards by row windows with no exchange when the dense "
              "operand is replicated, so N GPUs is N independent runs of this benchmark.",
              file=sys.stderr)
        return 2
    if args.copy_calibration:
        return copy_calibration()

    import spmm_npu

    w = workloads.make(args.config)
    if args.op == "preprocess":
        return preprocessing(spmm_npu, w, min(args.steps, 10), min(args.warmup, 2), not args.no_cpu)
    width = args.width or w.widths[0]
    B = w.dense(width)
    log(f"[bench] workload {w.name}: {w.rows}x{w.cols}, nnz={w.nnz}, N={width}, {w.dtype}")

    dev = torch.device("cuda:0")
    dense = torch.from_numpy(B).to(dev)
    alg_bytes = workloads.algorithmic_bytes(w, width)
    if args.op == "csr":
        crow, col, val = device_csr(w, dev)
        start = spmm_npu.make_start(crow, 40).to(dev)

        def step():
            return spmm_npu.spmm_csr(crow, col, val, dense, start)
        op_name = "spmm_csr"
    elif args.op == "mixed-empty":
        crow, col, val = device_csr(w, dev)
        e_i = torch.zeros(0, dtype=torch.int32, device=dev)
        e_v = torch.zeros(0, dtype=val.dtype, device=dev)
        z1 = torch.zeros(1, dtype=torch.int32, device=dev)
        z20 = torch.zeros(20, dtype=torch.int32, device=dev)
        start = spmm_npu.make_start(crow, 40).to(dev)

        def step():
            return spmm_npu.spmm_ascend_cube(z1, e_i, e_v, crow, col, val, dense, z20, start)
        op_name = "spmm_ascend_cube(vector part only)"
    elif args.op == "bcsr":
        crow, col, val = device_csr(w, dev)
        b = spmm_npu.csr_to_bcsr(crow, col, val, w.rows, w.cols, 16)
        i32 = torch.int32
        bops = (b["crow_window_ptr"].to(i32), b["unique_col_ids"].to(i32), b["value"],
                torch.zeros(1, dtype=i32, device=dev), torch.zeros(0, dtype=i32, device=dev),
                torch.zeros(0, dtype=val.dtype, device=dev))
        cstart = spmm_npu.make_start(b["crow_window_ptr"], 20).to(dev)
        vstart = torch.zeros(40, dtype=i32, device=dev)

        def step():
            return spmm_npu.spmm_ascend_cube(*bops, dense, cstart, vstart)
        op_name = "csr_to_bcsr -> spmm_ascend_cube (block part only; conversion untimed)"
    elif args.op == "mixed":
        ops, cstart, vstart, _ = mixed_operands(spmm_npu, w, dev, False)

        def step():
            return spmm_npu.spmm_ascend_cube(*ops, dense, cstart, vstart)
        op_name = "preprocess -> spmm_ascend_cube (preprocess untimed)"
    else:
        ops, cstart, vstart, p = mixed_operands(spmm_npu, w, dev, True)
        inv = p["inv_permutation"]
        packed_rows = int(p["packed_rows"][0].item())

        def step():
            packed = spmm_npu.pack_node_tensor(dense, inv, packed_rows)
            out = spmm_npu.spmm_ascend_cube(*ops, packed, cstart, vstart)
            return spmm_npu.restore_node_tensor(out, inv)
        op_name = "pack_node_tensor -> spmm_ascend_cube(P A P^T) -> restore_node_tensor"
        s = 2 if w.dtype == "fp16" else 4
        alg_bytes += 2 * s * w.cols * width + 2 * s * w.rows * width + 2 * 8 * w.rows

    log(f"[bench] {op_name}: warmup {args.warmup}, steps {args.steps}")
    wall_ms, event_ms = time_calls(step, args.steps, args.warmup)
    log(f"[bench] wall {wall_ms:.4f} ms/step, events {event_ms:.4f} ms/call")
    cold_ms = None
    if not args.no_cold:
        _, cold_ms = time_calls(step, min(args.steps, 10), 1, cold=True)
        log(f"[bench] cold-cache events {cold_ms:.4f} ms/call")

    graph_call_ms = None
    if args.op != "graph":  # the graph op's Python-side permutation checks read the device
        graph_call_ms = graph_ms(step)
        log(f"[bench] HIP graph replay {graph_call_ms:.4f} ms/call")

    copy_rate = copy_gbps(1 << 30, 5, 1)[1]
    log(f"[bench] 1 GiB device copy: {copy_rate:.1f} GB/s (read + write)")
    probe_ms, probe_note = None, "timed for the csr op only"
    if args.op == "csr":
        probe_note = probe_limits_note(w, width, 2 if w.dtype == "fp16" else 4)
        if probe_note is None:
            probe_ms = position_order_probe_ms(col, val, dense, w, args.steps, args.warmup)
            log(f"[bench] position-order gather probe {probe_ms:.4f} ms/call")

    flops = 2.0 * w.nnz * width
    t_s = wall_ms / 1e3
    achieved = alg_bytes / (event_ms / 1e3) / 1e9
    traffic, traffic_source = measured_traffic(args.config, args.op, width)
    s_b = 2 if w.dtype == "fp16" else 4
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
        "data": "synthetic (seeded generator of benchmark configuration %d)" % args.config,
        "config": {
            "workload": f"{w.name} {w.rows}x{w.cols} nnz={w.nnz} N={width} {w.dtype}",
            "op": op_name,
            "accumulate": "fp32",
            "index": "int32",
        },
        "hbm_gbps_algorithmic": round(alg_bytes / t_s / 1e9, 1),
        "cold_cache_ms_per_call": None if cold_ms is None else round(cold_ms, 5),
        "graph_replay_ms_per_call": None if graph_call_ms is None else round(graph_call_ms, 5),
        "roofline": {
            "bound": "hbm",
            "kernels": OP_KERNELS.get(args.op, ""),
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "kernel_sources_hash": kernel_sources_hash(),
            "traffic_gbps": None if traffic is None else round(traffic / (event_ms / 1e3) / 1e9, 1),
            "traffic_frac": None if traffic is None else round(traffic / (event_ms / 1e3) / 1e9 / HBM_PEAK_GBPS, 4),
            "copy_gbps": round(copy_rate, 1),
            "traffic_frac_of_copy": None if traffic is None else round(traffic / (event_ms / 1e3) / 1e9 / copy_rate, 4),
            "algorithmic_bytes_per_call": alg_bytes,
            "gather_model_bytes": int(w.nnz * width * s_b),
            "event_ms_per_call": round(event_ms, 5),
            # The position-order gather probe (op csr): the same dense-row
            # loads over the same ranges in position order, without rows or
            # output.  A reference rate, not a ceiling: spmm_csr's slab-dealt
            # segments can beat it.
            "position_order_probe_ms_per_call": None if probe_ms is None else round(probe_ms, 5),
            "position_order_probe_gather_model_gbps": None if probe_ms is None else round(
                w.nnz * width * s_b / (probe_ms / 1e3) / 1e9, 1),
            "spmm_time_over_probe_time": None if probe_ms is None else round(event_ms / probe_ms, 4),
            "position_order_probe_note": probe_note,
        },
    }
    if not args.no_block_path and args.config == 2 and args.op == "csr":
        log("[bench] block path (config 3, N=128) ...")
        result["block_path"] = block_path(spmm_npu, dev, 20, 5)
    if not args.no_cpu:
        log("[bench] CPU baseline ...")
        result["cpu_baseline"] = cpu_baseline(w, B, args.cpu_budget)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
