"""The bench.py contract: one JSON line with the driver's keys plus
``roofline`` (and ``cpu_baseline`` unless disabled); one GPU only."""

import json
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(REPO, "bench.py")


def run_bench(*args, timeout=240):
    return subprocess.run([sys.executable, BENCH, *args], cwd=REPO, capture_output=True, text=True,
                          timeout=timeout)


def test_bench_rejects_more_than_one_gpu():
    proc = run_bench("--gpus", "2")
    assert proc.returncode == 2
    assert "one GPU only" in proc.stderr
    assert proc.stdout.strip() == ""


def test_algorithmic_bytes_closed_form():
    """bytes = 4(M+1) + (4 + s)nnz + s N K_ref + s M N, K_ref = distinct
    columns: a hand-counted 3x5 CSR, and configuration 1 against the
    closed form with every column counted, 4*16385 + 8*131072 + 2*4*16384*128
    = 17,891,332 bytes at fp32 N=128 (the generated matrix leaves a few
    columns unused)."""
    import numpy as np

    import workloads as W

    class Tiny:
        rows, cols, nnz, dtype = 3, 5, 4, "fp16"
        crow = np.array([0, 2, 2, 4])
        col = np.array([1, 4, 1, 3])

    # M=3: 16 bytes of rowptr; 4 nonzeros of 6 bytes; K_ref = 3 distinct
    # columns {1, 3, 4} of 2*16 bytes each at N=16; output 3*16*2.
    assert W.algorithmic_bytes(Tiny, 16) == 16 + 24 + 3 * 32 + 96
    w = W.make(1)
    unused = w.cols - np.unique(w.col).size
    assert 0 <= unused < 32
    assert W.algorithmic_bytes(w, 128) + 4 * 128 * unused == 17_891_332


@pytest.mark.gpu
def test_bench_json_line():
    proc = run_bench("--steps", "3", "--warmup", "1", "--no-cpu", "--no-block-path", "--no-cold")
    assert proc.returncode == 0, proc.stderr[-2000:]
    lines = [line for line in proc.stdout.splitlines() if line.strip()]
    assert len(lines) == 1
    d = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline"):
        assert key in d, key
    assert d["n_gpus"] == 1 and d["steps"] == 3 and d["warmup"] == 1
    assert d["value"] > 0 and d["unit"] == "GFLOP/s" and d["dtype"] == "fp16"
    assert "C2" in d["config"]["workload"]
    r = d["roofline"]
    for key in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert key in r, key
    assert r["bound"] == "hbm" and r["unit"] == "GB/s" and r["peak"] == 8000.0
    assert abs(r["frac"] - r["achieved"] / r["peak"]) < 1e-3
    assert r["traffic"] is None or r["traffic"] > 0


@pytest.mark.gpu
def test_bench_preprocess_line():
    """--op preprocess: the four GPU pipelines timed, the oracle's C port
    beside them (kind "port"), one JSON line."""
    proc = run_bench("--op", "preprocess", "--config", "1", "--steps", "2", "--warmup", "1")
    assert proc.returncode == 0, proc.stderr[-2000:]
    lines = [line for line in proc.stdout.splitlines() if line.strip()]
    assert len(lines) == 1
    d = json.loads(lines[0])
    assert set(d["pipelines"]) == {"csr_to_bcsr", "csr_to_ascend_cube", "block_level_split", "preprocess"}
    for p in d["pipelines"].values():
        assert p["ms"] > 0 and p["bytes"] > 0 and p["cpu_ms"] > 0
    assert d["cpu_baseline"]["kind"] == "port" and d["cpu_baseline"]["cores"] == 1
    assert d["roofline"]["bound"] == "hbm" and d["value"] > 0


def test_probe_limits_note():
    """bench.py runs the position-order probe only within spmm_gather_probe's
    limits (64 lanes of 16 bytes per row, a 4 GB dense operand); elsewhere
    the line carries the reason instead of failing."""
    sys.path.insert(0, REPO)
    import bench

    class W:
        cols = 100000

    assert bench.probe_limits_note(W, 128, 2) is None
    assert bench.probe_limits_note(W, 512, 2) is None
    assert "64 lanes" in bench.probe_limits_note(W, 1024, 2)
    assert "64 lanes" in bench.probe_limits_note(W, 512, 4)
    W.cols = 1 << 24
    assert "4 GB" in bench.probe_limits_note(W, 256, 2)


@pytest.mark.gpu
def test_bench_fp32_width_512_line():
    """A csr line at fp32 N=512 (beyond the probe's rows) still prints its
    JSON line, with the probe fields null and the reason given."""
    proc = run_bench("--config", "1", "--width", "512", "--steps", "2", "--warmup", "1", "--no-cpu",
                     "--no-block-path", "--no-cold")
    assert proc.returncode == 0, proc.stderr[-2000:]
    d = json.loads([line for line in proc.stdout.splitlines() if line.strip()][-1])
    r = d["roofline"]
    assert r["position_order_probe_ms_per_call"] is None and "64 lanes" in r["position_order_probe_note"]
    assert d["value"] > 0


def test_traffic_table_is_keyed_to_the_kernel_sources():
    """roofline.traffic comes from the PMC table only when the entry was
    measured on the current kernel sources (their hash); otherwise it is
    null with the reason, never a stale figure."""
    import sys

    sys.path.insert(0, REPO)
    import bench

    h = bench.kernel_sources_hash()
    assert len(h) == 16 and h == bench.kernel_sources_hash()
    key = (99, "csr", 16)
    bench.PMC_KIB[key] = {"fetch_kib": 1.0, "write_kib": 3.0, "sources": h, "profile": "profiles/x.md"}
    try:
        assert bench.measured_traffic(*key) == (1024 * (2 * 1 + 3), "profiles/x.md")
        bench.PMC_KIB[key]["sources"] = "0" * 16
        traffic, note = bench.measured_traffic(*key)
        assert traffic is None and note.startswith("stale")
    finally:
        del bench.PMC_KIB[key]
    assert bench.measured_traffic(98, "csr", 16)[0] is None


def test_traffic_table_matches_its_profiles():
    """Every entry of the PMC table names a committed profile that records
    the same kernel-sources hash and whose per-kernel FETCH_SIZE and
    WRITE_SIZE columns sum to the entry's figures (spmm:: kernels of the op,
    the probe excluded; weighted by the dispatches per call where the table
    gives them, as for the graph op's column passes)."""
    import re

    sys.path.insert(0, REPO)
    import bench

    for key, e in bench.PMC_KIB.items():
        text = open(os.path.join(REPO, e["profile"])).read()
        assert f"Kernel sources of the run: {e['sources']}" in text, key
        per_call = "| dispatches per call |" in text
        fetch = write = 0.0
        for row in re.findall(r"^\| `spmm::[^`]*` \| (\d+) \| ([\d.]+) \| ([\d.]+) \|", text, flags=re.M):
            k = int(row[0]) if per_call else 1
            fetch += k * float(row[1])
            write += k * float(row[2])
        assert abs(fetch - e["fetch_kib"]) < 0.5 and abs(write - e["write_kib"]) < 0.5, key
