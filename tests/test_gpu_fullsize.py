"""Full-size GPU parity of every benchmark configuration (tests/workloads.py,
configurations 1-5 at their stated sizes) against the fp64 oracle, the way
the reference's harness checks whole matrices
(tests/task_mapping/correctness.py:170-182,
tests/aic_aiv_ablation/bitwise_correctness.py:138-175).

Each test runs the operator path bench.py times for that configuration, on
the same seeded inputs, and compares with the fp64 product at the
reference's tolerance (atol = rtol = 2e-2 for fp16, 1e-4 for fp32,
tests/task_mapping/correctness.py:140-143) with no slack, or bit for bit for
the layout operators:

* C1 (uniform 16384^2, fp32, N=128): spmm_csr, also against the reference's
  own CPU formula (torch sparse.mm fp32).
* C2 (power-law 100000^2, fp16, N=128): spmm_csr (test_gpu_spmm holds the
  same check; here beside the others at the generator's corrected size).
* C3 (block-banded 65536^2, fp16) at N=128 and N=256: spmm_csr;
  csr_to_bcsr -> spmm_ascend_cube; preprocess (bit-exact against the
  oracle) -> spmm_ascend_cube -> restore_node_tensor.
* C4 (mixed 200000^2, fp16) at N=64 and N=512: preprocess ->
  spmm_ascend_cube -> restore_node_tensor, and block_level_split (the
  harness ratio) -> spmm_ascend_cube.
* C5 (graph 1048576^2, ~32M nnz, fp32, N=512): preprocess(graph_layout=True)
  bit-exact against the oracle, then pack_node_tensor -> spmm_ascend_cube
  on the renumbered ids -> restore_node_tensor against fp64 on a seeded
  sample of 65,536 rows plus every row of more than 1024 nonzeros.
"""

import functools

import numpy as np
import pytest
import torch

import oracle as O
import workloads as W
from test_gpu_preprocess import assert_same

pytestmark = pytest.mark.gpu

TOL = {"fp16": 2e-2, "fp32": 1e-4}


@functools.lru_cache(maxsize=1)
def workload(config_id):
    print(f"[fullsize] generating configuration {config_id}", flush=True)
    return W.make(config_id)


def dev_csr(w):
    return (torch.from_numpy(w.crow.astype(np.int32)).cuda(), torch.from_numpy(w.col.astype(np.int32)).cuda(),
            torch.from_numpy(w.values).cuda())


def assert_close(actual, expected, dtype, degrees=None, what=""):
    """|actual - expected| <= tol + tol |expected| for every element (the
    reference's isclose), reporting the failing rows' degrees."""
    tol = TOL[dtype]
    a = actual.float().cpu().double().numpy() if torch.is_tensor(actual) else actual
    err = np.abs(a - expected)
    bad = ~(err <= tol + tol * np.abs(expected))
    if bad.any():
        rows = np.unique(np.nonzero(bad)[0])
        deg = "" if degrees is None else f", degrees of failing rows {np.sort(degrees[rows])[::-1][:10].tolist()}"
        pytest.fail(f"{what}: {int(bad.sum())} of {bad.size} elements outside {tol} in {rows.size} rows, "
                    f"max abs err {float(err.max()):.3e}{deg}")


def mixed(spmm_npu, p, dense, graph_layout=False):
    i32 = torch.int32
    ccol = p["renumbered_unique_col_ids"] if graph_layout else p["unique_col_ids"]
    vcol = p["renumbered_vcol_indices"] if graph_layout else p["vcol_indices"]
    return spmm_npu.spmm_ascend_cube(
        p["crow_window_ptr"].cuda().to(i32), ccol.cuda().to(i32), p["value"].cuda(),
        p["vrow_window_ptr"].cuda().to(i32), vcol.cuda().to(i32), p["vvalue"].cuda(), dense,
        spmm_npu.make_start(p["crow_window_ptr"], 20).cuda(), spmm_npu.make_start(p["vrow_window_ptr"], 40).cuda())


def test_c1_spmm_csr_full_size(spmm_npu):
    w = workload(1)
    B = w.dense(128)
    crow, col, val = dev_csr(w)
    out = spmm_npu.spmm_csr(crow, col, val, torch.from_numpy(B).cuda(), spmm_npu.make_start(crow, 40).cuda())
    assert out.shape == (16384, 128) and out.dtype == torch.float32
    assert_close(out, O.spmm_f64(w.crow, w.col, w.values, B), "fp32", what="C1 spmm_csr")
    ref = O.cpu_reference(w.rows, w.cols, w.crow, w.col, w.values, B)
    assert bool(torch.isclose(out.cpu(), ref, atol=1e-4, rtol=1e-4).all())


def test_c2_spmm_csr_full_size(spmm_npu):
    w = workload(2)
    B = w.dense(128)
    crow, col, val = dev_csr(w)
    out = spmm_npu.spmm_csr(crow, col, val, torch.from_numpy(B).cuda(), spmm_npu.make_start(crow, 40).cuda())
    assert_close(out, O.spmm_f64(w.crow, w.col, w.values, B), "fp16", np.diff(w.crow), "C2 spmm_csr")


@functools.lru_cache(maxsize=1)
def c3_layouts():
    """The GPU preprocess and csr_to_bcsr layouts of configuration 3 (int32
    device CSR, as bench.py builds them), the preprocess one checked bit for
    bit against the oracle."""
    import spmm_npu

    w = workload(3)
    crow, col, val = dev_csr(w)
    p = spmm_npu.preprocess(crow, col, val, w.rows, w.cols, 16, False)
    ref = O.preprocess(w.crow.astype(np.int32), w.col.astype(np.int32), w.values, w.rows, w.cols, 16, False)
    assert_same(p, ref)
    b = spmm_npu.csr_to_bcsr(crow, col, val, w.rows, w.cols, 16)
    assert_same(b, O.csr_to_bcsr(w.crow.astype(np.int32), w.col.astype(np.int32), w.values, w.rows, w.cols, 16))
    return p, b


@pytest.mark.parametrize("width", [128, 256])
def test_c3_full_size_every_path(spmm_npu, width):
    w = workload(3)
    p, b = c3_layouts()
    assert p["unique_col_ids"].numel() > 0 and p["vcol_indices"].numel() > 0  # both parts in use
    B = w.dense(width)
    expected = O.spmm_f64(w.crow, w.col, w.values, B)
    deg = np.diff(w.crow)
    dense = torch.from_numpy(B).cuda()
    crow, col, val = dev_csr(w)
    start = spmm_npu.make_start(crow, 40).cuda()
    assert_close(spmm_npu.spmm_csr(crow, col, val, dense, start), expected, "fp16", deg, f"C3 N={width} spmm_csr")
    i32 = torch.int32
    out = spmm_npu.spmm_ascend_cube(
        b["crow_window_ptr"].to(i32), b["unique_col_ids"].to(i32), b["value"],
        torch.zeros(1, dtype=i32, device="cuda"), torch.zeros(0, dtype=i32, device="cuda"),
        torch.zeros(0, dtype=torch.float16, device="cuda"), dense,
        spmm_npu.make_start(b["crow_window_ptr"], 20).cuda(), torch.zeros(40, dtype=i32, device="cuda"))
    assert out.shape == (w.rows, width)
    assert_close(out, expected, "fp16", deg, f"C3 N={width} csr_to_bcsr -> spmm_ascend_cube")
    out = mixed(spmm_npu, p, dense)
    restored = spmm_npu.restore_node_tensor(out, p["inv_permutation"].cuda())
    assert restored.shape == (w.rows, width)
    assert_close(restored, expected, "fp16", deg, f"C3 N={width} preprocess -> spmm_ascend_cube")


@functools.lru_cache(maxsize=1)
def c4_layouts():
    import spmm_npu

    w = workload(4)
    crow, col, val = dev_csr(w)
    p = spmm_npu.preprocess(crow, col, val, w.rows, w.cols, 16, False)
    h = spmm_npu.block_level_split(crow, col, val, w.rows, w.cols, (222.0 / 190.0) * 0.5, 16)
    c32, k32 = w.crow.astype(np.int32), w.col.astype(np.int32)
    assert_same(h, O.block_level_split(c32, k32, w.values, w.rows, w.cols, (222.0 / 190.0) * 0.5, 16))
    return p, h


@pytest.mark.parametrize("width", [64, 512])
def test_c4_full_size_mixed(spmm_npu, width):
    """preprocess (bit-exact at full size in test_gpu_preprocess) and
    block_level_split layouts of configuration 4 through spmm_ascend_cube."""
    w = workload(4)
    p, h = c4_layouts()
    assert p["unique_col_ids"].numel() > 0 and p["vcol_indices"].numel() > 0
    B = w.dense(width)
    expected = O.spmm_f64(w.crow, w.col, w.values, B)
    dense = torch.from_numpy(B).cuda()
    restored = spmm_npu.restore_node_tensor(mixed(spmm_npu, p, dense), p["inv_permutation"].cuda())
    assert restored.shape == (w.rows, width)
    deg = np.diff(w.crow)
    assert_close(restored, expected, "fp16", deg, f"C4 N={width} preprocess -> spmm_ascend_cube")
    out = mixed(spmm_npu, h, dense)
    assert_close(out[: w.rows], expected, "fp16", deg, f"C4 N={width} block_level_split -> spmm_ascend_cube")


@functools.lru_cache(maxsize=1)
def c5_layout():
    """GPU preprocess(graph_layout=True) of configuration 5 on the int32
    device CSR bench.py uses, checked bit for bit (every key, the transpose
    split included) against the oracle."""
    import spmm_npu

    w = workload(5)
    crow, col, val = dev_csr(w)
    print("[fullsize] C5 GPU preprocess", flush=True)
    p = spmm_npu.preprocess(crow, col, val, w.rows, w.cols, 16, True)
    print("[fullsize] C5 oracle preprocess", flush=True)
    ref = O.preprocess(w.crow.astype(np.int32), w.col.astype(np.int32), w.values, w.rows, w.cols, 16, True)
    assert_same(p, ref)
    return p


def test_c5_preprocess_graph_layout_bit_exact(spmm_npu):
    w = workload(5)
    assert abs(w.nnz - 32_000_000) < 32_000_000 * 1e-3 and int(np.diff(w.crow).max()) == 8192
    p = c5_layout()
    assert int(p["packed_layout_supported"][0]) == 1
    assert p["transpose_unique_col_ids"].numel() > 0 and p["transpose_vcol_indices"].numel() > 0


def test_c5_graph_path_full_size(spmm_npu):
    """pack -> spmm_ascend_cube(P A P^T) -> restore at full size, compared
    with fp64 on 65,536 seeded rows plus every row of more than 1024
    nonzeros (the hub rows, where fp32 accumulation is longest)."""
    w = workload(5)
    p = c5_layout()
    B = w.dense(512)
    dense = torch.from_numpy(B).cuda()
    inv = p["inv_permutation"].cuda()
    packed = spmm_npu.pack_node_tensor(dense, inv, int(p["packed_rows"][0]))
    out = spmm_npu.restore_node_tensor(mixed(spmm_npu, p, packed, graph_layout=True), inv)
    assert out.shape == (w.rows, 512) and out.dtype == torch.float32
    deg = np.diff(w.crow)
    rng = np.random.default_rng(2027 + 55)
    rows = np.union1d(rng.choice(w.rows, 65536, replace=False), np.nonzero(deg > 1024)[0])
    assert (deg[rows] > 1024).sum() == (deg > 1024).sum()
    pos = W._row_ranges(w.crow, rows)
    crow_s = np.concatenate([[0], np.cumsum(deg[rows])]).astype(np.int64)
    print(f"[fullsize] C5 fp64 on {rows.size} rows ({pos.size} nnz)", flush=True)
    expected = O.spmm_f64(crow_s, w.col[pos], w.values[pos], B)
    got = out[torch.from_numpy(rows).cuda()]
    assert_close(got, expected, "fp32", deg[rows], "C5 pack -> spmm_ascend_cube -> restore")
