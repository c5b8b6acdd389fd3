"""Partition methods of the task-mapping comparison (ascend-spmm_amd/
partition.py; reference tests/task_mapping/common.py:146-347) and the
correctness CLIs' argument handling (ascend-spmm_amd/checks.py; reference
tests/*/correctness.py, bitwise_correctness.py).  CPU only: the partition
logic is checked against per-edge brute force, the thresholds against their
closed form."""

import numpy as np
import pytest
import torch

import checks as C
import partition as PT


def random_csr(seed, rows, cols, max_deg, heavy=()):
    rng = np.random.default_rng(seed)
    parts = []
    for r in range(rows):
        d = int(rng.integers(0, max_deg + 1))
        if r in heavy:
            d = cols // 2
        parts.append(np.sort(rng.choice(cols, d, replace=False)))
    crow = np.zeros(rows + 1, np.int64)
    crow[1:] = np.cumsum([p.size for p in parts])
    col = np.concatenate(parts).astype(np.int64)
    vals = rng.uniform(-1, 1, col.size).astype(np.float32)
    return torch.from_numpy(crow), torch.from_numpy(col), torch.from_numpy(vals)


@pytest.mark.parametrize("rows,cols,nnz,want", [
    (0, 10, 0, 32),                       # no rows
    (100000, 100000, 1000000, 10),        # density 1e-4 < 2e-4, <= 1M rows: alpha 1.0
    (2000000, 2000000, 4000000, 4),       # > 1M rows: alpha 1.8 * 2 = 3.6 -> 3, floor 4
    (2000000, 2000000, 20000000, 18),     # alpha 1.8 * 10
    (100, 100, 5000, 12),                 # density 0.5 > 0.01: alpha 0.25 * 50
    (1000, 1000, 10000, 5),               # density 0.01 (not > 0.01): alpha 0.55 * 10 = 5.5
    (1000, 1000, 3000, 4),                # 0.55 * 3 = 1.65, floor 4
])
def test_neutronsparse_threshold_closed_form(rows, cols, nnz, want):
    assert PT.neutronsparse_threshold(rows, cols, nnz) == want


def brute_neutronsparse(crow, col, rows, cols, threshold, symmetric):
    crow, col = crow.numpy(), col.numpy()
    row_deg = [crow[r + 1] - crow[r] for r in range(rows)]
    if symmetric:
        col_deg = list(row_deg)
    else:
        col_deg = [0] * cols
        for c in col:
            col_deg[c] += 1
    dense_col = [col_deg[c] > threshold for c in range(cols)]
    cube, vec = [[] for _ in range(rows)], [[] for _ in range(rows)]
    dense_rows = 0
    for r in range(rows):
        in_dense = sum(1 for p in range(crow[r], crow[r + 1]) if dense_col[col[p]])
        dense_row = in_dense > threshold
        dense_rows += dense_row
        for p in range(crow[r], crow[r + 1]):
            (cube if dense_row and dense_col[col[p]] else vec)[r].append(p)
    return cube, vec, dense_rows, sum(dense_col)


def rows_of(part):
    crow, col, vals = part
    return [(col[crow[r]:crow[r + 1]].tolist(), vals[crow[r]:crow[r + 1]].tolist()) for r in range(crow.numel() - 1)]


@pytest.mark.parametrize("symmetric", [False, True])
@pytest.mark.parametrize("seed", [1, 2, 3])
def test_neutronsparse_parts_match_brute_force(seed, symmetric):
    rows = cols = 60
    crow, col, vals = random_csr(seed, rows, cols, 6, heavy=(3, 17, 40))
    # dense columns: make columns 5 and 9 appear in most rows
    cube, vector, meta = PT.neutronsparse_parts(crow, col, vals, rows, cols, symmetric)
    t = meta["threshold"]
    assert t == PT.neutronsparse_threshold(rows, cols, col.numel())
    bc, bv, dense_rows, dense_cols = brute_neutronsparse(crow, col, rows, cols, t, symmetric)
    c, v = col.numpy(), vals.numpy()
    assert rows_of(cube) == [(c[ps].tolist(), v[ps].tolist()) for ps in bc]
    assert rows_of(vector) == [(c[ps].tolist(), v[ps].tolist()) for ps in bv]
    assert (meta["dense_rows"], meta["dense_columns"]) == (dense_rows, dense_cols)
    assert meta["aic_nnz"] + meta["aiv_nnz"] == col.numel()
    assert meta["symmetry_shortcut_used"] == symmetric


def test_neutronsparse_selects_dense_rows():
    # 20 rows x 20 cols: rows 0..9 use every column (dense), the rest one column
    rows = cols = 20
    parts = [np.arange(cols)] * 10 + [np.array([r]) for r in range(10, 20)]
    crow = torch.from_numpy(np.concatenate([[0], np.cumsum([p.size for p in parts])]).astype(np.int64))
    col = torch.from_numpy(np.concatenate(parts).astype(np.int64))
    vals = torch.ones(col.numel())
    cube, vector, meta = PT.neutronsparse_parts(crow, col, vals, rows, cols, False)
    # density 210/400 > 0.01: threshold max(4, int(10.5 * 0.25)) = 4; column degree 10 or 11 > 4
    assert meta["threshold"] == 4 and meta["dense_columns"] == 20 and meta["dense_rows"] == 10
    assert meta["aic_nnz"] == 200 and meta["aiv_nnz"] == 10
    assert cube[0].tolist() == [20 * min(r, 10) for r in range(21)]


@pytest.mark.parametrize("fraction,pivot", [(1.0 / 3.0, None), (0.5, None), (0.0, 0), (1.0, None)])
def test_naive_parts_reassemble_the_matrix(fraction, pivot):
    crow, col, vals = random_csr(9, 40, 50, 7)
    nnz = col.numel()
    cube, vector, meta = PT.naive_parts(crow, col, vals, fraction)
    want = nnz // 3 if fraction == 1.0 / 3.0 else int(nnz * fraction)
    assert meta["pivot_nnz"] == want and meta["aic_nnz"] == want and meta["aiv_nnz"] == nnz - want
    assert cube[1].numel() == want and vector[1].numel() == nnz - want
    for r, ((cc, cv), (vc, vv)) in enumerate(zip(rows_of(cube), rows_of(vector))):
        a, b = int(crow[r]), int(crow[r + 1])
        assert cc + vc == col[a:b].tolist() and cv + vv == vals[a:b].tolist()


def test_prepare_partition_argument_errors():
    crow, col, vals = random_csr(4, 8, 8, 3)
    with pytest.raises(ValueError, match="unknown partition method"):
        PT.prepare_partition("greedy", 8, 8, crow, col, vals)
    with pytest.raises(ValueError, match="block_ratio must be positive"):
        PT.prepare_partition("naive", 8, 8, crow, col, vals, block_ratio=0)
    with pytest.raises(ValueError, match=r"naive_fraction must be in \[0, 1\]"):
        PT.prepare_partition("naive", 8, 8, crow, col, vals, naive_fraction=1.5)


def test_block_part_rejects_edges_past_last_row():
    crow = torch.tensor([0, 1, 1], dtype=torch.int64)
    with pytest.raises(ValueError, match="edges after its last nonempty row"):
        PT.block_part((crow, torch.tensor([0, 1]), torch.ones(2)), 4, "cpu")


def test_cli_defaults_and_errors():
    a = C.task_mapping_args([])
    assert a.methods == list(PT.METHODS) and a.dims == [128] and (a.atol, a.rtol) == (2e-2, 2e-2)
    assert C.task_mapping_args(["--dtype", "fp32"]).atol == 1e-4
    assert C.aiv_bitwise_args([]).dims == [16, 32, 64, 128, 256]
    assert C.aiv_bitwise_args(["--dims", "32", "64"]).dims == [32, 64]
    b = C.aic_aiv_args([])
    assert (b.aic_atol, b.aiv_atol, b.aiv_rtol) == (2e-2, 0.0, 0.0)
    for parse, argv in [(C.task_mapping_args, ["--dim", "24"]),
                        (C.task_mapping_args, ["--dim", "2048"]),
                        (C.task_mapping_args, ["--dtype", "fp32", "--dim", "1024"]),
                        (C.task_mapping_args, ["--dim", "32", "--dim", "32"]),
                        (C.task_mapping_args, ["--index", "0", "--limit", "2"]),
                        (C.task_mapping_args, ["--method", "naive", "--method", "naive"]),
                        (C.task_mapping_args, ["--block-ratio", "0"]),
                        (C.task_mapping_args, ["--naive-fraction", "2"]),
                        (C.task_mapping_args, ["--atol", "-1"]),
                        (C.aiv_bitwise_args, ["--dim", "16", "--dims", "32"]),
                        (C.aic_aiv_args, ["--aiv-atol", "-0.5"])]:
        with pytest.raises(SystemExit):
            parse(argv)
    assert C.main([]) == 2 and C.main(["bogus"]) == 2


def test_compare_reports_first_mismatch():
    e = torch.zeros(3, 4)
    a = e.clone()
    assert C.compare(a, e, 0, 0, "x") == {"bitwise_equal": True, "mismatch_count": 0, "max_abs_error": 0.0,
                                          "mean_abs_error": 0.0, "passed": True}
    a[1, 2], a[2, 0] = 0.5, 1e-3
    r = C.compare(a, e, 1e-2, 0, "x")
    assert r["mismatch_count"] == 1 and not r["passed"] and r["first_mismatch_row"] == 1
    assert (r["first_mismatch_column"], r["actual_value"], r["reference_value"]) == (2, 0.5, 0.0)
    a[0, 0] = float("nan")
    with pytest.raises(RuntimeError, match="NaN or Inf"):
        C.compare(a, e, 1, 1, "x")
