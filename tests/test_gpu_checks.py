"""The correctness CLIs end to end on the GPU (ascend-spmm_amd/checks.py,
the reference's scripts/run_tests.sh modes): synthetic payload datasets in
a temporary directory, every mode and partition method, and the JSON
reports' schema and verdicts."""

import json

import numpy as np
import pytest
import torch

import checks as C
import payloads as D
import workloads as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dataset_dir(tmp_path_factory):
    root = tmp_path_factory.mktemp("datasets_pt")
    w = W.config4(scale=0.02)  # mixed block / scattered windows
    D.save_payload(root / "mixed" / "mixed_csr.pt", "mixed", (w.rows, w.cols), w.crow, w.col)
    # hub rows and hub columns, so the NeutronSparse split has a block part
    rng = np.random.default_rng(5)
    n = 3000
    parts = []
    for r in range(n):
        deg = 400 if r % 97 == 0 else int(rng.integers(1, 12))
        cols = np.concatenate([np.arange(0, 60), rng.choice(n, deg, replace=False)]) if r % 97 == 0 else \
            rng.choice(n, deg, replace=False)
        parts.append(np.unique(cols))
    crow = np.concatenate([[0], np.cumsum([p.size for p in parts])]).astype(np.int64)
    D.save_payload(root / "hubs" / "hubs_csr.pt", "hubs", (n, n), crow, np.concatenate(parts))
    return root


def report(path):
    return json.loads(path.read_text())


@pytest.mark.parametrize("dtype", ["fp16", "fp32"])
def test_task_mapping_all_methods(spmm_npu, dataset_dir, tmp_path, dtype):
    out = tmp_path / "tm.json"
    assert C.main(["task-mapping", "--dataset-dir", str(dataset_dir), "--dim", "16", "--dim", "128",
                   "--dtype", dtype, "--output", str(out)]) == 0
    r = report(out)
    assert r["schema_version"] == 1 and r["passed"] is True and r["failed"] == 0
    assert r["methods"] == ["ours", "naive", "neutronsparse", "block-split"]
    assert r["comparisons"] == 2 * 4 * 2 == len(r["cases"]) and r["selected_datasets"] == 2
    for case in r["cases"]:
        assert case["aic_nnz"] + case["aiv_nnz"] == case["nnz"] and case["reference"] == "spmm_csr"
    hubs = next(d for d in r["datasets"] if d["dataset"] == "hubs")
    assert hubs["partitions"]["neutronsparse"]["aic_nnz"] > 0
    assert hubs["partitions"]["ours"]["aic_nnz"] + hubs["partitions"]["ours"]["aiv_nnz"] == hubs["nnz"]


def test_task_mapping_selection_and_naive_fraction(spmm_npu, dataset_dir, tmp_path):
    out = tmp_path / "tm.json"
    assert C.main(["task-mapping", "--dataset-dir", str(dataset_dir), "--name", "hubs", "--method", "naive",
                   "--naive-fraction", "0.75", "--output", str(out)]) == 0
    r = report(out)
    (case,) = r["cases"]
    assert case["dataset"] == "hubs" and case["method"] == "naive" and case["fraction"] == 0.75
    assert case["pivot_nnz"] == int(case["nnz"] * 0.75)


def test_aic_aiv_ablation(spmm_npu, dataset_dir, tmp_path):
    out = tmp_path / "ab.json"
    assert C.main(["aic-aiv", "--dataset-dir", str(dataset_dir), "--name", "mixed", "--dim", "64",
                   "--dim", "256", "--output", str(out)]) == 0
    r = report(out)
    assert r["passed"] is True and r["comparisons"] == 2 * 6 and r["dataset"] == "mixed"
    aiv = [c for c in r["cases"] if c["reference"] == "aiv-naive"]
    # the vector variants equal spmm_csr bitwise (zero tolerance)
    assert len(aiv) == 8 and all(c["bitwise_equal"] and c["atol"] == 0.0 for c in aiv)


def test_aiv_bitwise(spmm_npu, dataset_dir, tmp_path):
    out = tmp_path / "bw.json"
    assert C.main(["aiv-bitwise", "--dataset-dir", str(dataset_dir), "--output", str(out)]) == 0
    r = report(out)
    assert r["passed"] == r["comparisons"] == 2 * 5 and r["failed"] == 0
    assert [c["feature_width"] for c in r["cases"][:5]] == [16, 32, 64, 128, 256]
    assert all(c["mismatch_count"] == 0 and c["max_abs_error"] == 0.0 for c in r["cases"])


def test_failure_exits_nonzero(spmm_npu, dataset_dir, tmp_path, monkeypatch):
    # a wrong reference must fail the report (and exit non-zero), not pass silently
    import partition as PT
    real = PT.run_reference
    monkeypatch.setattr(PT, "run_reference", lambda *a: real(*a) + 1.0)
    out = tmp_path / "bad.json"
    with pytest.raises(SystemExit, match="comparisons failed"):
        C.main(["task-mapping", "--dataset-dir", str(dataset_dir), "--name", "mixed", "--method", "naive",
                "--output", str(out)])
    r = report(out)
    assert r["passed"] is False and r["failed"] == 1 and "first_mismatch_row" in r["cases"][0]


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("method", ["ours", "naive", "neutronsparse", "block-split"])
def test_partitions_match_fp64(spmm_npu, dataset_dir, dtype, method):
    """Every partition of the task-mapping comparison (tests/task_mapping/
    common.py:146-347), run through spmm_ascend_cube (run_mapping), against
    the fp64 oracle product at the reference's tolerance, on both datasets
    and at two widths; the naive split also at fractions 0 and 1 (all
    vector, all block)."""
    import oracle as O
    import partition as PT

    tol = 2e-2 if dtype == torch.float16 else 1e-4
    for path in sorted(dataset_dir.rglob("*.pt")):
        name, rows, cols, crow, col = D.load_payload(path)
        seed = D.stable_seed(2027, path.relative_to(dataset_dir).as_posix())
        values = D.make_values(col.numel(), dtype, seed)
        fractions = (PT.DEFAULT_NAIVE_FRACTION, 0.0, 1.0) if method == "naive" else (PT.DEFAULT_NAIVE_FRACTION,)
        for fraction in fractions:
            mapping, meta = PT.prepare_partition(method, rows, cols, crow, col, values, naive_fraction=fraction)
            assert meta["aic_nnz"] + meta["aiv_nnz"] == col.numel()
            if method != "ours":
                assert meta["aic_nnz"] > 0 or method == "neutronsparse" or fraction == 0.0
            for dim in (16, 128):
                dense = D.make_dense(cols, dim, dtype, seed + dim)
                out = PT.run_mapping(mapping, dense.cuda(), rows)
                expected = O.spmm_f64(crow.numpy(), col.numpy(), values.numpy(), dense.numpy())
                err = np.abs(out.double().cpu().numpy() - expected)
                bad = err > tol + tol * np.abs(expected)
                assert not bad.any(), (f"{name} {method} fraction={fraction} N={dim}: {int(bad.sum())} "
                                       f"mismatches, max abs err {float(err.max()):.3e}")
