"""The harness's dataset format (ascend-spmm_amd/payloads.py): payload
round trips, each validation error of the reference's load_payload
(tests/task_mapping/common.py:33-63), discovery and selection, stable_seed,
and Matrix Market conversion (tests/data/prepare_data.py:25-42)."""

import hashlib
import os
import sys

import numpy as np
import pytest
import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(REPO, "ascend-spmm_amd"))

import payloads as D  # noqa: E402


def write(path, **payload):
    path.parent.mkdir(parents=True, exist_ok=True)
    torch.save(payload, path)
    return path


def good(**over):
    p = {"name": "m", "shape": (3, 4), "nnz": 3, "crow_indices": torch.tensor([0, 1, 1, 3]),
         "col_indices": torch.tensor([3, 0, 2])}
    p.update(over)
    return p


def test_payload_round_trip(tmp_path):
    D.save_payload(tmp_path / "a" / "mat_csr.pt", "mat", (3, 4), [0, 1, 1, 3], [3, 0, 2])
    name, rows, cols, crow, col = D.load_payload(tmp_path / "a" / "mat_csr.pt")
    assert (name, rows, cols) == ("mat", 3, 4)
    assert crow.dtype == torch.int64 and crow.tolist() == [0, 1, 1, 3] and col.tolist() == [3, 0, 2]
    # name falls back to the stem without _csr
    p = write(tmp_path / "b_csr.pt", **{k: v for k, v in good().items() if k != "name"})
    assert D.load_payload(p)[0] == "b"


@pytest.mark.parametrize("over,msg", [
    ({"shape": None}, "missing payload fields: shape"),
    ({"shape": (0, 4)}, "invalid matrix shape"),
    ({"crow_indices": torch.tensor([0, 1, 3])}, "rows \\+ 1 entries"),
    ({"crow_indices": torch.tensor([1, 1, 1, 3])}, "invalid CSR pointer"),
    ({"crow_indices": torch.tensor([0, 2, 1, 3])}, "nondecreasing"),
    ({"col_indices": torch.tensor([3, 0, 4])}, "out-of-range"),
    ({"nnz": 5}, "nnz does not match"),
])
def test_payload_validation(tmp_path, over, msg):
    p = good(**over)
    if over.get("shape", 1) is None:
        del p["shape"]
    path = write(tmp_path / "x.pt", **p)
    with pytest.raises(ValueError, match=msg):
        D.load_payload(path)


def test_empty_matrix_rejected(tmp_path):
    path = write(tmp_path / "e.pt", **good(shape=(2, 2), nnz=0, crow_indices=torch.tensor([0, 0, 0]),
                                           col_indices=torch.zeros(0, dtype=torch.int64)))
    with pytest.raises(ValueError, match="empty matrices"):
        D.load_payload(path)


def test_discover_and_select(tmp_path):
    for rel in ("beta/beta_csr.pt", "alpha/alpha_csr.pt", "alpha/extra_csr.pt", "gamma/gamma_csr.pt"):
        write(tmp_path / rel, **good())
    names = [p.relative_to(tmp_path).as_posix() for p in D.discover_datasets(tmp_path)]
    assert names == ["alpha/alpha_csr.pt", "alpha/extra_csr.pt", "beta/beta_csr.pt", "gamma/gamma_csr.pt"]
    assert [p.name for p in D.discover_datasets(tmp_path, name="alpha")] == ["alpha_csr.pt", "extra_csr.pt"]
    assert [p.name for p in D.discover_datasets(tmp_path, name="extra")] == ["extra_csr.pt"]
    assert [p.name for p in D.discover_datasets(tmp_path, start=1, stop=3)] == ["extra_csr.pt", "beta_csr.pt"]
    assert [p.name for p in D.discover_datasets(tmp_path, limit=1)] == ["alpha_csr.pt"]
    assert D.select_dataset(tmp_path, "", 2).name == "beta_csr.pt"
    assert D.select_dataset(tmp_path, "gamma", 0).name == "gamma_csr.pt"
    with pytest.raises(ValueError, match="outside the discovered range"):
        D.discover_datasets(tmp_path, index=9)
    with pytest.raises(ValueError, match="expected exactly one"):
        D.select_dataset(tmp_path, "alpha", 0)
    with pytest.raises(ValueError, match="--limit must be positive"):
        D.discover_datasets(tmp_path, limit=0)
    with pytest.raises(ValueError, match="no .pt datasets"):
        D.discover_datasets(tmp_path, name="zzz")


def test_stable_seed_closed_form():
    s = D.stable_seed(2027, "a/a_csr.pt")
    digest = hashlib.sha256(b"a/a_csr.pt").digest()
    assert s == (2027 + int.from_bytes(digest[:8], "little")) % (2**63 - 1)
    assert s != D.stable_seed(2027, "b/b_csr.pt") and 0 <= s < 2**63 - 1


def test_seeded_operands_are_reproducible():
    v1, v2 = D.make_values(100, torch.float16, 7), D.make_values(100, torch.float16, 7)
    assert torch.equal(v1, v2) and v1.dtype == torch.float16 and float(v1.abs().max()) <= 1.0
    b = D.make_dense(10, 16, torch.float32, 3)
    assert b.shape == (10, 16) and not torch.equal(b, D.make_dense(10, 16, torch.float32, 4))


def test_matrix_market_conversion(tmp_path):
    from scipy import sparse
    from scipy.io import mmwrite

    coo = sparse.coo_matrix((np.array([1.0, 2.0, 0.0, 3.0, 4.0]), (np.array([0, 0, 1, 2, 0]), np.array([2, 2, 0, 1, 0]))),
                            shape=(3, 3))
    src = tmp_path / "g" / "g.mtx"
    src.parent.mkdir()
    mmwrite(str(src), coo)
    rows, cols, nnz = D.convert_matrix_market(src, tmp_path / "out" / "g_csr.pt")
    name, r, c, crow, col = D.load_payload(tmp_path / "out" / "g_csr.pt")
    # (0,2) duplicates summed, the explicit zero at (1,0) dropped, columns sorted
    assert (name, r, c, nnz) == ("g", 3, 3, 3)
    assert crow.tolist() == [0, 2, 2, 3] and col.tolist() == [0, 2, 1]
