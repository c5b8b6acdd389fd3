"""Dataset format of Ascend-SpMM's test harness: CSR structure payloads
(``*.pt``) converted from Matrix Market files, their discovery, and the
seeded values/dense operands the harness derives from them.

Same payload format, validation and error messages as the reference
(tests/task_mapping/common.py:33-63, 66-111, 114-116, 134-143;
tests/data/prepare_data.py:25-42), so datasets prepared for the reference
load unchanged.  Payloads are read with ``torch.load(weights_only=True)``
only: unlike the reference, there is no fallback to an unrestricted load.
"""

from __future__ import annotations

import hashlib
from pathlib import Path
from typing import List, Optional, Tuple

import numpy as np
import torch

REQUIRED_FIELDS = ("shape", "crow_indices", "col_indices")
INT32_MAX = int(np.iinfo(np.int32).max)


def load_payload(path) -> Tuple[str, int, int, torch.Tensor, torch.Tensor]:
    """Read and validate a CSR structure payload.

    Returns ``(name, rows, cols, crow_indices int64, col_indices int64)``.
    The name is the payload's ``name`` field, else the file stem without a
    trailing ``_csr``.  Raises ``ValueError`` exactly where the reference's
    ``load_payload`` does.
    """
    path = Path(path)
    payload = torch.load(path, map_location="cpu", weights_only=True)
    missing = sorted(f for f in REQUIRED_FIELDS if f not in payload)
    if missing:
        raise ValueError(f"missing payload fields: {', '.join(missing)}")
    rows, cols = (int(v) for v in payload["shape"])
    crow = torch.as_tensor(payload["crow_indices"]).to(torch.int64).contiguous()
    col = torch.as_tensor(payload["col_indices"]).to(torch.int64).contiguous()
    if rows <= 0 or cols <= 0:
        raise ValueError(f"invalid matrix shape: {(rows, cols)}")
    if crow.ndim != 1 or crow.numel() != rows + 1:
        raise ValueError("crow_indices must contain rows + 1 entries")
    if col.ndim != 1 or int(crow[0]) != 0 or int(crow[-1]) != col.numel():
        raise ValueError("invalid CSR pointer or column array")
    if bool((crow[1:] < crow[:-1]).any()):
        raise ValueError("crow_indices must be nondecreasing")
    if col.numel() == 0:
        raise ValueError("empty matrices are not supported")
    if int(col.min()) < 0 or int(col.max()) >= cols:
        raise ValueError("col_indices contains an out-of-range index")
    if max(rows, cols, col.numel()) > INT32_MAX:
        raise ValueError("matrix exceeds the 32-bit NPU index contract")
    if "nnz" in payload and int(payload["nnz"]) != col.numel():
        raise ValueError("payload nnz does not match col_indices")
    stem = path.stem
    default = stem[: -len("_csr")] if stem.endswith("_csr") else stem
    name = str(payload.get("name") or default)
    return name, rows, cols, crow, col


def save_payload(path, name: str, shape, crow_indices, col_indices) -> None:
    """Write a CSR structure payload (the fields ``load_payload`` reads)."""
    crow = torch.as_tensor(np.asarray(crow_indices, dtype=np.int64))
    col = torch.as_tensor(np.asarray(col_indices, dtype=np.int64))
    payload = {
        "name": str(name),
        "shape": (int(shape[0]), int(shape[1])),
        "nnz": int(col.numel()),
        "crow_indices": crow,
        "col_indices": col,
    }
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    torch.save(payload, path)


def convert_matrix_market(source, destination) -> Tuple[int, int, int]:
    """Matrix Market file -> CSR structure payload: duplicates summed,
    explicit zeros dropped, columns sorted per row (as the reference's
    tests/data/prepare_data.py:25-42).  Returns (rows, cols, nnz)."""
    from scipy import sparse
    from scipy.io import mmread

    source = Path(source)
    matrix = mmread(source)
    csr = matrix.tocsr() if sparse.issparse(matrix) else sparse.csr_matrix(np.asarray(matrix))
    csr.sum_duplicates()
    csr.eliminate_zeros()
    csr.sort_indices()
    rows, cols = csr.shape
    save_payload(destination, source.stem, (rows, cols), csr.indptr, csr.indices)
    return int(rows), int(cols), int(csr.nnz)


def discover_datasets(dataset_dir, name: str = "", index: Optional[int] = None, start: int = 0,
                      stop: Optional[int] = None, limit: Optional[int] = None) -> List[Path]:
    """``*.pt`` payloads under ``dataset_dir`` in relative-path order,
    filtered by ``name`` (directory name or a substring of the stem), then
    one ``index`` or the slice ``[start:stop]`` and at most ``limit``."""
    root = Path(dataset_dir)
    found = sorted(root.rglob("*.pt"), key=lambda p: p.relative_to(root).as_posix())
    if name:
        found = [p for p in found if p.parent.name == name or name in p.stem]
    if index is not None:
        if not 0 <= index < len(found):
            raise ValueError(f"--index {index} is outside the discovered range [0, {len(found)})")
        return [found[index]]
    if start < 0:
        raise ValueError("--start must be non-negative")
    if stop is not None and stop < start:
        raise ValueError("--stop must be greater than or equal to --start")
    found = found[start:stop]
    if limit is not None:
        if limit <= 0:
            raise ValueError("--limit must be positive")
        found = found[:limit]
    if not found:
        raise ValueError(f"no .pt datasets selected under {root}")
    return found


def select_dataset(dataset_dir, name: str, index: int) -> Path:
    """Exactly one dataset: by ``name`` if given, else by ``index``."""
    if name:
        found = discover_datasets(dataset_dir, name=name)
        if len(found) != 1:
            raise ValueError(f"--name selected {len(found)} datasets; expected exactly one")
        return found[0]
    return discover_datasets(dataset_dir, index=index)[0]


def stable_seed(base_seed: int, relative_path: str) -> int:
    """Per-dataset seed: base seed plus the first 8 bytes (little endian) of
    the SHA-256 of the relative path, modulo 2**63 - 1."""
    head = hashlib.sha256(relative_path.encode("utf-8")).digest()[:8]
    return (base_seed + int.from_bytes(head, "little")) % (2**63 - 1)


def make_values(nnz: int, dtype: torch.dtype, seed: int) -> torch.Tensor:
    """Nonzero values U(-1, 1) from a seeded torch generator."""
    g = torch.Generator().manual_seed(seed)
    return (torch.rand(nnz, generator=g) * 2 - 1).to(dtype).contiguous()


def make_dense(cols: int, dim: int, dtype: torch.dtype, seed: int) -> torch.Tensor:
    """Dense operand U(-1, 1) of shape [cols, dim] from a seeded generator."""
    g = torch.Generator().manual_seed(seed)
    return (torch.rand((cols, dim), generator=g) * 2 - 1).to(dtype).contiguous()
