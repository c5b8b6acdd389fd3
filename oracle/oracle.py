"""CPU oracle for the MI355X SpMM build — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker.  The product
(``ascend-spmm_amd/``) never imports it.

It wraps the C restatement in ``spmm_oracle.c`` (built to ``liboracle.so`` by
the Makefile next to it) and adds numpy closed forms.  Every function cites the
reference code it restates (paths relative to the Ascend-SpMM repository root).
Functions return numpy arrays whose dtypes follow the reference: index outputs
take the dtype of the input row pointer, value outputs the dtype of the input
values, permutations and scalar audit fields are int64 / float64.

Parity pinning of each function (what checks it beyond its own formula) is
listed in the tests that exercise it: ``tests/test_oracle_*.py``.
"""

from __future__ import annotations

import ctypes
import os
from typing import Dict

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_REF_PATH = os.path.join(_HERE, "_ref", "libref.so")

_I64P = ctypes.POINTER(ctypes.c_int64)
_U8P = ctypes.POINTER(ctypes.c_uint8)
_lib = None
_ref = None

_ERRORS = {1: ValueError, 2: IndexError, 3: OverflowError, 4: RuntimeError}


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run make -C oracle)")
        lib = ctypes.CDLL(_LIB_PATH)
        lib.or_last_error.restype = ctypes.c_char_p
        _lib = lib
    return _lib


def reference_library():
    """The reference's own std-only headers compiled into ``_ref/libref.so``
    (``make -C oracle ref``), or None when it was not built."""
    global _ref
    if _ref is None and os.path.exists(_REF_PATH):
        _ref = ctypes.CDLL(_REF_PATH)
    return _ref


def _check(rc: int) -> None:
    if rc != 0:
        msg = _load().or_last_error().decode()
        raise _ERRORS.get(rc, RuntimeError)(msg)


def _i64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a), dtype=np.int64)


def _p64(a: np.ndarray):
    return a.ctypes.data_as(_I64P)


def _pu8(a: np.ndarray):
    return a.ctypes.data_as(_U8P)


def _vals(values) -> np.ndarray:
    v = np.ascontiguousarray(np.asarray(values))
    if v.dtype not in (np.float16, np.float32, np.float64):
        raise TypeError(f"values must be fp16/fp32/fp64, got {v.dtype}")
    return v


# --------------------------------------------------------------------- SpMM

def spmm_f64(crow, col, values, dense) -> np.ndarray:
    """C = A @ B in fp64 (the mathematics the reference kernels approximate:
    kernels/op_kernel/spmm_csr.cpp:383-423, spmm_ascend_cube.cpp:16-311).
    Out-of-range columns contribute nothing."""
    lib = _load()
    crow = _i64(crow)
    col = _i64(col)
    val = np.ascontiguousarray(np.asarray(values, dtype=np.float64))
    B = np.ascontiguousarray(np.asarray(dense, dtype=np.float64))
    rows = crow.size - 1
    K, N = B.shape
    C = np.zeros((rows, N), dtype=np.float64)
    lib.or_spmm_f64(ctypes.c_int64(rows), _p64(crow), _p64(col),
                    val.ctypes.data_as(ctypes.POINTER(ctypes.c_double)),
                    ctypes.c_int64(K), ctypes.c_int64(N),
                    B.ctypes.data_as(ctypes.POINTER(ctypes.c_double)),
                    C.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
    return C


def spmm_cube_f64(rowptr, col, values, dense) -> np.ndarray:
    """The legacy spmm_cube operator in fp64 (kernels/op_kernel/spmm_cube.cpp:53-146):
    rowptr indexes 16-row windows, col = (dense row << 4) | row in window;
    runs of equal dense row form one 16x1 block, a later value of the same
    row in a run replacing an earlier one.  Returns [16 * windows, N]."""
    lib = _load()
    rowptr = _i64(rowptr)
    col = _i64(col)
    val = np.ascontiguousarray(np.asarray(values, dtype=np.float64))
    B = np.ascontiguousarray(np.asarray(dense, dtype=np.float64))
    windows = rowptr.size - 1
    K, N = B.shape
    C = np.zeros((16 * windows, N), dtype=np.float64)
    lib.or_spmm_cube_f64(ctypes.c_int64(windows), _p64(rowptr), _p64(col),
                         val.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), ctypes.c_int64(col.size),
                         ctypes.c_int64(K), ctypes.c_int64(N),
                         B.ctypes.data_as(ctypes.POINTER(ctypes.c_double)),
                         C.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
    return C


def cube_encode(crow, col, values, nrows):
    """Window-encoded form of a CSR matrix for spmm_cube: per 16-row window,
    nonzeros ordered by (column, row) with col = (column << 4) | row.
    Returns (rowptr[windows + 1], encoded col, values)."""
    crow = _i64(crow)
    col = _i64(col)
    vals = np.asarray(values)
    rows = np.repeat(np.arange(nrows, dtype=np.int64), np.diff(crow))
    windows = (nrows + 15) // 16
    order = np.lexsort((rows, col, rows // 16))
    w = (rows // 16)[order]
    rowptr = np.zeros(windows + 1, dtype=np.int64)
    rowptr[1:] = np.cumsum(np.bincount(w, minlength=windows))
    enc = (col[order] << 4) | (rows[order] & 15)
    return rowptr, enc, vals[order]


def cpu_reference(rows, cols, crow, col, values, dense):
    """The reference's CPU SpMM, ``cpu_reference``
    (tests/aic_aiv_ablation/common.py:173-177): torch CSR ``sparse.mm`` in
    fp32.  Takes and returns torch CPU tensors."""
    import torch

    matrix = torch.sparse_csr_tensor(
        torch.as_tensor(crow).long(), torch.as_tensor(col).long(),
        torch.as_tensor(values).float(), size=(rows, cols))
    return torch.sparse.mm(matrix, torch.as_tensor(dense).float())


def make_start(pointer, cores: int) -> np.ndarray:
    """Per-core start rows: ``searchsorted(pointer, k*ceil(total/cores),
    right=True) - 1`` clamped at 0 (tests/task_mapping/common.py:119-127)."""
    p = _i64(pointer)
    out = np.zeros(cores, dtype=np.int32)
    _load().or_make_start(_p64(p), ctypes.c_int64(p.size), ctypes.c_int64(cores),
                          out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)))
    return out


# -------------------------------------------------------- layout converters

def csr_to_bcsr(crow, col, values, nrows, ncols, window_size=16) -> Dict[str, np.ndarray]:
    """BCSR(16x1) conversion, ``ToBCSR`` (extension/custom_op.cpp:594-746)."""
    lib = _load()
    idx_dtype = np.asarray(crow).dtype
    c64, k64, v = _i64(crow), _i64(col), _vals(values)
    nwin = (nrows + window_size - 1) // window_size
    nnz = k64.size
    cwp = np.zeros(nwin + 1, dtype=np.int64)
    uniq = np.zeros(max(nnz, 1), dtype=np.int64)
    value = np.zeros(max(16 * nnz, 1), dtype=v.dtype)
    nb = ctypes.c_int64(0)
    _check(lib.or_csr_to_bcsr(_p64(c64), _p64(k64), _pu8(v), ctypes.c_int64(v.itemsize),
                              ctypes.c_int64(nrows), ctypes.c_int64(ncols),
                              ctypes.c_int64(window_size), _p64(cwp), _p64(uniq), _pu8(value),
                              ctypes.byref(nb)))
    n = nb.value
    return {
        "crow_window_ptr": cwp.astype(idx_dtype),
        "unique_col_ids": uniq[:n].astype(idx_dtype),
        "value": value[: 16 * n].copy(),
    }


def csr_to_ascend_cube(crow, col, values, nrows, ncols, window_size=16) -> Dict[str, np.ndarray]:
    """16x16 cube-tile conversion, ``your_logic_kernel``
    (extension/custom_op.cpp:429-592)."""
    lib = _load()
    idx_dtype = np.asarray(crow).dtype
    c64, k64, v = _i64(crow), _i64(col), _vals(values)
    nwin = (nrows + window_size - 1) // window_size
    nnz = k64.size
    cap_tiles = nnz + nwin + 1
    cwp = np.zeros(nwin + 1, dtype=np.int64)
    uniq = np.zeros(16 * cap_tiles, dtype=np.int64)
    value = np.zeros(256 * cap_tiles, dtype=v.dtype)
    nt = ctypes.c_int64(0)
    _check(lib.or_csr_to_cube(_p64(c64), _p64(k64), _pu8(v), ctypes.c_int64(v.itemsize),
                              ctypes.c_int64(nrows), ctypes.c_int64(ncols),
                              ctypes.c_int64(window_size), _p64(cwp), _p64(uniq), _pu8(value),
                              ctypes.byref(nt)))
    n = nt.value
    return {
        "crow_window_ptr": cwp.astype(idx_dtype),
        "unique_col_ids": uniq[: 16 * n].astype(idx_dtype),
        "value": value[: 256 * n].copy(),
    }


# ------------------------------------------------------------ hybrid split

class _SplitOut(ctypes.Structure):
    _fields_ = [
        ("crow_window_ptr", _I64P), ("n_crow", ctypes.c_int64),
        ("unique_col_ids", _I64P), ("n_unique", ctypes.c_int64),
        ("value", _U8P), ("n_value", ctypes.c_int64),
        ("vrow_window_ptr", _I64P), ("n_vrow", ctypes.c_int64),
        ("vcol_indices", _I64P), ("n_vnnz", ctypes.c_int64),
        ("vvalue", _U8P),
    ]


class _SplitBuffers:
    """Upper-bound buffers for one BCSR + CSR split (kept alive with the struct)."""

    def __init__(self, nwin: int, nnz: int, value_dtype, window_size: int = 16):
        self.cwp = np.zeros(nwin + 1, dtype=np.int64)
        self.uniq = np.zeros(max(nnz, 1), dtype=np.int64)
        self.value = np.zeros(max(window_size * nnz, 1), dtype=value_dtype)
        self.vrow = np.zeros(window_size * nwin + 1, dtype=np.int64)
        self.vcol = np.zeros(max(nnz, 1), dtype=np.int64)
        self.vval = np.zeros(max(nnz, 1), dtype=value_dtype)
        self.s = _SplitOut(_p64(self.cwp), 0, _p64(self.uniq), 0, _pu8(self.value), 0,
                           _p64(self.vrow), 0, _p64(self.vcol), 0, _pu8(self.vval))

    def result(self, idx_dtype, prefix: str = "") -> Dict[str, np.ndarray]:
        s = self.s
        return {
            prefix + "crow_window_ptr": self.cwp[: s.n_crow].astype(idx_dtype),
            prefix + "unique_col_ids": self.uniq[: s.n_unique].astype(idx_dtype),
            prefix + "value": self.value[: s.n_value].copy(),
            prefix + "vrow_window_ptr": self.vrow[: s.n_vrow].astype(idx_dtype),
            prefix + "vcol_indices": self.vcol[: s.n_vnnz].astype(idx_dtype),
            prefix + "vvalue": self.vval[: s.n_vnnz].copy(),
        }


def block_level_split(crow, col, values, nrows, ncols, a, window_size) -> Dict[str, np.ndarray]:
    """Density-threshold BCSR/CSR split, ``hybrid_split_impl``
    (extension/custom_op.cpp:1146-1348, entry :1390-1412)."""
    lib = _load()
    idx_dtype = np.asarray(crow).dtype
    c64, k64, v = _i64(crow), _i64(col), _vals(values)
    nwin = (nrows + window_size - 1) // window_size
    buf = _SplitBuffers(nwin, max(k64.size, int(c64[-1]) if c64.size else 0), v.dtype, window_size)
    _check(lib.or_hybrid_split(_p64(c64), _p64(k64), _pu8(v), ctypes.c_int64(v.itemsize),
                               ctypes.c_int64(nrows), ctypes.c_int64(ncols), ctypes.c_double(a),
                               ctypes.c_int64(window_size), ctypes.byref(buf.s)))
    return buf.result(idx_dtype)


# -------------------------------------------------------------- preprocess

class _PreOut(ctypes.Structure):
    _fields_ = [
        ("fwd", _SplitOut),
        ("renum_unique", _I64P), ("n_renum_unique", ctypes.c_int64),
        ("renum_vcol", _I64P), ("n_renum_vcol", ctypes.c_int64),
        ("tr", _SplitOut),
        ("permutation", _I64P), ("n_perm", ctypes.c_int64),
        ("inv_permutation", _I64P), ("n_inv", ctypes.c_int64),
        ("packed_rows", ctypes.c_int64), ("packed_layout_supported", ctypes.c_int64),
        ("marginal_window", ctypes.c_int64), ("marginal_aic_blocks", ctypes.c_int64),
        ("marginal_total_blocks", ctypes.c_int64), ("shared_windows", ctypes.c_int64),
        ("est_aic", ctypes.c_double), ("est_aiv", ctypes.c_double), ("est_max", ctypes.c_double),
    ]


def preprocess(crow, col, values, nrows, ncols, window_size=16, graph_layout=False):
    """Cost-model AIC/AIV task mapping, ``taskmapping``
    (extension/custom_op.cpp:765-1110, entry :1112-1137), with the graph
    layout (renumbering, packed transpose and its fixed split, :1003-1035,
    :1350-1384).  Returns the reference's dict keys."""
    lib = _load()
    idx_dtype = np.asarray(crow).dtype
    index_max = np.iinfo(idx_dtype).max
    c64, k64, v = _i64(crow), _i64(col), _vals(values)
    nnz = k64.size
    nwin = (nrows + 15) // 16
    fwd = _SplitBuffers(nwin, nnz, v.dtype)
    tr = _SplitBuffers(nwin, nnz, v.dtype)
    renum_u = np.zeros(max(nnz, 1), dtype=np.int64)
    renum_v = np.zeros(max(nnz, 1), dtype=np.int64)
    perm = np.zeros(max(16 * nwin, 1), dtype=np.int64)
    inv = np.zeros(max(nrows, 1), dtype=np.int64)
    out = _PreOut()
    out.fwd = fwd.s
    out.tr = tr.s
    out.renum_unique = _p64(renum_u)
    out.renum_vcol = _p64(renum_v)
    out.permutation = _p64(perm)
    out.inv_permutation = _p64(inv)
    _check(lib.or_preprocess(_p64(c64), _p64(k64), _pu8(v), ctypes.c_int64(v.itemsize),
                             ctypes.c_int64(nnz), ctypes.c_int64(nrows), ctypes.c_int64(ncols),
                             ctypes.c_int64(window_size), ctypes.c_int(bool(graph_layout)),
                             ctypes.c_int64(int(index_max)), ctypes.byref(out)))
    fwd.s = out.fwd
    tr.s = out.tr
    res = fwd.result(idx_dtype)
    res["renumbered_unique_col_ids"] = renum_u[: out.n_renum_unique].astype(idx_dtype)
    res["renumbered_vcol_indices"] = renum_v[: out.n_renum_vcol].astype(idx_dtype)
    res.update(tr.result(idx_dtype, prefix="transpose_"))
    res["permutation"] = perm[: out.n_perm].copy()
    res["inv_permutation"] = inv[: out.n_inv].copy()
    for key in ("packed_rows", "packed_layout_supported", "marginal_window",
                "marginal_aic_blocks", "marginal_total_blocks", "shared_windows"):
        res[key] = np.array([getattr(out, key)], dtype=np.int64)
    res["estimated_aic_cost"] = np.array([out.est_aic], dtype=np.float64)
    res["estimated_aiv_cost"] = np.array([out.est_aiv], dtype=np.float64)
    res["estimated_max_cost"] = np.array([out.est_max], dtype=np.float64)
    return res


# ------------------------------------------------- boundary / graph helpers

def bucket_sort(columns, occupancy, max_occupancy) -> np.ndarray:
    """``stable_bucket_sort_by_occupancy_desc``
    (extension/boundary_bucket_sort.h:13-56)."""
    c = _i64(columns).copy()
    occ = _i64(occupancy)
    _check(_load().or_bucket_sort(_p64(c), ctypes.c_int64(c.size), _p64(occ),
                                  ctypes.c_int64(occ.size), ctypes.c_int64(max_occupancy)))
    return c


def renumber(columns, inv_permutation, index_dtype=np.int64) -> np.ndarray:
    """``renumber_columns_for_packed_layout``
    (extension/packed_column_reindex.h:14-41)."""
    c = _i64(columns)
    inv = _i64(inv_permutation)
    out = np.zeros(max(c.size, 1), dtype=np.int64)
    imax = np.iinfo(np.dtype(index_dtype)).max
    _check(_load().or_renumber(_p64(c), ctypes.c_int64(c.size), _p64(inv),
                               ctypes.c_int64(inv.size), ctypes.c_int64(int(imax)), _p64(out)))
    return out[: c.size].astype(index_dtype)


def transpose(rowptr, cols, values, inv_permutation, packed_rows):
    """CSR of ``P A^T P^T``, ``transpose_into_packed_layout``
    (extension/packed_column_reindex.h:43-101).  Returns (rowptr, cols, values)."""
    rp, c, v, inv = _i64(rowptr), _i64(cols), _vals(values), _i64(inv_permutation)
    if rp.size != inv.size + 1 or c.size != v.size:
        raise ValueError("invalid CSR arrays for packed transpose")
    rt = np.zeros(packed_rows + 1, dtype=np.int64)
    ct = np.zeros(max(c.size, 1), dtype=np.int64)
    vt = np.zeros(max(c.size, 1), dtype=v.dtype)
    _check(_load().or_transpose(_p64(rp), _p64(c), _pu8(v), ctypes.c_int64(v.itemsize),
                                ctypes.c_int64(c.size), _p64(inv), ctypes.c_int64(inv.size),
                                ctypes.c_int64(packed_rows), _p64(rt), _p64(ct), _pu8(vt)))
    return rt, ct[: c.size], vt[: c.size]


def pack_node_tensor(x, inv_permutation, packed_rows=None) -> np.ndarray:
    """``packed[inv[i]] = x[i]``, other rows zero (spmm_npu.py:23-47)."""
    x = np.asarray(x)
    inv = _i64(inv_permutation).reshape(-1)
    minimum = int(inv.max()) + 1 if inv.size else 0
    rows = minimum if packed_rows is None else int(packed_rows)
    out = np.zeros((rows, *x.shape[1:]), dtype=x.dtype)
    out[inv] = x
    return out


def restore_node_tensor(packed, inv_permutation) -> np.ndarray:
    """``out[i] = packed[inv[i]]`` (spmm_npu.py:50-62)."""
    return np.asarray(packed)[_i64(inv_permutation).reshape(-1)]
