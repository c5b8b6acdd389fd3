"""Golden vectors written by the reference's own code (tests/golden/*.npz, made
by tests/golden/make_golden.py from oracle/_ref, which compiles the
reference's extension/boundary_bucket_sort.h and
extension/packed_column_reindex.h where they lie).

CPU: the oracle reproduces every vector, including the reference's error
cases.  GPU: the HIP preprocess(graph_layout=True) reproduces the
reference's renumbered ids, and its transpose_* keys are the fixed split
(a = 295/505, extension/custom_op.cpp:1350-1384) of the reference's packed
transpose.  The window layout keys that graph.npz also holds
(unique_col_ids, vcol_indices, inv_permutation) were written by the oracle
and serve as the reference routines' inputs; the GPU's equality with them
is a regression check, its pin is the oracle comparison of
test_gpu_preprocess and the hand-worked cases of preprocess_cases."""

import os

import numpy as np
import pytest
import torch

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
STATUS = {1: ValueError, 2: IndexError, 3: OverflowError}


def load(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"))  # allow_pickle=False (default)


def test_bucket_sort_golden():
    g = load("bucket_sort")
    for i in range(int(g["count"][0])):
        cols, occ, rc = g[f"c{i}_columns"], g[f"c{i}_occupancy"], int(g[f"c{i}_status"][0])
        if rc:
            with pytest.raises(STATUS[rc]):
                O.bucket_sort(cols, occ, 16)
        else:
            np.testing.assert_array_equal(O.bucket_sort(cols, occ, 16), g[f"c{i}_sorted"])
    assert any(int(g[f"c{i}_status"][0]) for i in range(int(g["count"][0])))


def test_renumber_golden():
    g = load("renumber")
    statuses = set()
    for i in range(int(g["count"][0])):
        cols, inv, rc = g[f"c{i}_cols"], g[f"c{i}_inv"], int(g[f"c{i}_status"][0])
        statuses.add(rc)
        if rc:
            with pytest.raises(STATUS[rc]):
                O.renumber(cols, inv, cols.dtype)
        else:
            got = O.renumber(cols, inv, cols.dtype)
            assert got.dtype == cols.dtype
            np.testing.assert_array_equal(got, g[f"c{i}_out"])
    assert statuses == {0, 1, 2, 3}


@pytest.mark.parametrize("i", [0, 1])
def test_graph_layout_golden_oracle(i):
    """graph.npz keeps, per matrix, the inputs the oracle's preprocess passed
    to the reference routines (unique_col_ids, vcol_indices,
    inv_permutation: written by the oracle, so they are inputs here, not
    pins) and what the reference's own code returned for them (the
    renumbered ids and the packed transpose: these are the pins)."""
    g = load("graph")
    crow, col, val = g[f"g{i}_crow"], g[f"g{i}_col"], g[f"g{i}_val"]
    inv = g[f"g{i}_inv_permutation"]
    packed = int(g[f"g{i}_packed_rows"][0])
    rt, ct, vt = O.transpose(crow, col, val, inv, packed)
    np.testing.assert_array_equal(rt, g[f"g{i}_transpose_rowptr"])
    np.testing.assert_array_equal(ct, g[f"g{i}_transpose_col"])
    np.testing.assert_array_equal(vt.view(np.uint32), g[f"g{i}_transpose_val"].view(np.uint32))
    for src, out in (("unique_col_ids", "renumbered_unique_col_ids"), ("vcol_indices", "renumbered_vcol_indices")):
        got = O.renumber(g[f"g{i}_{src}"], inv, np.int64)
        np.testing.assert_array_equal(got, g[f"g{i}_{out}"], err_msg=out)


@pytest.mark.gpu
@pytest.mark.parametrize("i", [0, 1])
def test_graph_layout_golden_gpu(spmm_npu, i):
    g = load("graph")
    crow, col, val = g[f"g{i}_crow"], g[f"g{i}_col"], g[f"g{i}_val"]
    n = crow.size - 1
    got = spmm_npu.preprocess(torch.from_numpy(crow).cuda(), torch.from_numpy(col).cuda(),
                              torch.from_numpy(val).cuda(), n, n, 16, True)
    for key in ("inv_permutation", "renumbered_unique_col_ids", "renumbered_vcol_indices"):
        np.testing.assert_array_equal(got[key].cpu().numpy().astype(np.int64), g[f"g{i}_{key}"], err_msg=key)
    assert int(got["packed_rows"][0]) == int(g[f"g{i}_packed_rows"][0])
    packed = int(g[f"g{i}_packed_rows"][0])
    split = O.block_level_split(g[f"g{i}_transpose_rowptr"], g[f"g{i}_transpose_col"],
                                g[f"g{i}_transpose_val"], packed, packed, 295.0 / 505.0, 16)
    for key, ref in split.items():
        mine = got["transpose_" + key].cpu().numpy()
        assert mine.dtype == ref.dtype, key
        if mine.dtype.kind == "f":
            np.testing.assert_array_equal(mine.view(np.uint32), ref.view(np.uint32), err_msg=key)
        else:
            np.testing.assert_array_equal(mine, ref, err_msg=key)
