"""Host-side logic of the Python mirror (``spmm_npu``) that runs without a
GPU: the module surface, ``make_start`` against the oracle, and the
``ValueError`` checks of pack/restore that fire before any device work
(reference: spmm_npu.py:23-62, tests/task_mapping/common.py:119-127)."""

import os
import sys

import numpy as np
import pytest
import torch

import oracle as O

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(REPO, "ascend-spmm_amd"))


@pytest.fixture(scope="module")
def api():
    import spmm_npu  # loads custom_ops_lib and libspmm_mi355x.so; no GPU call at import

    return spmm_npu


def test_surface_matches_reference_module(api):
    for name in ("spmm_csr", "spmm_ascend_cube", "csr_to_bcsr", "csr_to_ascend_cube", "preprocess",
                 "block_level_split", "pack_node_tensor", "restore_node_tensor",
                 "spmm_ascend_cube_aic_without_pipeline", "spmm_ascend_cube_aiv_mb",
                 "spmm_csr_aiv_mb_batch", "spmm_cube", "make_start"):
        assert callable(getattr(api, name)), name
    for op in ("spmm_csr", "spmm_cube", "spmm_ascend_cube", "spmm_csr_aiv_mb_batch",
               "spmm_ascend_cube_aic_without_pipeline", "spmm_ascend_cube_aiv_mb"):
        assert hasattr(torch.ops.myops, op), op


def test_make_start_matches_oracle(api):
    rng = np.random.default_rng(7)
    pointers = [np.zeros(1, np.int64), np.zeros(5, np.int64), np.array([0, 2, 4, 6]),
                np.array([0, 0, 9, 9, 9]), np.array([0, 100])]
    for _ in range(100):
        n = int(rng.integers(2, 60))
        pointers.append(np.concatenate([[0], np.cumsum(rng.integers(0, 6, n - 1))]))
    for p in pointers:
        for cores in (1, 3, 20, 40):
            got = api.make_start(torch.from_numpy(p), cores)
            assert got.dtype == torch.int32 and got.numel() == cores
            np.testing.assert_array_equal(got.numpy(), O.make_start(p, cores))
    assert api.make_start(torch.zeros(0, dtype=torch.int64), 4).tolist() == [0, 0, 0, 0]


def test_pack_restore_argument_errors(api):
    x = torch.zeros(3, 4)
    with pytest.raises(ValueError, match="at least one dimension"):
        api.pack_node_tensor(torch.tensor(1.0), torch.tensor([0]))
    with pytest.raises(ValueError, match="one entry per original node"):
        api.pack_node_tensor(x, torch.tensor([0, 1]))
    with pytest.raises(ValueError, match="does not map every original node"):
        api.pack_node_tensor(x, torch.tensor([0, -1, 2]))
    with pytest.raises(ValueError, match="smaller than the permutation extent"):
        api.pack_node_tensor(x, torch.tensor([0, 5, 2]), packed_rows=4)
    with pytest.raises(ValueError, match="at least one dimension"):
        api.restore_node_tensor(torch.tensor(1.0), torch.tensor([0]))
    with pytest.raises(ValueError, match="invalid packed node id"):
        api.restore_node_tensor(x, torch.tensor([0, 3]))
    with pytest.raises(ValueError, match="invalid packed node id"):
        api.restore_node_tensor(x, torch.tensor([-1]))


def test_operators_reject_cpu_tensors(api):
    """The operators run on the GPU only; CPU operands raise (no host fallback)."""
    crow = torch.tensor([0, 1], dtype=torch.int32)
    col = torch.tensor([0], dtype=torch.int32)
    val = torch.ones(1, dtype=torch.float16)
    dense = torch.ones(1, 16, dtype=torch.float16)
    with pytest.raises((RuntimeError, NotImplementedError)):
        api.spmm_csr(crow, col, val, dense, torch.zeros(40, dtype=torch.int32))
