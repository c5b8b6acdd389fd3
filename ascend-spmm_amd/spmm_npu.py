"""Public Python API of the MI355X SpMM build (drop-in for Ascend-SpMM's ``spmm_npu``).

The operators come from the ``custom_ops_lib`` PyTorch-ROCm extension, which
calls the HIP kernels of ``libspmm_mi355x.so``; both are built in this
directory by ``build.py``.  Importing this module fails if the extension is
missing: there is no host fallback.

For fixed square graphs, ``preprocess(..., graph_layout=True)`` returns
``P A P^T`` mappings; pack node tensors once with ``P`` and restore original
ids only when needed (reference: spmm_npu.py:1-5).
"""

import os
import sys

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
if _HERE not in sys.path:
    sys.path.insert(0, _HERE)

from custom_ops_lib import (  # noqa: E402
    block_level_split,
    csr_to_ascend_cube,
    csr_to_bcsr,
    pack_rows as _pack_rows,
    preprocess,
    restore_rows as _restore_rows,
    spmm_ascend_cube,
    spmm_ascend_cube_aic_without_pipeline,
    spmm_ascend_cube_aiv_mb,
    spmm_csr,
    spmm_csr_aiv_mb_batch,
    spmm_cube,
)


def make_start(pointer, cores):
    """Per-core start row (or window) of an even split of ``pointer[-1]``
    work items over ``cores``: ``searchsorted(pointer, k*ceil(total/cores),
    right=True) - 1`` clamped at 0, as int32 (the reference's test helper,
    tests/task_mapping/common.py:119-127).

    The HIP kernels partition work on the device and do not read ``start``;
    the operators accept it for interface compatibility and check its rank.
    Returns a CPU tensor.
    """
    p = torch.as_tensor(pointer).detach().to("cpu", torch.int64).reshape(-1)
    total = int(p[-1].item()) if p.numel() else 0
    if total <= 0:
        return torch.zeros(cores, dtype=torch.int32)
    step = -(-total // cores)
    keys = torch.arange(cores, dtype=torch.int64) * step
    idx = torch.searchsorted(p, keys, right=True) - 1
    return idx.clamp_min(0).to(torch.int32)


def pack_node_tensor(tensor, inv_permutation, packed_rows=None):
    """Apply ``P`` once to a tensor whose leading dimension is original node id.

    ``packed[inv_permutation[i]] = tensor[i]``; padding rows are zero.  Same
    argument handling and ``ValueError`` cases as the reference
    (spmm_npu.py:23-47); the row scatter runs as a HIP kernel.
    """
    if tensor.ndim < 1:
        raise ValueError("a node tensor must have at least one dimension")
    index = inv_permutation.to(device=tensor.device, dtype=torch.long).reshape(-1)
    if tensor.size(0) != index.numel():
        raise ValueError("inv_permutation must contain one entry per original node")
    if index.numel() and bool((index < 0).any().item()):
        raise ValueError("inv_permutation does not map every original node")
    minimum_rows = int(index.max().item()) + 1 if index.numel() else 0
    if packed_rows is None:
        packed_rows = minimum_rows
    elif torch.is_tensor(packed_rows):
        packed_rows = int(packed_rows.item())
    else:
        packed_rows = int(packed_rows)
    if packed_rows < minimum_rows:
        raise ValueError("packed_rows is smaller than the permutation extent")
    return _pack_rows(tensor, index.contiguous(), packed_rows)


def restore_node_tensor(packed_tensor, inv_permutation):
    """Apply ``P^T`` once and return rows in original node-id order.

    ``out[i] = packed_tensor[inv_permutation[i]]`` with the reference's
    validation (spmm_npu.py:50-62); the row gather runs as a HIP kernel.
    """
    if packed_tensor.ndim < 1:
        raise ValueError("a packed node tensor must have at least one dimension")
    index = inv_permutation.to(device=packed_tensor.device, dtype=torch.long).reshape(-1)
    if index.numel() and (
        bool((index < 0).any().item())
        or int(index.max().item()) >= packed_tensor.size(0)
    ):
        raise ValueError("inv_permutation contains an invalid packed node id")
    return _restore_rows(packed_tensor, index.contiguous())


__all__ = [
    "block_level_split",
    "csr_to_ascend_cube",
    "csr_to_bcsr",
    "make_start",
    "pack_node_tensor",
    "preprocess",
    "restore_node_tensor",
    "spmm_ascend_cube",
    "spmm_ascend_cube_aic_without_pipeline",
    "spmm_ascend_cube_aiv_mb",
    "spmm_csr",
    "spmm_csr_aiv_mb_batch",
    "spmm_cube",
]
