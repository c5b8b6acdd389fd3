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
)


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
    "pack_node_tensor",
    "preprocess",
    "restore_node_tensor",
    "spmm_ascend_cube",
    "spmm_ascend_cube_aic_without_pipeline",
    "spmm_ascend_cube_aiv_mb",
    "spmm_csr",
    "spmm_csr_aiv_mb_batch",
]
