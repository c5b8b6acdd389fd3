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


class _PackRows(torch.autograd.Function):
    """packed[inv[i]] = x[i] (HIP scatter); backward gathers grad[inv[i]]."""

    @staticmethod
    def forward(ctx, tensor, index, packed_rows):
        ctx.save_for_backward(index)
        return _pack_rows(tensor, index, packed_rows)

    @staticmethod
    def backward(ctx, grad):
        (index,) = ctx.saved_tensors
        return _restore_rows(grad.contiguous(), index), None, None


class _RestoreRows(torch.autograd.Function):
    """out[i] = packed[inv[i]] (HIP gather); backward scatters into a zero
    tensor of the packed shape (inv is a permutation: no two i share a row)."""

    @staticmethod
    def forward(ctx, packed, index):
        ctx.save_for_backward(index)
        ctx.packed_rows = packed.size(0)
        return _restore_rows(packed, index)

    @staticmethod
    def backward(ctx, grad):
        (index,) = ctx.saved_tensors
        return _pack_rows(grad.contiguous(), index, ctx.packed_rows), None


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
    # One reduction and one read-back for both checks.
    lowest, highest = torch.stack(torch.aminmax(index)).tolist() if index.numel() else (0, -1)
    if lowest < 0:
        raise ValueError("inv_permutation does not map every original node")
    minimum_rows = highest + 1
    if packed_rows is None:
        packed_rows = minimum_rows
    elif torch.is_tensor(packed_rows):
        packed_rows = int(packed_rows.item())
    else:
        packed_rows = int(packed_rows)
    if packed_rows < minimum_rows:
        raise ValueError("packed_rows is smaller than the permutation extent")
    return _PackRows.apply(tensor, index.contiguous(), packed_rows)


def restore_node_tensor(packed_tensor, inv_permutation):
    """Apply ``P^T`` once and return rows in original node-id order.

    ``out[i] = packed_tensor[inv_permutation[i]]`` with the reference's
    validation (spmm_npu.py:50-62); the row gather runs as a HIP kernel.
    """
    if packed_tensor.ndim < 1:
        raise ValueError("a packed node tensor must have at least one dimension")
    index = inv_permutation.to(device=packed_tensor.device, dtype=torch.long).reshape(-1)
    lowest, highest = torch.stack(torch.aminmax(index)).tolist() if index.numel() else (0, -1)
    if lowest < 0 or highest >= packed_tensor.size(0):
        raise ValueError("inv_permutation contains an invalid packed node id")
    return _RestoreRows.apply(packed_tensor, index.contiguous())


class _PackedGraphSpMM(torch.autograd.Function):
    """Y_p = (P A P^T) X_p on the mixed operator; dX_p = (P A^T P^T) dY_p on
    the same operator with the fixed-layout transpose split."""

    @staticmethod
    def forward(ctx, graph, x_packed):
        ctx.graph = graph
        return spmm_ascend_cube(*graph.forward_ops, x_packed, graph.cstart, graph.vstart)

    @staticmethod
    def backward(ctx, grad):
        g = ctx.graph
        return None, spmm_ascend_cube(*g.transpose_ops, grad.contiguous(), g.tcstart, g.tvstart)


class PackedGraph:
    """A fixed square graph in the packed layout of
    ``preprocess(..., graph_layout=True)``, as a differentiable operator on
    packed node tensors.

    ``graph(x_packed)`` returns ``P A P^T x_packed`` (``spmm_ascend_cube`` on
    the renumbered block and vector parts).  Its backward multiplies by
    ``P A^T P^T``: ``spmm_ascend_cube`` on the ``transpose_*`` keys, the
    fixed-layout split of the packed transpose that the reference computes
    (extension/custom_op.cpp:1072-1078, 1350-1384) but never consumes.
    Gradients flow to the node tensor only (the graph is constant).  Compose
    with ``pack_node_tensor`` / ``restore_node_tensor``, which are
    differentiable too.
    """

    def __init__(self, prep, device=None):
        if "transpose_crow_window_ptr" not in prep or int(prep["packed_layout_supported"][0]) == 0:
            raise ValueError("PackedGraph needs preprocess(..., graph_layout=True) on a square matrix")
        dev = torch.device(device) if device is not None else prep["crow_window_ptr"].device
        if dev.type == "cpu":
            dev = torch.device("cuda", torch.cuda.current_device())
        i32 = torch.int32

        def ix(t):
            return t.to(device=dev, dtype=i32).contiguous()

        def vx(t):
            return t.to(device=dev).contiguous()

        self.packed_rows = int(prep["packed_rows"][0].item())
        self.inv_permutation = prep["inv_permutation"].to(dev)
        self.forward_ops = (ix(prep["crow_window_ptr"]), ix(prep["renumbered_unique_col_ids"]), vx(prep["value"]),
                            ix(prep["vrow_window_ptr"]), ix(prep["renumbered_vcol_indices"]), vx(prep["vvalue"]))
        self.transpose_ops = (ix(prep["transpose_crow_window_ptr"]), ix(prep["transpose_unique_col_ids"]),
                              vx(prep["transpose_value"]), ix(prep["transpose_vrow_window_ptr"]),
                              ix(prep["transpose_vcol_indices"]), vx(prep["transpose_vvalue"]))
        self.cstart = make_start(prep["crow_window_ptr"], 20).to(dev)
        self.vstart = make_start(prep["vrow_window_ptr"], 40).to(dev)
        self.tcstart = make_start(prep["transpose_crow_window_ptr"], 20).to(dev)
        self.tvstart = make_start(prep["transpose_vrow_window_ptr"], 40).to(dev)

    def __call__(self, x_packed):
        if x_packed.size(0) != self.packed_rows:
            raise ValueError("x_packed must have packed_rows rows")
        return _PackedGraphSpMM.apply(self, x_packed)

    def pack(self, x):
        return pack_node_tensor(x, self.inv_permutation, self.packed_rows)

    def restore(self, y_packed):
        return restore_node_tensor(y_packed, self.inv_permutation)


__all__ = [
    "PackedGraph",
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
