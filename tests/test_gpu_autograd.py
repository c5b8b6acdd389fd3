"""Autograd of the graph layout: pack_node_tensor / restore_node_tensor are
differentiable (as the reference's index_copy_ / index_select are,
spmm_npu.py:45-46, 62), and PackedGraph multiplies by P A P^T forward and by
P A^T P^T backward using the transpose_* split the reference's preprocess
computes (extension/custom_op.cpp:1072-1078, 1350-1384).  Checked against
fp64 A x and A^T g of the oracle, at the reference's tolerances."""

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-2, torch.float32: 1e-4}
NP = {torch.float16: np.float16, torch.float32: np.float32}


def graph(seed, n, deg):
    rng = np.random.default_rng(seed)
    parts = []
    for r in range(n):
        d = int(min(n, rng.integers(0, deg + 1) if r % 9 else 4 * deg))
        parts.append(np.sort(rng.choice(n, d, replace=False)))
    crow = np.zeros(n + 1, np.int64)
    crow[1:] = np.cumsum([p.size for p in parts])
    return crow, np.concatenate(parts).astype(np.int64)


def transpose_csr(crow, col, val, n):
    rows = np.repeat(np.arange(n), np.diff(crow))
    order = np.lexsort((rows, col))
    tcrow = np.zeros(n + 1, np.int64)
    tcrow[1:] = np.cumsum(np.bincount(col, minlength=n))
    return tcrow, rows[order], val[order]


def test_pack_restore_gradients(spmm_npu):
    rng = np.random.default_rng(3)
    inv = torch.from_numpy(rng.permutation(48)[:40]).cuda()
    x = torch.randn(40, 16, device="cuda", requires_grad=True)
    w = torch.randn(48, 16, device="cuda")
    (spmm_npu.pack_node_tensor(x, inv, 48) * w).sum().backward()
    assert torch.equal(x.grad, w[inv])
    p = torch.randn(48, 16, device="cuda", requires_grad=True)
    g = torch.randn(40, 16, device="cuda")
    (spmm_npu.restore_node_tensor(p, inv) * g).sum().backward()
    want = torch.zeros(48, 16, device="cuda")
    want[inv] = g
    assert torch.equal(p.grad, want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("seed,n,deg", [(1, 90, 8), (2, 333, 20)])
def test_packed_graph_forward_and_backward(spmm_npu, dtype, seed, n, deg):
    crow, col = graph(seed, n, deg)
    rng = np.random.default_rng(seed + 100)
    val = rng.uniform(0, 1, col.size).astype(NP[dtype])
    width = 32
    prep = spmm_npu.preprocess(torch.from_numpy(crow).cuda(), torch.from_numpy(col).cuda(),
                               torch.from_numpy(val).cuda(), n, n, 16, True)
    G = spmm_npu.PackedGraph(prep)
    x_np = rng.standard_normal((n, width)).astype(NP[dtype])
    w_np = rng.standard_normal((n, width)).astype(NP[dtype])
    x = torch.from_numpy(x_np).cuda().requires_grad_(True)
    y = G.restore(G(G.pack(x)))
    (y.float() * torch.from_numpy(w_np).cuda().float()).sum().backward()
    tol = TOL[dtype]
    np.testing.assert_allclose(y.detach().double().cpu().numpy(), O.spmm_f64(crow, col, val, x_np),
                               atol=tol, rtol=tol)
    tcrow, tcol, tval = transpose_csr(crow, col, val, n)
    np.testing.assert_allclose(x.grad.double().cpu().numpy(), O.spmm_f64(tcrow, tcol, tval, w_np),
                               atol=tol, rtol=tol)


def test_packed_graph_rejects_unpacked_layout(spmm_npu):
    crow, col = graph(5, 40, 4)
    val = np.ones(col.size, np.float32)
    prep = spmm_npu.preprocess(torch.from_numpy(crow).cuda(), torch.from_numpy(col).cuda(),
                               torch.from_numpy(val).cuda(), 40, 40, 16, False)
    with pytest.raises(ValueError, match="graph_layout=True"):
        spmm_npu.PackedGraph(prep)
