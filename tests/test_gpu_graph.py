"""HIP graph capture of the SpMM operators.  spmm_csr and spmm_ascend_cube
launch kernels only (no host synchronisation, no memset nodes), so a caller
can capture them with torch.cuda.graph and replay them.  Each replay runs
after eager work that changes the dense operand in place, and must equal
the eager operator on the same operand bit for bit."""

import numpy as np
import pytest
import torch

import oracle as O
import workloads as W

pytestmark = pytest.mark.gpu


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dtype is None else t.to(dtype)


def check_replays(op, args, dense):
    """Capture op(*args) once, then replay it 4 times; between replays the
    dense operand is refilled by eager kernels and the eager op runs too."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            op(*args)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = op(*args)
    gen = torch.Generator(device="cuda")
    for i in range(4):
        gen.manual_seed(100 + i)
        dense.copy_(torch.randn(dense.shape, generator=gen, device="cuda").to(dense.dtype))
        eager = op(*args)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_out, eager), f"replay {i} differs from the eager call"
    return static_out


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_spmm_csr_graph_replays(spmm_npu, dtype):
    w = W.config2(scale=0.05)
    B = dev(w.dense(128)).to(dtype)
    args = (dev(w.crow, torch.int32), dev(w.col, torch.int32), dev(w.values).to(dtype), B,
            dev(O.make_start(w.crow, 40)))
    out = check_replays(spmm_npu.spmm_csr, args, B)
    assert out.shape == (w.rows, 128)


@pytest.mark.parametrize("graph_layout", [False, True])
def test_spmm_ascend_cube_graph_replays(spmm_npu, graph_layout):
    """The mixed op on a preprocess layout (block part, vector part, the
    block windows' hand-off and, at 512-byte rows, the window order)."""
    w = W.config4(scale=0.01)
    p = O.preprocess(w.crow, w.col, w.values, w.rows, w.cols, 16, graph_layout)
    i32 = torch.int32
    ccol = p["renumbered_unique_col_ids"] if graph_layout else p["unique_col_ids"]
    vcol = p["renumbered_vcol_indices"] if graph_layout else p["vcol_indices"]
    rows = int(p["packed_rows"][0]) if graph_layout else w.cols
    B = torch.zeros(rows, 256, dtype=dev(p["value"]).dtype, device="cuda")
    args = (dev(p["crow_window_ptr"], i32), dev(ccol, i32), dev(p["value"]), dev(p["vrow_window_ptr"], i32),
            dev(vcol, i32), dev(p["vvalue"]), B, dev(O.make_start(p["crow_window_ptr"], 20)),
            dev(O.make_start(p["vrow_window_ptr"], 40)))
    check_replays(spmm_npu.spmm_ascend_cube, args, B)
