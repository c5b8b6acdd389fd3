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


@pytest.mark.parametrize("width", [64, 128, 256])
def test_spmm_csr_graph_replays_segment_path(spmm_npu, width):
    """Config 2 at full size (2.0M nonzeros, dense operands of 12.8-51.2 MB):
    the segment path's three launches (classification, tiles with segment
    work-groups, post pass) replay from the graph like the eager call, at
    widths taking 1, 2 and 3 segment work-groups per slab."""
    w = W.config2()
    assert w.nnz >= 1 << 20
    B = dev(w.dense(width))
    args = (dev(w.crow, torch.int32), dev(w.col, torch.int32), dev(w.values), B, dev(O.make_start(w.crow, 40)))
    out = check_replays(spmm_npu.spmm_csr, args, B)
    assert out.shape == (w.rows, width)


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


# ---- C ABI calls under capture (ctypes, the current stream's handle) -------

import ctypes  # noqa: E402
import os  # noqa: E402

from test_cabi import CsrDesc  # noqa: E402

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "ascend-spmm_amd",
                   "libspmm_mi355x.so")


class CubeOpDesc(ctypes.Structure):
    _fields_ = [("windows", ctypes.c_int64), ("nnz", ctypes.c_int64), ("dense_rows", ctypes.c_int64),
                ("width", ctypes.c_int64), ("index_type", ctypes.c_int32), ("value_type", ctypes.c_int32)]


@pytest.fixture(scope="module")
def lib():
    h = ctypes.CDLL(LIB)
    h.spmm_last_error.restype = ctypes.c_char_p
    h.spmm_pack_workspace.restype = ctypes.c_size_t
    return h


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ok(lib, rc):
    assert rc == 0, lib.spmm_last_error()


def test_cabi_spmm_cube_op_graph_replays(spmm_npu, lib):
    """spmm_cube_op_run (window-encoded decode + MFMA block kernel) captured."""
    rng = np.random.default_rng(5)
    n, K = 400, 300
    deg = rng.integers(0, 25, n)
    crow = np.concatenate([[0], np.cumsum(deg)]).astype(np.int64)
    col = np.concatenate([np.sort(rng.choice(K, d, replace=False)) for d in deg]).astype(np.int64)
    val = rng.uniform(-1, 1, col.size).astype(np.float16)
    rp, enc, v = O.cube_encode(crow, col, val, n)
    d_rp, d_enc, d_v = dev(rp, torch.int32), dev(enc, torch.int32), dev(v)
    B = torch.zeros(K, 64, dtype=torch.float16, device="cuda")
    d = CubeOpDesc(rp.size - 1, enc.size, K, 64, 0, 0)
    need = ctypes.c_size_t(0)
    _ok(lib, lib.spmm_cube_op_workspace(ctypes.byref(d), ctypes.byref(need)))

    def op(dense):
        out = torch.empty(16 * (rp.size - 1), 64, dtype=torch.float16, device="cuda")
        ws = torch.empty(max(need.value, 1), dtype=torch.uint8, device="cuda")
        _ok(lib, lib.spmm_cube_op_run(ctypes.byref(d), _p(d_rp), _p(d_enc), _p(d_v), _p(dense), _p(out), _p(ws),
                                      ctypes.c_size_t(need.value), _stream()))
        return out

    out = check_replays(op, (B,), B)
    assert torch.equal(out, spmm_npu.spmm_cube(d_rp, d_enc, d_v, B, torch.zeros(20, dtype=torch.int32,
                                                                                    device="cuda")))


def test_cabi_pack_restore_graph_replays(spmm_npu, lib):
    """spmm_pack_rows and spmm_restore_rows captured (the Python
    pack_node_tensor / restore_node_tensor check inv_permutation on the host,
    which reads the device, so the C ABI calls are the capturable form)."""
    rng = np.random.default_rng(6)
    rows, packed_rows, width = 300, 320, 48
    inv = dev(rng.permutation(packed_rows)[:rows].astype(np.int64))
    X = torch.zeros(rows, width, dtype=torch.float32, device="cuda")
    row_bytes = width * 4
    need = lib.spmm_pack_workspace(ctypes.c_int64(packed_rows))

    def pack(src):
        packed = torch.empty(packed_rows, width, device="cuda")
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
        _ok(lib, lib.spmm_pack_rows(_p(src), ctypes.c_int64(rows), ctypes.c_int64(row_bytes), _p(inv), _p(packed),
                                    ctypes.c_int64(packed_rows), _p(ws), ctypes.c_size_t(need), _stream()))
        return packed

    def restore(src):
        out = torch.empty(rows, width, device="cuda")
        _ok(lib, lib.spmm_restore_rows(_p(pack(src)), ctypes.c_int64(packed_rows), ctypes.c_int64(row_bytes),
                                       _p(inv), ctypes.c_int64(rows), _p(out), _stream()))
        return out

    packed = check_replays(pack, (X,), X)
    assert torch.equal(packed, spmm_npu.pack_node_tensor(X, inv.cpu(), packed_rows))
    back = check_replays(restore, (X,), X)
    assert torch.equal(back, X)


def test_cabi_noalloc_graph_replays(spmm_npu, lib):
    """spmm_csr_run_noalloc (library scratch, nothing allocated) captured."""
    w = W.config2(scale=0.05)
    B = dev(w.dense(128))
    d = CsrDesc(w.rows, w.nnz, w.cols, 128, 0, 0)
    crow, col, val = dev(w.crow, torch.int32), dev(w.col, torch.int32), dev(w.values)

    def op(dense):
        out = torch.empty(w.rows, 128, dtype=torch.float16, device="cuda")
        _ok(lib, lib.spmm_csr_run_noalloc(ctypes.byref(d), _p(crow), _p(col), _p(val), _p(dense), _p(out),
                                          _stream()))
        return out

    out = check_replays(op, (B,), B)
    assert torch.equal(out, spmm_npu.spmm_csr(crow, col, val, B, dev(O.make_start(w.crow, 40))))
