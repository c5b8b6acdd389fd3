"""The C ABI of libspmm_mi355x.so: every function declared in include/*.h is
exported (CPU), host-side validation answers without a GPU (CPU), and direct
ctypes calls of the run entry points match the oracle (GPU)."""

import ctypes
import glob
import os
import re

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "ascend-spmm_amd", "libspmm_mi355x.so")


def declared_functions():
    names = []
    for header in glob.glob(os.path.join(REPO, "include", "*.h")):
        text = open(header).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(spmm_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


class CsrDesc(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_int64), ("nnz", ctypes.c_int64), ("dense_rows", ctypes.c_int64),
                ("width", ctypes.c_int64), ("index_type", ctypes.c_int32),
                ("value_type", ctypes.c_int32)]


class MixedDesc(ctypes.Structure):
    _fields_ = [("block_windows", ctypes.c_int64), ("block_count", ctypes.c_int64),
                ("block_values", ctypes.c_int64), ("vector_rows", ctypes.c_int64),
                ("vector_nnz", ctypes.c_int64), ("dense_rows", ctypes.c_int64),
                ("width", ctypes.c_int64), ("index_type", ctypes.c_int32),
                ("value_type", ctypes.c_int32)]


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built (python ascend-spmm_amd/build.py)")
    # torch first, also when this file runs alone: the library's
    # libamdhip64.so.7 dependency then resolves (by SONAME) to the HIP runtime
    # torch loaded.  Loaded the other way round, torch brings a second
    # runtime into the process, and the one initialised second finds no device.
    import torch  # noqa: F401

    lib = ctypes.CDLL(LIB)
    lib.spmm_last_error.restype = ctypes.c_char_p
    lib.spmm_version.restype = ctypes.c_char_p
    lib.spmm_mixed_out_rows.restype = ctypes.c_int64
    lib.spmm_pack_workspace.restype = ctypes.c_size_t
    return lib


def test_header_declares_entry_points():
    names = declared_functions()
    for required in ("spmm_csr_run", "spmm_csr_workspace", "spmm_mixed_run",
                     "spmm_mixed_workspace", "spmm_pack_rows", "spmm_restore_rows",
                     "spmm_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"
    assert lib.spmm_version().startswith(b"spmm_mi355x")


def test_host_validation_without_gpu(lib):
    d = CsrDesc(10, 5, 10, 24, 0, 0)  # fp16 width 24: not divisible by 16
    rc = lib.spmm_csr_run(ctypes.byref(d), None, None, None, None, None, None, 0, None)
    assert rc == 4 and b"divisible by 16" in lib.spmm_last_error()
    d = CsrDesc(10, 5, 10, 1040, 0, 0)
    assert lib.spmm_csr_run(ctypes.byref(d), None, None, None, None, None, None, 0, None) == 4
    assert b"<= 1024 for FP16" in lib.spmm_last_error()
    d = CsrDesc(10, 5, 10, 16, 7, 0)  # bad index type
    assert lib.spmm_csr_run(ctypes.byref(d), None, None, None, None, None, None, 0, None) == 4
    d = CsrDesc(10, 5, 10, 16, 0, 0)
    assert lib.spmm_csr_run(ctypes.byref(d), None, None, None, None, None, None, 0, None) == 1
    size = ctypes.c_size_t(0)
    assert lib.spmm_csr_workspace(ctypes.byref(d), ctypes.byref(size)) == 0
    m = MixedDesc(3, 0, 0, 100, 0, 10, 16, 0, 0)
    assert lib.spmm_mixed_out_rows(ctypes.byref(m)) == 100
    m.block_windows = 10
    assert lib.spmm_mixed_out_rows(ctypes.byref(m)) == 160
    assert lib.spmm_pack_workspace(ctypes.c_int64(100)) == 800
    # the allocation-free spmm_csr rejects a call whose scratch exceeds its
    # fixed array before any device call (40M nonzeros at fp16 N=1024)
    d = CsrDesc(1000, 40_000_000, 1000, 1024, 0, 0)
    assert lib.spmm_csr_run_noalloc(ctypes.byref(d), None, None, None, None, None, None) == 4
    assert b"more than the library's fixed" in lib.spmm_last_error()


@pytest.mark.gpu
def test_direct_cabi_calls_match_oracle(lib):
    import torch

    import oracle as O

    rng = np.random.default_rng(5)
    rows, K, N = 200, 150, 64
    deg = rng.integers(0, 30, rows)
    crow = np.zeros(rows + 1, np.int64)
    crow[1:] = np.cumsum(deg)
    col = np.concatenate([np.sort(rng.choice(K, d, replace=False)) for d in deg]).astype(np.int64)
    vals = rng.uniform(-1, 1, col.size).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    d_crow, d_col = t(crow.astype(np.int32)), t(col.astype(np.int32))
    d_val, d_B = t(vals), t(B)
    out = torch.empty(rows, N, device="cuda")
    d = CsrDesc(rows, col.size, K, N, 0, 1)
    ws_bytes = ctypes.c_size_t(0)
    assert lib.spmm_csr_workspace(ctypes.byref(d), ctypes.byref(ws_bytes)) == 0
    ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda x: ctypes.c_void_p(x.data_ptr())
    rc = lib.spmm_csr_run(ctypes.byref(d), p(d_crow), p(d_col), p(d_val), p(d_B), p(out), p(ws),
                          ctypes.c_size_t(ws_bytes.value), stream)
    assert rc == 0, lib.spmm_last_error()
    torch.cuda.synchronize()
    expected = O.spmm_f64(crow, col, vals, B)
    assert np.allclose(out.cpu().numpy(), expected, atol=1e-4, rtol=1e-4)

    # the mixed entry point with an empty block part is bitwise spmm_csr
    out2 = torch.empty(rows, N, device="cuda")
    zero = torch.zeros(1, dtype=torch.int32, device="cuda")
    m = MixedDesc(0, 0, 0, rows, col.size, K, N, 0, 1)
    assert lib.spmm_mixed_workspace(ctypes.byref(m), ctypes.byref(ws_bytes)) == 0
    ws2 = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device="cuda")
    rc = lib.spmm_mixed_run(ctypes.byref(m), p(zero), None, None, p(d_crow), p(d_col), p(d_val),
                            p(d_B), p(out2), p(ws2), ctypes.c_size_t(ws_bytes.value), stream)
    assert rc == 0, lib.spmm_last_error()
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), out2.cpu())


@pytest.mark.gpu
@pytest.mark.parametrize("vector_rows", [0, 16 * 6 + 5])
def test_mixed_block_only_writes_every_row(lib, vector_rows):
    """Block part only (no vector nonzeros) with windows that have no blocks:
    every output row is written (the block sums, zeros elsewhere), over an
    output pre-filled with NaN.  With vector_rows past the block windows, the
    rows beyond them are written as zeros too."""
    import torch

    import oracle as O

    rng = np.random.default_rng(8)
    K, N, windows = 300, 128, 5
    rows = 16 * windows
    deg = rng.integers(1, 25, rows)
    deg[16:32] = 0   # window 1 has no blocks
    deg[64:80] = 0   # nor the last window
    crow = np.zeros(rows + 1, np.int64)
    crow[1:] = np.cumsum(deg)
    col = np.concatenate([np.sort(rng.choice(K, d, replace=False)) for d in deg]).astype(np.int64)
    vals = rng.uniform(-1, 1, col.size).astype(np.float16)
    B = rng.standard_normal((K, N)).astype(np.float16)
    b = O.csr_to_bcsr(crow, col, vals, rows, K, 16)
    assert np.diff(b["crow_window_ptr"])[1] == 0 and np.diff(b["crow_window_ptr"])[4] == 0
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    p = lambda x: ctypes.c_void_p(x.data_ptr())
    i32 = np.int32
    d_crow, d_ucol, d_val = t(b["crow_window_ptr"].astype(i32)), t(b["unique_col_ids"].astype(i32)), t(b["value"])
    d_vrow = torch.zeros(vector_rows + 1, dtype=torch.int32, device="cuda")
    d_B = t(B)
    m = MixedDesc(windows, b["unique_col_ids"].size, b["value"].size, vector_rows, 0, K, N, 0, 0)
    out_rows = lib.spmm_mixed_out_rows(ctypes.byref(m))
    assert out_rows == max(rows, vector_rows)
    out = torch.full((out_rows, N), float("nan"), dtype=torch.float16, device="cuda")
    ws_bytes = ctypes.c_size_t(0)
    assert lib.spmm_mixed_workspace(ctypes.byref(m), ctypes.byref(ws_bytes)) == 0
    ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.spmm_mixed_run(ctypes.byref(m), p(d_crow), p(d_ucol), p(d_val), p(d_vrow), None, None,
                            p(d_B), p(out), p(ws), ctypes.c_size_t(ws_bytes.value), stream)
    assert rc == 0, lib.spmm_last_error()
    torch.cuda.synchronize()
    got = out.cpu().double().numpy()
    expected = np.zeros((out_rows, N))
    expected[:rows] = O.spmm_f64(crow, col, vals, B)
    assert not np.isnan(got).any()
    assert np.allclose(got, expected, atol=2e-2, rtol=2e-2)
    assert (got[16:32] == 0).all() and (got[64:] == 0).all()


def banded_csr(rng, rows, width=16, dmin=2, dmax=8):
    """Rows of dmin..dmax distinct sorted columns inside a band of `width`
    columns around the diagonal."""
    deg = rng.integers(dmin, dmax + 1, rows)
    pick = np.argsort(rng.random((rows, width)), axis=1)
    offs = np.sort(np.where(np.arange(width)[None, :] < deg[:, None], pick, width), axis=1)
    lo = np.clip(np.arange(rows) - width // 2, 0, rows - width)
    col = (lo[:, None] + offs)[offs < width].astype(np.int64)
    crow = np.zeros(rows + 1, np.int64)
    crow[1:] = np.cumsum(deg)
    return crow, col


@pytest.mark.gpu
@pytest.mark.parametrize("windows,invalid", [(1, False), (9, False), (1000, False), (1000, True), (16384, False)])
def test_window_order_writes_every_window(lib, windows, invalid):
    """Block part of a banded matrix plus a random vector part at N=128 fp16,
    so the block windows take the locality order when they are local (1000
    and 16384 windows; 1 and 9 windows span too much of K and keep theirs).
    The output is pre-filled with NaN and the workspace with 0xFF bytes:
    every row must be written, whatever the workspace held, and match
    A1 @ B + A2 @ B.  With `invalid`, some blocks get column ids -5 or K + 7
    (first and last blocks of windows included, which the order's keys
    read): they contribute zero."""
    import torch

    import oracle as O

    rng = np.random.default_rng(12 + windows)
    rows, N = 16 * windows, 128
    crow, col = banded_csr(rng, rows)
    vals = rng.uniform(-1, 1, col.size).astype(np.float16)
    vdeg = rng.integers(0, 3, rows)
    vcrow = np.zeros(rows + 1, np.int64)
    vcrow[1:] = np.cumsum(vdeg)
    vcol = rng.integers(0, rows, int(vcrow[-1])).astype(np.int64)
    vvals = rng.uniform(-1, 1, vcol.size).astype(np.float16)
    B = rng.standard_normal((rows, N)).astype(np.float16)
    b = O.csr_to_bcsr(crow, col, vals, rows, rows, 16)
    ucol = b["unique_col_ids"].astype(np.int64)
    if invalid:
        wp = b["crow_window_ptr"].astype(np.int64)
        nonempty = np.flatnonzero(np.diff(wp) > 0)
        bad = np.concatenate([wp[nonempty[::7]], wp[nonempty[3::7] + 1] - 1, rng.choice(ucol.size, 50)])
        ucol[bad[::2]] = -5
        ucol[bad[1::2]] = rows + 7
        # The block part's product without the invalid blocks: its CSR form.
        wins = np.repeat(np.arange(windows), np.diff(wp))
        r16 = (16 * wins[:, None] + np.arange(16)[None, :]).reshape(-1)
        c16 = np.repeat(ucol, 16)
        v16 = b["value"].reshape(-1)
        keep = (v16 != 0) & (c16 >= 0) & (c16 < rows)
        order = np.lexsort((c16[keep], r16[keep]))
        crow = np.zeros(rows + 1, np.int64)
        crow[1:] = np.cumsum(np.bincount(r16[keep], minlength=rows))
        col, vals = c16[keep][order], v16[keep][order]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    p = lambda x: ctypes.c_void_p(x.data_ptr())
    i32 = np.int32
    d = [t(b["crow_window_ptr"].astype(i32)), t(ucol.astype(i32)), t(b["value"]),
         t(vcrow.astype(i32)), t(vcol.astype(i32)), t(vvals)]
    m = MixedDesc(windows, b["unique_col_ids"].size, b["value"].size, rows, vcol.size, rows, N, 0, 0)
    out = torch.full((lib.spmm_mixed_out_rows(ctypes.byref(m)), N), float("nan"), dtype=torch.float16,
                     device="cuda")
    ws_bytes = ctypes.c_size_t(0)
    assert lib.spmm_mixed_workspace(ctypes.byref(m), ctypes.byref(ws_bytes)) == 0
    ws = torch.full((max(ws_bytes.value, 1),), 255, dtype=torch.uint8, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.spmm_mixed_run(ctypes.byref(m), *[p(x) for x in d], p(t(B)), p(out), p(ws),
                            ctypes.c_size_t(ws_bytes.value), stream)
    assert rc == 0, lib.spmm_last_error()
    torch.cuda.synchronize()
    got = out.cpu().double().numpy()
    assert not np.isnan(got).any()
    expected = O.spmm_f64(crow, col, vals, B) + O.spmm_f64(vcrow, vcol, vvals, B)
    assert np.allclose(got[:rows], expected, atol=2e-2, rtol=2e-2)


def test_rowscalar_host_validation(lib):
    d = CsrDesc(10, 5, 10, 24, 0, 0)
    assert lib.spmm_csr_rowscalar_run(ctypes.byref(d), None, None, None, None, None, None) == 4
    assert b"spmm_csr_rowscalar requires feature width divisible by 16" in lib.spmm_last_error()
    d = CsrDesc(10, 5, 10, 16, 0, 0)
    assert lib.spmm_csr_rowscalar_run(ctypes.byref(d), None, None, None, None, None, None) == 1


def test_gather_probe_host_validation(lib):
    """spmm_gather_probe refuses, before any device call, what it cannot run:
    int64 column ids, rows wider than 64 lanes of 16 bytes (fp16 N > 512,
    fp32 N > 256), null and misaligned pointers."""
    fake = ctypes.c_void_p(0x10000)  # aligned; never dereferenced: every check precedes the launch
    probe = lib.spmm_gather_probe
    d = CsrDesc(10, 5, 10, 128, 1, 0)
    assert probe(ctypes.byref(d), fake, fake, fake, fake, None) == 4
    assert b"int32 column ids only" in lib.spmm_last_error()
    for width, value_type in ((1024, 0), (512, 1)):
        d = CsrDesc(10, 5, 10, width, 0, value_type)
        assert probe(ctypes.byref(d), fake, fake, fake, fake, None) == 4
        assert b"rows wider than 64 lanes" in lib.spmm_last_error()
    d = CsrDesc(10, 5, 10, 128, 0, 0)
    assert probe(ctypes.byref(d), None, fake, fake, fake, None) == 1
    assert probe(ctypes.byref(d), fake, fake, ctypes.c_void_p(0x10004), fake, None) != 0


@pytest.mark.gpu
@pytest.mark.parametrize("value_type,N", [(0, 128), (0, 512), (1, 64), (1, 256)])
def test_gather_probe_sums(lib, value_type, N):
    """The probe accumulates value x dense row over every nonzero of its
    ranges and each thread writes the sum of its lanes' columns, so the sink
    adds up to sum_p value[p] * rowsum(dense[col[p]]) (invalid columns add
    zero); checked against that closed form in fp64."""
    import torch

    rng = np.random.default_rng(31 + N)
    nnz, K = 5000, 700
    col = rng.integers(0, K, nnz).astype(np.int32)
    col[::23] = K + 5
    npdt = np.float16 if value_type == 0 else np.float32
    vals = rng.uniform(-1, 1, nnz).astype(npdt)
    B = rng.standard_normal((K, N)).astype(npdt)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    d = CsrDesc(1, nnz, K, N, 0, value_type)
    lib.spmm_gather_probe_sink.restype = ctypes.c_size_t
    sink = torch.full((int(lib.spmm_gather_probe_sink(ctypes.byref(d))),), float("nan"), device="cuda")
    d_col, d_val, d_B = t(col), t(vals), t(B)
    p = lambda x: ctypes.c_void_p(x.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.spmm_gather_probe(ctypes.byref(d), p(d_col), p(d_val), p(d_B), p(sink), stream) == 0
    torch.cuda.synchronize()
    keep = col < K
    rowsum = B.astype(np.float64).sum(axis=1)
    expected = float((vals.astype(np.float64)[keep] * rowsum[col[keep]]).sum())
    got = float(sink.double().sum())
    assert abs(got - expected) <= 1e-3 * max(1.0, float(np.abs(vals.astype(np.float64)[keep] * rowsum[col[keep]]).sum()))


@pytest.mark.gpu
@pytest.mark.parametrize("value_type,N", [(0, 16), (0, 128), (1, 8), (1, 64)])
def test_rowscalar_baseline_matches_oracle_and_csr(lib, value_type, N):
    """The thread-per-row baseline computes the same row sums as spmm_csr:
    within tolerance of fp64 everywhere, bitwise on rows that spmm_csr sums
    in one piece (at most R/2 nonzeros; R = 16 for this size)."""
    import torch

    import oracle as O

    rng = np.random.default_rng(9 + N)
    rows, K = 300, 180
    deg = rng.integers(0, 25, rows)
    crow = np.zeros(rows + 1, np.int64)
    crow[1:] = np.cumsum(deg)
    col = np.concatenate([np.sort(rng.choice(K, d, replace=False)) for d in deg]).astype(np.int64)
    col[::17] = K + 3  # invalid columns contribute zero
    npdt = np.float16 if value_type == 0 else np.float32
    vals = rng.uniform(-1, 1, col.size).astype(npdt)
    B = rng.standard_normal((K, N)).astype(npdt)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    d_crow, d_col, d_val, d_B = t(crow.astype(np.int32)), t(col.astype(np.int32)), t(vals), t(B)
    out = torch.empty(rows, N, dtype=d_B.dtype, device="cuda")
    ref = torch.empty_like(out)
    d = CsrDesc(rows, col.size, K, N, 0, value_type)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda x: ctypes.c_void_p(x.data_ptr())
    assert lib.spmm_csr_rowscalar_run(ctypes.byref(d), p(d_crow), p(d_col), p(d_val), p(d_B), p(out), stream) == 0
    ws_bytes = ctypes.c_size_t(0)
    assert lib.spmm_csr_workspace(ctypes.byref(d), ctypes.byref(ws_bytes)) == 0
    ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device="cuda")
    assert lib.spmm_csr_run(ctypes.byref(d), p(d_crow), p(d_col), p(d_val), p(d_B), p(ref), p(ws),
                            ctypes.c_size_t(ws_bytes.value), stream) == 0, lib.spmm_last_error()
    torch.cuda.synchronize()
    tol = 2e-2 if value_type == 0 else 1e-4
    keep = col < K
    expected = O.spmm_f64(crow, np.where(keep, col, 0), np.where(keep, vals, 0).astype(npdt), B)
    assert np.allclose(out.float().cpu().numpy(), expected, atol=tol, rtol=tol)
    short = deg <= 8
    assert torch.equal(out.cpu()[torch.from_numpy(short)], ref.cpu()[torch.from_numpy(short)])


@pytest.mark.gpu
def test_segment_path_ignores_workspace_contents(lib):
    """spmm_csr on the segment path (config 2 at full size, 2.0M nonzeros, N=128
    fp16) keeps its segment words, chunk flags and tile first rows in the
    workspace.  The result must not depend on what the workspace held: a
    workspace of 0xFF bytes (every chunk flag set, every tile row -1), and
    the same workspace after a call on the row-reversed matrix (whose long
    rows, segments and tile rows sit elsewhere), give the bits of a call on a
    zeroed workspace, over outputs pre-filled with NaN."""
    import torch

    import workloads as W

    w = W.config2()
    N = 128
    crow = w.crow.astype(np.int64)
    deg = np.diff(crow)
    # The row-reversed matrix: row r of it is row rows-1-r of config 2.
    new_row = (w.rows - 1) - np.repeat(np.arange(w.rows), deg)
    perm = np.argsort(new_row, kind="stable")
    crow2 = np.concatenate([[0], np.cumsum(deg[::-1])])
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    p = lambda x: ctypes.c_void_p(x.data_ptr())
    first = [t(crow.astype(np.int32)), t(w.col.astype(np.int32)), t(w.values)]
    second = [t(crow2.astype(np.int32)), t(w.col[perm].astype(np.int32)), t(w.values[perm])]
    B = t(w.dense(N))
    d = CsrDesc(w.rows, w.nnz, w.cols, N, 0, 0)
    assert w.nnz >= 1 << 20 and B.dtype == torch.float16
    ws_bytes = ctypes.c_size_t(0)
    assert lib.spmm_csr_workspace(ctypes.byref(d), ctypes.byref(ws_bytes)) == 0
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def run(mat, ws):
        out = torch.full((w.rows, N), float("nan"), dtype=torch.float16, device="cuda")
        rc = lib.spmm_csr_run(ctypes.byref(d), *[p(x) for x in mat], p(B), p(out), p(ws),
                              ctypes.c_size_t(ws_bytes.value), stream)
        assert rc == 0, lib.spmm_last_error()
        return out

    expected = run(first, torch.zeros(ws_bytes.value, dtype=torch.uint8, device="cuda"))
    ws = torch.full((ws_bytes.value,), 255, dtype=torch.uint8, device="cuda")
    got_ff = run(first, ws)
    other = run(second, ws)
    got_reused = run(first, ws)
    torch.cuda.synchronize()
    assert not torch.isnan(expected).any()
    assert torch.equal(got_ff, expected)
    assert torch.equal(got_reused, expected)
    # the reversed matrix's rows are config 2's rows, reversed, summed in the
    # same ranges only where the row boundaries line up: compare with tolerance
    assert torch.allclose(other.flip(0).float(), expected.float(), atol=2e-2, rtol=2e-2)
