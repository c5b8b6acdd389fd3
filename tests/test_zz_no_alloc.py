"""The allocation-free entry point spmm_csr_run_noalloc, through the C ABI:
two calls in a row (the second on a smaller input, so the scratch holds the
first call's leftovers) each equal spmm_csr_run with a caller workspace bit
for bit (same kernels), and the oracle within the reference's tolerance; a
third call repeats the first; an input whose scratch exceeds the fixed size
is rejected before the device is touched."""

import ctypes
import os

import numpy as np
import pytest
import torch  # first: the library then shares torch's HIP runtime (loaded by SONAME)

from test_cabi import CsrDesc

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "ascend-spmm_amd", "libspmm_mi355x.so")


@pytest.fixture(scope="module")
def lib():
    lib = ctypes.CDLL(LIB)
    lib.spmm_last_error.restype = ctypes.c_char_p
    lib.spmm_csr_noalloc_max_scratch.restype = ctypes.c_size_t
    return lib


def case(seed, rows, K, N, max_deg, long_rows, npdt):
    rng = np.random.default_rng(seed)
    deg = rng.integers(0, max_deg + 1, rows)
    for r, d in long_rows:
        deg[r] = d
    crow = np.zeros(rows + 1, np.int64)
    crow[1:] = np.cumsum(deg)
    col = np.concatenate([np.sort(rng.choice(K, d, replace=False)) for d in deg]).astype(np.int64)
    vals = rng.uniform(-1, 1, col.size).astype(npdt)
    B = rng.standard_normal((K, N)).astype(npdt)
    return crow, col, vals, B


def run_both(lib, crow, col, vals, B):
    """(noalloc output, spmm_csr_run output) as CPU tensors."""
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    p = lambda x: ctypes.c_void_p(x.data_ptr())  # noqa: E731
    rows, (K, N) = crow.size - 1, B.shape
    vt = 0 if B.dtype == np.float16 else 1
    d = CsrDesc(rows, col.size, K, N, 0, vt)
    d_crow, d_col, d_val, d_B = t(crow.astype(np.int32)), t(col.astype(np.int32)), t(vals), t(B)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = torch.full((rows, N), float("nan"), dtype=d_B.dtype, device="cuda")
    rc = lib.spmm_csr_run_noalloc(ctypes.byref(d), p(d_crow), p(d_col), p(d_val), p(d_B), p(out), stream)
    assert rc == 0, lib.spmm_last_error()
    ref = torch.full_like(out, float("nan"))
    ws_bytes = ctypes.c_size_t(0)
    assert lib.spmm_csr_workspace(ctypes.byref(d), ctypes.byref(ws_bytes)) == 0
    assert ws_bytes.value <= lib.spmm_csr_noalloc_max_scratch()
    ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device="cuda")
    rc = lib.spmm_csr_run(ctypes.byref(d), p(d_crow), p(d_col), p(d_val), p(d_B), p(ref), p(ws),
                          ctypes.c_size_t(ws_bytes.value), stream)
    assert rc == 0, lib.spmm_last_error()
    torch.cuda.synchronize()
    return out.cpu(), ref.cpu()


def test_noalloc_matches_workspace_entry_point(lib):
    import oracle as O

    # First call: 60k rows, long rows crossing many ranges (partial slots in
    # use), fp16 N=128.  Second: a smaller fp32 input of 3000 rows at N=64.
    big = case(1, 60000, 40000, 128, 40, [(7, 5000), (30000, 12000), (59990, 3000)], np.float16)
    small = case(2, 3000, 2000, 64, 30, [(5, 1500), (2000, 900)], np.float32)
    for (crow, col, vals, B), tol in ((big, 2e-2), (small, 1e-4), (big, 2e-2)):
        out, ref = run_both(lib, crow, col, vals, B)
        assert torch.equal(out, ref), "noalloc differs from spmm_csr_run"
        expected = O.spmm_f64(crow, col, vals, B)
        assert np.allclose(out.double().numpy(), expected, atol=tol, rtol=tol)
    assert lib.spmm_csr_noalloc_max_scratch() == 64 << 20


def test_noalloc_rejects_inputs_beyond_its_scratch(lib):
    # 40M nonzeros at fp16 N=1024: about 1.3 GB of partial slots
    d = CsrDesc(1000, 40_000_000, 1000, 1024, 0, 0)
    assert lib.spmm_csr_run_noalloc(ctypes.byref(d), None, None, None, None, None, None) == 4
    assert b"fixed" in lib.spmm_last_error() and b"spmm_csr_run" in lib.spmm_last_error()
