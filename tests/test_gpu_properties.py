"""Property-based GPU parity (hypothesis, fixed examples): on generated CSR
matrices the HIP operators equal the oracle, bit for bit for the integer
and layout work (csr_to_bcsr, block_level_split, preprocess) and within
the reference's tolerance for the SpMM sums (spmm_csr, spmm_ascend_cube on
every layout), with widths and dtypes drawn too."""

import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

import oracle as O
from test_gpu_preprocess import assert_same
from test_properties import csr

pytestmark = pytest.mark.gpu

SETTINGS = settings(max_examples=25, deadline=None, derandomize=True,
                    suppress_health_check=[HealthCheck.too_slow, HealthCheck.function_scoped_fixture])
TOL = {np.float16: 2e-2, np.float32: 1e-4}


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dtype is None else t.to(dtype)


def close(out, expected, npdt):
    tol = TOL[npdt]
    a = out.float().cpu().double().numpy()
    assert np.allclose(a, expected, atol=tol, rtol=tol), float(np.abs(a - expected).max())


@SETTINGS
@given(m=csr(max_rows=300, max_cols=300, max_deg=80), width=st.sampled_from([16, 32, 64, 128, 256]),
       half=st.booleans(), i64=st.booleans())
def test_spmm_csr_matches_oracle(spmm_npu, m, width, half, i64):
    rows, cols, crow, col, vals = m
    npdt = np.float16 if half else np.float32
    v = vals.astype(npdt)
    B = np.random.default_rng(width + rows).standard_normal((cols, width)).astype(npdt)
    it = torch.int64 if i64 else torch.int32
    out = spmm_npu.spmm_csr(dev(crow, it), dev(col, it), dev(v), dev(B), dev(O.make_start(crow, 40)))
    assert out.shape == (rows, width)
    close(out, O.spmm_f64(crow, col, v, B), npdt)


@SETTINGS
@given(m=csr(max_rows=120, max_cols=120), half=st.booleans())
def test_converters_bit_exact(spmm_npu, m, half):
    rows, cols, crow, col, vals = m
    v = vals.astype(np.float16 if half else np.float32)
    assert_same(spmm_npu.csr_to_bcsr(dev(crow), dev(col), dev(v), rows, cols, 16),
                O.csr_to_bcsr(crow, col, v, rows, cols, 16))
    assert_same(spmm_npu.csr_to_ascend_cube(dev(crow), dev(col), dev(v), rows, cols, 16),
                O.csr_to_ascend_cube(crow, col, v, rows, cols, 16))


@SETTINGS
@given(m=csr(max_rows=120, max_cols=120), a=st.floats(0.05, 20.0), half=st.booleans())
def test_block_level_split_and_mixed_op(spmm_npu, m, a, half):
    rows, cols, crow, col, vals = m
    npdt = np.float16 if half else np.float32
    v = vals.astype(npdt)
    ref = O.block_level_split(crow, col, v, rows, cols, a, 16)
    got = spmm_npu.block_level_split(torch.from_numpy(crow), torch.from_numpy(col), torch.from_numpy(v),
                                     rows, cols, a, 16)
    assert_same(got, ref)
    B = np.random.default_rng(rows).standard_normal((cols, 64)).astype(npdt)
    i32 = torch.int32
    out = spmm_npu.spmm_ascend_cube(
        dev(ref["crow_window_ptr"], i32), dev(ref["unique_col_ids"], i32), dev(ref["value"]),
        dev(ref["vrow_window_ptr"], i32), dev(ref["vcol_indices"], i32), dev(ref["vvalue"]), dev(B),
        dev(O.make_start(ref["crow_window_ptr"], 20)), dev(O.make_start(ref["vrow_window_ptr"], 40)))
    close(out[:rows], O.spmm_f64(crow, col, v, B), npdt)


@SETTINGS
@given(m=csr(max_rows=120, square=True), graph_layout=st.booleans(), half=st.booleans())
def test_preprocess_bit_exact_and_unpermuted_product(spmm_npu, m, graph_layout, half):
    rows, cols, crow, col, vals = m
    npdt = np.float16 if half else np.float32
    v = vals.astype(npdt)
    ref = O.preprocess(crow, col, v, rows, cols, 16, graph_layout)
    got = spmm_npu.preprocess(dev(crow), dev(col), dev(v), rows, cols, 16, graph_layout)
    assert_same(got, ref)
    B = np.random.default_rng(rows + 1).standard_normal((cols, 32)).astype(npdt)
    i32 = torch.int32
    ccol = ref["renumbered_unique_col_ids"] if graph_layout else ref["unique_col_ids"]
    vcol = ref["renumbered_vcol_indices"] if graph_layout else ref["vcol_indices"]
    inv = torch.from_numpy(ref["inv_permutation"])
    dense = dev(B)
    if graph_layout:
        dense = spmm_npu.pack_node_tensor(dense, inv, int(ref["packed_rows"][0]))
    out = spmm_npu.spmm_ascend_cube(
        dev(ref["crow_window_ptr"], i32), dev(ccol, i32), dev(ref["value"]),
        dev(ref["vrow_window_ptr"], i32), dev(vcol, i32), dev(ref["vvalue"]), dense,
        dev(O.make_start(ref["crow_window_ptr"], 20)), dev(O.make_start(ref["vrow_window_ptr"], 40)))
    close(spmm_npu.restore_node_tensor(out, inv), O.spmm_f64(crow, col, v, B), npdt)
