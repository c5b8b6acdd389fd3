"""GPU preprocessing (csr_to_bcsr, csr_to_ascend_cube, block_level_split,
preprocess) against the CPU oracle: every output key must be bit-identical
(same dtype, same integers, same value bits), as the reference's host
routines produce (extension/custom_op.cpp:429-1412)."""

import numpy as np
import pytest
import torch

import oracle as O
import preprocess_cases as PC
import workloads as W

pytestmark = pytest.mark.gpu

NP_DT = {torch.float16: np.float16, torch.float32: np.float32, torch.float64: np.float64}


def random_csr(rng, rows, cols, max_deg, long_rows=(), empty_frac=0.2, dense_windows=0):
    deg = rng.integers(0, max_deg + 1, size=rows)
    deg[rng.random(rows) < empty_frac] = 0
    for r, d in long_rows:
        deg[r] = min(d, cols)
    parts = [np.sort(rng.choice(cols, int(d), replace=False)) for d in deg]
    for w in range(min(dense_windows, rows // 16)):  # a few near-dense 16-row windows
        base = rng.choice(max(cols - 24, 1))
        for r in range(16 * w, 16 * w + 16):
            parts[r] = np.union1d(parts[r], np.arange(base, min(base + 24, cols)))
    crow = np.zeros(rows + 1, dtype=np.int64)
    crow[1:] = np.cumsum([p.size for p in parts])
    col = np.concatenate(parts).astype(np.int64) if parts else np.zeros(0, np.int64)
    return crow, col


def assert_same(gpu: dict, ref: dict, keys=None):
    keys = keys or ref.keys()
    assert set(gpu.keys()) == set(ref.keys()), (sorted(gpu), sorted(ref))
    for k in keys:
        g = gpu[k].cpu().numpy()
        r = ref[k]
        assert g.dtype == r.dtype, f"{k}: dtype {g.dtype} != {r.dtype}"
        assert g.shape == r.shape, f"{k}: shape {g.shape} != {r.shape}"
        if g.dtype.kind == "f":
            assert np.array_equal(g.view(f"u{g.itemsize}"), r.view(f"u{r.itemsize}")), f"{k}: value bits differ"
        else:
            assert np.array_equal(g, r), f"{k}: differs at {np.nonzero(g != r)[0][:5]}"


def cases():
    rng = np.random.default_rng(2027)
    out = []
    c, k = random_csr(rng, 1, 5, 3)
    out.append(("one-row", c, k, 1, 5))
    c, k = random_csr(rng, 37, 50, 8)
    out.append(("small", c, k, 37, 50))
    c, k = random_csr(rng, 200, 200, 12, long_rows=[(3, 190), (100, 150)], dense_windows=4)
    out.append(("square-dense-windows", c, k, 200, 200))
    c, k = random_csr(rng, 333, 1000, 30, empty_frac=0.5)
    out.append(("rect-empty-rows", c, k, 333, 1000))
    w = W.config4(scale=0.02)
    out.append(("C4-scaled", w.crow, w.col, w.rows, w.cols))
    w = W.config3(scale=0.01)
    out.append(("C3-scaled", w.crow, w.col, w.rows, w.cols))
    w = W.config2(scale=0.02)
    out.append(("C2-scaled", w.crow, w.col, w.rows, w.cols))
    out.append(("empty", np.zeros(20, np.int64), np.zeros(0, np.int64), 19, 7))
    return out


CASES = cases()
IDS = [c[0] for c in CASES]


def values_for(col, dtype, seed=5):
    rng = np.random.default_rng(seed)
    return rng.uniform(-1, 1, col.size).astype(NP_DT[dtype])


@pytest.mark.parametrize("case", CASES, ids=IDS)
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_csr_to_bcsr_bit_exact(spmm_npu, case, index_dtype):
    name, crow, col, rows, cols = case
    for vdt in (torch.float16, torch.float32):
        val = values_for(col, vdt)
        c = crow.astype(np.int32 if index_dtype == torch.int32 else np.int64)
        k = col.astype(c.dtype)
        ref = O.csr_to_bcsr(c, k, val, rows, cols, 16)
        got = spmm_npu.csr_to_bcsr(torch.from_numpy(c), torch.from_numpy(k), torch.from_numpy(val), rows, cols, 16)
        assert all(not t.is_cuda for t in got.values())  # CPU in -> CPU out, as the reference
        assert_same(got, ref)


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_csr_to_ascend_cube_bit_exact(spmm_npu, case):
    name, crow, col, rows, cols = case
    val = values_for(col, torch.float16)
    ref = O.csr_to_ascend_cube(crow, col, val, rows, cols, 16)
    got = spmm_npu.csr_to_ascend_cube(torch.from_numpy(crow), torch.from_numpy(col), torch.from_numpy(val),
                                      rows, cols, 16)
    assert_same(got, ref)


def test_converters_window_sizes_and_gpu_inputs(spmm_npu):
    rng = np.random.default_rng(11)
    crow, col = random_csr(rng, 90, 70, 9)
    val = values_for(col, torch.float64)
    for ws in (1, 5, 8, 16):
        ref = O.csr_to_bcsr(crow, col, val, 90, 70, ws)
        got = spmm_npu.csr_to_bcsr(torch.from_numpy(crow).cuda(), torch.from_numpy(col).cuda(),
                                   torch.from_numpy(val).cuda(), 90, 70, ws)
        assert all(t.is_cuda for t in got.values())  # GPU in -> GPU out
        assert_same(got, ref)
        ref = O.csr_to_ascend_cube(crow, col, val, 90, 70, ws)
        got = spmm_npu.csr_to_ascend_cube(torch.from_numpy(crow), torch.from_numpy(col), torch.from_numpy(val),
                                          90, 70, ws)
        assert_same(got, ref)


def test_converters_duplicates_last_wins(spmm_npu):
    crow = np.array([0, 2, 3, 5], np.int64)
    col = np.array([3, 3, 3, 1, 1], np.int64)
    val = np.array([1, 2, 7, 4, 5], np.float32)
    for fn, ofn in ((spmm_npu.csr_to_bcsr, O.csr_to_bcsr), (spmm_npu.csr_to_ascend_cube, O.csr_to_ascend_cube)):
        ref = ofn(crow, col, val, 3, 4, 16)
        got = fn(torch.from_numpy(crow), torch.from_numpy(col), torch.from_numpy(val), 3, 4, 16)
        assert_same(got, ref)


@pytest.mark.parametrize("case", CASES, ids=IDS)
@pytest.mark.parametrize("a", [(222.0 / 190.0) * 0.5, 0.1, 3.0, 295.0 / 505.0])
def test_block_level_split_bit_exact(spmm_npu, case, a):
    name, crow, col, rows, cols = case
    val = values_for(col, torch.float32)
    ref = O.block_level_split(crow, col, val, rows, cols, a, 16)
    got = spmm_npu.block_level_split(torch.from_numpy(crow), torch.from_numpy(col), torch.from_numpy(val),
                                     rows, cols, a, 16)
    assert_same(got, ref)


@pytest.mark.parametrize("window", [2, 16])
def test_block_level_split_occupancy_beyond_the_window(spmm_npu, window):
    """Duplicate CSR entries give a block more entries than the window has
    rows (at least 5 at window 2, at least 42 at window 16).  The GPU split orders
    blocks with one sort on occupancy << position bits | first element when
    occupancies fit the window's bit width, and falls back to the two stable
    sorts when one does not: both must equal the oracle."""
    rng = np.random.default_rng(19)
    crow, col = random_csr(rng, 64, 40, 6)
    rows = [list(col[crow[r]:crow[r + 1]]) for r in range(64)]
    rows[0] = sorted(rows[0] + [7] * (3 if window == 2 else 40))
    rows[1] = sorted(rows[1] + [7] * 2)
    crow = np.zeros(65, np.int64)
    crow[1:] = np.cumsum([len(r) for r in rows])
    col = np.concatenate([np.asarray(r, np.int64) for r in rows])
    val = values_for(col, torch.float32)
    ref = O.block_level_split(crow, col, val, 64, 40, 0.5, window)
    got = spmm_npu.block_level_split(torch.from_numpy(crow), torch.from_numpy(col), torch.from_numpy(val),
                                     64, 40, 0.5, window)
    assert_same(got, ref)


@pytest.mark.parametrize("window", [2, 8, 32])
def test_block_level_split_window_sizes(spmm_npu, window):
    rng = np.random.default_rng(13)
    crow, col = random_csr(rng, 150, 120, 10, dense_windows=3)
    val = values_for(col, torch.float16)
    ref = O.block_level_split(crow.astype(np.int32), col.astype(np.int32), val, 150, 120, 0.5842, window)
    got = spmm_npu.block_level_split(torch.from_numpy(crow.astype(np.int32)), torch.from_numpy(col.astype(np.int32)),
                                     torch.from_numpy(val), 150, 120, 0.5842, window)
    assert_same(got, ref)


@pytest.mark.parametrize("case", CASES, ids=IDS)
@pytest.mark.parametrize("graph_layout", [False, True])
def test_preprocess_bit_exact(spmm_npu, case, graph_layout):
    name, crow, col, rows, cols = case
    for index_dtype, vdt in ((np.int64, torch.float16), (np.int32, torch.float32)):
        val = values_for(col, vdt)
        c, k = crow.astype(index_dtype), col.astype(index_dtype)
        ref = O.preprocess(c, k, val, rows, cols, 16, graph_layout)
        got = spmm_npu.preprocess(torch.from_numpy(c), torch.from_numpy(k), torch.from_numpy(val), rows, cols,
                                  16, graph_layout)
        assert_same(got, ref)


def test_preprocess_hand_example(spmm_npu):
    rows = [[0, 1]] * 16 + [[r] for r in range(16, 32)]
    crow = np.concatenate([[0], np.cumsum([len(x) for x in rows])]).astype(np.int64)
    col = np.concatenate(rows).astype(np.int64)
    val = (np.arange(col.size) + 1).astype(np.float32)
    got = spmm_npu.preprocess(torch.from_numpy(crow), torch.from_numpy(col), torch.from_numpy(val), 32, 32)
    assert int(got["marginal_window"][0]) == 1 and int(got["marginal_aic_blocks"][0]) == 5
    assert float(got["estimated_max_cost"][0]) == 7 / 295
    assert_same(got, O.preprocess(crow, col, val, 32, 32, 16, False))


def test_preprocess_config4_full_size(spmm_npu):
    """Benchmark configuration 4 (200000 rows, ~3.6M nnz) at full size, bit-exact."""
    w = W.config4()
    c32, k32 = w.crow.astype(np.int32), w.col.astype(np.int32)
    ref = O.preprocess(c32, k32, w.values, w.rows, w.cols, 16, False)
    got = spmm_npu.preprocess(torch.from_numpy(c32).cuda(), torch.from_numpy(k32).cuda(),
                              torch.from_numpy(w.values).cuda(), w.rows, w.cols, 16, False)
    assert_same(got, ref)


def test_preprocessing_errors(spmm_npu):
    t = torch.from_numpy
    # unsorted row: the converters require ascending columns per row
    crow = np.array([0, 2], np.int64)
    col = np.array([3, 1], np.int64)
    v = np.ones(2, np.float32)
    with pytest.raises(ValueError, match="sorted in ascending order"):
        spmm_npu.csr_to_bcsr(t(crow), t(col), t(v), 1, 4, 16)
    with pytest.raises(RuntimeError, match="16-row window"):
        spmm_npu.preprocess(t(crow), t(np.array([1, 3], np.int64)), t(v), 1, 4, 8)
    with pytest.raises(RuntimeError, match="column index out of range"):
        spmm_npu.preprocess(t(crow), t(np.array([1, 9], np.int64)), t(v), 1, 4)
    with pytest.raises(ValueError, match="row pointer"):
        spmm_npu.preprocess(t(np.array([0, 5], np.int64)), t(np.array([1, 3], np.int64)), t(v), 1, 4)
    with pytest.raises(ValueError, match="nrows \\+ 1"):
        spmm_npu.csr_to_bcsr(t(crow), t(np.array([1, 3], np.int64)), t(v), 5, 4, 16)
    # occupancy > 16 in the marginal window (duplicate coordinates)
    crow = np.array([0] + [17] * 16, np.int64)
    with pytest.raises(ValueError, match="coalesce duplicate CSR entries"):
        spmm_npu.preprocess(t(crow), t(np.zeros(17, np.int64)), t(np.ones(17, np.float32)), 16, 4)


@pytest.mark.parametrize("name", sorted(PC.CASES))
@pytest.mark.parametrize("graph_layout", [False, True])
def test_preprocess_hand_worked_order_and_tie(spmm_npu, name, graph_layout):
    """The hand-worked cases of preprocess_cases (vector windows in density
    order; an exact tie at the >= marginal test) on the GPU pipeline: the
    hand-derived fields, and every key bit for bit against the oracle."""
    crow, col, val, expected = PC.CASES[name]()
    n = expected["nrows"]
    for index_dtype in (np.int32, np.int64):
        c, k = crow.astype(index_dtype), col.astype(index_dtype)
        got = spmm_npu.preprocess(torch.from_numpy(c).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(val).cuda(),
                                  n, n, 16, graph_layout)
        PC.check_against_hand({key: t.cpu().numpy() for key, t in got.items()}, crow, col, expected)
        assert_same(got, O.preprocess(c, k, val, n, n, 16, graph_layout))
