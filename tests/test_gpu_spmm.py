"""GPU parity tests of the SpMM operators (spmm_csr, spmm_ascend_cube and the
ablation aliases) against the CPU oracle.

Tolerances are the reference's (tests/task_mapping/correctness.py:140-143):
atol = rtol = 2e-2 for fp16 and 1e-4 for fp32, applied to the fp64 oracle.
The vector path must also be bitwise identical across widths and bitwise
equal to spmm_csr when the block part is empty (the contract of
tests/aic_aiv_ablation/bitwise_correctness.py:138-175).
"""

import numpy as np
import pytest
import torch

import oracle as O
import workloads as W

# The segment path's dense-operand limit (kSegMaxDenseBytes): a larger dense
# operand takes the tile path.
SEG_MAX_DENSE = 128 << 20

pytestmark = pytest.mark.gpu

TOL = {"fp16": 2e-2, "fp32": 1e-4}
NP_DT = {"fp16": np.float16, "fp32": np.float32}


def random_csr(rng, rows, cols, max_deg, long_rows=(), empty_frac=0.2):
    """Distinct sorted columns per row; some empty rows; optional long rows."""
    deg = rng.integers(0, max_deg + 1, size=rows)
    deg[rng.random(rows) < empty_frac] = 0
    for r, d in long_rows:
        deg[r] = min(d, cols)
    parts = [np.sort(rng.choice(cols, int(d), replace=False)) for d in deg]
    crow = np.zeros(rows + 1, dtype=np.int64)
    crow[1:] = np.cumsum(deg)
    col = np.concatenate(parts).astype(np.int64) if parts else np.zeros(0, np.int64)
    return crow, col


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def zero_start(n):
    return torch.zeros(n, dtype=torch.int32, device="cuda")


def assert_close(actual, expected_f64, dtype):
    tol = TOL[dtype]
    a = actual.float().cpu().double()
    e = torch.from_numpy(expected_f64)
    close = torch.isclose(a, e, atol=tol, rtol=tol)
    bad = int((~close).sum())
    assert bad == 0, f"{bad} mismatches, max abs err {float((a - e).abs().max()):.3e}"


def run_csr(spmm_npu, crow, col, vals, B, index_dtype=torch.int32):
    return spmm_npu.spmm_csr(dev(crow, index_dtype), dev(col, index_dtype), dev(vals), dev(B),
                             dev(O.make_start(crow, 40)))


@pytest.mark.parametrize("dtype", ["fp16", "fp32"])
@pytest.mark.parametrize("width", [16, 32, 48, 64, 128, 256, 512])
def test_spmm_csr_matches_oracle(spmm_npu, dtype, width):
    rng = np.random.default_rng(100 + width)
    crow, col = random_csr(rng, 300, 257, 40, long_rows=[(7, 200), (150, 257)])
    vals = rng.uniform(-1, 1, col.size).astype(NP_DT[dtype])
    B = rng.standard_normal((257, width)).astype(NP_DT[dtype])
    out = run_csr(spmm_npu, crow, col, vals, B)
    torch.cuda.synchronize()
    assert out.shape == (300, width) and out.dtype == dev(vals).dtype
    assert_close(out, O.spmm_f64(crow, col, vals, B), dtype)


def test_spmm_csr_fp16_width_1024(spmm_npu):
    rng = np.random.default_rng(7)
    crow, col = random_csr(rng, 120, 90, 30, long_rows=[(3, 90)])
    vals = rng.uniform(-1, 1, col.size).astype(np.float16)
    B = rng.standard_normal((90, 1024)).astype(np.float16)
    out = run_csr(spmm_npu, crow, col, vals, B)
    assert_close(out, O.spmm_f64(crow, col, vals, B), "fp16")


@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_spmm_csr_long_rows_cross_ranges(spmm_npu, index_dtype):
    """Rows of 1000..5000 nonzeros cross many fixed ranges (fix-up path)."""
    rng = np.random.default_rng(11)
    crow, col = random_csr(rng, 64, 6000, 5, long_rows=[(0, 1000), (5, 5000), (6, 257), (7, 513), (63, 2500)])
    vals = rng.uniform(-1, 1, col.size).astype(np.float32)
    B = rng.standard_normal((6000, 64)).astype(np.float32)
    out = run_csr(spmm_npu, crow, col, vals, B, index_dtype)
    assert_close(out, O.spmm_f64(crow, col, vals, B), "fp32")


def _gather_range(nnz):
    """R of the CSR gather path: the largest power of two in [16, 256] with
    2 * R * 12288 <= nnz (nnz alone decides it)."""
    r = 16
    while r < 256 and 2 * r * 12288 <= nnz:
        r *= 2
    return r


def _piece_rows(crow, R):
    """Row pointer whose rows are the pieces a row is summed in: the whole
    row when it holds at most short_max(R) nonzeros (R/2, or R when R <= 32)
    or stays inside one range of R positions; else cut at the range ends
    (multiples of R).  Also returns each piece's source row."""
    short = R if R <= 32 else R // 2
    bounds, owner = [0], []
    for r in range(crow.size - 1):
        a, b = int(crow[r]), int(crow[r + 1])
        cuts = [a]
        if b - a > short and b > (a // R + 1) * R:
            cuts += list(range((a // R + 1) * R, b, R))
        cuts.append(b)
        for lo, hi in zip(cuts[:-1], cuts[1:]):
            bounds.append(hi)
            owner.append(r)
    return np.asarray(bounds, np.int64), np.asarray(owner, np.int64)


@pytest.mark.parametrize("dtype", ["fp16", "fp32"])
@pytest.mark.parametrize("nnz_target", [300_000, 600_000, 900_000])
def test_csr_pieces_bitwise(spmm_npu, dtype, nnz_target):
    """Every row is the fp32 sum of its pieces (each a sequential FMA sum
    from zero, cut at multiples of R when the row is longer than
    short_max(R) and crosses a range end), added in order and rounded once.
    The pieces' own sums come from spmm_csr in fp32 on a matrix whose rows
    are the pieces (same positions, so the same R, and no piece is cut
    again); fp16 values and dense rows are exact in fp32.  R = 16, 32 and
    64, with rows around R and 2R and rows over several tiles."""
    rng = np.random.default_rng(nnz_target // 1000)
    K, width = 3000, 64
    rows = nnz_target // 10
    deg = rng.integers(0, 20, size=rows)
    deg[rng.random(rows) < 0.1] = 0
    # rows around R and 2R, and long rows over several ranges and work-groups
    R = _gather_range(int(deg.sum()) + 40_000)
    for r, d in [(5, R), (6, R + 1), (7, 2 * R - 1), (8, 2 * R), (9, 2 * R + 1), (100, 3 * R + 5), (101, 700),
                 (rows // 2, 2900), (rows - 3, 1500), (rows - 1, 2 * R)]:
        deg[r] = d
    deg[rng.integers(0, rows, size=400)] = rng.integers(R // 2, 3 * R, size=400)
    parts = [np.sort(rng.choice(K, int(d), replace=False)) for d in deg]
    crow = np.zeros(rows + 1, np.int64)
    crow[1:] = np.cumsum(deg)
    col = np.concatenate(parts).astype(np.int64)
    assert _gather_range(col.size) == R
    vals = rng.uniform(-1, 1, col.size).astype(NP_DT[dtype])
    B = rng.standard_normal((K, width)).astype(NP_DT[dtype])
    out = run_csr(spmm_npu, crow, col, vals, B).cpu().numpy()
    pcrow, owner = _piece_rows(crow, R)
    pieces = run_csr(spmm_npu, pcrow, col, vals.astype(np.float32), B.astype(np.float32)).cpu().numpy()
    expected = np.zeros((rows, width), np.float32)
    first = np.ones(rows, bool)
    for p, r in enumerate(owner):
        expected[r] = pieces[p] if first[r] else expected[r] + pieces[p]
        first[r] = False
    assert np.array_equal(out.view(np.uint16 if dtype == "fp16" else np.uint32),
                          expected.astype(NP_DT[dtype]).view(np.uint16 if dtype == "fp16" else np.uint32))


def _wide_row_matrix(rng, cols):
    """About 1.13M nonzeros (above the segment workers' 2^20 threshold): one
    row of 110k columns (its ranges sweep a chunk inside one column slab, so
    the workers deal that chunk in eighths), 45 rows of 20k uniform columns
    (slab buckets) and short rows."""
    rows = 4000
    deg = rng.integers(0, 61, size=rows)
    deg[10] = 110_000
    deg[100:145] = 20_000
    parts = [np.sort(rng.choice(cols, int(d), replace=False)) for d in deg]
    crow = np.zeros(rows + 1, dtype=np.int64)
    crow[1:] = np.cumsum(deg)
    return crow, np.concatenate(parts).astype(np.int64)


@pytest.mark.parametrize("dtype,width", [("fp16", 128), ("fp16", 256), ("fp32", 64), ("fp32", 128)])
def test_segment_workers_equal_tile_path_bitwise(spmm_npu, dtype, width):
    """Segments of wide long rows summed by gather_segments (dense operand of
    at most 128 MiB) give the same bits as gather_tiles summing them (the same
    columns in a dense operand padded past 128 MiB, which switches the workers
    off), and both match the fp64 oracle.  fp32 uses positive operands: a
    signed sum of 110k fp32 products cancels to values whose absolute error
    (same bits on both paths) exceeds the 1e-4 tolerance; without
    cancellation the tolerance holds for every element."""
    rng = np.random.default_rng(4242 + width)
    cols = 120_000
    crow, col = _wide_row_matrix(rng, cols)
    assert col.size >= 1 << 20
    if dtype == "fp16":
        vals = rng.uniform(-1, 1, col.size).astype(np.float16)
        B = rng.standard_normal((cols, width)).astype(np.float16)
    else:
        vals = rng.uniform(0.5, 1, col.size).astype(np.float32)
        B = (np.abs(rng.standard_normal((cols, width))) + 0.1).astype(np.float32)
    elem = 2 if dtype == "fp16" else 4
    assert cols * width * elem <= SEG_MAX_DENSE
    pad_rows = SEG_MAX_DENSE // (width * elem) + 1024
    out = run_csr(spmm_npu, crow, col, vals, B)
    Bpad = torch.zeros((pad_rows, width), dtype=dev(vals).dtype, device="cuda")
    Bpad[:cols] = dev(B)
    out_tiles = spmm_npu.spmm_csr(dev(crow, torch.int32), dev(col, torch.int32), dev(vals), Bpad,
                                  dev(O.make_start(crow, 40)))
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), out_tiles.cpu())
    assert_close(out, O.spmm_f64(crow, col, vals, B), dtype)


def test_segment_workers_width_invariant_bitwise(spmm_npu):
    """Across the segment gate: fp16 widths up to 512 use the segment
    work-groups (K = 120k rows, at most 128 MiB), 1024 does not, and
    C_1024[:, :n] == C_n bit for bit for every width n; int64 indices give
    the same bits as int32."""
    rng = np.random.default_rng(99)
    cols = 120_000
    crow, col = _wide_row_matrix(rng, cols)
    vals = rng.uniform(-1, 1, col.size).astype(np.float16)
    B = rng.standard_normal((cols, 1024)).astype(np.float16)
    full = run_csr(spmm_npu, crow, col, vals, B).cpu()
    for n in (16, 64, 128, 256, 512):
        part = run_csr(spmm_npu, crow, col, vals, np.ascontiguousarray(B[:, :n])).cpu()
        assert torch.equal(part, full[:, :n]), f"width {n} differs"
    Bn = np.ascontiguousarray(B[:, :128])
    assert torch.equal(run_csr(spmm_npu, crow, col, vals, Bn, torch.int64).cpu(), full[:, :128])
    assert_close(full[:, :128], O.spmm_f64(crow, col, vals, Bn), "fp16")


def test_segment_workers_invalid_and_unsorted_columns(spmm_npu):
    """Wide long rows with invalid column ids (at a row's first and last
    position and inside it) and a long row with unsorted columns: invalid
    ids contribute nothing, and the segment path matches the fp64 oracle and
    the tile path bit for bit."""
    rng = np.random.default_rng(7)
    cols = 120_000
    crow, col = _wide_row_matrix(rng, cols)
    r10 = slice(crow[10], crow[11])
    col[r10] = rng.permutation(col[r10])  # unsorted columns in the 110k row
    for r in (100, 101, 102):
        a, b = crow[r], crow[r + 1]
        col[a] = cols + 5          # first position invalid
        col[b - 1] = -3 if r == 101 else cols  # last position invalid
        col[a + (b - a) // 2] = cols + 17
    vals = rng.uniform(-1, 1, col.size).astype(np.float16)
    B = rng.standard_normal((cols, 128)).astype(np.float16)
    out = spmm_npu.spmm_csr(dev(crow, torch.int32), dev(col, torch.int32), dev(vals), dev(B),
                            dev(O.make_start(crow, 40)))
    Bpad = torch.zeros((SEG_MAX_DENSE // 256 + 1024, 128), dtype=torch.float16, device="cuda")
    Bpad[:cols] = dev(B)
    colp = np.where((col >= 0) & (col < cols), col, Bpad.shape[0] + 3)  # invalid for the padded operand too
    out_tiles = spmm_npu.spmm_csr(dev(crow, torch.int32), dev(colp, torch.int32), dev(vals), Bpad,
                                  dev(O.make_start(crow, 40)))
    assert torch.equal(out.cpu(), out_tiles.cpu())
    keep = (col >= 0) & (col < cols)
    assert_close(out, O.spmm_f64(crow, np.where(keep, col, 0), np.where(keep, vals, 0).astype(np.float16), B),
                 "fp16")


def _boundary_matrix(rng, cols, target_nnz=1_700_000):
    """Rows whose ends fall on range and tile starts (multiples of 128 and
    of 2048 positions: the ranges and 16-range tiles of gather_tiles at
    R = 128, which the library picks for 1.57M-3.1M nonzeros), runs of empty
    rows right at tile starts, long rows (over R/2 nonzeros) crossing one or
    several tiles, and short rows; columns spread over [0, cols), so the
    long rows' segments go to the segment work-groups."""
    R, span = 128, 2048
    degs, pos = [], 0
    while pos < target_nnz:
        kind = int(rng.integers(0, 6))
        if kind == 0:  # run on to the next tile start, then empty rows
            new = [span - pos % span] + [0] * int(rng.integers(1, 4))
        elif kind == 1:  # run on to the next range start
            new = [R - pos % R]
        elif kind == 2:  # a long row over several tiles
            new = [int(rng.integers(3 * span, 5 * span))]
        elif kind == 3:  # a long row of one or a few ranges
            new = [int(rng.integers(R // 2 + 1, 1000))]
        else:
            new = [int(x) for x in rng.integers(1, 40, size=8)]
        degs += new
        pos += sum(new)
    deg = np.array(degs, dtype=np.int64)
    crow = np.zeros(deg.size + 1, dtype=np.int64)
    crow[1:] = np.cumsum(deg)
    col = np.concatenate([np.sort(rng.choice(cols, int(d), replace=False)) for d in deg if d > 0])
    return crow, col.astype(np.int64)


def test_segment_path_row_boundaries_on_tile_starts(spmm_npu):
    """The segment path's classification records each tile's first row for
    gather_tiles: tiles starting exactly at a row's first position, after a
    run of empty rows, or inside a long row crossing several tiles all read
    the right row.  Compared bit for bit with the tile path (the same columns
    in a dense operand padded past 128 MiB) and with the fp64 oracle."""
    rng = np.random.default_rng(2048)
    cols = 120_000
    crow, col = _boundary_matrix(rng, cols)
    nnz = col.size
    assert 1_572_864 <= nnz < 3_145_728  # R = 128: 2 R 12288 <= nnz < 4 R 12288
    ends = crow[1:]
    deg = np.diff(crow)
    empty_at_tile = (deg == 0) & (crow[:-1] % 2048 == 0)
    assert int((ends % 2048 == 0).sum()) > 50 and int(empty_at_tile.sum()) > 50
    assert int(((crow[:-1] // 2048) + 2 <= (ends - 1) // 2048).sum()) > 20  # rows crossing 2+ tile starts
    vals = rng.uniform(-1, 1, nnz).astype(np.float16)
    B = rng.standard_normal((cols, 128)).astype(np.float16)
    out = run_csr(spmm_npu, crow, col, vals, B)
    Bpad = torch.zeros((SEG_MAX_DENSE // 256 + 1024, 128), dtype=torch.float16, device="cuda")
    Bpad[:cols] = dev(B)
    out_tiles = spmm_npu.spmm_csr(dev(crow, torch.int32), dev(col, torch.int32), dev(vals), Bpad,
                                  dev(O.make_start(crow, 40)))
    assert torch.equal(out.cpu(), out_tiles.cpu())
    assert_close(out, O.spmm_f64(crow, col, vals, B), "fp16")
    assert bool((out[torch.from_numpy(deg == 0).cuda()] == 0).all())


@pytest.mark.parametrize("seed,dtype,width", [(1, "fp16", 64), (2, "fp16", 128), (3, "fp16", 256),
                                              (4, "fp32", 32), (5, "fp32", 64), (6, "fp32", 128)])
def test_segment_path_random_power_law_bitwise(spmm_npu, seed, dtype, width):
    """Seeded power-law matrices above the segment threshold (degrees from a
    Pareto tail up to 40k, some empty rows), at widths that take each
    segment split (1, 2 and 3 work-groups per slab): the segment path equals
    the tile path bit for bit and the fp64 oracle within tolerance.  fp32
    uses positive operands (long signed fp32 sums cancel past 1e-4)."""
    rng = np.random.default_rng(5000 + seed)
    cols, rows = 60_000, 30_000
    deg = np.minimum((rng.pareto(1.3, rows) * 12).astype(np.int64), 40_000)
    deg[rng.random(rows) < 0.05] = 0
    deg = (deg * (1_300_000 / max(int(deg.sum()), 1))).astype(np.int64).clip(0, 40_000)
    crow = np.zeros(rows + 1, dtype=np.int64)
    crow[1:] = np.cumsum(deg)
    col = np.concatenate([np.sort(rng.choice(cols, int(d), replace=False)) for d in deg if d > 0]).astype(np.int64)
    assert col.size >= 1 << 20 and int(deg.max()) > 4096
    if dtype == "fp16":
        vals = rng.uniform(-1, 1, col.size).astype(np.float16)
        B = rng.standard_normal((cols, width)).astype(np.float16)
    else:
        vals = rng.uniform(0.5, 1, col.size).astype(np.float32)
        B = (np.abs(rng.standard_normal((cols, width))) + 0.1).astype(np.float32)
    elem = 2 if dtype == "fp16" else 4
    out = run_csr(spmm_npu, crow, col, vals, B)
    Bpad = torch.zeros((SEG_MAX_DENSE // (width * elem) + 1024, width), dtype=dev(vals).dtype, device="cuda")
    Bpad[:cols] = dev(B)
    out_tiles = spmm_npu.spmm_csr(dev(crow, torch.int32), dev(col, torch.int32), dev(vals), Bpad,
                                  dev(O.make_start(crow, 40)))
    assert torch.equal(out.cpu(), out_tiles.cpu())
    assert_close(out, O.spmm_f64(crow, col, vals, B), dtype)


def test_spmm_csr_edge_shapes(spmm_npu):
    rng = np.random.default_rng(3)
    B = rng.standard_normal((10, 16)).astype(np.float32)
    # all rows empty (nnz = 0): zeros
    crow = np.zeros(6, dtype=np.int64)
    out = run_csr(spmm_npu, crow, np.zeros(0, np.int64), np.zeros(0, np.float32), B)
    assert out.shape == (5, 16) and bool((out == 0).all())
    # zero rows
    out = run_csr(spmm_npu, np.zeros(1, np.int64), np.zeros(0, np.int64), np.zeros(0, np.float32), B)
    assert out.shape == (0, 16)
    # identity -> C == B exactly; single nnz per row -> exact scaled copy
    crow = np.arange(11, dtype=np.int64)
    col = np.arange(10, dtype=np.int64)
    out = run_csr(spmm_npu, crow, col, np.ones(10, np.float32), B)
    assert torch.equal(out.cpu(), torch.from_numpy(B))
    Bh = B.astype(np.float16)
    out = run_csr(spmm_npu, crow, col[::-1].copy(), np.full(10, 2.0, np.float16), Bh)
    assert torch.equal(out.cpu(), torch.from_numpy((2 * Bh[::-1]).astype(np.float16)))


def test_spmm_csr_matches_torch_sparse_cpu(spmm_npu):
    """Against the reference's own CPU path (cpu_reference, torch CSR sparse.mm)."""
    w = W.config1(scale=1 / 16)
    B = w.dense(128)
    out = run_csr(spmm_npu, w.crow, w.col, w.values, B)
    ref = O.cpu_reference(w.rows, w.cols, w.crow, w.col, w.values, B)
    close = torch.isclose(out.cpu(), ref, atol=1e-4, rtol=1e-4)
    assert bool(close.all())


@pytest.mark.parametrize("dtype", ["fp16", "fp32"])
def test_vector_path_width_invariant_bitwise(spmm_npu, dtype):
    """C_maxwidth[:, :n] == C_n bit for bit for every width n."""
    rng = np.random.default_rng(21)
    crow, col = random_csr(rng, 200, 300, 25, long_rows=[(1, 300), (100, 260)])
    vals = rng.uniform(-1, 1, col.size).astype(NP_DT[dtype])
    maxw = 1024 if dtype == "fp16" else 512
    B = rng.standard_normal((300, maxw)).astype(NP_DT[dtype])
    full = run_csr(spmm_npu, crow, col, vals, B).cpu()
    for n in (16, 32, 64, 128, 256, 512, 1024):
        if n > maxw:
            continue
        part = run_csr(spmm_npu, crow, col, vals, np.ascontiguousarray(B[:, :n])).cpu()
        assert torch.equal(part, full[:, :n]), f"width {n} differs"


@pytest.mark.parametrize("dtype,rows", [("fp16", 320), ("fp32", 320), ("fp16", 16 * 3000), ("fp32", 16 * 3000)])
def test_block_path_width_invariant_bitwise(spmm_npu, dtype, rows):
    """Mixed operator on a preprocess layout (block part + vector part):
    C_maxwidth[:, :n] == C_n bit for bit.  fp16 outputs of 256 columns or
    more take 8-column lane pieces in the block kernel, narrower ones 4, and
    128 columns take 8 when there are at least 2048 block windows (the
    3000-window matrices), so this also checks that an element's MFMA
    sequence does not depend on that choice (widths 192 and 272 end in
    partial column groups)."""
    rng = np.random.default_rng(23)
    if rows == 320:
        crow, col = random_csr(rng, 320, 400, 60, long_rows=[(3, 400), (170, 380)])
        cols = 400
    else:
        # Windows of 16 rows with every row on the same 12 columns near the
        # window's diagonal (block windows for the cost model), and a few
        # scattered rows for the vector part.
        cols = 4096
        deg = np.where(rng.random(rows) < 0.97, 12, 3)
        crow = np.zeros(rows + 1, np.int64)
        crow[1:] = np.cumsum(deg)
        parts = []
        for r in range(rows):
            if deg[r] == 12:
                base = (r // 16 * 7) % (cols - 12)
                parts.append(np.arange(base, base + 12))
            else:
                parts.append(np.sort(rng.choice(cols, 3, replace=False)))
        col = np.concatenate(parts).astype(np.int64)
    vals = rng.uniform(-1, 1, col.size).astype(NP_DT[dtype])
    maxw = 1024 if dtype == "fp16" else 512
    B = rng.standard_normal((cols, maxw)).astype(NP_DT[dtype])
    p = spmm_npu.preprocess(torch.from_numpy(crow), torch.from_numpy(col), torch.from_numpy(vals), rows, cols, 16)
    if rows > 320:
        assert p["crow_window_ptr"].numel() - 1 >= 2048
    i32 = torch.int32
    assert p["unique_col_ids"].numel() > 0 and p["vcol_indices"].numel() > 0

    def t(key, dtype=None):
        return p[key].to("cuda", dtype)

    def run(Bn):
        return spmm_npu.spmm_ascend_cube(
            t("crow_window_ptr", i32), t("unique_col_ids", i32), t("value"),
            t("vrow_window_ptr", i32), t("vcol_indices", i32), t("vvalue"), dev(Bn),
            dev(O.make_start(p["crow_window_ptr"].numpy(), 20)),
            dev(O.make_start(p["vrow_window_ptr"].numpy(), 40))).cpu()

    full = run(B)
    for n in (16, 64, 128, 192, 256, 272, 512, 1024):
        if n > maxw:
            continue
        part = run(np.ascontiguousarray(B[:, :n]))
        assert torch.equal(part, full[:, :n]), f"width {n} differs"


@pytest.mark.parametrize("dtype", ["fp16", "fp32"])
def test_block_window_order_on_a_banded_layout(spmm_npu, dtype):
    """The preprocess layout of a banded matrix (windows sorted by density,
    each spanning a narrow band of columns) with dense rows of 256 bytes or
    more takes the block windows' locality order.  The order changes only
    which work-group runs first, so the result equals a narrower run without
    the order (128-byte rows: fp16 N=64, fp32 N=32) bit for bit on its
    columns, and the restored rows match A @ B."""
    rng = np.random.default_rng(97)
    rows, band = 3000, 48
    deg = rng.integers(0, 2 * band, rows)
    deg[rng.random(rows) < 0.2] = 2  # some sparse rows, for the vector part
    parts = []
    for r in range(rows):
        lo, hi = max(0, r - band), min(rows, r + band)
        parts.append(np.sort(rng.choice(np.arange(lo, hi), min(int(deg[r]), hi - lo), replace=False)))
    crow = np.zeros(rows + 1, np.int64)
    crow[1:] = np.cumsum([p.size for p in parts])
    col = np.concatenate(parts).astype(np.int64)
    vals = rng.uniform(-1, 1, col.size).astype(NP_DT[dtype])
    B = rng.standard_normal((rows, 512)).astype(NP_DT[dtype])
    p = spmm_npu.preprocess(torch.from_numpy(crow), torch.from_numpy(col), torch.from_numpy(vals), rows, rows, 16)
    assert p["unique_col_ids"].numel() > 0 and p["vcol_indices"].numel() > 0
    i32 = torch.int32

    def run(Bn):
        return spmm_npu.spmm_ascend_cube(
            p["crow_window_ptr"].to("cuda", i32), p["unique_col_ids"].to("cuda", i32), p["value"].cuda(),
            p["vrow_window_ptr"].to("cuda", i32), p["vcol_indices"].to("cuda", i32), p["vvalue"].cuda(),
            dev(Bn), dev(O.make_start(p["crow_window_ptr"].numpy(), 20)),
            dev(O.make_start(p["vrow_window_ptr"].numpy(), 40)))

    narrow = 64 if dtype == "fp16" else 32  # dense rows under 256 bytes: no order
    base = run(np.ascontiguousarray(B[:, :narrow])).cpu()
    for n in (128, 256, 512):
        out = run(np.ascontiguousarray(B[:, :n]))
        assert torch.equal(out[:, :narrow].cpu(), base), f"width {n} differs from {narrow}"
        got = spmm_npu.restore_node_tensor(out, p["inv_permutation"].cuda())[:rows]
        assert_close(got, O.spmm_f64(crow, col, vals, B[:, :n]), dtype)


@pytest.mark.parametrize("dtype", ["fp16", "fp32"])
@pytest.mark.parametrize("width", [16, 128, 256])
def test_mixed_with_empty_block_part_equals_csr_bitwise(spmm_npu, dtype, width):
    rng = np.random.default_rng(31 + width)
    crow, col = random_csr(rng, 333, 400, 30, long_rows=[(2, 400), (200, 390)])
    vals = rng.uniform(-1, 1, col.size).astype(NP_DT[dtype])
    B = rng.standard_normal((400, width)).astype(NP_DT[dtype])
    ref = run_csr(spmm_npu, crow, col, vals, B)
    i32 = torch.int32
    mixed = spmm_npu.spmm_ascend_cube(
        zero_start(1), torch.zeros(0, dtype=i32, device="cuda"),
        torch.zeros(0, dtype=dev(vals).dtype, device="cuda"),
        dev(crow, i32), dev(col, i32), dev(vals), dev(B), zero_start(20),
        dev(O.make_start(crow, 40)))
    assert torch.equal(mixed[:333].cpu(), ref.cpu())


@pytest.mark.parametrize("windows", [16384, 16385])
def test_window_order_at_its_limit(spmm_npu, windows):
    """Block part of a banded matrix (csr_to_bcsr: every window local) plus
    a random vector part, so the gather kernel runs beside it: with 16384
    windows (the most the locality order takes) the sort's key and scatter
    loops make several rounds; with 16385 the windows keep their order.  The
    result matches A1 @ B + A2 @ B in fp64, and at N=128 (ordered when
    16384) equals N=64 (never ordered) bit for bit on its columns."""
    rng = np.random.default_rng(61)
    rows = 16 * windows
    deg = rng.integers(2, 9, rows)
    lo = np.maximum(np.arange(rows) - 8, 0)
    parts = [np.sort(rng.choice(np.arange(lo[r], min(rows, lo[r] + 16)), int(deg[r]), replace=False))
             for r in range(rows)]
    crow = np.zeros(rows + 1, np.int64)
    crow[1:] = np.cumsum([p.size for p in parts])
    col = np.concatenate(parts).astype(np.int64)
    vals = rng.uniform(-1, 1, col.size).astype(np.float16)
    vcrow, vcol = random_csr(rng, rows, rows, 2, empty_frac=0.5)
    vvals = rng.uniform(-1, 1, vcol.size).astype(np.float16)
    b = O.csr_to_bcsr(crow, col, vals, rows, rows, 16)
    assert b["crow_window_ptr"].size - 1 == windows
    B = rng.standard_normal((rows, 128)).astype(np.float16)
    i32 = torch.int32

    def run(n):
        return spmm_npu.spmm_ascend_cube(
            dev(b["crow_window_ptr"], i32), dev(b["unique_col_ids"], i32), dev(b["value"]),
            dev(vcrow, i32), dev(vcol, i32), dev(vvals), dev(np.ascontiguousarray(B[:, :n])),
            dev(O.make_start(b["crow_window_ptr"], 20)), dev(O.make_start(vcrow, 40)))

    out = run(128)
    assert_close(out[:rows], O.spmm_f64(crow, col, vals, B) + O.spmm_f64(vcrow, vcol, vvals, B), "fp16")
    assert torch.equal(out[:, :64].cpu(), run(64).cpu())


def _evened_ranges_per_tile(nnz, cus, full=16):
    """Ranges per tile the launcher takes for a mixed op's vector part without
    a column split: the count in [full / 2, full] that gives the busiest CU
    the fewest ranges, when that is at least 5% fewer than with `full`."""
    nranges = -(-nnz // _gather_range(nnz))
    units = lambda r: -(-(-(-nranges // r)) // cus) * r
    best = min(range(full, full // 2 - 1, -1), key=lambda r: (units(r), -r))
    return best if units(best) * 20 <= units(full) * 19 else full


@pytest.mark.parametrize("dtype,width", [("fp16", 128), ("fp32", 64)])
def test_mixed_vector_part_tiles_evened_over_cus(spmm_npu, dtype, width):
    """A vector part of about 450k nonzeros (R = 32, 256-byte dense rows): on
    a 256-CU MI355X the launcher takes 14 ranges per tile instead of 16 so
    that no CU holds more than 56 ranges (64 with 16).  Rows of windows without blocks are
    the vector part's own sums, so they equal spmm_csr on the vector part
    (16 ranges per tile) bit for bit; the whole result matches
    A1 @ B + A2 @ B in fp64."""
    rng = np.random.default_rng(71)
    rows = 16384
    # Block part: 16x16 banded blocks in the first 64 windows only.
    brows = 64 * 16
    parts = [np.sort(rng.choice(np.arange(max(0, r - 24), min(rows, r + 24)), 12, replace=False))
             for r in range(brows)]
    crow = np.zeros(rows + 1, np.int64)
    crow[1:brows + 1] = np.cumsum([p.size for p in parts])
    crow[brows + 1:] = crow[brows]
    col = np.concatenate(parts).astype(np.int64)
    vals = rng.uniform(-1, 1, col.size).astype(NP_DT[dtype])
    vcrow, vcol = random_csr(rng, rows, rows, 69)
    vvals = rng.uniform(-1, 1, vcol.size).astype(NP_DT[dtype])
    nnz = int(vcrow[-1])
    assert _gather_range(nnz) == 32
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if cus == 256:
        assert _evened_ranges_per_tile(nnz, cus) == 14
    b = O.csr_to_bcsr(crow, col, vals, rows, rows, 16)
    B = rng.standard_normal((rows, width)).astype(NP_DT[dtype])
    i32 = torch.int32
    out = spmm_npu.spmm_ascend_cube(
        dev(b["crow_window_ptr"], i32), dev(b["unique_col_ids"], i32), dev(b["value"]),
        dev(vcrow, i32), dev(vcol, i32), dev(vvals), dev(B),
        dev(O.make_start(b["crow_window_ptr"], 20)), dev(O.make_start(vcrow, 40)))
    ref = run_csr(spmm_npu, vcrow, vcol, vvals, B)
    assert torch.equal(out[brows:rows].cpu(), ref[brows:].cpu())
    assert_close(out[:rows], O.spmm_f64(crow, col, vals, B) + O.spmm_f64(vcrow, vcol, vvals, B), dtype)


@pytest.mark.parametrize("dtype", ["fp16", "fp32"])
@pytest.mark.parametrize("width", [16, 64, 128, 192, 512])
def test_block_part_from_bcsr(spmm_npu, dtype, width):
    """Pure block part (csr_to_bcsr layout, empty vector part) vs fp64."""
    rng = np.random.default_rng(41 + width)
    crow, col = random_csr(rng, 250, 300, 60, long_rows=[(4, 300)])
    vals = rng.uniform(-1, 1, col.size).astype(NP_DT[dtype])
    B = rng.standard_normal((300, width)).astype(NP_DT[dtype])
    b = O.csr_to_bcsr(crow, col, vals, 250, 300, 16)
    i32 = torch.int32
    for op in (spmm_npu.spmm_ascend_cube, spmm_npu.spmm_ascend_cube_aic_without_pipeline):
        out = op(dev(b["crow_window_ptr"], i32), dev(b["unique_col_ids"], i32), dev(b["value"]),
                 zero_start(1), torch.zeros(0, dtype=i32, device="cuda"),
                 torch.zeros(0, dtype=dev(vals).dtype, device="cuda"), dev(B),
                 dev(O.make_start(b["crow_window_ptr"], 20)), zero_start(40))
        assert out.shape == (16 * 16, width)
        assert_close(out[:250], O.spmm_f64(crow, col, vals, B), dtype)
        assert bool((out[250:] == 0).all())


@pytest.mark.parametrize("dtype", ["fp16", "fp32"])
def test_mixed_block_level_split(spmm_npu, dtype):
    """block_level_split layout: BSR over all windows + CSR residual, original row order."""
    rng = np.random.default_rng(51)
    crow, col = random_csr(rng, 500, 500, 40, long_rows=[(9, 480)])
    vals = rng.uniform(-1, 1, col.size).astype(NP_DT[dtype])
    B = rng.standard_normal((500, 128)).astype(NP_DT[dtype])
    h = O.block_level_split(crow, col, vals, 500, 500, (222.0 / 190.0) * 0.5, 16)
    assert h["vcol_indices"].size > 0 and h["unique_col_ids"].size > 0
    i32 = torch.int32
    out = spmm_npu.spmm_ascend_cube(
        dev(h["crow_window_ptr"], i32), dev(h["unique_col_ids"], i32), dev(h["value"]),
        dev(h["vrow_window_ptr"], i32), dev(h["vcol_indices"], i32), dev(h["vvalue"]), dev(B),
        dev(O.make_start(h["crow_window_ptr"], 20)), dev(O.make_start(h["vrow_window_ptr"], 40)))
    assert_close(out[:500], O.spmm_f64(crow, col, vals, B), dtype)


@pytest.mark.parametrize("graph_layout", [False, True])
def test_mixed_preprocess_layout_unpermuted(spmm_npu, graph_layout):
    """preprocess layout: packed rows; restore with inv_permutation before comparing
    (the reference's task-mapping test omits this step, see its correctness.py:179-182)."""
    rng = np.random.default_rng(61)
    w = W.config4(scale=0.01)
    B = w.dense(64)
    p = O.preprocess(w.crow, w.col, w.values, w.rows, w.cols, 16, graph_layout)
    i32 = torch.int32
    ccol = p["renumbered_unique_col_ids"] if graph_layout else p["unique_col_ids"]
    vcol = p["renumbered_vcol_indices"] if graph_layout else p["vcol_indices"]
    dense = dev(B)
    if graph_layout:
        dense = spmm_npu.pack_node_tensor(dense, torch.from_numpy(p["inv_permutation"]),
                                          int(p["packed_rows"][0]))
    out = spmm_npu.spmm_ascend_cube(
        dev(p["crow_window_ptr"], i32), dev(ccol, i32), dev(p["value"]),
        dev(p["vrow_window_ptr"], i32), dev(vcol, i32), dev(p["vvalue"]), dense,
        dev(O.make_start(p["crow_window_ptr"], 20)), dev(O.make_start(p["vrow_window_ptr"], 40)))
    restored = spmm_npu.restore_node_tensor(out, torch.from_numpy(p["inv_permutation"]))
    assert restored.shape == (w.rows, 64)
    assert_close(restored, O.spmm_f64(w.crow, w.col, w.values, B), "fp16")
    del rng


def test_results_are_deterministic(spmm_npu):
    w = W.config2(scale=0.05)
    B = w.dense(128)
    a = run_csr(spmm_npu, w.crow, w.col, w.values, B).cpu()
    b = run_csr(spmm_npu, w.crow, w.col, w.values, B).cpu()
    assert torch.equal(a, b)


def test_aliases_match_base_ops(spmm_npu):
    rng = np.random.default_rng(71)
    crow, col = random_csr(rng, 100, 100, 20)
    vals = rng.uniform(-1, 1, col.size).astype(np.float16)
    B = rng.standard_normal((100, 64)).astype(np.float16)
    args = (dev(crow, torch.int32), dev(col, torch.int32), dev(vals), dev(B),
            dev(O.make_start(crow, 40)))
    assert torch.equal(spmm_npu.spmm_csr(*args), spmm_npu.spmm_csr_aiv_mb_batch(*args))
    i32 = torch.int32
    margs = (zero_start(1), torch.zeros(0, dtype=i32, device="cuda"),
             torch.zeros(0, dtype=torch.float16, device="cuda"), args[0], args[1], args[2],
             args[3], zero_start(20), args[4])
    assert torch.equal(spmm_npu.spmm_ascend_cube(*margs), spmm_npu.spmm_ascend_cube_aiv_mb(*margs))


def test_contract_errors(spmm_npu):
    i32 = torch.int32
    crow = dev(np.array([0, 1], np.int64), i32)
    col = dev(np.array([0], np.int64), i32)
    v = torch.ones(1, dtype=torch.float16, device="cuda")
    st = zero_start(40)
    with pytest.raises(RuntimeError, match="feature width divisible by 16"):
        spmm_npu.spmm_csr(crow, col, v, torch.ones(2, 24, dtype=torch.float16, device="cuda"), st)
    with pytest.raises(RuntimeError, match="0 < feature width <= 1024 for FP16"):
        spmm_npu.spmm_csr(crow, col, v, torch.ones(2, 1040, dtype=torch.float16, device="cuda"), st)
    with pytest.raises(RuntimeError, match="0 < feature width <= 512 for FP32"):
        spmm_npu.spmm_csr(crow, col, v.float(), torch.ones(2, 520, device="cuda"), st)
    with pytest.raises(RuntimeError, match="must have the same dtype as dense"):
        spmm_npu.spmm_csr(crow, col, v, torch.ones(2, 16, device="cuda"), st)
    with pytest.raises(RuntimeError, match="col and value must be same size"):
        spmm_npu.spmm_csr(crow, col, torch.ones(2, dtype=torch.float16, device="cuda"),
                          torch.ones(2, 16, dtype=torch.float16, device="cuda"), st)
    with pytest.raises(RuntimeError, match="must be a GPU tensor"):
        spmm_npu.spmm_csr(crow.cpu(), col, v, torch.ones(2, 16, dtype=torch.float16, device="cuda"), st)
    # fp32 spmm_csr accepts widths divisible by 8 (extension/custom_op.cpp:78)
    out = spmm_npu.spmm_csr(crow, col, v.float(), torch.ones(2, 24, device="cuda"), st)
    assert torch.equal(out.cpu(), torch.ones(1, 24))


def test_out_of_range_columns_contribute_zero(spmm_npu):
    """Column ids outside dense are skipped by the kernels (no out-of-bounds read)."""
    crow = np.array([0, 2, 3], np.int64)
    col = np.array([1, 99, 0], np.int64)
    vals = np.array([1.0, 5.0, 2.0], np.float32)
    B = np.arange(32, dtype=np.float32).reshape(2, 16)
    out = run_csr(spmm_npu, crow, col, vals, B).cpu().numpy()
    np.testing.assert_array_equal(out, np.stack([B[1], 2 * B[0]]))


def test_pack_restore_match_oracle(spmm_npu):
    rng = np.random.default_rng(81)
    x = rng.standard_normal((50, 24)).astype(np.float32)
    inv = rng.permutation(64)[:50].astype(np.int64)
    packed = spmm_npu.pack_node_tensor(dev(x), torch.from_numpy(inv), 64)
    np.testing.assert_array_equal(packed.cpu().numpy(), O.pack_node_tensor(x, inv, 64))
    back = spmm_npu.restore_node_tensor(packed, torch.from_numpy(inv))
    np.testing.assert_array_equal(back.cpu().numpy(), x)
    # odd row size (3 bytes per row) takes the byte path
    xb = rng.integers(0, 255, size=(50, 3)).astype(np.uint8)
    pb = spmm_npu.pack_node_tensor(dev(xb), torch.from_numpy(inv))
    np.testing.assert_array_equal(pb.cpu().numpy(), O.pack_node_tensor(xb, inv))
    with pytest.raises(ValueError, match="packed_rows is smaller"):
        spmm_npu.pack_node_tensor(dev(x), torch.from_numpy(inv), 10)
    with pytest.raises(ValueError, match="invalid packed node id"):
        spmm_npu.restore_node_tensor(packed[:10], torch.from_numpy(inv))


def test_config2_full_size_matches_oracle(spmm_npu):
    """Benchmark configuration 2 at full size (power-law, fp16, N=128) vs the fp64 oracle."""
    w = W.config2()
    B = w.dense(128)
    out = run_csr(spmm_npu, w.crow, w.col, w.values, B)
    assert_close(out, O.spmm_f64(w.crow, w.col, w.values, B), "fp16")


# ------------------------------------------------------------- spmm_cube

@pytest.mark.parametrize("dtype", ["fp16", "fp32"])
@pytest.mark.parametrize("width", [16, 128, 512])
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_spmm_cube_matches_oracle(spmm_npu, dtype, width, index_dtype):
    rng = np.random.default_rng(40 + width)
    n, K = 300, 257
    crow, col = random_csr(rng, n, K, 20, long_rows=[(5, 200), (17, 250)])
    val = rng.uniform(-1, 1, col.size).astype(NP_DT[dtype])
    B = rng.standard_normal((K, width)).astype(NP_DT[dtype])
    rp, enc, v = O.cube_encode(crow, col, val, n)
    out = spmm_npu.spmm_cube(dev(rp, index_dtype), dev(enc, index_dtype), dev(v), dev(B), zero_start(20))
    assert out.shape == (16 * (rp.size - 1), width) and out.dtype == dev(B).dtype
    ref = O.spmm_cube_f64(rp, enc, v, B)
    tol = TOL[dtype]
    np.testing.assert_allclose(out.double().cpu().numpy(), ref, atol=tol, rtol=tol)


@pytest.mark.parametrize("dtype", ["fp16", "fp32"])
def test_spmm_cube_equals_bcsr_block_part_bitwise(spmm_npu, dtype):
    """Encoded runs are the BCSR(16x1) blocks of csr_to_bcsr in the same
    order, so spmm_cube and spmm_ascend_cube on the BCSR run the same MFMA
    sequence."""
    rng = np.random.default_rng(9)
    n, K, width = 400, 600, 64
    crow, col = random_csr(rng, n, K, 30)
    val = rng.uniform(-1, 1, col.size).astype(NP_DT[dtype])
    B = rng.standard_normal((K, width)).astype(NP_DT[dtype])
    rp, enc, v = O.cube_encode(crow, col, val, n)
    cube = spmm_npu.spmm_cube(dev(rp, torch.int32), dev(enc, torch.int32), dev(v), dev(B), zero_start(20))
    b = O.csr_to_bcsr(crow, col, val, n, K, 16)
    i32 = torch.int32
    block = spmm_npu.spmm_ascend_cube(dev(b["crow_window_ptr"], i32), dev(b["unique_col_ids"], i32),
                                      dev(b["value"]), dev(np.zeros(1, np.int32)),
                                      torch.zeros(0, dtype=i32, device="cuda"),
                                      torch.zeros(0, dtype=dev(v).dtype, device="cuda"), dev(B),
                                      zero_start(20), zero_start(40))
    assert torch.equal(cube, block)


def test_spmm_cube_runs_overwrites_and_edges(spmm_npu):
    rowptr = np.array([0, 6, 6, 7], np.int64)
    col = np.array([(2 << 4) | 0, (2 << 4) | 0, (2 << 4) | 3, (1 << 4) | 1, (2 << 4) | 1, (9 << 4) | 2,
                    (0 << 4) | 15], np.int64)
    val = np.array([1.0, 5.0, 4.0, 2.0, 7.0, 100.0, 3.0], np.float32)
    B = np.tile(np.array([[1.0], [2.0], [3.0], [4.0]], np.float32), (1, 16))
    out = spmm_npu.spmm_cube(dev(rowptr), dev(col), dev(val), dev(B), zero_start(20))
    np.testing.assert_array_equal(out.cpu().numpy(), O.spmm_cube_f64(rowptr, col, val, B).astype(np.float32))
    # no nonzeros: all windows zero
    empty = spmm_npu.spmm_cube(dev(np.zeros(4, np.int64)), dev(np.zeros(0, np.int64)),
                               dev(np.zeros(0, np.float16)), dev(np.ones((5, 32), np.float16)), zero_start(20))
    assert empty.shape == (48, 32) and not empty.any()


def test_spmm_cube_contract_errors(spmm_npu):
    rp = dev(np.array([0, 1], np.int32))
    c = dev(np.array([0], np.int32))
    with pytest.raises(RuntimeError, match="spmm_cube requires feature width divisible by 16"):
        spmm_npu.spmm_cube(rp, c, dev(np.ones(1, np.float32)), dev(np.ones((2, 8), np.float32)), zero_start(20))
    with pytest.raises(RuntimeError, match="col and value must be same size"):
        spmm_npu.spmm_cube(rp, c, dev(np.ones(2, np.float16)), dev(np.ones((2, 16), np.float16)), zero_start(20))


def test_spmm_csr_sparse_rows_with_long_empty_gaps(spmm_npu):
    """Few nonzeros over many rows: a tile's rows run far past 256 (the
    marking walk takes several chunks), leading and trailing empty rows, and
    long runs of empty rows between nonzero rows are written as zeros."""
    rng = np.random.default_rng(71)
    rows, K = 200000, 5000
    nonempty = np.sort(rng.choice(np.arange(1000, rows - 1000), 2500, replace=False))
    deg = np.zeros(rows, np.int64)
    deg[nonempty] = rng.integers(1, 4, nonempty.size)
    deg[nonempty[::97]] = 40  # a few rows longer than half a range
    crow = np.zeros(rows + 1, np.int64)
    crow[1:] = np.cumsum(deg)
    col = np.concatenate([np.sort(rng.choice(K, d, replace=False)) for d in deg if d]).astype(np.int64)
    for dtype in ("fp16", "fp32"):
        vals = rng.uniform(-1, 1, col.size).astype(NP_DT[dtype])
        B = rng.standard_normal((K, 32)).astype(NP_DT[dtype])
        out = run_csr(spmm_npu, crow, col, vals, B)
        assert_close(out, O.spmm_f64(crow, col, vals, B), dtype)
        assert bool((out[torch.from_numpy(deg == 0).cuda()] == 0).all())


def test_invalid_columns_and_nonfinite_values_stay_in_their_rows(spmm_npu):
    """Negative and >= K column ids contribute nothing, even with an Inf
    value; Inf values of valid columns reach only their own rows (the masked
    edge positions of a range never leak into a neighbouring row)."""
    rng = np.random.default_rng(72)
    crow, col = random_csr(rng, 3000, 400, 12, long_rows=[(10, 300), (2000, 390)])
    vals = rng.uniform(-1, 1, col.size).astype(np.float32)
    bad = rng.choice(col.size, 60, replace=False)
    col[bad[:30]] = -5
    col[bad[30:]] = 400 + 7
    vals[bad] = np.inf  # invalid columns: ignored even though their value is Inf
    hot = rng.choice(np.setdiff1d(np.arange(col.size), bad), 25, replace=False)
    vals[hot] = np.inf
    B = (rng.standard_normal((400, 64)) + 8.0).astype(np.float32)  # no zeros: Inf * x stays +-Inf
    keep = (col >= 0) & (col < 400)
    expected = O.spmm_f64(crow, np.where(keep, col, 0), np.where(keep, vals, 0.0), B)
    for index_dtype in (torch.int32, torch.int64):
        out = run_csr(spmm_npu, crow, col, vals, B, index_dtype).cpu().double()
        e = torch.from_numpy(expected)
        finite = torch.isfinite(e)
        assert torch.equal(torch.isfinite(out), finite)
        assert torch.equal(torch.isnan(out), torch.isnan(e))
        assert bool(torch.isclose(out[finite], e[finite], atol=1e-4, rtol=1e-4).all())


@pytest.mark.parametrize("dtype,N", [("fp32", 512), ("fp16", 1024)])
def test_dense_operand_beyond_32bit_extent(spmm_npu, dtype, N):
    """A dense operand larger than 4 GB (K = 2.2M rows; fp32 N = 512 or fp16
    N = 1024) takes the gather's 64-bit global-load path; columns in the
    last rows are read."""
    K, rows = 2_200_000, 600
    tdt = torch.float32 if dtype == "fp32" else torch.float16
    rng = np.random.default_rng(73)
    B = torch.empty((K, N), dtype=tdt, device="cuda")
    B.normal_(generator=torch.Generator(device="cuda").manual_seed(5))
    assert K * N * B.element_size() > 0xFFFFF000
    deg = rng.integers(0, 20, rows)
    crow = np.zeros(rows + 1, np.int64)
    crow[1:] = np.cumsum(deg)
    col = np.concatenate([np.sort(rng.choice(K, d, replace=False)) for d in deg]).astype(np.int64)
    col[:50] = np.sort(rng.choice(np.arange(K - 1000, K), 50, replace=False))  # the far end of B
    col[60] = K + 1  # invalid
    vals = rng.uniform(-1, 1, col.size).astype(NP_DT[dtype])
    out = spmm_npu.spmm_csr(dev(crow, torch.int32), dev(col, torch.int32), dev(vals), B,
                            dev(O.make_start(crow, 40)))
    used = np.unique(col[col < K])
    Bsub = B[torch.from_numpy(used).cuda()].cpu().numpy()
    remap = np.where(col < K, np.searchsorted(used, np.minimum(col, K - 1)), used.size + 5)
    assert_close(out, O.spmm_f64(crow, remap, vals, Bsub), dtype)
    del B
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dtype,N", [("fp32", 512), ("fp16", 1024)])
def test_block_part_dense_beyond_32bit_extent(spmm_npu, dtype, N):
    """The block kernel on a dense operand larger than 4 GB (K = 2.2M rows)
    takes its 64-bit global-load path (fp32: 4-column pieces; fp16 at
    N = 1024: 8-column pieces); blocks in the last rows of B and an invalid
    block column (contributes zero) are included."""
    K, rows = 2_200_000, 200
    tdt = torch.float32 if dtype == "fp32" else torch.float16
    rng = np.random.default_rng(79)
    B = torch.empty((K, N), dtype=tdt, device="cuda")
    B.normal_(generator=torch.Generator(device="cuda").manual_seed(6))
    assert K * N * B.element_size() > 0xFFFFF000
    deg = rng.integers(0, 40, rows)
    crow = np.zeros(rows + 1, np.int64)
    crow[1:] = np.cumsum(deg)
    col = np.concatenate([np.sort(rng.choice(K, d, replace=False)) for d in deg]).astype(np.int64)
    col[: deg[0]] = np.sort(rng.choice(np.arange(K - 500, K), deg[0], replace=False))  # the far end of B
    vals = rng.uniform(-1, 1, col.size).astype(NP_DT[dtype])
    b = O.csr_to_bcsr(crow, col, vals, rows, K, 16)
    ucol = b["unique_col_ids"].copy()
    ucol[3] = K + 7  # one invalid block column
    i32 = torch.int32
    out = spmm_npu.spmm_ascend_cube(
        dev(b["crow_window_ptr"], i32), dev(ucol, i32), dev(b["value"]), zero_start(1),
        torch.zeros(0, dtype=i32, device="cuda"), torch.zeros(0, dtype=tdt, device="cuda"), B,
        dev(O.make_start(b["crow_window_ptr"], 20)), zero_start(40))
    # Expected: the blocks as a CSR over the used dense rows (the invalid block's
    # 16 values dropped), in fp64.
    nwin = b["crow_window_ptr"].size - 1
    bcol = ucol.astype(np.int64)
    blk_rows, blk_cols, blk_vals = [], [], []
    for s in range(nwin):
        for k in range(int(b["crow_window_ptr"][s]), int(b["crow_window_ptr"][s + 1])):
            if bcol[k] >= K:
                continue
            for r in range(16):
                blk_rows.append(16 * s + r)
                blk_cols.append(bcol[k])
                blk_vals.append(b["value"][16 * k + r])
    blk_rows = np.asarray(blk_rows)
    order = np.lexsort((np.asarray(blk_cols), blk_rows))
    ecrow = np.zeros(16 * nwin + 1, np.int64)
    np.add.at(ecrow, blk_rows + 1, 1)
    ecrow = np.cumsum(ecrow)
    ecol = np.asarray(blk_cols)[order]
    evals = np.asarray(blk_vals)[order]
    used = np.unique(ecol)
    Bsub = B[torch.from_numpy(used).cuda()].cpu().numpy()
    assert_close(out, O.spmm_f64(ecrow, np.searchsorted(used, ecol), evals, Bsub), dtype)
    del B
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dtype,width", [("fp16", 64), ("fp16", 512), ("fp32", 64), ("fp32", 512)])
def test_windows_longer_than_the_block_chunk(spmm_npu, dtype, width):
    """Windows of thousands of 16x1 blocks are cut into chunks summed by
    separate work-groups (overflow ranges) and added in order by the combine
    pass, which also adds the vector part of rows that have one."""
    rng = np.random.default_rng(91 + width)
    rows, K = 80, 20000
    deg = np.full(rows, 3)
    deg[16:32] = 1000          # window 1: ~11k distinct columns -> several chunks
    deg[48:56] = 2500          # window 3: half its rows long
    parts = [np.sort(rng.choice(K, d, replace=False)) for d in deg]
    crow = np.zeros(rows + 1, np.int64)
    crow[1:] = np.cumsum(deg)
    col = np.concatenate(parts).astype(np.int64)
    vals = rng.uniform(-1, 1, col.size).astype(NP_DT[dtype])
    B = rng.standard_normal((K, width)).astype(NP_DT[dtype])
    expected = O.spmm_f64(crow, col, vals, B)
    i32 = torch.int32
    b = O.csr_to_bcsr(crow, col, vals, rows, K, 16)
    nblk = np.diff(b["crow_window_ptr"])
    assert nblk.max() > 4096  # longer than any chunk for this block count
    bops = (dev(b["crow_window_ptr"], i32), dev(b["unique_col_ids"], i32), dev(b["value"]))
    bstart = dev(O.make_start(b["crow_window_ptr"], 20))
    out = spmm_npu.spmm_ascend_cube(*bops, zero_start(1), torch.zeros(0, dtype=i32, device="cuda"),
                                    torch.zeros(0, dtype=dev(vals).dtype, device="cuda"), dev(B), bstart,
                                    zero_start(40))
    assert_close(out[:rows], expected, dtype)
    # Without a vector part no gather pass runs, and each long window's own
    # work-group sums its overflow segments; with one (a single nonzero in
    # row 0) the gather's post pass zeroes the window counters and overflow
    # work-groups take the segments.  The long windows' rows agree bit for bit.
    vrow = np.ones(rows + 1, np.int64)
    vrow[0] = 0
    out_v = spmm_npu.spmm_ascend_cube(*bops, dev(vrow, i32), torch.zeros(1, dtype=i32, device="cuda"),
                                      dev(np.ones(1, NP_DT[dtype])), dev(B), bstart, dev(O.make_start(vrow, 40)))
    assert torch.equal(out_v[16:rows], out[16:rows])
    assert not torch.equal(out_v[0], out[0])
    # the same windows with part of every row in the vector part (vpart handed to the combine)
    h = O.block_level_split(crow, col, vals, rows, K, 1.0, 16)
    assert h["vcol_indices"].size > 0 and np.diff(h["crow_window_ptr"]).max() > 4096
    out = spmm_npu.spmm_ascend_cube(
        dev(h["crow_window_ptr"], i32), dev(h["unique_col_ids"], i32), dev(h["value"]),
        dev(h["vrow_window_ptr"], i32), dev(h["vcol_indices"], i32), dev(h["vvalue"]), dev(B),
        dev(O.make_start(h["crow_window_ptr"], 20)), dev(O.make_start(h["vrow_window_ptr"], 40)))
    assert_close(out[:rows], expected, dtype)


@pytest.mark.parametrize("dtype", ["fp32", "fp16"])
def test_column_passes_equal_single_pass_bitwise(spmm_npu, dtype):
    """A dense operand of more than 512 MiB (K = 600k rows: fp32 N = 512, or
    fp16 N = 1024) is swept in column passes (pass_width: 128 fp32 / 256 fp16
    columns).  Each slab of the result equals a one-pass call on that slab
    of the dense operand bit for bit, for spmm_csr and spmm_ascend_cube (a
    block_level_split layout, block and vector parts), and matches fp64."""
    K, rows = 600_000, 2048
    N = 512 if dtype == "fp32" else 1024
    w = 128 if dtype == "fp32" else 256
    tdt = torch.float32 if dtype == "fp32" else torch.float16
    rng = np.random.default_rng(97)
    B = torch.empty((K, N), dtype=tdt, device="cuda")
    B.normal_(generator=torch.Generator(device="cuda").manual_seed(9))
    crow, col = random_csr(rng, rows, K, 60, long_rows=[(5, 3000), (1000, 700)])
    vals = rng.uniform(-1, 1, col.size).astype(NP_DT[dtype])
    i32 = torch.int32
    start = dev(O.make_start(crow, 40))
    full = spmm_npu.spmm_csr(dev(crow, i32), dev(col, i32), dev(vals), B, start)
    h = O.block_level_split(crow, col, vals, rows, K, 0.5, 16)
    mops = (dev(h["crow_window_ptr"], i32), dev(h["unique_col_ids"], i32), dev(h["value"]),
            dev(h["vrow_window_ptr"], i32), dev(h["vcol_indices"], i32), dev(h["vvalue"]))
    mstarts = (dev(O.make_start(h["crow_window_ptr"], 20)), dev(O.make_start(h["vrow_window_ptr"], 40)))
    assert h["unique_col_ids"].size > 0 and h["vcol_indices"].size > 0
    mfull = spmm_npu.spmm_ascend_cube(*mops, B, *mstarts)
    for c in (0, N - w):
        slab = B[:, c:c + w].contiguous()
        one = spmm_npu.spmm_csr(dev(crow, i32), dev(col, i32), dev(vals), slab, start)
        assert torch.equal(full[:, c:c + w], one), f"spmm_csr slab {c}"
        mone = spmm_npu.spmm_ascend_cube(*mops, slab, *mstarts)
        assert torch.equal(mfull[:, c:c + w], mone), f"spmm_ascend_cube slab {c}"
        del slab
    used = np.unique(col)
    Bsub = B[:, :64][torch.from_numpy(used).cuda()].cpu().numpy()
    expected = O.spmm_f64(crow, np.searchsorted(used, col), vals, Bsub)
    assert_close(full[:, :64], expected, dtype)
    assert_close(mfull[:rows, :64], expected, dtype)
    del B
    torch.cuda.empty_cache()
