"""Seeded medium-scale GPU parity sweep: matrices of a few thousand to tens
of thousands of rows (several gather ranges per long row, many tiles, block
windows with overflow chunks, window orders), drawn from six structure
families (one rectangular), each checked through every operator path against the oracle:

* spmm_csr against the fp64 product (the reference's tolerance,
  tests/task_mapping/correctness.py:140-143) and bitwise against a
  narrower run on the shared columns (the vector path's width invariance,
  tests/aic_aiv_ablation/bitwise_correctness.py:138-175);
* csr_to_bcsr, block_level_split and preprocess (graph layout on and off,
  on for square matrices only) bit for bit against the oracle's layouts,
  with int32 indices on even seeds and int64 on odd;
* spmm_ascend_cube on each of those layouts against the fp64 product,
  after restore_node_tensor where rows are packed, and the legacy
  spmm_cube on the window encoding of the matrix;
* PackedGraph (graph layout, square families) forward against A x and
  backward against A^T g, at the same bound.

The bound is the reference's atol = rtol (2e-2 fp16, 1e-4 fp32) for every
row of at most SLACK_DEGREE (1024) nonzeros.  Rows longer than that (the
hub rows, up to tens of thousands of nonzeros) also get the rounding that
fp32 accumulation of d products p_k admits in any order,
4 u sqrt(d) sqrt(sum p_k^2), u = 2^-24 (about ten standard deviations of
recursive summation's error, whose size is u n sigma for n terms of rms
sigma): there no fp32 summation order stays inside 1e-4 where the result
cancels to near zero (a sequential fp32 CPU sum of those rows misses it
too).  For d <= 1024 and the U(-1, 1) x N(0, 1) products used here, that
error is about 2.4e-8 d rms, under a quarter of the fp32 tolerance, so
ordinary rows are held to the plain bound.
"""

import numpy as np
import pytest
import torch

import oracle as O
from test_gpu_autograd import transpose_csr
from test_gpu_preprocess import assert_same

pytestmark = pytest.mark.gpu

TOL = {np.float16: 2e-2, np.float32: 1e-4}
FAMILIES = ("powerlaw", "banded", "mixed", "community", "hubs", "rect")


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dtype is None else t.to(dtype)


def close(out, expected, npdt, slack):
    tol = TOL[npdt]
    a = out.float().cpu().double().numpy()
    bad = np.abs(a - expected) > tol + tol * np.abs(expected) + slack
    assert not bad.any(), f"{int(bad.sum())} mismatches, max abs err {float(np.abs(a - expected).max()):.3e}"


SLACK_DEGREE = 1024


def accumulation_slack(crow, col, vals, B):
    """4 u sqrt(d_r) sqrt(sum_k (a_rk B_kj)^2) per output element of a row
    of d_r > SLACK_DEGREE nonzeros, u = 2^-24; zero for every other row."""
    v = vals.astype(np.float64)
    d = np.diff(crow).astype(np.float64)[:, None]
    s2 = O.spmm_f64(crow, col, v * v, B.astype(np.float64) ** 2)
    return np.where(d > SLACK_DEGREE, 4.0 * 2.0 ** -24 * np.sqrt(d) * np.sqrt(s2), 0.0)


def from_pairs(rows, cols, r, c):
    """CSR with distinct sorted columns per row from (row, column) pairs
    (duplicates dropped)."""
    key = np.unique(r.astype(np.int64) * cols + c.astype(np.int64))
    r, c = key // cols, key % cols
    crow = np.zeros(rows + 1, np.int64)
    np.add.at(crow, r + 1, 1)
    return np.cumsum(crow), c.astype(np.int64)


def matrix(family, rng):
    """One matrix of the family (square but for "rect"); sizes are drawn
    per case.  Returns rows, cols, crow, col."""
    n = int(rng.integers(2000, 60000))
    if family == "rect":  # power-law rows over a column space 1/16 to 4 times the row count
        cols = max(1, int(n * 2.0 ** rng.uniform(-4, 2)))
        deg = np.minimum(rng.zipf(1.8, n), min(cols, 3000))
        r = np.repeat(np.arange(n), deg)
        crow, col = from_pairs(n, cols, r, rng.integers(0, cols, r.size))
        return n, cols, crow, col
    if family == "powerlaw":  # Zipf degrees, uniform columns (configuration 2's shape)
        deg = np.minimum(rng.zipf(float(rng.uniform(1.5, 2.2)), n), min(n, 3000))
        deg[rng.random(n) < 0.1] = 0
        r = np.repeat(np.arange(n), deg)
        c = rng.integers(0, n, r.size)
    elif family == "banded":  # 16x16 blocks on a band of block diagonals (configuration 3's shape)
        nb, band = (n + 15) // 16, int(rng.integers(1, 9))
        bi = np.repeat(np.arange(nb), 2 * band + 1)
        bj = bi + np.tile(np.arange(-band, band + 1), nb)
        keep = (bj >= 0) & (bj < nb) & (rng.random(bi.size) < 0.6)
        bi, bj = bi[keep], bj[keep]
        fill = rng.random((bi.size, 16, 16)) < float(rng.uniform(0.3, 0.9))
        k, y, x = np.nonzero(fill)
        r, c = bi[k] * 16 + y, bj[k] * 16 + x
        keep = (r < n) & (c < n)
        r, c = r[keep], c[keep]
    elif family == "mixed":  # block windows interleaved with sparse windows (configuration 4's shape)
        nw = (n + 15) // 16
        blocky = rng.random(nw) < 0.5
        rs, cs = [], []
        for w in np.nonzero(blocky)[0]:
            for bj in rng.integers(0, (n + 15) // 16, 4):
                y, x = np.nonzero(rng.random((16, 16)) < 0.5)
                rs.append(w * 16 + y)
                cs.append(bj * 16 + x)
        sparse_rows = np.nonzero(~blocky[np.arange(n) // 16])[0]
        rs.append(np.repeat(sparse_rows, 4))
        cs.append(rng.integers(0, n, sparse_rows.size * 4))
        r, c = np.concatenate(rs), np.concatenate(cs)
        keep = (r < n) & (c < n)
        r, c = r[keep], c[keep]
    elif family == "community":  # most columns within the row's community (configuration 5's shape)
        size = int(rng.integers(64, 2048))
        deg = np.minimum(rng.zipf(2.0, n), 2000)
        r = np.repeat(np.arange(n), deg)
        local = rng.random(r.size) < 0.7
        base = (r // size) * size
        c = np.where(local, base + rng.integers(0, size, r.size), rng.integers(0, n, r.size))
        c = np.minimum(c, n - 1)
    else:  # "hubs": a few rows holding most columns, long runs of empty rows
        deg = rng.integers(0, 6, n)
        deg[rng.random(n) < 0.5] = 0
        deg[rng.integers(0, n, 4)] = n
        r = np.repeat(np.arange(n), deg)
        c = rng.integers(0, n, r.size)
    crow, col = from_pairs(n, n, r, c)
    return n, n, crow, col


CASES = [(f, s) for s in range(8) for f in FAMILIES]


@pytest.mark.parametrize("family,seed", CASES, ids=[f"{f}-{s}" for f, s in CASES])
def test_sweep(spmm_npu, family, seed):
    rng = np.random.default_rng(1000 * seed + FAMILIES.index(family))
    n, cols, crow, col = matrix(family, rng)
    half = bool((seed + FAMILIES.index(family)) % 2)
    npdt = np.float16 if half else np.float32
    vals = rng.uniform(-1, 1, col.size).astype(npdt)
    widths = [16, 64, 128, 256, 512] + ([1024] if half else [])
    N = int(rng.choice(widths[1:4] if family == "rect" else widths[1:]))
    B = rng.standard_normal((cols, N)).astype(npdt)
    expected = O.spmm_f64(crow, col, vals, B)
    slack = accumulation_slack(crow, col, vals, B)
    print(f"[sweep] {family} seed={seed} rows={n} cols={cols} nnz={col.size} N={N} {npdt.__name__}", flush=True)

    # spmm_csr: tolerance, then width invariance on the first 16 columns.
    it = torch.int64 if seed % 2 else torch.int32
    start = dev(O.make_start(crow, 40))
    out = spmm_npu.spmm_csr(dev(crow, it), dev(col, it), dev(vals), dev(B), start)
    close(out, expected, npdt, slack)
    narrow = spmm_npu.spmm_csr(dev(crow, it), dev(col, it), dev(vals), dev(np.ascontiguousarray(B[:, :16])), start)
    assert torch.equal(out[:, :16].cpu(), narrow.cpu()), "vector path differs across widths"

    # The layout operators take int32 indices on even seeds, int64 on odd.
    ix = np.int64 if seed % 2 else np.int32
    crow_x, col_x = crow.astype(ix), col.astype(ix)
    i32 = torch.int32
    empty_i = torch.zeros(0, dtype=i32, device="cuda")
    empty_v = torch.zeros(0, dtype=dev(vals).dtype, device="cuda")

    # csr_to_bcsr: bit-exact layout, then the pure block part.
    b = O.csr_to_bcsr(crow_x, col_x, vals, n, cols, 16)
    assert_same(spmm_npu.csr_to_bcsr(dev(crow_x), dev(col_x), dev(vals), n, cols, 16), b)
    out = spmm_npu.spmm_ascend_cube(dev(b["crow_window_ptr"], i32), dev(b["unique_col_ids"], i32), dev(b["value"]),
                                    torch.zeros(1, dtype=i32, device="cuda"), empty_i, empty_v, dev(B),
                                    dev(O.make_start(b["crow_window_ptr"], 20)),
                                    torch.zeros(40, dtype=i32, device="cuda"))
    close(out[:n], expected, npdt, slack)

    # spmm_cube: the legacy window-encoded form of the same matrix.
    rp, enc, ev = O.cube_encode(crow, col, vals, n)
    out = spmm_npu.spmm_cube(dev(rp, it), dev(enc, it), dev(ev), dev(B), torch.zeros(20, dtype=i32, device="cuda"))
    close(out[:n], expected, npdt, slack)

    # block_level_split: bit-exact layout, then the mixed op.
    a = float(rng.choice([(222.0 / 190.0) * 0.5, 295.0 / 505.0, 0.1, 3.0]))
    h = O.block_level_split(crow_x, col_x, vals, n, cols, a, 16)
    assert_same(spmm_npu.block_level_split(torch.from_numpy(crow_x), torch.from_numpy(col_x), torch.from_numpy(vals),
                                           n, cols, a, 16), h)
    out = spmm_npu.spmm_ascend_cube(
        dev(h["crow_window_ptr"], i32), dev(h["unique_col_ids"], i32), dev(h["value"]),
        dev(h["vrow_window_ptr"], i32), dev(h["vcol_indices"], i32), dev(h["vvalue"]), dev(B),
        dev(O.make_start(h["crow_window_ptr"], 20)), dev(O.make_start(h["vrow_window_ptr"], 40)))
    close(out[:n], expected, npdt, slack)

    # preprocess: the graph layout needs a square matrix.
    for graph_layout in (False, True) if n == cols else (False,):
        p = O.preprocess(crow_x, col_x, vals, n, cols, 16, graph_layout)
        assert_same(spmm_npu.preprocess(dev(crow_x), dev(col_x), dev(vals), n, cols, 16, graph_layout), p)
        ccol = p["renumbered_unique_col_ids"] if graph_layout else p["unique_col_ids"]
        vcol = p["renumbered_vcol_indices"] if graph_layout else p["vcol_indices"]
        inv = torch.from_numpy(p["inv_permutation"])
        dense = dev(B)
        if graph_layout:
            dense = spmm_npu.pack_node_tensor(dense, inv, int(p["packed_rows"][0]))
        out = spmm_npu.spmm_ascend_cube(
            dev(p["crow_window_ptr"], i32), dev(ccol, i32), dev(p["value"]),
            dev(p["vrow_window_ptr"], i32), dev(vcol, i32), dev(p["vvalue"]), dense,
            dev(O.make_start(p["crow_window_ptr"], 20)), dev(O.make_start(p["vrow_window_ptr"], 40)))
        close(spmm_npu.restore_node_tensor(out, inv), expected, npdt, slack)


SQUARE_CASES = [(f, s) for s in range(4) for f in FAMILIES if f != "rect"]


@pytest.mark.parametrize("family,seed", SQUARE_CASES, ids=[f"{f}-{s}" for f, s in SQUARE_CASES])
def test_sweep_packed_graph(spmm_npu, family, seed):
    rng = np.random.default_rng(7000 + 1000 * seed + FAMILIES.index(family))
    n, _, crow, col = matrix(family, rng)
    npdt, tdt = (np.float16, torch.float16) if seed % 2 else (np.float32, torch.float32)
    vals = rng.uniform(0, 1, col.size).astype(npdt)
    width = 32
    print(f"[sweep-graph] {family} seed={seed} rows={n} nnz={col.size} {npdt.__name__}", flush=True)
    prep = spmm_npu.preprocess(dev(crow), dev(col), dev(vals), n, n, 16, True)
    G = spmm_npu.PackedGraph(prep)
    x_np = rng.standard_normal((n, width)).astype(npdt)
    w_np = rng.standard_normal((n, width)).astype(npdt)
    x = torch.from_numpy(x_np).cuda().requires_grad_(True)
    y = G.restore(G(G.pack(x)))
    assert y.dtype == tdt
    (y.float() * torch.from_numpy(w_np).cuda().float()).sum().backward()
    close(y.detach(), O.spmm_f64(crow, col, vals, x_np), npdt, accumulation_slack(crow, col, vals, x_np))
    tcrow, tcol, tval = transpose_csr(crow, col, vals, n)
    close(x.grad, O.spmm_f64(tcrow, tcol, tval, w_np), npdt, accumulation_slack(tcrow, tcol, tval, w_np))
