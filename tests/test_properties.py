"""Property-based checks (hypothesis) on random small CSR matrices.

CPU: the oracle's layout converters and splits rebuild A exactly (every
nonzero lands once, at its row and column; padding is zero), preprocess's
permutation and its un-permuted block + vector parts rebuild A, the graph
layout's renumbering and packed transpose are P A^T P^T, and spmm_f64 is
A @ B.  These pin the oracle against mathematics, independently of the
reference code it restates."""

import numpy as np
import pytest
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

import oracle as O

SETTINGS = settings(max_examples=60, deadline=None, derandomize=True,
                    suppress_health_check=[HealthCheck.too_slow])


@st.composite
def csr(draw, max_rows=70, max_cols=70, square=False, max_deg=24):
    rows = draw(st.integers(1, max_rows))
    cols = rows if square else draw(st.integers(1, max_cols))
    seed = draw(st.integers(0, 2**31 - 1))
    rng = np.random.default_rng(seed)
    deg = rng.integers(0, min(cols, max_deg) + 1, rows)
    deg[rng.random(rows) < 0.25] = 0
    if rows > 3 and draw(st.booleans()):
        deg[rng.integers(0, rows)] = cols  # a full row
    parts = [np.sort(rng.choice(cols, d, replace=False)) for d in deg]
    crow = np.zeros(rows + 1, np.int64)
    crow[1:] = np.cumsum(deg)
    col = np.concatenate(parts).astype(np.int64) if parts else np.zeros(0, np.int64)
    vals = rng.uniform(-1, 1, col.size).astype(np.float32)
    vals[vals == 0] = 0.5
    return rows, cols, crow, col, vals


def dense_of(rows, cols, crow, col, vals):
    A = np.zeros((rows, cols), np.float64)
    for r in range(rows):
        for p in range(crow[r], crow[r + 1]):
            A[r, col[p]] = vals[p]
    return A


def blocks_dense(nrows_pad, cols, cwp, uniq, value):
    """Rebuild from BCSR(16x1): value[16b + r] at (16w + r, uniq[b])."""
    A = np.zeros((nrows_pad, cols), np.float64)
    for w in range(cwp.size - 1):
        ids = uniq[cwp[w]:cwp[w + 1]]
        assert np.all(np.diff(ids) > 0), "block columns ascend within a window"
        for b in range(cwp[w], cwp[w + 1]):
            for r in range(16):
                v = value[16 * b + r]
                if v != 0:
                    assert A[16 * w + r, uniq[b]] == 0
                    A[16 * w + r, uniq[b]] = v
    return A


def csr_dense(nrows, cols, rp, ci, vv):
    return dense_of(nrows, cols, np.asarray(rp, np.int64), np.asarray(ci, np.int64), vv)


@SETTINGS
@given(csr())
def test_bcsr_rebuilds_the_matrix(m):
    rows, cols, crow, col, vals = m
    b = O.csr_to_bcsr(crow, col, vals, rows, cols, 16)
    nwin = (rows + 15) // 16
    assert b["crow_window_ptr"].size == nwin + 1 and np.all(np.diff(b["crow_window_ptr"]) >= 0)
    rebuilt = blocks_dense(16 * nwin, cols, b["crow_window_ptr"], b["unique_col_ids"], b["value"])
    np.testing.assert_array_equal(rebuilt[:rows], dense_of(*m))
    # one block per distinct (window, column)
    want = sum(len({int(c) for c in col[crow[16 * w]:crow[min(16 * w + 16, rows)]]}) for w in range(nwin))
    assert b["unique_col_ids"].size == want


@SETTINGS
@given(csr())
def test_cube_tiles_rebuild_the_matrix(m):
    rows, cols, crow, col, vals = m
    c = O.csr_to_ascend_cube(crow, col, vals, rows, cols, 16)
    nwin = (rows + 15) // 16
    A = np.zeros((16 * nwin, cols))
    cwp, uniq, value = c["crow_window_ptr"], c["unique_col_ids"], c["value"]
    for w in range(nwin):
        for t in range(cwp[w], cwp[w + 1]):
            for rr in range(16):
                for cc in range(16):
                    v = value[256 * t + 16 * rr + cc]
                    if v != 0:
                        A[16 * w + rr, uniq[16 * t + cc]] = v
    np.testing.assert_array_equal(A[:rows], dense_of(*m))


@SETTINGS
@given(csr(), st.floats(0.01, 50.0))
def test_block_level_split_rebuilds_the_matrix(m, a):
    rows, cols, crow, col, vals = m
    s = O.block_level_split(crow, col, vals, rows, cols, a, 16)
    nwin = (rows + 15) // 16
    blocks = blocks_dense(16 * nwin, cols, s["crow_window_ptr"], s["unique_col_ids"], s["value"])
    vrows = s["vrow_window_ptr"].size - 1
    vec = csr_dense(vrows, cols, s["vrow_window_ptr"], s["vcol_indices"], s["vvalue"])
    total = blocks[:rows].copy()
    total[:min(vrows, rows)] += vec[:rows]
    np.testing.assert_array_equal(total, dense_of(*m))
    assert int(np.count_nonzero(blocks)) + s["vcol_indices"].size == col.size


@SETTINGS
@given(csr(square=True), st.booleans())
def test_preprocess_parts_unpermute_to_the_matrix(m, graph_layout):
    rows, cols, crow, col, vals = m
    p = O.preprocess(crow, col, vals, rows, cols, 16, graph_layout)
    inv = p["inv_permutation"]
    perm = p["permutation"]
    assert inv.size == rows and len(set(inv.tolist())) == rows
    assert np.all(perm[inv] == np.arange(rows))  # perm is inv's inverse on real rows
    packed = int(p["packed_rows"][0]) if graph_layout else max(16 * (p["crow_window_ptr"].size - 1),
                                                               p["vrow_window_ptr"].size - 1)
    nblk_rows = 16 * (p["crow_window_ptr"].size - 1)
    blocks = blocks_dense(max(nblk_rows, 1), cols, p["crow_window_ptr"], p["unique_col_ids"], p["value"])
    vrows = p["vrow_window_ptr"].size - 1
    vec = csr_dense(vrows, cols, p["vrow_window_ptr"], p["vcol_indices"], p["vvalue"])
    out = np.zeros((max(packed, nblk_rows, vrows, 1), cols))
    out[:nblk_rows] += blocks[:nblk_rows]
    out[:vrows] += vec
    A = dense_of(*m)
    np.testing.assert_array_equal(out[inv], A)  # row i of A sits at packed row inv[i]
    assert int(np.count_nonzero(blocks)) + p["vcol_indices"].size == col.size
    if graph_layout:
        # renumbered ids are inv[original id]; the transpose part is P A^T P^T
        np.testing.assert_array_equal(p["renumbered_unique_col_ids"], inv[p["unique_col_ids"]])
        np.testing.assert_array_equal(p["renumbered_vcol_indices"], inv[p["vcol_indices"]])
        PAt = np.zeros((packed, packed))
        PAt[np.ix_(inv, inv)] = A.T
        tb = blocks_dense(16 * (p["transpose_crow_window_ptr"].size - 1), packed,
                          p["transpose_crow_window_ptr"], p["transpose_unique_col_ids"], p["transpose_value"])
        tv_rows = p["transpose_vrow_window_ptr"].size - 1
        tv = csr_dense(tv_rows, packed, p["transpose_vrow_window_ptr"], p["transpose_vcol_indices"],
                       p["transpose_vvalue"])
        T = np.zeros((max(tb.shape[0], tv_rows, packed), packed))
        T[:tb.shape[0]] += tb
        T[:tv_rows] += tv
        np.testing.assert_array_equal(T[:packed], PAt)


@SETTINGS
@given(csr(), st.integers(1, 40))
def test_spmm_f64_is_the_dense_product(m, width):
    rows, cols, crow, col, vals = m
    B = np.random.default_rng(width).standard_normal((cols, width))
    np.testing.assert_allclose(O.spmm_f64(crow, col, vals, B), dense_of(*m) @ B, rtol=1e-12, atol=1e-12)


@SETTINGS
@given(csr(), st.integers(1, 64))
def test_make_start_brackets_each_core_start(m, cores):
    rows, cols, crow, col, vals = m
    s = O.make_start(crow, cores)
    total = int(crow[-1])
    if total <= 0:
        assert not s.any()
        return
    chunk = -(-total // cores)
    assert np.all(np.diff(s) >= 0)
    for k in range(cores):
        t, i = k * chunk, int(s[k])
        # start[k] is the last pointer index whose pointer is <= t (leading
        # empty rows included), so core k's first item t lies in row i
        assert crow[i] <= t and (i == rows or crow[i + 1] > t)
