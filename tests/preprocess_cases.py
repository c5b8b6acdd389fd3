"""Hand-worked preprocess cases whose expected outputs are derived by hand
from the reference's rules (extension/custom_op.cpp:765-1110), not computed
by the oracle.  Both are checked against the oracle on the CPU
(test_oracle_pins.py) and against the GPU pipeline (test_gpu_preprocess.py).

The rules they pin:

* windows are visited by density nnz/blocks, descending, ties by window id
  (:806-809), and the vector (AIV) rows follow that order, not window-id
  order (:887-905 builds aiv_windows from the sorted positions after the
  marginal one; rows are laid out from it at :917-940);
* the marginal window is the first position where
  (prefix + blocks_w) / 295 >= (remaining - nnz_w) / 505, with >= (:818-820);
* the marginal split keeps the first q that minimises
  max((prefix + q) / 295, (remaining - assigned_q) / 505) over columns in
  stable descending-occupancy order (:846-870).

Case "density order": seven 16-row windows of distinct densities, the
marginal window second in density order, the vector windows in an order
that differs from their ids.

  window  columns                                   nnz   blocks  density
  w2      every row holds columns 0..63             1024  64      16
  w5      row r holds c in 0..63 with (c+r)%16 < 12  768  64      12
  w1      row r holds c in 0..7 with (c+r)%16 < 6     48   8       6
  w6      row r holds c in 0..7 with (c+r)%16 < 4     32   8       4
  w0      row r holds c in 0..7 with (c+r)%16 < 3     24   8       3
  w3      row r holds c in 0..7 with (c+r)%16 < 2     16   8       2
  w4      row r holds c in 0..7 with (c+r)%16 < 1      8   8       1

  nnz = 1920.  Density order: w2, w5, w1, w6, w0, w3, w4.
  pos 0 (w2): 64/295 = 0.217 < (1920-1024)/505 = 1.774: prefix 64, rem 896.
  pos 1 (w5): 128/295 = 0.434 >= (896-768)/505 = 0.253: marginal = w5.
  Every w5 column has occupancy 12, so the bucket sort keeps first-seen
  order: row 0's 48 columns (c%16 < 12, ascending), then row 1 adds
  15, 31, 47, 63, row 2 adds 14, 30, 46, 62, row 3 adds 13, 29, 45, 61 and
  row 4 adds 12, 28, 44, 60.
  q: max((64+q)/295, (896-12q)/505); q=57 gives 212/505 = 0.4198, q=58 gives
  122/295 = 0.4136 (aiv 200/505 = 0.3960), q=59 gives 123/295 = 0.4169:
  q* = 58, so the first 58 columns in that order go to the block part and
  45, 61, 12, 28, 44, 60 stay in the vector part (shared window).
  Block windows: w2 (slot 0), w5 (slot 1); vector windows in density order:
  w1, w6, w0, w3, w4.  Packed rows: w2's rows 32..47, w5's 80..95, then
  16..31, 96..111, 0..15, 48..63, 64..79.

Case "tie": four windows where the marginal test meets equality,
59 * 505 == 101 * 295.

  window  columns                                     nnz  blocks  density
  w2      every row holds columns 0..39                640  40      16
  w1      row r holds c in 0..18 with (r+c) even       152  19      8
  w3      row r holds c in 0..15 with (r+c)%4 == 0      64  16      4
  w0      37 distinct columns 0..36, rows 0..4 hold     37  37      1
          three consecutive ids, rows 5..15 two

  nnz = 893.  pos 0 (w2): 40/295 = 0.136 < 253/505 = 0.501: prefix 40,
  rem 253.  pos 1 (w1): 59/295 = 0.2 >= (253-152)/505 = 101/505 = 0.2
  (both quotients round to the same double): marginal = w1 under >=; a >
  would move on to w3.  q: every column has occupancy 8; the vector cost
  (253-8q)/505 reaches 0.2 only at q = 19, so q* = 19 = all of w1's blocks
  (not shared), estimated costs 59/295 and 101/505.  Block windows w2, w1;
  vector windows w3, w0.  Packed rows: 32..47, 16..31, 48..63, 0..15.
"""

import numpy as np


def _csr(rows):
    crow = np.concatenate([[0], np.cumsum([len(r) for r in rows])]).astype(np.int64)
    col = np.concatenate([np.asarray(r, np.int64) for r in rows]).astype(np.int64)
    val = (np.arange(col.size) + 1).astype(np.float32)
    return crow, col, val


def density_order_case():
    def mod_rows(ncols, keep):
        return [[c for c in range(ncols) if (c + r) % 16 < keep] for r in range(16)]

    windows = {2: [list(range(64))] * 16, 5: mod_rows(64, 12), 1: mod_rows(8, 6), 6: mod_rows(8, 4),
               0: mod_rows(8, 3), 3: mod_rows(8, 2), 4: mod_rows(8, 1)}
    rows = [row for w in range(7) for row in windows[w]]
    crow, col, val = _csr(rows)
    aiv_cols_w5 = [12, 28, 44, 45, 60, 61]
    window_rows = lambda w: list(range(16 * w, 16 * w + 16))  # noqa: E731
    expected = {
        "nrows": 112,
        "marginal_window": 5,
        "marginal_total_blocks": 64,
        "marginal_aic_blocks": 58,
        "shared_windows": 1,
        "estimated_aic_cost": 122 / 295,
        "estimated_aiv_cost": 200 / 505,
        "estimated_max_cost": 122 / 295,
        "crow_window_ptr": [0, 64, 122],
        "unique_col_ids": list(range(64)) + [c for c in range(64) if c not in aiv_cols_w5],
        "permutation": sum((window_rows(w) for w in (2, 5, 1, 6, 0, 3, 4)), []),
        "aiv_cols_w5": aiv_cols_w5,
        "vnnz": 200,
    }
    return crow, col, val, expected


def tie_case():
    w2 = [list(range(40))] * 16
    w1 = [[c for c in range(19) if (r + c) % 2 == 0] for r in range(16)]
    w3 = [[c for c in range(16) if (r + c) % 4 == 0] for r in range(16)]
    w0, nxt = [], 0
    for r in range(16):
        k = 3 if r < 5 else 2
        w0.append(list(range(nxt, nxt + k)))
        nxt += k
    assert nxt == 37
    crow, col, val = _csr(w0 + w1 + w2 + w3)
    window_rows = lambda w: list(range(16 * w, 16 * w + 16))  # noqa: E731
    expected = {
        "nrows": 64,
        "marginal_window": 1,
        "marginal_total_blocks": 19,
        "marginal_aic_blocks": 19,
        "shared_windows": 0,
        "estimated_aic_cost": 59 / 295,
        "estimated_aiv_cost": 101 / 505,
        "estimated_max_cost": 59 / 295,
        "crow_window_ptr": [0, 40, 59],
        "unique_col_ids": list(range(40)) + list(range(19)),
        "permutation": sum((window_rows(w) for w in (2, 1, 3, 0)), []),
        "vnnz": 101,
    }
    return crow, col, val, expected


CASES = {"density-order": density_order_case, "tie": tie_case}


def check_against_hand(p, crow, col, expected):
    """Asserts a preprocess result (numpy arrays) against the hand-derived
    fields; the vector rows' lengths follow from the permutation."""
    for key in ("marginal_window", "marginal_total_blocks", "marginal_aic_blocks", "shared_windows"):
        assert int(p[key][0]) == expected[key], key
    for key in ("estimated_aic_cost", "estimated_aiv_cost", "estimated_max_cost"):
        assert float(p[key][0]) == expected[key], key
    np.testing.assert_array_equal(p["crow_window_ptr"], expected["crow_window_ptr"])
    np.testing.assert_array_equal(p["unique_col_ids"], expected["unique_col_ids"])
    perm = np.asarray(expected["permutation"])
    np.testing.assert_array_equal(p["permutation"], perm)
    inv = np.empty(perm.size, np.int64)
    inv[perm] = np.arange(perm.size)
    np.testing.assert_array_equal(p["inv_permutation"], inv)
    assert p["vcol_indices"].size == expected["vnnz"]
    # Vector rows: block-window rows keep only the columns left out of the
    # block part; every vector-window row keeps its whole original row.
    deg = np.diff(crow)
    nblock_rows = 16 * (len(expected["crow_window_ptr"]) - 1)
    vlen = np.diff(p["vrow_window_ptr"])
    np.testing.assert_array_equal(vlen[nblock_rows:], deg[perm[nblock_rows:]])
    if "aiv_cols_w5" in expected:
        w5 = perm[16:32]
        for i, r in enumerate(w5):
            cols = col[crow[r]:crow[r + 1]]
            want = cols[np.isin(cols, expected["aiv_cols_w5"])]
            got = p["vcol_indices"][p["vrow_window_ptr"][16 + i]:p["vrow_window_ptr"][17 + i]]
            np.testing.assert_array_equal(got, want)  # original column order
    else:
        assert vlen[:nblock_rows].sum() == 0
