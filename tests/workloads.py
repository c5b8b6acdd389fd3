"""Seeded synthetic CSR workloads for the five benchmark configurations (1-5).

All generators use ``numpy.random.Generator(PCG64(2027 + config_id))`` (2027 is
the reference's default base seed, tests/task_mapping/correctness.py:92) and
return CSR with distinct, sorted column indices per row, as ``preprocess``
requires (extension/custom_op.cpp:1449-1450).  Index arrays are int64 here;
callers cast to int32 at the kernel boundary as the reference's tests do
(tests/task_mapping/common.py:352-360).

``scale`` < 1 shrinks a configuration (rows and nonzeros) for fast tests while
keeping its structure.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class Workload:
    name: str
    rows: int
    cols: int
    crow: np.ndarray      # int64 [rows + 1]
    col: np.ndarray       # int64 [nnz]
    values: np.ndarray    # float16 / float32 [nnz]
    widths: tuple         # feature widths N of the configuration
    dtype: str            # "fp16" or "fp32"
    seed: int

    @property
    def nnz(self) -> int:
        return int(self.col.size)

    def dense(self, width: int, seed_offset: int = 0) -> np.ndarray:
        """Dense operand B [cols, width] ~ N(0, 1) in the workload dtype."""
        rng = np.random.default_rng(self.seed + 1000 + width + seed_offset)
        b = rng.standard_normal((self.cols, width), dtype=np.float32)
        return b.astype(np.float16 if self.dtype == "fp16" else np.float32)


def _csr_from_coo(rows: int, r: np.ndarray, c: np.ndarray, cols: int):
    """Sort (row, col) pairs, drop duplicates, build the row pointer."""
    key = r.astype(np.int64) * cols + c.astype(np.int64)
    key = np.unique(key)
    r = key // cols
    c = key - r * cols
    crow = np.zeros(rows + 1, dtype=np.int64)
    counts = np.bincount(r, minlength=rows)
    crow[1:] = np.cumsum(counts)
    return crow, c.astype(np.int64)


def _distinct_rows(rng: np.random.Generator, degrees: np.ndarray, cols: int):
    """Distinct uniform columns per row (degree d_i, d_i <= cols), sorted."""
    rows = degrees.size
    r = np.repeat(np.arange(rows, dtype=np.int64), degrees)
    c = rng.integers(0, cols, size=r.size, dtype=np.int64)
    crow = np.concatenate([[0], np.cumsum(degrees)]).astype(np.int64)
    # Rows holding more than half the columns (only in scaled-down matrices)
    # are drawn without replacement: redrawing their repeats would take long.
    for row in np.nonzero(degrees > cols // 2)[0]:
        c[crow[row]:crow[row + 1]] = rng.choice(cols, int(degrees[row]), replace=False)
    c = _redraw_duplicates(rng, r, c, cols, crow,
                           lambda idx, final: rng.integers(0, cols, size=idx.size, dtype=np.int64))
    return _csr_from_coo(rows, r, c, cols)


def _zipf_degrees(rng, rows, alpha, max_deg, target_nnz):
    """Zipf(alpha) degrees clipped to [1, max_deg], then rescaled (scale,
    round, re-clip) so that they sum to target_nnz.  Rounding and the clip at
    either end move the sum off a plain target/sum factor (at config 2's
    factor of about 1.3 every degree-1 row rounds back to 1, losing 6.6%), so
    the factor is found by bisection on the rescaled sum, which is monotone
    in it; the sum lands within a few degrees of the target."""
    d0 = np.minimum(rng.zipf(alpha, size=rows), max_deg).astype(np.float64)

    def total(f):
        return np.clip(np.rint(d0 * f), 1, max_deg).sum()

    lo, hi = 0.0, target_nnz / d0.sum()
    while total(hi) < target_nnz and hi < 1e9:
        hi *= 2
    for _ in range(60):  # smallest factor whose sum reaches the target
        mid = 0.5 * (lo + hi)
        lo, hi = (mid, hi) if total(mid) < target_nnz else (lo, mid)
    return np.clip(np.rint(d0 * hi), 1, max_deg).astype(np.int64)


def _row_ranges(crow: np.ndarray, rows: np.ndarray) -> np.ndarray:
    """Positions of the entries of the given rows (CSR row pointer crow)."""
    starts, lens = crow[rows], crow[rows + 1] - crow[rows]
    if lens.sum() == 0:
        return np.zeros(0, np.int64)
    offs = np.repeat(starts - np.concatenate([[0], np.cumsum(lens)[:-1]]), lens)
    return offs + np.arange(int(lens.sum()), dtype=np.int64)


def _redraw_duplicates(rng, r, c, cols, crow, redraw, rounds=6):
    """Redraws every repeated (row, column) pair until each row's columns are
    distinct.  r is sorted (row-major entries, row pointer crow); redraw(idx,
    final) returns new columns for positions idx, with final=True after
    `rounds` rounds (the caller then draws from a larger space).  Only the rows that still hold a repeat are re-checked."""
    idx = np.arange(r.size, dtype=np.int64)
    for it in range(10 * rounds):
        key = r[idx] * cols + c[idx]
        order = np.argsort(key, kind="stable")
        ks = key[order]
        dup = ks[1:] == ks[:-1]
        if not dup.any():
            return c
        bad = idx[order[1:][dup]]
        c[bad] = redraw(bad, it >= rounds)
        idx = _row_ranges(crow, np.unique(r[bad]))
    raise RuntimeError("duplicate columns could not be redrawn")


def config1(scale: float = 1.0) -> Workload:
    """Uniform random 16384^2, 8 nnz/row, fp32, N=128 (the CPU-path anchor)."""
    seed = 2027 + 1
    rng = np.random.default_rng(seed)
    n = max(64, int(16384 * scale))
    crow, col = _distinct_rows(rng, np.full(n, 8, dtype=np.int64), n)
    vals = rng.uniform(-1, 1, col.size).astype(np.float32)
    return Workload("C1-uniform", n, n, crow, col, vals, (128,), "fp32", seed)


def config2(scale: float = 1.0) -> Workload:
    """Power-law 100000^2, Zipf(1.8) degrees in [1, 4096] rescaled to ~2M nnz, fp16, N=128."""
    seed = 2027 + 2
    rng = np.random.default_rng(seed)
    n = max(256, int(100000 * scale))
    deg = _zipf_degrees(rng, n, 1.8, min(4096, n), 2_000_000 * scale)
    crow, col = _distinct_rows(rng, deg, n)
    vals = rng.uniform(-1, 1, col.size).astype(np.float16)
    return Workload("C2-powerlaw", n, n, crow, col, vals, (128,), "fp16", seed)


def config3(scale: float = 1.0) -> Workload:
    """Block-banded 65536^2: 16x16 blocks on 33 block-diagonals, block kept with
    p=0.6, entries with p=0.7, fp16, N=256 (and 128 for the target)."""
    seed = 2027 + 3
    rng = np.random.default_rng(seed)
    nb = max(8, int(4096 * scale))
    n = nb * 16
    bi = np.repeat(np.arange(nb, dtype=np.int64), 33)
    bj = bi + np.tile(np.arange(-16, 17, dtype=np.int64), nb)
    ok = (bj >= 0) & (bj < nb)
    bi, bj = bi[ok], bj[ok]
    keep = rng.random(bi.size) < 0.6
    bi, bj = bi[keep], bj[keep]
    mask = rng.random((bi.size, 16, 16)) < 0.7
    blk, rr, cc = np.nonzero(mask)
    r = bi[blk] * 16 + rr
    c = bj[blk] * 16 + cc
    crow, col = _csr_from_coo(n, r, c, n)
    vals = rng.standard_normal(col.size, dtype=np.float32).astype(np.float16)
    return Workload("C3-blockband", n, n, crow, col, vals, (256, 128), "fp16", seed)


def config4(scale: float = 1.0) -> Workload:
    """Mixed 200000^2: half the 16-row windows hold 4 random 16x16 blocks at
    50% fill, the other half 4 uniform nnz per row; fp16, N=64 and 512."""
    seed = 2027 + 4
    rng = np.random.default_rng(seed)
    nwin = max(8, int(12500 * scale))
    n = nwin * 16
    nbcol = n // 16
    is_block = rng.permutation(np.arange(nwin) < nwin // 2)
    bw = np.nonzero(is_block)[0]
    # 4 distinct block columns per block window
    bcols = np.stack([rng.choice(nbcol, 4, replace=False) for _ in range(bw.size)]) if bw.size else np.zeros((0, 4), np.int64)
    mask = rng.random((bw.size, 4, 16, 16)) < 0.5
    w_i, b_i, rr, cc = np.nonzero(mask)
    r_block = bw[w_i] * 16 + rr
    c_block = bcols[w_i, b_i] * 16 + cc
    sw = np.nonzero(~is_block)[0]
    srows = (sw[:, None] * 16 + np.arange(16)[None, :]).reshape(-1)
    deg = np.zeros(n, dtype=np.int64)
    deg[srows] = 4
    crow_s, col_s = _distinct_rows(rng, deg, n)
    r_s = np.repeat(np.arange(n, dtype=np.int64), np.diff(crow_s))
    r = np.concatenate([r_block, r_s])
    c = np.concatenate([c_block, col_s])
    crow, col = _csr_from_coo(n, r, c, n)
    vals = rng.uniform(-1, 1, col.size).astype(np.float16)
    return Workload("C4-mixed", n, n, crow, col, vals, (64, 512), "fp16", seed)


def config5(scale: float = 1.0) -> Workload:
    """Graph-like 1048576^2 (~32M nnz): Zipf(2.0) degrees in [1, 8192], 70% of
    edges inside 4096-node communities, random relabelling; fp32, N=512.
    Repeated columns of a row are redrawn, so the rows keep their drawn
    degrees and nnz is the rescaled degree sum (32.0M at full size).  Rows of
    more than 4096 community edges cannot hold them all distinct, and the
    repeats that are still left after a few community redraws are drawn
    globally."""
    seed = 2027 + 5
    rng = np.random.default_rng(seed)
    n = max(4096, int(1048576 * scale))
    comm = 4096 if n >= 4096 * 4 else max(16, n // 16)
    deg = _zipf_degrees(rng, n, 2.0, min(8192, n), 32_000_000 * scale)
    r = np.repeat(np.arange(n, dtype=np.int64), deg)
    local = rng.random(r.size) < 0.7
    c = np.empty(r.size, dtype=np.int64)
    base = (r // comm) * comm
    c[local] = base[local] + rng.integers(0, comm, size=int(local.sum()), dtype=np.int64)
    c[~local] = rng.integers(0, n, size=int((~local).sum()), dtype=np.int64)
    c = np.minimum(c, n - 1)

    def redraw(idx, final):
        # A repeated column is drawn again the way it was drawn (inside the
        # row's community or globally); a row holding more community edges
        # than its community has nodes draws the rest globally.
        out = rng.integers(0, n, size=idx.size, dtype=np.int64)
        if not final:
            loc = local[idx]
            out[loc] = base[idx[loc]] + rng.integers(0, comm, size=int(loc.sum()), dtype=np.int64)
        return np.minimum(out, n - 1)

    crow0 = np.concatenate([[0], np.cumsum(deg)]).astype(np.int64)
    c = _redraw_duplicates(rng, r, c, n, crow0, redraw)
    q = rng.permutation(n).astype(np.int64)  # node relabelling Q
    crow, col = _csr_from_coo(n, q[r], q[c], n)
    vals = rng.uniform(0, 1, col.size).astype(np.float32)
    return Workload("C5-graph", n, n, crow, col, vals, (512,), "fp32", seed)


CONFIGS = {1: config1, 2: config2, 3: config3, 4: config4, 5: config5}


def make(config_id: int, scale: float = 1.0) -> Workload:
    return CONFIGS[config_id](scale)


def algorithmic_bytes(w: Workload, width: int, index_bytes: int = 4) -> int:
    """Format-independent compulsory bytes of one SpMM call:
    4*(M+1) + (4+s)*nnz + s*N*K_ref + s*M*N, K_ref = distinct columns of A."""
    s = 2 if w.dtype == "fp16" else 4
    k_ref = int(np.unique(w.col).size)
    return index_bytes * (w.rows + 1) + (index_bytes + s) * w.nnz + s * width * k_ref + s * w.rows * width
