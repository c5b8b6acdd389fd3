"""Writes the golden vectors of tests/golden/*.npz from the reference's own
code: oracle/_ref/libref.so, compiled (by ``make -C oracle ref``) from the
reference's std-only headers where they lie in the checkout
(extension/boundary_bucket_sort.h, extension/packed_column_reindex.h).

Run in the container that holds the reference checkout:
    make -C oracle all ref && python tests/golden/make_golden.py
The .npz files are data (inputs and the reference's outputs), loaded with
numpy's default allow_pickle=False; nothing here runs on the GPU box.

Cases:
  bucket_sort.npz  stable_bucket_sort_by_occupancy_desc (boundary_bucket_sort.h:13-56)
                   on seeded (columns, occupancy) inputs, including rejected
                   occupancies (status 1 = std::invalid_argument).
  renumber.npz     renumber_columns_for_packed_layout (packed_column_reindex.h:14-41)
                   for int32 and int64 ids, including -1 (status 1), out of
                   range (status 2) and int32 overflow (status 3) cases.
  graph.npz        two graph matrices: the oracle's preprocess(graph_layout=True)
                   inputs it passes to the reference routines (unique_col_ids,
                   vcol_indices, inv_permutation, packed_rows) and what the
                   reference routines return for them: the renumbered ids and
                   transpose_into_packed_layout (packed_column_reindex.h:43-101)
                   of the CSR.
"""

import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle"))
import oracle as O  # noqa: E402

P64 = ctypes.POINTER(ctypes.c_int64)
P32 = ctypes.POINTER(ctypes.c_int32)
U32 = ctypes.POINTER(ctypes.c_uint32)


def p(a, t=P64):
    return a.ctypes.data_as(t)


def bucket_sort_cases(lib):
    rng = np.random.default_rng(101)
    out = {}
    for i in range(24):
        n = int(rng.integers(0, 40))
        ncols = 64
        cols = rng.choice(ncols, n, replace=False).astype(np.int64)
        occ = np.zeros(ncols, np.int64)
        occ[cols] = rng.integers(1, 17, n)
        if i in (5, 17) and n:
            occ[cols[n // 2]] = 0 if i == 5 else 17
        res = cols.copy()
        rc = lib.ref_bucket_sort(p(res), ctypes.c_int64(n), p(occ), ctypes.c_int64(ncols), ctypes.c_int64(16))
        out[f"c{i}_columns"], out[f"c{i}_occupancy"] = cols, occ
        out[f"c{i}_status"] = np.array([rc], np.int64)
        out[f"c{i}_sorted"] = res if rc == 0 else np.zeros(0, np.int64)
    out["count"] = np.array([24], np.int64)
    return out


def renumber_cases(lib):
    rng = np.random.default_rng(202)
    out = {}
    i = 0
    for bits in (32, 64):
        dt = np.int32 if bits == 32 else np.int64
        for k in range(10):
            ninv = int(rng.integers(1, 40))
            inv = rng.permutation(ninv + 8)[:ninv].astype(np.int64)
            cols = rng.integers(0, ninv, size=int(rng.integers(0, 30))).astype(dt)
            if k == 3 and cols.size:
                inv[int(cols[0])] = -1
            if k == 5:
                cols = np.append(cols, dt(ninv))
            if k == 7 and bits == 32 and cols.size:
                inv[int(cols[0])] = 2**31 + 3
            res = np.zeros(max(cols.size, 1), dt)
            fn = lib.ref_renumber_i32 if bits == 32 else lib.ref_renumber_i64
            rc = fn(p(cols, P32 if bits == 32 else P64), ctypes.c_int64(cols.size), p(inv),
                    ctypes.c_int64(ninv), p(res, P32 if bits == 32 else P64))
            out[f"c{i}_cols"], out[f"c{i}_inv"] = cols, inv
            out[f"c{i}_status"] = np.array([rc], np.int64)
            out[f"c{i}_out"] = res[: cols.size] if rc == 0 else np.zeros(0, dt)
            i += 1
    out["count"] = np.array([i], np.int64)
    return out


def graph_matrix(seed, n, deg):
    rng = np.random.default_rng(seed)
    parts = []
    for r in range(n):
        d = int(min(n, rng.integers(0, deg + 1) if r % 7 else 3 * deg))
        parts.append(np.sort(rng.choice(n, d, replace=False)))
    crow = np.zeros(n + 1, np.int64)
    crow[1:] = np.cumsum([x.size for x in parts])
    col = np.concatenate(parts).astype(np.int64)
    val = rng.uniform(0, 1, col.size).astype(np.float32)
    return crow, col, val


def graph_cases(lib):
    out = {}
    for i, (seed, n, deg) in enumerate(((303, 70, 6), (304, 150, 12))):
        crow, col, val = graph_matrix(seed, n, deg)
        pre = O.preprocess(crow, col, val, n, n, 16, True)
        inv = pre["inv_permutation"].astype(np.int64)
        packed = int(pre["packed_rows"][0])
        renum = {}
        for key in ("unique_col_ids", "vcol_indices"):
            ids = pre[key].astype(np.int64)
            res = np.zeros(max(ids.size, 1), np.int64)
            rc = lib.ref_renumber_i64(p(ids), ctypes.c_int64(ids.size), p(inv), ctypes.c_int64(inv.size), p(res))
            assert rc == 0
            renum[key] = res[: ids.size]
        rt = np.zeros(packed + 1, np.int64)
        ct = np.zeros(max(col.size, 1), np.int64)
        vt = np.zeros(max(col.size, 1), np.uint32)
        rc = lib.ref_transpose(p(crow), ctypes.c_int64(crow.size), p(col), p(val.view(np.uint32), U32),
                               ctypes.c_int64(col.size), p(inv), ctypes.c_int64(n), ctypes.c_int64(packed),
                               p(rt), p(ct), p(vt, U32))
        assert rc == 0
        out.update({f"g{i}_crow": crow, f"g{i}_col": col, f"g{i}_val": val,
                    f"g{i}_unique_col_ids": pre["unique_col_ids"].astype(np.int64),
                    f"g{i}_vcol_indices": pre["vcol_indices"].astype(np.int64),
                    f"g{i}_inv_permutation": inv, f"g{i}_packed_rows": np.array([packed], np.int64),
                    f"g{i}_renumbered_unique_col_ids": renum["unique_col_ids"],
                    f"g{i}_renumbered_vcol_indices": renum["vcol_indices"],
                    f"g{i}_transpose_rowptr": rt, f"g{i}_transpose_col": ct[: col.size],
                    f"g{i}_transpose_val": vt[: col.size].view(np.float32)})
    out["count"] = np.array([2], np.int64)
    return out


def main():
    lib = O.reference_library()
    if lib is None:
        sys.exit("oracle/_ref/libref.so is not built: run `make -C oracle ref` where the reference checkout exists")
    for name, fn in (("bucket_sort", bucket_sort_cases), ("renumber", renumber_cases), ("graph", graph_cases)):
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **fn(lib))
        print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
