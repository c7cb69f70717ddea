"""gpre_dense (attention q/k/v and o projections on the card, gpu_pre.m:200-256) against maple.c's CPU
projections jobB_qkv / jobB_o (maple.c:459-470): prep of each input row (maple.c:183-194, the oracle's mo_prep,
pinned against maple.c) and tdot_multi's (float)(sum (c-1) q) * qs * s[row]. The integer sums are exact and
the two fp32 products are the same sequence, so the comparison is bit for bit."""
import numpy as np
import pytest

import maplemoe as M
import pyoracle as O
from helpers import SEED

pytestmark = pytest.mark.gpu


def random_ternary(rng, rows, cols):
    """packed codes (convert.py layout, codes 0..2 = w+1) and the natural-order codes they hold"""
    codes = rng.integers(0, 3, (rows, cols), dtype=np.uint8)
    packed = np.empty((rows, cols // 4), np.uint8)
    O.oracle().mo_pack(O._p(np.ascontiguousarray(codes)), rows, cols, O._p(packed))
    return packed, codes


def cpu_projection(x, mats):
    """maple.c's jobB_qkv / jobB_o for the rows of x: y[b] = concatenation over the group's matrices"""
    out = []
    for b in range(x.shape[0]):
        q, qs, qsum = O.prep(x[b])
        row = []
        for _, codes, scales in mats:
            d = (codes.astype(np.int64) - 1) @ q.astype(np.int64)          # sum (c - 1) q = sum c q - qsum, exact
            row.append(d.astype(np.float32) * qs * scales)                  # (float)(...) * qs, then * s (fp32 each)
        out.append(np.concatenate(row))
    return np.stack(out)


def test_gpre_dense_matches_cpu_projections():
    lib = M.lib()
    M.check(lib.mmoe_init(2048), "mmoe_init")
    M.check(lib.mmoe_dense_reset(), "dense reset")
    assert lib.gpre_dense(0, None, 1, None) < 0                              # before gpre_dense_done
    rng = np.random.default_rng(SEED + 7)
    groups = {0: [2048, 512, 512], 1: [2048]}                               # layer 0: q, k, v; then o
    mats = {}
    for g, rows_list in groups.items():
        mats[g] = []
        for rows in rows_list:
            packed, codes = random_ternary(rng, rows, 2048)
            scales = rng.uniform(0.01, 0.05, rows).astype(np.float32)
            lib.gpre_dense_add(g, M.ptr(packed), M.ptr(scales), rows, 2048)
            mats[g].append((packed, codes, scales))
    assert lib.gpre_dense_done(256) == 0, lib.mmoe_last_error()
    for g in (0, 1):
        ys = sum(r for r in groups[g])
        for nb in (1, 37, 64, 100, 256):
            x = rng.standard_normal((nb, 2048)).astype(np.float32)
            y = np.full((nb, ys), np.nan, np.float32)
            t = lib.gpre_dense(g, M.ptr(x), nb, M.ptr(y))
            assert t >= 0, lib.mmoe_last_error()
            want = cpu_projection(x, mats[g])
            assert np.array_equal(y.view(np.int32), want.view(np.int32)), f"group {g} nb {nb}"
        print(f"\n  group {g}: {ys} rows bit-exact at nb 1..256")
    assert lib.gpre_dense(1, None, 257, None) < 0                            # past maxtok
    assert lib.gpre_dense(5, None, 1, None) < 0                              # empty group
    lib.gpre_dense_add(0, M.ptr(mats[0][0][0]), M.ptr(mats[0][0][2]), 2048, 2048)
    assert b"after gpre_dense_done" in lib.mmoe_last_error()
    assert lib.gpre_dense_done(256) == -1                                   # a second upload needs a reset
    assert b"already" in lib.mmoe_last_error()
