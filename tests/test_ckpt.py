"""maple.c's checkpoint directory (csrc/ckpt.c): record table, region plan and location table, against an
independent restatement of maple.c:61-83 (load) and maple.c:1106-1131 (regions, GLOC) on a synthetic
checkpoint; the GPU test runs layers loaded from it against the oracle."""
import ctypes as C
import os

import numpy as np
import pytest

import maplemoe as M
import pyoracle as O
from ckpt_synth import NE, REC, distinct, write_checkpoint
from helpers import SEED, normed_hidden, relmax

PG = os.sysconf("SC_PAGE_SIZE")


def maple_plan(recs, L, nshard=9):
    """maple.c:1106-1131 for layer L: per shard the page-aligned span of the 256 x 6 expert tensors, slots in
    shard order; GLOC[e][2m] = slot, GLOC[e][2m+1] = offset - span start."""
    base = 3 + L * (9 + 3 * NE) + 9
    lo, hi = [None] * nshard, [0] * nshard
    spans = []
    for e in range(NE):
        for m in range(6):
            kind, f, off, soff, rows, cols = recs[base + 3 * e + m // 2]
            o, n = (soff, rows * 4) if m % 2 else (off, rows * cols // 4)
            spans.append((e, m, f, o))
            lo[f] = o if lo[f] is None else min(lo[f], o)
            hi[f] = max(hi[f], o + n)
    regions, slot = [], {}
    for k in range(nshard):
        if hi[k]:
            a, b = lo[k] // PG * PG, -(-hi[k] // PG) * PG
            slot[k] = len(regions)
            regions.append((k, a, b - a))
    loc = np.zeros((NE, 12), np.uint32)
    for e, m, f, o in spans:
        loc[e, 2 * m] = slot[f]
        loc[e, 2 * m + 1] = o - regions[slot[f]][1]
    return regions, loc


def lib_plan(L):
    sh = (C.c_int * 4)(); lo = (C.c_uint64 * 4)(); ln = (C.c_uint64 * 4)()
    loc = np.zeros((NE, 12), np.uint32)
    n = M.lib().mmoe_ckpt_layer_plan(L, sh, lo, ln, M.ptr(loc))
    return n, [(sh[i], lo[i], ln[i]) for i in range(max(n, 0))], loc


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = str(tmp_path_factory.mktemp("ckpt"))
    info = write_checkpoint(d, SEED)
    return d, info


def test_record_size_and_count(ckpt):
    d, info = ckpt
    assert REC.size == 26                                  # '<BBQQII', maple.c:39 Rec
    assert os.path.getsize(os.path.join(d, "layout.bin")) == 26 * (3 + 24 * (9 + 3 * NE)) == 26 * len(info["recs"])


def test_plan_matches_maple_region_math(ckpt):
    d, info = ckpt
    lib = M.lib()
    assert lib.mmoe_ckpt_open(d.encode()) == 0, lib.mmoe_ckpt_error()
    try:
        for L in (0, 1, 7, 23):
            n, regions, loc = lib_plan(L)
            want, wloc = maple_plan(info["recs"], L)
            assert n == len(want) == 3
            assert regions == want
            assert np.array_equal(loc, wloc)
            # every expert tensor lies inside its region (what gpre_moe's location lookup assumes)
            for e in range(NE):
                for m in range(6):
                    s_, off = loc[e, 2 * m], loc[e, 2 * m + 1]
                    n_ = (4 * (2048 if m == 5 else 512)) if m % 2 else 262144
                    assert off % 16 == 0 and off + n_ <= regions[s_][2]
    finally:
        lib.mmoe_ckpt_close()


def test_bf16_pointers(ckpt):
    d, info = ckpt
    lib = M.lib()
    assert lib.mmoe_ckpt_open(d.encode()) == 0, lib.mmoe_ckpt_error()
    try:
        for L in (0, 3):
            p = lib.mmoe_ckpt_bf16(L, 4)
            r = np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint16)), shape=(NE * 2048,)).reshape(NE, 2048)
            assert np.array_equal(r, info["routers"][L % 2])
            p = lib.mmoe_ckpt_bf16(L, 1)
            assert np.array_equal(np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint16)), shape=(2048,)), info["post_ln"])
        assert not lib.mmoe_ckpt_bf16(24, 4) and not lib.mmoe_ckpt_bf16(0, 5)
    finally:
        lib.mmoe_ckpt_close()


def rewrite_record(d, i, **kw):
    path = os.path.join(d, "layout.bin")
    raw = bytearray(open(path, "rb").read())
    f = list(REC.unpack_from(raw, 26 * i))
    names = ["kind", "file", "off", "soff", "rows", "cols"]
    for k, v in kw.items():
        f[names.index(k)] = v
    REC.pack_into(raw, 26 * i, *f)
    open(path, "wb").write(raw)


def expect_open_error(d, text):
    lib = M.lib()
    assert lib.mmoe_ckpt_open(d.encode()) == -1
    assert text in lib.mmoe_ckpt_error().decode(), lib.mmoe_ckpt_error()


def test_rejects_bad_checkpoints(tmp_path):
    lib = M.lib()
    d = str(tmp_path / "c")
    write_checkpoint(d, SEED, nexp=2)
    first_expert = 3 + 9
    rewrite_record(d, 4, kind=ord("t")); expect_open_error(d, "expected bf16")          # layer 0 input_layernorm
    rewrite_record(d, 4, kind=ord("b"))
    rewrite_record(d, first_expert, kind=ord("b")); expect_open_error(d, "expected ternary")
    rewrite_record(d, first_expert, kind=ord("t"))
    off = REC.unpack_from(open(os.path.join(d, "layout.bin"), "rb").read(), 26 * first_expert)[2]
    rewrite_record(d, first_expert, off=off + 8); expect_open_error(d, "16-byte")        # maple.c:1117
    rewrite_record(d, first_expert, off=off, rows=256); expect_open_error(d, "expected 512 x 2048")
    rewrite_record(d, first_expert, rows=512, off=1 << 40); expect_open_error(d, "outside shard")
    rewrite_record(d, first_expert, off=off, file=9); expect_open_error(d, "shard 9 outside")
    rewrite_record(d, first_expert, file=0)
    assert lib.mmoe_ckpt_open(d.encode()) == 0, lib.mmoe_ckpt_error()                    # repaired
    lib.mmoe_ckpt_close()
    with open(os.path.join(d, "layout.bin"), "r+b") as f:
        f.truncate(26 * 100)
    expect_open_error(d, "too short")
    os.remove(os.path.join(d, "shard-00007.bin"))
    expect_open_error(d, "shard-00007.bin")
    assert lib.mmoe_ckpt_layer_plan(0, (C.c_int * 4)(), (C.c_uint64 * 4)(), (C.c_uint64 * 4)(), None) == -1


def test_more_than_four_shards(tmp_path):
    """maple.c:1124 refuses a layer whose experts span more than 4 shards"""
    lib = M.lib()
    d = str(tmp_path / "c5")
    write_checkpoint(d, SEED, nexp=5, gu_shards=5)
    assert lib.mmoe_ckpt_open(d.encode()) == 0, lib.mmoe_ckpt_error()
    try:
        n, _, _ = lib_plan(0)
        assert n == -1 and "more than 4 shards" in lib.mmoe_ckpt_error().decode()
    finally:
        lib.mmoe_ckpt_close()


@pytest.mark.gpu
def test_layers_from_checkpoint(ckpt):
    """Layers 20 and 21 loaded from the checkpoint (regions, GLOC, router) give the oracle's results on the same
    expert bytes: top-8 identical, x within 1e-5."""
    d, info = ckpt
    lib = M.lib()
    M.check(lib.mmoe_init(2048), "mmoe_init")
    assert lib.mmoe_ckpt_open(d.encode()) == 0, lib.mmoe_ckpt_error()
    try:
        assert lib.mmoe_ckpt_load(20, 2) == 0, lib.mmoe_ckpt_error()
        for L in (20, 21):
            tab = (O.Expert * NE)()
            for e in range(NE):
                tab[e] = O.Expert(*[a.ctypes.data for a in info["experts"][distinct(L, e, 6)]])
            for nb in (1, 64):
                x, hn = normed_hidden(SEED, 300 + nb + L, nb)
                xg = x.copy()
                M.check(lib.mmoe_moe(L, M.ptr(hn), nb, M.ptr(xg), M.ORDER_BATCH), "mmoe_moe")
                xo = x.copy()
                o = O.moe_batch(hn, info["routers"][L % 2], tab, xo)
                top = M.read("TOP", (nb, 8), np.int32)
                assert np.array_equal(top, o["top"].reshape(nb, 8))
                assert relmax(xg - x, xo - x) <= 1e-5
                print(f"\n  layer {L} nb={nb}: x bit-exact {np.array_equal(xg, xo)}")
    finally:
        lib.mmoe_ckpt_close()
