"""The oracle's whole MoE block against maple.c's own (oracle/_ref) on a synthetic Maple-shaped layer:
step_batch (maple.c:733-834) and step (maple.c:605-665). Integer stages bit-exact; fp32 within 1e-5."""
import numpy as np
import pytest

import pyoracle as O
from helpers import SEED, HostLayer, normed_hidden, relmax

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref absent")


@pytest.fixture(scope="module")
def layer():
    hl = HostLayer(SEED, 2)
    if O.ref_available():
        import maplemoe as M
        R = O.ref(); R.ref_set_threads(1)
        R.ref_set_router(2, O._p(hl.router))
        for e in range(256):
            R.ref_set_expert(2, e, *[O._p(a) for a in M.expert_views(hl.blk, e)])
    return hl


@needs_ref
@pytest.mark.parametrize("nb", [1, 9, 48])
def test_moe_batch_vs_maple(layer, nb):
    x, hn = normed_hidden(SEED, 50 + nb, nb)
    P = nb * 8
    xr = x.copy()
    arr = {k: np.zeros(s, d) for k, s, d in [("rl", (nb, 256), np.float32), ("top", (nb, 8), np.int32), ("tw", (nb, 8), np.float32),
                                              ("nu", 1, np.int32), ("ue", 256, np.int32), ("us", 257, np.int32), ("ut", P, np.int32),
                                              ("uw", P, np.float32), ("G", (P, 512), np.float32), ("U", (P, 512), np.float32),
                                              ("A", (P, 512), np.float32), ("qa", (P, 512), np.int8), ("qsa", P, np.float32),
                                              ("D", (P, 2048), np.float32)]}
    O.ref().ref_moe_batch(2, O._p(hn), nb, O._p(xr), *[O._p(arr[k]) for k in ("rl", "top", "tw", "nu", "ue", "us", "ut", "uw", "G", "U", "A", "qa", "qsa", "D")])
    xo = x.copy()
    o = O.moe_batch(hn, layer.router, layer.table, xo)
    nu = int(arr["nu"][0])
    assert np.array_equal(arr["rl"].view(np.int32), o["rl"].view(np.int32))
    assert np.array_equal(arr["top"], o["top"])
    assert relmax(o["tw"], arr["tw"]) < 1e-6
    assert nu == int(o["nu"][0]) and np.array_equal(arr["ue"][:nu], o["ue"][:nu]) and np.array_equal(arr["us"][:nu + 1], o["ustart"][:nu + 1])
    assert np.array_equal(arr["ut"], o["utok"])
    assert relmax(o["gate"], arr["G"]) < 1e-6 and relmax(o["up"], arr["U"]) < 1e-6
    assert relmax(o["act"], arr["A"]) < 1e-6
    # maple.c's fast-math SiLU (libmvec expf, rcp + Newton) differs from IEEE by a few ulp, which moves a rare
    # re-quantised act value across a rounding boundary (|dq| = 1). Pairs without such a flip match to 1e-5;
    # tokens of flipped pairs differ by about one quantisation step of that pair.
    fl = (o["qa"] != arr["qa"])
    assert np.abs(o["qa"].astype(int) - arr["qa"].astype(int)).max() <= 1
    bad_pairs = np.nonzero(fl.any(1))[0]
    assert len(bad_pairs) <= max(1, P // 50), len(bad_pairs)
    ok = np.setdiff1d(np.arange(P), bad_pairs)
    assert relmax(o["down"][ok], arr["D"][ok]) < 1e-5
    bad_tok = np.unique(arr["ut"][bad_pairs])
    good_tok = np.setdiff1d(np.arange(nb), bad_tok)
    assert relmax((xo - x)[good_tok], (xr - x)[good_tok]) < 1e-5
    if len(bad_tok):
        assert relmax((xo - x)[bad_tok], (xr - x)[bad_tok]) < 1e-3
    print(f"\n  nb={nb}: {int(fl.sum())} act int8 values differ by 1 (fast-math SiLU) in {len(bad_pairs)} of {P} pairs")


@needs_ref
def test_moe_step_vs_maple(layer):
    x, hn = normed_hidden(SEED, 70, 1)
    xr = x[0].copy(); rl = np.zeros(256, np.float32); top = np.zeros(8, np.int32); tw = np.zeros(8, np.float32)
    act = np.zeros((8, 512), np.float32); down = np.zeros((8, 2048), np.float32)
    O.ref().ref_moe_step(2, O._p(hn[0]), O._p(xr), O._p(rl), O._p(top), O._p(tw), O._p(act), O._p(down))
    xo = x[0].copy()
    o = O.moe_step(hn[0], layer.router, layer.table, xo)
    assert np.array_equal(rl.view(np.int32), o["rl"].ravel().view(np.int32))
    assert np.array_equal(top, o["top"].ravel())
    assert relmax(o["act"], act) < 1e-6 and relmax(o["down"], down) < 1e-5
    assert relmax(xo - x[0], xr - x[0]) < 1e-5
