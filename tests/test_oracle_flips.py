"""Where the oracle (and so the GPU path, which matches it bit for bit) and maple.c's own build part ways, and
why that is benign. maple.c's -ffast-math build evaluates SiLU with libmvec expf and a reciprocal estimate
refined by Newton; the oracle uses IEEE division and its own exp. The act values then differ by a few ulp, and the
pair's absmax (so inv = 127 / max) by at most one. Re-quantising act (maple.c:832 prep) rounds act * inv to an
int8; a value within a few ulp of k + 0.5 can round to k on one side and k + 1 on the other. Every such flip is
shown to be that case: both pre-rounding values lie within a few ulp of the same half-integer.

Reported (printed) at BASELINE configs 0 (128 tokens) and 2 (2048 tokens, Zipf(1.1)-biased router): the flip
rate and the whole-batch relmax of the hidden state against maple.c. Config 2 runs maple.c on all 2048 tokens
and the oracle on a sample of them (a token's result depends only on that token)."""
import numpy as np
import pytest

import maplemoe as M
import pyoracle as O
from helpers import SEED, HostLayer, normed_hidden, relmax

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref absent")
ULP_TOL = 16      # pre-rounding values within this many ulp of the half-integer they straddle


def ref_batch(L, hn, x, bias=None):
    nb = hn.shape[0]; P = nb * 8
    a = {k: np.zeros(s, d) for k, s, d in [("rl", (nb, 256), np.float32), ("top", (nb, 8), np.int32), ("tw", (nb, 8), np.float32),
                                            ("nu", 1, np.int32), ("ue", 256, np.int32), ("us", 257, np.int32), ("ut", P, np.int32),
                                            ("uw", P, np.float32), ("A", (P, 512), np.float32), ("qa", (P, 512), np.int8),
                                            ("qsa", P, np.float32)]}
    R = O.ref()
    R.ref_set_bias(O._p(bias))
    try:
        R.ref_moe_batch(L, O._p(hn), nb, O._p(x), *[O._p(a[k]) for k in ("rl", "top", "tw", "nu", "ue", "us", "ut", "uw")],
                        None, None, O._p(a["A"]), O._p(a["qa"]), O._p(a["qsa"]), None)
    finally:
        R.ref_set_bias(None)
    return a


def pre_round(act):
    """act * inv of maple.c's prep under its build flags (inv = 127 / max|act|, both fp32), per pair row"""
    mx = np.abs(act).max(1, keepdims=True).astype(np.float32)
    inv = np.where(mx > 0, np.float32(127.0) / np.where(mx > 0, mx, 1), np.float32(1.0)).astype(np.float32)
    return (act * inv).astype(np.float32)


def check_flips(act_r, qa_r, act_o, qa_o):
    """every differing int8 is a near-tie: returns the count and the largest distance (in ulp) of a pre-rounding
    value from the half-integer the two sides straddle"""
    vr, vo = pre_round(act_r), pre_round(act_o)
    assert np.array_equal(np.rint(vr).astype(np.int8), qa_r) and np.array_equal(np.rint(vo).astype(np.int8), qa_o)
    d = qa_r.astype(np.int32) - qa_o.astype(np.int32)
    assert np.abs(d).max() <= 1
    idx = np.nonzero(d)
    if not len(idx[0]):
        return 0, 0.0
    m = (qa_r[idx].astype(np.float64) + qa_o[idx]) / 2              # the half-integer between the two results
    ulp = np.spacing(np.abs(m).astype(np.float32)).astype(np.float64)
    dist = np.maximum(np.abs(vr[idx] - m), np.abs(vo[idx] - m)) / ulp
    assert (np.abs(m - np.floor(m)) == 0.5).all()
    assert dist.max() <= ULP_TOL, dist.max()
    return len(idx[0]), float(dist.max())


@pytest.fixture(scope="module")
def layer():
    if not O.ref_available():
        pytest.skip("oracle/_ref absent")
    hl = HostLayer(SEED, 0)
    R = O.ref(); R.ref_set_threads(8)
    R.ref_set_router(0, O._p(hl.router))
    for e in range(256):
        R.ref_set_expert(0, e, *[O._p(a) for a in M.expert_views(hl.blk, e)])
    return hl


@needs_ref
def test_config0_flips_are_rounding_ties(layer):
    nb = 128
    x, hn = normed_hidden(SEED, 1128, nb)
    xr = x.copy()
    a = ref_batch(0, hn, xr)
    xo = x.copy()
    o = O.moe_batch(hn, layer.router, layer.table, xo, want=("top", "utok", "act", "qa", "qsa"))
    assert np.array_equal(a["top"], o["top"]) and np.array_equal(a["ut"], o["utok"])
    n, dmax = check_flips(a["A"], a["qa"], o["act"], o["qa"])
    P = nb * 8
    print(f"\n  config 0: {n} act int8 flips in {P * 512} values ({n / (P * 512):.1e}), farthest {dmax:.1f} ulp from "
          f"its half-integer; x relmax vs maple.c {relmax(xo - x, xr - x):.1e}")
    assert n >= 1     # this input holds a flip (the case the check is about)


@needs_ref
def test_config2_flips_are_rounding_ties(layer):
    T = 2048
    zb = M.zipf_bias(SEED, 1.1)
    x, hn = normed_hidden(SEED, 1129, T)
    xr = x.copy()
    a = ref_batch(0, hn, xr, zb)
    rng = np.random.default_rng(3)
    sample = np.sort(rng.choice(T, 128, replace=False))
    xo = x[sample].copy()
    o = O.moe_batch(hn[sample], layer.router, layer.table, xo, bias=zb, want=("rl", "top", "utok", "act", "qa"))
    assert np.array_equal(a["top"][sample], o["top"])
    # maple.c's pairs of the sampled tokens, in the oracle's grouped order (experts ascending, then tokens)
    pr = np.nonzero(np.isin(a["ut"], sample))[0]
    assert len(pr) == len(o["utok"]) and np.array_equal(sample[o["utok"]], a["ut"][pr])
    n, dmax = check_flips(a["A"][pr], a["qa"][pr], o["act"], o["qa"])
    e = relmax(xo - x[sample], xr[sample] - x[sample])
    print(f"\n  config 2 (sample of 128 of 2048 tokens): {n} act int8 flips in {len(pr) * 512} values, farthest "
          f"{dmax:.1f} ulp; x relmax vs maple.c {e:.1e}")
