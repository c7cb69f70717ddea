"""The oracle against golden vectors produced by maple.c itself (tests/golden/make_fixtures.py, from
oracle/_ref). Runs anywhere: inputs are regenerated from the seeds and checked by checksum first."""
import hashlib
import os

import numpy as np
import pytest

import maplemoe as M
import pyoracle as O
from helpers import HostLayer, normed_hidden, relmax

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "maple_moe_fixtures.npz")


def sha(a):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest(), np.uint8)


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX, allow_pickle=False) as z:
        d = {k: z[k] for k in z.files}
    seed, L, nb = (int(v) for v in d["seed"])
    hl = HostLayer(seed, L)
    assert np.array_equal(sha(hl.blk), d["sha_block"]) and np.array_equal(sha(hl.router), d["sha_router"]), \
        "synthetic generator no longer reproduces the fixture's inputs"
    return d, hl, seed, nb


def test_prep_vectors(fx):
    d = fx[0]
    for i in range(len(d["p_x"])):
        q, qs, s = O.prep(d["p_x"][i])
        assert np.array_equal(q, d["p_q"][i]) and np.float32(qs) == d["p_qs"][i] and s == d["p_qsum"][i]


def test_moe_batch_fixture(fx):
    d, hl, seed, nb = fx
    x, hn = normed_hidden(seed, 1, nb)
    assert np.array_equal(sha(hn), d["b_sha_hn"])
    xo = x.copy()
    o = O.moe_batch(hn, hl.router, hl.table, xo)
    nu = len(d["b_ue"])
    assert np.array_equal(o["rl"].view(np.int32), d["b_rl"].view(np.int32))   # router order: bit-exact
    assert np.array_equal(o["top"], d["b_top"])                                 # top-8 indices
    assert relmax(o["tw"], d["b_tw"]) < 1e-6
    assert int(o["nu"][0]) == nu and np.array_equal(o["ue"][:nu], d["b_ue"]) and np.array_equal(o["ustart"][:nu + 1], d["b_ustart"])
    assert np.array_equal(o["utok"], d["b_utok"]) and relmax(o["uw"], d["b_uw"]) < 1e-6
    assert relmax(o["gate"], d["b_gate"]) < 1e-6 and relmax(o["act"], d["b_act"]) < 1e-6
    assert np.array_equal(o["qa"], d["b_qa"])          # no rounding-boundary flips in this fixture
    assert relmax(o["qsa"], d["b_qsa"]) < 1e-6
    assert relmax(o["down"][:8], d["b_down8"]) < 1e-5
    assert relmax(xo - x, d["b_xout"] - x) < 1e-5


def test_moe_step_fixture(fx):
    d, hl, seed, _ = fx
    x, hn = normed_hidden(seed, 2, 1)
    assert np.array_equal(sha(hn), d["s_sha_hn"])
    xo = x[0].copy()
    o = O.moe_step(hn[0], hl.router, hl.table, xo)
    assert np.array_equal(o["rl"].ravel().view(np.int32), d["s_rl"].view(np.int32))
    assert np.array_equal(o["top"].ravel(), d["s_top"])
    assert relmax(o["tw"].ravel(), d["s_tw"]) < 1e-6 and relmax(o["act"], d["s_act"]) < 1e-6
    assert relmax(xo - x[0], d["s_xout"] - x[0]) < 1e-5
