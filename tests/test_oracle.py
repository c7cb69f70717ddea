"""Pins the C oracle (oracle/moe_oracle.c): against maple.c itself (oracle/_ref, built from /root/reference),
against closed forms and brute force, and against the committed golden fixtures (tests/test_golden.py).

Every check is chosen so that a plausible slip (wrong bit shift, dropped qsum term, transposed operand,
wrong summation lane, off-by-one tie-break) fails it."""
import math

import numpy as np
import pytest

import maplemoe as M
import pyoracle as O
from helpers import SEED, relmax

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref (maple.c built from /root/reference) absent")
rng = np.random.default_rng(12345)


def ulps(a, b):
    """|a - b| in units of the fp32 spacing at max(|a|, |b|) (sign-safe around zero)"""
    a = np.asarray(a, np.float32); b = np.asarray(b, np.float32)
    m = np.maximum(np.abs(a), np.abs(b)).astype(np.float32)
    sp = np.spacing(np.maximum(m, np.float32(np.finfo(np.float32).tiny))).astype(np.float64)
    return np.abs(a.astype(np.float64) - b.astype(np.float64)) / sp


# ------------------------------------------------------------------ a1 packed layout (convert.py:23-40)
def test_pack_layout_closed_form():
    # one nonzero code per position: column 37 of group 1 must land in byte 32+5 (group 1, j = 37-32 = 5) at bits 2..3
    codes = np.ones((1, 256), np.uint8)
    codes[0, 128 + 37] = 2
    packed = np.zeros((1, 64), np.uint8)
    O.oracle().mo_pack(O._p(codes), 1, 256, O._p(packed))
    expect = np.full(64, 0b01010101, np.uint8)
    expect[32 + 5] = 0b01011001
    assert np.array_equal(packed[0], expect)


def test_pack_unpack_roundtrip():
    codes = rng.integers(0, 3, size=(7, 512)).astype(np.uint8)
    packed = np.zeros((7, 128), np.uint8); back = np.zeros_like(codes)
    O.oracle().mo_pack(O._p(codes), 7, 512, O._p(packed))
    O.oracle().mo_unpack(O._p(packed), 7, 512, O._p(back))
    assert np.array_equal(codes, back)


def test_synth_codes_are_ternary_with_the_configured_mix():
    blk = M.page_aligned(M.EXPERT_BYTES)
    gc, gs, uc, us, dc, ds = (np.empty(s, d) for s, d in [((512, 512), np.uint8), (512, np.float32), ((512, 512), np.uint8),
                                                          (512, np.float32), ((2048, 128), np.uint8), (2048, np.float32)])
    M.slib().mmoe_synth_expert(SEED, 0, 5, *[M.ptr(a) for a in (gc, gs, uc, us, dc, ds)])
    codes = np.zeros((512, 2048), np.uint8)
    O.oracle().mo_unpack(O._p(gc), 512, 2048, O._p(codes))
    frac = np.bincount(codes.ravel(), minlength=4) / codes.size
    assert frac[3] == 0 and abs(frac[0] - 0.3) < 0.003 and abs(frac[1] - 0.4) < 0.003 and abs(frac[2] - 0.3) < 0.003
    assert gs.min() >= 0.01 and gs.max() <= 0.05 and ds.min() >= 0.01 and ds.max() <= 0.05


# ------------------------------------------------------------------ a3 prep, a7/a9 integer dots
def test_dot_i32_brute_force():
    rows, cols = 9, 2048
    codes = rng.integers(0, 3, size=(rows, cols)).astype(np.uint8)
    packed = np.zeros((rows, cols // 4), np.uint8)
    O.oracle().mo_pack(O._p(codes), rows, cols, O._p(packed))
    q = rng.integers(-127, 128, size=cols).astype(np.int8)
    w = codes.astype(np.int64) - 1                      # ternary weights
    for r in range(rows):
        tot = O.oracle().mo_dot_i32(O._p(packed[r]), O._p(q), cols)
        assert tot - int(q.astype(np.int64).sum()) == int(w[r] @ q.astype(np.int64))


def test_prep_special_cases():
    q, qs, s = O.prep(np.zeros(512, np.float32))
    assert qs == 1.0 and s == 0 and not q.any()           # maple.c:187: qs = 1 when max is 0
    x = np.zeros(2048, np.float32); x[10] = -3.0
    q, qs, s = O.prep(x)
    assert q[10] == -127 and s == -127 and qs == np.float32(3.0) * np.float32(1.0 / 127.0)
    # round half to even: with max 127, x*inv = x; 2.5 -> 2, 3.5 -> 4, -0.5 -> 0
    x = np.zeros(128, np.float32); x[0] = 127.0; x[1:4] = [2.5, 3.5, -0.5]
    q, qs, s = O.prep(x)
    assert list(q[:4]) == [127, 2, 4, 0]


@needs_ref
def test_prep_bit_exact_vs_maple():
    R = O.ref()
    for i in range(3000):
        n = 2048 if i % 2 else 512
        scale = 10.0 ** rng.uniform(-4, 3)
        x = (rng.standard_normal(n) * scale).astype(np.float32)
        if i % 7 == 0:
            x[rng.integers(0, n, 20)] = 0.0
        q1, qs1, s1 = O.prep(x)
        q2 = np.empty(n, np.int8); s2 = np.zeros(1, np.int32)
        qs2 = R.ref_prep(O._p(x), n, O._p(q2), O._p(s2))
        assert np.array_equal(q1, q2) and np.float32(qs1) == np.float32(qs2) and s1 == int(s2[0]), i


@needs_ref
def test_dot_i32_bit_exact_vs_maple():
    rows, cols, nv = 33, 2048, 70   # nv > 64 exercises tdot_multi's blocking
    codes = rng.integers(0, 3, size=(rows, cols)).astype(np.uint8)
    packed = np.zeros((rows, cols // 4), np.uint8)
    O.oracle().mo_pack(O._p(codes), rows, cols, O._p(packed))
    q = rng.integers(-127, 128, size=(nv, cols)).astype(np.int8)
    out = np.zeros((nv, rows), np.int32)
    O.ref().ref_dot_i32(O._p(packed), rows, cols, O._p(q), nv, O._p(out))
    mine = np.array([[O.oracle().mo_dot_i32(O._p(packed[r]), O._p(q[i]), cols) for r in range(rows)] for i in range(nv)])
    assert np.array_equal(out, mine)


# ------------------------------------------------------------------ a4 router logits
@pytest.fixture(scope="module")
def router():
    return M.synth_router(SEED, 3)


@needs_ref
@pytest.mark.parametrize("nb", [5, 40])
def test_router_batch_bit_exact_vs_maple(router, nb):
    R = O.ref(); R.ref_set_router(0, O._p(router))
    hn = rng.standard_normal((nb, 2048)).astype(np.float32)
    rl = np.zeros((nb, 256), np.float32)
    R.ref_route_batch(0, O._p(hn), nb, O._p(rl))
    mine = O.router_batch(hn, router)
    assert np.array_equal(rl.view(np.int32), mine.view(np.int32))


@needs_ref
def test_router_step_bit_exact_vs_maple(router):
    R = O.ref(); R.ref_set_router(0, O._p(router))
    hn = rng.standard_normal(2048).astype(np.float32)
    rl = np.zeros(256, np.float32)
    R.ref_route_step(0, O._p(hn), O._p(rl))
    assert np.array_equal(rl.view(np.int32), O.router_step(hn, router).view(np.int32))


def test_router_orders_vs_fp64(router):
    hn = rng.standard_normal((3, 2048)).astype(np.float32)
    w = (router.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    exact = hn.astype(np.float64) @ w.T
    assert relmax(O.router_batch(hn, router), exact) < 1e-6
    assert relmax(O.router_step(hn[0], router), exact[0]) < 1e-6
    # the two orders are genuinely different summations (not the same code path)
    b = O.router_batch(hn[:1], router)[0]; s = O.router_step(hn[0], router)
    assert not np.array_equal(b, s)


# ------------------------------------------------------------------ exp, a5 softmax/top-8
def test_exp_against_libm():
    xs = np.concatenate([np.linspace(-104, 88, 200001), rng.uniform(-20, 20, 100000)]).astype(np.float32)
    f = np.vectorize(lambda v: O.oracle().mo_exp(float(v)), otypes=[np.float32])(xs[::7])
    ref = np.array([np.float32(math.exp(float(v))) for v in xs[::7]], np.float32)
    fin = np.isfinite(ref) & (ref > 0)
    assert np.array_equal(f[~fin], ref[~fin])
    d = ulps(f[fin], ref[fin])
    assert d.max() <= 1 and (d > 0).mean() < 0.1  # faithful: within 1 ulp, mostly correctly rounded
    assert O.oracle().mo_exp(0.0) == 1.0 and O.oracle().mo_exp(-200.0) == 0.0 and math.isinf(O.oracle().mo_exp(200.0))


def test_topk_closed_forms():
    rl = np.zeros((2, 256), np.float32)
    rl[0, [200, 7, 100, 3]] = [4.0, 3.0, 2.0, 1.0]           # then ties at 0: lowest indices 0,1,2,4
    rl[1, :] = 1.0                                            # all tied: experts 0..7, equal weights
    top, tw = O.topk(rl)
    assert list(top[0]) == [200, 7, 100, 3, 0, 1, 2, 4]
    assert list(top[1]) == list(range(8)) and np.allclose(tw[1], 0.125, rtol=0, atol=1e-7)
    e = np.exp(np.array([4.0, 3.0, 2.0, 1.0, 0, 0, 0, 0]))
    assert relmax(tw[0], e / e.sum()) < 1e-6


def test_topk_invariants(router):
    rl = (rng.standard_normal((200, 256)) * 2).astype(np.float32)
    top, tw = O.topk(rl)
    for b in range(200):
        assert len(set(top[b])) == 8
        assert np.array_equal(top[b], np.argsort(-rl[b].astype(np.float64), kind="stable")[:8])
        assert abs(float(tw[b].astype(np.float64).sum()) - 1.0) < 1e-6 and np.all(np.diff(tw[b]) <= 0)


@needs_ref
def test_topk_vs_maple():
    rl = (rng.standard_normal((500, 256)) * 1.5).astype(np.float32)
    top = np.zeros((500, 8), np.int32); tw = np.zeros((500, 8), np.float32)
    O.ref().ref_topk(O._p(rl), 500, O._p(top), O._p(tw))
    t2, w2 = O.topk(rl)
    assert np.array_equal(top, t2)
    assert ulps(tw, w2).max() <= 8 and relmax(w2, tw) < 1e-6


# ------------------------------------------------------------------ a6 grouping
@needs_ref
def test_group_vs_maple_and_invariants():
    nb = 300
    top = np.stack([rng.choice(256, 8, replace=False) for _ in range(nb)]).astype(np.int32)
    top[:, :4] = np.sort(rng.choice(16, (nb, 4)), 1)  # crowd a few experts
    top = np.stack([np.array(list(dict.fromkeys(list(t) + list(rng.permutation(256))))[:8]) for t in top]).astype(np.int32)
    tw = rng.random((nb, 8)).astype(np.float32)
    g = O.group(top, tw)
    nu = np.zeros(1, np.int32); ue = np.zeros(256, np.int32); us = np.zeros(257, np.int32)
    ut = np.zeros(nb * 8, np.int32); uw = np.zeros(nb * 8, np.float32); tp = np.zeros(nb * 8, np.int32)
    O.ref().ref_group(O._p(top), O._p(tw), nb, O._p(nu), O._p(ue), O._p(us), O._p(ut), O._p(uw), O._p(tp))
    n = int(nu[0])
    assert n == g["nu"] and np.array_equal(ue[:n], g["ue"]) and np.array_equal(us[:n + 1], g["ustart"])
    assert np.array_equal(ut, g["utok"]) and np.array_equal(uw, g["uw"]) and np.array_equal(tp.reshape(nb, 8), g["tp"])
    # invariants: a stable counting sort
    cnt = np.bincount(top.ravel(), minlength=256)
    assert np.array_equal(g["ue"], np.nonzero(cnt)[0]) and np.array_equal(np.diff(g["ustart"]), cnt[cnt > 0])
    assert np.all(np.bincount(g["utok"], minlength=nb) == 8)
    for u in range(n):
        seg = g["utok"][g["ustart"][u]:g["ustart"][u + 1]]
        assert np.all(np.diff(seg) > 0)
    assert np.all(np.diff(g["tp"], axis=1) > 0)
    for b in range(nb):
        assert set(g["ue"][np.searchsorted(g["ustart"], g["tp"][b], side="right") - 1]) == set(top[b])


# ------------------------------------------------------------------ a8 act, a2 rmsnorm
@needs_ref
def test_act_vs_maple():
    G = (rng.standard_normal(200000) * 4).astype(np.float32); U = (rng.standard_normal(200000) * 4).astype(np.float32)
    G[:6] = [100, -100, 7, 7.5, -88, 0]; U[:6] = [100, -100, -8, 3, 1, 5]
    a1 = np.zeros_like(G); a2 = np.zeros_like(G)
    O.oracle().mo_act(O._p(G), O._p(U), O._p(a1), G.size)
    O.ref().ref_act(O._p(G), O._p(U), O._p(a2), G.size)
    # maple.c's -ffast-math build computes g / (1 + expf(-g)) as g * rcp-Newton(1 + expf(-g)); for g < -88.7 expf
    # overflows to inf and the Newton step turns rcp(inf) = 0 into NaN. The source's arithmetic (and the
    # oracle, and the GPU) give -0 there. Those inputs are checked separately.
    over = G < -88.7
    assert np.isnan(a2[over]).all() and (a1[over] == 0).all()
    # maple.c runs with flush-to-zero, so results below 1e-30 (g near -80) may be flushed there
    norm = ~over & (np.abs(a1) > 1e-30)
    assert relmax(a1[~over], a2[~over]) < 1e-5 and ulps(a1[norm], a2[norm]).max() <= 8
    # closed form: g = min(G, 7), u = clamp(U, +-7): G=100,U=100 -> 7/(1+e^-7)*7
    assert abs(a1[0] - 7.0 / (1.0 + math.exp(-7.0)) * 7.0) < 1e-5 and a1[5] == 0.0


@needs_ref
def test_rmsnorm_vs_maple():
    x = (rng.standard_normal(2048) * 3).astype(np.float32)
    w = M.synth_router(SEED, 0)[0]
    o1 = np.zeros_like(x); o2 = np.zeros_like(x)
    O.oracle().mo_rmsnorm(O._p(x), O._p(w), 2048, O._p(o1))
    O.ref().ref_rmsnorm(O._p(x), O._p(w), 2048, O._p(o2))
    assert ulps(o1, o2).max() <= 2
    wf = (w.astype(np.uint32) << 16).view(np.float32)
    exact = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-6) * wf
    assert relmax(o1, exact) < 1e-6
