"""mmoe_route: maple.c's job_topk + group_pairs (maple.c:910-938) and the tp table of its callers (maple.c:762,
1019) on the device, against the oracle's restatement (mo_topk / mo_group) bit for bit."""
import numpy as np
import pytest

import maplemoe as M
import pyoracle as O

pytestmark = pytest.mark.gpu


def route_gpu(rl):
    lib = M.lib()
    nb = rl.shape[0]; P = nb * 8
    top = np.full((nb, 8), -1, np.int32); tw = np.zeros((nb, 8), np.float32)
    ue = np.full(256, -1, np.int32); us = np.full(257, -1, np.int32)
    utok = np.full(P, -1, np.int32); uw = np.zeros(P, np.float32); tp = np.full((nb, 8), -1, np.int32)
    nu = lib.mmoe_route(M.ptr(np.ascontiguousarray(rl, np.float32)), nb, M.ptr(top), M.ptr(tw), M.ptr(ue), M.ptr(us),
                        M.ptr(utok), M.ptr(uw), M.ptr(tp))
    assert nu > 0, lib.mmoe_last_error()
    return dict(nu=nu, top=top, tw=tw, ue=ue[:nu], ustart=us[:nu + 1], utok=utok, uw=uw, tp=tp)


def check_route(rl):
    g = route_gpu(rl)
    top, tw = O.topk(rl)
    o = O.group(top, tw)
    assert np.array_equal(g["top"], top), "top-8 indices"
    assert np.array_equal(g["tw"].view(np.int32), tw.view(np.int32)), "top-8 weights"
    assert g["nu"] == o["nu"] and np.array_equal(g["ue"], o["ue"]) and np.array_equal(g["ustart"], o["ustart"]), "used experts"
    assert np.array_equal(g["utok"], o["utok"]) and np.array_equal(g["uw"].view(np.int32), o["uw"].view(np.int32)), "pairs"
    assert np.array_equal(g["tp"], o["tp"]), "tp"
    return g


@pytest.fixture(scope="module")
def ctx():
    M.check(M.lib().mmoe_init(2048), "mmoe_init")


@pytest.mark.parametrize("nb", [1, 5, 64, 65, 300, 2048])
def test_route_random_logits(ctx, nb):
    rl = np.random.default_rng(100 + nb).standard_normal((nb, 256)).astype(np.float32) * 0.5
    g = check_route(rl)
    print(f"\n  nb={nb}: {g['nu']} experts used, pairs {g['ustart'][-1]}")


def test_route_ties_and_skew(ctx):
    """Logits on a coarse grid (large tie classes, so maple.c's strict-> order decides), a Zipf-like skew that
    sends most tokens to a few experts, and rows where every logit is equal."""
    rng = np.random.default_rng(7)
    nb = 700
    rl = np.round(rng.standard_normal((nb, 256)) * 2.0).astype(np.float32) / 4.0
    rl[: nb // 2] += (3.0 / (1.0 + np.arange(256)) ** 1.1).astype(np.float32) * 8.0
    rl[-5:] = 0.0
    g = check_route(rl)
    assert (g["top"][-1] == np.arange(8)).all(), "all-equal row: experts 0..7 in order"


def test_route_null_outputs_and_limits(ctx):
    lib = M.lib()
    rl = np.random.default_rng(3).standard_normal((40, 256)).astype(np.float32)
    top = np.full((40, 8), -1, np.int32)
    nu = lib.mmoe_route(M.ptr(rl), 40, M.ptr(top), None, None, None, None, None, None)
    assert nu > 0 and np.array_equal(top, O.topk(rl)[0])
    assert lib.mmoe_route(M.ptr(rl), 0, None, None, None, None, None, None, None) == -1 and b"nb" in lib.mmoe_last_error()
    assert lib.mmoe_route(M.ptr(rl), 4096, None, None, None, None, None, None, None) == -1
    # no logits: the ones the call above uploaded stay on the device (40 tokens), none of 41
    assert lib.mmoe_route(None, 40, None, None, None, None, None, None, None) == nu
    assert lib.mmoe_route(None, 41, None, None, None, None, None, None, None) == -1


def test_route_between_layer_calls(ctx):
    """The routing's per-chunk counts are cleared by each call: a route after a whole-layer call and a second
    route of other logits still give the oracle's grouping."""
    from helpers import SEED, HostLayer, normed_hidden
    lib = M.lib()
    hl = HostLayer(SEED, 3)
    M.register_layer(3, hl.blk, hl.router)
    x, hn = normed_hidden(SEED, 55, 200)
    M.check(lib.mmoe_moe(3, M.ptr(hn), 200, M.ptr(x), M.ORDER_BATCH), "moe")
    for s in (11, 12):
        check_route(np.random.default_rng(s).standard_normal((257, 256)).astype(np.float32))


def route_dev(nb):
    """mmoe_route on the logits the last router call left on the device (rl = NULL)"""
    lib = M.lib()
    P = nb * 8
    top = np.full((nb, 8), -1, np.int32); tw = np.zeros((nb, 8), np.float32)
    ue = np.full(256, -1, np.int32); us = np.full(257, -1, np.int32)
    utok = np.full(P, -1, np.int32); uw = np.zeros(P, np.float32); tp = np.full((nb, 8), -1, np.int32)
    nu = lib.mmoe_route(None, nb, M.ptr(top), M.ptr(tw), M.ptr(ue), M.ptr(us), M.ptr(utok), M.ptr(uw), M.ptr(tp))
    return nu, dict(top=top, tw=tw, ue=ue[:max(nu, 0)], ustart=us[:max(nu, 0) + 1], utok=utok, uw=uw, tp=tp)


@pytest.mark.parametrize("nb", [1, 300])
def test_route_on_device_logits(ctx, nb):
    """rl = NULL: the routing of the logits a whole-layer call just computed on the device (the decode router at
    one token, the chain router below 512 tokens), without a host copy; equal to the oracle's routing of those
    logits and to the layer call's own top-8."""
    from helpers import SEED, HostLayer, normed_hidden
    lib = M.lib()
    hl = HostLayer(SEED, 4)
    M.register_layer(4, hl.blk, hl.router)
    x, hn = normed_hidden(SEED, 60 + nb, nb)
    M.check(lib.mmoe_moe(4, M.ptr(hn), nb, M.ptr(x), M.ORDER_BATCH), "moe")
    rl = M.read("LOGITS", (nb, 256), np.float32)
    top_layer = M.read("TOP", (nb, 8), np.int32)
    nu, g = route_dev(nb)
    assert nu > 0, lib.mmoe_last_error()
    top, tw = O.topk(rl)
    o = O.group(top, tw)
    assert np.array_equal(g["top"], top) and np.array_equal(g["top"], top_layer)
    assert np.array_equal(g["tw"].view(np.int32), tw.view(np.int32))
    assert nu == o["nu"] and np.array_equal(g["ue"], o["ue"]) and np.array_equal(g["ustart"], o["ustart"])
    assert np.array_equal(g["utok"], o["utok"]) and np.array_equal(g["uw"].view(np.int32), o["uw"].view(np.int32))
    assert np.array_equal(g["tp"], o["tp"])
    # another token count than the router call covered is refused
    assert route_dev(nb + 1)[0] == -1 and b"last router call" in lib.mmoe_last_error()


def test_route_device_logits_refused_after_mfma_router(ctx):
    """The default router of a 1024-token batch leaves approximate logits for the experts that cannot reach the
    top 8: rl = NULL is refused then, and accepted after the same call with the exact router option."""
    from helpers import SEED, HostLayer, normed_hidden
    lib = M.lib()
    hl = HostLayer(SEED, 5)
    M.register_layer(5, hl.blk, hl.router)
    nb = 1024
    x, hn = normed_hidden(SEED, 70, nb)
    xa = x.copy()   # held: the library writes through the pointer
    M.check(lib.mmoe_moe(5, M.ptr(hn), nb, M.ptr(xa), M.ORDER_BATCH), "moe")
    assert route_dev(nb)[0] == -1
    M.check(lib.mmoe_set_router_mode(1), "router mode")
    try:
        xb = x.copy()
        M.check(lib.mmoe_moe(5, M.ptr(hn), nb, M.ptr(xb), M.ORDER_BATCH), "moe")
        rl = M.read("LOGITS", (nb, 256), np.float32)
        nu, g = route_dev(nb)
        assert nu > 0 and np.array_equal(g["top"], O.topk(rl)[0])
    finally:
        M.check(lib.mmoe_set_router_mode(0), "router mode")
