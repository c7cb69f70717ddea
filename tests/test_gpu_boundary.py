"""Entry points of maple.c's boundary and library state that the main parity tests do not reach:
- gpux_begin_multi / gpux_end_multi, driven the way maple.c's step_batch decode does (maple.c:788-812):
  the cached subset of the used experts, pair runs pstart over tokens ptok, per-pair down outputs;
- every setter drops a captured HIP graph (a replay would otherwise run stale kernels or freed buffers);
- mmoe_gfull_post_norm / gfull_attn return exact chain logits in either router mode."""
import ctypes as C

import numpy as np
import pytest

import maplemoe as M
import pyoracle as O
from helpers import SEED, HostLayer, normed_hidden, relmax

pytestmark = pytest.mark.gpu
TOL = 1e-5


@pytest.fixture(scope="module")
def layer7():
    lib = M.lib()
    M.check(lib.mmoe_init(2048), "mmoe_init")
    hl = HostLayer(SEED, 7)
    hl.rid = M.register_layer(7, hl.blk, hl.router)
    return hl


@pytest.mark.parametrize("nb", [2, 9, 16])
def test_gpux_multi_as_maple_step_batch(layer7, nb):
    lib = M.lib()
    x, hn = normed_hidden(SEED, 500 + nb, nb)
    xo = x.copy()
    o = O.moe_batch(hn, layer7.router, layer7.table, xo, want=("top", "tw", "nu", "ue", "ustart", "utok", "uw", "down"))
    nu, ue, ustart, utok = o["nu"][0], o["ue"], o["ustart"], o["utok"]
    # the card holds every other used expert (maple.c's ESLOT cache), in slots of a shuffled order
    cached = [u for u in range(nu) if u % 2 == 0]
    rng = np.random.default_rng(nb)
    slot_of = {u: s for s, u in enumerate(rng.permutation(cached))}
    M.check(lib.gpux_init(1, len(cached)), "gpux_init")
    for u in cached:
        lib.gpux_upload(0, slot_of[u], *[M.ptr(a) for a in M.expert_views(layer7.blk, int(ue[u]))])
    gsl, gps, gtok, ga = [], [], [], []
    for u in cached:                                   # maple.c:791-797: runs of the cached experts in order
        gsl.append(slot_of[u]); gps.append(len(gtok))
        for a in range(ustart[u], ustart[u + 1]):
            gtok.append(int(utok[a])); ga.append(a)
    gps.append(len(gtok))
    gsl, gps, gtok = (np.array(v, np.int32) for v in (gsl, gps, gtok))
    h = lib.gpux_begin_multi(0, M.ptr(hn), nb, len(cached), M.ptr(gsl), M.ptr(gps), M.ptr(gtok))
    assert h, lib.mmoe_last_error()
    out = np.full((len(ga), 2048), np.nan, np.float32)
    lib.gpux_end_multi(h, M.ptr(out), len(ga))
    want = o["down"][np.array(ga)]
    print(f"\n  nb={nb}: {nu} experts used, {len(cached)} on the card, {len(ga)} pairs; bit-exact "
          f"{np.array_equal(out, want)}, relmax {relmax(out, want):.1e}")
    assert relmax(out, want) <= TOL
    # a pair count that does not match the call's is refused and writes nothing
    h = lib.gpux_begin_multi(0, M.ptr(hn), nb, len(cached), M.ptr(gsl), M.ptr(gps), M.ptr(gtok))
    bad = np.full((len(ga) + 1, 2048), 7.0, np.float32)
    lib.gpux_end_multi(h, M.ptr(bad), len(ga) + 1)
    assert b"outputs asked" in lib.mmoe_last_error() and (bad == 7.0).all()


def test_setters_drop_the_graph(layer7):
    lib = M.lib()
    x0 = M.synth_hidden(SEED, 600, 1)
    d_x = lib.mmoe_dev_alloc(x0.nbytes)
    M.check(lib.mmoe_h2d(d_x, M.ptr(x0), x0.nbytes), "h2d")
    bias = np.zeros(256, np.float32)
    setters = [("mmoe_set_debug(1)", lambda: lib.mmoe_set_debug(1)), ("mmoe_set_debug(0)", lambda: lib.mmoe_set_debug(0)),
               ("mmoe_set_decode_path", lambda: lib.mmoe_set_decode_path(1)),
               ("mmoe_set_router_mode", lambda: lib.mmoe_set_router_mode(0)),
               ("mmoe_set_bias", lambda: lib.mmoe_set_bias(7, M.ptr(bias))),
               ("mmoe_set_bias(NULL)", lambda: lib.mmoe_set_bias(7, None)),
               ("mmoe_set_layer", lambda: M.register_layer(7, layer7.blk, layer7.router) and 0)]
    try:
        for name, fn in setters:
            M.check(lib.mmoe_stack_graph(7, 1, d_x, 1, M.ORDER_STEP, 1), "graph")
            assert lib.mmoe_graph_held() == 1
            assert fn() == 0, name
            assert lib.mmoe_graph_held() == 0, f"{name} kept the captured graph"
        # after the last setter a replay captures again and still matches the eager step
        M.check(lib.mmoe_h2d(d_x, M.ptr(x0), x0.nbytes), "h2d")
        M.check(lib.mmoe_stack_graph(7, 1, d_x, 1, M.ORDER_STEP, 1), "graph")
        xg = np.empty_like(x0); M.check(lib.mmoe_d2h(M.ptr(xg), d_x, x0.nbytes), "d2h")
        M.check(lib.mmoe_h2d(d_x, M.ptr(x0), x0.nbytes), "h2d")
        M.check(lib.mmoe_stack_dev(7, 1, d_x, 1, M.ORDER_STEP), "eager")
        xe = np.empty_like(x0); M.check(lib.mmoe_d2h(M.ptr(xe), d_x, x0.nbytes), "d2h")
        assert np.array_equal(xg, xe)
    finally:
        lib.mmoe_graph_reset()
        lib.mmoe_set_debug(0)
        lib.mmoe_dev_free(d_x)
