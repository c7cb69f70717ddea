"""BASELINE configurations 1, 3 and 4 at their stated sizes, against the oracle.

- Config 1: one token through 24 stacked MoE layers with uniform random router weights (dist=1), in step()
  order, eager and as the HIP-graph replay the bench times; the whole trajectory against the oracle.
- Config 3: 64 sequences through the same 24 layers in step_batch order. A token's result depends on that token
  only (its router chains, its top-8, its pairs' combine order), so 4 sampled tokens run through the oracle.
- Config 4: a 2048-token chunk at positions 0-2047 and a second at 2048-4095 (4096-position fp16 cache) through
  a local (windowed) and a global layer, attention half and MoE block (Zipf(1.1)-biased router, as the bench).
  The oracle's attention for one token needs the cache of every earlier position: it gets the card's cache, whose
  rows are checked bit for bit on the sampled positions, then runs maple.c's chunk code for each sampled token.
  The first chunk runs with the exact router option, the second with the default MFMA router, under which
  gfull_attn must still return exact logits."""
import ctypes as C

import numpy as np
import pytest

import maplemoe as M
import pyoracle as O
from helpers import SEED, HostLayer, relmax

pytestmark = pytest.mark.gpu
NL, H = 24, 2048


def bf16_near_one(rng, n):
    return (np.asarray(rng.uniform(0.6, 1.4, n), np.float32).view(np.uint32) >> 16).astype(np.uint16)


@pytest.fixture(scope="module")
def stack24():
    lib = M.lib()
    M.check(lib.mmoe_init(2048), "mmoe_init")
    M.check(lib.mmoe_set_debug(0), "debug off")
    rng = np.random.default_rng(SEED + 70)
    layers, pln = [], []
    for L in range(NL):
        hl = HostLayer(SEED + 1, L, dist=1)             # config 1: uniform random router weights
        p = bf16_near_one(rng, H)
        M.register_layer(L, hl.blk, hl.router, p)
        layers.append(hl); pln.append(p)
    return lib, layers, pln


def oracle_stack(layers, pln, x, order):
    x = x.copy()
    for L in range(NL):
        hn = np.empty_like(x)
        for b in range(x.shape[0]):
            O.oracle().mo_rmsnorm(O._p(x[b]), O._p(pln[L]), H, O._p(hn[b]))
        if order == M.ORDER_STEP:
            O.moe_step(hn[0], layers[L].router, layers[L].table, x[0])
        else:
            O.moe_batch(hn, layers[L].router, layers[L].table, x, want=("top",))
    return x


def run_stack(lib, x0, order, graph=False):
    nb = x0.shape[0]
    d_x = lib.mmoe_dev_alloc(x0.nbytes)
    try:
        M.check(lib.mmoe_h2d(d_x, M.ptr(x0), x0.nbytes), "h2d")
        if graph:
            M.check(lib.mmoe_stack_graph(0, NL, d_x, nb, order, 1), "graph")
        else:
            M.check(lib.mmoe_stack_dev(0, NL, d_x, nb, order), "stack")
        out = np.empty_like(x0)
        M.check(lib.mmoe_d2h(M.ptr(out), d_x, x0.nbytes), "d2h")
    finally:
        lib.mmoe_graph_reset()
        lib.mmoe_dev_free(d_x)
    return out


def test_config1_decode_24_layers(stack24):
    lib, layers, pln = stack24
    for sid in (1, 2):
        x0 = M.synth_hidden(SEED, 700 + sid, 1)
        xe = run_stack(lib, x0, M.ORDER_STEP)
        xg = run_stack(lib, x0, M.ORDER_STEP, graph=True)
        xo = oracle_stack(layers, pln, x0, M.ORDER_STEP)
        print(f"\n  config 1, token {sid}: graph == eager {np.array_equal(xg, xe)}, bit-exact vs oracle "
              f"{np.array_equal(xe, xo)}, relmax {relmax(xe - x0, xo - x0):.1e}", flush=True)
        assert np.array_equal(xg.view(np.int32), xe.view(np.int32))
        assert relmax(xe - x0, xo - x0) <= 1e-5


def test_config3_batched_decode_24_layers(stack24):
    lib, layers, pln = stack24
    x0 = M.synth_hidden(SEED, 710, 64)
    xe = run_stack(lib, x0, M.ORDER_BATCH)
    xg = run_stack(lib, x0, M.ORDER_BATCH, graph=True)
    assert np.array_equal(xg.view(np.int32), xe.view(np.int32))
    sample = np.array([0, 17, 42, 63])
    xo = oracle_stack(layers, pln, x0[sample], M.ORDER_BATCH)
    e = relmax(xe[sample] - x0[sample], xo - x0[sample])
    print(f"\n  config 3, tokens {list(sample)}: bit-exact {np.array_equal(xe[sample], xo)}, relmax {e:.1e}")
    assert e <= 1e-5


@pytest.mark.parametrize("nb,order,nl", [(64, M.ORDER_BATCH, 4), (64, M.ORDER_BATCH, 5), (40, M.ORDER_STEP, 4),
                                         (100, M.ORDER_BATCH, 3), (300, M.ORDER_BATCH, 3)])
def test_stack_matches_layer_by_layer(stack24, nb, order, nl):
    """Stacked layers (one mmoe_stack_dev call over nl layers) against the same layers run one call at a time, bit
    for bit: both orders, several sizes on the chain-router path, and 300 tokens, whose down results travel as
    int16."""
    lib = stack24[0]
    x0 = M.synth_hidden(SEED, 720 + nb + nl, nb)
    d_x = lib.mmoe_dev_alloc(x0.nbytes)
    try:
        M.check(lib.mmoe_h2d(d_x, M.ptr(x0), x0.nbytes), "h2d")
        M.check(lib.mmoe_stack_dev(2, nl, d_x, nb, order), "stack")
        xs = np.empty_like(x0); M.check(lib.mmoe_d2h(M.ptr(xs), d_x, x0.nbytes), "d2h")
        M.check(lib.mmoe_h2d(d_x, M.ptr(x0), x0.nbytes), "h2d")
        for L in range(2, 2 + nl):
            M.check(lib.mmoe_stack_dev(L, 1, d_x, nb, order), "one layer")
        x1 = np.empty_like(x0); M.check(lib.mmoe_d2h(M.ptr(x1), d_x, x0.nbytes), "d2h")
    finally:
        lib.mmoe_dev_free(d_x)
    assert np.array_equal(xs.view(np.int32), x1.view(np.int32))
    assert not np.array_equal(xs, x0)


# ---------------------------------------------------------------- config 4
CTX, T = 4096, 2048
C4_LAYERS = [(0, 0), (3, 1)]          # (layer, glob): layer 3 attends to every earlier position


@pytest.fixture(scope="module")
def config4(stack24):
    lib = stack24[0]
    M.check(lib.mmoe_dense_reset(), "dense reset")
    att = [O.AttnLayer(SEED + 80 + k) for k in range(2)]
    for L in range(NL):
        a = att[L % 2]
        for n in "qkv":
            packed, s = a.mats[n]
            lib.gpre_dense_add(2 * L, M.ptr(packed), M.ptr(s), packed.shape[0], H)
        packed, s = a.mats["o"]
        lib.gpre_dense_add(2 * L + 1, M.ptr(packed), M.ptr(s), packed.shape[0], H)
    M.check(lib.gpre_dense_done(T), "gpre_dense_done")
    rng = np.random.default_rng(SEED + 81)
    blocks = [HostLayer(SEED + 2, k) for k in range(2)]
    post = [bf16_near_one(rng, H) for _ in range(2)]
    zb = M.zipf_bias(SEED, 1.1)
    norms = np.empty((NL, 4352), np.float32)
    routers = np.empty((NL, 256, H), np.uint16)
    f32 = lambda u: (u.astype(np.uint32) << 16).view(np.float32)
    for L in range(NL):
        a = att[L % 2]
        norms[L] = np.concatenate([f32(a.in_ln), f32(post[L % 2]), f32(a.q_norm), f32(a.k_norm)])
        routers[L] = blocks[L % 2].router
    cs = O.rope_table(CTX)
    M.check(lib.gfull_init(CTX, T, O.WIN, M.ptr(norms), M.ptr(routers), M.ptr(cs)), "gfull_init")
    for L, _ in C4_LAYERS:
        M.register_layer(L, blocks[L % 2].blk, blocks[L % 2].router, post[L % 2])
        M.check(lib.mmoe_set_bias(L, M.ptr(zb)), "bias")
    yield lib, att, blocks, post, zb, cs
    for L, _ in C4_LAYERS:
        lib.mmoe_set_bias(L, None)
    lib.mmoe_set_router_mode(0)


def test_config4_full_size_sampled(config4):
    lib, att, blocks, post, zb, cs = config4
    rng = np.random.default_rng(SEED + 82)
    kc = {L: np.zeros((CTX, 512), np.uint16) for L, _ in C4_LAYERS}
    vc = {L: np.zeros((CTX, 512), np.uint16) for L, _ in C4_LAYERS}
    for pos0, mode in ((0, 1), (2048, 0)):
        M.check(lib.mmoe_set_router_mode(mode), "router mode")
        x0 = rng.standard_normal((T, H)).astype(np.float32)
        lib.gfull_begin(M.ptr(x0), T, pos0)
        sample = np.unique(np.concatenate([[0, 1, 511, 512, 513, 1023, 2047], rng.integers(0, T, 9)]))
        for L, glob in C4_LAYERS:
            k = L % 2
            print(f"\n  chunk at {pos0} (router mode {mode}), layer {L} glob {glob}: {len(sample)} sampled tokens", flush=True)
            lib.gfull_write_x(M.ptr(x0))
            rl = np.empty((T, 256), np.float32)
            assert lib.gfull_attn(L, glob, M.ptr(rl)) >= 0, lib.mmoe_last_error()
            xa = np.empty((T, H), np.float32)
            kop = C.c_void_p()
            lib.gfull_read(M.ptr(xa), C.addressof(kop))
            ko = np.ctypeslib.as_array((C.c_uint16 * (NL * T * 1024)).from_address(kop.value)).reshape(NL, T, 1024)[L].copy()
            kc[L][pos0:pos0 + T] = ko[:, :512]; vc[L][pos0:pos0 + T] = ko[:, 512:]
            lib.gfull_write_x(M.ptr(x0))                       # the whole layer on the card: attention + MoE
            M.check(lib.mmoe_gfull_stack(L, 1), "gfull_stack")
            xf = np.empty((T, H), np.float32)
            lib.gfull_read(M.ptr(xf), None)
            top = M.read("TOP", (T, 8), np.int32)
            bad = []
            for b in sample:
                p = pos0 + int(b)
                xo, ko_o, _ = O.attn_chunk(att[k], x0[b:b + 1], p, glob, kc[L].copy(), vc[L].copy(), cs)
                hn = np.empty_like(xo)
                O.oracle().mo_rmsnorm(O._p(xo[0]), O._p(post[k]), H, O._p(hn[0]))
                xm = xo.copy()
                o = O.moe_batch(hn, blocks[k].router, blocks[k].table, xm, bias=zb, want=("rl", "top"))
                rl_o = O.router_batch(hn, blocks[k].router, zb)   # the layer's logit bias is part of its router
                ok = (np.array_equal(xa[b].view(np.uint32), xo[0].view(np.uint32)) and np.array_equal(ko[b], ko_o[0])
                      and np.array_equal(rl[b].view(np.uint32), rl_o[0].view(np.uint32))
                      and np.array_equal(top[b], o["top"][0]) and relmax(xf[b] - xo[0], xm[0] - xo[0]) <= 1e-5)
                if not ok:
                    bad.append(int(b))
            print(f"  attention x, k/v, router logits bit-exact and MoE within 1e-5 on all but {bad}", flush=True)
            assert not bad
