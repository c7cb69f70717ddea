"""gfull_attn, the attention half of a layer on the card (maple.c:706-724 as gpu_pre.m / gpu_full.metal run it),
against the oracle's mo_attn_chunk (pinned against maple.c's own statements): per-layer fp16 key/value cache,
local (windowed, roped) and global layers, chunks that start at 0, inside the window and past it. The q/k/v and o
projections are maple.c's int8 sequence and the attention kernels keep the oracle's order of operations, so k, v
and the updated hidden state are compared bit for bit; the router logits against the oracle's batch chains."""
import ctypes as C

import numpy as np
import pytest

import maplemoe as M
import pyoracle as O
from helpers import SEED, HostLayer, relmax

pytestmark = pytest.mark.gpu

H = 2048
CTX = 1024
MAXTOK = 256
NWL = 4352                       # per layer: in_ln | post_ln | q_norm | k_norm (fp32 holding bf16 values)
CHUNKS = [(0, 200), (200, 256), (456, 256), (712, 100)]   # positions 0..811: the last two chunks pass WIN = 512
LAYERS = [(0, 0), (3, 1)]        # (layer, glob): layer 3 is global ((L % 4) == 3, maple.c:709)


def bf2f(u16):
    return (u16.astype(np.uint32) << 16).view(np.float32)


@pytest.fixture(scope="module")
def gfull_model():
    lib = M.lib()
    M.check(lib.mmoe_init(2048), "mmoe_init")
    M.check(lib.mmoe_dense_reset(), "dense reset")
    layers = [O.AttnLayer(SEED + 40 + k) for k in range(2)]      # even layers use [0], odd layers [1]
    for L in range(24):
        al = layers[L % 2]
        for n in "qkv":
            packed, s = al.mats[n]
            lib.gpre_dense_add(2 * L, M.ptr(packed), M.ptr(s), packed.shape[0], H)
        packed, s = al.mats["o"]
        lib.gpre_dense_add(2 * L + 1, M.ptr(packed), M.ptr(s), packed.shape[0], H)
    M.check(lib.gpre_dense_done(2048), "gpre_dense_done")
    rng = np.random.default_rng(SEED + 41)
    post = [(np.asarray(rng.uniform(0.5, 1.5, H), np.float32).view(np.uint32) >> 16).astype(np.uint16) for _ in range(2)]
    routers = [M.synth_router(SEED, L, 0) for L in range(2)]
    norms = np.empty((24, NWL), np.float32)
    router_all = np.empty((24, 256, H), np.uint16)
    for L in range(24):
        al = layers[L % 2]
        norms[L] = np.concatenate([bf2f(al.in_ln), bf2f(post[L % 2]), bf2f(al.q_norm), bf2f(al.k_norm)])
        router_all[L] = routers[L % 2]
    cs = O.rope_table(CTX)
    M.check(lib.gfull_init(CTX, MAXTOK, O.WIN, M.ptr(norms), M.ptr(router_all), M.ptr(cs)), "gfull_init")
    return lib, layers, post, routers, cs, norms, router_all


def test_gfull_attn_matches_oracle(gfull_model):
    lib, layers, post, routers, cs = gfull_model[:5]
    rng = np.random.default_rng(SEED + 42)
    kc = {L: np.zeros((CTX, 512), np.uint16) for L, _ in LAYERS}
    vc = {L: np.zeros((CTX, 512), np.uint16) for L, _ in LAYERS}
    for pos0, nb in CHUNKS:
        x0 = rng.standard_normal((nb, H)).astype(np.float32)
        lib.gfull_begin(M.ptr(x0), nb, pos0)
        for L, glob in LAYERS:
            print(f"\n  chunk pos0={pos0} nb={nb} layer {L} glob={glob}", flush=True)
            lib.gfull_write_x(M.ptr(x0))
            rl = np.full((nb, 256), np.nan, np.float32)
            t = lib.gfull_attn(L, glob, M.ptr(rl))
            assert t >= 0, lib.mmoe_last_error()
            x = np.full((nb, H), np.nan, np.float32)
            kop = C.c_void_p()
            lib.gfull_read(M.ptr(x), C.addressof(kop))
            assert kop.value
            ko = np.ctypeslib.as_array((C.c_uint16 * (24 * MAXTOK * 1024)).from_address(kop.value))
            ko = ko.reshape(24, MAXTOK, 1024)[L, :nb].copy()
            xo, ko_o, _ = O.attn_chunk(layers[L % 2], x0, pos0, glob, kc[L], vc[L], cs)
            nk = int((ko[:, :512] != ko_o[:, :512]).sum()); nv = int((ko[:, 512:] != ko_o[:, 512:]).sum())
            nx = int((x.view(np.uint32) != xo.view(np.uint32)).sum())
            hn = np.empty_like(x)
            for b in range(nb):
                O.oracle().mo_rmsnorm(O._p(x[b]), O._p(post[L % 2]), H, O._p(hn[b]))
            rl_o = O.router_batch(hn, routers[L % 2])
            nr = int((rl.view(np.uint32) != rl_o.view(np.uint32)).sum())
            print(f"  {t * 1e6:.0f} us; differing: k {nk}, v {nv}, x {nx} (relmax {relmax(x - x0, xo - x0):.1e}), "
                  f"router logits {nr} (relmax {relmax(rl, rl_o):.1e})", flush=True)
            assert nk == 0 and nv == 0 and nx == 0
            assert nr == 0


def test_gfull_whole_layers(gfull_model):
    """maple.c's step_batch_card (maple.c:1001-1031): per layer gfull_attn, top-8 and grouping on the host from
    the card's logits, gfull_moe; two chunks through layers 0 (local) and 3 (global). As maple.c's GFULL_CHECK
    (maple.c:940-1000) each layer is checked from the card's own input: the oracle's attention half, then its
    MoE block on rmsnorm(x, post_ln) with the same top-8. The second chunk routes on the card instead
    (gfull_attn without a logits copy, then mmoe_route on the device logits, in place of maple.c's job_topk and
    group_pairs) and hands gfull_moe the tables mmoe_route returned."""
    lib, layers, post, routers, cs = gfull_model[:5]
    blocks = [HostLayer(SEED, k) for k in range(2)]                  # experts of even / odd layers
    rids = [lib.gpre_region(M.ptr(h.blk), h.blk.nbytes) for h in blocks]
    assert min(rids) >= 0, lib.mmoe_last_error()
    rng = np.random.default_rng(SEED + 43)
    kc = {L: np.zeros((CTX, 512), np.uint16) for L, _ in LAYERS}
    vc = {L: np.zeros((CTX, 512), np.uint16) for L, _ in LAYERS}
    for pos0, nb in [(0, 128), (128, 200)]:
        x = rng.standard_normal((nb, H)).astype(np.float32)
        lib.gfull_begin(M.ptr(x), nb, pos0)
        for L, glob in LAYERS:
            k = L % 2
            xin = np.empty((nb, H), np.float32)
            lib.gfull_read(M.ptr(xin), None)
            if pos0 == 0:
                rl = np.empty((nb, 256), np.float32)
                assert lib.gfull_attn(L, glob, M.ptr(rl)) >= 0, lib.mmoe_last_error()
                top, tw = O.topk(rl)
                g = O.group(top, tw)
            else:
                assert lib.gfull_attn(L, glob, None) >= 0, lib.mmoe_last_error()
                rl = M.read("LOGITS", (nb, 256), np.float32)
                top = np.empty((nb, 8), np.int32); tw = np.empty((nb, 8), np.float32)
                ue = np.empty(256, np.int32); us = np.empty(257, np.int32)
                utok = np.empty(nb * 8, np.int32); uw = np.empty(nb * 8, np.float32); tpr = np.empty((nb, 8), np.int32)
                nu = lib.mmoe_route(None, nb, M.ptr(top), M.ptr(tw), M.ptr(ue), M.ptr(us), M.ptr(utok), M.ptr(uw), M.ptr(tpr))
                assert nu > 0, lib.mmoe_last_error()
                g = dict(nu=nu, ue=ue[:nu].copy(), ustart=us[:nu + 1].copy(), utok=utok, uw=uw, tp=tpr)
            loc = M.block_loc(0, list(g["ue"]))
            regs = np.array([rids[k], -1, -1, -1], np.int32)
            tp = np.ascontiguousarray(g["tp"])
            lib.gfull_moe(g["nu"], M.ptr(loc), M.ptr(regs), M.ptr(g["ustart"]), M.ptr(g["utok"]), M.ptr(g["uw"]), M.ptr(tp))
            xg = np.empty((nb, H), np.float32)
            lib.gfull_read(M.ptr(xg), None)
            xa, _, _ = O.attn_chunk(layers[k], xin, pos0, glob, kc[L], vc[L], cs)
            hn = np.empty_like(xa)
            for b in range(nb):
                O.oracle().mo_rmsnorm(O._p(xa[b]), O._p(post[k]), H, O._p(hn[b]))
            xo = xa.copy()
            o = O.moe_batch(hn, routers[k], blocks[k].table, xo, want=("rl", "top", "tw", "nu", "ue", "ustart", "utok", "uw", "tp"))
            assert np.array_equal(rl.view(np.uint32), o["rl"].view(np.uint32)), "router logits"
            assert np.array_equal(top, o["top"]), "top-8"
            if pos0:   # the card's routing tables, as maple.c's group_pairs forms them
                assert g["nu"] == o["nu"] and np.array_equal(g["ustart"], np.ravel(o["ustart"])[:g["nu"] + 1]) and np.array_equal(g["utok"], o["utok"])
                assert np.array_equal(g["uw"].view(np.uint32), o["uw"].view(np.uint32)) and np.array_equal(g["tp"].ravel(), np.ravel(o["tp"]))
            e = relmax(xg - xin, xo - xin)
            print(f"\n  pos0={pos0} nb={nb} layer {L}: {g['nu']} experts, x bit-exact {np.array_equal(xg, xo)}, relmax {e:.1e}",
                  flush=True)
            assert e <= 1e-5


def test_gfull_stack_on_device(gfull_model):
    """mmoe_gfull_stack: the attention half and the device MoE block (router, top-8, grouping, experts, combine)
    per layer with no host step between them. Layers 0..3 (3 is global) one at a time from the card's own input,
    against the oracle's attention half followed by its MoE block; chunks of 5 tokens (the decode kernels) and
    of 256 tokens at positions past the window."""
    lib, layers, post, routers, cs = gfull_model[:5]
    blocks = [HostLayer(SEED, k) for k in range(2)]
    for L in range(4):
        M.register_layer(L, blocks[L % 2].blk, routers[L % 2], post[L % 2])
    rng = np.random.default_rng(SEED + 44)
    kc = {L: np.zeros((CTX, 512), np.uint16) for L in range(4)}
    vc = {L: np.zeros((CTX, 512), np.uint16) for L in range(4)}
    for pos0, nb in [(0, 5), (5, 256), (261, 256), (517, 256)]:
        x = rng.standard_normal((nb, H)).astype(np.float32)
        lib.gfull_begin(M.ptr(x), nb, pos0)
        for L in range(4):
            k, glob = L % 2, int(L % 4 == 3)
            print(f"\n  pos0={pos0} nb={nb} layer {L}", flush=True)
            xin = np.empty((nb, H), np.float32)
            lib.gfull_read(M.ptr(xin), None)
            M.check(lib.mmoe_gfull_stack(L, 1), "mmoe_gfull_stack")
            xg = np.empty((nb, H), np.float32)
            lib.gfull_read(M.ptr(xg), None)
            xa, _, _ = O.attn_chunk(layers[k], xin, pos0, glob, kc[L], vc[L], cs)
            hn = np.empty_like(xa)
            for b in range(nb):
                O.oracle().mo_rmsnorm(O._p(xa[b]), O._p(post[k]), H, O._p(hn[b]))
            xo = xa.copy()
            o = O.moe_batch(hn, routers[k], blocks[k].table, xo, want=("rl", "top", "tw"))
            top = M.read("TOP", (nb, 8), np.int32)
            e = relmax(xg - xin, xo - xin)
            print(f"  top-8 equal {np.array_equal(top, o['top'])}, x bit-exact {np.array_equal(xg, xo)}, relmax {e:.1e}", flush=True)
            assert np.array_equal(np.sort(top, 1), np.sort(o["top"], 1))
            assert e <= 1e-5


@pytest.mark.parametrize("nb,pos0", [(1030, 0), (602, 700)])
def test_gfull_attn_large_chunk(gfull_model, nb, pos0):
    """Chunks of 1030 tokens at position 0 and 602 tokens at 700 (above 256 tokens the weighted-sum kernel takes
    4-token groups; both sizes leave a partial group) on a fresh 2048-position set-up, local and global layer,
    against the oracle."""
    lib, layers, post, routers, cs, norms, router_all = gfull_model
    ctx = 2048
    cs = O.rope_table(ctx)
    M.check(lib.gfull_init(ctx, 2048, O.WIN, M.ptr(norms), M.ptr(router_all), M.ptr(cs)), "gfull_init 2048")
    rng = np.random.default_rng(SEED + 45 + nb)
    x0 = rng.standard_normal((nb, H)).astype(np.float32)
    lib.gfull_begin(M.ptr(x0), nb, pos0)
    assert not lib.mmoe_last_error().startswith(b"gfull_begin"), lib.mmoe_last_error()
    for L, glob in LAYERS:
        print(f"\n  nb={nb} layer {L} glob={glob}", flush=True)
        lib.gfull_write_x(M.ptr(x0))
        rl = np.empty((nb, 256), np.float32)
        assert lib.gfull_attn(L, glob, M.ptr(rl)) >= 0, lib.mmoe_last_error()
        x = np.empty((nb, H), np.float32)
        kop = C.c_void_p()
        lib.gfull_read(M.ptr(x), C.addressof(kop))
        ko = np.ctypeslib.as_array((C.c_uint16 * (24 * 2048 * 1024)).from_address(kop.value)).reshape(24, 2048, 1024)[L, :nb]
        kc = np.zeros((ctx, 512), np.uint16); vc = np.zeros((ctx, 512), np.uint16)   # positions before pos0: zeros on both sides
        xo, ko_o, _ = O.attn_chunk(layers[L % 2], x0, pos0, glob, kc, vc, cs)
        nx = int((x.view(np.uint32) != xo.view(np.uint32)).sum())
        print(f"  differing: k/v {int((ko != ko_o).sum())}, x {nx}", flush=True)
        assert np.array_equal(ko, ko_o) and nx == 0
