"""HIP path vs the C oracle on identical seeded inputs, through the C ABI (libmaplemoe).

Bar: bit-exact for router logits order, top-8 indices, grouping, int8 quantisation and every int32 code*q
sum; fp32 results within 1e-5 max-normalised (they are in fact compared bit for bit where the operation
sequence is shared, and the test reports it)."""
import ctypes as C
import numpy as np
import pytest

import maplemoe as M
import pyoracle as O
from helpers import SEED, HostLayer, normed_hidden, relmax

pytestmark = pytest.mark.gpu
TOL = 1e-5


@pytest.fixture(scope="module")
def layer0():
    lib = M.lib()
    M.check(lib.mmoe_init(2048), "mmoe_init")
    M.check(lib.mmoe_set_debug(1), "debug")
    hl = HostLayer(SEED, 0)
    hl.rid = M.register_layer(0, hl.blk, hl.router)
    return hl


def run_gpu(L, hn, x, order):
    x_out = x.copy()
    M.check(M.lib().mmoe_moe(L, M.ptr(hn), hn.shape[0], M.ptr(x_out), order), "mmoe_moe")
    return x_out


def compare_layer(hl, nb, order, bias_note="", refined=False):
    x, hn = normed_hidden(SEED, nb, nb)
    nb = hn.shape[0]; P = nb * 8
    xg = run_gpu(hl.L, hn, x, order)
    xo = x.copy()
    o = O.moe_batch(hn, hl.router, hl.table, xo) if order == M.ORDER_BATCH else O.moe_step(hn[0], hl.router, hl.table, xo[0])
    print(f"\n[nb={nb} order={order}{bias_note}]", flush=True)
    # refined: the MFMA router + exact refinement (mmoe_set_router_mode(0)); the logits of every token's
    # top-8 experts are maple.c's chain results bit for bit, the rest are approximate
    rl = M.read("LOGITS", (nb, 256), np.float32)
    orl = o["rl"].reshape(nb, 256)
    top = M.read("TOP", (nb, 8), np.int32)
    assert np.array_equal(top, o["top"].reshape(nb, 8)), "top-8 indices differ"
    if refined:
        sel = np.take_along_axis(rl, top, 1), np.take_along_axis(orl, top, 1)
        assert np.array_equal(sel[0].view(np.int32), sel[1].view(np.int32)), "top-8 logits not bit-exact"
        # the other logits are an intermediate (only their softmax sum reaches tw): two bf16 parts of the input
        # leave a 2^-15 remainder per term, so they sit ~1e-5 from the chain values; tw and x keep the 1e-5 bar
        assert relmax(rl, orl) <= 1e-4
        print("  approximate logits: relmax", relmax(rl, orl), "bit-exact share", float((rl == orl).mean()))
    else:
        assert np.array_equal(rl.view(np.int32), orl.view(np.int32)), "router logits not bit-exact"
    tw = M.read("TW", (nb, 8), np.float32)
    assert relmax(tw, o["tw"].reshape(nb, 8)) <= TOL
    print("  tw bit-exact:", np.array_equal(tw, o["tw"].reshape(nb, 8)), "relmax", relmax(tw, o["tw"].reshape(nb, 8)))
    plan = M.read_plan()
    qx = M.mfma_to_natural(M.read("QX", (nb, 2048), np.int8), 2048)
    assert np.array_equal(qx, o["qx"]), "int8 input quantisation differs"
    assert np.array_equal(M.read("QSX", (nb,), np.float32), o["qsx"])
    assert np.array_equal(M.read("QSUMX", (nb,), np.int32), o["qsumx"])
    if order == M.ORDER_BATCH:
        nu = int(o["nu"][0])
        assert plan["nu"] == nu and np.array_equal(plan["ue"], o["ue"][:nu]) and np.array_equal(plan["ustart"], o["ustart"][:nu + 1])
        assert np.array_equal(M.read("UTOK", (P,), np.int32), o["utok"])
        uw = M.read("UW", (P,), np.float32)
        assert relmax(uw, o["uw"]) <= TOL if refined else np.array_equal(uw, o["uw"])
        assert np.array_equal(M.read("TP", (nb, 8), np.int32), o["tp"])
        perm = np.arange(P)
    else:
        # decode: oracle indexes by slot, the device by pair; sp maps slot -> pair
        sp = M.read("SP", (1, 8), np.int32)[0]
        perm = sp
    gu = M.read("GU_I32", (P, 1024), np.int32)[perm]
    assert np.array_equal(gu, o["gu_i32"]), "gate/up int32 sums differ"
    act = M.read("ACT", (P, 512), np.float32)[perm]
    assert relmax(act, o["act"]) <= TOL
    print("  act bit-exact:", np.array_equal(act, o["act"]))
    qa = M.mfma_to_natural(M.read("QA", (P, 512), np.int8), 512)[perm]
    nflip = int((qa != o["qa"]).sum())
    print("  act int8 mismatches:", nflip)
    assert nflip == 0
    dn = M.read("DN_I32", (P, 2048), np.int32)[perm]
    assert np.array_equal(dn, o["dn_i32"]), "down int32 sums differ"
    down = M.read("DOWN", (P, 2048), np.float32)[perm]
    assert relmax(down, o["down"]) <= TOL
    print("  down bit-exact:", np.array_equal(down, o["down"]))
    assert relmax(xg - x, xo - x) <= TOL
    print("  x bit-exact:", np.array_equal(xg, xo), "rel", relmax(xg - x, xo - x))


@pytest.mark.parametrize("nb", [1, 3, 32, 64, 100, 128])   # 128: config 0 chunk
def test_moe_batch(layer0, nb):
    compare_layer(layer0, nb, M.ORDER_BATCH)


def test_silu_exhaustive():
    """The activation kernel's SiLU (refined reciprocal instead of IEEE division, ldexp instead of two power-of-two
    products) equals g / (1 + exp(-g)) with IEEE division for every finite fp32 g <= 7 (the gate clamp)."""
    lib = M.lib()
    M.check(lib.mmoe_init(8), "init")
    for lo, hi in [(0x00000000, 0x40E00000), (0x80000000, 0xFF7FFFFF)]:   # +0 .. 7, -0 .. -FLT_MAX
        nbad, first = C.c_ulonglong(), C.c_uint32()
        M.check(lib.mmoe_selftest_silu(lo, hi - lo + 1, C.byref(nbad), C.byref(first)), "selftest")
        assert nbad.value == 0, f"{nbad.value} mismatches in [{lo:#x}, {hi:#x}], first {first.value:#x}"


def test_moe_batch_gemm_router(layer0):
    # >= 512 tokens with the exact router option: the tiled fp32 chains (k_router_gemm); 520 leaves a ragged
    # last token tile
    M.check(M.lib().mmoe_set_router_mode(1), "router mode")
    try:
        compare_layer(layer0, 520, M.ORDER_BATCH)
    finally:
        M.check(M.lib().mmoe_set_router_mode(0), "router mode")


@pytest.mark.parametrize("nb,refined", [(255, False), (511, False), (512, True), (1023, True), (1024, True)])
def test_moe_batch_size_boundaries(layer0, nb, refined):
    """Sizes at the path switches: 255 tokens is the largest batch whose grouping forms inside the fused
    small-tile kernel; 511 the last one on the chain router and 512 the first on the MFMA router with exact
    refinement; 1023 runs the router in blocks of 128 experts (ragged last 32-token block), 1024 in blocks of
    all 256 experts."""
    compare_layer(layer0, nb, M.ORDER_BATCH, f" boundary {nb}", refined=refined)


def test_moe_batch_tn64(layer0):
    # 256 tokens -> 2048 pairs: the 64-token tile kernels
    compare_layer(layer0, 256, M.ORDER_BATCH)


def test_moe_step(layer0):
    compare_layer(layer0, 1, M.ORDER_STEP)


@pytest.mark.parametrize("nb", [48, 300])
def test_gpre_moe(layer0, nb):
    """gpre_moe with a host grouping (maple.c:757-763 call) vs the oracle's grouped experts; 300 tokens (2400
    pairs) take the 64-pair tile kernels with a plan built from the host grouping"""
    lib = M.lib()
    x, hn = normed_hidden(SEED, 900, nb)
    rl = O.router_batch(hn, layer0.router)
    top, tw = O.topk(rl)
    g = O.group(top, tw)
    nu = g["nu"]
    loc = M.block_loc(0, list(g["ue"]))
    regs = np.array([layer0.rid, -1, -1, -1], np.int32)
    y = np.zeros((nb, 2048), np.float32)
    tp = np.ascontiguousarray(g["tp"])
    sec = lib.gpre_moe(M.ptr(hn), nb, nu, M.ptr(loc), M.ptr(regs), None, M.ptr(g["ustart"]), M.ptr(g["utok"]),
                       M.ptr(g["uw"]), M.ptr(tp), M.ptr(y))
    assert sec >= 0, lib.mmoe_last_error()
    import ctypes as C
    exu = (O.Expert * nu)(*[layer0.table[int(e)] for e in g["ue"]])
    yo = np.zeros_like(y)
    O.oracle().mo_experts_grouped(O._p(hn), nb, nu, C.cast(exu, C.c_void_p), O._p(g["ustart"]), O._p(g["utok"]),
                                  O._p(g["uw"]), O._p(np.ascontiguousarray(g["tp"])), O._p(yo), None)
    print("\n  gpre_moe y bit-exact:", np.array_equal(y, yo), relmax(y, yo))
    assert relmax(y, yo) <= TOL


def test_gpux(layer0):
    """gpux_init/upload/begin/end (maple.c:628-642) vs the oracle's per-slot down outputs"""
    lib = M.lib()
    M.check(lib.gpux_init(1, 8), "gpux_init")
    experts = [3, 77, 150, 255, 0, 19]
    for s, e in enumerate(experts):
        lib.gpux_upload(0, s, *[M.ptr(a) for a in M.expert_views(layer0.blk, e)])
    x, hn = normed_hidden(SEED, 901, 1)
    slots = np.array([4, 1, 3], np.int32)
    h = lib.gpux_begin(0, M.ptr(hn[0]), 3, M.ptr(slots))
    assert h, lib.mmoe_last_error()
    out = np.zeros((3, 2048), np.float32)
    lib.gpux_end(h, M.ptr(out), 3)
    q, qs, qsum = O.prep(hn[0])
    for k, s in enumerate(slots):
        ex = layer0.table[experts[s]]
        # oracle: per-slot step MoE with a one-hot router is not needed; recompute directly
        o = O.oracle()
        import ctypes as C
        gate = np.zeros(512, np.float32); up = np.zeros(512, np.float32)
        gc, gs, uc, us, dc, ds = M.expert_views(layer0.blk, experts[s])
        for r in range(512):
            gate[r] = np.float32(np.float32(o.mo_dot_i32(O._p(gc[r]), O._p(q), 2048) - qsum) * qs) * gs[r]
            up[r] = np.float32(np.float32(o.mo_dot_i32(O._p(uc[r]), O._p(q), 2048) - qsum) * qs) * us[r]
        act = np.zeros(512, np.float32)
        o.mo_act(O._p(gate), O._p(up), O._p(act), 512)
        qa, qsa, qsuma = O.prep(act)
        d = np.array([np.float32(np.float32(o.mo_dot_i32(O._p(dc[r]), O._p(qa), 512) - qsuma) * qsa) * ds[r] for r in range(2048)], np.float32)
        assert relmax(out[k], d) <= TOL
    # a second gpux_init replaces the slots: upload one expert again and the hit gives the same output
    M.check(lib.gpux_init(2, 4), "gpux_init again")
    lib.gpux_upload(1, 2, *[M.ptr(a) for a in M.expert_views(layer0.blk, experts[4])])
    h = lib.gpux_begin(1, M.ptr(hn[0]), 1, M.ptr(np.array([2], np.int32)))
    assert h, lib.mmoe_last_error()
    again = np.zeros((1, 2048), np.float32)
    lib.gpux_end(h, M.ptr(again), 1)
    assert np.array_equal(again[0], out[0]), "slot 4 before and slot 2 after the second gpux_init differ"
    assert not lib.gpux_begin(1, M.ptr(hn[0]), 1, M.ptr(np.array([4], np.int32)))   # past the 4 slots now


@pytest.mark.parametrize("nb", [1, 5, 8])
def test_moe_grouped_path_small_batches(layer0, nb):
    """the grouped-GEMM kernels at decode sizes (the default there is the three-kernel decode path)"""
    M.check(M.lib().mmoe_set_decode_path(0), "decode off")
    try:
        compare_layer(layer0, nb, M.ORDER_BATCH)
        if nb == 1:
            compare_layer(layer0, 1, M.ORDER_STEP)
    finally:
        M.lib().mmoe_set_decode_path(1)


def test_stack_decode(layer0):
    """3 stacked layers (rmsnorm with a bf16 post-norm weight, then the MoE block of step()) on device memory,
    against the oracle applied layer by layer"""
    lib = M.lib()
    layers = [layer0]
    rng = np.random.default_rng(5)
    pln = (np.float32(1.0) + rng.standard_normal((3, 2048)).astype(np.float32) * 0.1).view(np.uint32)
    pln = ((pln + 0x7FFF + ((pln >> 16) & 1)) >> 16).astype(np.uint16)       # bf16 weights
    for L in (1, 2):
        hl = HostLayer(SEED, L)
        hl.rid = M.register_layer(L, hl.blk, hl.router, pln[L])
        layers.append(hl)
    M.register_layer(0, layer0.blk, layer0.router, pln[0])  # layer 0 again, now with its norm weight
    for nb, order in [(1, M.ORDER_STEP), (4, M.ORDER_BATCH), (64, M.ORDER_BATCH)]:   # 64: batched decode (config 3 shape)
        x0 = M.synth_hidden(SEED, 300 + nb, nb)
        d_x = lib.mmoe_dev_alloc(x0.nbytes)
        M.check(lib.mmoe_h2d(d_x, M.ptr(x0), x0.nbytes), "h2d")
        M.check(lib.mmoe_stack_dev(0, 3, d_x, nb, order), "stack")
        xg = np.empty_like(x0)
        M.check(lib.mmoe_d2h(M.ptr(xg), d_x, x0.nbytes), "d2h")
        lib.mmoe_dev_free(d_x)
        xo = x0.copy()
        for L in range(3):
            hn = np.empty_like(xo)
            for b in range(nb):
                O.oracle().mo_rmsnorm(O._p(xo[b]), O._p(pln[L]), 2048, O._p(hn[b]))
            if order == M.ORDER_STEP:
                O.moe_step(hn[0], layers[L].router, layers[L].table, xo[0])
            else:
                O.moe_batch(hn, layers[L].router, layers[L].table, xo)
        print(f"\n  stack nb={nb}: bit-exact {np.array_equal(xg, xo)}, rel {relmax(xg - x0, xo - x0):.2e}")
        assert relmax(xg - x0, xo - x0) <= TOL


def test_stack_graph_replays_match_eager(layer0):
    """mmoe_stack_graph (the HIP-graph replay the decode benchmarks time) against mmoe_stack_dev: three replays
    in a row, each with eager work of another shape in between, every replay bit-identical to the eager step.
    The second case changes the arguments, so the library must capture a new graph, not replay the old one.
    Runs after test_stack_decode, which set layers 0-2 with their norm weights."""
    lib = M.lib()
    M.check(lib.mmoe_graph_reset(), "graph reset")
    xo, ho = normed_hidden(SEED, 903, 8)
    for nb, order in [(1, M.ORDER_STEP), (64, M.ORDER_BATCH)]:
        x0 = M.synth_hidden(SEED, 400 + nb, nb)
        d_e = lib.mmoe_dev_alloc(x0.nbytes); d_g = lib.mmoe_dev_alloc(x0.nbytes)
        M.check(lib.mmoe_h2d(d_e, M.ptr(x0), x0.nbytes), "h2d"); M.check(lib.mmoe_h2d(d_g, M.ptr(x0), x0.nbytes), "h2d")
        xe = np.empty_like(x0); xg = np.empty_like(x0)
        try:
            for r in range(3):
                M.check(lib.mmoe_stack_dev(0, 3, d_e, nb, order), "stack eager")
                M.check(lib.mmoe_d2h(M.ptr(xe), d_e, x0.nbytes), "d2h")
                run_gpu(0, ho, xo, M.ORDER_BATCH)                            # other work between replays
                M.check(lib.mmoe_stack_graph(0, 3, d_g, nb, order, 1), "stack graph")
                M.check(lib.mmoe_d2h(M.ptr(xg), d_g, x0.nbytes), "d2h")
                assert np.array_equal(xg.view(np.int32), xe.view(np.int32)), f"nb {nb} replay {r} differs from eager"
            print(f"\n  graph nb={nb}: 3 replays bit-identical to the eager steps")
        finally:
            M.check(lib.mmoe_graph_reset(), "graph reset")   # before its buffers go
            lib.mmoe_dev_free(d_e); lib.mmoe_dev_free(d_g)


def test_moe_batch_mfma_router(layer0):
    """Batches of >= 512 tokens with the bf16-MFMA router (inputs split into two bf16 parts) and exact
    chain logits for each token's candidates (k_refine_topk): top-8 and their logits bit-exact, the rest close."""
    lib = M.lib()
    M.check(lib.mmoe_set_router_mode(0), "router mode")
    try:
        compare_layer(layer0, 520, M.ORDER_BATCH, " mfma router", refined=True)
    finally:
        M.check(lib.mmoe_set_router_mode(0), "router mode")


@pytest.fixture(scope="module", params=[52, 253, "round"])
def tie_layer(request):
    """Layers 19 and 20: router weights all zero and a bias with large tie classes, so every logit is its expert's
    bias exactly: 3 distinct leaders, then a class of equal logits across the 8th place. Layer 19: 52 experts
    (e * 37 % 5 == 4); layer 20: the 253 other experts all equal (every lane holds four tied experts, so each
    pick after the third must find the lowest lane and, inside it, the lowest slot).
    Layer 21 ("round"): leaders 0.03, 0.02, 0.015, every other logit 0 except expert 200 at 1e-30. Its logit is
    the 4th largest, but 1e-30 - 0.03 rounds to -0.03, so its p equals the tied class's and maple.c takes the
    lowest experts 0, 1, 2, 4, 5 first: a selection on logits alone picks 200, and only the check against p
    (then a selection on p) gives maple.c's picks."""
    lib = M.lib()
    M.check(lib.mmoe_init(2048), "mmoe_init")
    L = {52: 19, 253: 20, "round": 21}[request.param]
    hl = HostLayer(SEED, L)
    hl.router = np.zeros((256, 2048), np.uint16)
    hl.rid = M.register_layer(L, hl.blk, hl.router)
    if request.param == 52:
        hl.bias = ((np.arange(256) * 37) % 5).astype(np.float32) * 0.25
        hl.want = [250, 3, 180] + [e for e in range(256) if e * 37 % 5 == 4][:5]
    else:
        hl.bias = np.zeros(256, np.float32)
        hl.want = [250, 3, 180, 0, 1, 2, 4, 5]
    if request.param == "round":
        hl.bias[[250, 3, 180, 200]] = [0.03, 0.02, 0.015, 1e-30]
    else:
        hl.bias[[250, 3, 180]] = [3.0, 2.5, 2.25]
    M.check(lib.mmoe_set_bias(L, M.ptr(hl.bias)), "bias")
    yield hl
    M.check(lib.mmoe_set_bias(L, None), "bias off")


@pytest.mark.parametrize("nb,order", [(1, 1), (1, 0), (5, 0), (64, 0), (600, 0)])
def test_topk_ties_pick_lowest_index(tie_layer, nb, order):
    """Equal logits give equal softmax probabilities, and maple.c's repeated strict-> scans (maple.c:913-923)
    then pick the lowest expert index first: expected top-8 = 250, 3, 180, then the 5 lowest experts of the tied
    class. Checked against the oracle for the decode kernels (nb 1, both orders), small batches (nb 5), the
    fused small-tile path (nb 64) and the MFMA router with exact refinement (nb 600, where every tied expert is
    a candidate); top-8, weights, grouping and x."""
    lib = M.lib()
    M.check(lib.mmoe_set_debug(1), "debug")
    M.check(lib.mmoe_set_router_mode(0), "router mode")
    hl = tie_layer
    x, hn = normed_hidden(SEED, 700 + nb, nb)
    xg = run_gpu(hl.L, hn, x, order)
    xo = x.copy()
    if order == M.ORDER_STEP:
        o = O.moe_step(hn[0], hl.router, hl.table, xo[0], bias=hl.bias)
    else:
        o = O.moe_batch(hn, hl.router, hl.table, xo, bias=hl.bias)
    want = hl.want
    otop = o["top"].reshape(nb, 8)
    assert (otop == np.array(want)).all(), "oracle picks"
    assert np.array_equal(M.read("TOP", (nb, 8), np.int32), otop), "top-8 indices differ"
    assert np.array_equal(M.read("TW", (nb, 8), np.float32).view(np.int32), o["tw"].reshape(nb, 8).view(np.int32)), "weights differ"
    assert np.array_equal(M.read("UTOK", (nb * 8,), np.int32), o["utok"]), "grouping differs"
    assert relmax(xg - x, xo - x) <= TOL
    print(f"\n  nb={nb} order={order}: top-8 {want}; x bit-exact {np.array_equal(xg, xo)}")


def test_moe_batch_tn64_compact_sums(layer0):
    """With checks off the 64-token-tile path hands gate/up sums to k_act_quant and down results to k_combine as
    int16 (d = sum - qsum, int32 side buffer for the rare out-of-range entry): act int8 and x must still match."""
    lib = M.lib()
    M.check(lib.mmoe_set_debug(0), "debug off")
    try:
        nb = 256
        x, hn = normed_hidden(SEED, 77, nb)
        xg = run_gpu(layer0.L, hn, x, M.ORDER_BATCH)
        xo = x.copy()
        o = O.moe_batch(hn, layer0.router, layer0.table, xo)
        P = nb * 8
        qa = M.mfma_to_natural(M.read("QA", (P, 512), np.int8), 512)
        assert np.array_equal(qa, o["qa"]), "act int8 differs"
        assert np.array_equal(M.read("QSUMA", (P,), np.int32), o["qsuma"])
        assert relmax(xg - x, xo - x) <= TOL   # down results travel as int16 to the combine here
        print("\n  compact sums: x bit-exact", np.array_equal(xg, xo))
    finally:
        M.check(lib.mmoe_set_debug(1), "debug on")


@pytest.fixture(scope="module")
def zipf_layer():
    """Layer 6: its own experts and router plus the bench's Zipf(1.1) expert bias (config 2)"""
    lib = M.lib()
    M.check(lib.mmoe_init(2048), "mmoe_init")
    hl = HostLayer(SEED, 6)
    hl.rid = M.register_layer(6, hl.blk, hl.router)
    hl.bias = M.zipf_bias(SEED, 1.1)
    M.check(lib.mmoe_set_bias(6, M.ptr(hl.bias)), "bias")
    yield hl
    M.check(lib.mmoe_set_bias(6, None), "bias off")


@pytest.mark.parametrize("T", [2048, 2047])
def test_full_size_tokens_independent(zipf_layer, T):
    """BASELINE config 2 at full size (2048 Zipf-routed tokens, checks off: the int16 / fused-activation path).
    Each token's MoE output depends on that token only, and the batch combine sums a token's pairs in ascending
    expert order whatever the batch, so the full batch must reproduce, bit for bit, the rows of sub-batches run
    alone (two halves, and a scattered 48-token sample); the sample is also checked against the oracle. Runs
    with the exact router option, so that the 48-token sample (chain router) and the full batch share every
    logit; test_zipf_mfma_router_matches_exact covers the default MFMA router at this size."""
    lib = M.lib()
    L = zipf_layer.L
    M.check(lib.mmoe_set_debug(0), "debug off")
    M.check(lib.mmoe_set_router_mode(1), "router mode")
    try:
        x, hn = normed_hidden(SEED, 500 + T, T)
        xf = run_gpu(L, hn, x, M.ORDER_BATCH)
        h = T // 2
        for lo, hi in ((0, h), (h, T)):
            xs = run_gpu(L, np.ascontiguousarray(hn[lo:hi]), np.ascontiguousarray(x[lo:hi]), M.ORDER_BATCH)
            assert np.array_equal(xs, xf[lo:hi]), f"rows {lo}..{hi} differ from the full batch"
        rng = np.random.default_rng(T)
        idx = np.sort(rng.choice(T, 48, replace=False))
        hs, xsmp = np.ascontiguousarray(hn[idx]), np.ascontiguousarray(x[idx])
        xg = run_gpu(L, hs, xsmp, M.ORDER_BATCH)
        assert np.array_equal(xg, xf[idx]), "sampled rows differ from the full batch"
        xo = xsmp.copy()
        O.moe_batch(hs, zipf_layer.router, zipf_layer.table, xo, bias=zipf_layer.bias)
        assert relmax(xf[idx] - xsmp, xo - xsmp) <= TOL
        print(f"\n  T={T}: halves and sample bit-exact; sample vs oracle bit-exact {np.array_equal(xf[idx], xo)}")
    finally:
        M.check(lib.mmoe_set_router_mode(0), "router mode")
        M.check(lib.mmoe_set_debug(1), "debug on")


def test_rejects_sizes_outside_capacity(layer0):
    """Sizes outside what mmoe_init / gpux_init allocated are refused on the host with an error and no device
    work (maple.c never calls these hooks with an empty chunk; the refusal is this library's contract), and
    the library stays usable: a valid call afterwards still matches the oracle."""
    lib = M.lib()
    x, hn = normed_hidden(SEED, 902, 2)
    x_in = x.copy()
    for nb in (0, -1, 2049):
        assert lib.mmoe_moe(0, M.ptr(hn), nb, M.ptr(x), M.ORDER_BATCH) == -1
        assert b"outside" in lib.mmoe_last_error(), lib.mmoe_last_error()
    assert lib.mmoe_moe(-1, M.ptr(hn), 2, M.ptr(x), M.ORDER_BATCH) == -1
    assert lib.mmoe_moe(64, M.ptr(hn), 2, M.ptr(x), M.ORDER_BATCH) == -1      # past the 64 layer slots
    assert np.array_equal(x, x_in), "a refused call wrote the hidden state"
    # gpre_moe: an empty chunk, and a pair whose token lies outside the chunk
    ustart = np.array([0, 8], np.int32); utok = np.zeros(8, np.int32); uw = np.full(8, 0.125, np.float32)
    tp = np.tile(np.arange(8, dtype=np.int32), 2)
    loc = M.block_loc(0, [5]); regs = np.array([layer0.rid, -1, -1, -1], np.int32)
    y = np.zeros((2, 2048), np.float32)
    assert lib.gpre_moe(M.ptr(hn), 0, 1, M.ptr(loc), M.ptr(regs), None, M.ptr(ustart), M.ptr(utok), M.ptr(uw),
                        M.ptr(tp), M.ptr(y)) < 0
    bad = utok.copy(); bad[3] = 2
    assert lib.gpre_moe(M.ptr(hn), 2, 1, M.ptr(loc), M.ptr(regs), None, M.ptr(ustart), M.ptr(bad), M.ptr(uw),
                        M.ptr(tp), M.ptr(y)) < 0
    assert b"ptok" in lib.mmoe_last_error(), lib.mmoe_last_error()
    assert not y.any(), "a refused gpre_moe wrote its output"
    # gpux_begin: no slots
    assert not lib.gpux_begin(0, M.ptr(hn[0]), 0, M.ptr(np.zeros(1, np.int32)))
    # still usable
    compare_layer(layer0, 4, M.ORDER_BATCH)


def test_combine_int16_overflow():
    """Down results past int16 (the -32768 marker and the int32 side buffer): expert 5 of a layer gets gate, up and
    down codes all +1 and a large router bias, so every token routes to it; with positive inputs its gate and up
    clamp at 7, every act value quantises to 127 and each down sum is 512 x 127 = 65024. Checks off (int16 down
    results into k_combine16): x against the oracle."""
    lib = M.lib()
    M.check(lib.mmoe_init(2048), "mmoe_init")
    L, e = 7, 5
    blk = M.synth_layer_block(SEED, L)
    base = e * M.EXPERT_BYTES
    for m in (0, 2, 4):   # gate codes, up codes, down codes: bytes 0xAA = four codes 2 (w = +1)
        off = base + M.EXPERT_OFFS[m]
        blk[off:off + 262144] = 0xAA
    router = M.synth_router(SEED, L, 0)
    rid = M.register_layer(L, blk, router)
    bias = np.zeros(256, np.float32); bias[e] = 100.0
    M.check(lib.mmoe_set_bias(L, M.ptr(bias)), "bias")
    M.check(lib.mmoe_set_debug(0), "debug off")
    try:
        nb = 256
        rng = np.random.default_rng(SEED + 5)
        hn = np.abs(rng.standard_normal((nb, 2048))).astype(np.float32)
        x = rng.standard_normal((nb, 2048)).astype(np.float32)
        xg = run_gpu(L, hn, x, M.ORDER_BATCH)
        xo = x.copy()
        o = O.moe_batch(hn, router, O.experts_table(blk), xo, bias=bias, want=("top", "qa", "dn_i32"))
        assert (o["top"] == e).any(axis=1).all(), "every token routes to the all-ones expert"
        big = int((np.abs(o["dn_i32"].astype(np.int64) - o["qa"].astype(np.int64).sum(1, keepdims=True)) > 32767).sum())
        print(f"\n  down sums past int16: {big}; x bit-exact {np.array_equal(xg, xo)}, relmax {relmax(xg - x, xo - x):.1e}")
        assert big > 0
        assert relmax(xg - x, xo - x) <= TOL
    finally:
        M.check(lib.mmoe_set_debug(1), "debug on")
        M.check(lib.mmoe_set_bias(L, None), "bias off")


def test_flip_token_matches_oracle(layer0):
    """the golden token whose re-quantised act maple.c's AVX2 build rounds across an int8 boundary (a tie within
    an ulp, tests/test_golden.py): the card equals the oracle bit for bit, and differs from maple.c's AVX2 output
    in exactly that one value, which maple.c's -march=native build rounds as the card does"""
    from test_golden import flip_inputs
    f, hl, hn = flip_inputs()
    assert hl.L == 0 and np.array_equal(hl.router, layer0.router)
    for dec in (1, 0):                                   # the decode kernels and the grouped-GEMM kernels
        M.check(M.lib().mmoe_set_decode_path(dec), "decode path")
        xg = run_gpu(0, hn, np.zeros((1, 2048), np.float32), M.ORDER_BATCH)
        xo = np.zeros((1, 2048), np.float32)
        o = O.moe_batch(hn, hl.router, hl.table, xo, want=("top", "act", "qa"))
        qa = M.mfma_to_natural(M.read("QA", (8, 512), np.int8), 512)
        assert np.array_equal(qa, o["qa"]) and np.array_equal(xg.view(np.int32), xo.view(np.int32))
        assert int((qa != f["avx2_qa"]).sum()) == 1 and np.array_equal(qa, f["native_qa"])
        assert relmax(xg, f["native_xout"]) <= TOL
    M.lib().mmoe_set_decode_path(1)


def bound_share(router, hn, ra, rx):
    """largest |approximate - exact| logit as a share of the refinement's bound err_b = RG_ERRK x sw, sw the
    smaller of max|h| max_e sum|w_e| and |h|_2 max_e |w_e|_2 (both bound sum_c |w_ec h_c|), as the kernel forms it"""
    wf = (router.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    w1max = np.abs(wf).sum(1).max() * 1.001
    w2max = np.sqrt((wf ** 2).sum(1)).max() * 1.001
    h = hn.astype(np.float64)
    sw = np.minimum(np.abs(h).max(1) * w1max, np.sqrt((h ** 2).sum(1)) * 1.001 * w2max)
    err_b = 2.0 * (399.0 + 1024.0) * 1.01 / 2 ** 24 * sw   # RG_ERRK of the default two-part MFMA router
    return float((np.abs(ra.astype(np.float64) - rx) / err_b[:, None]).max())


def test_zipf_mfma_router_matches_exact(zipf_layer):
    """Config 2 (2048 Zipf-routed tokens) with the MFMA router against the exact chain router: identical top-8,
    the picked experts' logits bit for bit, tw and x within the bar; and, with the MFMA router too, each token's
    result independent of the rest of the batch (halves bit-exact)."""
    lib = M.lib()
    L, T = zipf_layer.L, 2048
    M.check(lib.mmoe_set_debug(0), "debug off")
    x, hn = normed_hidden(SEED, 4100, T)
    try:
        out = {}
        for mode in (1, 0):
            M.check(lib.mmoe_set_router_mode(mode), "router mode")
            xg = run_gpu(L, hn, x, M.ORDER_BATCH)
            out[mode] = (xg, M.read("TOP", (T, 8), np.int32), M.read("TW", (T, 8), np.float32), M.read("LOGITS", (T, 256), np.float32))
        (x1, t1, w1, r1), (x0, t0, w0, r0) = out[1], out[0]
        assert np.array_equal(t0, t1), f"top-8 differs on {int((t0 != t1).any(1).sum())} tokens"
        sel = np.take_along_axis(r0, t0, 1).view(np.int32), np.take_along_axis(r1, t1, 1).view(np.int32)
        assert np.array_equal(*sel), "the picked experts' logits differ"
        print(f"\n  mfma vs exact router: tw relmax {relmax(w0, w1):.1e}, x relmax {relmax(x0 - x, x1 - x):.1e}, "
              f"other logits relmax {relmax(r0, r1):.1e}")
        assert relmax(w0, w1) <= TOL and relmax(x0 - x, x1 - x) <= TOL
        # how close the MFMA logits came to the refinement's rounding bound: every approximate logit's distance
        # from its exact chain value, as a share of the token's bound err_b (the kernel's candidate margin is
        # twice err_b, so a share below 1 leaves every non-candidate provably outside the exact top 8)
        share = bound_share(zipf_layer.router, hn, r0, r1)
        print(f"  largest |approximate - exact| logit: {share:.3f} of the bound err_b")
        assert share < 1.0
        h = T // 2
        for lo, hi in ((0, h), (h, T)):
            xs = run_gpu(L, np.ascontiguousarray(hn[lo:hi]), np.ascontiguousarray(x[lo:hi]), M.ORDER_BATCH)
            assert np.array_equal(xs, x0[lo:hi]), f"rows {lo}..{hi} differ from the full batch"
    finally:
        M.check(lib.mmoe_set_router_mode(0), "router mode")
        M.check(lib.mmoe_set_debug(1), "debug on")


@pytest.mark.parametrize("nb", [9, 100, 255])
def test_expert16_fused_matches_three_kernels(zipf_layer, nb):
    """Tiles of 16 pairs: the fused whole-expert kernel (grouping, gate/up, act quantisation and down in one launch)
    against k_group and the three separate kernels, bit for bit in every intermediate (the grouping's utok, uw,
    tp, sp and plan, int32 sums, act, its int8 quantisation, down) and in x. The Zipf bias gives experts of many tiles (the hot expert gets most tokens) next to single-pair
    tiles, so ragged tiles, padding rows and several workgroups per expert all occur."""
    lib = M.lib()
    L = zipf_layer.L
    x, hn = normed_hidden(SEED, 4200 + nb, nb)
    P = nb * 8
    out = {}
    M.check(lib.mmoe_set_debug(1), "debug on")
    try:
        for fused in (0, 1):
            M.check(lib.mmoe_set_expert_path(fused), "expert path")
            xg = run_gpu(L, hn, x, M.ORDER_BATCH)
            out[fused] = [xg] + [M.read(n, (P, k), t) for n, k, t in (("GU_I32", 1024, np.int32), ("ACT", 512, np.float32),
                                                                     ("QA", 512, np.int8), ("QSA", 1, np.float32),
                                                                     ("QSUMA", 1, np.int32), ("DN_I32", 2048, np.int32),
                                                                     ("DOWN", 2048, np.float32), ("UTOK", 1, np.int32),
                                                                     ("UW", 1, np.float32), ("TP", 1, np.int32),
                                                                     ("SP", 1, np.int32))]
            plan = M.read_plan()
            out[fused] += [np.asarray(plan["ue"]), np.asarray(plan["ustart"]), np.array([plan["nu"], plan["np"], plan["ntile"], plan["tn"]])]
        cnt = np.diff(M.read_plan()["ustart"])
        print(f"\n  nb={nb}: {len(cnt)} experts, largest {cnt.max()} pairs ({int(((cnt + 15) // 16).sum())} tiles)")
        assert nb <= 16 or cnt.max() > 16
        for name, a, b in zip(("x", "GU_I32", "ACT", "QA", "QSA", "QSUMA", "DN_I32", "DOWN", "UTOK", "UW", "TP", "SP",
                               "plan ue", "plan ustart", "plan nu np ntile tn"), out[0], out[1]):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"{name} differs"
    finally:
        M.check(lib.mmoe_set_expert_path(1), "expert path")


@pytest.mark.parametrize("nb", [12, 40])
def test_step_order_batch_matches_oracle(layer0, nb):
    """A batch in step order above the decode path (the chain router's step order, the grouping inside the
    small-tile kernel, the combine over slots sp/tw): every token's x equals maple.c's step() on that token alone,
    here the oracle's step restatement on sampled tokens, bit for bit in the top-8 and within the bar in x."""
    x, hn = normed_hidden(SEED, 4300 + nb, nb)
    xg = run_gpu(layer0.L, hn, x, M.ORDER_STEP)
    top = M.read("TOP", (nb, 8), np.int32)
    for b in (0, nb // 2, nb - 1):
        xo = x[b].copy()
        o = O.moe_step(hn[b], layer0.router, layer0.table, xo)
        assert np.array_equal(top[b], o["top"].reshape(8)), f"token {b}: top-8 differs"
        e = relmax(xg[b] - x[b], xo - x[b])
        print(f"\n  nb={nb} token {b}: x bit-exact {np.array_equal(xg[b], xo)}, relmax {e:.1e}")
        assert e <= TOL


def test_mfma_router_large_bias(zipf_layer):
    """The MFMA router's candidate margin with a bias far larger than the logits themselves: the final bias add
    rounds relative to |logit + bias| (ulp 2^-5 at 2^18), and the margin covers that term too. Biases of 2^18 plus
    the Zipf values put many experts within a few ulp of the 8th place; the MFMA router with refinement must pick
    the exact chain router's top-8 (ties to the lowest index) with the same logits for the picks, at 600 tokens."""
    lib = M.lib()
    L, T = zipf_layer.L, 600
    big = (np.float32(262144.0) + zipf_layer.bias).astype(np.float32)
    M.check(lib.mmoe_set_bias(L, M.ptr(big)), "bias")
    x, hn = normed_hidden(SEED, 4400, T)
    try:
        out = {}
        for mode in (1, 0):
            M.check(lib.mmoe_set_router_mode(mode), "router mode")
            xg = run_gpu(L, hn, x, M.ORDER_BATCH)
            out[mode] = (xg, M.read("TOP", (T, 8), np.int32), M.read("LOGITS", (T, 256), np.float32))
        (x1, t1, r1), (x0, t0, r0) = out[1], out[0]
        assert np.array_equal(t0, t1), f"top-8 differs on {int((t0 != t1).any(1).sum())} tokens"
        sel = np.take_along_axis(r0, t0, 1).view(np.int32), np.take_along_axis(r1, t1, 1).view(np.int32)
        assert np.array_equal(*sel), "the picked experts' logits differ"
        assert relmax(x0 - x, x1 - x) <= TOL
        srt = np.sort(r1, 1)
        near = int((srt[:, -9] >= srt[:, -8] - 2 ** -4).sum())
        print(f"\n  bias 2^18: top-8 identical; tokens with a 9th expert within 2 ulp of the 8th: {near}")
    finally:
        M.check(lib.mmoe_set_router_mode(0), "router mode")
        M.check(lib.mmoe_set_bias(L, M.ptr(zipf_layer.bias)), "bias")


def test_mfma_router_outlier_coordinate(zipf_layer):
    """Hidden states with one dominant coordinate (x[c] 300 times the rest before the norm, as attention outputs
    can make them): max|h| is then close to |h|_2, and the refinement's bound takes the Cauchy-Schwarz form
    |h|_2 max_e |w_e|_2 instead of max|h| max_e sum|w_e| (about 30 times smaller here), so few experts need their
    exact chains. The MFMA router must still give the exact router's top-8 and picked logits bit for bit, and
    every approximate logit must lie within the bound."""
    lib = M.lib()
    L, T = zipf_layer.L, 1024
    x, _ = normed_hidden(SEED, 4300, T)
    rng = np.random.default_rng(11)
    x[np.arange(T), rng.integers(0, M.H, T)] *= 300.0
    hn = np.empty_like(x)
    for b in range(T):
        O.oracle().mo_rmsnorm(O._p(x[b]), None, M.H, O._p(hn[b]))
    M.check(lib.mmoe_set_debug(0), "debug off")
    try:
        out = {}
        for mode in (1, 0):
            M.check(lib.mmoe_set_router_mode(mode), "router mode")
            xg = run_gpu(L, hn, x, M.ORDER_BATCH)
            out[mode] = (xg, M.read("TOP", (T, 8), np.int32), M.read("TW", (T, 8), np.float32), M.read("LOGITS", (T, 256), np.float32))
        (x1, t1, w1, r1), (x0, t0, w0, r0) = out[1], out[0]
        assert np.array_equal(t0, t1)
        assert np.array_equal(np.take_along_axis(r0, t0, 1).view(np.int32), np.take_along_axis(r1, t1, 1).view(np.int32))
        assert relmax(w0, w1) <= TOL and relmax(x0 - x, x1 - x) <= TOL
        share = bound_share(zipf_layer.router, hn, r0, r1)
        wf = (zipf_layer.router.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        h = hn.astype(np.float64)
        ratio = float(np.median((np.abs(h).max(1) * np.abs(wf).sum(1).max()) / (np.sqrt((h ** 2).sum(1)) * np.sqrt((wf ** 2).sum(1)).max())))
        print(f"\n  outlier rows: largest |approximate - exact| {share:.3f} of err_b; Hoelder / Cauchy-Schwarz bound {ratio:.1f}x")
        assert share < 1.0
    finally:
        M.check(lib.mmoe_set_router_mode(0), "router mode")
        M.check(lib.mmoe_set_debug(1), "debug on")
