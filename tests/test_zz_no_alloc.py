"""mmoe_moe_dev_noalloc (work buffers in the library's static scratch, no allocation) against mmoe_moe_dev on
the same inputs, bit for bit: two calls in a row, the second with a smaller batch, on the decode kernels
(<= 8 tokens) and on the grouped 16-token-tile kernels (9..64 tokens), in both summation orders, and with the
other kernel choices (the separate gate/up, quantisation and down kernels with k_group's per-chunk counts in the
scratch; the grouped kernels for <= 8 tokens); sizes past the scratch are refused."""
import numpy as np
import pytest

import maplemoe as M
from helpers import SEED, HostLayer, normed_hidden

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def layer():
    lib = M.lib()
    M.check(lib.mmoe_init(2048), "mmoe_init")
    M.check(lib.mmoe_set_debug(0), "debug off")
    M.check(lib.mmoe_set_decode_path(1), "decode path")
    hl = HostLayer(SEED, 11)
    M.register_layer(11, hl.blk, hl.router)
    return lib


def run(lib, fn, hn, x, order):
    d_h = lib.mmoe_dev_alloc(hn.nbytes); d_x = lib.mmoe_dev_alloc(x.nbytes)
    try:
        M.check(lib.mmoe_h2d(d_h, M.ptr(hn), hn.nbytes), "h2d"); M.check(lib.mmoe_h2d(d_x, M.ptr(x), x.nbytes), "h2d")
        M.check(fn(11, d_h, hn.shape[0], d_x, order), "moe")
        out = np.empty_like(x)
        M.check(lib.mmoe_d2h(M.ptr(out), d_x, x.nbytes), "d2h")
    finally:
        lib.mmoe_dev_free(d_h); lib.mmoe_dev_free(d_x)
    return out


@pytest.mark.parametrize("sizes,order", [((64, 9), M.ORDER_BATCH), ((48, 5), M.ORDER_BATCH), ((8, 1), M.ORDER_BATCH),
                                         ((1, 1), M.ORDER_STEP)])
def test_noalloc_matches_moe_dev(layer, sizes, order):
    lib = layer
    for k, nb in enumerate(sizes):
        print(f"\n  call {k}: nb={nb} order={order}", flush=True)
        x, hn = normed_hidden(SEED, 800 + 10 * nb + k, nb)
        want = run(lib, lib.mmoe_moe_dev, hn, x, order)
        got = run(lib, lib.mmoe_moe_dev_noalloc, hn, x, order)
        assert np.array_equal(got.view(np.int32), want.view(np.int32)), f"nb={nb}: differs from mmoe_moe_dev"
        assert not np.array_equal(got, x)


@pytest.mark.parametrize("fused,dec", [(0, 1), (1, 0), (0, 0)])
def test_noalloc_other_kernel_paths(layer, fused, dec):
    lib = layer
    M.check(lib.mmoe_set_expert_path(fused), "expert path")
    M.check(lib.mmoe_set_decode_path(dec), "decode path")
    try:
        for k, nb in enumerate((64, 9, 8, 3)):
            print(f"\n  fused={fused} dec={dec} call {k}: nb={nb}", flush=True)
            x, hn = normed_hidden(SEED, 900 + 10 * nb + k, nb)
            want = run(lib, lib.mmoe_moe_dev, hn, x, M.ORDER_BATCH)
            got = run(lib, lib.mmoe_moe_dev_noalloc, hn, x, M.ORDER_BATCH)
            assert np.array_equal(got.view(np.int32), want.view(np.int32)), f"nb={nb}: differs from mmoe_moe_dev"
            assert not np.array_equal(got, x)
    finally:
        M.check(lib.mmoe_set_expert_path(1), "expert path")
        M.check(lib.mmoe_set_decode_path(1), "decode path")


def test_noalloc_refuses_past_scratch(layer):
    lib = layer
    assert lib.mmoe_moe_dev_noalloc(11, None, 65, None, M.ORDER_BATCH) == -1
    assert b"outside 1..64" in lib.mmoe_last_error()
    assert lib.mmoe_moe_dev_noalloc(11, None, 0, None, M.ORDER_BATCH) == -1
