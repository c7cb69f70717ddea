"""The oracle's attention half (mo_rope, mo_f16, mo_attend, mo_attn_chunk) pinned against maple.c itself
(oracle/_ref: rope, to_f16 and the statements of step_batch, maple.c:706-724) and against closed forms."""
import numpy as np
import pytest

import pyoracle as O
from helpers import relmax

H = 2048
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref (maple.c) not built")


def test_f16_closed_form():
    """mo_f16 is IEEE binary16 round-to-nearest-even (numpy's float16 cast); mo_h2f its exact inverse"""
    rng = np.random.default_rng(1)
    v = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
                        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 70000.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
                                  2.0 ** -14, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, np.inf, -np.inf], np.float32)])
    v = v.astype(np.float32)
    h = np.empty(v.size, np.uint16)
    O.oracle().mo_f16(O._p(v), O._p(h), v.size)
    assert np.array_equal(h, v.astype(np.float16).view(np.uint16))
    back = np.array([O.oracle().mo_h2f(int(x)) for x in h[:2000]], np.float32)
    assert np.array_equal(back, h[:2000].view(np.float16).astype(np.float32))


@needs_ref
def test_f16_matches_maple():
    rng = np.random.default_rng(2)
    v = (rng.standard_normal(4096) * 10.0 ** rng.integers(-8, 5, 4096)).astype(np.float32)
    a = np.empty(4096, np.uint16); b = np.empty(4096, np.uint16)
    O.oracle().mo_f16(O._p(v), O._p(a), 4096)
    O.ref().ref_f16(O._p(v), O._p(b), 4096)
    assert np.array_equal(a, b)


@needs_ref
def test_rope_table_and_rope_match_maple():
    npos = O.ref().ref_ctx()
    cs_ref = np.empty((npos, 32, 2), np.float32)
    O.ref().ref_cs(npos, O._p(cs_ref))
    cs = O.rope_table(npos)
    assert np.array_equal(cs.view(np.uint32), cs_ref.view(np.uint32))
    rng = np.random.default_rng(3)
    for pos in (0, 1, 7, 511, 512, 1000):
        v = rng.standard_normal(128).astype(np.float32)
        a, b = v.copy(), v.copy()
        O.oracle().mo_rope(O._p(a), O._p(cs[pos]))
        O.ref().ref_rope(O._p(b), pos)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), pos
    # closed form: a rotation of each (i, i+32) pair keeps its length
    v = rng.standard_normal(128).astype(np.float32); a = v.copy()
    O.oracle().mo_rope(O._p(a), O._p(cs[300]))
    n0 = v[:32] ** 2 + v[32:64] ** 2; n1 = a[:32] ** 2 + a[32:64] ** 2
    assert np.allclose(n0, n1, rtol=1e-5) and np.array_equal(a[64:], v[64:])


def attend_bruteforce(q, kc, vc, kvh, pos, glob, win=512):
    """float64 softmax attention over the fp16 cache, the definition the chains approximate"""
    lo = 0 if glob else max(0, pos - win)
    k = kc[lo:pos + 1, kvh * 128:(kvh + 1) * 128].view(np.float16).astype(np.float64)
    v = vc[lo:pos + 1, kvh * 128:(kvh + 1) * 128].view(np.float16).astype(np.float64)
    s = (q.reshape(4, 128).astype(np.float64) @ k.T) / np.sqrt(128.0)
    p = np.exp(s - s.max(1, keepdims=True)); p /= p.sum(1, keepdims=True)
    return p @ v


def test_attend_against_float64():
    rng = np.random.default_rng(4)
    ctx = 700
    kc = rng.standard_normal((ctx, 512)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((ctx, 512)).astype(np.float16).view(np.uint16)
    for pos, glob in ((0, 0), (5, 1), (600, 0), (600, 1)):
        q = rng.standard_normal(512).astype(np.float32)
        out = np.empty(512, np.float32); sc = np.empty(4 * ctx, np.float32)
        O.oracle().mo_attend(O._p(q), O._p(kc), O._p(vc), 2, pos, glob, 512, O._p(out), O._p(sc))
        want = attend_bruteforce(q, kc, vc, 2, pos, glob).ravel()
        assert relmax(out, want) < 2e-6, (pos, glob)


@needs_ref
@pytest.mark.parametrize("glob,pos0,nb", [(0, 600, 8), (1, 100, 16), (0, 0, 4)])
def test_attn_chunk_matches_maple(glob, pos0, nb):
    """mo_attn_chunk against maple.c's step_batch attention half on the same tensors, cache and input:
    the fp16 k/v written bit for bit; attention output and x within the documented bounds."""
    layer = O.AttnLayer(11)
    ref = O.ref()
    L = 0
    ref.ref_set_attn(L, O._p(layer.in_ln), O._p(layer.q_norm), O._p(layer.k_norm),
                     *[O._p(a) for n in "qkvo" for a in layer.mats[n]])
    ctx = ref.ref_ctx()
    rng = np.random.default_rng(12 + pos0)
    kc = np.zeros((ctx, 512), np.uint16); vc = np.zeros((ctx, 512), np.uint16)
    kc[:pos0] = rng.standard_normal((pos0, 512)).astype(np.float16).view(np.uint16)
    vc[:pos0] = rng.standard_normal((pos0, 512)).astype(np.float16).view(np.uint16)
    ref.ref_cache(L, pos0, O._p(kc), O._p(vc), 1)
    x0 = rng.standard_normal((nb, H)).astype(np.float32)
    cs = O.rope_table(ctx)
    xo, ko, att_o = O.attn_chunk(layer, x0, pos0, glob, kc, vc, cs)
    xr = x0.copy(); att_r = np.zeros((nb, H), np.float32)
    ref.ref_attn_chunk(L, glob, O._p(xr), nb, pos0, O._p(att_r))
    kr = np.zeros((pos0 + nb, 512), np.uint16); vr = np.zeros((pos0 + nb, 512), np.uint16)
    ref.ref_cache(L, pos0 + nb, O._p(kr), O._p(vr), 0)
    # v bit for bit; k within one fp16 ulp (maple.c's -ffast-math build may reorder the fp64 sum of squares of
    # its per-head rmsnorm, which moves a k value by an fp32 ulp and, rarely, its fp16 rounding)
    assert np.array_equal(vr[pos0:], vc[pos0:pos0 + nb])
    dk = np.abs(kr[pos0:].astype(np.int32) - kc[pos0:pos0 + nb].astype(np.int32))
    assert dk.max() <= 1 and (dk > 0).mean() < 1e-3
    assert np.array_equal(ko[:, :512], kc[pos0:pos0 + nb]) and np.array_equal(ko[:, 512:], vc[pos0:pos0 + nb])
    ea, ex = relmax(att_o, att_r), relmax(xo - x0, xr - x0)
    # x: the o projection quantises the attention output to int8 (prep); an att difference at the 1e-6 level
    # can move a value across a rounding boundary, which moves y by one quantum. Count those flips.
    flips = sum(int((O.prep(att_o[b])[0] != O.prep(att_r[b])[0]).sum()) for b in range(nb))
    print(f"\n  glob={glob} pos0={pos0} nb={nb}: k differs {int((dk > 0).sum())}/{dk.size} (1 ulp), att relmax "
          f"{ea:.2e}, x relmax {ex:.2e}, int8 flips {flips}/{nb * H}")
    assert ea < 2e-5
    assert flips <= 2e-3 * nb * H
    assert ex < (1e-5 if flips == 0 else 1e-3)
