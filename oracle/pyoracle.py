"""ctypes bindings of the checker: liboracle.so (the C restatement) and _ref/libmaple_ref.so (maple.c itself).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
H, NE, TOPK, FF = 2048, 256, 8, 512


def _p(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


class Expert(C.Structure):
    _fields_ = [("gc", C.c_void_p), ("gs", C.c_void_p), ("uc", C.c_void_p), ("us", C.c_void_p),
                ("dc", C.c_void_p), ("ds", C.c_void_p)]


class T2(C.Structure):
    """maple.c:36 T2 / mo_t2: packed codes, row scales, rows, cols"""
    _fields_ = [("p", C.c_void_p), ("s", C.c_void_p), ("rows", C.c_int), ("cols", C.c_int)]


class Trace(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("rl", "top", "tw", "nu", "ue", "ustart", "utok", "uw", "tp", "qx", "qsx",
                                           "qsumx", "gu_i32", "gate", "up", "act", "qa", "qsa", "qsuma", "dn_i32", "down")]


_or = None
_ref = None
_ref_native = None


def oracle():
    global _or
    if _or is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError("oracle/liboracle.so not built (make -C oracle)")
        _or = C.CDLL(path)
        vp, i = C.c_void_p, C.c_int
        for n, r, a in [("mo_prep", C.c_float, [vp, i, vp, vp]), ("mo_dot_i32", C.c_int32, [vp, vp, i]),
                        ("mo_router_batch", None, [vp, i, vp, vp, vp]), ("mo_router_step", None, [vp, vp, vp, vp]),
                        ("mo_exp", C.c_float, [C.c_float]), ("mo_topk", None, [vp, i, vp, vp]),
                        ("mo_group", i, [vp, vp, i, vp, vp, vp, vp, vp, vp]), ("mo_act", None, [vp, vp, vp, i]),
                        ("mo_rmsnorm", None, [vp, vp, i, vp]), ("mo_pack", None, [vp, i, i, vp]),
                        ("mo_unpack", None, [vp, i, i, vp]),
                        ("mo_moe_batch", None, [vp, i, vp, vp, vp, vp, vp, vp]),
                        ("mo_moe_step", None, [vp, vp, vp, vp, vp, vp]),
                        ("mo_experts_grouped", None, [vp, i, i, vp, vp, vp, vp, vp, vp, vp]),
                        ("mo_rope", None, [vp, vp]), ("mo_f16", None, [vp, vp, i]), ("mo_h2f", C.c_float, [C.c_uint16]),
                        ("mo_attend", None, [vp, vp, vp, i, i, i, i, vp, vp]),
                        ("mo_attn_chunk", None, [vp, i, i, i, i, vp, vp, vp, T2, T2, T2, T2, vp, vp, vp, vp, vp])]:
            f = getattr(_or, n)
            f.restype, f.argtypes = r, a
    return _or


def ref_available():
    return os.path.exists(os.path.join(HERE, "_ref", "libmaple_ref.so"))


def ref(native=False):
    """maple.c compiled from /root/reference (oracle/Makefile `ref`): -mavx2 -mfma -mf16c (the reference's
    AVX2 target), or native=True: its documented -march=native build on the build host."""
    global _ref, _ref_native
    lib = _ref_native if native else _ref
    if lib is None:
        name = "libmaple_ref_native.so" if native else "libmaple_ref.so"
        path = os.path.join(HERE, "_ref", name)
        if not os.path.exists(path):
            raise RuntimeError(f"oracle/_ref/{name} not built (make -C oracle ref)")
        lib = C.CDLL(path)
        if native:
            _ref_native = lib
        else:
            _ref = lib
        vp, i = C.c_void_p, C.c_int
        for n, r, a in [("ref_set_threads", i, [i]), ("ref_set_router", None, [i, vp]),
                        ("ref_set_expert", None, [i, i, vp, vp, vp, vp, vp, vp]),
                        ("ref_prep", C.c_float, [vp, i, vp, vp]), ("ref_dot_i32", None, [vp, i, i, vp, i, vp]),
                        ("ref_route_batch", None, [i, vp, i, vp]), ("ref_route_step", None, [i, vp, vp]),
                        ("ref_topk", None, [vp, i, vp, vp]), ("ref_group", i, [vp, vp, i, vp, vp, vp, vp, vp, vp]),
                        ("ref_rmsnorm", None, [vp, vp, i, vp]), ("ref_act", None, [vp, vp, vp, i]),
                        ("ref_moe_batch", None, [i, vp, i, vp] + [vp] * 14),
                        ("ref_moe_step", None, [i, vp, vp, vp, vp, vp, vp, vp]), ("ref_now", C.c_double, []), ("ref_set_bias", None, [vp]),
                        ("ref_ctx", i, []), ("ref_rope", None, [vp, i]), ("ref_f16", None, [vp, vp, i]),
                        ("ref_cs", None, [i, vp]), ("ref_set_attn", None, [i] + [vp] * 11),
                        ("ref_cache", None, [i, i, vp, vp, i]), ("ref_attn_chunk", None, [i, i, vp, i, i, vp])]:
            f = getattr(lib, n)
            f.restype, f.argtypes = r, a
    return lib


# ------------------------------------------------------------------ oracle wrappers
def prep(x):
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(x.shape[-1], np.int8); s = np.zeros(1, np.int32)
    qs = oracle().mo_prep(_p(x), x.shape[-1], _p(q), _p(s))
    return q, np.float32(qs), int(s[0])


def router_batch(hn, w, bias=None):
    hn = np.ascontiguousarray(hn, np.float32)
    rl = np.empty((hn.shape[0], NE), np.float32)
    oracle().mo_router_batch(_p(hn), hn.shape[0], _p(w), _p(bias), _p(rl))
    return rl


def router_step(hn, w, bias=None):
    hn = np.ascontiguousarray(hn, np.float32)
    rl = np.empty(NE, np.float32)
    oracle().mo_router_step(_p(hn), _p(w), _p(bias), _p(rl))
    return rl


def topk(rl):
    rl = np.ascontiguousarray(rl, np.float32).reshape(-1, NE)
    top = np.empty((rl.shape[0], TOPK), np.int32); tw = np.empty((rl.shape[0], TOPK), np.float32)
    oracle().mo_topk(_p(rl), rl.shape[0], _p(top), _p(tw))
    return top, tw


def group(top, tw):
    nb = top.shape[0]; P = nb * TOPK
    nu = np.zeros(1, np.int32); ue = np.zeros(NE, np.int32); us = np.zeros(NE + 1, np.int32)
    utok = np.zeros(P, np.int32); uw = np.zeros(P, np.float32); tp = np.zeros(P, np.int32)
    oracle().mo_group(_p(np.ascontiguousarray(top, np.int32)), _p(np.ascontiguousarray(tw, np.float32)), nb,
                      _p(nu), _p(ue), _p(us), _p(utok), _p(uw), _p(tp))
    n = int(nu[0])
    return dict(nu=n, ue=ue[:n], ustart=us[:n + 1], utok=utok, uw=uw, tp=tp.reshape(nb, TOPK))


def experts_table(blk):
    """Expert structs (oracle layout) for all 256 experts of a synthetic layer block"""
    from_base = blk.ctypes.data
    tab = (Expert * NE)()
    offs = (0, 262144, 264192, 526336, 528384, 790528)
    for e in range(NE):
        b = from_base + e * 798720
        tab[e] = Expert(*[b + o for o in offs])
    return tab


def new_trace(nb, P, want=("rl", "top", "tw", "nu", "ue", "ustart", "utok", "uw", "tp", "qx", "qsx", "qsumx", "gu_i32",
                           "gate", "up", "act", "qa", "qsa", "qsuma", "dn_i32", "down")):
    shapes = dict(rl=((nb, NE), np.float32), top=((nb, TOPK), np.int32), tw=((nb, TOPK), np.float32),
                  nu=((1,), np.int32), ue=((NE,), np.int32), ustart=((NE + 1,), np.int32), utok=((P,), np.int32),
                  uw=((P,), np.float32), tp=((nb, TOPK), np.int32), qx=((nb, H), np.int8), qsx=((nb,), np.float32),
                  qsumx=((nb,), np.int32), gu_i32=((P, 2 * FF), np.int32), gate=((P, FF), np.float32),
                  up=((P, FF), np.float32), act=((P, FF), np.float32), qa=((P, FF), np.int8), qsa=((P,), np.float32),
                  qsuma=((P,), np.int32), dn_i32=((P, H), np.int32), down=((P, H), np.float32))
    arrs = {k: np.zeros(*shapes[k]) for k in want}
    tr = Trace(**{k: v.ctypes.data for k, v in arrs.items()})
    return tr, arrs


def moe_batch(hn, router, experts, x, bias=None, rl_in=None, want=None):
    hn = np.ascontiguousarray(hn, np.float32); nb = hn.shape[0]
    tr, arrs = new_trace(nb, nb * TOPK, **({} if want is None else dict(want=want)))
    oracle().mo_moe_batch(_p(hn), nb, _p(router), _p(bias), _p(rl_in), C.cast(experts, C.c_void_p), _p(x), C.byref(tr))
    return arrs


def moe_step(hn, router, experts, x, bias=None):
    hn = np.ascontiguousarray(hn, np.float32)
    tr, arrs = new_trace(1, TOPK)
    oracle().mo_moe_step(_p(hn), _p(router), _p(bias), C.cast(experts, C.c_void_p), _p(x), C.byref(tr))
    return arrs


# ------------------------------------------------------------------ attention half (maple.c:706-724)
WIN = 512


def rope_table(npos):
    """maple.c:1151-1152: (cos, sin) of pos * INV_FREQ[i] in double, stored as fp32; INV_FREQ (maple.c:1085)"""
    inv = 1.0 / np.power(10000.0, (2.0 * np.arange(32)) / 64)
    f = np.arange(npos, dtype=np.float64)[:, None] * inv[None, :]
    cs = np.empty((npos, 32, 2), np.float32)
    cs[..., 0] = np.cos(f).astype(np.float32); cs[..., 1] = np.sin(f).astype(np.float32)
    return cs


class AttnLayer:
    """Attention tensors of one layer in the reference layout (maple.c:38 Layer: in_ln, q_norm, k_norm bf16;
    q 2048x2048, k and v 512x2048, o 2048x2048 ternary with fp32 row scales), seeded."""

    def __init__(self, seed):
        rng = np.random.default_rng(seed)
        bf = lambda a: (np.asarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)
        self.in_ln = bf(rng.uniform(0.5, 1.5, H)); self.q_norm = bf(rng.uniform(0.5, 1.5, 128))
        self.k_norm = bf(rng.uniform(0.5, 1.5, 128))
        self.mats = {}
        for name, rows in (("q", 2048), ("k", 512), ("v", 512), ("o", 2048)):
            c = rng.choice(np.array([0, 1, 2], np.uint8), size=(rows, H), p=[0.3, 0.4, 0.3])
            packed = np.empty((rows, H // 4), np.uint8)
            oracle().mo_pack(_p(np.ascontiguousarray(c)), rows, H, _p(packed))
            self.mats[name] = (packed, rng.uniform(0.01, 0.05, rows).astype(np.float32))

    def t2(self, name):
        packed, s = self.mats[name]
        return T2(packed.ctypes.data, s.ctypes.data, packed.shape[0], H)


def attn_chunk(layer, x, pos0, glob, kc, vc, cs, win=WIN):
    """mo_attn_chunk: x [nb][2048] updated in a copy; kc/vc [ctx][512] fp16 updated in place; returns
    (x, ko [nb][1024], att [nb][2048])"""
    x = np.ascontiguousarray(x, np.float32).copy(); nb = x.shape[0]
    ko = np.zeros((nb, 1024), np.uint16); att = np.zeros((nb, H), np.float32)
    oracle().mo_attn_chunk(_p(x), nb, pos0, glob, win, _p(layer.in_ln), _p(layer.q_norm), _p(layer.k_norm),
                           layer.t2("q"), layer.t2("k"), layer.t2("v"), layer.t2("o"), _p(cs), _p(kc), _p(vc),
                           _p(ko), _p(att))
    return x, ko, att
