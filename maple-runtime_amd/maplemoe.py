"""ctypes binding of libmaplemoe (include/maplemoe.h) plus synthetic Maple-shaped layers.

The library is the product: a C ABI over hand-written gfx950 kernels. This module only loads it, declares the
signatures and offers numpy-friendly wrappers; it never computes anything itself and raises if the library
is missing (there is no fallback path).

Layer storage follows maple.c: a layer's 256 experts live in a region (gpre_region, maple.c:1125) and are
addressed through a location table loc[256][12] of (region slot, byte offset) pairs for gate codes, gate
scales, up codes, up scales, down codes, down scales (maple.c:276-277, 1106-1131).
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmaplemoe.so")
SYNTH_PATH = os.path.join(HERE, "libmaplesynth.so")   # synthetic data (bench and test tooling, not the path)

H, NE, TOPK, FF = 2048, 256, 8, 512
EXPERT_BYTES = 798720
# byte offsets of the six tensors inside one synthetic expert block (see csrc/synth.c)
EXPERT_OFFS = (0, 262144, 264192, 526336, 528384, 790528)
ORDER_BATCH, ORDER_STEP = 0, 1
COMBINE_OVERWRITE, COMBINE_BATCH, COMBINE_ADD, COMBINE_STEP = 0, 1, 4, 6
R = dict(LOGITS=0, TOP=1, TW=2, PLAN=3, UTOK=4, UW=5, TP=6, SP=7, QX=8, QSX=9, QSUMX=10, ACT=11, QA=12, QSA=13,
         QSUMA=14, DOWN=15, GU_I32=16, DN_I32=17, X=18, HN=19)
KERNELS = ["rmsnorm", "router", "topk", "group", "quant", "gateup", "quant_act", "down", "combine", "dense", "qkn",
           "att_scores", "att_softmax", "att_pv"]

_lib = None
_slib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (run __graft_entry__.build() or make -C maple-runtime_amd)")
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def slib():
    """libmaplesynth.so: seeded synthetic Maple-shaped data (include/maplesynth.h)"""
    global _slib
    if _slib is None:
        if not os.path.exists(SYNTH_PATH):
            raise RuntimeError(f"{SYNTH_PATH} is not built (make -C maple-runtime_amd)")
        _slib = C.CDLL(SYNTH_PATH)
        u64, i, d, vp, sz = C.c_uint64, C.c_int, C.c_double, C.c_void_p, C.c_size_t
        for name, (res, args) in {
            "mmoe_synth_expert": (None, [u64, i, i, vp, vp, vp, vp, vp, vp]), "mmoe_synth_expert_bytes": (sz, []),
            "mmoe_synth_layer": (None, [u64, i, vp, i]), "mmoe_synth_router": (None, [u64, i, i, vp]),
            "mmoe_synth_hidden": (None, [u64, i, i, vp]), "mmoe_synth_zipf_bias": (None, [u64, d, vp]),
        }.items():
            f = getattr(_slib, name)
            f.restype, f.argtypes = res, args
    return _slib


def _declare(L):
    vp, ip, fp, sz, i, d = C.c_void_p, C.POINTER(C.c_int), C.POINTER(C.c_float), C.c_size_t, C.c_int, C.c_double
    u8p, u16p, u32p, u64 = C.POINTER(C.c_uint8), C.POINTER(C.c_uint16), C.POINTER(C.c_uint32), C.c_uint64
    sig = {
        "gpre_init": (i, [i, i]), "gpre_region": (i, [vp, sz]), "gpre_stage": (i, [sz]),
        "gpre_moe": (d, [vp, i, i, vp, vp, vp, vp, vp, vp, vp, vp]), "gpre_blit_seconds": (d, []),
        "gpre_dense_done": (i, [i]), "gpre_dense_add": (None, [i, vp, vp, i, i]), "gpre_dense": (d, [i, vp, i, vp]), "mmoe_dense_reset": (i, []), "gfull_init": (i, [i, i, i, vp, vp, vp]),
        "gfull_begin": (None, [vp, i, i]), "gfull_attn": (d, [i, i, vp]),
        "gfull_moe": (None, [i, vp, vp, vp, vp, vp, vp]), "gfull_read": (None, [vp, vp]),
        "gfull_write_x": (None, [vp]), "gfull_maxtok": (i, []), "gfull_report": (None, []),
        "gpux_init": (i, [i, i]), "gpux_upload": (None, [i, i, vp, vp, vp, vp, vp, vp]),
        "gpux_begin": (vp, [i, vp, i, vp]), "gpux_end": (None, [vp, vp, i]),
        "gpux_begin_multi": (vp, [i, vp, i, i, vp, vp, vp]), "gpux_end_multi": (None, [vp, vp, i]),
        "gpu_head_init": (i, [vp, i, i]),
        "mmoe_init": (i, [i]), "mmoe_set_layer": (i, [i, vp, vp, vp, vp]), "mmoe_set_bias": (i, [i, vp]),
        "mmoe_moe": (i, [i, vp, i, vp, i]), "mmoe_moe_dev": (i, [i, vp, i, vp, i]), "mmoe_moe_dev_noalloc": (i, [i, vp, i, vp, i]),
        "mmoe_route": (i, [vp, i, vp, vp, vp, vp, vp, vp, vp]),
        "mmoe_rmsnorm_dev": (i, [vp, vp, i, vp]), "mmoe_stack_dev": (i, [i, i, vp, i, i]),
        "mmoe_stack_graph": (i, [i, i, vp, i, i, i]), "mmoe_graph_reset": (i, []), "mmoe_graph_held": (i, []),
        "mmoe_gfull_setup": (i, [i]), "mmoe_gfull_post_norm": (i, [i, vp]), "mmoe_gfull_stack": (i, [i, i]),
        "mmoe_read": (i, [i, vp, sz]), "mmoe_set_debug": (i, [i]), "mmoe_set_decode_path": (i, [i]), "mmoe_set_expert_path": (i, [i]), "mmoe_set_router_mode": (i, [i]), "mmoe_last_error": (C.c_char_p, []),
        "mmoe_dev_alloc": (vp, [sz]), "mmoe_dev_free": (i, [vp]), "mmoe_h2d": (i, [vp, vp, sz]),
        "mmoe_d2h": (i, [vp, vp, sz]), "mmoe_d2d": (i, [vp, vp, sz]), "mmoe_sync": (i, []), "mmoe_stream": (vp, []),
        "mmoe_event_record": (i, [i]), "mmoe_event_elapsed_ms": (d, []), "mmoe_prof": (i, [i]),
        "mmoe_prof_reset": (i, []), "mmoe_prof_get": (i, [i, C.POINTER(C.c_double), C.POINTER(C.c_long)]),
        "mmoe_device_info": (i, [C.c_char_p, i, ip, ip]),
        "mmoe_selftest_silu": (i, [C.c_uint32, C.c_uint32, C.POINTER(C.c_ulonglong), u32p]),
        "mmoe_ckpt_open": (i, [C.c_char_p]), "mmoe_ckpt_close": (None, []), "mmoe_ckpt_error": (C.c_char_p, []),
        "mmoe_ckpt_layer_plan": (i, [i, ip, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), vp]),
        "mmoe_ckpt_bf16": (vp, [i, i]), "mmoe_ckpt_load": (i, [i, i]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype, f.argtypes = res, args


def ptr(a):
    """data pointer of a numpy array; the caller must keep the array referenced until the call returns"""
    return None if a is None else C.c_void_p(a.ctypes.data)


def check(rc, what=""):
    if rc != 0:
        raise RuntimeError(f"{what}: {lib().mmoe_last_error().decode()}")


# ---------------------------------------------------------------- synthetic data (host)
def page_aligned(nbytes):
    """uint8 array of nbytes whose data pointer is page aligned (regions must be, maple.c:1117-1124)."""
    pg = os.sysconf("SC_PAGE_SIZE")
    raw = np.empty(nbytes + pg, np.uint8)
    off = (-raw.ctypes.data) % pg
    a = raw[off:off + nbytes]
    assert a.ctypes.data % pg == 0
    return a


def synth_layer_block(seed, L, nthreads=8):
    """All 256 experts of layer L, contiguous (EXPERT_BYTES each), page aligned."""
    blk = page_aligned(NE * EXPERT_BYTES)
    slib().mmoe_synth_layer(seed, L, ptr(blk), nthreads)
    return blk


def expert_views(blk, e):
    """(gc, gs, uc, us, dc, ds) numpy views of expert e inside a layer block"""
    b = blk[e * EXPERT_BYTES:(e + 1) * EXPERT_BYTES]
    o = EXPERT_OFFS
    return (b[o[0]:o[1]].reshape(FF, H // 4), b[o[1]:o[2]].view(np.float32),
            b[o[2]:o[3]].reshape(FF, H // 4), b[o[3]:o[4]].view(np.float32),
            b[o[4]:o[5]].reshape(H, FF // 4), b[o[5]:].view(np.float32))


def synth_router(seed, L, dist=0):
    w = np.empty((NE, H), np.uint16)
    slib().mmoe_synth_router(seed, L, dist, ptr(w))
    return w


def synth_hidden(seed, sid, nb):
    x = np.empty((nb, H), np.float32)
    slib().mmoe_synth_hidden(seed, sid, nb, ptr(x))
    return x


def zipf_bias(seed, s=1.1):
    b = np.empty(NE, np.float32)
    slib().mmoe_synth_zipf_bias(seed, s, ptr(b))
    return b


def block_loc(region_slot=0, experts=range(NE)):
    """loc table (maple.c:276 GLOC[L] layout) of a contiguous layer block registered as one region"""
    loc = np.zeros((len(list(experts)), 12), np.uint32)
    for u, e in enumerate(experts):
        for m in range(6):
            loc[u, 2 * m] = region_slot
            loc[u, 2 * m + 1] = e * EXPERT_BYTES + EXPERT_OFFS[m]
    return loc


def register_layer(L, blk, router, post_ln=None):
    """gpre_region the block, then mmoe_set_layer with its location table. Returns the region id."""
    rid = lib().gpre_region(ptr(blk), blk.nbytes)
    if rid < 0:
        raise RuntimeError("gpre_region: " + lib().mmoe_last_error().decode())
    regs = np.array([rid, -1, -1, -1], np.int32)
    loc = block_loc()  # keep every array alive across the call
    rw = np.ascontiguousarray(router)
    check(lib().mmoe_set_layer(L, ptr(loc), ptr(regs), ptr(rw), ptr(post_ln)), "mmoe_set_layer")
    return rid


def read(what, shape, dtype):
    a = np.empty(shape, dtype)
    check(lib().mmoe_read(R[what], ptr(a), a.nbytes), f"mmoe_read {what}")
    return a


def read_plan():
    p = np.empty(4 + 256 + 257 + 257, np.int32)
    check(lib().mmoe_read(R["PLAN"], ptr(p), p.nbytes), "mmoe_read plan")
    nu, np_, nt, tn = (int(v) for v in p[:4])
    ue = p[4:4 + 256][:nu].copy()
    ustart = p[260:260 + 257][:nu + 1].copy()
    return dict(nu=nu, np=np_, ntile=nt, tn=tn, ue=ue, ustart=ustart)


def mfma_to_natural(q, n):
    """int8 rows in mfma order (kernels.h) -> natural column order. q: [rows][n] int8."""
    rows = q.shape[0]
    g = q.reshape(rows, n // 128, 2, 4, 4, 4)        # [g][h][t][s][b]
    return g.transpose(0, 1, 4, 2, 3, 5).reshape(rows, n)  # column = s*32 + h*16 + t*4 + b


def device_info():
    name = C.create_string_buffer(64)
    cu, clk = C.c_int(0), C.c_int(0)
    check(lib().mmoe_device_info(name, 64, C.byref(cu), C.byref(clk)), "device_info")
    return name.value.decode(), cu.value, clk.value
