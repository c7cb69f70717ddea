"""A small checkpoint directory in maple.c's on-disk format (maple.c:61-83, layout.py), for the loader tests.

Nine shard files and layout.bin with the full 24-layer record table (packed '<BBQQII' records in layout.py's
order). Only `nexp` distinct synthetic experts are stored; expert e of layer L points at distinct expert
(7 e + L) % nexp, so the files stay a few MB while every record is valid. A record names one shard for its
codes and its scales (maple.c:70-72): gate and up tensors of even distinct experts sit in shard 1, of odd ones
in shard 2, down tensors in shard 3 (three regions per layer); the routers of even and odd layers in shard 4;
norms and the attention/embedding records (small stand-ins: the MoE path does not read them) in shard 5;
shards 6-9 hold 16 bytes each. Tensors start at 16-byte offsets that are not page multiples."""
import os
import struct

import numpy as np

import maplemoe as M

REC = struct.Struct("<BBQQII")
NL, NE = 24, 256


def distinct(L, e, nexp):
    return (7 * e + L) % nexp


class Shard:
    def __init__(self):
        self.buf = bytearray(b"\x5a" * 5008)        # a prefix, so spans do not start on a page

    def put(self, arr):
        off = len(self.buf)
        self.buf += np.ascontiguousarray(arr).tobytes()
        self.buf += b"\0" * (-len(self.buf) % 16)
        return off


def write_checkpoint(d, seed, nexp=6, gu_shards=2):
    """Writes the directory (gate/up of distinct expert k in shard k % gu_shards + 1); returns dict(experts=[(gc, gs, uc, us, dc, ds) numpy arrays], routers=[2 arrays],
    post_ln=array, recs=list of record tuples)."""
    os.makedirs(d, exist_ok=True)
    sh = [Shard() for _ in range(9)]
    experts, eoff = [], []
    for k in range(nexp):
        gc = np.empty((M.FF, M.H // 4), np.uint8); gs = np.empty(M.FF, np.float32)
        uc = np.empty((M.FF, M.H // 4), np.uint8); us = np.empty(M.FF, np.float32)
        dc = np.empty((M.H, M.FF // 4), np.uint8); ds = np.empty(M.H, np.float32)
        M.lib().mmoe_synth_expert(seed, 0, k, M.ptr(gc), M.ptr(gs), M.ptr(uc), M.ptr(us), M.ptr(dc), M.ptr(ds))
        experts.append((gc, gs, uc, us, dc, ds))
        g = sh[k % gu_shards]
        o_gc = g.put(gc); o_gs = g.put(gs); o_uc = g.put(uc); o_us = g.put(us)
        o_dc = sh[2].put(dc); o_ds = sh[2].put(ds)
        eoff.append((k % gu_shards, o_gc, o_gs, o_uc, o_us, o_dc, o_ds))
    routers = [M.synth_router(seed, L, 0) for L in range(2)]
    r_off = [sh[3].put(r) for r in routers]
    post_ln = (0x3F80 + (np.arange(M.H) % 7) - 3).astype(np.uint16)      # bf16 values near 1
    o_post = sh[4].put(post_ln)
    o_norm = sh[4].put(np.full(M.H, 0x3F80, np.uint16))
    o_small = sh[4].put(np.zeros(256, np.uint8))
    recs = []
    b = lambda off, rows, cols: (ord("b"), 4, off, 0, rows, cols)
    t_small = (ord("t"), 4, o_small, o_small + 128, 4, 128)               # 4 x 128: 128 B codes, 16 B scales
    recs += [b(o_norm, 1, 8), b(o_norm, 1, 8), b(o_norm, 1, M.H)]          # embeddings, lm_head, norm stand-ins
    for L in range(NL):
        recs += [b(o_norm, 1, M.H), b(o_post, 1, M.H), b(o_norm, 1, 128), b(o_norm, 1, 128)]
        recs.append((ord("b"), 3, r_off[L % 2], 0, NE, M.H))
        recs += [t_small] * 4
        for e in range(NE):
            o = eoff[distinct(L, e, nexp)]
            recs.append((ord("t"), o[0], o[1], o[2], M.FF, M.H))      # gate
            recs.append((ord("t"), o[0], o[3], o[4], M.FF, M.H))      # up
            recs.append((ord("t"), 2, o[5], o[6], M.H, M.FF))         # down
    for k, s_ in enumerate(sh):
        data = bytes(s_.buf) if k < 5 else b"\0" * 16
        with open(os.path.join(d, f"shard-{k + 1:05d}.bin"), "wb") as f:
            f.write(data)
    with open(os.path.join(d, "layout.bin"), "wb") as f:
        for r in recs:
            f.write(REC.pack(*r))
    return dict(experts=experts, routers=routers, post_ln=post_ln, recs=recs)
