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
        M.slib().mmoe_synth_expert(seed, 0, k, M.ptr(gc), M.ptr(gs), M.ptr(uc), M.ptr(us), M.ptr(dc), M.ptr(ds))
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


VOCAB, NKV, HD = 151936, 4, 128


def pack_codes(c):
    """codes[rows][cols] in {0,1,2} -> the packed layout of convert.py:29-33 (128-column groups of 32 bytes, byte j
    holding columns j, j+32, j+64, j+96 at bits 0,2,4,6)"""
    r, n = c.shape
    g = c.reshape(r, n // 128, 4, 32).astype(np.uint8)
    return (g[:, :, 0] | (g[:, :, 1] << 2) | (g[:, :, 2] << 4) | (g[:, :, 3] << 6)).reshape(r, n // 4)


def write_model_checkpoint(d, seed, nexp=16, vocab_rows=4096):
    """A whole-model directory in maple.c's format (every record at its real shape) that maple.c itself can run:
    embeddings and lm_head share one record of VOCAB x 2048 bf16 whose first `vocab_rows` rows are random and the
    rest a sparse (unwritten, zero) tail of the shard; 2 variants of norms, router and attention projections,
    alternating over the layers; `nexp` distinct experts (expert e of layer L is distinct (7 e + L) % nexp).
    Returns the number of vocabulary rows with data (prompt ids must lie below it)."""
    os.makedirs(d, exist_ok=True)
    rng = np.random.default_rng(seed)
    sh = [Shard() for _ in range(9)]
    bf = lambda a: (np.asarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)
    eoff = []
    for k in range(nexp):
        gc = np.empty((M.FF, M.H // 4), np.uint8); gs = np.empty(M.FF, np.float32)
        uc = np.empty((M.FF, M.H // 4), np.uint8); us = np.empty(M.FF, np.float32)
        dc = np.empty((M.H, M.FF // 4), np.uint8); ds = np.empty(M.H, np.float32)
        M.slib().mmoe_synth_expert(seed, 0, k, M.ptr(gc), M.ptr(gs), M.ptr(uc), M.ptr(us), M.ptr(dc), M.ptr(ds))
        g = sh[k % 2]
        o = (k % 2, g.put(gc), g.put(gs), g.put(uc), g.put(us), sh[2].put(dc), sh[2].put(ds))
        eoff.append(o)
    r_off = [sh[3].put(M.synth_router(seed, L, 0)) for L in range(2)]
    norm = lambda n: bf(rng.uniform(0.7, 1.3, n))
    var = []
    for v in range(2):
        t = {}
        for name, rows in (("q", NE // 16 * 128), ("k", NKV * HD), ("v", NKV * HD), ("o", M.H)):
            c = rng.choice(np.array([0, 1, 2], np.uint8), size=(rows, M.H), p=[0.3, 0.4, 0.3])
            t[name] = (sh[4].put(pack_codes(c)), sh[4].put(rng.uniform(0.01, 0.05, rows).astype(np.float32)), rows)
        t["in"] = sh[4].put(norm(M.H)); t["post"] = sh[4].put(norm(M.H))
        t["qn"] = sh[4].put(norm(HD)); t["kn"] = sh[4].put(norm(HD))
        var.append(t)
    o_norm = sh[4].put(np.full(M.H, 0x3F80, np.uint16))
    emb = sh[5].put(bf(rng.standard_normal((vocab_rows, M.H)) * 0.05))
    recs = [(ord("b"), 5, emb, 0, VOCAB, M.H), (ord("b"), 5, emb, 0, VOCAB, M.H), (ord("b"), 4, o_norm, 0, 1, M.H)]
    for L in range(NL):
        t = var[L % 2]
        recs += [(ord("b"), 4, t["in"], 0, 1, M.H), (ord("b"), 4, t["post"], 0, 1, M.H),
                 (ord("b"), 4, t["qn"], 0, 1, HD), (ord("b"), 4, t["kn"], 0, 1, HD),
                 (ord("b"), 3, r_off[L % 2], 0, NE, M.H)]
        for name in "qkvo":
            off, soff, rows = t[name]
            recs.append((ord("t"), 4, off, soff, rows, M.H))
        for e in range(NE):
            o = eoff[distinct(L, e, nexp)]
            recs.append((ord("t"), o[0], o[1], o[2], M.FF, M.H))
            recs.append((ord("t"), o[0], o[3], o[4], M.FF, M.H))
            recs.append((ord("t"), 2, o[5], o[6], M.H, M.FF))
    for k, s_ in enumerate(sh):
        with open(os.path.join(d, f"shard-{k + 1:05d}.bin"), "wb") as f:
            f.write(bytes(s_.buf) if k < 6 else b"\0" * 16)
            if k == 5:
                f.truncate(emb + VOCAB * M.H * 2)              # the zero tail of the vocabulary, not written
    with open(os.path.join(d, "layout.bin"), "wb") as f:
        for r in recs:
            f.write(REC.pack(*r))
    return vocab_rows
