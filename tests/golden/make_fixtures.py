"""Writes tests/golden/maple_moe_fixtures.npz: input/output vectors of maple.c's own MoE code (oracle/_ref,
compiled from /root/reference/maple.c), on seeded synthetic inputs that tests regenerate bit for bit.

Run in the build container (where /root/reference exists): python3 tests/golden/make_fixtures.py
The fixture holds only data: seeds, input checksums and expected outputs."""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "maple-runtime_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")]

import maplemoe as M  # noqa: E402
import pyoracle as O  # noqa: E402
from helpers import HostLayer, normed_hidden  # noqa: E402

SEED, LAYER, NB = 424242, 5, 6


def sha(a):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest(), np.uint8)


def main():
    R = O.ref(); R.ref_set_threads(1)
    hl = HostLayer(SEED, LAYER)
    R.ref_set_router(LAYER, O._p(hl.router))
    for e in range(256):
        R.ref_set_expert(LAYER, e, *[O._p(a) for a in M.expert_views(hl.blk, e)])
    out = dict(seed=np.array([SEED, LAYER, NB], np.int64), sha_block=sha(hl.blk), sha_router=sha(hl.router))
    # step_batch MoE block
    x, hn = normed_hidden(SEED, 1, NB)
    P = NB * 8
    xr = x.copy()
    a = {k: np.zeros(s, d) for k, s, d in [("rl", (NB, 256), np.float32), ("top", (NB, 8), np.int32), ("tw", (NB, 8), np.float32),
                                            ("nu", 1, np.int32), ("ue", 256, np.int32), ("us", 257, np.int32), ("ut", P, np.int32),
                                            ("uw", P, np.float32), ("G", (P, 512), np.float32), ("U", (P, 512), np.float32),
                                            ("A", (P, 512), np.float32), ("qa", (P, 512), np.int8), ("qsa", P, np.float32),
                                            ("D", (P, 2048), np.float32)]}
    R.ref_moe_batch(LAYER, O._p(hn), NB, O._p(xr), *[O._p(a[k]) for k in ("rl", "top", "tw", "nu", "ue", "us", "ut", "uw", "G", "U", "A", "qa", "qsa", "D")])
    nu = int(a["nu"][0])
    out.update(b_sha_hn=sha(hn), b_rl=a["rl"], b_top=a["top"], b_tw=a["tw"], b_ue=a["ue"][:nu], b_ustart=a["us"][:nu + 1],
               b_utok=a["ut"], b_uw=a["uw"], b_gate=a["G"], b_act=a["A"], b_qa=a["qa"], b_qsa=a["qsa"], b_down8=a["D"][:8],
               b_xout=xr)
    # step() MoE block, one token
    x1, hn1 = normed_hidden(SEED, 2, 1)
    xs = x1[0].copy(); rl = np.zeros(256, np.float32); top = np.zeros(8, np.int32); tw = np.zeros(8, np.float32)
    act = np.zeros((8, 512), np.float32); down = np.zeros((8, 2048), np.float32)
    R.ref_moe_step(LAYER, O._p(hn1[0]), O._p(xs), O._p(rl), O._p(top), O._p(tw), O._p(act), O._p(down))
    out.update(s_sha_hn=sha(hn1), s_rl=rl, s_top=top, s_tw=tw, s_act=act, s_xout=xs)
    # prep vectors of assorted scales
    rng = np.random.default_rng(SEED)
    px = (rng.standard_normal((24, 512)) * (10.0 ** rng.uniform(-3, 3, (24, 1)))).astype(np.float32)
    px[3] = 0.0
    pq = np.zeros((24, 512), np.int8); pqs = np.zeros(24, np.float32); pqsum = np.zeros(24, np.int32)
    for i in range(24):
        s = np.zeros(1, np.int32)
        pqs[i] = R.ref_prep(O._p(px[i]), 512, O._p(pq[i]), O._p(s)); pqsum[i] = s[0]
    out.update(p_x=px, p_q=pq, p_qs=pqs, p_qsum=pqsum)
    path = os.path.join(HERE, "maple_moe_fixtures.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {os.path.getsize(path)} bytes, {nu} experts used")


if __name__ == "__main__":
    main()
