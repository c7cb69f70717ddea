"""Writes the golden vectors of maple.c's own MoE code (oracle/_ref, compiled from /root/reference/maple.c) on
seeded synthetic inputs that tests regenerate bit for bit:
  maple_moe_fixtures.npz         maple.c built for its AVX2 target (-O3 -ffast-math -mavx2 -mfma -mf16c)
  maple_moe_fixtures_native.npz  the same inputs through maple.c's documented build (-O3 -ffast-math
                                 -march=native, AVX-512 on the build host)
  maple_moe_flip_fixture.npz     one token of a 128-token chunk (BASELINE config 0 inputs) whose re-quantised
                                 act holds a value that maple.c's fast-math SiLU rounds across an int8 boundary
                                 relative to IEEE arithmetic; both builds' outputs for it

Run in the build container (where /root/reference exists): python3 tests/golden/make_fixtures.py
The fixtures hold only data: seeds, input checksums and expected outputs."""
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


FLIP_SEED, FLIP_SID, FLIP_NB, FLIP_LAYER = 20261201, 1128, 128, 0   # the config-0 chunk of tests/test_oracle_flips.py


def ref_token(R, L, hn):
    """maple.c's step_batch MoE block on one token (nb = 1): the token's top-8, act, qa, qsa and x out"""
    P = 8
    a = {k: np.zeros(s, d) for k, s, d in [("top", (1, 8), np.int32), ("tw", (1, 8), np.float32), ("A", (P, 512), np.float32),
                                            ("qa", (P, 512), np.int8), ("qsa", P, np.float32)]}
    x = np.zeros((1, 2048), np.float32)
    R.ref_moe_batch(L, O._p(hn), 1, O._p(x), None, O._p(a["top"]), O._p(a["tw"]), None, None, None, None, None, None, None,
                    O._p(a["A"]), O._p(a["qa"]), O._p(a["qsa"]), None)
    return a, x


def flip_fixture():
    """the first token of the config-0 chunk whose act int8 differ between maple.c and the oracle"""
    hl = HostLayer(FLIP_SEED, FLIP_LAYER)
    _, hn = normed_hidden(FLIP_SEED, FLIP_SID, FLIP_NB)
    out = dict(seed=np.array([FLIP_SEED, FLIP_LAYER, FLIP_SID, FLIP_NB], np.int64), sha_block=sha(hl.blk),
               sha_router=sha(hl.router))
    Rs = {}
    for tag, native in (("avx2", False), ("native", True)):
        R = O.ref(native); R.ref_set_threads(1)
        R.ref_set_router(FLIP_LAYER, O._p(hl.router))
        for e in range(256):
            R.ref_set_expert(FLIP_LAYER, e, *[O._p(a) for a in M.expert_views(hl.blk, e)])
        Rs[tag] = R
    for b in range(FLIP_NB):
        a, x = ref_token(Rs["avx2"], FLIP_LAYER, hn[b:b + 1])
        o = O.moe_batch(hn[b:b + 1], hl.router, hl.table, np.zeros((1, 2048), np.float32), want=("qa",))
        if (o["qa"] != a["qa"]).any():
            break
    else:
        raise SystemExit("no act flip in the config-0 chunk")
    out.update(token=np.array([b], np.int64), sha_hn=sha(hn[b:b + 1]))
    for tag, R in Rs.items():
        a, x = ref_token(R, FLIP_LAYER, hn[b:b + 1])
        out.update({f"{tag}_top": a["top"], f"{tag}_tw": a["tw"], f"{tag}_act": a["A"], f"{tag}_qa": a["qa"],
                    f"{tag}_qsa": a["qsa"], f"{tag}_xout": x})
    path = os.path.join(HERE, "maple_moe_flip_fixture.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {os.path.getsize(path)} bytes, token {b}")


def main(native=False):
    R = O.ref(native); R.ref_set_threads(1)
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
    path = os.path.join(HERE, "maple_moe_fixtures_native.npz" if native else "maple_moe_fixtures.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {os.path.getsize(path)} bytes, {nu} experts used")


if __name__ == "__main__":
    main(False)
    main(True)
    flip_fixture()
