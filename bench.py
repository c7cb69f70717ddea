#!/usr/bin/env python3
"""Benchmark of the MI355X MoE hot path on synthetic Maple-shaped data.

Default (the line the driver records): config 1, decode of 1 token through 24 stacked MoE layers
(rmsnorm + router + top-8 + grouping + int8 quant + gate/up/SiLU + re-quant + down + combine per layer),
expert codes resident in HBM. A "step" = one token through the 24 layers; value = tokens/s.
The same line carries the 2048-token prefill layer with Zipf-skewed routing (config 2) under "prefill".

roofline: the dominant kernel's algorithmic bytes (decode) or int8 ops (prefill) per launch divided by its
average launch time, measured with HIP events on the library stream in a separate profiling pass.
cpu_baseline: maple.c's own int8 AVX2 path (oracle/_ref, built from the reference sources) on the host.
"""
import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "maple-runtime_amd"), os.path.join(ROOT, "oracle")]

import numpy as np  # noqa: E402

import maplemoe as M  # noqa: E402

METRIC = "MoE tokens/s (2048-tok prefill, 1-tok decode); % int8-MFMA / HBM peak"   # BASELINE.json's metric
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
NL = 24
SEED = 20261201
CODES_SCALES_PER_EXPERT = 2 * (262144 + 2048) + (262144 + 8192)   # gate+up, down: 798,720 B
GU_BYTES_PER_EXPERT = 2 * (262144 + 2048)
DN_BYTES_PER_EXPERT = 262144 + 8192
OPS_GU_PER_PAIR = 2 * 1024 * 2048
OPS_DN_PER_PAIR = 2 * 2048 * 512


def pmc_traffic(kernel):
    """HBM bytes per dispatch of `kernel` from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary, or None."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        cols = [c.strip() for c in line.split("|")]
        # "k<a>" also names an instantiation with further template arguments, "k<a, ...>"
        if len(cols) > 6 and (cols[1] == kernel or (kernel.endswith(">") and cols[1].startswith(kernel[:-1] + ","))):
            return int(cols[6])
    return None


def pmc_mfma(kernel, workload):
    """counter-based MFMA figures of `kernel` (a prefix of its instantiation) at `workload` from the committed
    rocprofv3 summary: busy share of the 1024 SIMDs at the published clock over the kernel's duration, and the
    ops the MFMA pipes ran over the algorithmic ops (tile padding). None if the summary is absent."""
    path = os.path.join(ROOT, "profiles", "mfma_util.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        cols = [c.strip() for c in line.split("|")]
        if len(cols) > 12 and cols[1].startswith(kernel) and cols[2] == workload:
            try:
                return dict(busy_frac_at_peak_clock=float(cols[9]), mfma_util_rocprof=float(cols[8]),
                            padded_ops_ratio=round(float(cols[10]) / float(cols[11]), 3),
                            avg_launch_us_profiled=float(cols[4]), source="profiles/mfma_util.md")
            except ValueError:
                return None
    return None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def prof_pass(fn, reps):
    """per-kernel device execution time: every launch carries start/stop events on its own dispatch
    (hipExtLaunchKernel), so a kernel's figure is its run on the device, as rocprofv3 reports it.
    fn(i) is called for i in range(reps)."""
    lib = M.lib()
    lib.mmoe_prof_reset(); lib.mmoe_prof(1)
    for i in range(reps):
        fn(i)
    lib.mmoe_sync(); lib.mmoe_prof(0)
    out = {}
    import ctypes as C
    for k, name in enumerate(M.KERNELS):
        ms, n = C.c_double(0), C.c_long(0)
        lib.mmoe_prof_get(k, C.byref(ms), C.byref(n))
        if n.value:
            out[name] = (ms.value, n.value)
    return out


def timed(fn, steps, warmup):
    """fn(i) for the warm-up and the timed steps; events on the library stream around the timed ones"""
    lib = M.lib()
    for i in range(warmup):
        fn(i)
    lib.mmoe_sync()
    lib.mmoe_event_record(0)
    t0 = time.perf_counter()
    for i in range(steps):
        fn(warmup + i)
    lib.mmoe_event_record(1)
    lib.mmoe_sync()
    t1 = time.perf_counter()
    ev_ms = lib.mmoe_event_elapsed_ms()
    return ev_ms / steps, (t1 - t0) * 1e3 / steps


def cpu_topology():
    """lscpu's model name and physical core count of the host, and the cores this process may run on (its
    affinity mask: the box's CPU share). Falls back to /proc/cpuinfo when lscpu is absent."""
    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            info[k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    model = info.get("Model name")
    if not model:
        model = "unknown"
        try:
            for line in open("/proc/cpuinfo"):
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
        except OSError:
            pass
    try:
        phys = int(info["Socket(s)"]) * int(info["Core(s) per socket"])
    except (KeyError, ValueError):
        phys = None
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return model, phys, usable


def cpu_baselines(blocks, routers, seconds):
    """maple.c's own int8 AVX2 MoE code (oracle/_ref, built from the reference sources) on the host cores, on the
    same synthetic weights: step()'s MoE block for config 1 (24 layers per token) and step_batch's MoE block
    (maple.c:733-834) for configs 0 (128 tokens) and 2 (2048 tokens, Zipf-biased router). Each first on one
    thread (maple.c's run() with NT = 1: every job inline), then on all host threads (up to 16, NT-1 spinning
    workers as maple.c's main starts them; they are started once per process, so the one-thread legs go first)."""
    import pyoracle as O
    if not O.ref_available():
        return None
    R = O.ref()
    for L in range(NL):
        R.ref_set_router(L, O._p(routers[L]))
        for e in range(M.NE):
            R.ref_set_expert(L, e, *[O._p(a) for a in M.expert_views(blocks[L], e)])
    rp = M.synth_router(SEED, 0, dist=0)                 # prefill legs: layer 0's experts with a N(0, 0.02) router
    zb = M.zipf_bias(SEED, 1.1)
    ones = np.full(M.H, 0x3F80, np.uint16)
    x = M.synth_hidden(SEED, 77, 1)[0].copy()
    hn = np.empty_like(x)

    def token():
        for L in range(NL):
            R.ref_rmsnorm(O._p(x), O._p(ones), M.H, O._p(hn))
            R.ref_moe_step(L, O._p(hn), O._p(x), None, None, None, None, None)

    pre = {}
    for T in (128, 2048):
        xs = M.synth_hidden(SEED, 2 if T == 2048 else 4, T)
        pre[T] = ((xs / np.sqrt((xs.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6)).astype(np.float32), xs)

    def prefill(T):
        hnT, xT = pre[T]
        xw = xT.copy()
        R.ref_set_router(0, O._p(rp))                    # maple.c holds 24 layers: borrow layer 0's slot
        R.ref_set_bias(O._p(zb) if T == 2048 else None)
        R.ref_moe_batch(0, O._p(hnT), T, O._p(xw), *([None] * 14))
        R.ref_set_bias(None)
        R.ref_set_router(0, O._p(routers[0]))

    def rate(fn, units, secs, min_reps=1):
        fn()                                              # touch the pages once
        n, t0 = 0, time.perf_counter()
        while True:
            fn(); n += 1
            if n >= min_reps and time.perf_counter() - t0 >= secs:
                break
        return n, units * n / (time.perf_counter() - t0)

    res = {}
    model, phys, usable = cpu_topology()
    # every core this process may use (the affinity mask), at most the host's physical cores (maple.c runs one
    # thread per core) and at most the thread budget the environment sets (OMP_NUM_THREADS on the GPU boxes)
    budget = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    nt_all = min(x for x in (usable, phys, budget or None) if x)
    for nt in (1, nt_all):
        if nt > 1:
            nt = R.ref_set_threads(nt)
        d_n, d_v = rate(token, 1, seconds)
        p1_n, p1_v = rate(lambda: prefill(128), 128, seconds / 4)
        p2_n, p2_v = rate(lambda: prefill(2048), 2048, 0.0)
        res[nt] = dict(decode=(d_n, d_v), p128=(p1_n, p1_v), p2048=(p2_n, p2_v))
        log(f"cpu baseline, {nt} thread(s): decode {d_v:.1f} tok/s, prefill-128 {p1_v:.0f} tok/s, prefill-2048 {p2_v:.0f} tok/s")
    flags = "-O3 -ffast-math -mavx2 -mfma -mf16c"
    r1, ra = res[1], res[max(res)]
    return dict(value=round(ra["decode"][1], 2), unit="tokens/s", cores=max(res), kind="reference",
                cpu=model, host_physical_cores=phys, cores_usable=usable, thread_budget=budget or None,
                value_1_thread=round(r1["decode"][1], 2),
                sample=f"{ra['decode'][0]} decode tokens x 24 layers through maple.c's step() MoE block (int8, {flags}, "
                       f"{max(res)} threads of run()), same synthetic weights; {r1['decode'][0]} tokens on 1 thread",
                prefill=dict(workload="maple.c step_batch MoE block (maple.c:733-834), one layer, layer-0 experts",
                             config0_128_tokens=dict(tokens_per_s_1_thread=round(r1["p128"][1], 1),
                                                     tokens_per_s_all=round(ra["p128"][1], 1)),
                             config2_2048_tokens_zipf=dict(tokens_per_s_1_thread=round(r1["p2048"][1], 1),
                                                           tokens_per_s_all=round(ra["p2048"][1], 1))))


def valid_ternary_bytes():
    """the 81 byte values whose four 2-bit fields are all codes 0..2 (w = -1, 0, +1)"""
    v = np.arange(256)
    ok = ((v & 3) < 3) & (((v >> 2) & 3) < 3) & (((v >> 4) & 3) < 3) & ((v >> 6) < 3)
    return v[ok].astype(np.uint8)


def rope_table(npos):
    """maple.c:1151-1152: (cos, sin) of pos * 10000^(-2i/64), i < 32, computed in double, stored as fp32"""
    f = np.arange(npos, dtype=np.float64)[:, None] * (1.0 / np.power(10000.0, 2.0 * np.arange(32) / 64))[None, :]
    return np.ascontiguousarray(np.stack([np.cos(f), np.sin(f)], -1).astype(np.float32))


def full_prefill(lib, rids, args):
    T, CTX = 2048, 4096
    rng = np.random.default_rng(SEED + 4)
    vb = valid_ternary_bytes()
    keep = []
    M.check(lib.mmoe_dense_reset(), "dense reset")
    for L in range(NL):
        for g, rows_list in ((2 * L, (2048, 512, 512)), (2 * L + 1, (2048,))):
            for rows in rows_list:
                packed = rng.choice(vb, size=(rows, 512))
                sc = rng.uniform(0.01, 0.05, rows).astype(np.float32)
                lib.gpre_dense_add(g, M.ptr(packed), M.ptr(sc), rows, 2048); keep += [packed, sc]
    if lib.gpre_dense_done(T) != 0:
        log("gpre_dense_done:", lib.mmoe_last_error().decode()); return None, None
    del keep
    # dense q/k/v projections of layer 0 alone (gpre_dense, k_dense): kernel time only
    xq = rng.standard_normal((T, 2048)).astype(np.float32); yq = np.empty((T, 3072), np.float32)
    lib.gpre_dense(0, M.ptr(xq), T, M.ptr(yq))
    dk = prof_pass(lambda i: lib.gpre_dense(0, M.ptr(xq), T, M.ptr(yq)), 5)
    kt_ms = dk["dense"][0] / dk["dense"][1]
    dops = 2 * T * 3072 * 2048
    log(f"dense q/k/v 2048 tokens: k_dense {kt_ms * 1e3:.1f} us, {dops / kt_ms / 1e9:.0f} TOPS")
    dense = dict(workload="q/k/v projections (3072 x 2048 ternary) of a 2048-token chunk, gpre_dense",
                 kernel_us=round(kt_ms * 1e3, 2), tops=round(dops / kt_ms / 1e9, 1),
                 frac_int8_peak=round(dops / kt_ms / 1e9 / INT8_PEAK_TOPS, 4))
    bf = lambda a: (np.asarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)
    norms = np.empty((NL, 4352), np.float32)
    routers = np.empty((NL, 256, 2048), np.uint16)
    zb = M.zipf_bias(SEED, 1.1)
    for L in range(NL):
        w = bf(rng.uniform(0.5, 1.5, 4352))
        norms[L] = (w.astype(np.uint32) << 16).view(np.float32)
        routers[L] = M.synth_router(SEED, L, dist=0)
    M.check(lib.gfull_init(CTX, T, 512, M.ptr(norms), M.ptr(routers), M.ptr(rope_table(CTX))), "gfull_init")
    loc = M.block_loc()
    for L in range(NL):   # expert tables (the layer blocks of the decode run), router and post-norm as above
        regs = np.array([rids[L], -1, -1, -1], np.int32)
        M.check(lib.mmoe_set_layer(L, M.ptr(loc), M.ptr(regs), M.ptr(routers[L]), M.ptr(bf(norms[L, 2048:4096]))), "set_layer")
        M.check(lib.mmoe_set_bias(L, M.ptr(zb)), "bias")
    x = M.synth_hidden(SEED, 5, T)
    out = dict(workload="config 4: 2048-token chunk x 24 whole layers (attention 16q/4kv x 128, q/k norms, rope, "
                        "fp16 cache; MoE with Zipf(1.1) bias), mmoe_gfull_stack",
               unit="tokens/s")
    for pos0 in (0, 2048):
        lib.gfull_begin(M.ptr(x), T, pos0)   # the chunk's hidden state in HBM; each step runs it through 24 layers

        def fstep(i=0):
            M.check(lib.mmoe_gfull_stack(0, NL), "gfull_stack")
        fms, _ = timed(fstep, 3, 1)
        # per kernel, the pass (of 3, each 24 layers) with its lowest average: an occasional slow dispatch in one
        # pass does not set a kernel's figure; attention and MoE times are the sums of those per-pass figures
        passes = [prof_pass(fstep, 1) for _ in range(3)]
        fk = {k: min((p[k] for p in passes if k in p), key=lambda v: v[0] / v[1]) for k in passes[0]}
        att = sum(v[0] for k, v in fk.items() if k in ("dense", "qkn", "att_scores", "att_softmax", "att_pv"))
        tot = sum(v[0] for v in fk.values())
        log(f"full prefill 2048 at pos0 {pos0}: {fms:.2f} ms / 24 layers, {T / fms * 1e3:.0f} tok/s; "
            f"kernel time attention half {att:.2f} ms, MoE {tot - att:.2f} ms")
        for k, (tt, n) in sorted(fk.items(), key=lambda kv: -kv[1][0]):
            log(f"  {k:12s} {tt / n * 1e3:8.2f} us avg x {n}")
        # scores and weighted sum: 16 heads x 128 dims x (window length) fp32 FMAs per token each, in maple.c's
        # order (no MFMA); averaged over the 24 layers (every fourth global, the rest a 512-position window)
        pos = np.arange(pos0, pos0 + T)
        win_len = {0: np.minimum(pos, 512) + 1, 1: pos + 1}
        fma = sum(16 * 128 * int(win_len[int(L % 4 == 3)].sum()) for L in range(NL)) / NL
        fma_peak = 256 * 4 * 16 * 2.4e9   # fp32 FMA without packed operations
        frac = {k: round(fma / (fk[k][0] / fk[k][1] * 1e-3) / fma_peak, 4) for k in ("att_scores", "att_pv") if k in fk}
        key = "first_chunk" if pos0 == 0 else "second_chunk"
        out[key] = dict(pos0=pos0, value=round(T / fms * 1e3, 1), ms_per_chunk=round(fms, 3),
                        attention_ms=round(att, 3), moe_ms=round(tot - att, 3),
                        attention_fma_per_layer=int(fma), attention_frac_fp32_fma_peak=frac,
                        kernels_us={k: round(v[0] / v[1] * 1e3, 2) for k, v in fk.items()})
    lib.gfull_read(None, None)
    return out, dense

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-decode", action="store_true", help="skip the config-1 decode timing (development runs)")
    ap.add_argument("--no-full", action="store_true", help="skip config 4 (24 whole layers with attention)")
    ap.add_argument("--no-floor", action="store_true",
                    help="skip the decode-floor probe (libmaplefloor); profiled runs leave it out")
    ap.add_argument("--graph", type=int, default=1, help="replay the 24-layer decode as a HIP graph")
    ap.add_argument("--router", choices=["exact", "mfma"], default="mfma",
                    help="router of the 2048-token prefill: bf16 MFMA logits with each token's near-top-8 experts recomputed "
                         "exactly (default), or fp32 FMA chains for every logit")
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                    help="also run 3 plain device copies of MIB MiB (scale reference for rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures one GPU only: the MoE path of one MI355X; "
                                   "multi-GPU sharding is a design note only; run with --gpus 1"}))
        sys.exit(2)
    lib = M.lib()
    M.check(lib.mmoe_init(2048), "mmoe_init")
    if args.calib_copy:
        nbytes = args.calib_copy << 20
        a, b = lib.mmoe_dev_alloc(nbytes), lib.mmoe_dev_alloc(nbytes)
        for _ in range(3):
            M.check(lib.mmoe_d2d(b, a, nbytes), "calibration copy")
        lib.mmoe_sync(); lib.mmoe_dev_free(a); lib.mmoe_dev_free(b)
    name, cus, clk = M.device_info()
    log(f"device {name}, {cus} CUs, {clk / 1e3:.0f} MHz")

    # ---- 24 synthetic layers, codes resident in HBM (config 1: uniform router weights)
    t = time.perf_counter()
    blocks, routers = [], []
    ones = np.full(M.H, 0x3F80, np.uint16)
    rids = []
    for L in range(NL):
        blk = M.synth_layer_block(SEED, L, nthreads=min(os.cpu_count() or 1, 16))
        rw = M.synth_router(SEED, L, dist=1)
        rids.append(M.register_layer(L, blk, rw, ones))
        blocks.append(blk); routers.append(rw)
    log(f"24 layers generated and resident in HBM in {time.perf_counter() - t:.1f} s")

    # Each decode step takes the next of NX distinct tokens: different tokens route to different experts, so the
    # codes a step reads are not the ones the step before left in the caches (24 layers x 8 experts x 0.8 MB =
    # 153 MB per token; the whole model is 4.9 GB). The first pass repeats one token to show the warm case.
    NX = 64
    xs0 = M.synth_hidden(SEED, 1, NX)
    d_x = lib.mmoe_dev_alloc(M.H * 4)
    d_xs = lib.mmoe_dev_alloc(xs0.nbytes)
    lib.mmoe_h2d(d_xs, M.ptr(xs0), xs0.nbytes)
    import ctypes as C
    tok = lambda i: C.c_void_p(d_xs + (i % NX) * M.H * 4)

    def step_plain(i):
        lib.mmoe_d2d(d_x, tok(i), M.H * 4)
        M.check(lib.mmoe_stack_dev(0, NL, d_x, 1, M.ORDER_STEP), "stack")

    def step_graph(i):
        lib.mmoe_d2d(d_x, tok(i), M.H * 4)
        M.check(lib.mmoe_stack_graph(0, NL, d_x, 1, M.ORDER_STEP, 1), "graph")
    step = step_graph if args.graph else step_plain
    bytes_tok = NL * 8 * CODES_SCALES_PER_EXPERT
    gu_bytes = 8 * GU_BYTES_PER_EXPERT
    if args.no_decode:   # development runs: no decode timing, no headline figures
        ms = wall_ms = tok_s = None
        kt, roof = {}, None
    else:
        warm_ms, _ = timed(lambda i: step(0), max(5, args.steps // 2), args.warmup)
        ms, wall_ms = timed(step, args.steps, args.warmup)
        tok_s = 1e3 / ms
        log(f"decode: {ms * 1e3:.1f} us/token (wall {wall_ms * 1e3:.1f} us), {tok_s:.0f} tok/s, "
            f"{bytes_tok / ms / 1e6:.0f} GB/s on codes+scales over the whole step; one token repeated: {warm_ms * 1e3:.1f} us")
        kt = prof_pass(step_plain, 2 * NX)
        for k, (tot, n) in sorted(kt.items(), key=lambda kv: -kv[1][0]):
            log(f"  {k:10s} {tot / n * 1e3:8.2f} us avg x {n}")
        gu_us = kt["gateup"][0] / kt["gateup"][1] * 1e3
        roof = dict(bound="hbm", kernel="k_dec_gateup (decode, 8 experts x 1024 rows)", achieved=round(gu_bytes / gu_us / 1e3, 1),
                    peak=HBM_PEAK_GBS, unit="GB/s", frac=round(gu_bytes / gu_us / 1e3 / HBM_PEAK_GBS, 4),
                    traffic=pmc_traffic("k_dec_gateup"), algorithmic_bytes_per_launch=gu_bytes, avg_launch_us=round(gu_us, 2),
                    timing=f"device execution of each of its {kt['gateup'][1]} launches in 24-layer steps over {NX} distinct "
                           "tokens (events on the dispatch, as rocprofv3)",
                    step_gbs=round(bytes_tok / ms / 1e6, 1), step_frac=round(bytes_tok / ms / 1e6 / HBM_PEAK_GBS, 4))

    # ---- the floor under the decode layer: 3 x 24 dependent kernels at the decode grid shapes, one HIP graph
    floor = None
    fpath = os.path.join(ROOT, "maple-runtime_amd", "libmaplefloor.so")
    if not args.no_decode and not args.no_floor and os.path.exists(fpath):
        fl = C.CDLL(fpath)
        fl.floor_layer_us.restype, fl.floor_layer_us.argtypes = C.c_double, [C.c_int, C.c_int, C.c_int]
        fv = [fl.floor_layer_us(f, NL, 200) for f in (0, 1, 2)]
        floor = dict(unit="us per layer (3 dependent kernels)", empty_kernels=round(fv[0], 2),
                     one_dependent_load=round(fv[1], 2), dependent_load_then_cold_load=round(fv[2], 2),
                     measured_layer=round(ms * 1e3 / NL, 2))
        log(f"decode floor per layer (graph of 3 x 24 kernels at the decode grids): empty {fv[0]:.2f} us, "
            f"one dependent load {fv[1]:.2f} us, dependent + cold load {fv[2]:.2f} us; measured layer {ms * 1e3 / NL:.2f} us")

    # ---- config 2: 2048-token prefill, one layer, Zipf(1.1)-skewed routing. Steps rotate over 4 layers with
    # different experts (4 x 204 MB, more than the 256 MB last-level cache holds)
    prefill = None
    if not args.no_prefill:
        LPS = (40, 41, 42, 43)
        rw = M.synth_router(SEED, 0, dist=0)
        loc = M.block_loc()
        zb = M.zipf_bias(SEED, 1.1)
        for k, LP in enumerate(LPS):
            regs = np.array([rids[k], -1, -1, -1], np.int32)
            M.check(lib.mmoe_set_layer(LP, M.ptr(loc), M.ptr(regs), M.ptr(rw), None), "set_layer")
            M.check(lib.mmoe_set_bias(LP, M.ptr(zb)), "bias")
        T = 2048
        xs = M.synth_hidden(SEED, 2, T)
        hn = xs / np.sqrt((xs.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6).astype(np.float32)
        hn = hn.astype(np.float32)
        d_hn = lib.mmoe_dev_alloc(hn.nbytes); d_xp = lib.mmoe_dev_alloc(hn.nbytes)
        lib.mmoe_h2d(d_hn, M.ptr(hn), hn.nbytes); lib.mmoe_h2d(d_xp, M.ptr(xs), xs.nbytes)

        M.check(lib.mmoe_set_router_mode(1 if args.router == "exact" else 0), "router mode")

        def pstep(i):
            M.check(lib.mmoe_moe_dev(LPS[i % len(LPS)], d_hn, T, d_xp, M.ORDER_BATCH), "moe_dev")
        pms, pwall = timed(pstep, max(8, args.steps // 5), 4)
        plan = M.read_plan()
        cnt = np.diff(plan["ustart"])
        ops = T * 8 * (OPS_GU_PER_PAIR + OPS_DN_PER_PAIR)
        log(f"prefill 2048: {pms * 1e3:.1f} us/layer, {T / pms * 1e3:.0f} tok/s, {ops / pms / 1e9:.1f} TOPS "
            f"({ops / pms / 1e9 / INT8_PEAK_TOPS * 100:.1f}% of int8 MFMA peak); {plan['nu']} experts used, max load {cnt.max()}")
        pk = prof_pass(pstep, 8)
        for k, (tot, n) in sorted(pk.items(), key=lambda kv: -kv[1][0]):
            log(f"  {k:10s} {tot / n * 1e3:8.2f} us avg x {n}")
        g_us = pk["gateup"][0] / pk["gateup"][1] * 1e3
        g_ops = T * 8 * OPS_GU_PER_PAIR
        prefill = dict(workload="config 2: 2048-token prefill chunk, 1 MoE layer, Zipf(1.1) expert bias",
                       value=round(T / pms * 1e3, 1), unit="tokens/s", ms_per_layer=round(pms, 4),
                       layer_tops=round(ops / pms / 1e9, 1), layer_frac_int8_peak=round(ops / pms / 1e9 / INT8_PEAK_TOPS, 4),
                       experts_used=plan["nu"], max_expert_load=int(cnt.max()),
                       roofline=dict(bound="mfma", kernel="k_gateup_pk<true> (grouped int8 MFMA)", achieved=round(g_ops / g_us / 1e6, 1),
                                     peak=INT8_PEAK_TOPS, unit="TOPS", frac=round(g_ops / g_us / 1e6 / INT8_PEAK_TOPS, 4),
                                     traffic=pmc_traffic("k_gateup_pk<true>"), avg_launch_us=round(g_us, 2),
                                     counters=pmc_mfma("k_gateup_pk<true", "config 2")),
                       kernels_us={k: round(v[0] / v[1] * 1e3, 2) for k, v in pk.items()})

    # ---- config 3: batched decode, 64 sequences x 24 layers (batch order), and config 0: a 128-token chunk
    extra = {}
    if not args.no_prefill:
        xb0 = M.synth_hidden(SEED, 3, 64)
        d_xb = lib.mmoe_dev_alloc(xb0.nbytes); d_xb0 = lib.mmoe_dev_alloc(xb0.nbytes)
        lib.mmoe_h2d(d_xb0, M.ptr(xb0), xb0.nbytes)

        def bstep(i):
            lib.mmoe_d2d(d_xb, d_xb0, xb0.nbytes)
            M.check(lib.mmoe_stack_graph(0, NL, d_xb, 64, M.ORDER_BATCH, 1) if args.graph else
                    lib.mmoe_stack_dev(0, NL, d_xb, 64, M.ORDER_BATCH), "batched decode")
        lib.mmoe_graph_reset()
        bms, _ = timed(bstep, max(5, args.steps // 5), 2)
        lib.mmoe_graph_reset()
        # untimed: the experts each layer uses (for the step's algorithmic bytes) and per-kernel device times
        lib.mmoe_d2d(d_xb, d_xb0, xb0.nbytes)
        nus = []
        for L in range(NL):
            M.check(lib.mmoe_stack_dev(L, 1, d_xb, 64, M.ORDER_BATCH), "batched decode layer")
            nus.append(int(M.read_plan()["nu"]))
        bbytes = sum(nus) * CODES_SCALES_PER_EXPERT
        bk = prof_pass(lambda i: (lib.mmoe_d2d(d_xb, d_xb0, xb0.nbytes), M.check(lib.mmoe_stack_dev(0, NL, d_xb, 64, M.ORDER_BATCH), "stack")), 2)
        log(f"batched decode 64 x 24 layers: {bms * 1e3:.1f} us/step, {64 / bms * 1e3:.0f} tok/s, "
            f"{bbytes / bms / 1e6:.0f} GB/s on the used experts' codes+scales ({sum(nus) / NL:.1f} experts per layer)")
        extra["batched_decode"] = dict(workload="config 3: 64 sequences x 1 token x 24 MoE layers (batch order)",
                                       value=round(64 / bms * 1e3, 1), unit="tokens/s", ms_per_step=round(bms, 4),
                                       experts_per_layer=round(sum(nus) / NL, 1), step_gbs=round(bbytes / bms / 1e6, 1),
                                       step_frac_hbm=round(bbytes / bms / 1e6 / HBM_PEAK_GBS, 4),
                                       kernels_us_per_layer={k: round(v[0] / v[1] * 1e3, 2) for k, v in bk.items()})
        T0 = 128
        for LP in LPS:
            M.check(lib.mmoe_set_bias(LP, None), "bias off")
        x128 = M.synth_hidden(SEED, 4, T0)
        h128 = (x128 / np.sqrt((x128.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6)).astype(np.float32)
        d_h128 = lib.mmoe_dev_alloc(h128.nbytes); d_x128 = lib.mmoe_dev_alloc(h128.nbytes)
        lib.mmoe_h2d(d_h128, M.ptr(h128), h128.nbytes); lib.mmoe_h2d(d_x128, M.ptr(x128), x128.nbytes)

        def cstep(i):
            M.check(lib.mmoe_moe_dev(LPS[i % len(LPS)], d_h128, T0, d_x128, M.ORDER_BATCH), "moe_dev 128")
        cms, _ = timed(cstep, max(5, args.steps // 5), 2)
        ck = prof_pass(cstep, 8)
        log(f"prefill 128 (config 0): {cms * 1e3:.1f} us/layer, {T0 / cms * 1e3:.0f} tok/s")
        extra["prefill_128"] = dict(workload="config 0: 128-token chunk, 1 MoE layer, unbiased router",
                                    value=round(T0 / cms * 1e3, 1), unit="tokens/s", ms_per_layer=round(cms, 4),
                                    kernels_us={k: round(v[0] / v[1] * 1e3, 2) for k, v in ck.items()})

    # ---- config 4: a 2048-token chunk through 24 whole layers (attention + MoE) on the card, positions 0..2047
    # and 2048..4095 of a 4096-position key/value cache (mmoe_gfull_stack); the dense q/k/v/o projections of all
    # 24 layers (random ternary, per-row fp32 scales) sit in HBM beside the experts
    if not args.no_prefill and not args.no_full:
        full, dense = full_prefill(lib, rids, args)
        if full:
            extra["full_prefill_2048"] = full
        if dense:
            extra["dense_qkv_2048"] = dense

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baselines(blocks, routers, args.cpu_seconds)

    rnd = lambda v, k: None if v is None else round(v, k)
    out = {"metric": METRIC, "value": rnd(tok_s, 1),
           "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": rnd(ms, 5),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8xternary->int32, fp32",
           "data": "synthetic (seeded Maple-shaped ternary experts, uniform router, N(0,1) hidden)",
           "config": {"workload": "config 1: decode 1 token x 24 stacked MoE layers (d=2048, 256 experts, top-8, FF=512)",
                      "tokens_per_step": 1, "layers": NL, "hip_graph": bool(args.graph), "device": name},
           "roofline": roof, "cpu_baseline": cpu, "prefill": prefill,
           "decode_kernels_us": {k: round(v[0] / v[1] * 1e3, 2) for k, v in kt.items()}, "decode_floor": floor, **extra}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
