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
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "maple-runtime_amd"), os.path.join(ROOT, "oracle")]

import numpy as np  # noqa: E402

import maplemoe as M  # noqa: E402

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
        if len(cols) > 6 and cols[1] == kernel:
            return int(cols[6])
    return None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def prof_pass(fn, reps):
    lib = M.lib()
    lib.mmoe_prof_reset(); lib.mmoe_prof(1)
    for _ in range(reps):
        fn()
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
    lib = M.lib()
    for _ in range(warmup):
        fn()
    lib.mmoe_sync()
    lib.mmoe_event_record(0)
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    lib.mmoe_event_record(1)
    lib.mmoe_sync()
    t1 = time.perf_counter()
    ev_ms = lib.mmoe_event_elapsed_ms()
    return ev_ms / steps, (t1 - t0) * 1e3 / steps


def cpu_baseline_decode(blocks, routers, seconds):
    """maple.c's step() MoE block (oracle/_ref) for 24 layers per token, on the host cores."""
    import pyoracle as O
    if not O.ref_available():
        return None
    R = O.ref()
    nt = min(os.cpu_count() or 1, 16)
    nt = R.ref_set_threads(nt)
    for L in range(NL):
        R.ref_set_router(L, O._p(routers[L]))
        for e in range(M.NE):
            R.ref_set_expert(L, e, *[O._p(a) for a in M.expert_views(blocks[L], e)])
    ones = np.full(M.H, 0x3F80, np.uint16)
    x = M.synth_hidden(SEED, 77, 1)[0].copy()
    hn = np.empty_like(x)

    def token():
        for L in range(NL):
            R.ref_rmsnorm(O._p(x), O._p(ones), M.H, O._p(hn))
            R.ref_moe_step(L, O._p(hn), O._p(x), None, None, None, None, None)
    token()  # touch the pages once
    n, t0 = 0, time.perf_counter()
    while True:
        token(); n += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    return dict(value=n / dt, unit="tokens/s", cores=nt, kind="reference",
                sample=f"{n} decode tokens x 24 layers through maple.c's step() MoE block (int8 AVX2, "
                       f"-O3 -ffast-math -mavx2 -mfma -mf16c, {nt} threads of run()), same synthetic weights")



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
    dk = prof_pass(lambda: lib.gpre_dense(0, M.ptr(xq), T, M.ptr(yq)), 5)
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

        def fstep():
            M.check(lib.mmoe_gfull_stack(0, NL), "gfull_stack")
        fms, _ = timed(fstep, 3, 1)
        fk = prof_pass(fstep, 1)
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
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-full", action="store_true", help="skip config 4 (24 whole layers with attention)")
    ap.add_argument("--graph", type=int, default=1, help="replay the 24-layer decode as a HIP graph")
    ap.add_argument("--router", choices=["exact", "mfma"], default="exact",
                    help="router of the 2048-token prefill: fp32 FMA chains for every logit, or bf16 MFMA logits "
                         "with each token's near-top-8 experts recomputed exactly")
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

    x0 = M.synth_hidden(SEED, 1, 1)
    d_x = lib.mmoe_dev_alloc(x0.nbytes)
    d_x0 = lib.mmoe_dev_alloc(x0.nbytes)
    lib.mmoe_h2d(d_x0, M.ptr(x0), x0.nbytes)
    lib.mmoe_h2d(d_x, M.ptr(x0), x0.nbytes)

    def step_plain():
        lib.mmoe_d2d(d_x, d_x0, x0.nbytes)
        M.check(lib.mmoe_stack_dev(0, NL, d_x, 1, M.ORDER_STEP), "stack")

    if args.graph:
        def step():
            lib.mmoe_d2d(d_x, d_x0, x0.nbytes)
            M.check(lib.mmoe_stack_graph(0, NL, d_x, 1, M.ORDER_STEP, 1), "graph")
    else:
        step = step_plain
    ms, wall_ms = timed(step, args.steps, args.warmup)
    tok_s = 1e3 / ms
    bytes_tok = NL * 8 * CODES_SCALES_PER_EXPERT
    log(f"decode: {ms * 1e3:.1f} us/token (wall {wall_ms * 1e3:.1f} us), {tok_s:.0f} tok/s, "
        f"{bytes_tok / ms / 1e6:.0f} GB/s on codes+scales over the whole step")
    kt = prof_pass(step_plain, 5)
    for k, (tot, n) in sorted(kt.items(), key=lambda kv: -kv[1][0]):
        log(f"  {k:10s} {tot / n * 1e3:8.2f} us avg x {n}")
    step_plain(); lib.mmoe_sync()
    gu_ms = lib.mmoe_bench_stage(5, 200)  # k_gateup of the last layer, back to back
    dn_ms = lib.mmoe_bench_stage(7, 200)
    log(f"  back-to-back: gateup {gu_ms * 1e3:.2f} us, down {dn_ms * 1e3:.2f} us per launch")
    gu_bytes = 8 * GU_BYTES_PER_EXPERT
    roof = dict(bound="hbm", kernel="k_dec_gateup (decode, 8 experts x 1024 rows)", achieved=round(gu_bytes / gu_ms / 1e6, 1),
                peak=HBM_PEAK_GBS, unit="GB/s", frac=round(gu_bytes / gu_ms / 1e6 / HBM_PEAK_GBS, 4),
                traffic=pmc_traffic("k_dec_gateup"),
                algorithmic_bytes_per_launch=gu_bytes, avg_launch_us=round(gu_ms * 1e3, 2),
                step_gbs=round(bytes_tok / ms / 1e6, 1), step_frac=round(bytes_tok / ms / 1e6 / HBM_PEAK_GBS, 4))

    # ---- config 2: 2048-token prefill, one layer, Zipf(1.1)-skewed routing
    prefill = None
    if not args.no_prefill:
        LP = 40
        rw = M.synth_router(SEED, 0, dist=0)
        regs = np.array([rids[0], -1, -1, -1], np.int32)
        loc = M.block_loc()
        zb = M.zipf_bias(SEED, 1.1)
        M.check(lib.mmoe_set_layer(LP, M.ptr(loc), M.ptr(regs), M.ptr(rw), None), "set_layer")
        M.check(lib.mmoe_set_bias(LP, M.ptr(zb)), "bias")
        T = 2048
        xs = M.synth_hidden(SEED, 2, T)
        hn = xs / np.sqrt((xs.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6).astype(np.float32)
        hn = hn.astype(np.float32)
        d_hn = lib.mmoe_dev_alloc(hn.nbytes); d_xp = lib.mmoe_dev_alloc(hn.nbytes)
        lib.mmoe_h2d(d_hn, M.ptr(hn), hn.nbytes); lib.mmoe_h2d(d_xp, M.ptr(xs), xs.nbytes)

        M.check(lib.mmoe_set_router_mode(1 if args.router == "exact" else 0), "router mode")

        def pstep():
            M.check(lib.mmoe_moe_dev(LP, d_hn, T, d_xp, M.ORDER_BATCH), "moe_dev")
        pms, pwall = timed(pstep, max(5, args.steps // 5), 2)
        plan = M.read_plan()
        cnt = np.diff(plan["ustart"])
        ops = T * 8 * (OPS_GU_PER_PAIR + OPS_DN_PER_PAIR)
        log(f"prefill 2048: {pms * 1e3:.1f} us/layer, {T / pms * 1e3:.0f} tok/s, {ops / pms / 1e9:.1f} TOPS "
            f"({ops / pms / 1e9 / INT8_PEAK_TOPS * 100:.1f}% of int8 MFMA peak); {plan['nu']} experts used, max load {cnt.max()}")
        pk = prof_pass(pstep, 3)
        for k, (tot, n) in sorted(pk.items(), key=lambda kv: -kv[1][0]):
            log(f"  {k:10s} {tot / n * 1e3:8.2f} us avg x {n}")
        pstep(); lib.mmoe_sync()
        g_ms = lib.mmoe_bench_stage(5, 20)
        d_ms = lib.mmoe_bench_stage(7, 20)
        log(f"  back-to-back: gateup {g_ms * 1e3:.2f} us ({T * 8 * OPS_GU_PER_PAIR / g_ms / 1e9:.0f} TOPS), "
            f"down {d_ms * 1e3:.2f} us ({T * 8 * OPS_DN_PER_PAIR / d_ms / 1e9:.0f} TOPS)")
        g_ops = T * 8 * OPS_GU_PER_PAIR
        prefill = dict(workload="config 2: 2048-token prefill chunk, 1 MoE layer, Zipf(1.1) expert bias",
                       value=round(T / pms * 1e3, 1), unit="tokens/s", ms_per_layer=round(pms, 4),
                       layer_tops=round(ops / pms / 1e9, 1), layer_frac_int8_peak=round(ops / pms / 1e9 / INT8_PEAK_TOPS, 4),
                       experts_used=plan["nu"], max_expert_load=int(cnt.max()),
                       roofline=dict(bound="mfma", kernel="k_gateup_pk<true> (grouped int8 MFMA)", achieved=round(g_ops / g_ms / 1e9, 1),
                                     peak=INT8_PEAK_TOPS, unit="TOPS", frac=round(g_ops / g_ms / 1e9 / INT8_PEAK_TOPS, 4),
                                     traffic=pmc_traffic("k_gateup_pk<true>"), avg_launch_us=round(g_ms * 1e3, 2)),
                       kernels_us={k: round(v[0] / v[1] * 1e3, 2) for k, v in pk.items()})

    # ---- config 3: batched decode, 64 sequences x 24 layers (batch order), and config 0: a 128-token chunk
    extra = {}
    if not args.no_prefill:
        xb0 = M.synth_hidden(SEED, 3, 64)
        d_xb = lib.mmoe_dev_alloc(xb0.nbytes); d_xb0 = lib.mmoe_dev_alloc(xb0.nbytes)
        lib.mmoe_h2d(d_xb0, M.ptr(xb0), xb0.nbytes)

        def bstep():
            lib.mmoe_d2d(d_xb, d_xb0, xb0.nbytes)
            M.check(lib.mmoe_stack_graph(0, NL, d_xb, 64, M.ORDER_BATCH, 1) if args.graph else
                    lib.mmoe_stack_dev(0, NL, d_xb, 64, M.ORDER_BATCH), "batched decode")
        lib.mmoe_graph_reset()
        bms, _ = timed(bstep, max(5, args.steps // 5), 2)
        lib.mmoe_graph_reset()
        log(f"batched decode 64 x 24 layers: {bms * 1e3:.1f} us/step, {64 / bms * 1e3:.0f} tok/s")
        extra["batched_decode"] = dict(workload="config 3: 64 sequences x 1 token x 24 MoE layers (batch order)",
                                       value=round(64 / bms * 1e3, 1), unit="tokens/s", ms_per_step=round(bms, 4))
        T0 = 128
        M.check(lib.mmoe_set_bias(LP, None), "bias off")
        x128 = M.synth_hidden(SEED, 4, T0)
        h128 = (x128 / np.sqrt((x128.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6)).astype(np.float32)
        d_h128 = lib.mmoe_dev_alloc(h128.nbytes); d_x128 = lib.mmoe_dev_alloc(h128.nbytes)
        lib.mmoe_h2d(d_h128, M.ptr(h128), h128.nbytes); lib.mmoe_h2d(d_x128, M.ptr(x128), x128.nbytes)

        def cstep():
            M.check(lib.mmoe_moe_dev(LP, d_h128, T0, d_x128, M.ORDER_BATCH), "moe_dev 128")
        cms, _ = timed(cstep, max(5, args.steps // 5), 2)
        log(f"prefill 128 (config 0): {cms * 1e3:.1f} us/layer, {T0 / cms * 1e3:.0f} tok/s")
        extra["prefill_128"] = dict(workload="config 0: 128-token chunk, 1 MoE layer, unbiased router",
                                    value=round(T0 / cms * 1e3, 1), unit="tokens/s", ms_per_layer=round(cms, 4))

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
        cpu = cpu_baseline_decode(blocks, routers, args.cpu_seconds)
        if cpu:
            log(f"cpu baseline: {cpu['value']:.2f} tok/s on {cpu['cores']} threads")

    out = {"metric": "MoE decode tokens/s (1 token x 24 MoE layers); % HBM peak", "value": round(tok_s, 1),
           "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8xternary->int32, fp32",
           "data": "synthetic (seeded Maple-shaped ternary experts, uniform router, N(0,1) hidden)",
           "config": {"workload": "config 1: decode 1 token x 24 stacked MoE layers (d=2048, 256 experts, top-8, FF=512)",
                      "tokens_per_step": 1, "layers": NL, "hip_graph": bool(args.graph), "device": name},
           "roofline": roof, "cpu_baseline": cpu, "prefill": prefill,
           "decode_kernels_us": {k: round(v[0] / v[1] * 1e3, 2) for k, v in kt.items()}, **extra}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
