// mmoe.hip -- libmaplemoe: the MI355X (gfx950) MoE hot path behind maple.c's GPU entry points.
//
// Exports, with maple.c's own C signatures (maple.c:247-272), the entry points maple.c links against when
// built with -DGPU_HEAD: gpre_* (experts of a prompt chunk and the dense q/k/v/o projections), gfull_*
// (device-resident hidden state and the attention half of a layer), gpux_* (decode experts) and gpu_head_*.
// The output head is outside the built scope: gpu_head_init returns the failure value maple.c handles by
// keeping the head on its CPU. New mmoe_* entry points run the whole MoE layer on the device: router logits,
// softmax/top-8, grouping, int8 quantisation, gate/up + SiLU, re-quantisation, down and the combine
// (declared in include/maplemoe.h).
//
// One global context, like the reference (gpu_pre.m keeps file-scope state); not thread-safe; all work is
// queued on one default-priority HIP stream owned by the library.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>
#include <tuple>
#include <vector>
#include "kernels.h"
#include "decode.h"
#include "attn.h"
#ifndef GU16_W
#define GU16_W 4    // small-tile gate/up: waves per workgroup, 16-row fragments per wave
#define GU16_RF 1
#endif
#ifndef DN16_W
#define DN16_W 4    // small-tile down: waves per workgroup, 16-row fragments per wave
#define DN16_RF 2
#endif
#ifndef E16_W
#define E16_W 16   // fused small-tile expert kernel: waves per workgroup, code groups in the register ring
#define E16_RING 3
#define E16_GL 4     // 16-byte code loads per lane in one ring group
#endif
#ifndef DN_RPB
#define DN_RPB 2   // down row blocks of 256 per workgroup
#endif

extern "C" {
#include "../../include/maplemoe.h"
}

#define NLMAX 64
#define EXPERT_BYTES 798720u

static char g_err[512];
static void seterr(const char *fmt, ...) {
    va_list ap; va_start(ap, fmt); vsnprintf(g_err, sizeof g_err, fmt, ap); va_end(ap);
    fprintf(stderr, "maplemoe: %s\n", g_err);
}
#define HC(call) do { hipError_t e_ = (call); if (e_ != hipSuccess) { seterr("%s failed: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__, __LINE__); return -1; } } while (0)
#define HCV(call) do { hipError_t e_ = (call); if (e_ != hipSuccess) { seterr("%s failed: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__, __LINE__); return; } } while (0)
#define HCN(call) do { hipError_t e_ = (call); if (e_ != hipSuccess) { seterr("%s failed: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__, __LINE__); return NULL; } } while (0)

// ------------------------------------------------------------------------------------------------------
// Device work buffers for up to maxtok tokens (maxp = maxtok * 8 pairs)
// ------------------------------------------------------------------------------------------------------
struct Work {
    int maxtok = 0, maxp = 0;
    float *hn = nullptr, *x = nullptr, *rl = nullptr, *tw = nullptr, *uw = nullptr;
    int *top = nullptr, *hist = nullptr, *utok = nullptr, *tp = nullptr, *sp = nullptr, *ustart = nullptr;
    Plan *plan = nullptr;
    Tile *tiles = nullptr;
    ExpPtr *eptr = nullptr;
    int8_t *qx = nullptr, *qa = nullptr;
    float *qsx = nullptr, *qsa = nullptr, *act = nullptr, *down = nullptr;
    int *qsumx = nullptr, *qsuma = nullptr;
    int *dbg_gu = nullptr, *dbg_dn = nullptr;
    int *dov = nullptr;             // the same for the int16 down results
    int *eu = nullptr, *pu = nullptr;   // expert -> used-expert index [256], pair -> used-expert index [P]
    bool compact = false;           // the last expert stage left down as int16 (k_combine16)
    int hist_used = 0;              // entries of hist the device grouping filled; the combine clears them
    const float *norm_x = nullptr;  // set by mmoe_stack_dev: the router normalises this x into hn (post_ln norm_w)
    const uint16_t *norm_w = nullptr;
    float *rpart = nullptr;         // partial router logits [4][T][256] (approximate router)
    bool grp16 = false;             // the last device routing left the grouping to k_expert16 (no k_group launch)
    bool routed = false;            // the last chain-router launch also ran the top-8 and the quantisation
    int *rcnt = nullptr;            // per token: router blocks done (that launch's arrival counts, back to 0 after)
    int grp_nb = 0;
    const ExpPtr *grp_tab = nullptr;
    bool refine = false;            // the last router call left approximate logits for k_refine_topk
    int rl_nb = 0;                  // rl holds exact logits of this many tokens (last router call), else 0
};

// Where a Work set's buffers come from: hipMalloc (c == nullptr) or a fixed device span carved in order
// (the no-alloc entry point's static scratch).
struct Carve { uint8_t *base = nullptr; size_t used = 0, cap = 0; };
template <typename T> static int wbuf(T *&p, size_t bytes, Carve *c) {
    if (!c) { HC(hipMalloc(&p, bytes)); return 0; }
    size_t o = (c->used + 255) / 256 * 256;
    if (o + bytes > c->cap) { seterr("scratch of %zu bytes too small (%zu needed)", c->cap, o + bytes); return -1; }
    p = (T *)(c->base + o);
    c->used = o + bytes;
    return 0;
}
__global__ void k_fill_zero(int *p, int n) { int i = blockIdx.x * 256 + threadIdx.x; if (i < n) p[i] = 0; }

// ------------------------------------------------------------------------------------------------------
// Global state
// ------------------------------------------------------------------------------------------------------
struct Region { const void *host; size_t len; uint8_t *dev; };
struct LayerW { ExpPtr *tab = nullptr; uint16_t *router = nullptr; uint16_t *rc16 = nullptr, *rc8 = nullptr; float *rf8 = nullptr, *w1max = nullptr; uint16_t *post_ln = nullptr; float *bias = nullptr; };

static struct {
    bool ready = false;
    ExpPtr *zero_tab = nullptr;     // mmoe_route: the expert table k_group reads when no layer is involved
    hipStream_t st = nullptr;
    Work main;                 // gpre / gfull / mmoe
    Work dec;                  // gpux
    Work na;                   // mmoe_moe_dev_noalloc: carved from `scratch` (its device address in na_ptr)
    uint8_t *na_ptr = nullptr;
    bool debug = false;
    std::vector<Region> regions;
    LayerW layers[NLMAX];
    double t_region = 0.0;     // seconds spent copying regions into HBM
    // gpux
    int gx_layers = 0, gx_slots = 0; uint8_t *gx_mem = nullptr;
    hipEvent_t gx_ev = nullptr; int gx_np = 0;
    // gfull
    bool gfull = false; int gfull_nb = 0;
    double t_moe = 0.0;
    // profiling
    bool prof = false;
    hipEvent_t pe[2];
    double prof_ms[MMOE_PROF_NKERNELS]; long prof_n[MMOE_PROF_NKERNELS];
    hipGraphExec_t graph = nullptr;
    struct { int L0, nl, nb, order; float *x; } gkey = {};   // the arguments the graph was captured with
    int ncu = 256;             // compute units of the device (persistent grids)
} S;

// Kernel launch on the library stream. The arguments are converted to the kernel's parameter types and passed
// by address (hipLaunchKernel). While a launch() profiles, the dispatch itself carries start/stop events
// (hipExtLaunchKernel): their interval is the kernel's execution on the device, the duration rocprofv3 reports,
// without the extra barrier packets that events recorded around the launch would add.
static hipEvent_t g_ke[2];          // set by launch() while profiling, else null
static hipError_t g_klerr = hipSuccess;
template <typename... P, typename... A>
static void kl(void (*f)(P...), dim3 g, dim3 b, size_t shm, A &&...a) {
    static_assert(sizeof...(P) == sizeof...(A), "kernel argument count");
    std::tuple<P...> v(static_cast<P>(a)...);
    void *ptr[sizeof...(P)];
    std::apply([&](auto &...x) { int i = 0; ((ptr[i++] = (void *)&x), ...); }, v);
    hipError_t e = g_ke[0] ? hipExtLaunchKernel((const void *)f, g, b, ptr, shm, S.st, g_ke[0], g_ke[1], 0)
                           : hipLaunchKernel((const void *)f, g, b, ptr, shm, S.st);
    if (e != hipSuccess) g_klerr = e;
}

// small (carved sets): at most 64 tokens, so only the decode and 16-token-tile paths run: no int16 down side
// buffer (2048+ pairs only), no approximate-router buffers (512+ tokens), no host-side hidden state copy.
static int work_alloc(Work &w, int maxtok, Carve *c = nullptr) {
    if (maxtok < 1 || maxtok > MMOE_MAXTOK || (c && maxtok > 64)) { seterr("maxtok %d outside 1..%d", maxtok, c ? 64 : MMOE_MAXTOK); return -1; }
    w.maxtok = maxtok; w.maxp = maxtok * MTOPK;
    int nch = (maxtok + 63) / 64;
    size_t T = maxtok, P = w.maxp;
    if (wbuf(w.hn, T * MH * 4, c) || wbuf(w.rl, T * MNE * 4, c) || wbuf(w.top, T * MTOPK * 4, c) ||
        wbuf(w.tw, T * MTOPK * 4, c) || wbuf(w.hist, (size_t)nch * MNE * 4, c) || wbuf(w.plan, sizeof(Plan), c) ||
        wbuf(w.tiles, sizeof(Tile) * ((size_t)w.maxp / 16 + MNE + 8), c) || wbuf(w.eptr, MNE * sizeof(ExpPtr), c) ||
        wbuf(w.utok, P * 4, c) || wbuf(w.uw, P * 4, c) || wbuf(w.tp, P * 4, c) || wbuf(w.sp, P * 4, c) ||
        wbuf(w.ustart, (MNE + 1) * 4, c) || wbuf(w.qx, T * MH, c) || wbuf(w.qsx, T * 4, c) || wbuf(w.qsumx, T * 4, c) ||
        wbuf(w.act, P * MFF * 4, c) || wbuf(w.qa, P * MFF, c) || wbuf(w.qsa, P * 4, c) || wbuf(w.qsuma, P * 4, c) ||
        wbuf(w.down, P * MH * 4, c) || wbuf(w.eu, MNE * 4, c) || wbuf(w.pu, P * 4, c) || wbuf(w.rcnt, T * 4, c))
        return -1;
    // the per-chunk expert counts start at zero; the combine after k_group clears what it used
    kl(k_fill_zero, (nch * MNE + 255) / 256, 256, 0, w.hist, nch * MNE);
    kl(k_fill_zero, (maxtok + 255) / 256, 256, 0, w.rcnt, maxtok);
    HC(hipGetLastError());
    if (c) return 0;
    HC(hipMalloc(&w.x, T * MH * 4));
    HC(hipMalloc(&w.dov, P * MH * 4));
    HC(hipMalloc(&w.rpart, 4 * T * MNE * 4));
    HC(hipStreamSynchronize(S.st));
    return 0;
}

static int work_debug(Work &w, int on) {
    if (on && !w.dbg_gu) {
        HC(hipMalloc(&w.dbg_gu, (size_t)w.maxp * 2 * MFF * 4));
        HC(hipMalloc(&w.dbg_dn, (size_t)w.maxp * MH * 4));
    }
    if (!on && w.dbg_gu) { HC(hipFree(w.dbg_gu)); HC(hipFree(w.dbg_dn)); w.dbg_gu = w.dbg_dn = nullptr; }
    return 0;
}

// Work buffers of mmoe_moe_dev_noalloc, for callers that cannot allocate (see that entry point): a fixed device
// array, held by the device the library runs on until the process ends. Host code never passes the array's
// name to a kernel or a copy: it stands for a host-side shadow there. The device address comes from
// hipGetSymbolAddress once, in ctx_ready, and every use goes through S.na_ptr.
#define NOALLOC_SCRATCH_BYTES (7u << 20)
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

static int ctx_ready() {
    if (S.ready) return 0;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n < 1) { seterr("no HIP device"); return -1; }
    HC(hipStreamCreateWithFlags(&S.st, hipStreamNonBlocking));
    HC(hipEventCreate(&S.pe[0])); HC(hipEventCreate(&S.pe[1]));
    HC(hipEventCreate(&S.gx_ev));
    int dev = 0; HC(hipGetDevice(&dev));
    HC(hipDeviceGetAttribute(&S.ncu, hipDeviceAttributeMultiprocessorCount, dev));
    // the no-alloc work set: carved from the static scratch of this device (one device per process here)
    void *sp = nullptr;
    HC(hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)));
    S.na_ptr = (uint8_t *)sp;
    Carve c{S.na_ptr, 0, NOALLOC_SCRATCH_BYTES};
    if (work_alloc(S.na, MMOE_NOALLOC_MAXTOK, &c)) return -1;
    HC(hipStreamSynchronize(S.st));
    S.ready = true;
    return 0;
}

// Launch helper: one kernel (f calls kl once); while profiling, its device execution time is added to kid's.
template <typename F>
static int launch(int kid, F &&f) {
    g_klerr = hipSuccess;
    if (S.prof) { g_ke[0] = S.pe[0]; g_ke[1] = S.pe[1]; }
    f();
    g_ke[0] = g_ke[1] = nullptr;
    if (g_klerr != hipSuccess) { seterr("kernel launch failed: %s", hipGetErrorString(g_klerr)); (void)hipGetLastError(); return -1; }
    HC(hipGetLastError());
    if (S.prof) {
        HC(hipEventSynchronize(S.pe[1]));
        float ms = 0; HC(hipEventElapsedTime(&ms, S.pe[0], S.pe[1]));
        S.prof_ms[kid] += ms; S.prof_n[kid]++;
    }
    return 0;
}

// ------------------------------------------------------------------------------------------------------
// Pipeline stages
// ------------------------------------------------------------------------------------------------------
static int tile_tn(int np) { return np >= 2048 ? 64 : 16; }
static bool S_expert16 = true;   // tiles of 16: the fused whole-expert kernel (else three kernels)

// Router logits of nb tokens (d_hn) with layer L's router; order 0 = batch (maple.c:853-889), 1 = step (bf_row)
static bool S_router_exact = false;
#ifndef ROUTER_TK
#define ROUTER_TK 1
#endif
#ifndef ROUTER_TPB
#define ROUTER_TPB 2   // tokens per block of the chain router with the top-8 tail (below 512 tokens)
#endif
static bool S_router_tk = ROUTER_TK;   // batches below 512: top-8 and quantisation in the router launch   // batches of 512+: MFMA logits + exact refinement (else the exact chain GEMM)
// exact_only: never the approximate large-batch router (callers that hand the logits themselves to the host)
// tk (batches below 512 tokens): the router launch also runs each token's softmax/top-8 (per-chunk counts into
// hist unless hist is null) and its int8 quantisation, in the last of the token's router blocks
static int stage_router_launch(Work &w, int L, const float *d_hn, int nb, int order, bool exact_only, bool tk, int *hist) {
    LayerW &lw = S.layers[L];
    w.refine = false;
    w.routed = false;
    if (!lw.router) { seterr("layer %d has no router (mmoe_set_layer)", L); return -1; }
    // w.norm_x set (stacked path): the chain routers form hn = rmsnorm(x, post_ln) into d_hn themselves
    float *hn_w = const_cast<float *>(d_hn);
    if (tk && nb < 512) {
        RouteTail rt{w.top, w.tw, w.qx, w.qsx, w.qsumx, hist, w.rcnt};
        w.routed = true;
        unsigned g8 = (unsigned)((nb + 7) / 8 * 8);
        if (ROUTER_TPB == 2) {   // two tokens per block
            unsigned p8 = (unsigned)(((nb + 1) / 2 + 7) / 8 * 8);
            if (order == MMOE_ORDER_STEP) {
                if (w.norm_x) return launch(MMOE_K_ROUTER, [&] { kl(k_router_chains2<16, true>, p8 * 16, 256, 0, w.norm_x, nb, lw.rc16, lw.bias, w.rl, w.norm_w, hn_w, rt); });
                return launch(MMOE_K_ROUTER, [&] { kl(k_router_chains2<16, false>, p8 * 16, 256, 0, d_hn, nb, lw.rc16, lw.bias, w.rl, (const uint16_t *)nullptr, (float *)nullptr, rt); });
            }
            if (w.norm_x) return launch(MMOE_K_ROUTER, [&] { kl(k_router_chains2<8, true>, p8 * 8, 256, 0, w.norm_x, nb, lw.rc8, lw.bias, w.rl, w.norm_w, hn_w, rt); });
            return launch(MMOE_K_ROUTER, [&] { kl(k_router_chains2<8, false>, p8 * 8, 256, 0, d_hn, nb, lw.rc8, lw.bias, w.rl, (const uint16_t *)nullptr, (float *)nullptr, rt); });
        }
        if (order == MMOE_ORDER_STEP) {
            if (w.norm_x) return launch(MMOE_K_ROUTER, [&] { kl(k_router_chains<16, true, true>, g8 * 16, 256, 0, w.norm_x, nb, lw.rc16, lw.bias, w.rl, w.norm_w, hn_w, rt); });
            return launch(MMOE_K_ROUTER, [&] { kl(k_router_chains<16, false, true>, g8 * 16, 256, 0, d_hn, nb, lw.rc16, lw.bias, w.rl, nullptr, nullptr, rt); });
        }
        if (w.norm_x) return launch(MMOE_K_ROUTER, [&] { kl(k_router_chains<8, true, true>, g8 * 8, 256, 0, w.norm_x, nb, lw.rc8, lw.bias, w.rl, w.norm_w, hn_w, rt); });
        return launch(MMOE_K_ROUTER, [&] { kl(k_router_chains<8, false, true>, g8 * 8, 256, 0, d_hn, nb, lw.rc8, lw.bias, w.rl, nullptr, nullptr, rt); });
    }
    if (order == MMOE_ORDER_STEP) {
        if (w.norm_x) return launch(MMOE_K_ROUTER, [&] { kl(k_router_chains<16, true>, dim3(MNE * 16 / 256, nb), 256, 0, w.norm_x, nb, lw.rc16, lw.bias, w.rl, w.norm_w, hn_w, RouteTail{}); });
        return launch(MMOE_K_ROUTER, [&] { kl(k_router_chains<16>, dim3(MNE * 16 / 256, nb), 256, 0, d_hn, nb, lw.rc16, lw.bias, w.rl, nullptr, nullptr, RouteTail{}); });
    }
    if (nb < 512) {   // one block per (token, 32 experts): 8 nb blocks, router reread from L2 per token
        if (w.norm_x) return launch(MMOE_K_ROUTER, [&] { kl(k_router_chains<8, true>, dim3(MNE * 8 / 256, nb), 256, 0, w.norm_x, nb, lw.rc8, lw.bias, w.rl, w.norm_w, hn_w, RouteTail{}); });
        return launch(MMOE_K_ROUTER, [&] { kl(k_router_chains<8>, dim3(MNE * 8 / 256, nb), 256, 0, d_hn, nb, lw.rc8, lw.bias, w.rl, nullptr, nullptr, RouteTail{}); });
    }
    if (S_router_exact || exact_only)
        return launch(MMOE_K_ROUTER, [&] { kl(k_router_gemm<4>, dim3((nb + 15) / 16, MNE / RG_BE), 256, 0, d_hn, nb, lw.rf8, lw.bias, w.rl); });
    // approximate logits on the bf16 MFMA; k_refine_topk makes the top-8 exact
    w.refine = true;
    if (nb >= 1024) return launch(MMOE_K_ROUTER, [&] { kl(k_router_mfma<8, 1>, dim3((nb + 31) / 32, MNE / 256, 4), 512, 0, lw.router, d_hn, nb, w.rpart); });
    return launch(MMOE_K_ROUTER, [&] { kl(k_router_mfma<4, 1>, dim3((nb + 31) / 32, MNE / 128, 4), 256, 0, lw.router, d_hn, nb, w.rpart); });
}

// the router launch, recording whether rl now holds every logit exactly (mmoe_route may then take them as they are)
static int stage_router(Work &w, int L, const float *d_hn, int nb, int order, bool exact_only = false, bool tk = false,
                        int *hist = nullptr) {
    w.rl_nb = 0;
    int rc = stage_router_launch(w, L, d_hn, nb, order, exact_only, tk, hist);
    if (!rc && !w.refine) w.rl_nb = nb;
    return rc;
}

// softmax/top-8, the int8 quantisation of hn and the grouping of nb tokens; eptr filled from layer L's table
static int stage_route_group(Work &w, int L, int nb, int tn, const float *d_hn) {
    int nch = (nb + 63) / 64;
    w.grp16 = false;
    if (!w.refine && tn == 16 && S_expert16 && nb <= E16_GRP_MAXTOK) {   // top-8 only: k_expert16 forms the grouping
        w.grp16 = true; w.grp_nb = nb; w.grp_tab = S.layers[L].tab;
        if (w.routed) return 0;   // the router launch ran the top-8 and the quantisation
        return launch(MMOE_K_TOPK, [&] { kl(k_topk_quant, dim3((nb + 3) / 4, 2), 256, 0, w.rl, d_hn, nb, w.top, w.tw, w.qx, w.qsx, w.qsumx, (int *)nullptr); });
    }
    if (w.refine) {   // exact logits of each token's candidates, then its softmax/top-8 (and the quantisation)
        const LayerW &lw = S.layers[L];
        if (launch(MMOE_K_TOPK, [&] { kl(k_refine_topk, dim3((nb + 3) / 4, 2), 256, 0, w.rpart, d_hn, nb, lw.rc8, lw.bias, lw.w1max, w.rl, w.top, w.tw,
                                          w.hist, w.qx, w.qsx, w.qsumx); }))
            return -1;
    } else if (!w.routed && launch(MMOE_K_TOPK, [&] { kl(k_topk_quant, dim3((nb + 3) / 4, 2), 256, 0, w.rl, d_hn, nb, w.top, w.tw, w.qx, w.qsx, w.qsumx, w.hist); })) return -1;
    w.hist_used = nch * MNE;   // cleared by this call's combine
    return launch(MMOE_K_GROUP, [&] {
        kl(k_group, nch, 512, 0, w.hist, nb, w.plan, S.layers[L].tab, w.eptr, tn, w.tiles, w.eu, w.top, w.tw, w.utok, w.uw,
                                       w.tp, w.sp, w.pu);
    });
}

static int stage_quant_x(Work &w, const float *d_hn, int nb) {
    return launch(MMOE_K_QUANT, [&] { kl(k_quant<MH>, (nb + 3) / 4, 256, 0, d_hn, nb, w.qx, w.qsx, w.qsumx); });
}

// gate/up (+SiLU), act quantisation, down for np pairs under w.plan / w.eptr / w.utok

static inline unsigned grid8(int items) { return (unsigned)((items + 7) / 8 * 8); }  // xcd_item needs a multiple of 8
#ifndef GU_OCC
#define GU_OCC 3   // k_gateup_pk: persistent workgroups per CU, code / activation prefetch distances in chunks
#define GU_PD 1     // (3 / 2 / 2, the deeper prefetch at two workgroups per CU, measured 64.5 against 60 us at config 2)
#define GU_PA 1
#endif
static int launch_gateup(Work &w, int maxtiles, int tn, int *dg) {
    if (tn == 64) {   // checks on: int32 sums into the debug buffer; else the fp32 activation into w.act
        int nblk = (int)grid8(S.ncu * GU_OCC < maxtiles * (MFF / 128) ? S.ncu * GU_OCC : maxtiles * (MFF / 128));   // persistent blocks, GU_OCC per CU
        if (dg) return launch(MMOE_K_GATEUP, [&] { kl(k_gateup_pk<false, GU_PD, GU_PA, GU_OCC>, nblk, 256, 0, w.plan, w.tiles, w.eptr, w.utok, w.qx, w.qsx, w.qsumx, dg); });
        return launch(MMOE_K_GATEUP, [&] { kl(k_gateup_pk<true, GU_PD, GU_PA, GU_OCC>, nblk, 256, 0, w.plan, w.tiles, w.eptr, w.utok, w.qx, w.qsx, w.qsumx, w.act); });
    }
    return launch(MMOE_K_GATEUP, [&] { kl(k_gateup<16, GU16_W, GU16_RF>, grid8(maxtiles * (MFF / (16 * GU16_W * GU16_RF))), 64 * GU16_W, 0, w.plan, w.tiles, w.eptr, w.utok, w.qx, w.qsx, w.qsumx, w.act, dg); });
}
static int launch_down(Work &w, int maxtiles, int tn, int *dd, bool compact) {
    // large batches: 4 row blocks per workgroup (half the activation staging per row); else 2 (more workgroups)
    // compact: act arrives in fp32 and each tile is quantised inside the down kernel (no k_quant_act launch)
    if (tn == 64 && compact && maxtiles >= S.ncu)
        return launch(MMOE_K_DOWN, [&] { kl(k_down_tile<4, true, true>, grid8(maxtiles * (MH / 256 / 4)), 256, 0, w.plan, w.tiles, w.eptr, w.qa, w.qsa, w.qsuma, w.down, w.dov, dd,
                                            (const float *)w.act, w.qa, w.qsa, w.qsuma); });
    if (tn == 64 && compact) return launch(MMOE_K_DOWN, [&] { kl(k_down_tile<DN_RPB, true, true>, grid8(maxtiles * (MH / 256 / DN_RPB)), 256, 0, w.plan, w.tiles, w.eptr, w.qa, w.qsa, w.qsuma, w.down, w.dov, dd,
                                                                 (const float *)w.act, w.qa, w.qsa, w.qsuma); });
    if (tn == 64) return launch(MMOE_K_DOWN, [&] { kl(k_down_tile<DN_RPB, false>, grid8(maxtiles * (MH / 256 / DN_RPB)), 256, 0, w.plan, w.tiles, w.eptr, w.qa, w.qsa, w.qsuma, w.down, nullptr, dd,
                                                       nullptr, nullptr, nullptr, nullptr); });
    return launch(MMOE_K_DOWN, [&] { kl(k_down<16, DN16_W, DN16_RF>, grid8(maxtiles * (MH / (16 * DN16_W * DN16_RF))), 64 * DN16_W, 0, w.plan, w.tiles, w.eptr, w.qa, w.qsa, w.qsuma, w.down, dd); });
}

// tiles of 16 with the fused path: one workgroup per tile does gate/up, the act quantisation and down
// grp: the grouping is formed in the kernel from w.top / w.tw (device routing), else read from the plan
static int launch_expert16(Work &w, int maxtiles, int *dg, int *dd, bool grp) {
    if (grp) {   // workgroup e < 256: expert e's first tile; then one per further tile (at most np / 16 of them)
        GroupIn gi{w.top, w.tw, w.grp_nb, w.grp_tab, w.plan, w.tiles, w.eptr, w.eu, w.utok, w.uw, w.tp, w.sp, w.pu};
        return launch(MMOE_K_GATEUP, [&] { kl(k_expert16<E16_W, E16_RING, 2, E16_GL>, MNE + w.grp_nb * MTOPK / 16, 64 * E16_W, 0, w.plan, w.tiles, w.eptr, w.utok, w.qx, w.qsx,
                                              w.qsumx, w.down, dg ? w.act : nullptr, w.qa, w.qsa, w.qsuma, dg, dd, gi); });
    }
    return launch(MMOE_K_GATEUP, [&] { kl(k_expert16<E16_W, E16_RING, 0, E16_GL>, grid8(maxtiles), 64 * E16_W, 0, w.plan, w.tiles, w.eptr, w.utok, w.qx, w.qsx, w.qsumx,
                                          w.down, dg ? w.act : nullptr, w.qa, w.qsa, w.qsuma, dg, dd, GroupIn{}); });
}
static int launch_quant_act(Work &w, int maxtiles, int tn, int np, int *dg) {
    if (tn == 64) {
        // checks on: activation from the int32 sums in the debug buffer; else gate/up wrote it already
        if (dg) return launch(MMOE_K_QUANT_ACT, [&] { kl(k_act_quant, maxtiles * 8, 256, 0, w.plan, w.tiles, w.eptr, w.utok, w.qsx, w.qsumx, dg, w.act, w.qa, w.qsa, w.qsuma); });
        return launch(MMOE_K_QUANT_ACT, [&] { kl(k_quant_act, (np + 7) / 8, 256, 0, w.act, np, w.qa, w.qsa, w.qsuma); });
    }
    return launch(MMOE_K_QUANT_ACT, [&] { kl(k_quant<MFF>, (np + 3) / 4, 256, 0, w.act, np, w.qa, w.qsa, w.qsuma); });
}
// device_grouping: the grouping came from k_group (pu is valid), so the 64-token-tile path may
// hand the down results to k_combine as int16 (not with checks on: the tests read them as fp32)
static int stage_experts(Work &w, int np, int nu_max, int tn, bool device_grouping) {
    int maxtiles = np / tn + (nu_max < np ? nu_max : np);
    int *dg = S.debug ? w.dbg_gu : nullptr, *dd = S.debug ? w.dbg_dn : nullptr;
    w.compact = device_grouping && tn == 64 && !S.debug;
    if (tn == 16 && S_expert16) return launch_expert16(w, maxtiles, dg, dd, device_grouping && w.grp16);
    if (launch_gateup(w, maxtiles, tn, dg)) return -1;
    if (!w.compact && launch_quant_act(w, maxtiles, tn, np, dg)) return -1;
    if (launch_down(w, maxtiles, tn, dd, w.compact)) return -1;
    return 0;
}

static int stage_combine(Work &w, int nb, float *d_x, int mode) {
    int n = nb * (MH / 4);
    int hzn = w.hist_used;   // the device grouping's counts (k_group) go back to zero here
    w.hist_used = 0;
    int *hz = hzn ? w.hist : nullptr;
    if (w.compact)
        return launch(MMOE_K_COMBINE, [&] { kl(k_combine16, nb, 256, 0, (const int16_t *)w.down, w.uw, w.tp, w.sp, w.tw, nb, d_x, mode, w.pu, w.eptr, w.qsa, w.dov, hz, hzn); });
    return launch(MMOE_K_COMBINE, [&] { kl(k_combine, (n + 255) / 256, 256, 0, w.down, w.uw, w.tp, w.sp, w.tw, nb, d_x, mode, hz, hzn); });
}

// Small batches (decode): three kernels, see decode.h. in = hn (do_norm 0) or the hidden state x whose
// rmsnorm(post_ln) is the MoE input (do_norm 1); hn is also written to w.hn.
static bool S_dec_enabled = true;
static int launch_dec_gateup(Work &w, int nb, int L) {
    int maxu = nb * MTOPK < MNE ? nb * MTOPK : MNE;
    int *dg = S.debug ? w.dbg_gu : nullptr;
    const ExpPtr *tab = S.layers[L].tab;
    return launch(MMOE_K_GATEUP, [&] { kl(k_dec_gateup, dim3(MFF / 8, maxu), 256, 0, w.rl, w.hn, nb, tab, w.top, w.tw, w.plan, w.utok, w.uw, w.tp, w.sp, w.eptr, w.qx, w.qsx, w.qsumx, w.act, dg); });
}
static int launch_dec_down(Work &w, int nb, float *d_x, int order) {
    int *dd = S.debug ? w.dbg_dn : nullptr;
    int mode = order == MMOE_ORDER_STEP ? MMOE_COMBINE_STEP : MMOE_COMBINE_BATCH;
    return launch(MMOE_K_DOWN, [&] { kl(k_dec_down, MH / 8, 256, 0, w.plan, w.eptr, w.act, w.qa, w.qsa, w.qsuma, w.tp, w.sp, w.uw, w.tw, nb, d_x, mode, w.down, dd); });
}
static int moe_dec(Work &w, int L, const float *in, int do_norm, int nb, float *d_x, int order) {
    LayerW &lw = S.layers[L];
    const uint16_t *pln = do_norm ? lw.post_ln : nullptr;
    w.rl_nb = 0;
    if (order == MMOE_ORDER_STEP) {
        if (launch(MMOE_K_ROUTER, [&] { kl(k_dec_route<16>, MNE * 16 / 64, 64, 0, in, nb, pln, do_norm, lw.rc16, lw.bias, w.hn, w.rl); })) return -1;
    } else {
        if (launch(MMOE_K_ROUTER, [&] { kl(k_dec_route<8>, MNE * 8 / 64, 64, 0, in, nb, pln, do_norm, lw.rc8, lw.bias, w.hn, w.rl); })) return -1;
    }
    w.rl_nb = nb;
    if (launch_dec_gateup(w, nb, L)) return -1;
    return launch_dec_down(w, nb, d_x, order);
}

// Whole MoE layer on device buffers: x[b] += MoE_L(hn[b]), with the work set w (no allocation here)
static int moe_dev(Work &w, int L, const float *d_hn, int nb, float *d_x, int order) {
    if (nb < 1 || nb > w.maxtok) { seterr("nb %d outside 1..%d (mmoe_init)", nb, w.maxtok); return -1; }
    if (L < 0 || L >= NLMAX || !S.layers[L].tab) { seterr("layer %d not set (mmoe_set_layer)", L); return -1; }
    if (nb <= DEC_MAXTOK && S_dec_enabled) return moe_dec(w, L, d_hn, 0, nb, d_x, order);
    int np = nb * MTOPK, tn = tile_tn(np);
    // below 512 tokens the router launch also runs the top-8 and the quantisation; the per-chunk counts are for
    // k_group, which the fused small-tile kernel does without (it groups itself)
    bool grp16 = tn == 16 && S_expert16 && nb <= E16_GRP_MAXTOK;
    if (stage_router(w, L, d_hn, nb, order, false, S_router_tk, grp16 ? nullptr : w.hist)) return -1;
    int rc = stage_route_group(w, L, nb, tn, d_hn);
    if (!rc) rc = stage_experts(w, np, MNE, tn, true);
    if (!rc) rc = stage_combine(w, nb, d_x, order == MMOE_ORDER_STEP ? MMOE_COMBINE_STEP : MMOE_COMBINE_BATCH);
    if (rc && w.hist_used) {   // a stage failed before the combine cleared the expert counts: clear them here
        // a fill kernel, not hipMemsetAsync: this may run under a caller's (or mmoe_stack_graph's) capture
        kl(k_fill_zero, (w.hist_used + 255) / 256, 256, 0, w.hist, w.hist_used);
        (void)hipGetLastError();
        w.hist_used = 0;
    }
    return rc;
}

// Experts for a host-given grouping (gpre_moe, gfull_moe, gpux): ustart[nu+1], ptok, pw, tp on the host,
// eptr[nu] resolved on the host. Input activations in w.hn.
static int experts_host_grouping(Work &w, int nb, int nu, const ExpPtr *eptr_h, const int *ustart, const int *ptok,
                                 const float *pw, const int *tp) {
    if (nu < 1 || nu > MNE) { seterr("nu %d outside 1..256", nu); return -1; }
    int np = ustart[nu];
    if (nb < 1 || nb > w.maxtok || np < 1 || np > w.maxp) { seterr("nb %d / pairs %d exceed capacity %d / %d", nb, np, w.maxtok, w.maxp); return -1; }
    for (int u = 0; u < nu; u++) if (ustart[u + 1] < ustart[u]) { seterr("ustart not ascending at %d", u); return -1; }
    for (int a = 0; a < np; a++) if (ptok[a] < 0 || ptok[a] >= nb) { seterr("ptok[%d] = %d outside 0..%d", a, ptok[a], nb - 1); return -1; }
    if (tp) for (int i = 0; i < nb * MTOPK; i++) if (tp[i] < 0 || tp[i] >= np) { seterr("tp[%d] = %d outside 0..%d", i, tp[i], np - 1); return -1; }
    int tn = tile_tn(np);
    HC(hipMemcpyAsync(w.eptr, eptr_h, sizeof(ExpPtr) * nu, hipMemcpyHostToDevice, S.st));
    HC(hipMemcpyAsync(w.ustart, ustart, sizeof(int) * (nu + 1), hipMemcpyHostToDevice, S.st));
    HC(hipMemcpyAsync(w.utok, ptok, sizeof(int) * np, hipMemcpyHostToDevice, S.st));
    if (pw) HC(hipMemcpyAsync(w.uw, pw, sizeof(float) * np, hipMemcpyHostToDevice, S.st));
    if (tp) HC(hipMemcpyAsync(w.tp, tp, sizeof(int) * nb * MTOPK, hipMemcpyHostToDevice, S.st));
    if (launch(MMOE_K_GROUP, [&] { kl(k_plan_from_ustart, 1, 64, 0, w.ustart, nu, w.plan, tn, w.tiles); })) return -1;
    if (stage_quant_x(w, w.hn, nb)) return -1;
    return stage_experts(w, np, nu, tn, false);
}

// loc (maple.c:276-277: per used expert 6 x (region slot, byte offset)) + regs -> device pointers
static int resolve_loc(const uint32_t *loc, const int *regs, int n, ExpPtr *out) {
    for (int u = 0; u < n; u++) {
        const uint8_t *p[6];
        for (int m = 0; m < 6; m++) {
            uint32_t slot = loc[u * 12 + 2 * m], off = loc[u * 12 + 2 * m + 1];
            if (slot > 3 || regs[slot] < 0 || regs[slot] >= (int)S.regions.size()) { seterr("loc[%d][%d]: region slot %u has no region", u, m, slot); return -1; }
            const Region &R = S.regions[regs[slot]];
            size_t len = m == 1 || m == 3 ? 512 * 4 : m == 5 ? 2048 * 4 : 262144;
            if ((size_t)off + len > R.len || (off & 15)) { seterr("loc[%d][%d]: offset %u outside region %d or not 16-byte aligned", u, m, off, regs[slot]); return -1; }
            p[m] = R.dev + off;
        }
        out[u] = ExpPtr{p[0], (const float *)p[1], p[2], (const float *)p[3], p[4], (const float *)p[5]};
    }
    return 0;
}

// ======================================================================================================
// maple.c's entry points (maple.c:247-272)
// ======================================================================================================
extern "C" {

// gpu_pre.m:266-316. Allocates the work buffers for chunks of up to maxtok tokens.
int gpre_init(int maxtok, int topk) {
    if (topk != MTOPK) { seterr("gpre_init: topk %d unsupported (this build is for TOPK = 8)", topk); return -1; }
    if (ctx_ready()) return -1;
    if (S.main.maxtok) return maxtok <= S.main.maxtok ? 0 : (seterr("gpre_init: already initialised for %d tokens", S.main.maxtok), -1);
    if (work_alloc(S.main, maxtok)) return -1;
    if (work_debug(S.main, S.debug)) return -1;
    fprintf(stderr, "maplemoe: MI355X MoE path, chunks up to %d tokens, expert codes resident in HBM\n", maxtok);
    return 0;
}

// gpu_pre.m:173-181. A page-aligned span of an mmapped shard becomes a region. On MI355X the span is copied
// into HBM once (it stays resident; the reference read it over PCIe in place).
int gpre_region(const void *p, size_t len) {
    if (ctx_ready()) return -1;
    size_t pg = (size_t)getpagesize();
    if (((uintptr_t)p % pg) || (len % pg) || !len) { seterr("gpre_region: region not page-aligned"); return -1; }
    if (S.regions.size() >= MMOE_MAXREG) { seterr("gpre_region: more than %d regions", MMOE_MAXREG); return -1; }
    uint8_t *d = nullptr;
    HC(hipMalloc(&d, len));
    hipEvent_t a = nullptr, b = nullptr;
    float ms = 0;
    hipError_t e = hipEventCreate(&a);
    if (e == hipSuccess) e = hipEventCreate(&b);
    if (e == hipSuccess) e = hipEventRecord(a, S.st);
    if (e == hipSuccess) e = hipMemcpyAsync(d, p, len, hipMemcpyHostToDevice, S.st);
    if (e == hipSuccess) e = hipEventRecord(b, S.st);
    if (e == hipSuccess) e = hipEventSynchronize(b);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    if (e != hipSuccess) { (void)hipFree(d); seterr("gpre_region: copy into HBM: %s", hipGetErrorString(e)); return -1; }
    S.t_region += ms * 1e-3;
    S.regions.push_back(Region{p, len, d});
    return (int)S.regions.size() - 1;
}

// gpu_pre.m:183-188. Weights are already resident in HBM: nothing to stage.
int gpre_stage(size_t bytes) { (void)bytes; return 0; }

// gpu_pre.m:321-385. Synchronous: x[nb][2048] post-norm (host), grouping from the host, y[nb][2048] =
// sum over each token's pairs of pw * down (overwritten). Returns device seconds. next: unused (resident).
double gpre_moe(const float *x, int nb, int nu, const uint32_t *loc, const int *regs, const int *next, const int *ustart,
                const int *ptok, const float *pw, const int *tp, float *y) {
    (void)next;
    Work &w = S.main;
    if (!w.maxtok) { seterr("gpre_moe before gpre_init"); return -1.0; }
    if (nb < 1 || nb > w.maxtok) { seterr("gpre_moe: nb %d outside 1..%d", nb, w.maxtok); return -1.0; }
    ExpPtr ep[MNE];
    if (nu < 1 || nu > MNE || resolve_loc(loc, regs, nu, ep)) { if (nu < 1 || nu > MNE) seterr("gpre_moe: nu %d", nu); return -1.0; }
    hipEvent_t a, b;
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) { seterr("gpre_moe: event"); return -1.0; }
    auto fail = [&] { (void)hipEventDestroy(a); (void)hipEventDestroy(b); return -1.0; };
    (void)hipEventRecord(a, S.st);
    if (hipMemcpyAsync(w.hn, x, (size_t)nb * MH * 4, hipMemcpyHostToDevice, S.st) != hipSuccess) { seterr("gpre_moe: copy x"); return fail(); }
    if (experts_host_grouping(w, nb, nu, ep, ustart, ptok, pw, tp)) return fail();
    if (stage_combine(w, nb, w.x, MMOE_COMBINE_OVERWRITE)) return fail();
    (void)hipEventRecord(b, S.st);
    if (hipMemcpyAsync(y, w.x, (size_t)nb * MH * 4, hipMemcpyDeviceToHost, S.st) != hipSuccess || hipStreamSynchronize(S.st) != hipSuccess) {
        seterr("gpre_moe: %s", hipGetErrorString(hipGetLastError())); return fail();
    }
    float ms = 0; (void)hipEventElapsedTime(&ms, a, b);
    (void)hipEventDestroy(a); (void)hipEventDestroy(b);
    S.t_moe += ms * 1e-3;
    return ms * 1e-3;
}

// gpu_pre.m:257-264: seconds spent moving weights to the card (here: the one-time region copies)
double gpre_blit_seconds(void) { return S.t_region; }

// ---- dense ternary projections: attention q/k/v (group 2L) and o (group 2L + 1), gpu_pre.m:200-256 ----
// The matrices are staged on the host by gpre_dense_add and copied into one HBM buffer by gpre_dense_done.
// gpre_dense quantises x as maple.c's prep (maple.c:183-194) and runs k_dense, the int8 GEMM with maple.c's
// integer and fp32 sequence (tdot_multi), so y equals maple.c's CPU projections (jobB_qkv / jobB_o) bit for
// bit (the Metal version multiplies fp32 activations instead).
#define DGRP 48
#ifndef DENSE_W
#define DENSE_W 2   // k_dense waves per workgroup (64 rows each)
#endif
static struct {
    std::vector<uint8_t> host;                   // staging until gpre_dense_done
    struct Mat { size_t codes, scales; int rows; } mat[DGRP][3];
    int n[DGRP], rows[DGRP], maxtok;
    uint8_t *dev;                                // all matrices in HBM
    DenseMat *dmat;                              // per group, 3 slots
    int *drbs;                                   // per group, 4 row-block offsets
    float *y;                                    // [maxtok][max rows]
    int ymax, ready, bad;
    double t;
} DN;

void gpre_dense_add(int g, const uint8_t *codes, const float *scales, int rows, int cols) {
    if (DN.ready) { seterr("gpre_dense_add after gpre_dense_done: ignored"); return; }
    if (g < 0 || g >= DGRP || DN.n[g] >= 3 || cols != MH || rows < 256 || rows % 256 || !codes || !scales) {
        DN.bad = 1;   // reported by gpre_dense_done (this call returns nothing, as in gpu_pre.m)
        return;
    }
    auto put = [&](const void *p, size_t n) {
        size_t o = (DN.host.size() + 255) / 256 * 256;
        DN.host.resize(o + n);
        memcpy(DN.host.data() + o, p, n);
        return o;
    };
    auto &m = DN.mat[g][DN.n[g]++];
    m.codes = put(codes, (size_t)rows * cols / 4);
    m.scales = put(scales, (size_t)rows * 4);
    m.rows = rows;
    DN.rows[g] += rows;
}

int gpre_dense_done(int maxtok) {
    if (ctx_ready()) return -1;
    if (DN.ready) { seterr("gpre_dense_done: the projections are already on the card (mmoe_dense_reset first)"); return -1; }
    if (DN.bad) { seterr("gpre_dense_add: a matrix was not 256k x 2048 (or more than 3 per group)"); fprintf(stderr, "maplemoe: %s\n", mmoe_last_error()); return -1; }
    if (DN.host.empty() || maxtok < 1 || maxtok > 2048 || maxtok > S.main.maxtok) {
        seterr("gpre_dense_done: nothing added, or maxtok %d outside 1..%d (gpre_init)", maxtok, S.main.maxtok);
        return -1;
    }
    HC(hipMalloc(&DN.dev, DN.host.size()));
    HC(hipMemcpy(DN.dev, DN.host.data(), DN.host.size(), hipMemcpyHostToDevice));
    DenseMat hm[DGRP][3] = {};
    int hr[DGRP][4] = {};
    DN.ymax = 0;
    for (int g = 0; g < DGRP; g++) {
        int yo = 0;
        for (int k = 0; k < DN.n[g]; k++) {
            hm[g][k] = DenseMat{DN.dev + DN.mat[g][k].codes, (const float *)(DN.dev + DN.mat[g][k].scales), DN.mat[g][k].rows, yo};
            hr[g][k + 1] = hr[g][k] + DN.mat[g][k].rows / (64 * DENSE_W);
            yo += DN.mat[g][k].rows;
        }
        for (int k = DN.n[g] + 1; k < 4; k++) hr[g][k] = hr[g][DN.n[g]];
        if (yo > DN.ymax) DN.ymax = yo;
    }
    HC(hipMalloc(&DN.dmat, sizeof hm)); HC(hipMemcpy(DN.dmat, hm, sizeof hm, hipMemcpyHostToDevice));
    HC(hipMalloc(&DN.drbs, sizeof hr)); HC(hipMemcpy(DN.drbs, hr, sizeof hr, hipMemcpyHostToDevice));
    HC(hipMalloc(&DN.y, (size_t)maxtok * DN.ymax * 4));
    DN.maxtok = maxtok;
    fprintf(stderr, "maplemoe: attention projections in HBM, %.0f MB\n", DN.host.size() / 1e6);
    std::vector<uint8_t>().swap(DN.host);
    DN.ready = 1;
    return 0;
}

// Drops the projections from HBM; gpre_dense_add may stage a new set.
int mmoe_dense_reset(void) {
    if (DN.dev) HC(hipFree(DN.dev));
    if (DN.dmat) HC(hipFree(DN.dmat));
    if (DN.drbs) HC(hipFree(DN.drbs));
    if (DN.y) HC(hipFree(DN.y));
    std::vector<uint8_t>().swap(DN.host);
    memset(DN.mat, 0, sizeof DN.mat); memset(DN.n, 0, sizeof DN.n); memset(DN.rows, 0, sizeof DN.rows);
    DN.maxtok = 0; DN.dev = nullptr; DN.dmat = nullptr; DN.drbs = nullptr; DN.y = nullptr;
    DN.ymax = DN.ready = DN.bad = 0;
    return 0;
}

// y[nb][rows of group g] = group g's matrices times x[nb][2048] (host arrays); returns device seconds
double gpre_dense(int g, const float *x, int nb, float *y) {
    if (!DN.ready) { seterr("gpre_dense before gpre_dense_done"); return -1.0; }
    if (g < 0 || g >= DGRP || !DN.n[g]) { seterr("gpre_dense: group %d has no matrices", g); return -1.0; }
    if (nb < 1 || nb > DN.maxtok) { seterr("gpre_dense: nb %d outside 1..%d", nb, DN.maxtok); return -1.0; }
    Work &w = S.main;
    int ys = DN.rows[g], nrb = ys / (64 * DENSE_W);
    hipEvent_t a, b;
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) { seterr("gpre_dense: event"); return -1.0; }
    auto fail = [&] { (void)hipEventDestroy(a); (void)hipEventDestroy(b); return -1.0; };
    (void)hipEventRecord(a, S.st);
    if (hipMemcpyAsync(w.hn, x, (size_t)nb * MH * 4, hipMemcpyHostToDevice, S.st) != hipSuccess) { seterr("gpre_dense: copy x"); return fail(); }
    if (stage_quant_x(w, w.hn, nb)) return fail();
    if (launch(MMOE_K_DENSE, [&] {
            kl(k_dense<DENSE_W>, dim3(nrb, (nb + 63) / 64), 64 * DENSE_W, 0, DN.dmat + g * 3, DN.drbs + g * 4, DN.n[g], nb, ys, w.qx, w.qsx, w.qsumx, DN.y);
        })) return fail();
    (void)hipEventRecord(b, S.st);
    if (hipMemcpyAsync(y, DN.y, (size_t)nb * ys * 4, hipMemcpyDeviceToHost, S.st) != hipSuccess || hipStreamSynchronize(S.st) != hipSuccess) {
        seterr("gpre_dense: %s", hipGetErrorString(hipGetLastError())); return fail();
    }
    float ms = 0; (void)hipEventElapsedTime(&ms, a, b);
    (void)hipEventDestroy(a); (void)hipEventDestroy(b);
    DN.t += ms * 1e-3;
    return ms * 1e-3;
}

// Output head (gpu_head.m): not part of the MoE path; init failure makes maple.c use its CPU head.
int gpu_head_init(const uint16_t *w, int rows, int cols) { (void)w; (void)rows; (void)cols; return -1; }
int gpu_head_init_i8(const int8_t *w, const float *scale, int rows, int cols) { (void)w; (void)scale; (void)rows; (void)cols; return -1; }
void gpu_head_run(const float *x, float *y) { (void)x; (void)y; seterr("gpu_head_run: not part of this build"); }
void gpu_head_run_multi(const float *x, int n, float *y) { (void)x; (void)n; (void)y; seterr("gpu_head_run_multi: not part of this build"); }

static int set_router(int L, const uint16_t *router);

// ---- whole layers on the card (gpu_pre.m:387-594): the hidden state of a chunk stays in HBM; per layer
// gfull_attn runs rmsnorm -> q/k/v (k_dense) -> q/k norm + rope + fp16 cache -> attention -> o (x += o) ->
// post-norm -> router logits (exact chains), and gfull_moe the experts of the pairs the host picked.
// One sequence; the chunk's nb tokens sit at positions pos0 .. pos0+nb-1 of a cache of ctx positions.
#define AT_SC_NB 2    // tokens per k_att_scores workgroup
#define GF_NWL 4352   // per layer in the norms gfull_init receives: in_ln 2048 | post_ln 2048 | q_norm 128 | k_norm 128
static struct {
    int ready, ctx, win, maxtok, pos0;
    uint16_t *nw;                 // bf16 [24][4352] (the fp32 norms are bf16 values: exact)
    float *cs;                    // [ctx][32][2]
    __half *kc, *vc, *ko;         // [24][ctx][512] x 2, [24][maxtok][1024]
    uint16_t *ko_host;            // gfull_read's copy
    float *qkv, *att, *sc, *inv, *mx;  // [maxtok][3072], [maxtok][2048], [maxtok * 16][ctx], [maxtok * 16] x 2
    double t_attn;
} GF;

int gfull_init(int ctx, int maxtok, int win, const float *norms, const uint16_t *router, const float *cs) {
    if (ctx_ready()) return -1;
    if (!DN.ready) { seterr("gfull_init: the dense projections are not on the card (gpre_dense_done)"); fprintf(stderr, "maplemoe: %s\n", mmoe_last_error()); return -1; }
    if (ctx < 1 || maxtok < 1 || maxtok > S.main.maxtok || maxtok > DN.maxtok || win < 0 || !norms || !router || !cs) {
        seterr("gfull_init: ctx %d / maxtok %d (context %d) / win %d", ctx, maxtok, S.main.maxtok, win); return -1;
    }
    // a second set-up replaces the first; buffers of a set-up that failed part way are released here too
    GF.ready = 0;
    void **dbuf[] = {(void **)&GF.nw, (void **)&GF.cs, (void **)&GF.kc, (void **)&GF.vc, (void **)&GF.ko,
                     (void **)&GF.qkv, (void **)&GF.att, (void **)&GF.sc, (void **)&GF.inv, (void **)&GF.mx};
    for (void **pp : dbuf) if (*pp) { HC(hipFree(*pp)); *pp = nullptr; }
    free(GF.ko_host); GF.ko_host = nullptr;
    std::vector<uint16_t> nw((size_t)24 * GF_NWL);
    for (size_t i = 0; i < nw.size(); i++) { uint32_t u; memcpy(&u, &norms[i], 4); nw[i] = (uint16_t)(u >> 16); }
    HC(hipMalloc(&GF.nw, nw.size() * 2)); HC(hipMemcpy(GF.nw, nw.data(), nw.size() * 2, hipMemcpyHostToDevice));
    HC(hipMalloc(&GF.cs, (size_t)ctx * 64 * 4)); HC(hipMemcpy(GF.cs, cs, (size_t)ctx * 64 * 4, hipMemcpyHostToDevice));
    size_t kvb = (size_t)24 * ctx * 512 * 2, kob = (size_t)24 * maxtok * 1024 * 2;
    HC(hipMalloc(&GF.kc, kvb)); HC(hipMalloc(&GF.vc, kvb)); HC(hipMalloc(&GF.ko, kob));
    HC(hipMemset(GF.kc, 0, kvb)); HC(hipMemset(GF.vc, 0, kvb));
    GF.ko_host = (uint16_t *)malloc(kob);
    if (!GF.ko_host) { seterr("gfull_init: %zu bytes of host memory", kob); return -1; }
    HC(hipMalloc(&GF.qkv, (size_t)maxtok * 3072 * 4)); HC(hipMalloc(&GF.att, (size_t)maxtok * MH * 4));
    HC(hipMalloc(&GF.sc, (size_t)maxtok * 16 * ctx * 4)); HC(hipMalloc(&GF.inv, (size_t)maxtok * 16 * 4)); HC(hipMalloc(&GF.mx, (size_t)maxtok * 16 * 4));
    for (int L = 0; L < 24; L++) {
        if (set_router(L, router + (size_t)L * MNE * MH)) return -1;
        LayerW &lw = S.layers[L];
        if (!lw.post_ln) HC(hipMalloc(&lw.post_ln, MH * 2));
        HC(hipMemcpy(lw.post_ln, nw.data() + (size_t)L * GF_NWL + MH, MH * 2, hipMemcpyHostToDevice));
    }
    GF.ctx = ctx; GF.win = win; GF.maxtok = maxtok; GF.ready = 1;
    S.gfull = true;
    fprintf(stderr, "maplemoe: whole layers on the card, key/value cache %.0f MB\n", 2.0 * kvb / 1e6);
    return 0;
}
// a new chunk: nb hidden vectors (embeddings) at positions pos0..
void gfull_begin(const float *x, int nb, int pos0) {
    S.gfull_nb = 0;   // a rejected chunk leaves no chunk: gfull_attn / gfull_moe then report it
    if (!S.gfull || nb < 1 || nb > S.main.maxtok) { seterr("gfull_begin: not set up or nb %d out of range", nb); return; }
    if (GF.ready && (nb > GF.maxtok || pos0 < 0 || pos0 + nb > GF.ctx)) { seterr("gfull_begin: positions %d..%d past ctx %d", pos0, pos0 + nb - 1, GF.ctx); return; }
    S.gfull_nb = nb; GF.pos0 = pos0;
    HCV(hipMemcpyAsync(S.main.x, x, (size_t)nb * MH * 4, hipMemcpyHostToDevice, S.st));
}
// The attention half of layer L (asynchronous): x += o(attention(q, k, v of rmsnorm(x, in_ln))), k and v into
// the layer's cache and ko.
static int gfull_attn_launch(int L, int glob) {
    if (!GF.ready || !S.gfull_nb) { seterr("gfull_attn: gfull_init / gfull_begin first"); return -1; }
    if (L < 0 || L >= 24) { seterr("gfull_attn: layer %d", L); return -1; }
    if (DN.rows[2 * L] != 3072 || DN.rows[2 * L + 1] != 2048) {
        seterr("gfull_attn: layer %d projections are not q,k,v (3072 rows) and o (2048) (gpre_dense_add)", L); return -1;
    }
    Work &w = S.main;
    int nb = S.gfull_nb, pos0 = GF.pos0, ctx = GF.ctx, win = GF.win, g = 2 * L;
    const uint16_t *nwl = GF.nw + (size_t)L * GF_NWL;
    __half *kcl = GF.kc + (size_t)L * ctx * 512, *vcl = GF.vc + (size_t)L * ctx * 512, *kol = GF.ko + (size_t)L * GF.maxtok * 1024;
    if (launch(MMOE_K_RMSNORM, [&] { kl(k_rmsnorm, nb, 256, 0, w.x, nwl, w.hn, nb); })) return -1;
    if (stage_quant_x(w, w.hn, nb)) return -1;
    if (launch(MMOE_K_DENSE, [&] {
        kl(k_dense<DENSE_W>, dim3(3072 / (64 * DENSE_W), (nb + 63) / 64), 64 * DENSE_W, 0, DN.dmat + g * 3, DN.drbs + g * 4, DN.n[g], nb, 3072, w.qx, w.qsx, w.qsumx, GF.qkv);
    })) return -1;
    if (launch(MMOE_K_QKN, [&] {
        kl(k_qkn, nb, 256, 0, GF.qkv, pos0, glob, nwl + 4096, nwl + 4224, GF.cs, kcl, vcl, kol, GF.mx);
    })) return -1;
    int span = glob ? pos0 + nb : std::min(pos0 + nb, win + AT_SC_NB);   // positions one token group can see
    if (launch(MMOE_K_ATT_SCORES, [&] {
        kl(k_att_scores<AT_SC_NB>, dim3((nb + AT_SC_NB - 1) / AT_SC_NB * 4, (span + 63) / 64), 64, 0, GF.qkv, nb, pos0, glob, win, kcl, GF.sc, GF.mx, ctx);
    })) return -1;
    if (launch(MMOE_K_ATT_SOFTMAX, [&] { kl(k_att_softmax, nb, 256, 0, pos0, glob, win, GF.sc, GF.mx, GF.inv, ctx); })) return -1;
    if (launch(MMOE_K_ATT_PV, [&] {   // small chunks: fewer tokens per workgroup, more workgroups
        if (nb > 256) kl(k_att_pv<4>, (nb + 3) / 4 * 4, 256, 0, nb, pos0, glob, win, GF.sc, GF.mx, GF.inv, vcl, GF.att, ctx);
        else kl(k_att_pv<2>, (nb + 1) / 2 * 4, 256, 0, nb, pos0, glob, win, GF.sc, GF.mx, GF.inv, vcl, GF.att, ctx);
    })) return -1;
    if (stage_quant_x(w, GF.att, nb)) return -1;
    return launch(MMOE_K_DENSE, [&] {
        kl(k_dense<DENSE_W, true>, dim3(MH / (64 * DENSE_W), (nb + 63) / 64), 64 * DENSE_W, 0, DN.dmat + (g + 1) * 3, DN.drbs + (g + 1) * 4, DN.n[g + 1], nb, MH, w.qx, w.qsx, w.qsumx, w.x);
    });
}
// The attention half of layer L and the router: rl gets nb x 256 logits. Synchronous; returns device seconds.
double gfull_attn(int L, int glob, float *rl) {
    hipEvent_t a, b;
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) { seterr("gfull_attn: event"); return -1.0; }
    (void)hipEventRecord(a, S.st);
    int rc = gfull_attn_launch(L, glob);
    (void)hipEventRecord(b, S.st);
    if (!rc) rc = mmoe_gfull_post_norm(L, rl);
    if (!rc && hipStreamSynchronize(S.st) != hipSuccess) { seterr("gfull_attn: stream"); rc = -1; }
    float ms = 0;
    if (!rc) (void)hipEventElapsedTime(&ms, a, b);
    (void)hipEventDestroy(a); (void)hipEventDestroy(b);
    if (rc) return -1.0;
    GF.t_attn += ms * 1e-3;
    return ms * 1e-3;
}
// gpu_pre.m:508-566: asynchronous; adds each token's weighted expert outputs into the device hidden state
void gfull_moe(int nu, const uint32_t *loc, const int *regs, const int *ustart, const int *ptok, const float *pw, const int *tp) {
    if (!S.gfull || !S.gfull_nb) { seterr("gfull_moe: gfull state not set up (gfull_begin)"); return; }
    ExpPtr ep[MNE];
    if (nu < 1 || nu > MNE) { seterr("gfull_moe: nu %d", nu); return; }
    if (resolve_loc(loc, regs, nu, ep)) return;
    if (experts_host_grouping(S.main, S.gfull_nb, nu, ep, ustart, ptok, pw, tp)) return;
    stage_combine(S.main, S.gfull_nb, S.main.x, MMOE_COMBINE_ADD);
}
// gpu_pre.m:569-584: waits, copies the hidden state back; *ko -> the chunk's k,v of every layer
// (24 x maxtok x 1024 fp16, k | v per token; NULL before gfull_init)
void gfull_read(float *x, const uint16_t **ko) {
    HCV(hipStreamSynchronize(S.st));
    if (x && S.gfull) HCV(hipMemcpy(x, S.main.x, (size_t)S.gfull_nb * MH * 4, hipMemcpyDeviceToHost));
    if (ko) {
        *ko = NULL;
        if (GF.ready) {   // the chunk's nb rows of every layer only (the [24][maxtok][1024] layout is kept)
            size_t pitch = (size_t)GF.maxtok * 1024 * 2, rows = (size_t)(S.gfull_nb ? S.gfull_nb : GF.maxtok) * 1024 * 2;
            HCV(hipMemcpy2D(GF.ko_host, pitch, GF.ko, pitch, rows, 24, hipMemcpyDeviceToHost));
            *ko = GF.ko_host;
        }
    }
}
void gfull_write_x(const float *x) {
    if (!S.gfull) { seterr("gfull_write_x: not set up"); return; }
    HCV(hipMemcpyAsync(S.main.x, x, (size_t)S.gfull_nb * MH * 4, hipMemcpyHostToDevice, S.st));
}
int gfull_maxtok(void) { return GF.ready ? GF.maxtok : S.main.maxtok; }
void gfull_report(void) { fprintf(stderr, "maplemoe: card %.3f s attention half, %.3f s expert work\n", GF.t_attn, S.t_moe); }

// ---- decode expert cache (gpu_exp.m:155-291). Slots hold experts in the reference layout in HBM; a hit
// runs prep, gate/up, SiLU, re-quant and down on the device with maple.c's int8 semantics.
int gpux_init(int layers, int slots) {
    if (ctx_ready()) return -1;
    if (layers < 1 || layers > NLMAX || slots < 1 || slots > 256) { seterr("gpux_init: layers %d / slots %d out of range", layers, slots); return -1; }
    if (!S.dec.maxtok && work_alloc(S.dec, MMOE_GPUX_MAXTOK)) return -1;
    if (work_debug(S.dec, S.debug)) return -1;
    if (S.gx_mem) {   // a second set-up replaces the first (its slots are gone until uploaded again)
        uint8_t *old = S.gx_mem;
        S.gx_mem = nullptr; S.gx_layers = S.gx_slots = 0;
        HC(hipFree(old));
    }
    HC(hipMalloc(&S.gx_mem, (size_t)layers * slots * EXPERT_BYTES));
    S.gx_layers = layers; S.gx_slots = slots;
    return 0;
}
static ExpPtr slot_ptr(int L, int slot) {
    uint8_t *b = S.gx_mem + ((size_t)L * S.gx_slots + slot) * EXPERT_BYTES;
    return ExpPtr{b, (const float *)(b + 262144), b + 264192, (const float *)(b + 526336), b + 528384, (const float *)(b + 790528)};
}
void gpux_upload(int L, int slot, const uint8_t *gc, const float *gs, const uint8_t *uc, const float *us, const uint8_t *dc, const float *ds) {
    if (!S.gx_mem || L < 0 || L >= S.gx_layers || slot < 0 || slot >= S.gx_slots) { seterr("gpux_upload: L %d slot %d out of range", L, slot); return; }
    ExpPtr p = slot_ptr(L, slot);
    HCV(hipMemcpyAsync((void *)p.gc, gc, 262144, hipMemcpyHostToDevice, S.st));
    HCV(hipMemcpyAsync((void *)p.gs, gs, 2048, hipMemcpyHostToDevice, S.st));
    HCV(hipMemcpyAsync((void *)p.uc, uc, 262144, hipMemcpyHostToDevice, S.st));
    HCV(hipMemcpyAsync((void *)p.us, us, 2048, hipMemcpyHostToDevice, S.st));
    HCV(hipMemcpyAsync((void *)p.dc, dc, 262144, hipMemcpyHostToDevice, S.st));
    HCV(hipMemcpyAsync((void *)p.ds, ds, 8192, hipMemcpyHostToDevice, S.st));
    HCV(hipStreamSynchronize(S.st));  // the host buffers are the caller's mmap; keep the copy synchronous
}
static void *gpux_start(int L, const float *x, int nb, int nu, const int *slots, const int *pstart, const int *ptok) {
    if (!S.gx_mem || L < 0 || L >= S.gx_layers) { seterr("gpux: not initialised or layer %d out of range", L); return NULL; }
    Work &w = S.dec;
    if (nb < 1 || nb > w.maxtok) { seterr("gpux: %d vectors exceed %d", nb, w.maxtok); return NULL; }
    ExpPtr ep[MNE];
    if (nu < 1 || nu > MNE) { seterr("gpux: %d experts", nu); return NULL; }
    for (int k = 0; k < nu; k++) {
        if (slots[k] < 0 || slots[k] >= S.gx_slots) { seterr("gpux: slot %d out of range", slots[k]); return NULL; }
        ep[k] = slot_ptr(L, slots[k]);
    }
    HCN(hipMemcpyAsync(w.hn, x, (size_t)nb * MH * 4, hipMemcpyHostToDevice, S.st));
    if (experts_host_grouping(w, nb, nu, ep, pstart, ptok, NULL, NULL)) return NULL;
    HCN(hipEventRecord(S.gx_ev, S.st));
    S.gx_np = pstart[nu];
    return (void *)&S.gx_ev;
}
static void gpux_finish(void *h, float *out, int np) {
    if (h != (void *)&S.gx_ev) { seterr("gpux_end: unknown handle"); return; }
    if (np != S.gx_np) { seterr("gpux_end: %d outputs asked, %d computed", np, S.gx_np); return; }
    HCV(hipMemcpyAsync(out, S.dec.down, (size_t)np * MH * 4, hipMemcpyDeviceToHost, S.st));
    HCV(hipStreamSynchronize(S.st));
}
// n hits of one token: outputs out[k][2048] = down of slot k's expert (unweighted), maple.c:628-642
void *gpux_begin(int L, const float *x, int n, const int *slots) {
    int ps[MNE + 1], pt[MNE];
    if (n < 1 || n > MNE) { seterr("gpux_begin: n %d", n); return NULL; }
    for (int k = 0; k <= n; k++) ps[k] = k;
    for (int k = 0; k < n; k++) pt[k] = 0;
    return gpux_start(L, x, 1, n, slots, ps, pt);
}
void gpux_end(void *h, float *out, int n) { gpux_finish(h, out, n); }
void *gpux_begin_multi(int L, const float *x, int nb, int nu, const int *slots, const int *pstart, const int *ptok) {
    return gpux_start(L, x, nb, nu, slots, pstart, ptok);
}
void gpux_end_multi(void *h, float *out, int np) { gpux_finish(h, out, np); }

// ======================================================================================================
// mmoe_*: the whole MoE layer on the device
// ======================================================================================================
const char *mmoe_last_error(void) { return g_err; }

int mmoe_init(int maxtok) {
    if (ctx_ready()) return -1;
    if (S.main.maxtok) return maxtok <= S.main.maxtok ? 0 : (seterr("mmoe_init: already initialised for %d tokens", S.main.maxtok), -1);
    if (work_alloc(S.main, maxtok)) return -1;
    return work_debug(S.main, S.debug);
}

// Small batches take the three-kernel decode path unless switched off (tests compare both paths).
// Every setter below changes what a captured graph holds (kernels, pointers it passes): each drops the graph
// before the change, so the next mmoe_stack_graph captures again and no replay touches freed memory.
int mmoe_set_router_mode(int exact) { if (mmoe_graph_reset()) return -1; S_router_exact = exact != 0; return 0; }
int mmoe_set_decode_path(int on) { if (mmoe_graph_reset()) return -1; S_dec_enabled = on != 0; return 0; }
int mmoe_set_expert_path(int fused) { if (mmoe_graph_reset()) return -1; S_expert16 = fused != 0; return 0; }

int mmoe_set_debug(int on) {
    if (mmoe_graph_reset()) return -1;
    S.debug = on != 0;
    if (S.main.maxtok && work_debug(S.main, S.debug)) return -1;
    if (S.dec.maxtok && work_debug(S.dec, S.debug)) return -1;
    return 0;
}

int mmoe_set_layer(int L, const uint32_t *loc, const int *regs, const uint16_t *router, const uint16_t *post_ln) {
    if (ctx_ready()) return -1;
    if (L < 0 || L >= NLMAX) { seterr("mmoe_set_layer: layer %d outside 0..%d", L, NLMAX - 1); return -1; }
    if (mmoe_graph_reset()) return -1;
    LayerW &lw = S.layers[L];
    ExpPtr ep[MNE];
    if (resolve_loc(loc, regs, MNE, ep)) return -1;
    if (!lw.tab) HC(hipMalloc(&lw.tab, sizeof(ExpPtr) * MNE));
    HC(hipMemcpy(lw.tab, ep, sizeof ep, hipMemcpyHostToDevice));
    if (set_router(L, router)) return -1;
    if (post_ln) {
        if (!lw.post_ln) HC(hipMalloc(&lw.post_ln, MH * 2));
        HC(hipMemcpy(lw.post_ln, post_ln, MH * 2, hipMemcpyHostToDevice));
    }
    return 0;
}

// Layer L's router (bf16 [256][2048]) into HBM with its chain-major copies (both orders, and fp32 for the
// tiled batch router) and the bound the MFMA router option uses.
static int set_router(int L, const uint16_t *router) {
    if (mmoe_graph_reset()) return -1;
    LayerW &lw = S.layers[L];
    if (!lw.router) HC(hipMalloc(&lw.router, (size_t)MNE * MH * 2));
    HC(hipMemcpy(lw.router, router, (size_t)MNE * MH * 2, hipMemcpyHostToDevice));
    if (!lw.rc16) HC(hipMalloc(&lw.rc16, (size_t)MNE * MH * 2));
    if (!lw.rc8) HC(hipMalloc(&lw.rc8, (size_t)MNE * MH * 2));
    kl(k_router_chainmajor<16>, MNE * MH / 256, 256, 0, lw.router, lw.rc16);
    kl(k_router_chainmajor<8>, MNE * MH / 256, 256, 0, lw.router, lw.rc8);
    if (!lw.rf8) HC(hipMalloc(&lw.rf8, (size_t)MNE * MH * 4));
    kl(k_router_chain8_f32, MNE * MH / 256, 256, 0, lw.router, lw.rf8);
    if (!lw.w1max) HC(hipMalloc(&lw.w1max, 2 * sizeof(float)));
    kl(k_router_l1max, 1, 256, 0, lw.router, lw.w1max);
    HC(hipGetLastError());
    HC(hipStreamSynchronize(S.st));
    return 0;
}

int mmoe_set_bias(int L, const float *bias) {
    if (ctx_ready()) return -1;
    if (L < 0 || L >= NLMAX) { seterr("mmoe_set_bias: layer %d", L); return -1; }
    if (mmoe_graph_reset()) return -1;
    LayerW &lw = S.layers[L];
    if (!bias) { if (lw.bias) HC(hipFree(lw.bias)); lw.bias = nullptr; return 0; }
    if (!lw.bias) HC(hipMalloc(&lw.bias, MNE * 4));
    HC(hipMemcpy(lw.bias, bias, MNE * 4, hipMemcpyHostToDevice));
    return 0;
}

int mmoe_moe(int L, const float *hn, int nb, float *x, int order) {
    Work &w = S.main;
    if (!w.maxtok) { seterr("mmoe_moe before mmoe_init"); return -1; }
    if (nb < 1 || nb > w.maxtok) { seterr("mmoe_moe: nb %d outside 1..%d", nb, w.maxtok); return -1; }
    HC(hipMemcpyAsync(w.hn, hn, (size_t)nb * MH * 4, hipMemcpyHostToDevice, S.st));
    HC(hipMemcpyAsync(w.x, x, (size_t)nb * MH * 4, hipMemcpyHostToDevice, S.st));
    if (moe_dev(w, L, w.hn, nb, w.x, order)) return -1;
    HC(hipMemcpyAsync(x, w.x, (size_t)nb * MH * 4, hipMemcpyDeviceToHost, S.st));
    HC(hipStreamSynchronize(S.st));
    return 0;
}

int mmoe_moe_dev(int L, const float *d_hn, int nb, float *d_x, int order) { return moe_dev(S.main, L, d_hn, nb, d_x, order); }

// maple.c's softmax/top-8 (job_topk, maple.c:910-922) and grouping (group_pairs, maple.c:924-938, plus the tp table
// its callers build before gpre_moe / gfull_moe, maple.c:762 and 1019) of nb tokens' logits, on the device: the top-8
// kernel (its quantisation row of blocks left out) and k_group, which also fill the plan and tiles the expert
// kernels would use. k_group publishes the used experts' pointers from a layer table: routing alone has no layer,
// so a zeroed table stands in. rl = NULL takes the logits already in the work set's rl (exact ones only, of nb tokens):
// after gfull_attn(L, glob, NULL) the chunk's routing then needs no logits on the host at all.
int mmoe_route(const float *rl, int nb, int *top, float *tw, int *ue, int *ustart, int *utok, float *uw, int *tp) {
    Work &w = S.main;
    if (!w.maxtok) { seterr("mmoe_route before mmoe_init"); return -1; }
    if (nb < 1 || nb > w.maxtok) { seterr("mmoe_route: nb %d outside 1..%d", nb, w.maxtok); return -1; }
    if (!rl && w.rl_nb != nb) {
        seterr("mmoe_route: no logits given and the last router call did not leave exact logits of %d tokens", nb);
        return -1;
    }
    if (!S.zero_tab) {
        HC(hipMalloc(&S.zero_tab, sizeof(ExpPtr) * MNE));
        HC(hipMemset(S.zero_tab, 0, sizeof(ExpPtr) * MNE));
    }
    const int nch = (nb + 63) / 64, P = nb * MTOPK;
    if (rl) { HC(hipMemcpyAsync(w.rl, rl, (size_t)nb * MNE * 4, hipMemcpyHostToDevice, S.st)); w.rl_nb = nb; }
    if (launch(MMOE_K_TOPK, [&] { kl(k_topk_quant, dim3((nb + 3) / 4, 1), 256, 0, (const float *)w.rl, (const float *)nullptr, nb, w.top, w.tw,
                                     (int8_t *)nullptr, (float *)nullptr, (int *)nullptr, w.hist); }))
        return -1;
    int rc = launch(MMOE_K_GROUP, [&] { kl(k_group, nch, 512, 0, w.hist, nb, w.plan, S.zero_tab, w.eptr, 64, w.tiles, w.eu, w.top, w.tw, w.utok,
                                           w.uw, w.tp, w.sp, w.pu); });
    kl(k_fill_zero, (nch * MNE + 255) / 256, 256, 0, w.hist, nch * MNE);   // the per-chunk counts, for the next call
    if (rc) { (void)hipGetLastError(); return -1; }
    HC(hipGetLastError());
    Plan pl;   // pageable: the copy completes before the synchronisation below returns
    HC(hipMemcpyAsync(&pl, w.plan, sizeof(Plan), hipMemcpyDeviceToHost, S.st));
    if (top) HC(hipMemcpyAsync(top, w.top, (size_t)P * 4, hipMemcpyDeviceToHost, S.st));
    if (tw) HC(hipMemcpyAsync(tw, w.tw, (size_t)P * 4, hipMemcpyDeviceToHost, S.st));
    if (utok) HC(hipMemcpyAsync(utok, w.utok, (size_t)P * 4, hipMemcpyDeviceToHost, S.st));
    if (uw) HC(hipMemcpyAsync(uw, w.uw, (size_t)P * 4, hipMemcpyDeviceToHost, S.st));
    if (tp) HC(hipMemcpyAsync(tp, w.tp, (size_t)P * 4, hipMemcpyDeviceToHost, S.st));
    HC(hipStreamSynchronize(S.st));
    if (ue) memcpy(ue, pl.ue, sizeof(int) * pl.nu);
    if (ustart) memcpy(ustart, pl.ustart, sizeof(int) * (pl.nu + 1));
    return pl.nu;
}

// mmoe_moe_dev for batches of up to MMOE_NOALLOC_MAXTOK tokens with every work buffer in the library's static
// scratch: no allocation of any kind. Calls on one device share that scratch (and queue on one stream).
int mmoe_moe_dev_noalloc(int L, const float *d_hn, int nb, float *d_x, int order) {
    if (!S.ready || !S.na.maxtok) { seterr("mmoe_moe_dev_noalloc: set the layers up first (mmoe_set_layer)"); return -1; }
    if (nb < 1 || nb > MMOE_NOALLOC_MAXTOK) { seterr("mmoe_moe_dev_noalloc: nb %d outside 1..%d (the fixed scratch)", nb, MMOE_NOALLOC_MAXTOK); return -1; }
    return moe_dev(S.na, L, d_hn, nb, d_x, order);
}

int mmoe_rmsnorm_dev(const float *d_x, const uint16_t *d_w, int nb, float *d_out) {
    if (ctx_ready()) return -1;
    return launch(MMOE_K_RMSNORM, [&] { kl(k_rmsnorm, nb, 256, 0, d_x, d_w, d_out, nb); });
}

int mmoe_stack_dev(int L0, int nl, float *d_x, int nb, int order) {
    Work &w = S.main;
    if (!w.maxtok || nb < 1 || nb > w.maxtok) { seterr("mmoe_stack_dev: nb %d outside capacity %d", nb, w.maxtok); return -1; }
    for (int L = L0; L < L0 + nl; L++) {
        if (L < 0 || L >= NLMAX || !S.layers[L].tab) { seterr("mmoe_stack_dev: layer %d not set", L); return -1; }
        if (nb <= DEC_MAXTOK && S_dec_enabled) { if (moe_dec(w, L, d_x, 1, nb, d_x, order)) return -1; continue; }
        const uint16_t *pw = S.layers[L].post_ln;
        if (order == MMOE_ORDER_STEP || nb < 512) {   // the chain router forms hn itself (no rmsnorm launch)
            w.norm_x = d_x; w.norm_w = pw;
            int rc = moe_dev(w, L, w.hn, nb, d_x, order);
            w.norm_x = nullptr; w.norm_w = nullptr;
            if (rc) return -1;
            continue;
        }
        if (launch(MMOE_K_RMSNORM, [&] { kl(k_rmsnorm, nb, 256, 0, d_x, pw, w.hn, nb); })) return -1;
        if (moe_dev(w, L, w.hn, nb, d_x, order)) return -1;
    }
    return 0;
}

int mmoe_gfull_stack(int L0, int nl) {
    if (ctx_ready()) return -1;
    if (L0 < 0 || nl < 1 || L0 + nl > 24) { seterr("mmoe_gfull_stack: layers %d..%d outside 0..23", L0, L0 + nl - 1); return -1; }
    if (!GF.ready || !S.gfull_nb) { seterr("mmoe_gfull_stack: gfull_init / gfull_begin first"); return -1; }
    for (int L = L0; L < L0 + nl; L++) {
        if (!S.layers[L].tab) { seterr("mmoe_gfull_stack: layer %d has no experts (mmoe_set_layer)", L); return -1; }
        if (gfull_attn_launch(L, (L % 4) == 3)) return -1;
        if (mmoe_stack_dev(L, 1, S.main.x, S.gfull_nb, MMOE_ORDER_BATCH)) return -1;
    }
    return 0;
}

// Capture mmoe_stack_dev into a HIP graph and replay it (launch-bound decode). Profiling must be off.
int mmoe_stack_graph(int L0, int nl, float *d_x, int nb, int order, int replays) {
    if (S.prof) { seterr("mmoe_stack_graph: profiling is on"); return -1; }
    if (replays < 0) { seterr("mmoe_stack_graph: replays %d", replays); return -1; }
    // the graph holds its arguments: other arguments need a new capture
    if (S.graph && (S.gkey.L0 != L0 || S.gkey.nl != nl || S.gkey.x != d_x || S.gkey.nb != nb || S.gkey.order != order))
        if (mmoe_graph_reset()) return -1;
    if (!S.graph) {
        hipGraph_t g;
        HC(hipStreamBeginCapture(S.st, hipStreamCaptureModeThreadLocal));
        int rc = mmoe_stack_dev(L0, nl, d_x, nb, order);
        hipError_t e = hipStreamEndCapture(S.st, &g);
        if (rc || e != hipSuccess) {
            if (e == hipSuccess) (void)hipGraphDestroy(g);
            if (!rc) seterr("graph capture failed: %s", hipGetErrorString(e));
            return -1;
        }
        HC(hipGraphInstantiate(&S.graph, g, nullptr, nullptr, 0));
        HC(hipGraphDestroy(g));
        S.gkey = {L0, nl, nb, order, d_x};   // setters that change what a capture holds drop the graph
    }
    for (int i = 0; i < replays; i++) HC(hipGraphLaunch(S.graph, S.st));
    return 0;
}
int mmoe_graph_reset(void) {
    if (S.graph) { hipGraphExec_t g = S.graph; S.graph = nullptr; HC(hipGraphExecDestroy(g)); }
    return 0;
}
int mmoe_graph_held(void) { return S.graph != nullptr; }

// Intermediate results of the last main-context call (debug/test access)
int mmoe_read(int what, void *dst, size_t bytes) {
    Work &w = S.main;
    const void *src = nullptr; size_t cap = 0;
    size_t T = w.maxtok, P = w.maxp;
    switch (what) {
        case MMOE_R_LOGITS: src = w.rl; cap = T * MNE * 4; break;
        case MMOE_R_TOP: src = w.top; cap = T * MTOPK * 4; break;
        case MMOE_R_TW: src = w.tw; cap = T * MTOPK * 4; break;
        case MMOE_R_PLAN: src = w.plan; cap = sizeof(Plan); break;
        case MMOE_R_UTOK: src = w.utok; cap = P * 4; break;
        case MMOE_R_UW: src = w.uw; cap = P * 4; break;
        case MMOE_R_TP: src = w.tp; cap = P * 4; break;
        case MMOE_R_SP: src = w.sp; cap = P * 4; break;
        case MMOE_R_QX: src = w.qx; cap = T * MH; break;
        case MMOE_R_QSX: src = w.qsx; cap = T * 4; break;
        case MMOE_R_QSUMX: src = w.qsumx; cap = T * 4; break;
        case MMOE_R_ACT: src = w.act; cap = P * MFF * 4; break;
        case MMOE_R_QA: src = w.qa; cap = P * MFF; break;
        case MMOE_R_QSA: src = w.qsa; cap = P * 4; break;
        case MMOE_R_QSUMA: src = w.qsuma; cap = P * 4; break;
        case MMOE_R_DOWN: src = w.down; cap = P * MH * 4; break;
        case MMOE_R_GU_I32: src = w.dbg_gu; cap = P * 2 * MFF * 4; break;
        case MMOE_R_DN_I32: src = w.dbg_dn; cap = P * MH * 4; break;
        case MMOE_R_X: src = w.x; cap = T * MH * 4; break;
        case MMOE_R_HN: src = w.hn; cap = T * MH * 4; break;
        default: seterr("mmoe_read: unknown item %d", what); return -1;
    }
    if (!src) { seterr("mmoe_read: item %d not allocated (init / debug)", what); return -1; }
    if (bytes > cap) { seterr("mmoe_read: %zu bytes asked, %zu held", bytes, cap); return -1; }
    HC(hipStreamSynchronize(S.st));
    HC(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return 0;
}

int mmoe_gfull_setup(int maxtok) {
    if (mmoe_init(maxtok)) return -1;
    S.gfull = true;
    return 0;
}
// The router stage of gfull_attn (gpu_full.metal rms + rtr): hn = rmsnorm(x, post_ln[L]), rl = router logits
int mmoe_gfull_post_norm(int L, float *rl) {
    if (!S.gfull || !S.gfull_nb || L < 0 || L >= NLMAX || !S.layers[L].router) { seterr("mmoe_gfull_post_norm: not set up (gfull_begin) / layer %d", L); return -1; }
    Work &w = S.main; int nb = S.gfull_nb;
    const uint16_t *pw = S.layers[L].post_ln;
    if (launch(MMOE_K_RMSNORM, [&] { kl(k_rmsnorm, nb, 256, 0, w.x, pw, w.hn, nb); })) return -1;
    // exact chains whatever the router mode: maple.c takes these logits as they are (its own softmax/top-8)
    if (stage_router(w, L, w.hn, nb, MMOE_ORDER_BATCH, true)) return -1;
    if (rl) { HC(hipMemcpyAsync(rl, w.rl, (size_t)nb * MNE * 4, hipMemcpyDeviceToHost, S.st)); HC(hipStreamSynchronize(S.st)); }
    return 0;
}

// ---- device memory helpers (plain pointers; the caller owns them) ----
void *mmoe_dev_alloc(size_t bytes) { if (ctx_ready()) return NULL; void *p = nullptr; HCN(hipMalloc(&p, bytes)); return p; }
int mmoe_dev_free(void *p) { HC(hipFree(p)); return 0; }
int mmoe_h2d(void *d, const void *h, size_t bytes) { if (ctx_ready()) return -1; HC(hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, S.st)); HC(hipStreamSynchronize(S.st)); return 0; }
int mmoe_d2h(void *h, const void *d, size_t bytes) { if (ctx_ready()) return -1; HC(hipStreamSynchronize(S.st)); HC(hipMemcpy(h, d, bytes, hipMemcpyDeviceToHost)); return 0; }
int mmoe_d2d(void *d, const void *s, size_t bytes) { if (ctx_ready()) return -1; HC(hipMemcpyAsync(d, s, bytes, hipMemcpyDeviceToDevice, S.st)); return 0; }
int mmoe_sync(void) { if (ctx_ready()) return -1; HC(hipStreamSynchronize(S.st)); return 0; }
void *mmoe_stream(void) { return ctx_ready() ? NULL : (void *)S.st; }

// ---- timing on the library stream ----
int mmoe_event_record(int slot) { if (ctx_ready() || slot < 0 || slot > 1) return -1; HC(hipEventRecord(S.pe[slot], S.st)); return 0; }
double mmoe_event_elapsed_ms(void) {
    if (hipEventSynchronize(S.pe[1]) != hipSuccess) return -1.0;
    float ms = 0; if (hipEventElapsedTime(&ms, S.pe[0], S.pe[1]) != hipSuccess) return -1.0;
    return ms;
}
// Exhaustive check of the SiLU used by k_act_quant against its IEEE-division form over the bit patterns
// [lo, lo + n). Blocks until done; *nbad = mismatches, *first = smallest mismatching pattern (0xffffffff
// if none).
int mmoe_selftest_silu(uint32_t lo, uint32_t n, unsigned long long *nbad, uint32_t *first) {
    if (ctx_ready()) return -1;
    struct R { unsigned long long bad; uint32_t first; } h = {0, 0xffffffffu};
    R *d = nullptr;
    HC(hipMalloc(&d, sizeof(R)));
    int rc = -1;
    if (hipMemcpy(d, &h, sizeof h, hipMemcpyHostToDevice) == hipSuccess) {
        kl(k_selftest_silu, S.ncu * 16, 256, 0, lo, n, &d->bad, &d->first);
        if (hipGetLastError() == hipSuccess && hipStreamSynchronize(S.st) == hipSuccess &&
            hipMemcpy(&h, d, sizeof h, hipMemcpyDeviceToHost) == hipSuccess) rc = 0;
    }
    (void)hipFree(d);
    if (rc) { seterr("mmoe_selftest_silu: HIP error"); return -1; }
    *nbad = h.bad; *first = h.first;
    return 0;
}

int mmoe_prof(int on) { S.prof = on != 0; return 0; }
int mmoe_prof_reset(void) { memset(S.prof_ms, 0, sizeof S.prof_ms); memset(S.prof_n, 0, sizeof S.prof_n); return 0; }
int mmoe_prof_get(int kid, double *ms_total, long *count) {
    if (kid < 0 || kid >= MMOE_PROF_NKERNELS) return -1;
    *ms_total = S.prof_ms[kid]; *count = S.prof_n[kid]; return 0;
}
int mmoe_device_info(char *name, int len, int *cus, int *clock_khz) {
    if (ctx_ready()) return -1;
    hipDeviceProp_t p; HC(hipGetDeviceProperties(&p, 0));
    if (name && len > 0) { strncpy(name, p.gcnArchName, len - 1); name[len - 1] = 0; }
    if (cus) *cus = p.multiProcessorCount;
    if (clock_khz) *clock_khz = p.clockRate;
    return 0;
}

}  // extern "C"

