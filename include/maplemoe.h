/* maplemoe.h -- C ABI of libmaplemoe, the MI355X (gfx950) MoE hot path for maple-runtime.
 *
 * Part 1 declares the entry points maple.c binds when built with -DGPU_HEAD, with maple.c's own signatures
 * (maple.c:247-272, implemented in the reference by gpu_pre.m, gpu_exp.m and gpu_head.m). A maple.c build
 * that links libmaplemoe.so instead of the Objective-C/Metal files runs its expert work on the MI355X.
 * Part 2 declares new mmoe_* entry points that keep the whole MoE layer on the device (router logits,
 * softmax/top-8, grouping, quantisation, expert products, combine), which maple.c would call in place of its
 * CPU routing (maple.c:734-755) and expert block (maple.c:824-834).
 *
 * Conventions, as in the reference: plain C; int returns are 0 on success and -1 on failure, double
 * returns are seconds (or -1.0 on failure); messages go to stderr (and mmoe_last_error()); host arrays
 * stay owned by the caller and are copied; one global context, not thread-safe.
 * Shapes are fixed by the model: H = 2048, 256 experts, top-8, expert width 512 (maple.c:21-30).
 */
#ifndef MAPLEMOE_H
#define MAPLEMOE_H
#include <stddef.h>
#include <stdint.h>

#define MMOE_MAXTOK 2048      /* largest chunk (maple.c:413 BMAX) */
#define MMOE_MAXREG 256       /* regions (gpu_pre.m:21 MAXREG is 64: a model whose layers span 3 shards needs 72) */
#define MMOE_GPUX_MAXTOK 64   /* vectors per gpux call (maple.c:322 MAXSEQ) */
#define MMOE_NOALLOC_MAXTOK 64   /* tokens per mmoe_moe_dev_noalloc call (its fixed scratch) */

/* ============================ Part 1: maple.c:247-272 ============================ */

/* gpu_head.m: output head. Not part of the MoE path: init returns -1, maple.c keeps its CPU head
 * (maple.c:1096, 1100). Replaces gpu_head.m's gpu_head_init / _init_i8 / _run / _run_multi. */
int gpu_head_init(const uint16_t *w, int rows, int cols);
int gpu_head_init_i8(const int8_t *w, const float *scale, int rows, int cols);
void gpu_head_run(const float *x, float *y);
void gpu_head_run_multi(const float *x, int n, float *y);

/* Decode expert cache, replaces gpu_exp.m:155-291 (declared maple.c:251-256).
 * gpux_init: slots per layer in HBM; 0 / -1.
 * gpux_upload: one expert's six tensors (reference layout) into slot `slot` of layer L.
 * gpux_begin: x[2048] (post-norm), n hit experts given by slot -> handle; gpux_end waits and writes
 *   out[n][2048] = each hit expert's down output (unweighted), computed with maple.c's int8 semantics.
 * gpux_begin_multi/_end_multi: nb vectors, nu slot experts with pair runs pstart[nu+1] over tokens ptok[]
 *   -> out[np][2048] per pair. */
int gpux_init(int layers, int slots);
void gpux_upload(int L, int slot, const uint8_t *gc, const float *gs, const uint8_t *uc, const float *us,
                 const uint8_t *dc, const float *ds);
void *gpux_begin(int L, const float *x, int n, const int *slots);
void gpux_end(void *h, float *out, int n);
void *gpux_begin_multi(int L, const float *x, int nb, int nu, const int *slots, const int *pstart, const int *ptok);
void gpux_end_multi(void *h, float *out, int np);

/* Prompt experts, replaces gpu_pre.m:173-385 (declared maple.c:257-262).
 * gpre_init(maxtok, topk): work buffers for chunks of up to maxtok (<= 2048) tokens, topk must be 8; 0 / -1.
 * gpre_region(p, len): page-aligned span of an mmapped shard -> region id (copied once into HBM), or -1.
 * gpre_moe: synchronous. x[nb][2048] post-norm input; nu used experts; loc[nu][12] = (region slot, byte
 *   offset) of gate codes, gate scales, up codes, up scales, down codes, down scales (maple.c:276-277);
 *   regs[4] region ids behind slots 0..3; next: ignored (weights are resident); ustart[nu+1], ptok[P], pw[P]
 *   the grouping of maple.c:924-938; tp[nb][8] pair ids per token. y[nb][2048] = sum of pw * down over the
 *   token's pairs (overwritten, not added). Returns device seconds or -1.0.
 * gpre_stage: no-op (weights are already in HBM), returns 0.
 * gpre_blit_seconds: seconds spent copying regions into HBM. */
int gpre_init(int maxtok, int topk);
int gpre_region(const void *p, size_t len);
double gpre_moe(const float *x, int nb, int nu, const uint32_t *loc, const int *regs, const int *next,
                const int *ustart, const int *ptok, const float *pw, const int *tp, float *y);
int gpre_stage(size_t bytes);
/* Dense q/k/v/o projections, replaces gpu_pre.m:200-256 (declared maple.c:261-263, called maple.c:1136-1141,
 * 692, 723). gpre_dense_add(g, codes, scales, rows, cols) stages one ternary matrix of group g (2L: q, k, v;
 * 2L+1: o), rows a multiple of 256, cols 2048, at most 3 per group; its outputs follow the group's earlier
 * ones. gpre_dense_done(maxtok) copies them to HBM (0, or -1 when a matrix was malformed or the context is
 * missing: maple.c then keeps the projections on the CPU). gpre_dense(g, x, nb, y): synchronous,
 * y[nb][rows of g] = the matrices times x[nb][2048] (host arrays), with maple.c's int8 arithmetic (prep,
 * tdot_multi): equal to its CPU projections bit for bit. Returns device seconds, or -1. */
void gpre_dense_add(int g, const uint8_t *codes, const float *scales, int rows, int cols);
int gpre_dense_done(int maxtok);
double gpre_dense(int g, const float *x, int nb, float *y);
double gpre_blit_seconds(void);
/* Drops the dense projections from HBM so gpre_dense_add can stage a new set (no counterpart in maple.c,
 * which loads them once per run; for callers and tests that load several models in one process). */
int mmoe_dense_reset(void);

/* Whole layers on the card, replaces gpu_pre.m:387-594 (declared maple.c:265-272, driven by maple.c:1001-1031,
 * set up at maple.c:1140-1154). gfull_init needs the dense projections (gpre_dense_add per layer: group 2L = q,
 * k, v, group 2L+1 = o; gpre_dense_done) and takes norms[24][4352] (in_ln | post_ln | q_norm | k_norm, fp32
 * holding bf16 values), the 24 routers (bf16 [256][2048] each) and the rope table cs[ctx][32][2]; it keeps a
 * per-layer fp16 key/value cache of ctx positions in HBM. gfull_begin loads a chunk of nb hidden vectors at
 * positions pos0..; gfull_attn(L, glob) runs the attention half of layer L (maple.c:706-724: rmsnorm, q/k/v,
 * head norms, rope unless glob, cache, causal attention over the window win (all positions when glob), o,
 * x += o), then post-norm and the router: rl gets nb x 256 logits; synchronous, returns device seconds (-1.0 on
 * error). gfull_moe adds the experts of the host's grouping into x (asynchronous). gfull_read waits, copies x
 * back and sets *ko to the chunk's fp16 k | v of every layer ([24][gfull_maxtok()][1024]; rows 0..nb-1 of each
 * layer are the chunk's, the rest are not refreshed). Results: k, v, x
 * after attention and the logits equal maple.c's CPU statements bit for bit. */
int gfull_init(int ctx, int maxtok, int win, const float *norms, const uint16_t *router, const float *cs);
void gfull_begin(const float *x, int nb, int pos0);
double gfull_attn(int L, int glob, float *rl);
void gfull_moe(int nu, const uint32_t *loc, const int *regs, const int *ustart, const int *ptok, const float *pw, const int *tp);
void gfull_read(float *x, const uint16_t **ko);
void gfull_write_x(const float *x);
int gfull_maxtok(void);
void gfull_report(void);

/* ============================ Part 2: the layer on the device ============================ */

/* Summation orders (maple.c has two router and two combine orders) */
#define MMOE_ORDER_BATCH 0    /* step_batch: router maple.c:853-889, combine maple.c:834 */
#define MMOE_ORDER_STEP 1     /* step (one token): router bf_row maple.c:146-157, combine maple.c:664 */

/* Combine modes (flag bits; used internally and by tests): 1 start from x, 2 slot order, 4 add at end */
#define MMOE_COMBINE_OVERWRITE 0
#define MMOE_COMBINE_BATCH 1
#define MMOE_COMBINE_ADD 4
#define MMOE_COMBINE_STEP 6

/* mmoe_init(maxtok): context and work buffers for up to maxtok (<= 2048) tokens. Same buffers as gpre_init. */
int mmoe_init(int maxtok);
/* Layer L's experts (all 256) through maple.c's location table GLOC[L] (loc[256][12], maple.c:276) and
 * region ids GREG[L] (regs[4]); router[256][2048] bf16 (maple.c:38 Layer.router); post_ln[2048] bf16 or
 * NULL (used by the stacked path only). The router is copied to HBM. */
int mmoe_set_layer(int L, const uint32_t *loc, const int *regs, const uint16_t *router, const uint16_t *post_ln);
/* Optional per-expert logit bias[256] added after the router dot (no counterpart in maple.c: it skews
 * expert loads for the imbalance workload); NULL removes it. */
int mmoe_set_bias(int L, const float *bias);
/* The MoE block of step_batch (order BATCH, maple.c:733-834) or step (order STEP, maple.c:605-665) on host
 * arrays: hn[nb][2048] post-norm input; x[nb][2048] updated in place (x += MoE). Synchronous. */
int mmoe_moe(int L, const float *hn, int nb, float *x, int order);
/* The same on device pointers, queued on the library stream (mmoe_stream) without waiting. */
int mmoe_moe_dev(int L, const float *d_hn, int nb, float *d_x, int order);
/* No counterpart in the reference. For callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): mmoe_moe_dev for nb <= MMOE_NOALLOC_MAXTOK
 * tokens whose work buffers all live in a fixed 7 MiB static device array of the library (set up when the
 * library context is, by mmoe_init / mmoe_set_layer; held until the process ends). The call allocates and
 * frees nothing; larger nb is refused with -1. Every call on the GPU shares that scratch: calls that overlap
 * on one GPU (from several host threads) race. Results equal mmoe_moe_dev's. */
int mmoe_moe_dev_noalloc(int L, const float *d_hn, int nb, float *d_x, int order);
/* Routing only, in place of maple.c's job_topk + group_pairs (maple.c:910-938) and the tp table its callers
 * build (maple.c:762, 1019), for a caller that keeps its own gpre_moe / gfull_moe (maple.c:763, 1021): rl[nb][256]
 * router logits (host), or NULL for the logits the last router call left on the device (gfull_attn,
 * mmoe_gfull_post_norm, and mmoe_moe* when every logit was computed exactly: below 512 tokens or with
 * mmoe_set_router_mode(1)); NULL is refused with -1 unless that call covered exactly nb tokens.
 * -> maple.c's TOPB/TWB (top[nb][8], tw[nb][8]: softmax, the 8 largest p in pick order, renormalised), the pairs grouped by expert (ue[nu] used experts ascending, ustart[nu+1], utok[nb*8] and
 * uw[nb*8] = UTOK/UW) and tp[nb][8] (each token's pair ids, ascending). Any output may be NULL. Synchronous;
 * returns nu, or -1 (mmoe_last_error). nb <= mmoe_init's maxtok. */
int mmoe_route(const float *rl, int nb, int *top, float *tw, int *ue, int *ustart, int *utok, float *uw, int *tp);
/* maple.c:398-402 rmsnorm on device pointers; d_w bf16[2048] or NULL (unit weight). */
int mmoe_rmsnorm_dev(const float *d_x, const uint16_t *d_w, int nb, float *d_out);
/* nl stacked MoE layers: for L in L0..L0+nl-1: hn = rmsnorm(x, post_ln[L]); x += MoE_L(hn). */
int mmoe_stack_dev(int L0, int nl, float *d_x, int nb, int order);
/* The same captured once into a HIP graph, then replayed `replays` times; mmoe_graph_reset drops it. A call
 * with other arguments captures anew. The graph holds the kernels and device buffers it was captured with, so
 * every setter that changes them (mmoe_set_layer, mmoe_set_bias, mmoe_set_debug, mmoe_set_decode_path,
 * mmoe_set_expert_path, mmoe_set_router_mode, gfull_init) drops it first. Profiling must be off. mmoe_graph_held: 1 while a
 * captured graph is kept, else 0. */
int mmoe_stack_graph(int L0, int nl, float *d_x, int nb, int order, int replays);
int mmoe_graph_reset(void);
int mmoe_graph_held(void);
/* Router stage of gfull_attn (gpu_full.metal:12-27 rms, 169-209 rtr) on the gfull hidden state:
 * hn = rmsnorm(x, post_ln[L]), rl[nb][256] = router logits (copied to the host if rl != NULL). */
int mmoe_gfull_setup(int maxtok);
int mmoe_gfull_post_norm(int L, float *rl);
/* Layers L0 .. L0+nl-1 of the gfull chunk entirely on the device, asynchronous (no counterpart in maple.c,
 * whose step_batch_card, maple.c:1005-1022, brings the logits to the host for top-8 and grouping between the
 * halves): per layer the attention half of gfull_attn (glob = (L % 4) == 3, maple.c:1008) and then the MoE
 * block of mmoe_stack_dev on the hidden state (post-norm, router, top-8, grouping, experts, combine). Needs
 * gfull_init, gfull_begin and mmoe_set_layer for every layer (expert tables); gfull_read waits for it. */
int mmoe_gfull_stack(int L0, int nl);

/* Intermediate results of the last call on the main context (tests and checks, like GPRE_CHECK) */
#define MMOE_R_LOGITS 0   /* float [nb][256] */
#define MMOE_R_TOP 1      /* int [nb][8] */
#define MMOE_R_TW 2       /* float [nb][8] */
#define MMOE_R_PLAN 3     /* int nu, np, ntile, tn, ue[256], ustart[257], tstart[257] */
#define MMOE_R_UTOK 4     /* int [P] */
#define MMOE_R_UW 5       /* float [P] */
#define MMOE_R_TP 6       /* int [nb][8] pair ids, ascending */
#define MMOE_R_SP 7       /* int [nb][8] pair id of each slot */
#define MMOE_R_QX 8       /* int8 [nb][2048] in mfma order (see kernels.h) */
#define MMOE_R_QSX 9      /* float [nb] */
#define MMOE_R_QSUMX 10   /* int [nb] */
#define MMOE_R_ACT 11     /* float [P][512] */
#define MMOE_R_QA 12      /* int8 [P][512] in mfma order */
#define MMOE_R_QSA 13     /* float [P] */
#define MMOE_R_QSUMA 14   /* int [P] */
#define MMOE_R_DOWN 15    /* float [P][2048] */
#define MMOE_R_GU_I32 16  /* int [P][1024] gate then up code*q sums (needs mmoe_set_debug(1)) */
#define MMOE_R_DN_I32 17  /* int [P][2048] down code*q sums (needs mmoe_set_debug(1)) */
#define MMOE_R_X 18       /* float [nb][2048] work hidden state */
#define MMOE_R_HN 19      /* float [nb][2048] work input */
int mmoe_read(int what, void *dst, size_t bytes);
int mmoe_set_debug(int on);
/* Batches of <= 8 tokens use three fused decode kernels (default on); off = the grouped-GEMM path. */
int mmoe_set_decode_path(int on);
/* Batches whose pairs are tiled by 16 (fewer than 2048 pairs, above the decode path): 1 (default) = one fused
 * kernel per tile (gate/up, SiLU*up, act quantisation and down; the act never leaves the chip), 0 = the three
 * separate kernels. Both give identical results. */
int mmoe_set_expert_path(int fused);
/* Router of batches of >= 512 tokens in batch order: 0 (default) = bf16 MFMA logits on the input split into
 * three exact bf16 parts, with every expert that a rounding bound cannot exclude from a token's top 8 recomputed
 * in maple.c's exact chain order (top-8 indices and their logits stay maple.c's; the other logits, and through
 * the softmax sum the weights, differ by about 1e-7); 1 = exact fp32 FMA chains for every logit. gfull_attn's
 * logits, which maple.c consumes itself, always use the exact chains. */
int mmoe_set_router_mode(int exact);
const char *mmoe_last_error(void);

/* Device memory on the library's device, and the library stream */
void *mmoe_dev_alloc(size_t bytes);
int mmoe_dev_free(void *p);
int mmoe_h2d(void *d, const void *h, size_t bytes);
int mmoe_d2h(void *h, const void *d, size_t bytes);
int mmoe_d2d(void *d, const void *s, size_t bytes);
int mmoe_sync(void);
void *mmoe_stream(void);

/* Timing with HIP events on the library stream: record slot 0 and 1, elapsed ms between them.
 * mmoe_prof(1) brackets every kernel launch with events and sums the time per kernel id (serialises). */
#define MMOE_K_RMSNORM 0
#define MMOE_K_ROUTER 1
#define MMOE_K_TOPK 2
#define MMOE_K_GROUP 3
#define MMOE_K_QUANT 4
#define MMOE_K_GATEUP 5
#define MMOE_K_QUANT_ACT 6
#define MMOE_K_DOWN 7
#define MMOE_K_COMBINE 8
#define MMOE_K_DENSE 9          /* k_dense: q/k/v and o projections */
#define MMOE_K_QKN 10           /* k_qkn: head norms, rope, fp16 cache */
#define MMOE_K_ATT_SCORES 11
#define MMOE_K_ATT_SOFTMAX 12
#define MMOE_K_ATT_PV 13
#define MMOE_PROF_NKERNELS 14
int mmoe_event_record(int slot);
double mmoe_event_elapsed_ms(void);
int mmoe_prof(int on);
int mmoe_prof_reset(void);
int mmoe_prof_get(int kid, double *ms_total, long *count);
int mmoe_device_info(char *name, int len, int *cus, int *clock_khz);

/* ---- maple.c's checkpoint directory (csrc/ckpt.c) ----
 * shard-00001.bin .. shard-00009.bin, mapped read-only, and layout.bin (26-byte packed records <kind u8, shard u8,
 * data offset u64, scale offset u64, rows u32, cols u32> in layout.py's order), as maple.c:61-83 load().
 * mmoe_ckpt_open checks the record kinds (maple.c:69-80) and, for the MoE tensors, shapes, bounds and 16-byte
 * alignment (maple.c:1116-1117); 0 or -1 (mmoe_ckpt_error says why). */
int mmoe_ckpt_open(const char *dir);
void mmoe_ckpt_close(void);
const char *mmoe_ckpt_error(void);
/* Layer L's device regions and location table as maple.c:1106-1131 computes them: per shard (ascending), the
 * page-aligned span of the layer's 256 x 6 expert tensors; shard[i], lo[i], len[i] for i < return value (<= 4);
 * loc (may be NULL) receives GLOC[L] (256 x 12: region slot, byte offset for gate codes, gate scales, up codes,
 * up scales, down codes, down scales). No GPU work. */
int mmoe_ckpt_layer_plan(int L, int shard[4], uint64_t lo[4], uint64_t len[4], uint32_t *loc);
/* Layer L's bf16 tensor `which` (0 input_layernorm, 1 post_attention_layernorm, 2 q_norm, 3 k_norm, 4 router)
 * inside the mapping, or NULL. */
const uint16_t *mmoe_ckpt_bf16(int L, int which);
/* Layers L0 .. L0+nl-1: gpre_region for each planned span, then mmoe_set_layer with the location table, the
 * router and the post-attention norm (maple.c:1106-1131 followed by the mmoe_set_layer call of INTEGRATION).
 * Needs mmoe_init (or gpre_init) first. */
int mmoe_ckpt_load(int L0, int nl);
/* Diagnostic, no counterpart in the reference: checks the branch-light SiLU of the activation kernel
 * against g / (1 + exp(-g)) with IEEE division, bit for bit, over the fp32 bit patterns [lo, lo + n).
 * *nbad = number of mismatches, *first = smallest mismatching pattern (0xffffffff if none). */
int mmoe_selftest_silu(uint32_t lo, uint32_t n, unsigned long long *nbad, uint32_t *first);

#endif
