/* moe_oracle.h -- CPU restatement of maple-runtime's MoE hot path, for checking only.
 *
 * TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this code, and only as the checker. The product library (libmaplemoe) never links or calls it.
 *
 * Every function follows a function or block of maple.c (the reference's C runtime); the citation is on
 * each declaration. Arithmetic is plain IEEE fp32/fp64 with no fast-math and no FMA contraction
 * (-ffp-contract=off); where maple.c's AVX2 build uses an FMA the oracle calls fmaf() explicitly, and
 * where maple.c's documented -ffast-math build computes something other than its source text says, the
 * oracle follows the compiled behaviour and says so.
 *
 * Pinning (how each function is checked, tests/test_oracle*.py):
 *   mo_pack/mo_unpack      closed form of convert.py:23-40 + brute-force round trip
 *   mo_prep                maple.c built here (oracle/_ref) on 10^5 vectors, bit-exact; x=0 special case
 *   mo_dot_i32             brute force sum (c-1)*q on unpacked codes; maple.c tdot_multi with qs=s=1, bit-exact
 *   mo_router_*            maple.c job_route_multi / bf_row, bit-exact; fp64 dot within 1e-6
 *   mo_exp                 within 2 ulp of libm exp over a sweep, mostly exact (the function the GPU repeats)
 *   mo_topk                maple.c job_topk indices identical; weights within 2 ulp; permutation invariants
 *   mo_group               maple.c group_pairs identical; counting-sort invariants
 *   mo_act                 maple.c's act loop (fast-math expf/rcp) within 4 ulp
 *   mo_rmsnorm             maple.c rmsnorm within 2 ulp
 *   mo_moe_batch/step      maple.c step_batch / step MoE blocks, integer stages bit-exact, fp32 1e-5
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#define MO_H 2048   /* d_model, maple.c:21 */
#define MO_NE 256   /* experts, maple.c:26 */
#define MO_TOPK 8   /* maple.c:27-29 */
#define MO_FF 512   /* expert width, maple.c:30 */

#ifdef __cplusplus
extern "C" {
#endif

/* One expert of one layer, in the packed layout of convert.py:23-33 (codes c in {0,1,2} = w+1, 128-column
 * groups, byte j of a group holds columns j, j+32, j+64, j+96 at bits 0,2,4,6; one fp32 scale per row).
 * maple.c:37 T2 and maple.c:39 Layer.eg/eu/ed. */
typedef struct {
    const uint8_t *gc; const float *gs;   /* gate: 512 rows x 2048 cols -> 512 B/row */
    const uint8_t *uc; const float *us;   /* up:   512 rows x 2048 cols */
    const uint8_t *dc; const float *ds;   /* down: 2048 rows x 512 cols -> 128 B/row */
} mo_expert;

/* convert.py:23-33 pack_ternary for codes already in {0,1,2}: codes[rows][cols] -> packed[rows][cols/4] */
void mo_pack(const uint8_t *codes, int rows, int cols, uint8_t *packed);
/* convert.py:36-40 unpack_ternary (codes only): packed -> codes[rows][cols] in {0,1,2} */
void mo_unpack(const uint8_t *packed, int rows, int cols, uint8_t *codes);

/* maple.c:183-194 prep: per-vector int8 quantisation. Follows the -ffast-math build of maple.c:
 * qs = mx * fl(1/127), inv = 127/mx (source text: qs = mx/127, inv = 1/qs); qs = inv = 1 when mx == 0;
 * q = round-half-even(x * inv). Returns qs; q[n], *qsum = sum of q. */
float mo_prep(const float *x, int n, int8_t *q, int32_t *qsum);

/* maple.c:195-227 tdot / 423-458 tdot_multi, integer part: sum over columns of code * q (codes 0..2,
 * NOT yet minus qsum). The reference's result is (float)(tot - qsum) * qs * s[r]. */
int32_t mo_dot_i32(const uint8_t *row, const int8_t *q, int cols);
float mo_tdot(const uint8_t *row, float s, const int8_t *q, float qs, int32_t qsum, int cols);

/* Router logits, maple.c:853-889 (job_route_small / job_route_multi, nb > 1) summation order: 8 lanes,
 * lane j accumulates columns j, j+8, ... with FMA, then hsum (maple.c:115-119). bias may be NULL
 * (an extension for the skewed-load workload: added after the dot). rl[nb][256]. */
void mo_router_batch(const float *hn, int nb, const uint16_t *w_bf16, const float *bias, float *rl);
/* maple.c:146-157 bf_row order (decode step(), maple.c:609): two 8-lane accumulators with stride 16. */
void mo_router_step(const float *hn, const uint16_t *w_bf16, const float *bias, float *rl);

/* exp used by softmax and SiLU: a fixed fp32 evaluation (range reduction with split ln2, degree-7 Taylor by
 * Horner with FMA, exponent scaling). The HIP kernels evaluate the same sequence of IEEE operations. */
float mo_exp(float x);

/* maple.c:910-923 job_topk (== the inline block maple.c:735-748 and step's 608-617): softmax with
 * max subtraction, sum as 8 interleaved partial sums folded like hsum (an order maple.c's vectorised
 * build may use; the source's order is sequential), 8 rounds of argmax over probabilities (strict >, lowest index wins),
 * picked set to -1, weights / (sum of picked + 1e-20). rl is not modified. top[nb][8], tw[nb][8]. */
void mo_topk(const float *rl, int nb, int32_t *top, float *tw);

/* maple.c:924-938 group_pairs + maple.c:1018-1019 tp: counting sort of (token, expert) pairs by expert.
 * Outputs nu, ue[nu], ustart[nu+1], utok[P], uw[P], tp[nb*8] (pair ids of token b, ascending). Returns P. */
int mo_group(const int32_t *top, const float *tw, int nb, int *nu, int32_t *ue, int32_t *ustart,
             int32_t *utok, float *uw, int32_t *tp);

/* maple.c:825-832 (and 655-662): g = min(G, 7), u = clamp(U, -7, 7), act = g / (1 + exp(-g)) * u */
void mo_act(const float *g, const float *u, float *act, int n);

/* maple.c:398-402 rmsnorm (sum of squares in double) with bf16 weight w (NULL = all ones) */
void mo_rmsnorm(const float *x, const uint16_t *w_bf16, int n, float *out);

/* Intermediate results of one MoE layer, all optional (NULL = not wanted). Sizes for P pairs. */
typedef struct {
    float *rl;          /* [nb][256] router logits */
    int32_t *top;       /* [nb][8] */
    float *tw;          /* [nb][8] */
    int *nu;            /* [1] */
    int32_t *ue;        /* [256] */
    int32_t *ustart;    /* [257] */
    int32_t *utok;      /* [P] */
    float *uw;          /* [P] */
    int32_t *tp;        /* [nb][8] */
    int8_t *qx;         /* [nb][2048] prep of the input */
    float *qsx;         /* [nb] */
    int32_t *qsumx;     /* [nb] */
    int32_t *gu_i32;    /* [P][1024] raw code*q sums, gate rows then up rows */
    float *gate;        /* [P][512] */
    float *up;          /* [P][512] */
    float *act;         /* [P][512] */
    int8_t *qa;         /* [P][512] prep of act */
    float *qsa;         /* [P] */
    int32_t *qsuma;     /* [P] */
    int32_t *dn_i32;    /* [P][2048] raw code*q sums of down */
    float *down;        /* [P][2048] */
} mo_trace;

/* The MoE block of step_batch (maple.c:732-755, 824-834): hn[nb][2048] is the post-norm input; router
 * logits in job_route_* order (+bias), top-8, grouping, gate/up, act + re-quant, down, and the combine
 * x[tok] += uw * down pair by pair in grouped order, as an FMA. x is updated in place.
 * experts[256] give each expert's tensors. If rl_in is not NULL the router is skipped and rl_in used. */
void mo_moe_batch(const float *hn, int nb, const uint16_t *router, const float *bias, const float *rl_in,
                  const mo_expert *experts, float *x, mo_trace *tr);

/* The MoE block of step() (maple.c:605-665), one token: router in bf_row order, top-8, gate/up per slot,
 * act, down per slot, y = sum over slots (FMA, slot order), x += y. */
void mo_moe_step(const float *hn, const uint16_t *router, const float *bias, const mo_expert *experts,
                 float *x, mo_trace *tr);

/* Expert products for a given grouping (what gpre_moe computes, gpu_pre.m:321-385 semantics):
 * y[tok] = sum over that token's pairs in ascending pair order of uw * down (FMA chain from 0).
 * ex[u] gives used expert u's tensors. y is overwritten. */
void mo_experts_grouped(const float *hn, int nb, int nu, const mo_expert *ex, const int32_t *ustart,
                        const int32_t *utok, const float *uw, const int32_t *tp, float *y, mo_trace *tr);

/* ---- attention half of a layer (maple.c step_batch CPU path, 706-724) ----
 * Pinning: mo_rope / mo_f16 bit-exact against maple.c's rope / to_f16 (oracle/_ref); mo_attend and
 * mo_attn_chunk within 1e-6 of maple.c's attend_group / step_batch (its -ffast-math build vectorises the
 * softmax loop with libmvec's expf; this restatement fixes one order, with mo_exp). */
#define MO_NH 16
#define MO_NKV 4
#define MO_HD 128
#define MO_ROT 64
typedef struct { const uint8_t *p; const float *s; int rows, cols; } mo_t2;   /* maple.c:36 T2 */
/* maple.c:403-411 rope on the first 64 dims of a head, pairs (i, i+32), as its FMA-contracted build computes
 * it; cs = the position's 32 (cos, sin) pairs as maple.c:1151-1152 tabulates them ((float)cos / sin of
 * pos * INV_FREQ[i] in double) */
void mo_rope(float *v, const float *cs);
/* maple.c:314-320 to_f16: fp32 -> fp16 with round to nearest even (F16C rounding mode 0); and back (exact) */
void mo_f16(const float *s, uint16_t *d, int n);
float mo_h2f(uint16_t h);
/* maple.c:516-558 attend_group (AVX2 path): the 4 query heads q[4][128] of key/value head kvh attend over
 * positions lo..pos (lo = 0 on global layers, max(0, pos - win) else) of the fp16 cache kc/vc [pos][512]:
 * score = hsum of 8 FMA lanes (lane l: dims l, l+8, ...) times 1/sqrtf(128); p = mo_exp(score - max); the
 * sum over positions in order; out[j][d] = FMA chain over positions of (p * (1/sum)) * v. sc: 4 x (pos+1) */
void mo_attend(const float *q, const uint16_t *kc, const uint16_t *vc, int kvh, int pos, int glob, int win,
               float *out, float *sc);
/* maple.c:706-724 for one sequence: x[nb][2048] of positions pos0 .. pos0+nb-1 -> hn = rmsnorm(x, in_ln),
 * prep, q/k/v = tdot rows (wq 2048, wk 512, wv 512 rows); per token q/k heads rmsnorm (q_norm, k_norm, 128)
 * then rope (local layers, glob == 0); k, v to fp16 into the layer's cache kc/vc [pos][512] and ko[b][1024]
 * (k | v, may be NULL); attention per (token, kv head); prep of the attention output, o = tdot rows of wo;
 * x += o. cs: the rope table [pos][32][2]. att (may be NULL) receives the attention output [nb][2048]. */
void mo_attn_chunk(float *x, int nb, int pos0, int glob, int win, const uint16_t *in_ln, const uint16_t *q_norm,
                   const uint16_t *k_norm, mo_t2 wq, mo_t2 wk, mo_t2 wv, mo_t2 wo, const float *cs,
                   uint16_t *kc, uint16_t *vc, uint16_t *ko, float *att);

#ifdef __cplusplus
}
#endif
#endif
