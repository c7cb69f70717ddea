/* ref_harness.c -- exposes maple.c's own MoE functions (compiled from /root/reference/maple.c as it lies)
 * through a small C API, so tests can check the oracle and the HIP path against the reference itself.
 *
 * TEST INFRASTRUCTURE. Built by oracle/Makefile into oracle/_ref/libmaple_ref.so with maple.c's documented
 * flags (-O3 -ffast-math) for the AVX2 ISA it targets (-mavx2 -mfma -mf16c). No reference source is copied:
 * maple.c is included by path; its `main` is renamed so the file links as a library.
 *
 * What runs is maple.c's code: prep, tdot_multi, bf_row, job_route_small/multi, job_topk, group_pairs,
 * job_gateup/job_down, jobB_gateup/jobB_down and run(). Three statements that maple.c writes inline inside
 * step()/step_batch() are restated here because they are not functions of their own: the SiLU*up loop
 * (maple.c:825-830 / 655-660), the batched combine (maple.c:834) and the decode combine (maple.c:664).
 * They are compiled with the same flags, in the same translation unit.
 */
#define main maple_reference_main_unused
#include "maple.c"
#undef main

static int REF_WORKERS;

/* A maple.c executable linked with -ffast-math starts with flush-to-zero and denormals-are-zero set
 * (crtfastmath). This library is linked without it so that it does not change the floating-point mode of
 * the process that loads it; instead every ref_* entry point runs maple.c's code under FTZ/DAZ and restores
 * the caller's mode on return. Worker threads inherit the mode from ref_set_threads. */
#include <xmmintrin.h>
#define FAST_ENTER unsigned int csr_saved_ = _mm_getcsr(); _mm_setcsr(csr_saved_ | 0x8040u)
#define FAST_LEAVE _mm_setcsr(csr_saved_)

/* maple.c starts NT = 4 (maple.c:85) and main() spawns the workers; without main, run() must not wait for
 * workers that do not exist, so the library starts single-threaded until ref_set_threads. */
__attribute__((constructor)) static void ref_single_thread(void) { NT = 1; }

/* maple.c:1095 starts NT-1 spinning workers; the caller thread takes the first slice of each job */
static int ref_set_threads_impl(int nt) {
    if (nt < 1) nt = 1;
    if (REF_WORKERS) return NT;  /* workers are started once, like maple.c's main */
    NT = nt;
    pthread_t th;
    for (int i = 1; i < NT; i++) pthread_create(&th, NULL, worker, (void *)(intptr_t)i);
    REF_WORKERS = NT > 1;
    return NT;
}
int ref_set_threads(int nt) {
    FAST_ENTER;
    int r_ = ref_set_threads_impl(nt);
    FAST_LEAVE;
    return r_;
}

/* Point layer L's router and experts at caller memory (maple.c:61-81 does this from layout.bin) */
void ref_set_router(int L, const uint16_t *w) {
    FAST_ENTER;
    LY[L].router.p = w; LY[L].router.rows = NE; LY[L].router.cols = H;
    FAST_LEAVE;
}
void ref_set_expert(int L, int e, const uint8_t *gc, const float *gs, const uint8_t *uc, const float *us,
                    const uint8_t *dc, const float *ds) {
    FAST_ENTER;
    Layer *l = &LY[L];
    l->eg[e] = (T2){gc, gs, FF, H};
    l->eu[e] = (T2){uc, us, FF, H};
    l->ed[e] = (T2){dc, ds, H, FF};
    FAST_LEAVE;
}

/* maple.c:183-194 */
static float ref_prep_impl(const float *x, int n, int8_t *q, int32_t *qsum) {
    static Vin v;
    prep(&v, x, n);
    memcpy(q, v.q, (size_t)n);
    *qsum = v.qsum;
    return v.qs;
}
float ref_prep(const float *x, int n, int8_t *q, int32_t *qsum) {
    FAST_ENTER;
    float r_ = ref_prep_impl(x, n, q, qsum);
    FAST_LEAVE;
    return r_;
}

/* maple.c:423-458 tdot_multi with qs = 1, qsum = 0 and unit row scale: the fp32 result is the exact
 * integer sum of code*q (|sum| < 2^24). rows x cols codes, nv int8 vectors (each cols long). */
void ref_dot_i32(const uint8_t *codes, int rows, int cols, const int8_t *q, int nv, int32_t *out) {
    FAST_ENTER;
    static Vin *vs[BMAX]; static Vin pool[64];
    float *ones = malloc(sizeof(float) * rows), *res = malloc(sizeof(float) * (size_t)rows * nv);
    for (int r = 0; r < rows; r++) ones[r] = 1.0f;
    T2 w = {codes, ones, rows, cols};
    for (int i0 = 0; i0 < nv; i0 += 64) {
        int n = nv - i0 < 64 ? nv - i0 : 64;
        for (int i = 0; i < n; i++) { memcpy(pool[i].q, q + (size_t)(i0 + i) * cols, (size_t)cols); pool[i].qs = 1.0f; pool[i].qsum = 0; vs[i] = &pool[i]; }
        for (int r = 0; r < rows; r++) tdot_multi(&w, r, vs, n, res + (size_t)r * nv + i0, 1);
    }
    for (int r = 0; r < rows; r++) for (int i = 0; i < nv; i++) out[(size_t)i * rows + r] = (int32_t)res[(size_t)r * nv + i];
    free(ones); free(res);
    FAST_LEAVE;
}

/* maple.c:734: router logits of nb tokens of layer L the way step_batch does (<= 32: route_small) */
void ref_route_batch(int L, const float *hn, int nb, float *rl) {
    FAST_ENTER;
    BN = nb; BL = &LY[L];
    memcpy(HNB, hn, sizeof(float) * (size_t)nb * H);
    if (nb <= 32) run(job_route_small, NULL, NE); else run(job_route_multi, NULL, (nb + 7) / 8);
    memcpy(rl, RLG, sizeof(float) * (size_t)nb * NE);
    FAST_LEAVE;
}
/* maple.c:609: decode router, bf_row per expert */
void ref_route_step(int L, const float *hn, float *rl) {
    FAST_ENTER;
    for (int e = 0; e < NE; e++) rl[e] = bf_row(&LY[L].router, e, hn);
    FAST_LEAVE;
}
/* maple.c:910-923 */
void ref_topk(const float *rl, int nb, int32_t *top, float *tw) {
    FAST_ENTER;
    memcpy(RLG, rl, sizeof(float) * (size_t)nb * NE);
    run(job_topk, NULL, nb);
    memcpy(top, TOPB, sizeof(int) * (size_t)nb * TOPK);
    memcpy(tw, TWB, sizeof(float) * (size_t)nb * TOPK);
    FAST_LEAVE;
}
/* maple.c:924-938 + 1018-1019, on TOPB/TWB given by the caller */
static int ref_group_impl(const int32_t *top, const float *tw, int nb, int *nu, int32_t *ue, int32_t *ustart,
              int32_t *utok, float *uw, int32_t *tp) {
    memcpy(TOPB, top, sizeof(int) * (size_t)nb * TOPK);
    memcpy(TWB, tw, sizeof(float) * (size_t)nb * TOPK);
    int pos[BMAX]; for (int b = 0; b < nb; b++) pos[b] = b;
    int na = group_pairs(nb, pos, 0);
    *nu = NU;
    memcpy(ue, UE, sizeof(int) * NU); memcpy(ustart, USTART, sizeof(int) * (NU + 1));
    memcpy(utok, UTOK, sizeof(int) * na); memcpy(uw, UW, sizeof(float) * na);
    int fl[BMAX]; memset(fl, 0, sizeof(int) * nb);
    for (int a = 0; a < na; a++) { int b = UTOK[a]; tp[b * TOPK + fl[b]++] = a; }
    return na;
}
int ref_group(const int32_t *top, const float *tw, int nb, int *nu, int32_t *ue, int32_t *ustart,
              int32_t *utok, float *uw, int32_t *tp) {
    FAST_ENTER;
    int r_ = ref_group_impl(top, tw, nb, nu, ue, ustart, utok, uw, tp);
    FAST_LEAVE;
    return r_;
}
/* maple.c:398-402 */
void ref_rmsnorm(const float *x, const uint16_t *w, int n, float *out) {
    FAST_ENTER;
    BF bw = {w, 1, n};
    rmsnorm(out, x, &bw, n);
    FAST_LEAVE;
}
/* the act loop maple.c:825-830 */
void ref_act(const float *G, const float *U, float *act, int n) {
    FAST_ENTER;
    for (int k = 0; k < n; k++) {
        float g = G[k] < 7.0f ? G[k] : 7.0f, u = U[k];
        u = u < -7.0f ? -7.0f : (u > 7.0f ? 7.0f : u);
        act[k] = g / (1.0f + expf(-g)) * u;
    }
    FAST_LEAVE;
}

/* Optional per-expert logit bias for ref_moe_batch (NULL: none). Not a maple.c feature: the Zipf-skewed
 * workload adds it to each logit after the router dot, as the oracle's mo_router_batch
 * and the library do (one fp32 addition). */
static const float *REF_BIAS;
void ref_set_bias(const float *bias) { REF_BIAS = bias; }

/* The MoE block of step_batch (maple.c:733-755, 824-834) for layer L: hn[nb][2048] post-norm input,
 * x[nb][2048] updated in place. Optional outputs as in the oracle's mo_trace (NULL = skip). */
void ref_moe_batch(int L, const float *hn, int nb, float *x, float *rl_out, int32_t *top_out, float *tw_out,
                   int *nu_out, int32_t *ue_out, int32_t *ustart_out, int32_t *utok_out, float *uw_out,
                   float *gate_out, float *up_out, float *act_out, int8_t *qa_out, float *qsa_out, float *down_out) {
    FAST_ENTER;
    BN = nb; BL = &LY[L];
    memcpy(HNB, hn, sizeof(float) * (size_t)nb * H);
    for (int b = 0; b < nb; b++) prep(&VHB[b], HNB[b], H);
    if (nb <= 32) run(job_route_small, NULL, NE); else run(job_route_multi, NULL, (nb + 7) / 8);
    if (REF_BIAS) for (int b = 0; b < nb; b++) for (int e = 0; e < NE; e++) RLG[b][e] = RLG[b][e] + REF_BIAS[e];
    if (rl_out) memcpy(rl_out, RLG, sizeof(float) * (size_t)nb * NE);
    run(job_topk, NULL, nb);
    if (top_out) memcpy(top_out, TOPB, sizeof(int) * (size_t)nb * TOPK);
    if (tw_out) memcpy(tw_out, TWB, sizeof(float) * (size_t)nb * TOPK);
    int pos[BMAX]; for (int b = 0; b < nb; b++) pos[b] = b;
    int na = group_pairs(nb, pos, L);
    if (nu_out) *nu_out = NU;
    if (ue_out) memcpy(ue_out, UE, sizeof(int) * NU);
    if (ustart_out) memcpy(ustart_out, USTART, sizeof(int) * (NU + 1));
    if (utok_out) memcpy(utok_out, UTOK, sizeof(int) * na);
    if (uw_out) memcpy(uw_out, UW, sizeof(float) * na);
    run(jobB_gateup, NULL, NU * 2 * FF);
    for (int a = 0; a < na; a++) {
        ref_act(GATEB[a], UPB[a], ACTB[a], FF);
        prep(&VAB[a], ACTB[a], FF);
    }
    run(jobB_down, NULL, NU * H);
    for (int a = 0; a < na; a++) { float *xb = x + (size_t)UTOK[a] * H; for (int i = 0; i < H; i++) xb[i] += UW[a] * DOWNB[a][i]; }
    if (gate_out) memcpy(gate_out, GATEB, sizeof(float) * (size_t)na * FF);
    if (up_out) memcpy(up_out, UPB, sizeof(float) * (size_t)na * FF);
    if (act_out) memcpy(act_out, ACTB, sizeof(float) * (size_t)na * FF);
    if (qa_out) for (int a = 0; a < na; a++) memcpy(qa_out + (size_t)a * FF, VAB[a].q, FF);
    if (qsa_out) for (int a = 0; a < na; a++) qsa_out[a] = VAB[a].qs;
    if (down_out) memcpy(down_out, DOWNB, sizeof(float) * (size_t)na * H);
    FAST_LEAVE;
}

/* The MoE block of step() (maple.c:606-665, no expert cache) for layer L: one token. */
void ref_moe_step(int L, const float *hn, float *x, float *rl_out, int32_t *top_out, float *tw_out,
                  float *act_out, float *down_out) {
    FAST_ENTER;
    const Layer *l = &LY[L];
    memcpy(HN, hn, sizeof(float) * H);
    prep(&V_H, HN, H);
    for (int e = 0; e < NE; e++) RLG[0][e] = bf_row(&l->router, e, HN);
    if (rl_out) memcpy(rl_out, RLG[0], sizeof(float) * NE);
    run(job_topk, NULL, 1);
    for (int s = 0; s < TOPK; s++) { TOPI[s] = TOPB[0][s]; TOPW[s] = TWB[0][s]; }
    if (top_out) memcpy(top_out, TOPI, sizeof TOPI);
    if (tw_out) memcpy(tw_out, TOPW, sizeof TOPW);
    run(job_gateup, (void *)l, TOPK * 2 * FF);
    for (int s = 0; s < TOPK; s++) { ref_act(GATE[s], UP[s], ACT[s], FF); prep(&V_A[s], ACT[s], FF); }
    run(job_down, (void *)l, TOPK * H);
    for (int i = 0; i < H; i++) { float y = 0; for (int s = 0; s < TOPK; s++) y += TOPW[s] * DOWN[s][i]; x[i] += y; }
    if (act_out) memcpy(act_out, ACT, sizeof(float) * TOPK * FF);
    if (down_out) memcpy(down_out, DOWN, sizeof(float) * TOPK * H);
    FAST_LEAVE;
}

/* Wall-clock helper for the CPU baseline (maple.c:47) */
double ref_now(void) { return now(); }

/* ---- attention half (maple.c:706-724), for pinning the oracle's mo_rope / mo_f16 / mo_attn_chunk ----
 * maple.c's main() sets INV_FREQ (maple.c:1085) and allocates the fp16 caches and the score rows
 * (maple.c:1088-1090); these entry points do the same once, with a context of REF_CTX positions. */
#define REF_CTX 1024
static int REF_ATT_READY;
static void ref_att_init(void) {
    if (REF_ATT_READY) return;
    for (int i = 0; i < ROT / 2; i++) INV_FREQ[i] = 1.0 / pow(10000.0, (2.0 * i) / ROT);   /* maple.c:1085 */
    CTX = REF_CTX;
    KC = calloc((size_t)NL * CTX * NKV * HD, sizeof(uint16_t));
    VC = calloc((size_t)NL * CTX * NKV * HD, sizeof(uint16_t));
    SCR = malloc(sizeof(float) * (size_t)BMAX * NH * CTX);
    REF_ATT_READY = 1;
}
int ref_ctx(void) { return REF_CTX; }
/* maple.c:403-411 */
void ref_rope(float *v, int pos) { FAST_ENTER; ref_att_init(); rope(v, pos); FAST_LEAVE; }
/* maple.c:314-320 */
void ref_f16(const float *s, uint16_t *d, int n) { FAST_ENTER; to_f16(d, s, n); FAST_LEAVE; }
/* maple.c:1151-1152: the (cos, sin) table gfull_init receives, npos positions x 32 pairs */
void ref_cs(int npos, float *cs) {
    FAST_ENTER; ref_att_init();
    for (int pos = 0; pos < npos; pos++) for (int i = 0; i < ROT / 2; i++) {
        double f = pos * INV_FREQ[i]; cs[(pos * 32 + i) * 2] = (float)cos(f); cs[(pos * 32 + i) * 2 + 1] = (float)sin(f);
    }
    FAST_LEAVE;
}
/* Layer L's attention tensors (maple.c:71-77 does this from layout.bin) */
void ref_set_attn(int L, const uint16_t *in_ln, const uint16_t *q_norm, const uint16_t *k_norm,
                  const uint8_t *qc, const float *qs, const uint8_t *kc, const float *ks, const uint8_t *vc, const float *vs,
                  const uint8_t *oc, const float *os) {
    FAST_ENTER;
    Layer *l = &LY[L];
    l->in_ln = (BF){in_ln, 1, H}; l->q_norm = (BF){q_norm, 1, HD}; l->k_norm = (BF){k_norm, 1, HD};
    l->q = (T2){qc, qs, NH * HD, H}; l->k = (T2){kc, ks, NKV * HD, H}; l->v = (T2){vc, vs, NKV * HD, H};
    l->o = (T2){oc, os, H, NH * HD};
    FAST_LEAVE;
}
/* Layer L's cache of sequence 0 (maple.c KC/VC at KOFF(0, L, .)): set positions 0..npos-1, or read them */
void ref_cache(int L, int npos, uint16_t *kc, uint16_t *vc, int set) {
    FAST_ENTER; ref_att_init();
    size_t n = (size_t)npos * NKV * HD * 2;
    if (set) { memcpy(KC + KOFF(0, L, 0), kc, n); memcpy(VC + KOFF(0, L, 0), vc, n); }
    else { memcpy(kc, KC + KOFF(0, L, 0), n); memcpy(vc, VC + KOFF(0, L, 0), n); }
    FAST_LEAVE;
}
/* The attention half of step_batch (maple.c:706-724, the CPU path) for nb tokens of sequence 0 at positions
 * pos0..: statements restated, every function maple.c's own. x[nb][2048] is updated in place; att (may be
 * NULL) receives maple.c's attention output ATTB. */
void ref_attn_chunk(int L, int glob, float *x, int nb, int pos0, float *att) {
    FAST_ENTER; ref_att_init();
    BN = nb; BL = &LY[L];
    for (int b = 0; b < nb; b++) memcpy(XB[b], x + (size_t)b * H, H * sizeof(float));
    for (int b = 0; b < nb; b++) { rmsnorm(HNB[b], XB[b], &BL->in_ln, H); prep(&VHB[b], HNB[b], H); }
    run(jobB_qkv, NULL, NH * HD + 2 * NKV * HD);
    for (int b = 0; b < nb; b++) {
        int pos = pos0 + b;
        for (int h = 0; h < NH; h++) { rmsnorm(QB[b] + h * HD, QB[b] + h * HD, &BL->q_norm, HD); if (!glob) rope(QB[b] + h * HD, pos); }
        for (int h = 0; h < NKV; h++) { rmsnorm(KB_[b] + h * HD, KB_[b] + h * HD, &BL->k_norm, HD); if (!glob) rope(KB_[b] + h * HD, pos); }
        to_f16(KC + KOFF(0, L, pos), KB_[b], NKV * HD);
        to_f16(VC + KOFF(0, L, pos), VB_[b], NKV * HD);
        ASEQ[b] = 0; APOS[b] = pos;
    }
    AL = L; AGLOB = glob;
    run(jobB_att, NULL, nb * NKV);
    for (int b = 0; b < nb; b++) prep(&VATTB[b], ATTB[b], H);
    run(jobB_o, NULL, H);
    for (int b = 0; b < nb; b++) for (int i = 0; i < H; i++) XB[b][i] += YB[b][i];
    for (int b = 0; b < nb; b++) memcpy(x + (size_t)b * H, XB[b], H * sizeof(float));
    if (att) for (int b = 0; b < nb; b++) memcpy(att + (size_t)b * H, ATTB[b], H * sizeof(float));
    FAST_LEAVE;
}
