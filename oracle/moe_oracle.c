/* moe_oracle.c -- CPU restatement of maple-runtime's MoE hot path, for checking only.
 *
 * TEST INFRASTRUCTURE: loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
 * checker. Never linked into the product. Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math).
 * See moe_oracle.h for the reference citation of every function and how each one is pinned.
 */
#include "moe_oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

static inline float bf2f(uint16_t v) { union { uint32_t u; float f; } c; c.u = (uint32_t)v << 16; return c.f; }

/* convert.py:29-33: group of 128 columns -> 32 bytes; byte j = c[j] | c[j+32]<<2 | c[j+64]<<4 | c[j+96]<<6 */
void mo_pack(const uint8_t *codes, int rows, int cols, uint8_t *packed) {
    for (int r = 0; r < rows; r++)
        for (int g = 0; g < cols / 128; g++)
            for (int j = 0; j < 32; j++) {
                const uint8_t *c = codes + (size_t)r * cols + g * 128 + j;
                packed[(size_t)r * (cols / 4) + g * 32 + j] = (uint8_t)(c[0] | (c[32] << 2) | (c[64] << 4) | (c[96] << 6));
            }
}

/* convert.py:36-40 */
void mo_unpack(const uint8_t *packed, int rows, int cols, uint8_t *codes) {
    for (int r = 0; r < rows; r++)
        for (int g = 0; g < cols / 128; g++)
            for (int j = 0; j < 32; j++) {
                uint8_t b = packed[(size_t)r * (cols / 4) + g * 32 + j];
                for (int s = 0; s < 4; s++) codes[(size_t)r * cols + g * 128 + s * 32 + j] = (b >> (2 * s)) & 3;
            }
}

/* maple.c:183-194. The documented build (-O3 -ffast-math, AVX2) compiles `mx / 127.0f` to a multiply by
 * the rounded constant 1/127 (0x3C010204) and `1.0f / qs` to `127.0f / mx`; lrintf is cvtss2si
 * (round half to even). Those compiled semantics are the ones restated here. */
float mo_prep(const float *x, int n, int8_t *q, int32_t *qsum) {
    float mx = 0.0f;
    for (int i = 0; i < n; i++) { float a = fabsf(x[i]); if (a > mx) mx = a; }
    float qs = 1.0f, inv = 1.0f;
    if (mx > 0.0f) { qs = mx * (1.0f / 127.0f); inv = 127.0f / mx; }
    int32_t s = 0;
    for (int i = 0; i < n; i++) { int v = (int)rintf(x[i] * inv); q[i] = (int8_t)v; s += v; }
    *qsum = s;
    return qs;
}

/* maple.c:195-227 (tdot), 423-458 (tdot_multi): integer sum of code * q; AVX2 maddubs lanes cannot
 * saturate (maple.c:208) so the integer result is exact whatever the summation order. */
int32_t mo_dot_i32(const uint8_t *row, const int8_t *q, int cols) {
    int32_t tot = 0;
    for (int g = 0; g < cols / 128; g++) {
        const uint8_t *p = row + g * 32; const int8_t *qg = q + g * 128;
        for (int j = 0; j < 32; j++) {
            uint8_t b = p[j];
            tot += (b & 3) * qg[j] + ((b >> 2) & 3) * qg[32 + j] + ((b >> 4) & 3) * qg[64 + j] + (b >> 6) * qg[96 + j];
        }
    }
    return tot;
}

/* maple.c:226 / 452: (float)(tot - qsum) * qs * s[r], left to right */
float mo_tdot(const uint8_t *row, float s, const int8_t *q, float qs, int32_t qsum, int cols) {
    return (float)(mo_dot_i32(row, q, cols) - qsum) * qs * s;
}

/* maple.c:111-115 hsum of 8 lanes: ((v0+v4)+(v1+v5)) + ((v2+v6)+(v3+v7)) */
static inline float hsum8(const float *v) {
    float a0 = v[0] + v[4], a1 = v[1] + v[5], a2 = v[2] + v[6], a3 = v[3] + v[7];
    return (a0 + a1) + (a2 + a3);
}

/* maple.c:853-889: acc lane j += w[c+j] * x[c+j] (FMA) for c = 0, 8, ..., then hsum */
void mo_router_batch(const float *hn, int nb, const uint16_t *w, const float *bias, float *rl) {
    for (int b = 0; b < nb; b++) {
        const float *x = hn + (size_t)b * MO_H;
        for (int e = 0; e < MO_NE; e++) {
            const uint16_t *p = w + (size_t)e * MO_H;
            float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int c = 0; c < MO_H; c += 8)
                for (int j = 0; j < 8; j++) acc[j] = fmaf(bf2f(p[c + j]), x[c + j], acc[j]);
            float v = hsum8(acc);
            if (bias) v = v + bias[e];
            rl[(size_t)b * MO_NE + e] = v;
        }
    }
}

/* maple.c:146-157 bf_row: a0 lane j takes columns c+j, a1 lane j takes c+8+j, c = 0, 16, ...;
 * hsum(a0 + a1) */
void mo_router_step(const float *hn, const uint16_t *w, const float *bias, float *rl) {
    for (int e = 0; e < MO_NE; e++) {
        const uint16_t *p = w + (size_t)e * MO_H;
        float a0[8] = {0, 0, 0, 0, 0, 0, 0, 0}, a1[8] = {0, 0, 0, 0, 0, 0, 0, 0}, s[8];
        for (int c = 0; c < MO_H; c += 16)
            for (int j = 0; j < 8; j++) {
                a0[j] = fmaf(bf2f(p[c + j]), hn[c + j], a0[j]);
                a1[j] = fmaf(bf2f(p[c + 8 + j]), hn[c + 8 + j], a1[j]);
            }
        for (int j = 0; j < 8; j++) s[j] = a0[j] + a1[j];
        float v = hsum8(s);
        if (bias) v = v + bias[e];
        rl[e] = v;
    }
}

/* exp(x) in fp32 arithmetic: k = rint(x * log2(e)), r = x - k ln2 with ln2 split in two (two FMAs, exact
 * for |k| < 2^12), exp(r) by its Taylor series to r^7 (|r| <= 0.347: truncation 6e-9 relative) by Horner with
 * FMA, then times 2^k as exponent-field arithmetic in two steps (2^(k/2) * 2^(k - k/2)) so that results in
 * the subnormal range are rounded once more like any product. Overflow gives inf, x < -104 gives 0.
 * The HIP kernels run the identical operation sequence, so both sides produce the same bits. */
static inline float pow2i(int k) { union { uint32_t u; float f; } c; c.u = (uint32_t)(k + 127) << 23; return c.f; }
float mo_exp(float x) {
    if (x > 88.8f) return (float)INFINITY;
    if (x < -104.0f) return 0.0f;
    float k = rintf(x * 1.44269504f);
    float r = fmaf(-k, 0.693145752f, x);
    r = fmaf(-k, 1.42860677e-06f, r);
    float p = 1.98412698e-04f;
    p = fmaf(p, r, 1.38888889e-03f);
    p = fmaf(p, r, 8.33333333e-03f);
    p = fmaf(p, r, 4.16666667e-02f);
    p = fmaf(p, r, 1.66666667e-01f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int ki = (int)k, k1 = ki / 2, k2 = ki - k1;
    return p * pow2i(k1) * pow2i(k2);
}

/* maple.c:910-923 */
void mo_topk(const float *rl, int nb, int32_t *top, float *tw) {
    for (int b = 0; b < nb; b++) {
        float lg[MO_NE], mx = -1e30f, sum = 0.0f, tsum = 0.0f;
        memcpy(lg, rl + (size_t)b * MO_NE, sizeof lg);
        for (int e = 0; e < MO_NE; e++) if (lg[e] > mx) mx = lg[e];
        /* maple.c's -O3 -ffast-math AVX2 build sums this loop in 8-wide vector lanes; the oracle pins
         * one such order: lane j sums experts j, j+8, ... in order, lanes folded by hsum8 */
        float part[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int e = 0; e < MO_NE; e++) { lg[e] = mo_exp(lg[e] - mx); part[e & 7] = part[e & 7] + lg[e]; }
        sum = hsum8(part);
        for (int e = 0; e < MO_NE; e++) lg[e] = lg[e] / sum;
        for (int k = 0; k < MO_TOPK; k++) {
            int best = -1;
            for (int e = 0; e < MO_NE; e++) if (best < 0 || lg[e] > lg[best]) best = e;
            top[b * MO_TOPK + k] = best; tw[b * MO_TOPK + k] = lg[best]; tsum += lg[best]; lg[best] = -1.0f;
        }
        for (int k = 0; k < MO_TOPK; k++) tw[b * MO_TOPK + k] = tw[b * MO_TOPK + k] / (tsum + 1e-20f);
    }
}

/* maple.c:924-938 and 1018-1019 */
int mo_group(const int32_t *top, const float *tw, int nb, int *nu_out, int32_t *ue, int32_t *ustart,
             int32_t *utok, float *uw, int32_t *tp) {
    int cnt[MO_NE] = {0}, uidx[MO_NE], fillc[MO_NE] = {0}, nu = 0, na = 0;
    for (int b = 0; b < nb; b++) for (int s = 0; s < MO_TOPK; s++) cnt[top[b * MO_TOPK + s]]++;
    for (int e = 0; e < MO_NE; e++) if (cnt[e]) { uidx[e] = nu; ue[nu] = e; ustart[nu++] = na; na += cnt[e]; }
    ustart[nu] = na;
    for (int b = 0; b < nb; b++) for (int s = 0; s < MO_TOPK; s++) {
        int u = uidx[top[b * MO_TOPK + s]], slot = ustart[u] + fillc[u]++;
        utok[slot] = b; uw[slot] = tw[b * MO_TOPK + s];
    }
    if (tp) {
        int *fl = (int *)calloc((size_t)nb, sizeof(int));
        for (int a = 0; a < na; a++) { int b = utok[a]; tp[b * MO_TOPK + fl[b]++] = a; }
        free(fl);
    }
    *nu_out = nu;
    return na;
}

/* maple.c:826-830 */
void mo_act(const float *G, const float *U, float *act, int n) {
    for (int k = 0; k < n; k++) {
        float g = G[k] < 7.0f ? G[k] : 7.0f, u = U[k];
        u = u < -7.0f ? -7.0f : (u > 7.0f ? 7.0f : u);
        act[k] = g / (1.0f + mo_exp(-g)) * u;
    }
}

/* maple.c:398-402 */
void mo_rmsnorm(const float *x, const uint16_t *w, int n, float *out) {
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * x[i];
    float k = 1.0f / sqrtf((float)(ss / n) + 1e-6f);
    for (int i = 0; i < n; i++) out[i] = x[i] * k * (w ? bf2f(w[i]) : 1.0f);
}

/* gate/up of one pair (maple.c:471-479 via tdot_multi): G[512], U[512], optional raw i32 [1024] */
static void gateup_pair(const mo_expert *ex, const int8_t *q, float qs, int32_t qsum, float *G, float *U, int32_t *raw) {
    for (int k = 0; k < MO_FF; k++) {
        int32_t tg = mo_dot_i32(ex->gc + (size_t)k * (MO_H / 4), q, MO_H);
        int32_t tu = mo_dot_i32(ex->uc + (size_t)k * (MO_H / 4), q, MO_H);
        if (raw) { raw[k] = tg; raw[MO_FF + k] = tu; }
        G[k] = (float)(tg - qsum) * qs * ex->gs[k];
        U[k] = (float)(tu - qsum) * qs * ex->us[k];
    }
}

/* down of one pair (maple.c:498-505): D[2048], optional raw i32 [2048] */
static void down_pair(const mo_expert *ex, const int8_t *qa, float qs, int32_t qsum, float *D, int32_t *raw) {
    for (int r = 0; r < MO_H; r++) {
        int32_t t = mo_dot_i32(ex->dc + (size_t)r * (MO_FF / 4), qa, MO_FF);
        if (raw) raw[r] = t;
        D[r] = (float)(t - qsum) * qs * ex->ds[r];
    }
}

typedef struct { int8_t *q; float *qs; int32_t *qsum; } qvec;

/* Shared body of the batched path: prep, gate/up, act, re-quant, down for each pair. Per-pair outputs
 * go to D[P][2048]. */
static void experts_body(const float *hn, int nb, int nu, const mo_expert *const *exu, const int32_t *ustart,
                         const int32_t *utok, float *D, mo_trace *tr) {
    int P = ustart[nu];
    int8_t *qx = (int8_t *)malloc((size_t)nb * MO_H); float *qsx = (float *)malloc(sizeof(float) * nb);
    int32_t *qsumx = (int32_t *)malloc(sizeof(int32_t) * nb);
    for (int b = 0; b < nb; b++) qsx[b] = mo_prep(hn + (size_t)b * MO_H, MO_H, qx + (size_t)b * MO_H, &qsumx[b]);
    float G[MO_FF], U[MO_FF], A[MO_FF]; int8_t qa[MO_FF];
    for (int u = 0; u < nu; u++)
        for (int a = ustart[u]; a < ustart[u + 1]; a++) {
            int b = utok[a];
            gateup_pair(exu[u], qx + (size_t)b * MO_H, qsx[b], qsumx[b], G, U, tr && tr->gu_i32 ? tr->gu_i32 + (size_t)a * 2 * MO_FF : NULL);
            mo_act(G, U, A, MO_FF);
            int32_t qsa; float qsa_s = mo_prep(A, MO_FF, qa, &qsa);
            down_pair(exu[u], qa, qsa_s, qsa, D + (size_t)a * MO_H, tr && tr->dn_i32 ? tr->dn_i32 + (size_t)a * MO_H : NULL);
            if (tr) {
                if (tr->gate) memcpy(tr->gate + (size_t)a * MO_FF, G, sizeof G);
                if (tr->up) memcpy(tr->up + (size_t)a * MO_FF, U, sizeof U);
                if (tr->act) memcpy(tr->act + (size_t)a * MO_FF, A, sizeof A);
                if (tr->qa) memcpy(tr->qa + (size_t)a * MO_FF, qa, sizeof qa);
                if (tr->qsa) tr->qsa[a] = qsa_s;
                if (tr->qsuma) tr->qsuma[a] = qsa;
            }
        }
    if (tr) {
        if (tr->qx) memcpy(tr->qx, qx, (size_t)nb * MO_H);
        if (tr->qsx) memcpy(tr->qsx, qsx, sizeof(float) * nb);
        if (tr->qsumx) memcpy(tr->qsumx, qsumx, sizeof(int32_t) * nb);
        if (tr->down) memcpy(tr->down, D, sizeof(float) * (size_t)P * MO_H);
    }
    free(qx); free(qsx); free(qsumx);
}

/* maple.c:732-755 (route, top-8, grouping) and 824-834 (experts, act, combine) */
void mo_moe_batch(const float *hn, int nb, const uint16_t *router, const float *bias, const float *rl_in,
                  const mo_expert *experts, float *x, mo_trace *tr) {
    float *rl = (float *)malloc(sizeof(float) * (size_t)nb * MO_NE);
    if (rl_in) memcpy(rl, rl_in, sizeof(float) * (size_t)nb * MO_NE);
    else mo_router_batch(hn, nb, router, bias, rl);
    int32_t *top = (int32_t *)malloc(sizeof(int32_t) * nb * MO_TOPK); float *tw = (float *)malloc(sizeof(float) * nb * MO_TOPK);
    mo_topk(rl, nb, top, tw);
    int P = nb * MO_TOPK, nu;
    int32_t ue[MO_NE], ustart[MO_NE + 1];
    int32_t *utok = (int32_t *)malloc(sizeof(int32_t) * P), *tp = (int32_t *)malloc(sizeof(int32_t) * P);
    float *uw = (float *)malloc(sizeof(float) * P);
    mo_group(top, tw, nb, &nu, ue, ustart, utok, uw, tp);
    const mo_expert *exu[MO_NE];
    for (int u = 0; u < nu; u++) exu[u] = &experts[ue[u]];
    float *D = (float *)malloc(sizeof(float) * (size_t)P * MO_H);
    experts_body(hn, nb, nu, exu, ustart, utok, D, tr);
    /* maple.c:834: x[tok] += UW[a] * DOWNB[a][i], pairs in grouped order; the AVX2 build contracts to FMA */
    for (int a = 0; a < P; a++) {
        float *xb = x + (size_t)utok[a] * MO_H; const float *d = D + (size_t)a * MO_H;
        for (int i = 0; i < MO_H; i++) xb[i] = fmaf(uw[a], d[i], xb[i]);
    }
    if (tr) {
        if (tr->rl) memcpy(tr->rl, rl, sizeof(float) * (size_t)nb * MO_NE);
        if (tr->top) memcpy(tr->top, top, sizeof(int32_t) * nb * MO_TOPK);
        if (tr->tw) memcpy(tr->tw, tw, sizeof(float) * nb * MO_TOPK);
        if (tr->nu) *tr->nu = nu;
        if (tr->ue) memcpy(tr->ue, ue, sizeof(int32_t) * nu);
        if (tr->ustart) memcpy(tr->ustart, ustart, sizeof(int32_t) * (nu + 1));
        if (tr->utok) memcpy(tr->utok, utok, sizeof(int32_t) * P);
        if (tr->uw) memcpy(tr->uw, uw, sizeof(float) * P);
        if (tr->tp) memcpy(tr->tp, tp, sizeof(int32_t) * P);
    }
    free(rl); free(top); free(tw); free(utok); free(tp); free(uw); free(D);
}

/* maple.c:605-665 (without the gpux branch) */
void mo_moe_step(const float *hn, const uint16_t *router, const float *bias, const mo_expert *experts,
                 float *x, mo_trace *tr) {
    float rl[MO_NE]; int32_t top[MO_TOPK]; float tw[MO_TOPK];
    mo_router_step(hn, router, bias, rl);
    mo_topk(rl, 1, top, tw);
    int8_t qx[MO_H]; int32_t qsumx; float qsx = mo_prep(hn, MO_H, qx, &qsumx);
    float G[MO_FF], U[MO_FF], A[MO_FF]; int8_t qa[MO_FF];
    float *D = (float *)malloc(sizeof(float) * MO_TOPK * MO_H);
    for (int s = 0; s < MO_TOPK; s++) {
        const mo_expert *ex = &experts[top[s]];
        gateup_pair(ex, qx, qsx, qsumx, G, U, tr && tr->gu_i32 ? tr->gu_i32 + (size_t)s * 2 * MO_FF : NULL);
        mo_act(G, U, A, MO_FF);
        int32_t qsa; float qsa_s = mo_prep(A, MO_FF, qa, &qsa);
        down_pair(ex, qa, qsa_s, qsa, D + (size_t)s * MO_H, tr && tr->dn_i32 ? tr->dn_i32 + (size_t)s * MO_H : NULL);
        if (tr) {
            if (tr->gate) memcpy(tr->gate + (size_t)s * MO_FF, G, sizeof G);
            if (tr->up) memcpy(tr->up + (size_t)s * MO_FF, U, sizeof U);
            if (tr->act) memcpy(tr->act + (size_t)s * MO_FF, A, sizeof A);
            if (tr->qa) memcpy(tr->qa + (size_t)s * MO_FF, qa, sizeof qa);
            if (tr->qsa) tr->qsa[s] = qsa_s;
            if (tr->qsuma) tr->qsuma[s] = qsa;
        }
    }
    /* maple.c:664: y = sum over slots of TOPW[s] * DOWN[s][i] (FMA), X[i] += y */
    for (int i = 0; i < MO_H; i++) {
        float y = 0.0f;
        for (int s = 0; s < MO_TOPK; s++) y = fmaf(tw[s], D[(size_t)s * MO_H + i], y);
        x[i] = x[i] + y;
    }
    if (tr) {
        if (tr->rl) memcpy(tr->rl, rl, sizeof rl);
        if (tr->top) memcpy(tr->top, top, sizeof top);
        if (tr->tw) memcpy(tr->tw, tw, sizeof tw);
        if (tr->qx) memcpy(tr->qx, qx, sizeof qx);
        if (tr->qsx) *tr->qsx = qsx;
        if (tr->qsumx) *tr->qsumx = qsumx;
        if (tr->down) memcpy(tr->down, D, sizeof(float) * MO_TOPK * MO_H);
    }
    free(D);
}

/* gpre_moe semantics (gpu_pre.m:321-385 + cmb gpu_pre.m:158-163): y[b] = sum over tp[b][j] of the
 * weighted down outputs; the weighting and the sum use the FMA chain y = fma(uw, D, y) from 0. */
void mo_experts_grouped(const float *hn, int nb, int nu, const mo_expert *ex, const int32_t *ustart,
                        const int32_t *utok, const float *uw, const int32_t *tp, float *y, mo_trace *tr) {
    int P = ustart[nu];
    const mo_expert *exu[MO_NE];
    for (int u = 0; u < nu; u++) exu[u] = &ex[u];
    float *D = (float *)malloc(sizeof(float) * (size_t)P * MO_H);
    experts_body(hn, nb, nu, exu, ustart, utok, D, tr);
    for (int b = 0; b < nb; b++)
        for (int i = 0; i < MO_H; i++) {
            float s = 0.0f;
            for (int j = 0; j < MO_TOPK; j++) { int a = tp[b * MO_TOPK + j]; s = fmaf(uw[a], D[(size_t)a * MO_H + i], s); }
            y[(size_t)b * MO_H + i] = s;
        }
    free(D);
}

/* ---------------------------------------------------------------- attention half (maple.c:706-724) */
/* maple.c:403-411. Its build (-O3 -ffast-math -mfma) contracts each line into one FMA whose addend is the
 * rounded second product: t[i] = fma(v[i], c, -(v[i+32] s)), t[i+32] = fma(v[i+32], c, v[i] s) (the form
 * that matches the compiled maple.c bit for bit; tests/test_oracle_attn.py). */
void mo_rope(float *v, const float *cs) {
    float t[MO_ROT];
    for (int i = 0; i < MO_ROT / 2; i++) {
        float c = cs[2 * i], s = cs[2 * i + 1], a = v[i], w = v[i + MO_ROT / 2];
        t[i] = fmaf(a, c, -(w * s));
        t[i + MO_ROT / 2] = fmaf(w, c, a * s);
    }
    memcpy(v, t, sizeof t);
}

/* maple.c:314-320: IEEE binary16, round to nearest even */
static uint16_t f2h(float f) {
    union { float f; uint32_t u; } c = {f};
    uint32_t sign = (c.u >> 16) & 0x8000u, a = c.u & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0));   /* inf / nan */
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);                /* rounds past 65504 */
    if (a < 0x38800000u) {                                                  /* subnormal half (or zero) */
        if (a < 0x33000000u) return (uint16_t)sign;                         /* below half the smallest */
        uint32_t m = (a & 0x7fffffu) | 0x800000u; int e = (int)(a >> 23);  /* value = m * 2^(e - 150) */
        int sh = 126 - e;                                                   /* half units of 2^-24: m >> (sh) */
        uint32_t q = m >> sh, rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t h = ((a >> 13) - ((127 - 15) << 10)), rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;
    return (uint16_t)(sign | h);
}
void mo_f16(const float *s, uint16_t *d, int n) { for (int i = 0; i < n; i++) d[i] = f2h(s[i]); }
float mo_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31, m = h & 0x3ffu;
    union { uint32_t u; float f; } c;
    if (e == 31) c.u = sign | 0x7f800000u | (m << 13);
    else if (e) c.u = sign | ((e + 112) << 23) | (m << 13);
    else { c.f = (float)m * (1.0f / 16777216.0f); c.u |= sign; }
    return c.f;
}

/* maple.c:516-558 */
void mo_attend(const float *q, const uint16_t *kc, const uint16_t *vc, int kvh, int pos, int glob, int win,
               float *out, float *sc) {
    int lo = glob ? 0 : (pos - win > 0 ? pos - win : 0), T = pos - lo + 1;
    const float scale = 1.0f / sqrtf((float)MO_HD);
    float mx[4], inv[4];
    for (int j = 0; j < 4; j++) { mx[j] = -1e30f; memset(out + j * MO_HD, 0, MO_HD * sizeof(float)); }
    for (int t = 0; t < T; t++) {
        const uint16_t *kk = kc + (size_t)(lo + t) * 512 + kvh * MO_HD;
        float kf[MO_HD];
        for (int d = 0; d < MO_HD; d++) kf[d] = mo_h2f(kk[d]);
        for (int j = 0; j < 4; j++) {
            float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int d = 0; d < MO_HD; d += 8)
                for (int l = 0; l < 8; l++) a[l] = fmaf(kf[d + l], q[j * MO_HD + d + l], a[l]);
            float s = hsum8(a) * scale;
            sc[j * T + t] = s;
            if (s > mx[j]) mx[j] = s;
        }
    }
    for (int j = 0; j < 4; j++) {
        float sum = 0, *sj = sc + j * T;
        for (int t = 0; t < T; t++) { sj[t] = mo_exp(sj[t] - mx[j]); sum += sj[t]; }
        inv[j] = 1.0f / sum;
    }
    for (int t = 0; t < T; t++) {
        const uint16_t *vv = vc + (size_t)(lo + t) * 512 + kvh * MO_HD;
        for (int j = 0; j < 4; j++) {
            float w = sc[j * T + t] * inv[j];
            for (int d = 0; d < MO_HD; d++) out[j * MO_HD + d] = fmaf(w, mo_h2f(vv[d]), out[j * MO_HD + d]);
        }
    }
}

/* maple.c:706-724 (CPU path), one sequence */
void mo_attn_chunk(float *x, int nb, int pos0, int glob, int win, const uint16_t *in_ln, const uint16_t *q_norm,
                   const uint16_t *k_norm, mo_t2 wq, mo_t2 wk, mo_t2 wv, mo_t2 wo, const float *cs,
                   uint16_t *kc, uint16_t *vc, uint16_t *ko, float *att) {
    float *hn = malloc(sizeof(float) * MO_H), *qkv = malloc(sizeof(float) * (size_t)nb * 3072);
    float *at = malloc(sizeof(float) * (size_t)nb * MO_H), *sc = malloc(sizeof(float) * 4 * (size_t)(pos0 + nb));
    int8_t *q8 = malloc(MO_H);
    for (int b = 0; b < nb; b++) {
        float qs; int32_t qsum;
        mo_rmsnorm(x + (size_t)b * MO_H, in_ln, MO_H, hn);
        qs = mo_prep(hn, MO_H, q8, &qsum);
        float *o = qkv + (size_t)b * 3072;
        for (int r = 0; r < 2048; r++) o[r] = mo_tdot(wq.p + (size_t)r * (wq.cols / 4), wq.s[r], q8, qs, qsum, wq.cols);
        for (int r = 0; r < 512; r++) o[2048 + r] = mo_tdot(wk.p + (size_t)r * (wk.cols / 4), wk.s[r], q8, qs, qsum, wk.cols);
        for (int r = 0; r < 512; r++) o[2560 + r] = mo_tdot(wv.p + (size_t)r * (wv.cols / 4), wv.s[r], q8, qs, qsum, wv.cols);
    }
    for (int b = 0; b < nb; b++) {
        int pos = pos0 + b;
        float *o = qkv + (size_t)b * 3072;
        for (int h = 0; h < MO_NH; h++) {
            mo_rmsnorm(o + h * MO_HD, q_norm, MO_HD, o + h * MO_HD);
            if (!glob) mo_rope(o + h * MO_HD, cs + (size_t)pos * MO_ROT);
        }
        for (int h = 0; h < MO_NKV; h++) {
            mo_rmsnorm(o + 2048 + h * MO_HD, k_norm, MO_HD, o + 2048 + h * MO_HD);
            if (!glob) mo_rope(o + 2048 + h * MO_HD, cs + (size_t)pos * MO_ROT);
        }
        mo_f16(o + 2048, kc + (size_t)pos * 512, 512);
        mo_f16(o + 2560, vc + (size_t)pos * 512, 512);
        if (ko) { memcpy(ko + (size_t)b * 1024, kc + (size_t)pos * 512, 1024); memcpy(ko + (size_t)b * 1024 + 512, vc + (size_t)pos * 512, 1024); }
    }
    for (int b = 0; b < nb; b++)
        for (int kvh = 0; kvh < MO_NKV; kvh++)
            mo_attend(qkv + (size_t)b * 3072 + kvh * 4 * MO_HD, kc, vc, kvh, pos0 + b, glob, win,
                      at + (size_t)b * MO_H + kvh * 4 * MO_HD, sc);
    for (int b = 0; b < nb; b++) {
        float qs; int32_t qsum;
        qs = mo_prep(at + (size_t)b * MO_H, MO_H, q8, &qsum);
        for (int r = 0; r < MO_H; r++) {
            float y = mo_tdot(wo.p + (size_t)r * (wo.cols / 4), wo.s[r], q8, qs, qsum, wo.cols);
            x[(size_t)b * MO_H + r] = x[(size_t)b * MO_H + r] + y;
        }
    }
    if (att) memcpy(att, at, sizeof(float) * (size_t)nb * MO_H);
    free(hn); free(qkv); free(at); free(sc); free(q8);
}
