/* synth.c -- seeded synthetic Maple-shaped MoE data in the reference's packed layout.
 *
 * There is no checkpoint here (convert.py streams it from the network, convert.py:43-125), so the workloads
 * are synthetic: ternary codes drawn iid with P(w=0) = 0.4 and P(w=+1) = P(w=-1) = 0.3, packed 2 bits each in
 * the layout of convert.py:29-33 (byte j of a 128-column group holds columns j, j+32, j+64, j+96 at bits
 * 0,2,4,6; code = w+1), one fp32 scale per row uniform in [0.01, 0.05] (convert.py keeps one scale per row),
 * router rows as bf16 (layout.py:14 stores mlp.gate.weight as bf16), hidden states N(0,1).
 *
 * Every value is a pure function of (seed, tensor id, element index) through splitmix64, so any subset can
 * be regenerated anywhere (host or test) and compared bit for bit.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "maplesynth.h"

#define SY_H 2048
#define SY_NE 256
#define SY_FF 512
#define SY_CODE_MAT 262144u                 /* 512 x 2048 codes, 2 bits each */
#define SY_EXPERT_BYTES (3u * SY_CODE_MAT + (512u + 512u + 2048u) * 4u)  /* 798,720 */

static inline uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static inline uint64_t stream_key(uint64_t seed, uint64_t a, uint64_t b, uint64_t c) {
    return mix64(mix64(mix64(seed ^ 0x6D61706C65ull) + a) + (b << 8) + c);
}
/* one 16-bit draw -> code: < 0.3 -> 0 (w=-1), < 0.7 -> 1 (w=0), else 2 (w=+1) */
static inline uint32_t code16(uint32_t h) { return h < 19661u ? 0u : (h < 45875u ? 1u : 2u); }

static void fill_codes(uint64_t key, uint8_t *dst, size_t nbytes) {
    for (size_t i = 0; i < nbytes; i++) {
        uint64_t h = mix64(key + i);
        dst[i] = (uint8_t)(code16((uint32_t)(h & 0xFFFF)) | (code16((uint32_t)((h >> 16) & 0xFFFF)) << 2) |
                           (code16((uint32_t)((h >> 32) & 0xFFFF)) << 4) | (code16((uint32_t)(h >> 48)) << 6));
    }
}
static void fill_scales(uint64_t key, float *dst, int n) {
    for (int i = 0; i < n; i++) {
        uint64_t h = mix64(key + (uint64_t)i);
        float u = (float)(uint32_t)(h >> 40) * (1.0f / 16777216.0f);
        float s = 0.04f * u;
        dst[i] = 0.01f + s;
    }
}

/* One expert (layer L, expert e): gate/up codes 512 rows x 512 B, down 2048 rows x 128 B, fp32 row scales */
void mmoe_synth_expert(uint64_t seed, int L, int e, uint8_t *gc, float *gs, uint8_t *uc, float *us, uint8_t *dc, float *ds) {
    fill_codes(stream_key(seed, (uint64_t)L, (uint64_t)e, 0), gc, SY_CODE_MAT);
    fill_scales(stream_key(seed, (uint64_t)L, (uint64_t)e, 1), gs, SY_FF);
    fill_codes(stream_key(seed, (uint64_t)L, (uint64_t)e, 2), uc, SY_CODE_MAT);
    fill_scales(stream_key(seed, (uint64_t)L, (uint64_t)e, 3), us, SY_FF);
    fill_codes(stream_key(seed, (uint64_t)L, (uint64_t)e, 4), dc, SY_CODE_MAT);
    fill_scales(stream_key(seed, (uint64_t)L, (uint64_t)e, 5), ds, SY_H);
}

/* Bytes of one expert in the contiguous per-layer block written by mmoe_synth_layer. Offsets inside an
 * expert: gate codes 0, gate scales 262144, up codes 264192, up scales 526336, down codes 528384,
 * down scales 790528. Every tensor is 16-byte aligned, as maple.c:1117 requires of a region. */
size_t mmoe_synth_expert_bytes(void) { return SY_EXPERT_BYTES; }

typedef struct { uint64_t seed; int L, e0, e1; uint8_t *base; } synth_job;
static void *synth_worker(void *p) {
    synth_job *j = (synth_job *)p;
    for (int e = j->e0; e < j->e1; e++) {
        uint8_t *b = j->base + (size_t)e * SY_EXPERT_BYTES;
        mmoe_synth_expert(j->seed, j->L, e, b, (float *)(b + SY_CODE_MAT), b + SY_CODE_MAT + 2048,
                          (float *)(b + 2 * SY_CODE_MAT + 2048), b + 2 * SY_CODE_MAT + 4096, (float *)(b + 3 * SY_CODE_MAT + 4096));
    }
    return NULL;
}
/* All 256 experts of layer L into base (256 * 798,720 bytes), with nthreads host threads */
void mmoe_synth_layer(uint64_t seed, int L, uint8_t *base, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 64) nthreads = 64;
    pthread_t th[64]; synth_job jobs[64];
    for (int t = 0; t < nthreads; t++) {
        jobs[t] = (synth_job){seed, L, SY_NE * t / nthreads, SY_NE * (t + 1) / nthreads, base};
        pthread_create(&th[t], NULL, synth_worker, &jobs[t]);
    }
    for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
}

static inline uint16_t f2bf(float f) {  /* round to nearest even; inputs are finite */
    uint32_t u; memcpy(&u, &f, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
static inline double unit01(uint64_t h) { return ((double)(h >> 11) + 0.5) * (1.0 / 9007199254740992.0); }

/* Router of layer L, 256 x 2048 bf16: dist 0 = N(0, 0.02^2) (Box-Muller), dist 1 = uniform with the same
 * variance, U(-0.02*sqrt(3), 0.02*sqrt(3)) */
void mmoe_synth_router(uint64_t seed, int L, int dist, uint16_t *w) {
    uint64_t key = stream_key(seed, 1000u + (uint64_t)L, 0, 7);
    for (size_t i = 0; i < (size_t)SY_NE * SY_H; i += 2) {
        double u1 = unit01(mix64(key + 2 * i)), u2 = unit01(mix64(key + 2 * i + 1));
        double a, b;
        if (dist == 0) {
            double r = sqrt(-2.0 * log(u1)) * 0.02;
            a = r * cos(6.283185307179586 * u2); b = r * sin(6.283185307179586 * u2);
        } else {
            const double h = 0.02 * 1.7320508075688772;
            a = (2.0 * u1 - 1.0) * h; b = (2.0 * u2 - 1.0) * h;
        }
        w[i] = f2bf((float)a); w[i + 1] = f2bf((float)b);
    }
}

/* nb hidden vectors of 2048, N(0,1), stream id sid */
void mmoe_synth_hidden(uint64_t seed, int sid, int nb, float *x) {
    uint64_t key = stream_key(seed, 2000u + (uint64_t)sid, 0, 9);
    size_t n = (size_t)nb * SY_H;
    for (size_t i = 0; i < n; i += 2) {
        double u1 = unit01(mix64(key + 2 * i)), u2 = unit01(mix64(key + 2 * i + 1));
        double r = sqrt(-2.0 * log(u1));
        x[i] = (float)(r * cos(6.283185307179586 * u2));
        x[i + 1] = (float)(r * sin(6.283185307179586 * u2));
    }
}

/* Per-expert logit bias b_e = ln(rank_e^-s / sum_r r^-s), ranks 1..256 assigned by a seeded permutation */
void mmoe_synth_zipf_bias(uint64_t seed, double s, float *bias) {
    int perm[SY_NE];
    for (int i = 0; i < SY_NE; i++) perm[i] = i;
    uint64_t key = stream_key(seed, 3000u, 0, 11);
    for (int i = SY_NE - 1; i > 0; i--) {  /* Fisher-Yates */
        int j = (int)(mix64(key + (uint64_t)i) % (uint64_t)(i + 1));
        int t = perm[i]; perm[i] = perm[j]; perm[j] = t;
    }
    double z = 0.0;
    for (int r = 1; r <= SY_NE; r++) z += pow((double)r, -s);
    for (int i = 0; i < SY_NE; i++) bias[perm[i]] = (float)log(pow((double)(i + 1), -s) / z);
}
