/* san_driver.c -- host code of the library and the oracle under AddressSanitizer + UBSan (CPU only).
 *
 * Built by tests/test_sanitize.py together with maple-runtime_amd/csrc/ckpt.c, csrc/synth.c and
 * oracle/moe_oracle.c, all with -fsanitize=address,undefined. ckpt.c's three calls into the GPU library are
 * replaced by the host stand-ins below: gpre_region reads every byte of the span it is given (so a span
 * outside its shard mapping is an ASan error) and mmoe_set_layer checks the location table against the
 * registered spans (so a bad table is a test failure).
 *
 *   san_driver ckpt DIR     open, plan, load and close a checkpoint; prints "open rc" and the error text
 *   san_driver synth        synthetic experts, a layer block, router, hidden state, Zipf bias
 *   san_driver oracle       one small MoE layer through the oracle (batch and step) plus its pieces
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "maplemoe.h"
#include "maplesynth.h"
#include "moe_oracle.h"

#define STUB_MAXREG 64   /* the stand-in's own region table (gpu_pre.m:21's size) */
static const uint8_t *REG_P[STUB_MAXREG];
static size_t REG_N[STUB_MAXREG];
static int NREG;
static volatile unsigned SINK;

int gpre_region(const void *p, size_t len) {
    if (NREG >= STUB_MAXREG) return -1;
    const uint8_t *b = (const uint8_t *)p;
    unsigned s = 0;
    for (size_t i = 0; i < len; i++) s += b[i];
    SINK += s;
    REG_P[NREG] = b; REG_N[NREG] = len;
    return NREG++;
}
int mmoe_set_layer(int L, const uint32_t *loc, const int *regs, const uint16_t *router, const uint16_t *post_ln) {
    (void)L;
    for (int e = 0; e < 256; e++)
        for (int m = 0; m < 6; m++) {
            uint32_t slot = loc[e * 12 + 2 * m], off = loc[e * 12 + 2 * m + 1];
            size_t len = m == 1 || m == 3 ? 2048 : m == 5 ? 8192 : 262144;
            if (slot > 3 || regs[slot] < 0 || regs[slot] >= NREG || off + len > REG_N[regs[slot]]) {
                fprintf(stderr, "bad location e %d m %d\n", e, m);
                exit(3);
            }
            SINK += REG_P[regs[slot]][off] + REG_P[regs[slot]][off + len - 1];
        }
    unsigned s = 0;
    for (int i = 0; i < 256 * 2048; i++) s += router[i];
    for (int i = 0; i < 2048; i++) s += post_ln[i];
    SINK += s;
    return 0;
}
const char *mmoe_last_error(void) { return "host stand-in"; }

static int run_ckpt(const char *dir) {
    int rc = mmoe_ckpt_open(dir);
    printf("open rc %d: %s\n", rc, rc ? mmoe_ckpt_error() : "ok");
    if (rc) return 0;
    static uint32_t loc[256 * 12];
    for (int L = 0; L < 24; L++) {
        int sh[4]; uint64_t lo[4], len[4];
        int n = mmoe_ckpt_layer_plan(L, sh, lo, len, loc);
        if (n < 1) { printf("plan %d failed: %s\n", L, mmoe_ckpt_error()); return 2; }
        for (int w = 0; w < 5; w++) if (!mmoe_ckpt_bf16(L, w)) { printf("bf16 %d %d missing\n", L, w); return 2; }
    }
    if (mmoe_ckpt_bf16(24, 0) || mmoe_ckpt_bf16(0, 5) || mmoe_ckpt_layer_plan(-1, NULL, NULL, NULL, NULL) != -1) return 2;
    rc = mmoe_ckpt_load(0, 21);              /* 3 regions a layer: 63 of the 64 region slots */
    printf("load rc %d regions %d\n", rc, NREG);
    int full = mmoe_ckpt_load(21, 3);         /* past the region table: refused, not overrun */
    printf("load past the region table rc %d: %s\n", full, full ? mmoe_ckpt_error() : "ok");
    mmoe_ckpt_close();
    mmoe_ckpt_close();   /* twice: idempotent */
    return rc || !full ? 2 : 0;
}

static int run_synth(void) {
    size_t eb = mmoe_synth_expert_bytes();
    uint8_t *blk = malloc(256 * eb);
    if (!blk) return 2;
    mmoe_synth_layer(7, 3, blk, 4);
    uint8_t *gc = malloc(262144), *uc = malloc(262144), *dc = malloc(262144);
    float *gs = malloc(2048), *us = malloc(2048), *ds = malloc(8192);
    mmoe_synth_expert(7, 3, 255, gc, gs, uc, us, dc, ds);
    int same = !memcmp(gc, blk + 255 * eb, 262144) && !memcmp(ds, blk + 255 * eb + eb - 8192, 8192);
    uint16_t *w = malloc(256 * 2048 * 2);
    for (int dist = 0; dist < 2; dist++) mmoe_synth_router(7, 3, dist, w);
    float *x = malloc(5 * 2048 * 4), bias[256];
    mmoe_synth_hidden(7, 1, 5, x);
    mmoe_synth_zipf_bias(7, 1.1, bias);
    printf("synth ok, expert 255 matches the block: %d\n", same);
    free(blk); free(gc); free(uc); free(dc); free(gs); free(us); free(ds); free(w); free(x);
    return same ? 0 : 2;
}

static int run_oracle(void) {
    enum { NB = 5 };
    size_t eb = mmoe_synth_expert_bytes();
    uint8_t *blk = malloc(256 * eb);
    mmoe_synth_layer(11, 0, blk, 4);
    mo_expert ex[256];
    for (int e = 0; e < 256; e++) {
        uint8_t *b = blk + e * eb;
        ex[e] = (mo_expert){b, (const float *)(b + 262144), b + 264192, (const float *)(b + 526336), b + 528384,
                            (const float *)(b + 790528)};
    }
    uint16_t *w = malloc(256 * 2048 * 2);
    mmoe_synth_router(11, 0, 0, w);
    float *x = malloc(NB * 2048 * 4), *hn = malloc(NB * 2048 * 4), *x2 = malloc(NB * 2048 * 4);
    mmoe_synth_hidden(11, 2, NB, x);
    for (int b = 0; b < NB; b++) mo_rmsnorm(x + b * 2048, NULL, 2048, hn + b * 2048);
    memcpy(x2, x, NB * 2048 * 4);
    enum { P = NB * 8 };
    static float rl[NB * 256], tw[P], uw[P], act[P * 512], down[P * 2048], gate[P * 512], up[P * 512];
    static int32_t top[P], ue[256], us_[257], utok[P], tp[P], gu[P * 1024], dn[P * 2048];
    int nu = 0;
    mo_trace tr = {.rl = rl, .top = top, .tw = tw, .nu = &nu, .ue = ue, .ustart = us_, .utok = utok, .uw = uw, .tp = tp,
                   .gu_i32 = gu, .gate = gate, .up = up, .act = act, .dn_i32 = dn, .down = down};
    mo_moe_batch(hn, NB, w, NULL, NULL, ex, x, &tr);
    mo_moe_step(hn, w, NULL, ex, x2, NULL);
    /* the pieces on their own, including the special cases */
    int8_t q[2048]; int32_t qsum;
    float z[2048] = {0};
    float qs = mo_prep(z, 2048, q, &qsum);
    uint8_t codes[4 * 128], packed[4 * 32], back[4 * 128];
    for (int i = 0; i < 4 * 128; i++) codes[i] = (uint8_t)(i * 7 % 3);
    mo_pack(codes, 4, 128, packed);
    mo_unpack(packed, 4, 128, back);
    float y[NB * 2048];
    mo_experts_grouped(hn, NB, nu, ex, us_, utok, uw, tp, y, NULL);
    printf("oracle ok: nu %d, prep(0) qs %g qsum %d, pack round trip %d\n", nu, qs, qsum, !memcmp(codes, back, sizeof codes));
    free(blk); free(w); free(x); free(hn); free(x2);
    return (qs == 1.0f && qsum == 0 && !memcmp(codes, back, sizeof codes)) ? 0 : 2;
}

int main(int argc, char **argv) {
    if (argc >= 3 && !strcmp(argv[1], "ckpt")) return run_ckpt(argv[2]);
    if (argc >= 2 && !strcmp(argv[1], "synth")) return run_synth();
    if (argc >= 2 && !strcmp(argv[1], "oracle")) return run_oracle();
    fprintf(stderr, "usage: san_driver ckpt DIR | synth | oracle\n");
    return 1;
}
