/* ckpt.c -- maple.c's on-disk checkpoint, read for the MoE path (host code, no GPU calls of its own).
 *
 * A checkpoint directory holds shard-00001.bin .. shard-00009.bin and layout.bin (maple.c:61-83; written by
 * layout.py). layout.bin is a table of packed records <kind u8 ('t' ternary, 'b' bf16), shard u8 (0..8), data
 * offset u64, scale offset u64, rows u32, cols u32>, struct format '<BBQQII' = 26 bytes (maple.c:39 Rec; the
 * docstring of layout.py says 24), in one fixed order (layout.py:1-5): word embeddings, lm_head, final norm;
 * then per layer input_layernorm, post_attention_layernorm, q_norm, k_norm, router (bf16), q, k, v, o
 * (ternary), and gate, up, down of each of the 256 experts (ternary).
 *
 * mmoe_ckpt_open maps the shards read-only and checks the table as maple.c's load() does (record kinds), plus
 * what the MoE path relies on: every expert, router and post-norm tensor lies inside its shard, has the
 * shapes of the packed layout and starts 16-byte aligned (the check of maple.c:1116-1117).
 * mmoe_ckpt_layer_plan computes one layer's device regions and location table exactly as maple.c:1106-1131:
 * per shard, the page-aligned span of the layer's 256 x 6 expert tensors becomes one region (shards in
 * ascending order, at most 4), and GLOC[e][2m] = region slot, GLOC[e][2m+1] = byte offset inside it for
 * m = gate codes, gate scales, up codes, up scales, down codes, down scales.
 * mmoe_ckpt_load registers the regions (gpre_region) and the layer (mmoe_set_layer). */
#define _DEFAULT_SOURCE
#include "maplemoe.h"
#include <fcntl.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#define CK_NSHARD 9
#define CK_NL 24
#define CK_NE 256
#define CK_H 2048
#define CK_FF 512
#define CK_GLOBAL 3                       /* embeddings, lm_head, norm */
#define CK_PER_LAYER (9 + 3 * CK_NE)       /* 4 norms + router, q k v o, 256 x (gate, up, down) */
#define CK_NREC (CK_GLOBAL + CK_NL * CK_PER_LAYER)

typedef struct __attribute__((packed)) { uint8_t kind, file; uint64_t off, soff; uint32_t rows, cols; } CkRec;
_Static_assert(sizeof(CkRec) == 26, "layout.bin record: 26 bytes, struct.pack('<BBQQII')");

static struct {
    int open;
    const uint8_t *file[CK_NSHARD];
    size_t size[CK_NSHARD];
    CkRec rec[CK_NREC];
} C;

static char ck_err[256];
static int fail(const char *fmt, ...) {
    va_list ap; va_start(ap, fmt); vsnprintf(ck_err, sizeof ck_err, fmt, ap); va_end(ap);
    return -1;
}
const char *mmoe_ckpt_error(void) { return ck_err; }

void mmoe_ckpt_close(void) {
    for (int k = 0; k < CK_NSHARD; k++)
        if (C.file[k]) munmap((void *)C.file[k], C.size[k]);
    memset(&C, 0, sizeof C);
}

static int map_file(const char *path, const uint8_t **p, size_t *sz) {
    int fd = open(path, O_RDONLY);
    if (fd < 0) return fail("cannot open %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0) { close(fd); return fail("cannot stat %s", path); }
    *sz = (size_t)st.st_size;
    void *m = *sz ? mmap(NULL, *sz, PROT_READ, MAP_SHARED, fd, 0) : MAP_FAILED;
    close(fd);
    if (m == MAP_FAILED) return fail("cannot map %s", path);
    *p = (const uint8_t *)m;
    return 0;
}

/* record index of layer L's tensor: j = 0..8 the per-layer tensors in order, then expert e part m (0 gate,
 * 1 up, 2 down) */
static int rec_layer(int L, int j) { return CK_GLOBAL + L * CK_PER_LAYER + j; }
static int rec_expert(int L, int e, int m) { return rec_layer(L, 9 + 3 * e + m); }

/* byte span [off, off + len) of record r inside its shard: part 0 = data, 1 = scales (ternary only) */
static int rec_span(const CkRec *r, int part, uint64_t *off, uint64_t *len) {
    if (r->kind == 't') {
        *off = part ? r->soff : r->off;
        *len = part ? (uint64_t)r->rows * 4 : (uint64_t)r->rows * r->cols / 4;
    } else {
        *off = r->off;
        *len = (uint64_t)r->rows * r->cols * 2;
    }
    return 0;
}

static int check_inside(const CkRec *r, int part, const char *what, int L) {
    uint64_t o, n;
    rec_span(r, part, &o, &n);
    if (r->file >= CK_NSHARD) return fail("layer %d %s: shard %d outside 0..8", L, what, r->file);
    if (o + n < o || o + n > C.size[r->file]) return fail("layer %d %s: bytes outside shard %d", L, what, r->file + 1);
    return 0;
}

int mmoe_ckpt_open(const char *dir) {
    char path[1024];
    mmoe_ckpt_close();
    for (int k = 0; k < CK_NSHARD; k++) {
        snprintf(path, sizeof path, "%s/shard-%05d.bin", dir, k + 1);
        if (map_file(path, &C.file[k], &C.size[k])) { mmoe_ckpt_close(); return -1; }
    }
    snprintf(path, sizeof path, "%s/layout.bin", dir);
    FILE *f = fopen(path, "rb");
    if (!f) { mmoe_ckpt_close(); return fail("cannot open %s", path); }
    size_t got = fread(C.rec, sizeof(CkRec), CK_NREC, f);
    fclose(f);
    if (got != CK_NREC) { mmoe_ckpt_close(); return fail("layout.bin too short: %zu of %d records", got, CK_NREC); }
    /* kinds, as maple.c:69-80 (GETB / GETT) */
    for (int i = 0; i < CK_NREC; i++) {
        int want_b = i < CK_GLOBAL || ((i - CK_GLOBAL) % CK_PER_LAYER) < 5;
        if (C.rec[i].kind != (want_b ? 'b' : 't')) {
            mmoe_ckpt_close();
            return fail("layout.bin record %d: expected %s", i, want_b ? "bf16" : "ternary");
        }
    }
    /* what the MoE path reads: shapes, bounds, 16-byte alignment */
    for (int L = 0; L < CK_NL; L++) {
        const CkRec *post = &C.rec[rec_layer(L, 1)], *router = &C.rec[rec_layer(L, 4)];
        int bad = 0;
        if ((uint64_t)post->rows * post->cols != CK_H) bad = fail("layer %d post_attention_layernorm: %u x %u", L, post->rows, post->cols);
        else if (router->rows != CK_NE || router->cols != CK_H) bad = fail("layer %d router: %u x %u", L, router->rows, router->cols);
        else if (check_inside(post, 0, "post_attention_layernorm", L) || check_inside(router, 0, "router", L)) bad = -1;
        for (int e = 0; e < CK_NE && !bad; e++)
            for (int m = 0; m < 3 && !bad; m++) {
                const CkRec *r = &C.rec[rec_expert(L, e, m)];
                uint32_t rows = m == 2 ? CK_H : CK_FF, cols = m == 2 ? CK_FF : CK_H;
                if (r->rows != rows || r->cols != cols)
                    bad = fail("layer %d expert %d %s: %u x %u, expected %u x %u", L, e, m == 0 ? "gate" : m == 1 ? "up" : "down",
                               r->rows, r->cols, rows, cols);
                else if (check_inside(r, 0, "expert codes", L) || check_inside(r, 1, "expert scales", L)) bad = -1;
                else if ((r->off & 15) || (r->soff & 15))
                    bad = fail("layer %d expert %d: tensor not 16-byte aligned in its shard", L, e);
            }
        if (bad) { mmoe_ckpt_close(); return -1; }
    }
    C.open = 1;
    return 0;
}

int mmoe_ckpt_layer_plan(int L, int shard[4], uint64_t lo[4], uint64_t len[4], uint32_t *loc) {
    if (!C.open) return fail("no checkpoint open");
    if (L < 0 || L >= CK_NL) return fail("layer %d outside 0..%d", L, CK_NL - 1);
    size_t pg = (size_t)getpagesize();
    uint64_t flo[CK_NSHARD], fhi[CK_NSHARD];
    int slot[CK_NSHARD], ns = 0;
    for (int k = 0; k < CK_NSHARD; k++) { flo[k] = UINT64_MAX; fhi[k] = 0; slot[k] = -1; }
    for (int e = 0; e < CK_NE; e++)
        for (int m = 0; m < 6; m++) {
            const CkRec *r = &C.rec[rec_expert(L, e, m / 2)];
            uint64_t o, n;
            rec_span(r, m % 2, &o, &n);
            if (o < flo[r->file]) flo[r->file] = o;
            if (o + n > fhi[r->file]) fhi[r->file] = o + n;
        }
    for (int k = 0; k < CK_NSHARD; k++) {
        if (!fhi[k]) continue;
        if (ns == 4) return fail("layer %d spans more than 4 shards", L);
        flo[k] = flo[k] / pg * pg;
        fhi[k] = (fhi[k] + pg - 1) / pg * pg;         /* within the mapping: it covers the file's last page whole */
        slot[k] = ns;
        shard[ns] = k; lo[ns] = flo[k]; len[ns] = fhi[k] - flo[k];
        ns++;
    }
    for (int j = ns; j < 4; j++) { shard[j] = -1; lo[j] = len[j] = 0; }
    if (loc)
        for (int e = 0; e < CK_NE; e++)
            for (int m = 0; m < 6; m++) {
                const CkRec *r = &C.rec[rec_expert(L, e, m / 2)];
                uint64_t o, n;
                rec_span(r, m % 2, &o, &n);
                loc[e * 12 + 2 * m] = (uint32_t)slot[r->file];
                loc[e * 12 + 2 * m + 1] = (uint32_t)(o - flo[r->file]);
            }
    return ns;
}

const uint16_t *mmoe_ckpt_bf16(int L, int which) {
    if (!C.open || L < 0 || L >= CK_NL || which < 0 || which > 4) return NULL;
    const CkRec *r = &C.rec[rec_layer(L, which)];
    return (const uint16_t *)(C.file[r->file] + r->off);
}

int mmoe_ckpt_load(int L0, int nl) {
    if (!C.open) return fail("no checkpoint open");
    if (L0 < 0 || nl < 1 || L0 + nl > CK_NL) return fail("layers %d..%d outside 0..%d", L0, L0 + nl - 1, CK_NL - 1);
    static uint32_t loc[CK_NE * 12];
    for (int L = L0; L < L0 + nl; L++) {
        int shard[4], regs[4];
        uint64_t lo[4], len[4];
        int ns = mmoe_ckpt_layer_plan(L, shard, lo, len, loc);
        if (ns < 0) return -1;
        for (int j = 0; j < 4; j++) {
            regs[j] = -1;
            if (j >= ns) continue;
            regs[j] = gpre_region(C.file[shard[j]] + lo[j], (size_t)len[j]);
            if (regs[j] < 0) return fail("layer %d: gpre_region: %s", L, mmoe_last_error());
        }
        if (mmoe_set_layer(L, loc, regs, mmoe_ckpt_bf16(L, 4), mmoe_ckpt_bf16(L, 1)))
            return fail("layer %d: mmoe_set_layer: %s", L, mmoe_last_error());
    }
    return 0;
}
