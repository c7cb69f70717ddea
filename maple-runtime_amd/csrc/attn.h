// attn.h -- the attention half of a Maple layer on the card (gfull_attn): per-head norms, rope and the fp16
// key/value cache, then causal grouped-query attention, for one sequence whose chunk of nb tokens sits at
// positions pos0 .. pos0+nb-1. The arithmetic follows maple.c's step_batch (maple.c:706-724) in the order
// the oracle's mo_attn_chunk fixes (oracle/moe_oracle.c), so the results equal the oracle's bit for bit:
//   head rmsnorm  maple.c:398-402 with n = 128: fp64 sum of squares in index order
//   rope          maple.c:403-411, in the FMA-contracted form maple.c's build computes
//   fp16 cache    maple.c:314-320, round to nearest even
//   attention     maple.c:516-558 (attend_group, AVX2 path): scores as 8 FMA lanes over the head dimension
//                 folded by hsum8, softmax with the library's exp and a sum in position order, output as an
//                 FMA chain over positions.
// Work split: scores and the weighted sum of values take groups of consecutive tokens of one key/value head per
// workgroup, so each cached key or value row is read once for the group and feeds all its query heads; a
// token's own window is enforced with a zero weight outside it (an FMA with weight 0 leaves a chain unchanged,
// exactly), so a group shares one loop over positions.
#pragma once
#include <hip/hip_fp16.h>
#include "kernels.h"

#define AT_HD 128
#define AT_QKV 3072   // q 16 x 128 | k 4 x 128 | v 4 x 128 per token
#define AT_XS 129     // LDS row stride of a head (a lane per head reads its own row without bank conflicts)

__device__ __forceinline__ int att_lo(int pos, int glob, int win) { return glob ? 0 : (pos - win > 0 ? pos - win : 0); }

// Raises *a to v (float maximum through integer atomics: non-negative floats order as signed integers,
// negative ones in reverse as unsigned integers).
__device__ __forceinline__ void atomic_max_f32(float *a, float v) {
    if (__float_as_int(v) >= 0) atomicMax((int *)a, __float_as_int(v));
    else atomicMin((unsigned int *)a, __float_as_uint(v));
}

// One workgroup per token b (it also sets the token's 16 score maxima to -1e30). q heads 0..15 and k heads 16..19 are normalised (q_norm / k_norm, sum of squares
// in fp64 in index order, one lane per head), roped on local layers (glob == 0); q stays fp32 in qkv, k and v
// go to the layer's cache kc/vc [position][512] and to ko[b][1024] (k | v) as fp16.
__global__ void __launch_bounds__(256) k_qkn(float *__restrict__ qkv, int pos0, int glob, const uint16_t *__restrict__ qn,
                                             const uint16_t *__restrict__ kn, const float *__restrict__ cs,
                                             __half *__restrict__ kc, __half *__restrict__ vc, __half *__restrict__ ko,
                                             float *__restrict__ mx) {
    __shared__ float xs[20 * AT_XS];
    __shared__ float kk[20];
    int b = blockIdx.x, t = threadIdx.x, pos = pos0 + b;
    float *row = qkv + (size_t)b * AT_QKV;
    if (t < 16) mx[b * 16 + t] = -1e30f;   // the score maxima k_att_scores raises
    // every element a thread ropes has dim t % 128 (elements t + 256 m): its cos / sin pair, loaded up front
    float rc = 0.0f, rsn = 0.0f;
    if (!glob && (t & 127) < 64) {
        float2 cv = *(const float2 *)(cs + ((size_t)pos * 32 + (t & 31)) * 2);
        rc = cv.x; rsn = cv.y;
    }
    {   // all of the thread's loads first (10 q/k values, 2 v values), then the LDS and cache stores
        float qk[10], vv[2];
#pragma unroll
        for (int m = 0; m < 10; m++) qk[m] = row[t + 256 * m];
#pragma unroll
        for (int m = 0; m < 2; m++) vv[m] = row[2560 + t + 256 * m];
#pragma unroll
        for (int m = 0; m < 10; m++) { int i = t + 256 * m; xs[(i >> 7) * AT_XS + (i & 127)] = qk[m]; }
#pragma unroll
        for (int m = 0; m < 2; m++) {
            int i = t + 256 * m;
            __half h = __float2half_rn(vv[m]);
            vc[(size_t)pos * 512 + i] = h; ko[(size_t)b * 1024 + 512 + i] = h;
        }
    }
    __syncthreads();
    if (t < 20) {
        const float *x = xs + t * AT_XS;
        double ss = 0.0;
        for (int i = 0; i < AT_HD; i++) ss += (double)x[i] * (double)x[i];
        kk[t] = 1.0f / sqrtf((float)(ss / (double)AT_HD) + 1e-6f);
    }
    __syncthreads();
    float y[10];   // elements t + 256 m of the 20 heads
#pragma unroll
    for (int m = 0; m < 10; m++) {
        int i = t + m * 256, h = i >> 7, d = i & 127;
        y[m] = xs[h * AT_XS + d] * kk[h] * bf16f((h < 16 ? qn : kn)[d]);
    }
    if (!glob) {   // rope on dims 0..63 of every head: pairs (i, i + 32)
        __syncthreads();
#pragma unroll
        for (int m = 0; m < 10; m++) { int i = t + m * 256; xs[(i >> 7) * AT_XS + (i & 127)] = y[m]; }
        __syncthreads();
#pragma unroll
        for (int m = 0; m < 10; m++) {
            int i = t + m * 256, h = i >> 7, d = i & 127;
            if (d >= 64) continue;
            if (d < 32) y[m] = __builtin_fmaf(y[m], rc, -(xs[h * AT_XS + d + 32] * rsn));
            else y[m] = __builtin_fmaf(y[m], rc, xs[h * AT_XS + d - 32] * rsn);
        }
    }
#pragma unroll
    for (int m = 0; m < 10; m++) {
        int i = t + m * 256;
        if (i < 2048) { row[i] = y[m]; continue; }
        __half h = __float2half_rn(y[m]);
        kc[(size_t)pos * 512 + i - 2048] = h; ko[(size_t)b * 1024 + i - 2048] = h;
    }
}

// Scores of the 4 query heads of key/value head kvh for a group of NB consecutive tokens (block x = (group,
// kvh)), one thread per cached position (block y = a run of 64 positions from the group's first window start):
// sc[(b * 16 + kvh * 4 + j) * ctx + p - lo_b] = hsum8(8 FMA lanes over the dims) * 1/sqrtf(128), for the tokens b
// whose window [lo_b, pos_b] holds p; mx[b * 16 + h] is raised to the row maximum. The q values are the same for
// every lane and are read with wave-uniform loads (scalar registers feed the FMAs).
template <int NB>
__global__ void __launch_bounds__(64) k_att_scores(const float *__restrict__ qkv, int nb, int pos0, int glob, int win,
                                                    const __half *__restrict__ kc, float *__restrict__ sc,
                                                    float *__restrict__ mx, int ctx) {
    int grp = blockIdx.x >> 2, kvh = blockIdx.x & 3, tid = threadIdx.x;
    int b0 = grp * NB, nbt = min(NB, nb - b0);
    int lo0 = att_lo(pos0 + b0, glob, win), phi = pos0 + b0 + nbt - 1, pstart = lo0 + blockIdx.y * 64;
    if (pstart > phi) return;   // the whole block past the group's last position
    int p = pstart + tid;
    const uint4 *kr = (const uint4 *)(kc + (size_t)min(p, phi) * 512 + kvh * AT_HD);
    const float *qb[NB];
#pragma unroll
    for (int bi = 0; bi < NB; bi++) qb[bi] = qkv + (size_t)min(b0 + bi, nb - 1) * AT_QKV + kvh * 4 * AT_HD;
    float a[NB][4][8];
#pragma unroll
    for (int bi = 0; bi < NB; bi++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int l = 0; l < 8; l++) a[bi][j][l] = 0.0f;
#pragma unroll 2
    for (int d8 = 0; d8 < AT_HD / 8; d8++) {
        uint4 u = kr[d8];
        const __half *hh = (const __half *)&u;
        float kf[8];
#pragma unroll
        for (int l = 0; l < 8; l++) kf[l] = __half2float(hh[l]);
#pragma unroll
        for (int bi = 0; bi < NB; bi++)
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int l = 0; l < 8; l++) a[bi][j][l] = __builtin_fmaf(kf[l], qb[bi][j * AT_HD + d8 * 8 + l], a[bi][j][l]);
    }
    const float scale = 1.0f / sqrtf((float)AT_HD);
    float mv[NB * 4];   // the 4 NB scores of this position, -1e30 outside a token's window
#pragma unroll
    for (int bi = 0; bi < NB; bi++) {
        int pb = pos0 + b0 + bi, lb = att_lo(pb, glob, win);
        bool in = bi < nbt && p >= lb && p <= pb;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float v = hsum8(a[bi][j]) * scale;
            if (in) sc[((size_t)(b0 + bi) * 16 + kvh * 4 + j) * ctx + p - lb] = v;
            mv[bi * 4 + j] = in ? v : -1e30f;
        }
    }
    // the maxima of the 8 rows (NB = 2) over the wave at once: lane-half swaps across lane bits 32 and 16 put
    // row k of both halves into one register pair (the lower half keeps rows 0..h-1, the upper rows h..2h-1),
    // then a rotation by 8 within 16-lane rows; then the maximum over each aligned group of 8 lanes
    static_assert(NB == 2, "the row-maximum exchange is written for 8 rows");
    int lane = tid & 63;
    float m4[4], m2[2];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mv[k]), __float_as_uint(mv[4 + k]), false, false);
        m4[k] = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    }
#pragma unroll
    for (int k = 0; k < 2; k++) {
        auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(m4[k]), __float_as_uint(m4[2 + k]), false, false);
        m2[k] = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    }
    float t0 = fmaxf(m2[0], __int_as_float(dpp<0x128>(__float_as_int(m2[0]))));   // row_ror:8: lane i gets lane i ^ 8
    float t1 = fmaxf(m2[1], __int_as_float(dpp<0x128>(__float_as_int(m2[1]))));
    float m = (lane & 8) ? t1 : t0;
    int r = ((lane >> 5) & 1) * 4 + ((lane >> 4) & 1) * 2 + ((lane >> 3) & 1);
    m = fmaxf(m, __int_as_float(dpp<0xB1>(__float_as_int(m))));    // quad xor 1
    m = fmaxf(m, __int_as_float(dpp<0x4E>(__float_as_int(m))));    // quad xor 2
    m = fmaxf(m, __int_as_float(dpp<0x12C>(__float_as_int(m))));   // row_ror:12: lane i gets lane i + 4 of its 16-lane row
    if ((lane & 7) == 0 && (r >> 2) < nbt) atomic_max_f32(mx + (b0 + (r >> 2)) * 16 + kvh * 4 + (r & 3), m);
}

// Softmax sums of the 16 rows (heads) of token b, one workgroup per token: p = exp(s - max) (max from
// k_att_scores), summed in position order by 16 lanes of wave 0 (one row each); inv[b * 16 + h] = 1 / sum.
// k_att_pv recomputes the same p. Waves 1-3 produce the p of 64-position chunks into two LDS buffers while
// wave 0 sums the previous chunk, and load the raw scores one chunk further ahead into registers, so the
// serial sums (the critical path) never wait for a load or an exp.
#define AT_SMCH 64
#define AT_SMPT ((16 * AT_SMCH + 191) / 192)   // p values per producer thread and chunk
__global__ void __launch_bounds__(256) k_att_softmax(int pos0, int glob, int win, const float *__restrict__ sc,
                                                     const float *__restrict__ mx, float *__restrict__ inv, int ctx) {
    constexpr int LD = AT_SMCH + 4;   // 16-byte aligned rows; the 16 summing lanes hit distinct bank groups
    __shared__ __attribute__((aligned(16))) float pl[2][16 * LD];
    __shared__ float smx[16];
    int b = blockIdx.x, tid = threadIdx.x, pos = pos0 + b;
    int T = pos - att_lo(pos, glob, win) + 1, nch = (T + AT_SMCH - 1) / AT_SMCH;
    const float *rows = sc + (size_t)b * 16 * ctx;
    const float *mr = mx + b * 16;
    int pt = tid - 64;                 // producer index (waves 1-3)
    float sv[AT_SMPT];                 // raw scores of the next chunk to produce
    auto load = [&](int c0) {
#pragma unroll
        for (int k = 0; k < AT_SMPT; k++) {
            int i = pt + 192 * k, r = i / AT_SMCH, p = i % AT_SMCH;
            sv[k] = (i < 16 * AT_SMCH && c0 + p < T) ? rows[(size_t)r * ctx + c0 + p] : 0.0f;
        }
    };
    auto produce = [&](float *buf) {
#pragma unroll
        for (int k = 0; k < AT_SMPT; k++) {
            int i = pt + 192 * k;
            if (i < 16 * AT_SMCH) buf[(i / AT_SMCH) * LD + i % AT_SMCH] = dexp(sv[k] - smx[i / AT_SMCH]);
        }
    };
    if (tid < 16) smx[tid] = mr[tid];
    if (pt >= 0) load(0);
    __syncthreads();
    if (pt >= 0) {
        produce(pl[0]);
        if (nch > 1) load(AT_SMCH);
    }
    __syncthreads();
    float sum = 0.0f;
    for (int c = 0; c < nch; c++) {
        if (pt >= 0) {
            if (c + 1 < nch) produce(pl[(c + 1) & 1]);
            if (c + 2 < nch) load((c + 2) * AT_SMCH);
        } else if (tid < 16) {   // in position order; 16 values are read ahead of their additions
            int n = min(AT_SMCH, T - c * AT_SMCH);
            const float *q = pl[c & 1] + tid * LD;
            const float4 *q4 = (const float4 *)q;
            int t = 0;
            for (; t + 16 <= n; t += 16) {
                float4 a = q4[t / 4], bq = q4[t / 4 + 1], cq = q4[t / 4 + 2], d = q4[t / 4 + 3];
                sum += a.x; sum += a.y; sum += a.z; sum += a.w; sum += bq.x; sum += bq.y; sum += bq.z; sum += bq.w;
                sum += cq.x; sum += cq.y; sum += cq.z; sum += cq.w; sum += d.x; sum += d.y; sum += d.z; sum += d.w;
            }
            for (; t < n; t++) sum += q[t];
        }
        __syncthreads();
    }
    if (tid < 16) inv[b * 16 + tid] = 1.0f / sum;
}

// Output of a group of NB consecutive tokens for key/value head kvh (block = (group, kvh), groups with the
// longest windows first): wave j is query head kvh * 4 + j, lane l dims 2l and 2l + 1. Per run of positions
// (512 / NB, at most 128) the weights w = exp(s - max) * inv of the group's tokens are staged in LDS (0 outside a token's window; the
// next run's are loaded into registers while the current one is consumed) and each output is the FMA chain over
// positions of w * v, into att[b][2048].
template <int NB>
__global__ void __launch_bounds__(256) k_att_pv(int nb, int pos0, int glob, int win, const float *__restrict__ sc,
                                                const float *__restrict__ mx, const float *__restrict__ inv, const __half *__restrict__ vc,
                                                float *__restrict__ att, int ctx) {
    constexpr int AT_PVCH = NB >= 4 ? 512 / NB : 128;   // positions per staged run
    constexpr int PER = 4 * NB * AT_PVCH / 256;       // staged weights per thread (8, or 4 for NB = 2)
    __shared__ __attribute__((aligned(16))) float wl[4][AT_PVCH][NB];
    int ngrp = (nb + NB - 1) / NB;
    int grp = ngrp - 1 - (int)(blockIdx.x >> 2), kvh = blockIdx.x & 3;
    int tid = threadIdx.x, j = tid >> 6, lane = tid & 63;
    int b0 = grp * NB, nbt = min(NB, nb - b0);
    int lo0 = att_lo(pos0 + b0, glob, win), phi = pos0 + b0 + nbt - 1;
    const uint32_t *vp = (const uint32_t *)(vc + kvh * AT_HD) + lane;   // dims 2 lane, 2 lane + 1 (256 words a position)
    // the staging slots of this thread: i = tid + 256 k -> (jj, bi, tt), tt fastest (coalesced rows of sc)
    const float *src[PER];
    int lbk[PER], pbk[PER];
    float ivk[PER], mxk[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        int i = tid + 256 * k, tt = i % AT_PVCH, bi = (i / AT_PVCH) % NB, jj = i / (AT_PVCH * NB);
        int pb = pos0 + b0 + bi, lb = att_lo(pb, glob, win), r = (b0 + bi) * 16 + kvh * 4 + jj;
        bool ok = bi < nbt;
        pbk[k] = ok ? pb : -1; lbk[k] = ok ? lb : 1 << 30;
        src[k] = sc + (size_t)(ok ? r : 0) * ctx - lb + tt;   // + p0 gives the entry of position p0 + tt
        ivk[k] = ok ? inv[r] : 0.0f; mxk[k] = ok ? mx[r] : 0.0f;
    }
    // the raw scores of a run are loaded together (out-of-window slots read a valid address and are zeroed
    // later) and turned into weights only after the current run's FMAs, so their latency hides behind them
    float raw[PER];
    auto load = [&](int p0) {
#pragma unroll
        for (int k = 0; k < PER; k++) {
            int p = p0 + (tid + 256 * k) % AT_PVCH;
            raw[k] = *((p >= lbk[k] && p <= pbk[k]) ? src[k] + p0 : sc);
        }
    };
    auto weights = [&](int p0, float *w) {
#pragma unroll
        for (int k = 0; k < PER; k++) {
            int p = p0 + (tid + 256 * k) % AT_PVCH;
            w[k] = (p >= lbk[k] && p <= pbk[k]) ? dexp(raw[k] - mxk[k]) * ivk[k] : 0.0f;
        }
    };
    float acc[NB][2];
#pragma unroll
    for (int bi = 0; bi < NB; bi++) acc[bi][0] = acc[bi][1] = 0.0f;
    float wn[PER];
    load(lo0);
    weights(lo0, wn);
    for (int p0 = lo0; p0 <= phi; p0 += AT_PVCH) {
        __syncthreads();
#pragma unroll
        for (int k = 0; k < PER; k++) {
            int i = tid + 256 * k, tt = i % AT_PVCH, bi = (i / AT_PVCH) % NB, jj = i / (AT_PVCH * NB);
            wl[jj][tt][bi] = wn[k];
        }
        __syncthreads();
        const bool more = p0 + AT_PVCH <= phi;
        if (more) load(p0 + AT_PVCH);
        int n = min(AT_PVCH, phi + 1 - p0);
        const uint32_t *vr = vp + (size_t)p0 * 256;
#pragma unroll 8
        for (int tt = 0; tt < n; tt++) {
            uint32_t h2 = vr[(size_t)tt * 256];
            float v0 = __half2float(__ushort_as_half((unsigned short)(h2 & 0xffff)));
            float v1 = __half2float(__ushort_as_half((unsigned short)(h2 >> 16)));
#pragma unroll
            for (int bi = 0; bi < NB; bi++) {
                float w = wl[j][tt][bi];
                acc[bi][0] = __builtin_fmaf(w, v0, acc[bi][0]);
                acc[bi][1] = __builtin_fmaf(w, v1, acc[bi][1]);
            }
        }
        if (more) weights(p0 + AT_PVCH, wn);
    }
#pragma unroll
    for (int bi = 0; bi < NB; bi++)
        if (bi < nbt) *(float2 *)(att + (size_t)(b0 + bi) * MH + (kvh * 4 + j) * AT_HD + 2 * lane) = make_float2(acc[bi][0], acc[bi][1]);
}
