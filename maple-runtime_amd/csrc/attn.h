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
// These kernels are correctness-first: one thread per score and per output element, no MFMA.
#pragma once
#include <hip/hip_fp16.h>
#include "kernels.h"

#define AT_HD 128
#define AT_QKV 3072   // q 16 x 128 | k 4 x 128 | v 4 x 128 per token

// One wave per (token b, head h): h < 16 query heads, 16..19 key heads, 20..23 value heads. q/k heads are
// normalised (q_norm / k_norm), roped on local layers (glob == 0); q stays fp32 in qkv, k and v go to the
// layer's cache kc/vc [position][512] and to ko[b][1024] (k | v) as fp16.
__global__ void __launch_bounds__(64) k_qkn(float *__restrict__ qkv, int pos0, int glob, const uint16_t *__restrict__ qn,
                                            const uint16_t *__restrict__ kn, const float *__restrict__ cs,
                                            __half *__restrict__ kc, __half *__restrict__ vc, __half *__restrict__ ko) {
    __shared__ float xs[AT_HD];
    __shared__ float kk;
    int b = blockIdx.x, h = blockIdx.y, l = threadIdx.x, pos = pos0 + b;
    float *src = qkv + (size_t)b * AT_QKV + h * AT_HD;   // q 0..2047, k 2048..2559, v 2560..3071
    float a0 = src[l], a1 = src[l + 64];
    if (h >= 20) {
        int c = (h - 20) * AT_HD;
        __half h0 = __float2half_rn(a0), h1 = __float2half_rn(a1);
        vc[(size_t)pos * 512 + c + l] = h0; vc[(size_t)pos * 512 + c + l + 64] = h1;
        ko[(size_t)b * 1024 + 512 + c + l] = h0; ko[(size_t)b * 1024 + 512 + c + l + 64] = h1;
        return;
    }
    xs[l] = a0; xs[l + 64] = a1;
    __syncthreads();
    if (l == 0) {
        double ss = 0.0;
        for (int i = 0; i < AT_HD; i++) ss += (double)xs[i] * (double)xs[i];
        kk = 1.0f / sqrtf((float)(ss / (double)AT_HD) + 1e-6f);
    }
    __syncthreads();
    float k = kk;
    const uint16_t *w = h < 16 ? qn : kn;
    a0 = a0 * k * bf16f(w[l]); a1 = a1 * k * bf16f(w[l + 64]);
    if (!glob) {   // rope on dims 0..63 (lane l holds dim l in a0): pairs (i, i + 32)
        __syncthreads();
        xs[l] = a0;
        __syncthreads();
        int i = l & 31;
        float c = cs[((size_t)pos * 32 + i) * 2], s = cs[((size_t)pos * 32 + i) * 2 + 1];
        if (l < 32) a0 = __builtin_fmaf(a0, c, -(xs[l + 32] * s));
        else a0 = __builtin_fmaf(a0, c, xs[l - 32] * s);
    }
    if (h < 16) { src[l] = a0; src[l + 64] = a1; return; }
    int c = (h - 16) * AT_HD;
    __half h0 = __float2half_rn(a0), h1 = __float2half_rn(a1);
    kc[(size_t)pos * 512 + c + l] = h0; kc[(size_t)pos * 512 + c + l + 64] = h1;
    ko[(size_t)b * 1024 + c + l] = h0; ko[(size_t)b * 1024 + c + l + 64] = h1;
}

__device__ __forceinline__ int att_lo(int pos, int glob, int win) { return glob ? 0 : (pos - win > 0 ? pos - win : 0); }

// Scores of the 4 query heads of key/value head kvh of token b (block = (b, kvh), thread = position t):
// sc[(b * 16 + kvh * 4 + j) * ctx + t - lo] = hsum8(8 FMA lanes over the dims) * 1/sqrtf(128).
__global__ void __launch_bounds__(256) k_att_scores(const float *__restrict__ qkv, int pos0, int glob, int win,
                                                    const __half *__restrict__ kc, float *__restrict__ sc, int ctx) {
    __shared__ float qs[4][AT_HD];
    int b = blockIdx.x >> 2, kvh = blockIdx.x & 3, tid = threadIdx.x, pos = pos0 + b;
    int lo = att_lo(pos, glob, win), T = pos - lo + 1;
    for (int i = tid; i < 4 * AT_HD; i += 256) qs[i >> 7][i & 127] = qkv[(size_t)b * AT_QKV + (kvh * 4 + (i >> 7)) * AT_HD + (i & 127)];
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)AT_HD);
    for (int t = tid; t < T; t += 256) {
        const uint4 *kr = (const uint4 *)(kc + (size_t)(lo + t) * 512 + kvh * AT_HD);
        float a[4][8];
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int l = 0; l < 8; l++) a[j][l] = 0.0f;
#pragma unroll 4
        for (int d8 = 0; d8 < AT_HD / 8; d8++) {
            uint4 u = kr[d8];
            const __half *hh = (const __half *)&u;
            float kf[8];
#pragma unroll
            for (int l = 0; l < 8; l++) kf[l] = __half2float(hh[l]);
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int l = 0; l < 8; l++) a[j][l] = __builtin_fmaf(kf[l], qs[j][d8 * 8 + l], a[j][l]);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) sc[((size_t)b * 16 + kvh * 4 + j) * ctx + t] = hsum8(a[j]) * scale;
    }
}

// Per (token, head) row r = b * 16 + head: max over the row, p = exp(s - max) in place, the sum in position
// order (lane 0 over LDS chunks), inv[r] = 1 / sum.
#define AT_SMCH 1024
__global__ void __launch_bounds__(64) k_att_softmax(int pos0, int glob, int win, float *__restrict__ sc,
                                                    float *__restrict__ inv, int ctx) {
    __shared__ float pl[AT_SMCH];
    int r = blockIdx.x, b = r >> 4, l = threadIdx.x, pos = pos0 + b;
    int T = pos - att_lo(pos, glob, win) + 1;
    float *row = sc + (size_t)r * ctx;
    float mx = -1e30f;
    for (int t = l; t < T; t += 64) mx = fmaxf(mx, row[t]);
    mx = wave_max(mx);
    float sum = 0.0f;
    for (int c0 = 0; c0 < T; c0 += AT_SMCH) {
        int n = min(AT_SMCH, T - c0);
        for (int t = l; t < n; t += 64) { float p = dexp(row[c0 + t] - mx); row[c0 + t] = p; pl[t] = p; }
        __syncthreads();
        if (l == 0) for (int t = 0; t < n; t++) sum += pl[t];
        __syncthreads();
    }
    if (l == 0) inv[r] = 1.0f / sum;
}

// Output of head (kvh * 4 + j), dim d of token b (block = (b, kvh), thread = (j, d)): the FMA chain over
// positions of (p * inv) * v, into att[b][2048].
__global__ void __launch_bounds__(512) k_att_pv(int pos0, int glob, int win, const float *__restrict__ sc,
                                                const float *__restrict__ inv, const __half *__restrict__ vc,
                                                float *__restrict__ att, int ctx) {
    int b = blockIdx.x >> 2, kvh = blockIdx.x & 3, tid = threadIdx.x, j = tid >> 7, d = tid & 127, pos = pos0 + b;
    int lo = att_lo(pos, glob, win), T = pos - lo + 1;
    int r = b * 16 + kvh * 4 + j;
    const float *p = sc + (size_t)r * ctx;
    const __half *v = vc + (size_t)lo * 512 + kvh * AT_HD + d;
    float iv = inv[r], o = 0.0f;
#pragma unroll 8
    for (int t = 0; t < T; t++) o = __builtin_fmaf(p[t] * iv, __half2float(v[(size_t)t * 512]), o);
    att[(size_t)b * MH + (kvh * 4 + j) * AT_HD + d] = o;
}
