// decode.h -- the MoE layer for small batches (decode: 1..8 tokens) in three kernels per layer.
//
// Decode reads each used expert's codes once per token step and is bound by memory latency, not by MFMA
// throughput: 8 experts of one token are 6.4 MB of codes, less than what the GPU keeps in flight. What costs
// time is the number of dependent steps, so the layer is three launches and no block waits for another
// inside a launch (device-scope fences that would publish data between blocks flush L2 on this part):
//   k_dec_route   rmsnorm (optional) + router logits in maple.c's FMA-chain order, from a chain-order copy
//                 of the router so every thread issues all its loads at once
//   k_dec_gateup  every block first repeats the small routing step (softmax/top-8 and the grouping of
//                 maple.c:924-938 for <= 8 tokens, the int8 quantisation of its tokens), then computes its
//                 gate/up rows as a GEMV (codes decoded in registers, v_dot4 on int8) and SiLU * up.
//                 Block (0, 0) also publishes the routing for the next kernel and for checks.
//   k_dec_down    every block re-quantises the act vectors (maple.c:832), then a wave computes 8 down rows
//                 over all used experts and runs the combine chain in maple.c's order into the hidden state.
// Results are bit-identical to the grouped-GEMM path and the oracle: same integer sums, same fp32 sequence.
#pragma once
#include "kernels.h"

#define DEC_MAXTOK 8
#define DEC_MAXP (DEC_MAXTOK * MTOPK)  // 64 pairs
#define DEC_GS 144                      // LDS bytes per 128-column group of int8 vectors (16 bytes padding)
#define DEC_HP 4                        // LDS floats of padding per router chain

__device__ __forceinline__ int dot16(const uint32_t *c, const uint32_t *q, int acc) {
#pragma unroll
    for (int i = 0; i < 16; i++) acc = __builtin_amdgcn_sdot4((int)c[i], (int)q[i], acc, false);
    return acc;
}
__device__ __forceinline__ void decode4(uint32_t w, uint32_t *o) {
    const uint32_t M = 0x03030303u;
    o[0] = w & M; o[1] = (w >> 2) & M; o[2] = (w >> 4) & M; o[3] = (w >> 6) & M;
}

// ---------------------------------------------------------------------------------------------------------
// Router logits. One wave per block, 64/NCH experts per block (grid = MNE*NCH/64), lane = (expert, chain j):
// chain j of expert e runs over columns j, j+NCH, ... (NCH = 16: maple.c:146-157, step; NCH = 8:
// maple.c:853-889, batch). wc is the router in chain order (k_router_chainmajor: word q of chain j holds its steps
// 8q .. 8q+7, the words q of an expert's NCH chains side by side); a lane
// issues all loads of its chain at kernel start and keeps them in registers for every token. hn sits in
// LDS in the same chain-major order (padded against bank conflicts). do_norm: hn = rmsnorm(x, post_ln)
// (maple.c:398-402, as k_rmsnorm), else hn = x. Block 0 writes hn.
// ---------------------------------------------------------------------------------------------------------
template <int NCH>
__global__ void __launch_bounds__(64) k_dec_route(const float *__restrict__ x, int nb, const uint16_t *__restrict__ post_ln, int do_norm,
                                                  const uint16_t *__restrict__ wc, const float *__restrict__ bias,
                                                  float *__restrict__ hn, float *__restrict__ rl) {
    constexpr int LEN = MH / NCH;                     // chain length
    __shared__ __attribute__((aligned(16))) float hs[NCH * (LEN + DEC_HP)];
    int l = threadIdx.x, j = l % NCH, e = blockIdx.x * (64 / NCH) + l / NCH;
    // token 0's x and the norm weights first, the router weights after them: loads return in issue order, so
    // the norm need not wait for the router weights (the scheduling barrier keeps that order)
    float4 x0[8];
#pragma unroll
    for (int i = 0; i < 8; i++) x0[i] = *(const float4 *)(x + 4 * l + 256 * i);
    uint2 pw[8];                                      // post_ln at columns 4l + 256i + 0..3
#pragma unroll
    for (int i = 0; i < 8; i++) pw[i] = (do_norm && post_ln) ? *(const uint2 *)(post_ln + 4 * l + 256 * i) : make_uint2(0x3f803f80u, 0x3f803f80u);
    __builtin_amdgcn_sched_barrier(0);
    const gptr_u4 *wp = (const gptr_u4 *)(wc + (size_t)e * MH + j * 8);   // 16 bytes i of the chain at wp[i * NCH]
    v4i wv[LEN / 8];
#pragma unroll
    for (int i = 0; i < LEN / 8; i++) wv[i] = wp[i * NCH];
    float lw[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        uint2 pv = pw[i];
        lw[4 * i] = bf16f(pv.x & 0xffff); lw[4 * i + 1] = bf16f(pv.x >> 16); lw[4 * i + 2] = bf16f(pv.y & 0xffff); lw[4 * i + 3] = bf16f(pv.y >> 16);
    }
    float bv = bias && j == 0 ? bias[e] : 0.0f;
    for (int b = 0; b < nb; b++) {
        const float *xb = x + (size_t)b * MH;
        float v[32]; double ss = 0.0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float4 f = b == 0 ? x0[i] : *(const float4 *)(xb + 4 * l + 256 * i);
            v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
        }
        if (do_norm) {
            double s4[4] = {0.0, 0.0, 0.0, 0.0};     // squares are exact in fp64; only the additions round
#pragma unroll
            for (int i = 0; i < 32; i++) s4[i & 3] += (double)v[i] * (double)v[i];
            ss = (s4[0] + s4[1]) + (s4[2] + s4[3]);
            ss = wave_sum_d(ss);
            float k = 1.0f / sqrtf((float)(ss / (double)MH) + 1e-6f);
#pragma unroll
            for (int i = 0; i < 32; i++) v[i] = v[i] * k * lw[i];
        }
        __syncthreads();                              // previous token's chains are done with hs
#pragma unroll
        for (int i = 0; i < 32; i++) { int c = 4 * l + 256 * (i >> 2) + (i & 3); hs[(c % NCH) * (LEN + DEC_HP) + c / NCH] = v[i]; }
        if (blockIdx.x == 0)
#pragma unroll
            for (int i = 0; i < 8; i++) *(float4 *)(hn + (size_t)b * MH + 4 * l + 256 * i) = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
        __syncthreads();
        const float *hc = hs + j * (LEN + DEC_HP);
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < LEN / 8; i++) {
            float4 h0 = *(const float4 *)(hc + 8 * i), h1 = *(const float4 *)(hc + 8 * i + 4);
            uint32_t q0 = (uint32_t)wv[i].x, q1 = (uint32_t)wv[i].y, q2 = (uint32_t)wv[i].z, q3 = (uint32_t)wv[i].w;
            acc = __builtin_fmaf(__uint_as_float(q0 << 16), h0.x, acc); acc = __builtin_fmaf(__uint_as_float(q0 & 0xffff0000u), h0.y, acc);
            acc = __builtin_fmaf(__uint_as_float(q1 << 16), h0.z, acc); acc = __builtin_fmaf(__uint_as_float(q1 & 0xffff0000u), h0.w, acc);
            acc = __builtin_fmaf(__uint_as_float(q2 << 16), h1.x, acc); acc = __builtin_fmaf(__uint_as_float(q2 & 0xffff0000u), h1.y, acc);
            acc = __builtin_fmaf(__uint_as_float(q3 << 16), h1.z, acc); acc = __builtin_fmaf(__uint_as_float(q3 & 0xffff0000u), h1.w, acc);
        }
        float r = hsum8_lanes<NCH>(acc);
        if (j == 0) {
            if (bias) r = r + bv;
            rl[(size_t)b * MNE + e] = r;
        }
    }
}

// The router in chain order for the kernels that run maple.c's FMA chains (NCH chains per expert, chain j over
// columns j, j + NCH, j + 2 NCH, ...): wc[e][q][j][t] = w[e][j + NCH (8 q + t)]. Steps 8q .. 8q+7 of chain j are
// one 16-byte word, and the words of step group q of all NCH chains are contiguous, so when lane j of a group of
// NCH lanes loads its chain's word q, the group reads NCH x 16 contiguous bytes.
template <int NCH>
__global__ void k_router_chainmajor(const uint16_t *__restrict__ w, uint16_t *__restrict__ wc) {
    int i = blockIdx.x * 256 + threadIdx.x;      // over 256 * 2048 elements of wc
    int e = i / MH, r = i % MH, q = r / (NCH * 8), j = (r / 8) % NCH, t = r % 8;
    wc[i] = w[(size_t)e * MH + j + NCH * (8 * q + t)];
}

// Grouping of the nb <= 8 tokens' top-8 (R.top) by one wave of the block, the counting sort of
// maple.c:924-938 (experts ascending, stable in token order) computed per pair from counts. Results in LDS: nu, ue, ustart, utok, uw, sp (slot -> pair), tp (pair ids of a token ascending).
struct DecRoute {
    int top[DEC_MAXP]; float tw[DEC_MAXP];
    int nu, ue[DEC_MAXP], ustart[DEC_MAXP + 1];
    int utok[DEC_MAXP]; float uw[DEC_MAXP]; int sp[DEC_MAXP], tp[DEC_MAXP];
};
__device__ void dec_group_block(int nb, DecRoute &R) {
    int t = threadIdx.x, P = nb * MTOPK;
    if (t < 64) {                                     // one wave, lane i = pair i (P <= 64)
        int i = t, e = i < P ? R.top[i] : 0x7fffffff, cl = 0, ce = 0;
        for (int j0 = 0; j0 < P; j0 += MTOPK) {       // P is a multiple of 8: 8 LDS reads issued together
            int ej[MTOPK];
#pragma unroll
            for (int k = 0; k < MTOPK; k++) ej[k] = R.top[j0 + k];
#pragma unroll
            for (int k = 0; k < MTOPK; k++) { cl += ej[k] < e; ce += (j0 + k < i) & (ej[k] == e); }
        }
        bool first = i < P && ce == 0;
        unsigned long long fm = __ballot(first);
        int du = 0;
        for (int j0 = 0; j0 < P; j0 += MTOPK) {
            int ej[MTOPK];
#pragma unroll
            for (int k = 0; k < MTOPK; k++) ej[k] = R.top[j0 + k];
#pragma unroll
            for (int k = 0; k < MTOPK; k++) du += (int)((fm >> (j0 + k)) & 1) & (ej[k] < e);
        }
        int slot = cl + ce;                           // experts ascending, tokens ascending within one
        if (first) { R.ue[du] = e; R.ustart[du] = cl; }
        if (i == 0) { R.nu = popc64(fm); R.ustart[popc64(fm)] = P; }
        if (i < P) { R.utok[slot] = i / MTOPK; R.uw[slot] = R.tw[i]; R.sp[i] = slot; }
        // tp: a token's slots ascending (maple.c:1018-1019); the 8 pairs of a token are lanes 8b..8b+7
        int rank = 0;
#pragma unroll
        for (int k = 0; k < MTOPK; k++) rank += __shfl(slot, (i & ~(MTOPK - 1)) + k, 64) < slot;
        if (i < P) R.tp[(i & ~(MTOPK - 1)) + rank] = slot;
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------------------------------------
// Gate/up GEMV. grid (64 row blocks of 8 rows, 8*nb expert slots); block 256. Every block routes (above);
// slot u >= nu exits. Waves 0-1: gate rows, 2-3: up rows; 16 lanes per row, a lane = one 128-column group
// (8 code words). Block (0, 0) publishes the routing (top, tw, plan, utok, uw, tp, sp, eptr, qx, qsx, qsumx).
// ---------------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_dec_gateup(const float *__restrict__ rl, const float *__restrict__ hn, int nb,
                                                    const ExpPtr *__restrict__ layer_tab, int *__restrict__ top,
                                                    float *__restrict__ tw, Plan *__restrict__ plan, int *__restrict__ utok,
                                                    float *__restrict__ uw, int *__restrict__ tp, int *__restrict__ sp,
                                                    ExpPtr *__restrict__ eptr, int8_t *__restrict__ qx, float *__restrict__ qsx,
                                                    int *__restrict__ qsumx, float *__restrict__ act, int *__restrict__ dbg) {
    __shared__ DecRoute R;
    __shared__ __attribute__((aligned(16))) float E[4][MNE];
    __shared__ __attribute__((aligned(16))) float Pl[MNE];   // one token: p of every expert (wave 2)
    __shared__ __attribute__((aligned(16))) int8_t qs_l[DEC_MAXTOK][MH / 128 * DEC_GS];
    __shared__ float qsv_l[DEC_MAXTOK];
    __shared__ int qsum_l[DEC_MAXTOK];
    __shared__ int sums[2][8][DEC_MAXTOK];
    __shared__ float sgu[2][8];
    __shared__ __attribute__((aligned(16))) ExpPtr tab[MNE];
    int t = threadIdx.x, wv = t >> 6, l = t & 63;
    static_assert(sizeof(ExpPtr) == 48, "ExpPtr: 6 pointers");
    const v4i *ltp = (const v4i *)(layer_tab + t);   // the layer's expert table, stored to LDS after top-8 (three
    v4i my0 = ltp[0], my1 = ltp[1], my2 = ltp[2];     // vectors: held as a struct it went to scratch memory)

    // one token: the 8 picks are selected on the logits (wave 0) while wave 2 computes the softmax and wave 1
    // quantises x; p = exp(l - max) / sum is non-decreasing in l, so after the barrier a check against p proves the
    // selection is maple.c's (below), and only a token that fails it (ties in p) runs the selection on p again.
    // More tokens: top-8 (topk_wave) and quantisation (maple.c:908-923) of every token, spread over waves.
    if (nb == 1) {
        if (wv == 0) {
            v4f lv = *(const gptr_f4 *)(rl + 4 * l);
            int ek[MTOPK];
            topk_logit_rounds(make_float4(lv.x, lv.y, lv.z, lv.w), l, ek);
            if (l < MTOPK) {   // the one-token grouping: picks in ascending expert order (pair = rank)
                int e = 0, rank = 0;
#pragma unroll
                for (int k = 0; k < MTOPK; k++) e = l == k ? ek[k] : e;
#pragma unroll
                for (int k = 0; k < MTOPK; k++) rank += ek[k] < e;
                R.top[l] = e; R.ue[rank] = e; R.ustart[rank] = rank; R.utok[rank] = 0; R.sp[l] = rank; R.tp[rank] = rank;
                if (l == 0) { R.nu = MTOPK; R.ustart[MTOPK] = MTOPK; }
            }
        } else if (wv == 1) {
            quant_wave<MH, DEC_GS - 128>(hn, l, qs_l[0], &qsv_l[0], &qsum_l[0]);
        } else if (wv == 2) {
            v4f lv = *(const gptr_f4 *)(rl + 4 * l);
            float pv[4];
            softmax_wave(make_float4(lv.x, lv.y, lv.z, lv.w), E[2], l, pv);
            *(float4 *)(&Pl[4 * l]) = make_float4(pv[0], pv[1], pv[2], pv[3]);
        }
    } else {
        for (int it = wv; it < 2 * nb; it += 4) {
            if (it < nb) topk_wave(rl + (size_t)it * MNE, E[wv], l, R.top + it * MTOPK, R.tw + it * MTOPK);
            else quant_wave<MH, DEC_GS - 128>(hn + (size_t)(it - nb) * MH, l, qs_l[it - nb], &qsv_l[it - nb], &qsum_l[it - nb]);
        }
    }
    { v4i *tp4 = (v4i *)(tab + t); tp4[0] = my0; tp4[1] = my1; tp4[2] = my2; }
    __syncthreads();
    int u = blockIdx.y;
    int kind = wv >> 1, rr = (wv & 1) * 4 + (l >> 4), grp = l & 15;
    int r0 = blockIdx.x * 8, row = r0 + rr;
    v4i c0, c1;
    float srow = 0.0f;   // row scales, loaded with the codes (one load per thread: no wait between two)
    // the block's gate/up codes: for one token the grouping is written by the top-8 wave (its 8 picks ascending),
    // so slot u's expert is R.ue[u] right after the barrier; for more tokens after dec_group_block
    auto load_codes = [&](int e) {
        const ExpPtr &ex = tab[e];
        const gptr_u4 *cp = (const gptr_u4 *)((kind ? ex.uc : ex.gc) + (size_t)row * (MH / 4) + grp * 32);
        c0 = cp[0]; c1 = cp[1];
        if (t < 16) srow = *(const gptr_f *)(t < 8 ? ex.gs + r0 + t : ex.us + r0 + t - 8);
    };
    if (nb == 1) {
        load_codes(R.ue[u]);   // slot u = the u-th pick in ascending expert order (above)
        // the check, by every thread alike: with the picks s_0..s_7 in logit order, p(s_0) > ... > p(s_7) and every
        // other expert's p < p(s_7) mean the 8 largest p are s_0..s_7 in that order with no ties, i.e. maple.c's
        // picks; otherwise (a tie in p) the selection runs again on p keys (topk_wave) and the codes are reloaded
        int sk[MTOPK]; float ps[MTOPK];
#pragma unroll
        for (int k = 0; k < MTOPK; k++) sk[k] = R.top[k];
        if (!picks_exact(sk, Pl, l, ps)) {   // uniform: every wave computes the same values
            __syncthreads();                  // all reads of R.top above are done
            if (wv == 0) {
                v4f lv = *(const gptr_f4 *)(rl + 4 * l);
                topk_wave_v(make_float4(lv.x, lv.y, lv.z, lv.w), E[0], l, R.top, R.tw);
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                if (l < MTOPK) {
                    int e = R.top[l], rank = 0;
#pragma unroll
                    for (int j = 0; j < MTOPK; j++) rank += R.top[j] < e;
                    R.ue[rank] = e; R.uw[rank] = R.tw[l]; R.sp[l] = rank;
                }
            }
            __syncthreads();
            load_codes(R.ue[u]);
        } else if (blockIdx.x == 0 && blockIdx.y == 0) {   // the publishing block: weights in pick order
            if (wv == 0 && l < MTOPK) {
                float tsum = 0.0f;
#pragma unroll
                for (int k = 0; k < MTOPK; k++) tsum = tsum + ps[k];
                float w = 0.0f;
#pragma unroll
                for (int k = 0; k < MTOPK; k++) w = l == k ? ps[k] : w;
                w = w / (tsum + 1e-20f);
                R.tw[l] = w; R.uw[R.sp[l]] = w;
            }
            __syncthreads();
        }
    } else {
        dec_group_block(nb, R);
    }
    bool pub = blockIdx.x == 0 && blockIdx.y == 0;
    if (u >= R.nu && !pub) return;                    // whole block
    if (pub) {
        int P = nb * MTOPK;
        if (t < P) { top[t] = R.top[t]; tw[t] = R.tw[t]; utok[t] = R.utok[t]; uw[t] = R.uw[t]; tp[t] = R.tp[t]; sp[t] = R.sp[t]; }
        if (t < R.nu) { plan->ue[t] = R.ue[t]; plan->ustart[t] = R.ustart[t]; eptr[t] = tab[R.ue[t]]; }
        if (t == 0) { plan->nu = R.nu; plan->np = P; plan->ustart[R.nu] = P; plan->tn = 16; }
        for (int bb = 0; bb < nb; bb++) {
            for (int i = t; i < MH / 16; i += 256) *(uint4 *)(qx + (size_t)bb * MH + i * 16) = *(const uint4 *)(&qs_l[bb][(i >> 3) * DEC_GS + (i & 7) * 16]);
            if (t == 0) { qsx[bb] = qsv_l[bb]; qsumx[bb] = qsum_l[bb]; }
        }
        if (u >= R.nu) return;
    }
    if (nb != 1) load_codes(R.ue[u]);
    uint32_t cd[32];
    uint32_t cwd[8] = {(uint32_t)c0.x, (uint32_t)c0.y, (uint32_t)c0.z, (uint32_t)c0.w, (uint32_t)c1.x, (uint32_t)c1.y, (uint32_t)c1.z, (uint32_t)c1.w};
#pragma unroll
    for (int k = 0; k < 8; k++) decode4(cwd[k], cd + 4 * k);
    int a0 = R.ustart[u], n = R.ustart[u + 1] - a0;
    for (int i = 0; i < n; i++) {
        int tok = R.utok[a0 + i];
        const uint32_t *qd = (const uint32_t *)(&qs_l[tok][grp * DEC_GS]);
        int acc = 0;
#pragma unroll
        for (int k = 0; k < 32; k++) acc = __builtin_amdgcn_sdot4((int)cd[k], (int)qd[k], acc, false);
        acc += dpp<0xB1>(acc); acc += dpp<0x4E>(acc); acc += dpp<0x141>(acc); acc += dpp<0x140>(acc);   // 16-lane row sum
        if (grp == 0) sums[kind][rr][i] = acc;
    }
    if (t < 16) sgu[t >> 3][t & 7] = srow;
    __syncthreads();
    if (t < n * 8) {
        int i = t >> 3, r8 = t & 7, a = a0 + i, tok = R.utok[a];
        float qs = qsv_l[tok]; int qsum = qsum_l[tok];
        int ag = sums[0][r8][i], au = sums[1][r8][i];
        float gv = (float)(ag - qsum) * qs * sgu[0][r8];
        float uv = (float)(au - qsum) * qs * sgu[1][r8];
        float g = gv < 7.0f ? gv : 7.0f;
        float uu = uv < -7.0f ? -7.0f : (uv > 7.0f ? 7.0f : uv);
        act[(size_t)a * MFF + r0 + r8] = g / (1.0f + dexp(-g)) * uu;
        if (dbg) { dbg[(size_t)a * 2 * MFF + r0 + r8] = ag; dbg[(size_t)a * 2 * MFF + MFF + r0 + r8] = au; }
    }
}

// ---------------------------------------------------------------------------------------------------------
// Down GEMV + combine. grid = 2048 / 8 row blocks of 256 threads. Every block quantises all act vectors into
// LDS (wave w takes pairs 8k + 2w, 8k + 2w + 1; block 0 also publishes them). Wave w computes the 8 rows for
// the used experts u = w, w+4, ... (lane = row l/8, 64-column slice l%8); its code vectors are loaded while
// the act vectors are quantised. Last, thread (token, row) runs the combine chain: mode 6 = step
// (maple.c:664), mode 1 = step_batch (maple.c:834), as k_combine.
// ---------------------------------------------------------------------------------------------------------
#define DEC_DU (DEC_MAXP / 4)   // experts per wave
struct ActChunk { float v[16]; };
// lanes 0-31 load vector a0 = a, lanes 32-63 the vector the caller passes for them; lane = 16-column chunk
__device__ __forceinline__ void act_load(const float *__restrict__ act, int a, int l, ActChunk &c) {
    int o = l & 31, g = o >> 3, h = (o >> 2) & 1, tq = o & 3;
    const float *xr = act + (size_t)a * MFF;
#pragma unroll
    for (int s = 0; s < 4; s++) {
        float4 f = *(const float4 *)(xr + g * 128 + s * 32 + h * 16 + tq * 4);
        c.v[s * 4] = f.x; c.v[s * 4 + 1] = f.y; c.v[s * 4 + 2] = f.z; c.v[s * 4 + 3] = f.w;
    }
}
__global__ void __launch_bounds__(256) k_dec_down(const Plan *__restrict__ plan, const ExpPtr *__restrict__ eptr,
                                                  const float *__restrict__ act, int8_t *__restrict__ qa_out, float *__restrict__ qsa_out,
                                                  int *__restrict__ qsuma_out, const int *__restrict__ tp, const int *__restrict__ sp,
                                                  const float *__restrict__ uw, const float *__restrict__ tw, int nb,
                                                  float *__restrict__ x, int mode, float *__restrict__ down, int *__restrict__ dbg) {
    __shared__ float Dl[DEC_MAXP][8];
    __shared__ __attribute__((aligned(16))) int8_t qa[DEC_MAXP][MFF / 128 * DEC_GS];
    __shared__ float qsa[DEC_MAXP];
    __shared__ int qsuma[DEC_MAXP];
    int t = threadIdx.x, wv = t >> 6, l = t & 63, rr = l >> 3, sl = l & 7;
    int r0 = blockIdx.x * 8, row = r0 + rr;
    ActChunk c0;
    act_load(act, 2 * wv + (l >> 5), l, c0);          // first act vectors, issued before anything else
    int nu = plan->nu;
    // expert pointers through scalar loads (the wave index made provably uniform), so the code loads that use
    // them wait on those loads only and not on the act loads issued before
    int wvu = __builtin_amdgcn_readfirstlane(wv);
    // the combine's inputs (thread (token, row) < nb * 8): the hidden-state value and the token's 8 pair ids and
    // weights, loaded now so the combine at the end waits for nothing
    int cb = t >> 3, cr8 = t & 7, ca[MTOPK]; float cw[MTOPK], cx = 0.0f;
    float *cxp = x + (size_t)cb * MH + r0 + cr8;
    if (t < nb * 8) {
        cx = *cxp;
#pragma unroll
        for (int jj = 0; jj < MTOPK; jj++) {
            ca[jj] = (mode & 2) ? sp[cb * MTOPK + jj] : tp[cb * MTOPK + jj];
            cw[jj] = (mode & 2) ? tw[cb * MTOPK + jj] : uw[ca[jj]];
        }
    }
    int us0[2], us1[2];   // ustart of the wave's first two experts (scalar loads; clamped like the pointers)
#pragma unroll
    for (int k = 0; k < 2; k++) { us0[k] = plan->ustart[wvu + 4 * k]; us1[k] = plan->ustart[wvu + 4 * k + 1]; }
    v4i cv[DEC_DU]; float sd[DEC_DU];
    // the first two experts of the wave (all of them for one token, nu <= 8) unconditionally, a slot past nu
    // reading expert 0's rows instead (never used), so the pointer and code loads are issued back to back
    const uint8_t *dc0 = eptr[0].dc; const float *ds0 = eptr[0].ds;
#pragma unroll
    for (int k = 0; k < 2; k++) {   // entry and plan->nu loaded together, the pointer picked after
        const uint8_t *dc = eptr[wvu + 4 * k].dc; const float *ds = eptr[wvu + 4 * k].ds;
        bool live = wvu + 4 * k < nu;
        dc = live ? dc : dc0; ds = live ? ds : ds0;
        cv[k] = *(const gptr_u4 *)(dc + (size_t)row * (MFF / 4) + sl * 16); sd[k] = *(const gptr_f *)(ds + row);
    }
#pragma unroll
    for (int k = 2; k < DEC_DU; k++)
        if (wvu + 4 * k < nu) {
            const ExpPtr &ep = eptr[wvu + 4 * k];
            cv[k] = *(const gptr_u4 *)(ep.dc + (size_t)row * (MFF / 4) + sl * 16); sd[k] = *(const gptr_f *)(ep.ds + row);
        }
    for (int k = 0; k < nb; k++) {
        int a = 8 * k + 2 * wv + (l >> 5);
        if (k > 0) act_load(act, a, l, c0);
        quant_half<DEC_GS>(c0.v, l, qa[a], &qsa[a], &qsuma[a]);
    }
    __syncthreads();
    if (blockIdx.x == 0)
        for (int a = wv; a < nb * MTOPK; a += 4) {
            if (l < MFF / 16) *(uint4 *)(qa_out + (size_t)a * MFF + l * 16) = *(const uint4 *)(&qa[a][(l >> 3) * DEC_GS + (l & 7) * 16]);
            if (l == 0) { qsa_out[a] = qsa[a]; qsuma_out[a] = qsuma[a]; }
        }
#pragma unroll
    for (int k = 0; k < DEC_DU; k++) {
        int u = wvu + 4 * k;
        if (u >= nu) break;
        uint32_t cd[16];
        decode4((uint32_t)cv[k].x, cd); decode4((uint32_t)cv[k].y, cd + 4); decode4((uint32_t)cv[k].z, cd + 8); decode4((uint32_t)cv[k].w, cd + 12);
        int a0 = k < 2 ? us0[k] : plan->ustart[u], a1 = k < 2 ? us1[k] : plan->ustart[u + 1];
        for (int a = a0; a < a1; a++) {
            const uint32_t *qd = (const uint32_t *)(&qa[a][(sl >> 1) * DEC_GS + (sl & 1) * 64]);
            int acc = dot16(cd, qd, 0);
            acc += dpp<0xB1>(acc); acc += dpp<0x4E>(acc); acc += dpp<0x141>(acc);   // the 8 lanes of the row half
            if (sl == 0) {
                float d = (float)(acc - qsuma[a]) * qsa[a] * sd[k];
                Dl[a][rr] = d;
                if (dbg) { down[(size_t)a * MH + row] = d; dbg[(size_t)a * MH + row] = acc; }   // checks only
            }
        }
    }
    __syncthreads();
    if (t < nb * 8) {
        float acc = (mode & 1) ? cx : 0.0f;
#pragma unroll
        for (int jj = 0; jj < MTOPK; jj++) acc = __builtin_fmaf(cw[jj], Dl[ca[jj]][cr8], acc);
        if (mode & 4) acc = cx + acc;
        *cxp = acc;
    }
}
