// kernels.h -- gfx950 (CDNA4) kernels of the Maple MoE hot path. Included by mmoe.hip only.
//
// Data layouts in HBM (shapes of maple.c:21-30: H = 2048, NE = 256, TOPK = 8, FF = 512):
//   expert codes      the reference's packed layout, unchanged (convert.py:29-33): rows of cols/4 bytes,
//                     128-column groups of 32 bytes, byte j holding columns j, j+32, j+64, j+96 at bits
//                     0,2,4,6, code c = w+1 in {0,1,2}; one fp32 scale per row. Read in place from the
//                     regions (gpre_region) or expert slots (gpux_upload).
//   int8 activations  "mfma order": within each 128-column group, column s*32 + h*16 + t*4 + b is stored at
//                     byte h*64 + t*16 + s*4 + b (s,t,b in 0..3, h in 0..1). Then the 16 bytes one MFMA lane
//                     needs for one code dword are contiguous (see the gate/up kernel).
//   pairs             (token, expert) assignments grouped by expert exactly as maple.c:924-938: used experts
//                     ascending, tokens ascending inside an expert; ustart[u] is the first pair of used expert u.
//
// Integer work (quantisation, code*q sums, routing indices, grouping) is exact. Floating-point work follows
// the fixed IEEE operation sequence of the C oracle: no FMA contraction (-ffp-contract=off), explicit fmaf where
// maple.c's AVX2 build has an FMA, correctly rounded division and sqrt.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define MH 2048
#define MNE 256
#define MTOPK 8
#define MFF 512

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(1))) v4i gptr_u4;   // global-memory 16 bytes (global_load, not flat_load)
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) v4f gptr_f4;
typedef __attribute__((address_space(1))) float gptr_f;      // global-memory float

struct ExpPtr {  // one expert's six tensors (maple.c:276-277 GLOC order: gate codes/scales, up, down)
    const uint8_t *gc; const float *gs;
    const uint8_t *uc; const float *us;
    const uint8_t *dc; const float *ds;
};

// Plan of one grouped launch, written on the device by the grouping kernels (or from a host grouping).
struct Plan {
    int nu;                 // used experts
    int np;                 // pairs
    int ntile_gu;           // token tiles of the gate/up GEMM (sum over u of ceil(cnt_u / TN))
    int tn;                 // token-tile width the tile starts were computed for
    int ue[MNE];            // used expert -> expert id
    int ustart[MNE + 1];    // pair offsets
    int tstart[MNE + 1];    // token-tile offsets
};
// One token tile of a grouped launch: used expert, first pair, pairs in the tile (<= TN)
struct Tile { int u, p0, n, pad; };

__device__ __forceinline__ float bf16f(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }

// exp in fp32 arithmetic: k = rint(x * log2(e)), r = x - k ln2 with ln2 split in two (two FMAs), Taylor
// series to r^7 by Horner with FMA, times 2^k in two exponent-field steps. Overflow gives inf, x < -104
// gives 0. Identical operation-for-operation to the oracle's mo_exp.
__device__ __forceinline__ float pow2i(int k) { return __uint_as_float((uint32_t)(k + 127) << 23); }
__device__ __forceinline__ float dexp(float x) {
    if (x > 88.8f) return __int_as_float(0x7f800000);
    if (x < -104.0f) return 0.0f;
    float k = __builtin_rintf(x * 1.44269504f);
    float r = __builtin_fmaf(-k, 0.693145752f, x);
    r = __builtin_fmaf(-k, 1.42860677e-06f, r);
    float p = 1.98412698e-04f;
    p = __builtin_fmaf(p, r, 1.38888889e-03f);
    p = __builtin_fmaf(p, r, 8.33333333e-03f);
    p = __builtin_fmaf(p, r, 4.16666667e-02f);
    p = __builtin_fmaf(p, r, 1.66666667e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    // p 2^k, k in [-150, 128]. The oracle forms it as (p 2^(k/2)) 2^(k - k/2); the first product is exact,
    // so both round once, identically.
    return __builtin_amdgcn_ldexpf(p, (int)k);
}

// SiLU of a gate value g <= 7: g / (1 + dexp(-g)), bit-identical to that expression with IEEE division
// (mmoe_selftest_silu checks every finite g <= 7). For -g <= 80 the quotient is a refined reciprocal
// y = rcp(d) + one Newton step, q = g y, then one residual correction q += (g - d q) y (Markstein's
// scheme); d = 1 + e lies in [1, 2^116] there, so y stays a normal number. -g > 80 (rare) takes the IEEE
// division, with dexp's overflow to +inf (g / inf = -0).
__device__ __forceinline__ float silu_le7(float g) {
    float x = fminf(-g, 88.8f);
    float k = __builtin_rintf(x * 1.44269504f);
    float r = __builtin_fmaf(-k, 0.693145752f, x);
    r = __builtin_fmaf(-k, 1.42860677e-06f, r);
    float p = 1.98412698e-04f;
    p = __builtin_fmaf(p, r, 1.38888889e-03f);
    p = __builtin_fmaf(p, r, 8.33333333e-03f);
    p = __builtin_fmaf(p, r, 4.16666667e-02f);
    p = __builtin_fmaf(p, r, 1.66666667e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    float e = __builtin_amdgcn_ldexpf(p, (int)k);   // = p 2^k1 2^k2 of dexp (one rounding either way)
    float d = 1.0f + e;
    if (__builtin_expect(-g > 80.0f, 0)) return g / (-g > 88.8f ? __int_as_float(0x7f800000) : d);
    float y = __builtin_amdgcn_rcpf(d);
    y = __builtin_fmaf(__builtin_fmaf(-d, y, 1.0f), y, y);
    float q = g * y;
    // the correction turns g = -0 into +0; d > 0, so the quotient carries the sign of g
    return __builtin_copysignf(__builtin_fmaf(__builtin_fmaf(-d, q, g), y, q), g);
}

// Exhaustive check of silu_le7 against g / (1 + dexp(-g)): thread i tests bit patterns lo + i + n * stride.
__global__ void k_selftest_silu(uint32_t lo, uint32_t n, unsigned long long *nbad, uint32_t *first) {
    unsigned long long bad = 0;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        float g = __uint_as_float(lo + i);
        float a = silu_le7(g), b = g / (1.0f + dexp(-g));
        if (__float_as_uint(a) != __float_as_uint(b)) { bad++; atomicMin(first, lo + i); }
    }
    if (bad) atomicAdd(nbad, bad);
}

// ---- wave64 reductions (order-free operations only: max, integer sum). DPP inside each 16-lane row
// (quad swaps, half-row mirror, row mirror), then the four row results are read as scalars. The whole wave
// must be active.
template <int CTRL> __device__ __forceinline__ int dpp(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false); }
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, __int_as_float(dpp<0xB1>(__float_as_int(v))));    // quad_perm [1,0,3,2]
    v = fmaxf(v, __int_as_float(dpp<0x4E>(__float_as_int(v))));    // quad_perm [2,3,0,1]
    v = fmaxf(v, __int_as_float(dpp<0x141>(__float_as_int(v))));   // row_half_mirror
    v = fmaxf(v, __int_as_float(dpp<0x140>(__float_as_int(v))));   // row_mirror
    int b = __float_as_int(v);
    float r0 = __int_as_float(__builtin_amdgcn_readlane(b, 0)), r1 = __int_as_float(__builtin_amdgcn_readlane(b, 16));
    float r2 = __int_as_float(__builtin_amdgcn_readlane(b, 32)), r3 = __int_as_float(__builtin_amdgcn_readlane(b, 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
// sum over the wave in an arbitrary fixed order (used only where the order does not matter: bounds)
__device__ __forceinline__ float wave_sumf(float v) {
    v = v + __int_as_float(dpp<0xB1>(__float_as_int(v)));
    v = v + __int_as_float(dpp<0x4E>(__float_as_int(v)));
    v = v + __int_as_float(dpp<0x141>(__float_as_int(v)));
    v = v + __int_as_float(dpp<0x140>(__float_as_int(v)));
    int b = __float_as_int(v);
    float r0 = __int_as_float(__builtin_amdgcn_readlane(b, 0)), r1 = __int_as_float(__builtin_amdgcn_readlane(b, 16));
    float r2 = __int_as_float(__builtin_amdgcn_readlane(b, 32)), r3 = __int_as_float(__builtin_amdgcn_readlane(b, 48));
    return (r0 + r1) + (r2 + r3);
}
__device__ __forceinline__ int wave_sum_i(int v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    v += dpp<0x140>(v);
    return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) + __builtin_amdgcn_readlane(v, 32) +
           __builtin_amdgcn_readlane(v, 48);
}
__device__ __forceinline__ int popc64(unsigned long long m) { return __popcll(m); }
// fp64 sum over the wave (DPP on both halves of each double; the order is fixed, not maple.c's)
template <int CTRL> __device__ __forceinline__ double dpp_d(double v) {
    unsigned long long b = __double_as_longlong(v);
    int hi = dpp<CTRL>((int)(b >> 32)), lo = dpp<CTRL>((int)(uint32_t)b);
    return __longlong_as_double((long long)(((unsigned long long)(uint32_t)hi << 32) | (uint32_t)lo));
}
__device__ __forceinline__ double wave_sum_d(double v) {
    v += dpp_d<0xB1>(v); v += dpp_d<0x4E>(v); v += dpp_d<0x141>(v); v += dpp_d<0x140>(v);
    unsigned long long b = __double_as_longlong(v);
    double r[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t hi = __builtin_amdgcn_readlane((int)(b >> 32), 16 * i), lo = __builtin_amdgcn_readlane((int)(uint32_t)b, 16 * i);
        r[i] = __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
    }
    return (r[0] + r[1]) + (r[2] + r[3]);
}

// =====================================================================================================
// RMSNorm, maple.c:398-402: k = 1 / sqrtf((float)(sum x^2 / n) + 1e-6), out = x * k * w. The sum of squares
// is in fp64 as in maple.c; each square is exact in fp64, so only the fp64 additions depend on order.
// One block of 256 threads per row.
// =====================================================================================================
__global__ void __launch_bounds__(256) k_rmsnorm(const float *__restrict__ x, const uint16_t *__restrict__ w,
                                                  float *__restrict__ out, int nb) {
    __shared__ double red[256];
    __shared__ float kk;
    int b = blockIdx.x, t = threadIdx.x;
    const float *xr = x + (size_t)b * MH;
    float v[8]; double s = 0.0;
    for (int i = 0; i < 8; i++) { v[i] = xr[t + i * 256]; s += (double)v[i] * (double)v[i]; }
    red[t] = s;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) { if (t < o) red[t] += red[t + o]; __syncthreads(); }
    if (t == 0) kk = 1.0f / sqrtf((float)(red[0] / (double)MH) + 1e-6f);
    __syncthreads();
    float k = kk;
    float *o = out + (size_t)b * MH;
    for (int i = 0; i < 8; i++) { float wv = w ? bf16f(w[t + i * 256]) : 1.0f; o[t + i * 256] = v[i] * k * wv; }
}

// =====================================================================================================
// Router logits, maple.c:853-889 (batch, NCH = 8) and maple.c:146-157 (decode bf_row, NCH = 16).
// A logit is NCH independent FMA chains: chain j runs over columns j, j+NCH, j+2NCH, ... in order,
// acc = fma(w, x, acc). Batch: v[j] = chain j; decode: v[j] = chain j + chain j+8. Then
// ((v0+v4)+(v1+v5)) + ((v2+v6)+(v3+v7)) (maple.c:111-115 hsum). Bias (optional) is added last.
// =====================================================================================================
__device__ __forceinline__ float hsum8(const float *v) {
    float a0 = v[0] + v[4], a1 = v[1] + v[5], a2 = v[2] + v[6], a3 = v[3] + v[7];
    return (a0 + a1) + (a2 + a3);
}
// The same fold over the chain values of NCH (16 or 8) consecutive lanes of one 16-lane row, one value per
// lane (16 chains first pair chain i with chain i + 8, as the step router does): DPP row shifts pair the same
// operands as hsum8 (row_ror:8, then row_shl:4, 1, 2: lane i adds lane i + n), so the group's first lane holds
// hsum8's result bit for bit. Every lane of the row must be active.
template <int NCH>
__device__ __forceinline__ float hsum8_lanes(float v) {
    if (NCH == 16) v = v + __int_as_float(dpp<0x128>(__float_as_int(v)));   // row_ror:8
    v = v + __int_as_float(dpp<0x104>(__float_as_int(v)));                   // row_shl:4
    v = v + __int_as_float(dpp<0x101>(__float_as_int(v)));                   // row_shl:1
    return v + __int_as_float(dpp<0x102>(__float_as_int(v)));                // row_shl:2
}

// Mid-size batches: one thread per (expert, chain) of one token, block = 256/NCH experts of token
// blockIdx.y. The token's row sits in LDS chain-major (hc[j][m] = hn[j + NCH m]) and the router comes from
// its chain-order copy (wc[e][q][j][t] = w[e][j + NCH (8 q + t)], k_router_chainmajor), so the NCH lanes of an
// expert read NCH x 16 contiguous bytes per load; its loads are
// issued 16 at a time ahead of the FMAs. Chain j runs over columns j, j + NCH, ... with fma(w, x, acc); the
// chains are then folded as described above (NCH = 16: chain j + chain j+8 first).
// NORM: `in` is the hidden state x and the block first forms hn = rmsnorm(x, post_ln) for its token with
// exactly k_rmsnorm's arithmetic (thread t sums columns t, t+256, ... in fp64, then the same 256-wide tree);
// blocks with blockIdx.x == 0 write hn to hn_out. Else `in` is hn.
// the top-8 / quantisation outputs of a router launch that also routes its tokens (TK); defined further down:
struct RouteTail { int *top; float *tw; int8_t *qx; float *qsx; int *qsumx; int *hist; int *cnt; };
__device__ __forceinline__ int topk_wave(const float *__restrict__ r, float *E, int l, int *__restrict__ top, float *__restrict__ tw);

template <int N, int GPAD = 0>
__device__ __forceinline__ void quant_wave(const float *__restrict__ xr, int l, int8_t *__restrict__ q, float *__restrict__ qs,
                                           int *__restrict__ qsum);
template <int NCH, bool NORM = false, bool TK = false>
__global__ void __launch_bounds__(256) k_router_chains(const float *__restrict__ in, int nb, const uint16_t *__restrict__ wc,
                                                       const float *__restrict__ bias, float *__restrict__ rl,
                                                       const uint16_t *__restrict__ post_ln = nullptr, float *__restrict__ hn_out = nullptr,
                                                       RouteTail tail = RouteTail{}) {
    constexpr int LEN = MH / NCH, HP = LEN + 4;
    __shared__ __attribute__((aligned(16))) float hc[NCH * HP];
    __shared__ double red[NORM ? 256 : 1];
    __shared__ float kk;
    // TK: a 1-D grid in which the NCH blocks of token b (expert groups y) all get ids = b mod 8, i.e. run on
    // XCD b mod 8 (workgroup ids go to the 8 XCDs round robin) and share its L2; else grid (NCH, nb)
    int b = TK ? (int)(blockIdx.x / (8 * NCH)) * 8 + (int)(blockIdx.x % 8) : (int)blockIdx.y;
    int y = TK ? (int)(blockIdx.x / 8) % NCH : (int)blockIdx.x;
    if (TK && b >= nb) return;   // whole block
    int tid = threadIdx.x, j = tid % NCH, e = y * (256 / NCH) + tid / NCH;
    const float *xr = in + (size_t)b * MH;
    float xv[8];
    uint32_t pw[8];   // bf16 bits, one per register (no packing between the loads and the barrier)
    if (NORM) {   // the token's x and norm weights first: loads return in issue order, so the norm need not
#pragma unroll    // wait for the router weights issued after them (the scheduling barrier keeps that order)
        for (int i = 0; i < 8; i++) xv[i] = xr[tid + i * 256];
        if (post_ln) {
#pragma unroll
            for (int i = 0; i < 8; i++) pw[i] = post_ln[tid + i * 256];
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) pw[i] = 0x3f80;   // bf16 1.0
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    const gptr_u4 *wp = (const gptr_u4 *)(wc + (size_t)e * MH + j * 8);   // 16 bytes q of the chain at wp[q * NCH]
    v4i wv[16];
#pragma unroll
    for (int q = 0; q < 16; q++) wv[q] = wp[q * NCH];
    float be = 0.0f;
    if (bias && j == 0) be = bias[e];   // with the weights' loads, added at the end
    if (NORM) {
        double sq = 0.0;
#pragma unroll
        for (int i = 0; i < 8; i++) sq += (double)xv[i] * (double)xv[i];
        red[tid] = sq;
        __syncthreads();
        for (int o = 128; o > 0; o >>= 1) { if (tid < o) red[tid] += red[tid + o]; __syncthreads(); }
        if (tid == 0) kk = 1.0f / sqrtf((float)(red[0] / (double)MH) + 1e-6f);
        __syncthreads();
        float k = kk;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            int c = tid + i * 256;
            float wn = __uint_as_float(pw[i] << 16);
            float h = xv[i] * k * wn;
            hc[(c % NCH) * HP + c / NCH] = h;
            if (y == 0) hn_out[(size_t)b * MH + c] = h;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            int c = (tid + 256 * i) * 4;
            float4 f = *(const float4 *)(xr + c);
            hc[((c + 0) % NCH) * HP + (c + 0) / NCH] = f.x; hc[((c + 1) % NCH) * HP + (c + 1) / NCH] = f.y;
            hc[((c + 2) % NCH) * HP + (c + 2) / NCH] = f.z; hc[((c + 3) % NCH) * HP + (c + 3) / NCH] = f.w;
        }
    }
    __syncthreads();
    const float *h = hc + j * HP;
    float acc = 0.0f;
#pragma unroll
    for (int half = 0; half < LEN / 128; half++) {
        if (half > 0) {
#pragma unroll
            for (int q = 0; q < 16; q++) wv[q] = wp[(half * 16 + q) * NCH];
        }
#pragma unroll
        for (int q = 0; q < 16; q++) {
            float4 h0 = *(const float4 *)(h + half * 128 + q * 8), h1 = *(const float4 *)(h + half * 128 + q * 8 + 4);
            uint32_t q0 = (uint32_t)wv[q].x, q1 = (uint32_t)wv[q].y, q2 = (uint32_t)wv[q].z, q3 = (uint32_t)wv[q].w;
            acc = __builtin_fmaf(__uint_as_float(q0 << 16), h0.x, acc); acc = __builtin_fmaf(__uint_as_float(q0 & 0xffff0000u), h0.y, acc);
            acc = __builtin_fmaf(__uint_as_float(q1 << 16), h0.z, acc); acc = __builtin_fmaf(__uint_as_float(q1 & 0xffff0000u), h0.w, acc);
            acc = __builtin_fmaf(__uint_as_float(q2 << 16), h1.x, acc); acc = __builtin_fmaf(__uint_as_float(q2 & 0xffff0000u), h1.y, acc);
            acc = __builtin_fmaf(__uint_as_float(q3 << 16), h1.z, acc); acc = __builtin_fmaf(__uint_as_float(q3 & 0xffff0000u), h1.w, acc);
        }
    }
    float r = hsum8_lanes<NCH>(acc);
    if (j == 0) {
        if (bias) r = r + be;
        rl[(size_t)b * MNE + e] = r;
    }
    if (TK) {
        // the token's softmax/top-8 and int8 quantisation in the last of its NCH blocks to arrive: every block's
        // stores (logits; hn from block 0) reach the XCD's L2 before its arrival is counted, and the last one
        // reads them there (its L1 holds none of those lines: nothing in this kernel read them before)
        __shared__ int last;
        __shared__ __attribute__((aligned(16))) float E[MNE];
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) last = atomicAdd(&tail.cnt[b], 1) == NCH - 1;
        __syncthreads();
        if (!last) return;
        int wv = tid >> 6, l = tid & 63;
        if (wv == 0) {
            int ek = topk_wave(rl + (size_t)b * MNE, E, l, tail.top + b * MTOPK, tail.tw + b * MTOPK);
            if (tail.hist && l < MTOPK) atomicAdd(&tail.hist[(b >> 6) * MNE + ek], 1);   // per-chunk counts for k_group
        } else if (wv == 1) {
            const float *hr = (NORM ? hn_out : in) + (size_t)b * MH;
            quant_wave<MH>(hr, l, tail.qx + (size_t)b * MH, tail.qsx + b, tail.qsumx + b);
        } else if (tid == 128) {
            tail.cnt[b] = 0;   // for the next launch (every block of the token has counted)
        }
    }
}

// k_router_chains for two tokens per block (the TK form: top-8 and quantisation in the last block): every thread
// runs its chain for both tokens side by side from the same router words in registers, so a block reads its 32
// experts' weights once for two tokens (half the blocks, half the L2 traffic) and the two FMA chains are
// independent. Token pair q = (2q, 2q + 1) takes the NCH blocks with ids congruent to q mod 8 (one XCD). The
// arithmetic per token is k_router_chains' exactly (the rmsnorm of each token as k_rmsnorm, the chains, the fold).
template <int NCH, bool NORM>
__global__ void __launch_bounds__(256) k_router_chains2(const float *__restrict__ in, int nb, const uint16_t *__restrict__ wc,
                                                        const float *__restrict__ bias, float *__restrict__ rl,
                                                        const uint16_t *__restrict__ post_ln, float *__restrict__ hn_out,
                                                        RouteTail tail) {
    constexpr int LEN = MH / NCH, HP = LEN + 4;
    __shared__ __attribute__((aligned(16))) float hc[2][NCH * HP];
    __shared__ double red[NORM ? 2 : 1][NORM ? 256 : 1];
    __shared__ float kk[2];
    int q = (int)(blockIdx.x / (8 * NCH)) * 8 + (int)(blockIdx.x % 8);
    int y = (int)(blockIdx.x / 8) % NCH;
    int b0 = 2 * q;
    if (b0 >= nb) return;   // whole block
    const bool two = b0 + 1 < nb;
    int tid = threadIdx.x, j = tid % NCH, e = y * (256 / NCH) + tid / NCH;
    float xv[2][8];
    uint32_t pw[8];
    if (NORM) {
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const float *xr = in + (size_t)(two ? b0 + t : b0) * MH;
#pragma unroll
            for (int i = 0; i < 8; i++) xv[t][i] = xr[tid + i * 256];
        }
        if (post_ln) {
#pragma unroll
            for (int i = 0; i < 8; i++) pw[i] = post_ln[tid + i * 256];
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) pw[i] = 0x3f80;
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    const gptr_u4 *wp = (const gptr_u4 *)(wc + (size_t)e * MH + j * 8);
    v4i wv[16];
#pragma unroll
    for (int qq = 0; qq < 16; qq++) wv[qq] = wp[qq * NCH];
    float be = 0.0f;
    if (bias && j == 0) be = bias[e];
    if (NORM) {
#pragma unroll
        for (int t = 0; t < 2; t++) {
            double sq = 0.0;
#pragma unroll
            for (int i = 0; i < 8; i++) sq += (double)xv[t][i] * (double)xv[t][i];
            red[t][tid] = sq;
        }
        __syncthreads();
        for (int o = 128; o > 0; o >>= 1) {
            if (tid < o) { red[0][tid] += red[0][tid + o]; red[1][tid] += red[1][tid + o]; }
            __syncthreads();
        }
        if (tid < 2) kk[tid] = 1.0f / sqrtf((float)(red[tid][0] / (double)MH) + 1e-6f);
        __syncthreads();
#pragma unroll
        for (int t = 0; t < 2; t++) {
            float k = kk[t];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                int c = tid + i * 256;
                float h = xv[t][i] * k * __uint_as_float(pw[i] << 16);
                hc[t][(c % NCH) * HP + c / NCH] = h;
                if (y == 0 && (t == 0 || two)) hn_out[(size_t)(b0 + t) * MH + c] = h;
            }
        }
    } else {
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const float *xr = in + (size_t)(two ? b0 + t : b0) * MH;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                int c = (tid + 256 * i) * 4;
                float4 f = *(const float4 *)(xr + c);
                hc[t][((c + 0) % NCH) * HP + (c + 0) / NCH] = f.x; hc[t][((c + 1) % NCH) * HP + (c + 1) / NCH] = f.y;
                hc[t][((c + 2) % NCH) * HP + (c + 2) / NCH] = f.z; hc[t][((c + 3) % NCH) * HP + (c + 3) / NCH] = f.w;
            }
        }
    }
    __syncthreads();
    const float *h0p = hc[0] + j * HP, *h1p = hc[1] + j * HP;
    float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
    for (int half = 0; half < LEN / 128; half++) {
        if (half > 0) {
#pragma unroll
            for (int qq = 0; qq < 16; qq++) wv[qq] = wp[(half * 16 + qq) * NCH];
        }
#pragma unroll
        for (int qq = 0; qq < 16; qq++) {
            int o = half * 128 + qq * 8;
            float4 a0 = *(const float4 *)(h0p + o), a1 = *(const float4 *)(h0p + o + 4);
            float4 c0 = *(const float4 *)(h1p + o), c1 = *(const float4 *)(h1p + o + 4);
            uint32_t w4[4] = {(uint32_t)wv[qq].x, (uint32_t)wv[qq].y, (uint32_t)wv[qq].z, (uint32_t)wv[qq].w};
            float hv0[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w}, hv1[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
            for (int u = 0; u < 8; u++) {
                float wf = __uint_as_float((u & 1) ? (w4[u >> 1] & 0xffff0000u) : (w4[u >> 1] << 16));
                acc0 = __builtin_fmaf(wf, hv0[u], acc0);
                acc1 = __builtin_fmaf(wf, hv1[u], acc1);
            }
        }
    }
    float r0 = hsum8_lanes<NCH>(acc0), r1 = hsum8_lanes<NCH>(acc1);
    if (j == 0) {
        if (bias) { r0 = r0 + be; r1 = r1 + be; }
        rl[(size_t)b0 * MNE + e] = r0;
        if (two) rl[(size_t)(b0 + 1) * MNE + e] = r1;
    }
    // the pair's softmax/top-8 and quantisation in the last of its NCH blocks to arrive (as k_router_chains)
    __shared__ int last;
    __shared__ __attribute__((aligned(16))) float E[2][MNE];
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) last = atomicAdd(&tail.cnt[q], 1) == NCH - 1;
    __syncthreads();
    if (!last) return;
    int wvi = tid >> 6, l = tid & 63, t = wvi & 1, b = b0 + t;
    if (t == 1 && !two) return;   // whole wave
    if (wvi < 2) {
        int ek = topk_wave(rl + (size_t)b * MNE, E[t], l, tail.top + b * MTOPK, tail.tw + b * MTOPK);
        if (tail.hist && l < MTOPK) atomicAdd(&tail.hist[(b >> 6) * MNE + ek], 1);
    } else {
        const float *hr = (NORM ? hn_out : in) + (size_t)b * MH;
        quant_wave<MH>(hr, l, tail.qx + (size_t)b * MH, tail.qsx + b, tail.qsumx + b);
        if (tid == 128) tail.cnt[q] = 0;   // every block of the pair has counted
    }
}

// Large batches (batch order, NCH = 8) as a register-tiled GEMM that keeps maple.c's chains: one thread
// owns one chain j for a TPT-token x 8-expert tile (independent FMA chains in registers), a block
// covers 4 TPT tokens x 64 experts x 8 chains. Operands sit in LDS chain-major, hs[j][m][token] and
// ws[j][m][expert] for column j + 8m, so a chain step reads 2 + 2 16-byte words. The router comes
// pre-converted to fp32 in that order, wT[j][m][e] = w[e][j + 8m] (k_router_chain8_f32). Columns advance
// in chunks of RG_MC steps, the next chunk loaded into registers while the current one is used.
// After the last column the 8 chain values meet in LDS and are folded by hsum8.
#define RG_BE 64
#define RG_MC 16
__global__ void k_router_chain8_f32(const uint16_t *__restrict__ w, float *__restrict__ wT) {
    int i = blockIdx.x * 256 + threadIdx.x;          // over wT: [8][256][256]
    int j = i >> 16, m = (i >> 8) & 255, e = i & 255;
    wT[i] = bf16f(w[(size_t)e * MH + j + 8 * m]);
}
// TPT tokens per thread: the block covers BT = 4 TPT tokens (TPT = 4: 16 tokens, 512 blocks at T = 2048 and
// 32 accumulators per thread, so two or more waves share a SIMD).
template <int TPT>
__global__ void __launch_bounds__(256) k_router_gemm(const float *__restrict__ hn, int nb, const float *__restrict__ wT,
                                                     const float *__restrict__ bias, float *__restrict__ rl) {
    constexpr int BT = 4 * TPT, HP = BT + 4;        // tokens per block; token stride of hs (padded, 16-byte aligned)
    constexpr int NH = BT * 128 / 4 / 256;           // float4 pieces of the token chunk per thread
    constexpr int SM_CHUNK = 8 * RG_MC * HP + 8 * RG_MC * RG_BE, SM_RED = 8 * BT * RG_BE;
    __shared__ __attribute__((aligned(16))) float smem[SM_CHUNK > SM_RED ? SM_CHUNK : SM_RED];
    float *hs = smem, *ws = smem + 8 * RG_MC * HP;
    int t = threadIdx.x, j = t >> 5, tg = (t >> 3) & 3, eg = t & 7;
    int b0 = blockIdx.x * BT, e0 = blockIdx.y * RG_BE;
    static_assert(RG_BE == 64, "the output loop gives thread t expert e0 + t % 64 in every round");
    float be = 0.0f;
    if (bias) be = bias[e0 + (t & 63)];   // loaded at entry, added to the thread's logits at the end
    typedef float f4v __attribute__((ext_vector_type(4)));
    f4v hr[NH], wr[8];
    float acc[TPT][8];
#pragma unroll
    for (int a = 0; a < TPT; a++)
#pragma unroll
        for (int b = 0; b < 8; b++) acc[a][b] = 0.0f;
#define RG_LOAD(cn)                                                                                             \
    {                                                                                                           \
        _Pragma("unroll") for (int k = 0; k < NH; k++) {                                                        \
            int idx = t + 256 * k, b = idx >> 5, c4 = idx & 31;                                                 \
            hr[k] = *(const f4v *)(hn + (size_t)min(b0 + b, nb - 1) * MH + (cn) + 4 * c4);                      \
        }                                                                                                       \
        _Pragma("unroll") for (int k = 0; k < 8; k++) {                                                         \
            int idx = t + 256 * k, jj = idx >> 8, mm = (idx >> 4) & 15, e4 = idx & 15;                          \
            wr[k] = *(const f4v *)(wT + ((size_t)jj * 256 + (cn) / 8 + mm) * 256 + e0 + 4 * e4);                 \
        }                                                                                                       \
    }
    RG_LOAD(0);
    for (int c0 = 0; c0 < MH; c0 += 8 * RG_MC) {
        __syncthreads();                             // the previous chunk is no longer read
#pragma unroll
        for (int k = 0; k < NH; k++) {
            int idx = t + 256 * k, b = idx >> 5, c4 = idx & 31;
            int c = 4 * c4, base = (c >> 3) * HP + b, j0 = c & 7;
            hs[((j0 + 0) * RG_MC) * HP + base] = hr[k].x;
            hs[((j0 + 1) * RG_MC) * HP + base] = hr[k].y;
            hs[((j0 + 2) * RG_MC) * HP + base] = hr[k].z;
            hs[((j0 + 3) * RG_MC) * HP + base] = hr[k].w;
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            int idx = t + 256 * k, jj = idx >> 8, mm = (idx >> 4) & 15, e4 = idx & 15;
            *(f4v *)(ws + (jj * RG_MC + mm) * RG_BE + 4 * e4) = wr[k];
        }
        __syncthreads();
        if (c0 + 8 * RG_MC < MH) RG_LOAD(c0 + 8 * RG_MC);
#pragma unroll 4
        for (int m = 0; m < RG_MC; m++) {
            const float *hp = hs + (j * RG_MC + m) * HP + tg * TPT, *wp = ws + (j * RG_MC + m) * RG_BE + eg * 8;
            float hv[TPT];
#pragma unroll
            for (int a = 0; a < TPT; a += 4) { float4 h = *(const float4 *)(hp + a); hv[a] = h.x; hv[a + 1] = h.y; hv[a + 2] = h.z; hv[a + 3] = h.w; }
            float4 w0 = *(const float4 *)wp, w1 = *(const float4 *)(wp + 4);
            float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int a = 0; a < TPT; a++)
#pragma unroll
                for (int b = 0; b < 8; b++) acc[a][b] = __builtin_fmaf(wv[b], hv[a], acc[a][b]);
        }
    }
#undef RG_LOAD
    __syncthreads();
    float *red = smem;                               // red[j][token][expert]
#pragma unroll
    for (int a = 0; a < TPT; a++)
#pragma unroll
        for (int b = 0; b < 8; b += 4)
            *(float4 *)(red + (j * BT + tg * TPT + a) * RG_BE + eg * 8 + b) = make_float4(acc[a][b], acc[a][b + 1], acc[a][b + 2], acc[a][b + 3]);
    __syncthreads();
#pragma unroll
    for (int q = 0; q < BT * RG_BE / 256; q++) {
        int o = q * 256 + t, tok = o >> 6, e = o & 63;
        float v[8];
#pragma unroll
        for (int jj = 0; jj < 8; jj++) v[jj] = red[(jj * BT + tok) * RG_BE + e];
        float r = hsum8(v);
        if (bias) r = r + be;
        if (b0 + tok < nb) rl[(size_t)(b0 + tok) * MNE + e0 + e] = r;
    }
}

// Large batches, approximate logits on the bf16 MFMA + exact refinement (k_refine_topk).
// Each fp32 input h is split into bf16 parts by truncation: h1 = the top 8 significant bits of h, h2 = the top 8
// of h - h1 (both subtractions exact), h3 = what is left, |h3| < 2^-7 |h - h1| < 2^-14 |h|. The MFMA takes h1 and
// h2 (RM_PARTS = 2, the default: h3's share of a logit, below 2^-14 sum |w h|, goes into the refinement's bound)
// or all three (RM_PARTS = 3: h = h1 + h2 + h3 exactly, for |h| above 2^-110). The router is bf16 already, so
// every product w * h_i is exact in fp32: besides h3, only the fp32 accumulation of the MFMA makes the
// approximate logit A differ from maple.c's chain result L, bounded in k_refine_topk.
//
// Partial logits on v_mfma_f32_32x32x16_bf16: P[q][b][e] = sum over columns [512 q, 512 q + 512) and the
// parts of w[e][c] * h_i[b][c], accumulated per chunk of 64 columns from zero (64 RM_PARTS products a chunk, in
// 16-column steps, each step over the parts) and the 8 chunk sums added in order, which keeps the rounding
// bound of k_refine_topk small. A block of WAVES waves takes 32 tokens x 32 WAVES EW experts x one column
// quarter q (grid.z); wave w owns experts w * 32 EW .. +32 EW as EW fragments of 32 against the block's 32
// tokens, so each input chunk is split into its parts once per block. Columns advance in chunks of 64: the
// router chunk (bf16) and the input chunk (fp32) are read with coalesced 16-byte loads into registers two
// chunks ahead, then stored to LDS (the input as its bf16 parts; rows padded to 72 bf16).
#define RM_KC 64
#ifndef RM_PARTS
#define RM_PARTS 2   // bf16 parts of each input value on the MFMA (3: the third, below 2^-14 |h|, too)
#endif
#define RM_PF 2   // router chunks loaded ahead (registers); 4 and 8 measured slower
#define RM_LR 72
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
__device__ __forceinline__ void split3(v4i f, uint2 &p1, uint2 &p2, uint2 &p3) {
    uint32_t v[4] = {(uint32_t)f.x, (uint32_t)f.y, (uint32_t)f.z, (uint32_t)f.w}, a[4], b[4], c[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        uint32_t b1 = v[u] & 0xffff0000u;
        float r1 = __uint_as_float(v[u]) - __uint_as_float(b1);
        uint32_t b2 = __float_as_uint(r1) & 0xffff0000u;
        float r2 = r1 - __uint_as_float(b2);
        a[u] = b1 >> 16; b[u] = b2 >> 16; c[u] = __float_as_uint(r2) >> 16;
    }
    p1 = make_uint2(a[0] | a[1] << 16, a[2] | a[3] << 16);
    p2 = make_uint2(b[0] | b[1] << 16, b[2] | b[3] << 16);
    p3 = make_uint2(c[0] | c[1] << 16, c[2] | c[3] << 16);
}
template <int WAVES, int EW>
__global__ void __launch_bounds__(WAVES * 64) k_router_mfma(const uint16_t *__restrict__ w, const float *__restrict__ hn, int nb,
                                                              float *__restrict__ P) {
    constexpr int NT = WAVES * 64, ER = 32 * WAVES * EW;
    constexpr int NW = ER * 8 / NT;              // router pieces (16 bytes) staged per thread: rows wrow + (NT / 8) i
    constexpr int NH = 32 * 16 / NT;             // input pieces (4 floats) per thread: rows hrow + (NT / 16) i
    // LDS stages (2 for the 8-wave block, one per CU anyway; 1 for the 4-wave block, several per CU): chunk ck
    // is stored to stage ck % NB, so with 2 stages one barrier per chunk suffices (a stage is rewritten two chunks
    // later, after every wave has passed the barrier of the chunk in between)
    constexpr int NB = WAVES == 8 ? 2 : 1;
    __shared__ __attribute__((aligned(16))) uint16_t ws_[NB][ER * RM_LR];
    __shared__ __attribute__((aligned(16))) uint16_t hsl_[NB][RM_PARTS][32 * RM_LR];
    int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, r = l & 31, kg = l >> 5;
    int e0 = blockIdx.y * ER, t0 = blockIdx.x * 32, kq = blockIdx.z * (MH / 4);
    int wrow = tid >> 3, wpc = tid & 7, hrow = tid >> 4, hq = tid & 15;
    const uint16_t *wsrc = w + (size_t)(e0 + wrow) * MH + kq + wpc * 8;
    const float *hsrc[NH];
#pragma unroll
    for (int i = 0; i < NH; i++) hsrc[i] = hn + (size_t)min(t0 + hrow + (NT / 16) * i, nb - 1) * MH + kq + hq * 4;
    constexpr int NCK = MH / 4 / RM_KC;          // chunks of this column quarter
    v4i rw[RM_PF][NW], rh[RM_PF][NH];            // chunk ck in slot ck % RM_PF, loaded RM_PF chunks ahead
#define RMW_LOAD(q_, k_)                                                                                 {                                                                                                        _Pragma("unroll") for (int i = 0; i < NW; i++)                                                           rw[q_][i] = *(const gptr_u4 *)(wsrc + (size_t)(NT / 8) * i * MH + (k_));                         _Pragma("unroll") for (int i = 0; i < NH; i++) rh[q_][i] = *(const gptr_u4 *)(hsrc[i] + (k_));     }
#pragma unroll
    for (int c = 0; c < RM_PF; c++) RMW_LOAD(c, c * RM_KC);
    f32x16 acc[EW];
#pragma unroll
    for (int f = 0; f < EW; f++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[f][i] = 0.0f;
#pragma unroll
    for (int ck = 0; ck < NCK; ck++) {
        const int q = ck % RM_PF;
        uint16_t *ws = ws_[ck % NB];
        uint16_t (*hsl)[32 * RM_LR] = hsl_[ck % NB];
        if (NB == 1) __syncthreads();
#pragma unroll
        for (int i = 0; i < NW; i++) *(v4i *)(&ws[(wrow + (NT / 8) * i) * RM_LR + wpc * 8]) = rw[q][i];
#pragma unroll
        for (int i = 0; i < NH; i++) {
            int o = (hrow + (NT / 16) * i) * RM_LR + hq * 4;
            uint2 p1, p2, p3;
            split3(rh[q][i], p1, p2, p3);
            *(uint2 *)(&hsl[0][o]) = p1; *(uint2 *)(&hsl[1][o]) = p2;
            if (RM_PARTS == 3) *(uint2 *)(&hsl[RM_PARTS - 1][o]) = p3;
        }
        __syncthreads();
        if (ck + RM_PF < NCK) RMW_LOAD(q, (ck + RM_PF) * RM_KC);
        f32x16 cacc[EW];
#pragma unroll
        for (int f = 0; f < EW; f++)
#pragma unroll
            for (int i = 0; i < 16; i++) cacc[f][i] = 0.0f;
#pragma unroll
        for (int kk = 0; kk < RM_KC; kk += 16) {
            bf16x8 av[EW];
#pragma unroll
            for (int f = 0; f < EW; f++) av[f] = *(const bf16x8 *)(&ws[(wv * 32 * EW + f * 32 + r) * RM_LR + kk + kg * 8]);
#pragma unroll
            for (int sp = 0; sp < RM_PARTS; sp++) {
                bf16x8 bv = *(const bf16x8 *)(&hsl[sp][r * RM_LR + kk + kg * 8]);
#pragma unroll
                for (int f = 0; f < EW; f++) cacc[f] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[f], bv, cacc[f], 0, 0, 0);
            }
        }
#pragma unroll
        for (int f = 0; f < EW; f++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[f][i] = acc[f][i] + cacc[f][i];
    }
#undef RMW_LOAD
    // D: register i -> expert row (i/4)*8 + kg*4 + i%4 of fragment f, token column r
    float *Pq = P + (size_t)blockIdx.z * nb * MNE;
    int tk = t0 + r;
    if (tk < nb) {
#pragma unroll
        for (int f = 0; f < EW; f++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                int e = e0 + wv * 32 * EW + f * 32 + g * 8 + kg * 4;
                *(float4 *)(Pq + (size_t)tk * MNE + e) = make_float4(acc[f][g * 4], acc[f][g * 4 + 1], acc[f][g * 4 + 2], acc[f][g * 4 + 3]);
            }
    }
}

// out[0] = max over experts of sum_c |w_ec|, out[1] = max over experts of sqrt(sum_c w_ec^2) (one block). Each
// carries a 1.001 margin for its own float arithmetic (2048 rounded additions: relative error below 1.3e-4).
__global__ void __launch_bounds__(256) k_router_l1max(const uint16_t *__restrict__ w, float *__restrict__ out) {
    __shared__ float red[2][256];
    int e = threadIdx.x;
    float s = 0.0f, q = 0.0f;
    for (int c = 0; c < MH; c++) { float v = bf16f(w[(size_t)e * MH + c]); s += fabsf(v); q += v * v; }
    red[0][e] = s; red[1][e] = sqrtf(q);
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (e < o) { red[0][e] = fmaxf(red[0][e], red[0][e + o]); red[1][e] = fmaxf(red[1][e], red[1][e + o]); }
        __syncthreads();
    }
    if (e == 0) { out[0] = red[0][0] * 1.001f; out[1] = red[1][0] * 1.001f; }
}

// =====================================================================================================
// Softmax + top-8 + renormalisation, maple.c:910-923. One wave per token; lane l holds experts 4l .. 4l+3.
// Probabilities: p_e = exp(l_e - max) / sum, the sum taken as 8 interleaved partial sums
// (lane j: experts j, j+8, ... in order) folded by hsum8 -- the same order the oracle uses. Top-8: 8 rounds
// of argmax on p with the lowest index winning ties (maple.c's strict >), picked entries set to -1; weights
// p / (sum of picked, in pick order, + 1e-20). Also writes slot -> expert (top) and weight (tw).
// =====================================================================================================
// One wave, one token: rl_row[256] -> top[8], tw[8] (written by lane 0); lane l returns the expert of slot
// l % 8. E = 256 floats of LDS scratch. Lane l holds experts 4l .. 4l+3. Selection: p >= 0 and p <= 1, so
// key = (p_bits + 1) << 2 | (3 - slot) fits 32 bits, orders like p and, within a lane, puts the lower expert
// first among equal p; a picked expert gets key 0. Each of the 8 rounds takes the largest key (lane-local
// over 4, DPP within 16-lane rows, the 4 row results as scalars); the lowest lane whose best key has that p
// holds the lowest expert index with it, and that lane's best key names it: the pick order of maple.c's
// repeated strict-> scans, ties included.
// topk_wave_v takes the lane's 4 logits; topk_wave loads them from a row in global memory.
// maple.c's softmax (maple.c:608-610) of the wave's token: p of the lane's 4 experts 4l .. 4l+3 (E: 256 floats of
// LDS scratch).
__device__ __forceinline__ void softmax_wave(float4 lv, float *E, int l, float *pv) {
    float lg[4] = {lv.x, lv.y, lv.z, lv.w};
    float mx = fmaxf(fmaxf(lg[0], lg[1]), fmaxf(lg[2], lg[3]));
    mx = wave_max(mx);
    mx = fmaxf(mx, -1e30f);  // maple.c starts its max at -1e30
#pragma unroll
    for (int i = 0; i < 4; i++) lg[i] = dexp(lg[i] - mx);
    *(float4 *)(E + 4 * l) = make_float4(lg[0], lg[1], lg[2], lg[3]);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    float part = 0.0f;
    if (l < 8) {
        float ev[MNE / 8];
#pragma unroll
        for (int m = 0; m < MNE / 8; m++) ev[m] = E[l + 8 * m];
#pragma unroll
        for (int m = 0; m < MNE / 8; m++) part = part + ev[m];
    }
    float p8[8];
#pragma unroll
    for (int i = 0; i < 8; i++) p8[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), i));
    float sum = hsum8(p8);
#pragma unroll
    for (int i = 0; i < 4; i++) pv[i] = lg[i] / sum;
}
// The 8 selection rounds on 32-bit keys whose low 2 bits are 3 - slot (key 0 = taken): picks in order (ek) and,
// for p keys ((p_bits + 1) << 2 | (3 - slot)), their p (pk) and the sum of picked p in pick order (tsum).
__device__ __forceinline__ void topk_rounds(uint32_t *key, int l, float *pk, int *ek, float &tsum) {
#pragma unroll
    for (int k = 0; k < MTOPK; k++) {
        uint32_t b = max(max(key[0], key[1]), max(key[2], key[3]));
        uint32_t lb = b;
        b = max(b, (uint32_t)dpp<0xB1>((int)b));
        b = max(b, (uint32_t)dpp<0x4E>((int)b));
        b = max(b, (uint32_t)dpp<0x141>((int)b));
        b = max(b, (uint32_t)dpp<0x140>((int)b));
        uint32_t m = max(max((uint32_t)__builtin_amdgcn_readlane((int)b, 0), (uint32_t)__builtin_amdgcn_readlane((int)b, 16)),
                         max((uint32_t)__builtin_amdgcn_readlane((int)b, 32), (uint32_t)__builtin_amdgcn_readlane((int)b, 48)));
        // the lowest lane whose best p equals the largest p holds the lowest expert with it; its own best key
        // (the lowest of its slots with that p) names the expert
        int L = __ffsll((long long)__ballot((lb >> 2) == (m >> 2))) - 1;
        uint32_t mL = (uint32_t)__builtin_amdgcn_readlane((int)lb, L);
        int e = 4 * L + 3 - (int)(mL & 3u);
        pk[k] = __uint_as_float((m >> 2) - 1u); ek[k] = e;
        tsum = tsum + pk[k];
        if (l == L) {
#pragma unroll
            for (int i = 0; i < 4; i++) key[i] = key[i] == mL ? 0u : key[i];
        }
    }
}
// Selection on the logits themselves (no softmax first): keys are the order-preserving bits of each logit with the
// low 2 bits replaced by 3 - slot, so the lower expert comes first among keys that tie. ek: the 8 picks in order.
__device__ __forceinline__ void topk_logit_rounds(float4 lv, int l, int *ek) {
    float lg[4] = {lv.x, lv.y, lv.z, lv.w};
    uint32_t key[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t b = __float_as_uint(lg[i]);
        b = (b >> 31) ? ~b : (b | 0x80000000u);
        key[i] = (b & ~3u) | (uint32_t)(3 - i);
    }
    float pk[MTOPK]; float ts = 0.0f;
    topk_rounds(key, l, pk, ek, ts);
}
// Whether picks sk[0..7] taken on the logits are maple.c's picks on p (P: the token's 256 p in LDS). p = exp(l - max)
// / sum does not decrease with the logit, so p(s_0) > ... > p(s_7) > every other expert's p means the 8 largest p
// are s_0..s_7 in that order with no ties: exactly what maple.c's strict-> scans select. A tie in p (distinct
// logits may round to one p) fails the check. ps: p of the picks. The result is uniform over the wave.
__device__ __forceinline__ bool picks_exact(const int *sk, const float *P, int l, float *ps) {
#pragma unroll
    for (int k = 0; k < MTOPK; k++) ps[k] = P[sk[k]];
    bool dec = true;
#pragma unroll
    for (int k = 0; k + 1 < MTOPK; k++) dec = dec && ps[k] > ps[k + 1];
    float4 pv = *(const float4 *)(&P[4 * l]);
    float pl4[4] = {pv.x, pv.y, pv.z, pv.w}, mo = -1.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        bool picked = false;
#pragma unroll
        for (int k = 0; k < MTOPK; k++) picked = picked || sk[k] == 4 * l + i;
        mo = picked ? mo : fmaxf(mo, pl4[i]);
    }
    mo = wave_max(mo);
    return dec && ps[MTOPK - 1] > mo;
}
__device__ __forceinline__ int topk_wave_v(float4 lv, float *E, int l, int *__restrict__ top, float *__restrict__ tw) {
    float pv[4];
    softmax_wave(lv, E, l, pv);
    uint32_t key[4];
#pragma unroll
    for (int i = 0; i < 4; i++) key[i] = ((__float_as_uint(pv[i]) + 1u) << 2) | (uint32_t)(3 - i);
    float pk[MTOPK]; int ek[MTOPK];
    float tsum = 0.0f;
    topk_rounds(key, l, pk, ek, tsum);
    if (l == 0) {
#pragma unroll
        for (int k = 0; k < MTOPK; k++) { top[k] = ek[k]; tw[k] = pk[k] / (tsum + 1e-20f); }
    }
    int mine = 0;   // lane l returns the expert of slot l % 8
#pragma unroll
    for (int k = 0; k < MTOPK; k++) mine = (l & (MTOPK - 1)) == k ? ek[k] : mine;
    return mine;
}
__device__ __forceinline__ int topk_wave(const float *__restrict__ r, float *E, int l, int *__restrict__ top, float *__restrict__ tw) {
    v4f lv = *(const gptr_f4 *)(r + 4 * l);
    return topk_wave_v(make_float4(lv.x, lv.y, lv.z, lv.w), E, l, top, tw);
}

// Top-8 and the int8 quantisation of the MoE input (maple.c:909-923 and 908 prep) of 4 tokens per block,
// one wave per token, blocks (x, 0) the top-8 and blocks (x, 1) the quantisation; adds each token's 8 experts to hist (per chunk of 64 tokens) when hist is given.
__global__ void __launch_bounds__(256) k_topk_quant(const float *__restrict__ rl, const float *__restrict__ hn, int nb,
                                                    int *__restrict__ top, float *__restrict__ tw, int8_t *__restrict__ qx,
                                                    float *__restrict__ qsx, int *__restrict__ qsumx, int *__restrict__ hist);
// Grouping of a large batch (maple.c:924-938, 1018-1019) in one launch: block c (chunk of 64 tokens, 512
// threads) reads the per-chunk expert counts hist[chunk][expert] that k_topk_quant accumulated (read only; the
// combine of the same call clears them) and forms in LDS the per-expert totals and their exclusive scans: pair
// offsets (ustart), used-expert indices (ue, eu) and tile offsets. Block 0 also publishes the plan, the tile
// table and the used experts' pointer table. Then thread (token, slot) places its pair: slot = the expert's
// offset + pairs of earlier chunks + the number of earlier tokens of the chunk that picked the expert
// (popcount of a 64-bit token mask), stable in token order as maple.c's counting sort; it writes utok/uw
// (maple.c:934-936), tp (pair ids of token b ascending), sp (pair of slot s) and pu (used expert of a pair).
__global__ void __launch_bounds__(512) k_group(const int *__restrict__ hist, int nb, Plan *__restrict__ plan,
                                               const ExpPtr *__restrict__ layer_tab, ExpPtr *__restrict__ eptr_u, int tn,
                                               Tile *__restrict__ tiles, int *__restrict__ eu_out, const int *__restrict__ top,
                                               const float *__restrict__ tw, int *__restrict__ utok, float *__restrict__ uw,
                                               int *__restrict__ tp, int *__restrict__ sp, int *__restrict__ pu) {
    constexpr int MAXCH = (2048 + 63) / 64;
    __shared__ int sc[MNE], su[MNE], st[MNE], sbase[MNE], seu[MNE];
    __shared__ unsigned long long msk[MNE];
    __shared__ int slots[64][MTOPK];
    int c = blockIdx.x, t = threadIdx.x, nchunk = (nb + 63) / 64;
    int run = 0, pre = 0, used = 0, nt = 0;
    // loads that do not depend on the counts go out first: block 0's copies of the used experts' table entries
    // and every thread's pair (token, slot) for the placement
    v4i lt0 = {0, 0, 0, 0}, lt1 = lt0, lt2 = lt0;
    if (c == 0 && layer_tab && t < MNE) { const v4i *lp = (const v4i *)(layer_tab + t); lt0 = lp[0]; lt1 = lp[1]; lt2 = lp[2]; }
    int tk = t >> 3, s = t & 7, b = c * 64 + tk;
    bool live = b < nb;
    int e = live ? top[b * MTOPK + s] : 0;
    float wv = live ? tw[b * MTOPK + s] : 0.0f;
    if (t < MNE) {
        int cnt[MAXCH];
#pragma unroll
        for (int k = 0; k < MAXCH; k++) cnt[k] = k < nchunk ? hist[k * MNE + t] : 0;   // independent loads
#pragma unroll
        for (int k = 0; k < MAXCH; k++) { if (k == c) pre = run; run += cnt[k]; }
        used = run > 0; nt = (run + tn - 1) / tn;
        sc[t] = run; su[t] = used; st[t] = nt; msk[t] = 0ull;
    }
    // inclusive scans over the 256 experts: within each of waves 0-3 by shuffles, then the totals of the waves
    // before (one barrier instead of two per doubling step)
    __shared__ int wtot[4][3];
    int isc = run, isu = used, ist = nt, l = t & 63, w4 = t >> 6;
    if (t < MNE) {
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            int a = __shfl_up(isc, o, 64), bq = __shfl_up(isu, o, 64), cq = __shfl_up(ist, o, 64);
            if (l >= o) { isc += a; isu += bq; ist += cq; }
        }
        if (l == 63) { wtot[w4][0] = isc; wtot[w4][1] = isu; wtot[w4][2] = ist; }
    }
    __syncthreads();
    if (t < MNE) {
        for (int w2 = 0; w2 < w4; w2++) { isc += wtot[w2][0]; isu += wtot[w2][1]; ist += wtot[w2][2]; }
        sc[t] = isc; su[t] = isu; st[t] = ist;
    }
    __syncthreads();
    if (t < MNE) {
        int e = t, pstart = sc[e] - run, uidx = su[e] - used, tstart = st[e] - nt;
        sbase[e] = pstart + pre;
        seu[e] = used ? uidx : -1;
        if (c == 0) {
            eu_out[e] = seu[e];
            if (used) {
                plan->ue[uidx] = e;
                plan->ustart[uidx] = pstart;
                plan->tstart[uidx] = tstart;
                if (layer_tab) { v4i *d = (v4i *)(eptr_u + uidx); d[0] = lt0; d[1] = lt1; d[2] = lt2; }
                for (int i = 0; i < nt; i++) tiles[tstart + i] = Tile{uidx, pstart + i * tn, min(tn, run - i * tn), 0};
            }
            if (e == MNE - 1) {
                int nu = su[e];
                plan->nu = nu; plan->np = sc[e]; plan->ntile_gu = st[e]; plan->tn = tn;
                plan->ustart[nu] = sc[e]; plan->tstart[nu] = st[e];
            }
        }
    }
    __syncthreads();
    // placement: thread (token tk of the chunk, slot s)
    int bs = live ? sbase[e] : 0;
    if (live) atomicOr(&msk[e], 1ull << tk);
    __syncthreads();
    int slot = bs + __popcll(msk[e] & ((1ull << tk) - 1ull));
    if (live) {
        utok[slot] = b; uw[slot] = wv;
        if (sp) sp[b * MTOPK + s] = slot;
        if (pu) pu[slot] = seu[e];
    }
    slots[tk][s] = slot;
    __syncthreads();
    if (live) {
        int rank = 0;
#pragma unroll
        for (int k = 0; k < MTOPK; k++) rank += slots[tk][k] < slot;
        tp[b * MTOPK + rank] = slot;
    }
}

// Host-given grouping (gpre_moe / gfull_moe / gpux): plan from ustart; one thread.
__global__ void k_plan_from_ustart(const int *__restrict__ ustart, int nu, Plan *__restrict__ plan, int tn, Tile *__restrict__ tiles) {
    if (threadIdx.x != 0) return;
    int t = 0;
    for (int u = 0; u < nu; u++) {
        int c = ustart[u + 1] - ustart[u];
        plan->ue[u] = u; plan->ustart[u] = ustart[u]; plan->tstart[u] = t;
        for (int i = 0; i * tn < c; i++) tiles[t++] = Tile{u, ustart[u] + i * tn, min(tn, c - i * tn), 0};
    }
    plan->ustart[nu] = ustart[nu]; plan->tstart[nu] = t;
    plan->nu = nu; plan->np = ustart[nu]; plan->ntile_gu = t; plan->tn = tn;
}

// rint of four values |v| <= 2^22 as four int8 in one word (byte i = value i), and their sum added to *sum.
// v + 1.5 * 2^23 lies in [2^23, 2^24), where the float spacing is 1, so the addition rounds v to the nearest
// integer, ties to even (rintf's rounding), and the low byte of the sum's bit pattern is that integer mod 256.
// The word's signed bytes are summed with one v_dot4 against 1,1,1,1.
__device__ __forceinline__ uint32_t rint_pack4(float a, float b, float c, float d, int *sum) {
    const float MAG = 12582912.0f;
    uint32_t ua = __float_as_uint(a + MAG), ub = __float_as_uint(b + MAG), uc = __float_as_uint(c + MAG), ud = __float_as_uint(d + MAG);
    uint32_t lo = __builtin_amdgcn_perm(ub, ua, 0x0c0c0400u), hi = __builtin_amdgcn_perm(ud, uc, 0x0c0c0400u);
    uint32_t w = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
    *sum = __builtin_amdgcn_sdot4((int)w, 0x01010101, *sum, false);
    return w;
}

// =====================================================================================================
// Per-vector int8 quantisation, maple.c:183-194 as compiled with maple.c's -ffast-math flags:
// qs = mx * fl(1/127), inv = 127 / mx (both 1 when mx = 0), q = rint(x * inv). One wave per vector of
// n = 2048 or 512 values; output in mfma order (see top of file) plus qs and qsum. Optionally the source
// rows are gathered (src_row = rows ? rows[i] : i) -- not used by the current path.
// =====================================================================================================
// One wave quantises one vector of N (2048 or 512) floats into q (mfma order), *qs, *qsum (lane 0 writes).
// GPAD: bytes of padding after each 128-column group of q (LDS copies read by lanes one group apart).
template <int N, int GPAD>
__device__ __forceinline__ void quant_wave(const float *__restrict__ xr, int l, int8_t *__restrict__ q, float *__restrict__ qs,
                                           int *__restrict__ qsum) {
    constexpr int NCHK = N / 16;                    // 16-byte output chunks per vector
    constexpr int PER = (NCHK + 63) / 64;           // chunks per lane
    float v[PER][16];
    float mx = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        int o = l + 64 * k;
        if (o < NCHK) {
            int g = o >> 3, h = (o >> 2) & 1, t = o & 3;
#pragma unroll
            for (int s = 0; s < 4; s++) {
                float4 f = *(const float4 *)(xr + g * 128 + s * 32 + h * 16 + t * 4);
                v[k][s * 4 + 0] = f.x; v[k][s * 4 + 1] = f.y; v[k][s * 4 + 2] = f.z; v[k][s * 4 + 3] = f.w;
            }
#pragma unroll
            for (int i = 0; i < 16; i++) mx = fmaxf(mx, fabsf(v[k][i]));
        }
    }
    mx = wave_max(mx);
    float qsv = 1.0f, inv = 1.0f;
    if (mx > 0.0f) { qsv = mx * (1.0f / 127.0f); inv = 127.0f / mx; }
    int sum = 0;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        int o = l + 64 * k;
        if (o < NCHK) {
            uint32_t wds[4];
#pragma unroll
            for (int d = 0; d < 4; d++)
                wds[d] = rint_pack4(v[k][d * 4] * inv, v[k][d * 4 + 1] * inv, v[k][d * 4 + 2] * inv, v[k][d * 4 + 3] * inv, &sum);
            *(uint4 *)(q + (o >> 3) * (128 + GPAD) + (o & 7) * 16) = make_uint4(wds[0], wds[1], wds[2], wds[3]);
        }
    }
    sum = wave_sum_i(sum);
    if (l == 0) { *qs = qsv; *qsum = sum; }
}

template <int N>
__global__ void __launch_bounds__(256) k_quant(const float *__restrict__ x, int nrows, int8_t *__restrict__ q,
                                               float *__restrict__ qs, int *__restrict__ qsum) {
    int wv = threadIdx.x >> 6, l = threadIdx.x & 63;
    int row = blockIdx.x * 4 + wv;
    if (row >= nrows) return;
    quant_wave<N>(x + (size_t)row * N, l, q + (size_t)row * N, qs + row, qsum + row);
}

__global__ void __launch_bounds__(256) k_topk_quant(const float *__restrict__ rl, const float *__restrict__ hn, int nb,
                                                    int *__restrict__ top, float *__restrict__ tw, int8_t *__restrict__ qx,
                                                    float *__restrict__ qsx, int *__restrict__ qsumx, int *__restrict__ hist) {
    __shared__ __attribute__((aligned(16))) float E[4][MNE];
    int wv = threadIdx.x >> 6, l = threadIdx.x & 63;
    int b = blockIdx.x * 4 + wv;
    if (b >= nb) return;  // whole wave exits together
    if (blockIdx.y == 0) {   // grid y = 2: the top-8 and the quantisation of a token run in different blocks
        int ek = topk_wave(rl + (size_t)b * MNE, E[wv], l, top + b * MTOPK, tw + b * MTOPK);
        if (hist && l < MTOPK) atomicAdd(&hist[(b >> 6) * MNE + ek], 1);   // per-chunk expert counts for k_group
    } else {
        quant_wave<MH>(hn + (size_t)b * MH, l, qx + (size_t)b * MH, qsx + b, qsumx + b);
    }
}

// Exact top-8 from the approximate logits of k_router_mfma, fused with the softmax/top-8 of the token.
// |A - L| <= RG_ERRK * sw = err_b bounds the gap between the MFMA logit A and maple.c's chain logit L, where sw
// bounds sum_c |w_ec h_c| for every expert: the smaller of max|h_b| max_e sum_c |w_ec| (Hoelder) and
// |h_b|_2 max_e |w_e|_2 (Cauchy-Schwarz, far smaller when a few coordinates of h dominate). Of the gap to
// L: on the MFMA side a product of a column and an input part is exact and passes through at most 64 RM_PARTS
// roundings inside its chunk's accumulation (every product of the chunk rounded on its own, the worst case for the
// MFMA's internal sums), 8 for the chunk sums of its quarter, 3 for the quarter partials and 1 for the bias; on
// the chain side through 256 FMAs and 3 hsum additions. Each rounding is at most 2^-24 times the running
// magnitude (at most sum |w h|): (64 RM_PARTS + 271) x 2^-24 x sum |w h|, plus 1024 x 2^-24 x sum |w h| for the
// left-out part h3 when RM_PARTS = 2; times 1.01 for the parts' sum of magnitudes, and 2 for safety (which also
// covers an accumulator that truncates: 2^-23 per operation). Every expert with A >= a8 - 2 err_b (a8 = the 8th largest A) is a candidate and gets its exact chain
// logit in maple.c's batch order; no other expert can reach the top 8 of the exact logits, because the 8
// experts with A >= a8 have L >= a8 - err_b while the rest have L < a8 - err_b. The softmax/top-8 then runs on
// the row of exact (candidates) and approximate (the rest) logits, so the picks and their order are maple.c's;
// p, and so tw, differ only through the softmax sum's approximate small terms.
#if RM_PARTS == 3
#define RG_ERRK (2.0f * 463.0f * 1.01f / 16777216.0f)
#else
#define RG_ERRK (2.0f * (399.0f + 1024.0f) * 1.01f / 16777216.0f)
#endif
#define RT_HP 260    // LDS floats per chain of the staged input (256 + 4 against bank conflicts)
// One wave per token, 4 tokens per block (grid = (ceil(nb / 4), 2)); the blocks of grid row 1 quantise the
// tokens instead (in the same wave they would raise the register count of the refinement). The input row sits in LDS chain-major
// (hc[j][m] = hn[j + 8m]); lane = (candidate slot l / 8, chain l % 8), so 8 candidates are resolved per pass,
// each lane's 256-long FMA chain reading the router's chain-order copy (k_router_chainmajor, NCH = 8) with all
// 32 of its 16-byte loads issued before the FMAs. Writes rl (exact for candidates, else approximate), top, tw
// and the per-chunk expert counts for k_group.
__global__ void __launch_bounds__(256) k_refine_topk(const float *__restrict__ P, const float *__restrict__ hn, int nb,
                                                     const uint16_t *__restrict__ wc8, const float *__restrict__ bias,
                                                     const float *__restrict__ w1max, float *__restrict__ rl,
                                                     int *__restrict__ top, float *__restrict__ tw, int *__restrict__ hist,
                                                     int8_t *__restrict__ qx, float *__restrict__ qsx, int *__restrict__ qsumx) {
    __shared__ __attribute__((aligned(16))) float hsc[4][8 * RT_HP];
    __shared__ __attribute__((aligned(16))) float row[4][MNE];
    __shared__ __attribute__((aligned(16))) float E[4][MNE];
    __shared__ int cand[4][MNE];
    int wv = threadIdx.x >> 6, l = threadIdx.x & 63, b = blockIdx.x * 4 + wv;
    if (b >= nb) return;   // whole wave; no block-wide barrier below
    if (blockIdx.y == 1) {   // grid y = 2: the tokens' int8 quantisation (maple.c prep) in blocks of their own
        quant_wave<MH>(hn + (size_t)b * MH, l, qx + (size_t)b * MH, qsx + b, qsumx + b);
        return;
    }
    const float *xr = hn + (size_t)b * MH;
    float4 f[8];
#pragma unroll
    for (int i = 0; i < 8; i++) f[i] = *(const float4 *)(xr + (l + 64 * i) * 4);
    float a[4], bb[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (bias) {   // issued with the partials' loads (one wait for all)
#pragma unroll
        for (int i = 0; i < 4; i++) bb[i] = bias[l + 64 * i];
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        size_t o = (size_t)b * MNE + l + 64 * i, qs = (size_t)nb * MNE;
        float v = (P[o] + P[o + qs]) + (P[o + 2 * qs] + P[o + 3 * qs]);
        if (bias) v = v + bb[i];
        a[i] = v;
    }
    float *hc = &hsc[wv][0];
    float hm = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        int c = (l + 64 * i) * 4;
        float v4[4] = {f[i].x, f[i].y, f[i].z, f[i].w};
#pragma unroll
        for (int u = 0; u < 4; u++) { hc[((c + u) & 7) * RT_HP + ((c + u) >> 3)] = v4[u]; hm = fmaxf(hm, fabsf(v4[u])); }
    }
    hm = wave_max(hm);
    float h2 = 0.0f;   // sum of squares of the row (fp32; below 2^-18 relative error, covered by the 1.001 below)
#pragma unroll
    for (int i = 0; i < 8; i++) h2 += (f[i].x * f[i].x + f[i].y * f[i].y) + (f[i].z * f[i].z + f[i].w * f[i].w);
    h2 = wave_sumf(h2);
    // a8: the 8th largest approximate logit (8 rounds of the wave maximum, lowest index first)
    float rem[4] = {a[0], a[1], a[2], a[3]}, a8 = 0.0f;
    for (int k = 0; k < MTOPK; k++) {
        float m = wave_max(fmaxf(fmaxf(rem[0], rem[1]), fmaxf(rem[2], rem[3])));
        a8 = m;
        unsigned long long m0 = __ballot(rem[0] == m), m1 = __ballot(rem[1] == m), m2 = __ballot(rem[2] == m), m3 = __ballot(rem[3] == m);
        int e = m0 ? __ffsll((long long)m0) - 1 : m1 ? 64 + __ffsll((long long)m1) - 1 : m2 ? 128 + __ffsll((long long)m2) - 1 : 192 + __ffsll((long long)m3) - 1;
        if (l == (e & 63)) { int i = e >> 6; rem[0] = i == 0 ? -INFINITY : rem[0]; rem[1] = i == 1 ? -INFINITY : rem[1]; rem[2] = i == 2 ? -INFINITY : rem[2]; rem[3] = i == 3 ? -INFINITY : rem[3]; }
    }
    // the bias add rounds relative to |logit + bias| on both sides (MFMA sum and exact chain): with a bias much
    // larger than sum|w h| that error is not covered by RG_ERRK's term, so add 2^-24 (|bias| + sum|w h|) per side
    float bm = wave_max(fmaxf(fmaxf(fabsf(bb[0]), fabsf(bb[1])), fmaxf(fabsf(bb[2]), fabsf(bb[3]))));
    // sum_c |w_ec h_c| <= min(max|h| max_e sum_c |w_ec|, |h|_2 max_e |w_e|_2) (Hoelder, Cauchy-Schwarz): the second
    // is far tighter when a few columns of h dominate (one outlier coordinate: max|h| ~ |h|_2 while sum |w| ~ 45 |w|_2)
    float sw = fminf(hm * w1max[0], sqrtf(h2) * 1.001f * w1max[1]);
    float thr = a8 - 2.0f * (RG_ERRK * sw + (2.0f / 16777216.0f) * (bm + 1.01f * sw));
    int nc = 0;
    unsigned long long lanemask = (1ull << l) - 1ull;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        row[wv][l + 64 * i] = a[i];
        bool c = a[i] >= thr;
        unsigned long long m = __ballot(c);
        if (c) cand[wv][nc + popc64(m & lanemask)] = l + 64 * i;
        nc += popc64(m);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    // exact chain logits of the candidates, 8 per pass (nc is at least 8 and at most 256)
    int slot = l >> 3, j = l & 7;
    const float *hj = hc + j * RT_HP;
    for (int c0 = 0; c0 < nc; c0 += 8) {   // c0 and nc are uniform over the wave
        bool on = c0 + slot < nc;
        int e = cand[wv][on ? c0 + slot : 0];
        const gptr_u4 *wp = (const gptr_u4 *)(wc8 + (size_t)e * MH + j * 8);   // 16 bytes q of the chain at wp[q * 8]
        float be = 0.0f;
        if (bias && j == 0) be = bias[e];   // loaded before the chain, added after it
        float acc = 0.0f;
#pragma unroll
        for (int hb = 0; hb < 2; hb++) {   // the chain's weights in two halves of 16 x 16 bytes (registers)
            v4i wq[16];
#pragma unroll
            for (int q = 0; q < 16; q++) wq[q] = wp[(hb * 16 + q) * 8];
#pragma unroll
            for (int q16 = 0; q16 < 16; q16++) {
                int q = hb * 16 + q16;
                if ((q & 1) == 0) __builtin_amdgcn_sched_barrier(0);   // two steps per scheduling region (registers)
                float4 h0 = *(const float4 *)(hj + q * 8), h1 = *(const float4 *)(hj + q * 8 + 4);
                uint32_t q0 = (uint32_t)wq[q16].x, q1 = (uint32_t)wq[q16].y, q2 = (uint32_t)wq[q16].z, q3 = (uint32_t)wq[q16].w;
                acc = __builtin_fmaf(__uint_as_float(q0 << 16), h0.x, acc); acc = __builtin_fmaf(__uint_as_float(q0 & 0xffff0000u), h0.y, acc);
                acc = __builtin_fmaf(__uint_as_float(q1 << 16), h0.z, acc); acc = __builtin_fmaf(__uint_as_float(q1 & 0xffff0000u), h0.w, acc);
                acc = __builtin_fmaf(__uint_as_float(q2 << 16), h1.x, acc); acc = __builtin_fmaf(__uint_as_float(q2 & 0xffff0000u), h1.y, acc);
                acc = __builtin_fmaf(__uint_as_float(q3 << 16), h1.z, acc); acc = __builtin_fmaf(__uint_as_float(q3 & 0xffff0000u), h1.w, acc);
            }
        }
        float rv = hsum8_lanes<8>(acc);
        if (j == 0 && on) {
            if (bias) rv = rv + be;
            row[wv][e] = rv;
        }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
    for (int i = 0; i < 4; i++) rl[(size_t)b * MNE + l + 64 * i] = row[wv][l + 64 * i];
    int ek = topk_wave_v(*(const float4 *)(&row[wv][4 * l]), E[wv], l, top + b * MTOPK, tw + b * MTOPK);
    if (hist && l < MTOPK) atomicAdd(&hist[(b >> 6) * MNE + ek], 1);   // per-chunk expert counts for k_group
}

// Quantisation of two FF-long (512) vectors by one wave, as quant_wave: lanes 0-31 hold one vector, lanes
// 32-63 the other, lane = one 16-column chunk o (values v[s*4+b] = columns (o>>3)*128 + s*32 +
// ((o>>2)&1)*16 + (o&3)*4 + b). Output in mfma order with GS bytes per 128-column group (128 in global
// memory, more in padded LDS copies); lane 0 of each half writes qs and qsum. store = false: the half takes
// part in the wave-wide reductions but writes nothing.
template <int GS>
__device__ __forceinline__ void quant_half(const float *v, int l, int8_t *q, float *qs, int *qsum, bool store = true) {
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) mx = fmaxf(mx, fabsf(v[i]));
    mx = fmaxf(mx, __int_as_float(dpp<0xB1>(__float_as_int(mx))));
    mx = fmaxf(mx, __int_as_float(dpp<0x4E>(__float_as_int(mx))));
    mx = fmaxf(mx, __int_as_float(dpp<0x141>(__float_as_int(mx))));
    mx = fmaxf(mx, __int_as_float(dpp<0x140>(__float_as_int(mx))));
    int mb = __float_as_int(mx);
    float m0 = fmaxf(__int_as_float(__builtin_amdgcn_readlane(mb, 0)), __int_as_float(__builtin_amdgcn_readlane(mb, 16)));
    float m1 = fmaxf(__int_as_float(__builtin_amdgcn_readlane(mb, 32)), __int_as_float(__builtin_amdgcn_readlane(mb, 48)));
    mx = l < 32 ? m0 : m1;
    float qsv = 1.0f, inv = 1.0f;
    if (mx > 0.0f) { qsv = mx * (1.0f / 127.0f); inv = 127.0f / mx; }
    int sum = 0; uint32_t wds[4];
#pragma unroll
    for (int d = 0; d < 4; d++) wds[d] = rint_pack4(v[d * 4] * inv, v[d * 4 + 1] * inv, v[d * 4 + 2] * inv, v[d * 4 + 3] * inv, &sum);
    int o = l & 31;
    if (store) *(uint4 *)(q + (o >> 3) * GS + (o & 7) * 16) = make_uint4(wds[0], wds[1], wds[2], wds[3]);
    sum += dpp<0xB1>(sum); sum += dpp<0x4E>(sum); sum += dpp<0x141>(sum); sum += dpp<0x140>(sum);
    int s0 = __builtin_amdgcn_readlane(sum, 0) + __builtin_amdgcn_readlane(sum, 16);
    int s1 = __builtin_amdgcn_readlane(sum, 32) + __builtin_amdgcn_readlane(sum, 48);
    if (store && (l & 31) == 0) { *qs = qsv; *qsum = l < 32 ? s0 : s1; }
}

// int8 quantisation of np activation vectors of 512 (maple.c:830-832), two per wave (quant_half), output
// in mfma order. grid = ceil(np / 8) blocks of 256.
__global__ void __launch_bounds__(256) k_quant_act(const float *__restrict__ act, int np, int8_t *__restrict__ qa,
                                                   float *__restrict__ qsa, int *__restrict__ qsuma) {
    int t = threadIdx.x, l = t & 63;
    int pair = blockIdx.x * 8 + (t >> 6) * 2 + (l >> 5);
    bool live = pair < np;
    const float *ar = act + (size_t)(live ? pair : 0) * MFF;
    int o = l & 31, g = o >> 3, h = (o >> 2) & 1, tq = o & 3;
    float v[16];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        float4 f = *(const float4 *)(ar + g * 128 + s * 32 + h * 16 + tq * 4);
        v[s * 4] = f.x; v[s * 4 + 1] = f.y; v[s * 4 + 2] = f.z; v[s * 4 + 3] = f.w;
    }
    quant_half<128>(v, l, qa + (size_t)pair * MFF, qsa + pair, qsuma + pair, live);
}

// SiLU(min(g,7)) * clamp(u,-7,7) from the int32 gate/up sums, then the int8 quantisation of act
// (maple.c:825-832); the path with checks on (the sums stay readable). gu[pair][0..511] gate, [512..1023] up,
// as written by k_gateup_pk<false>; G = (float)(sum - qsum) * qs * s_gate[row], likewise U. grid = tiles x 8
// blocks of 8 pairs; a wave takes 2 pairs (half-wave each). act (fp32) is written when act != NULL.
__global__ void __launch_bounds__(256) k_act_quant(const Plan *__restrict__ plan, const Tile *__restrict__ tiles,
                                                   const ExpPtr *__restrict__ eptr, const int *__restrict__ utok,
                                                   const float *__restrict__ qsx, const int *__restrict__ qsumx,
                                                   const int *__restrict__ gu, float *__restrict__ act,
                                                   int8_t *__restrict__ qa, float *__restrict__ qsa, int *__restrict__ qsuma) {
    int tile = blockIdx.x >> 3, part = blockIdx.x & 7;
    if (tile >= plan->ntile_gu) return;
    Tile tl = tiles[tile];
    if (part * 8 >= tl.n) return;
    int t = threadIdx.x, wv = t >> 6, l = t & 63;
    int tk = part * 8 + wv * 2 + (l >> 5);
    bool live = tk < tl.n;
    int pair = tl.p0 + (live ? tk : 0);
    ExpPtr ex = eptr[tl.u];
    int tok = utok[pair];
    int o = l & 31, g = o >> 3, h = (o >> 2) & 1, tq = o & 3;
    int ag[4][4], au[4][4]; float4 sg[4], su[4];
    int qsum = qsumx[tok];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        int col = g * 128 + s * 32 + h * 16 + tq * 4;
        size_t o = (size_t)pair * 2 * MFF + col;
        int4 a4 = *(const int4 *)(gu + o), u4 = *(const int4 *)(gu + o + MFF);
        ag[s][0] = a4.x - qsum; ag[s][1] = a4.y - qsum; ag[s][2] = a4.z - qsum; ag[s][3] = a4.w - qsum;
        au[s][0] = u4.x - qsum; au[s][1] = u4.y - qsum; au[s][2] = u4.z - qsum; au[s][3] = u4.w - qsum;
        sg[s] = *(const float4 *)(ex.gs + col);
        su[s] = *(const float4 *)(ex.us + col);
    }
    float qs = qsx[tok];
    float v[16];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        float sgv[4] = {sg[s].x, sg[s].y, sg[s].z, sg[s].w}, suv[4] = {su[s].x, su[s].y, su[s].z, su[s].w};
#pragma unroll
        for (int b = 0; b < 4; b++) {
            float gv = (float)ag[s][b] * qs * sgv[b];
            float uv = (float)au[s][b] * qs * suv[b];
            float gg = gv < 7.0f ? gv : 7.0f;
            float uu = __builtin_amdgcn_fmed3f(uv, -7.0f, 7.0f);   // finite uv: the clamp of maple.c
            v[s * 4 + b] = silu_le7(gg) * uu;
        }
        if (act && live)
            *(float4 *)(act + (size_t)pair * MFF + g * 128 + s * 32 + h * 16 + tq * 4) = make_float4(v[s * 4], v[s * 4 + 1], v[s * 4 + 2], v[s * 4 + 3]);
    }
    quant_half<128>(v, l, qa + (size_t)pair * MFF, qsa + pair, qsuma + pair, live);
}

// =====================================================================================================
// Grouped ternary x int8 GEMM on CDNA4 int8 MFMA (v_mfma_i32_16x16x64_i8), shared by gate/up and down.
//
// MFMA operand mapping. A = codes (16 weight rows x 64 k), B = activations (64 k x 16 tokens). A lane
// (G = lane/16, r = lane%16) holds 16 int8 of row r; B lane (G, n) holds the same 16 k positions of token n;
// which 16 k positions a (G, byte) slot stands for is the same for A and B, so any consistent assignment of
// columns to slots gives the exact integer dot product. We assign them so that one 32-bit word of packed
// codes is one lane's A operand: code word at byte j0 of a 128-group, shifted by 2s and masked with
// 0x03030303, is the int8 codes of columns s*32 + j0 + 0..3 (s = 0..3). Lane (G, r) loads 16 code bytes
// (group G/2 of a 256-column chunk, bytes (G%2)*16 .. +16) = 4 code words = the A operands of 4 MFMA steps;
// the matching activation bytes are 64 contiguous bytes in mfma order. Codes stay {0,1,2}: the sum of
// (c - 1) q is the MFMA result minus qsum, exactly as maple.c does (maple.c:226).
// Result D lane (G, n): rows 4G..4G+3 of the 16-row block, token n.
// =====================================================================================================
__device__ __forceinline__ v4i decode_word(uint32_t w) {
    const uint32_t M = 0x03030303u;
    v4i a;
    a.x = (int)(w & M); a.y = (int)((w >> 2) & M); a.z = (int)((w >> 4) & M); a.w = (int)((w >> 6) & M);
    return a;
}

// Work-item order for the 8 XCDs: the hardware hands consecutive workgroup ids to XCDs round robin, so
// workgroup id b runs on XCD b % 8. The n real items (known on the device only; the grid is sized for the
// worst case) are split into 8 contiguous runs of ceil(n / 8), and workgroup b takes item b / 8 of run b % 8
// (-1: nothing to do). Items are ordered (token tile, row block) with the row block fastest, so the tiles of
// one expert -- sharing its codes -- and the row blocks of one tile -- sharing its activations -- meet in the
// same XCD's L2, and all 8 XCDs get the same number of items whatever the grid size.
__device__ __forceinline__ int xcd_item(int b, int n) {
    int per = (n + 7) >> 3, j = b >> 3, item = (b & 7) * per + j;
    return j < per && item < n ? item : -1;
}

// Gate+up with fused SiLU*up (maple.c:471-479, 825-830). Block = WAVES waves; wave w owns RF 16-row
// fragments of gate rows and the same RF fragments of up rows; the block covers WAVES*RF*16 rows of both.
// 1-D grid of (token tile x row block) items, n = gridDim.x (multiple of 8); items past the plan exit.
//
// Pipeline over the 8 chunks of 256 columns, two chunks deep, ordinary loads only:
//   iteration ch: barrier; issue the loads of chunk ch+2 (code words into a 3-deep register ring, the tile's
//   activation pieces into a 2-deep register ring); MFMAs of chunk ch (codes from registers, activations from
//   LDS stage ch%2); store the activation pieces of chunk ch+1 into LDS stage (ch+1)%2.
// LDS activation rows: token tk, 256 bytes, its 16-byte part p at slot p ^ (tk & 15), so the 16 lanes that
// read one B fragment (16 tokens, one part) hit 16 different banks. Padding tokens of a partial tile load a
// valid token's row; their result columns are never stored. MODE is an experiment knob (0 = normal).
template <int TN, int WAVES, int RF, int MODE = 0>
__global__ void __launch_bounds__(WAVES * 64) k_gateup(const Plan *__restrict__ plan, const Tile *__restrict__ tiles,
                                                        const ExpPtr *__restrict__ eptr,
                                                        const int *__restrict__ utok, const int8_t *__restrict__ qx,
                                                        const float *__restrict__ qsx, const int *__restrict__ qsumx,
                                                        float *__restrict__ act, int *__restrict__ dbg) {
    constexpr int NT = WAVES * 64;
    constexpr int NF = TN / 16;                 // token fragments
    constexpr int NA = 2 * RF;                  // code fragments per wave (gate then up)
    constexpr int RB = MFF / (WAVES * RF * 16);
    constexpr int NCH = MH / 256;               // 8 chunks of 256 columns
    constexpr int BB = TN * 256;                // activation bytes per LDS stage
    constexpr int NPC = (TN * 16 + NT - 1) / NT;  // 16-byte activation pieces per thread per chunk
    __shared__ __attribute__((aligned(16))) int8_t bs[2][BB];
    __shared__ int toks[TN];
    int item = xcd_item(blockIdx.x, plan->ntile_gu * RB);
    if (item < 0) return;
    int tile = item / RB, rb = item % RB;
    Tile tl = tiles[tile];
    int p0 = tl.p0, ntok = tl.n;
    ExpPtr ex = eptr[tl.u];
    int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, G = l >> 4, r16 = l & 15;
    if (tid < TN) toks[tid] = utok[p0 + (tid < ntok ? tid : 0)];
    __syncthreads();

    // activation pieces of this thread: piece i = tid + k*NT -> token i/16, part i%16 (slot part ^ (tk & 15))
    const gptr_u4 *bsrc[NPC]; int bdst[NPC]; bool blive[NPC];   // padding tokens of a short tile: zeros, not loaded
#pragma unroll
    for (int k = 0; k < NPC; k++) {
        int i = tid + k * NT, tk = (i < TN * 16 ? i : 0) >> 4, part = i & 15;
        bsrc[k] = (const gptr_u4 *)(qx + (size_t)toks[tk] * MH + part * 16);
        blive[k] = i < TN * 16 && tk < ntok;
        bdst[k] = i < TN * 16 ? tk * 256 + ((part ^ (tk & 15)) * 16) : -1;
    }
    int rowblk = rb * (WAVES * RF * 16) + wv * RF * 16;   // first gate (and up) row of this wave
    const gptr_u4 *arow[NA];
    int aoff = (G >> 1) * 32 + (G & 1) * 16;  // byte offset of this lane's 16 code bytes in a 64-byte chunk
#pragma unroll
    for (int f = 0; f < RF; f++) {
        arow[f] = (const gptr_u4 *)(ex.gc + (size_t)(rowblk + f * 16 + r16) * (MH / 4) + aoff);
        arow[RF + f] = (const gptr_u4 *)(ex.uc + (size_t)(rowblk + f * 16 + r16) * (MH / 4) + aoff);
    }
    v4i acc[NA][NF];
#pragma unroll
    for (int f = 0; f < NA; f++)
#pragma unroll
        for (int j = 0; j < NF; j++) acc[f][j] = v4i{0, 0, 0, 0};

    v4i cw[3][NA];      // code words of chunks ch, ch+1, ch+2
    v4i br[2][NPC];     // activation pieces of chunks ch+1, ch+2
#pragma unroll
    for (int c = 0; c < 2; c++) {
#pragma unroll
        for (int f = 0; f < NA; f++) cw[c][f] = arow[f][c * 4];
#pragma unroll
        for (int k = 0; k < NPC; k++) br[c][k] = blive[k] ? bsrc[k][c * 16] : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int k = 0; k < NPC; k++) if (bdst[k] >= 0) *(v4i *)(&bs[0][bdst[k]]) = br[0][k];
#pragma unroll
    for (int ch = 0; ch < NCH; ch++) {
        __syncthreads();                                   // stage ch%2 written by everyone
        if (ch + 2 < NCH) {
#pragma unroll
            for (int f = 0; f < NA; f++) cw[(ch + 2) % 3][f] = arow[f][(ch + 2) * 4];
            if (MODE != 1) {
#pragma unroll
                for (int k = 0; k < NPC; k++) br[ch % 2][k] = blive[k] ? bsrc[k][(ch + 2) * 16] : v4i{0, 0, 0, 0};
            }
        }
        const int8_t *sp = &bs[ch % 2][0];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            int part = (G >> 1) * 8 + (G & 1) * 4 + t;
            v4i bv[NF];
#pragma unroll
            for (int j = 0; j < NF; j++) bv[j] = *(const v4i *)(sp + (j * 16 + r16) * 256 + ((part ^ r16) * 16));
#pragma unroll
            for (int f = 0; f < NA; f++) {
                v4i c4 = cw[ch % 3][f];
                uint32_t w = (uint32_t)(t == 0 ? c4.x : t == 1 ? c4.y : t == 2 ? c4.z : c4.w);
                v4i av = decode_word(w);
#pragma unroll
                for (int j = 0; j < NF; j++) acc[f][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv[j], acc[f][j], 0, 0, 0);
            }
        }
        if (ch + 1 < NCH) {
            __builtin_amdgcn_sched_barrier(0);  // the store (and its wait on chunk ch+1's loads) after the MFMAs
#pragma unroll
            for (int k = 0; k < NPC; k++) if (bdst[k] >= 0) *(v4i *)(&bs[(ch + 1) % 2][bdst[k]]) = br[(ch + 1) % 2][k];
        }
    }
    // epilogue: G, U -> act
#pragma unroll
    for (int j = 0; j < NF; j++) {
        int tk = j * 16 + r16;
        if (tk >= ntok) continue;
        int tok = toks[tk];
        float qs = qsx[tok]; int qsum = qsumx[tok];
        int pair = p0 + tk;
#pragma unroll
        for (int f = 0; f < RF; f++) {
            int row0 = rowblk + f * 16 + 4 * G;
            float4 sg = *(const float4 *)(ex.gs + row0), su = *(const float4 *)(ex.us + row0);
            float sgv[4] = {sg.x, sg.y, sg.z, sg.w}, suv[4] = {su.x, su.y, su.z, su.w};
            int ag[4] = {acc[f][j].x, acc[f][j].y, acc[f][j].z, acc[f][j].w};
            int au[4] = {acc[RF + f][j].x, acc[RF + f][j].y, acc[RF + f][j].z, acc[RF + f][j].w};
            float o[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float gv = (float)(ag[i] - qsum) * qs * sgv[i];
                float uv = (float)(au[i] - qsum) * qs * suv[i];
                float g = gv < 7.0f ? gv : 7.0f;
                float uu = uv < -7.0f ? -7.0f : (uv > 7.0f ? 7.0f : uv);
                o[i] = MODE == 3 ? g + uu : g / (1.0f + dexp(-g)) * uu;
            }
            *(float4 *)(act + (size_t)pair * MFF + row0) = make_float4(o[0], o[1], o[2], o[3]);
            if (dbg) {
                *(int4 *)(dbg + (size_t)pair * 2 * MFF + row0) = make_int4(ag[0], ag[1], ag[2], ag[3]);
                *(int4 *)(dbg + (size_t)pair * 2 * MFF + MFF + row0) = make_int4(au[0], au[1], au[2], au[3]);
            }
        }
    }
}

// One 256-column chunk of a gate/up tile for one wave: 8 steps of 32 columns; at each step the gate and up code
// words (NA = 2 fragments) are decoded once and multiplied with NFU token fragments of 32 (NFU = 1 when the
// tile has <= 32 tokens). Activation operands come from the LDS stage sp one
// step ahead of their use; the body is branch-free so the scheduler can overlap LDS reads, decode and MFMA.
// LDS stage layout: token tk's 256 bytes at tk * GU_LROW (16 bytes of padding per row: the 16 lanes of a
// 16-byte read pass fall in 16 different bank groups, and a step is a constant offset).
#define GU_LROW 272
template <int NFU>
__device__ __forceinline__ void gu_chunk(v16i (&acc)[2][2], const v4i (&cwc)[2][2], const int8_t *sp, int G2, int r32,
                                         bool two = true) {
    v4i bv[2][NFU];
#pragma unroll
    for (int j = 0; j < NFU; j++) bv[0][j] = *(const v4i *)(sp + (j * 32 + r32) * GU_LROW + G2 * 128);
#pragma unroll
    for (int t = 0; t < 8; t++) {
        if (t + 1 < 8) {
#pragma unroll
            for (int j = 0; j < NFU; j++) bv[(t + 1) & 1][j] = *(const v4i *)(sp + (j * 32 + r32) * GU_LROW + G2 * 128 + (t + 1) * 16);
        }
#pragma unroll
        for (int f = 0; f < 2; f++) {
            v4i c4 = cwc[f][t >> 2];
            int tt = t & 3;
            v4i av = decode_word((uint32_t)(tt == 0 ? c4.x : tt == 1 ? c4.y : tt == 2 ? c4.z : c4.w));
#pragma unroll
            for (int j = 0; j < NFU; j++)
                if (j == 0 || two) acc[f][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv[t & 1][j], acc[f][j], 0, 0, 0);
        }
        // issue order of one step: next step's LDS reads, gate decode, gate MFMAs, up decode, up MFMAs
        if (t + 1 < 8) __builtin_amdgcn_sched_group_barrier(0x100, NFU, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 7, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, NFU, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 7, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, NFU, 0);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Persistent gate+up on v_mfma_i32_32x32x32_i8 (twice the rate of the 16x16x64 form on gfx950), int32 sums
// out. Operand mapping: A lane (G2 = lane/32, r = lane%32) holds 16 int8 of row r, B lane (G2, n) the same 16
// k positions of token n. Lane group G2 takes 128-column group G2 of each 256-column chunk; at step t (0..7)
// its A operand is code word t of that group decoded in registers, and its B operand the 16 contiguous
// bytes 16t.. of the group in mfma order (see the top of this file). D (16 int32 per lane): register i
// holds row (i/4)*8 + G2*4 + i%4 of the 32-row block, token lane%32. An item is 128 gate + 128 up rows (wave w:
// 32 of each) x a tile of 64 tokens (two fragments of 32). grid = 8 * NB workgroups; the ones on XCD x = blockIdx % 8 walk that XCD's
// contiguous run of items (as xcd_item) with stride NB, so an XCD's L2 sees the tiles of few experts at a
// time. The chunk pipeline runs on across items: while the last chunks of one item are multiplied, the first
// ones of the next are loaded (codes PD chunks ahead in a ring of PD + 1 register slots, activations PA chunks
// ahead, then through two LDS stages), so no item starts with an empty pipeline. The default, PD = PA = 1 at
// three workgroups per CU (168 VGPRs), beats PD = 3 / PA = 2 at two (214 VGPRs): the third wave per SIMD
// fills the MFMA and VALU pipes better than the deeper prefetch hides latency.
template <bool ACT, int PD = 1, int PA = 1, int OCC = 3>
__global__ void __launch_bounds__(256, OCC) k_gateup_pk(const Plan *__restrict__ plan, const Tile *__restrict__ tiles,
                                                      const ExpPtr *__restrict__ eptr, const int *__restrict__ utok,
                                                      const int8_t *__restrict__ qx, const float *__restrict__ qsx,
                                                      const int *__restrict__ qsumx, void *__restrict__ out) {
    constexpr int TN = 64, NT = 256, NF = 2, NA = 2, RB = MFF / 128, NCH = MH / 256, BB = TN * GU_LROW;
    constexpr int NPC = TN * 16 / NT;          // 4 activation pieces of 16 bytes per thread per chunk
    // PD: prefetch distance of the codes in chunks (ring of CR = PD + 1 slots, a divisor of NCH); PA: that of the
    // activations (ring of PA, then 2 LDS stages); OCC: workgroups per CU the register budget is held to
    constexpr int CR = PD + 1;
    static_assert(NCH % CR == 0 && (PA == 1 || PA == 2), "k_gateup_pk pipeline shape");
    __shared__ __attribute__((aligned(16))) int8_t bs[2][BB];
    __shared__ int toks[2][TN];
    __shared__ __attribute__((aligned(16))) float ssc[2][128];   // ACT: the item's gate and up row scales (epilogue)
    int nitems = plan->ntile_gu * RB;
    int per = (nitems + 7) >> 3, xcd = blockIdx.x & 7, nbx = gridDim.x >> 3;
    int last = min(nitems, (xcd + 1) * per);
    int cur = xcd * per + (blockIdx.x >> 3);
    if (cur >= last) return;
    int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, G2 = l >> 5, r32 = l & 31;
    // a thread's activation pieces k: token tk = (tid >> 4) + 16 k, 16-byte part tid & 15 of the chunk
    int part = tid & 15, bdst = (tid >> 4) * GU_LROW + part * 16;

    // current item: uniform bases (scalar registers) + 32-bit per-lane offsets
    Tile tl = tiles[cur / RB];
    int p0 = tl.p0, ntok = tl.n, cu = tl.u, rowblk = (cur % RB) * 128 + wv * 32;
    const uint8_t *gcb = eptr[tl.u].gc, *ucb = eptr[tl.u].uc;
    if (tid < TN) toks[0][tid] = utok[p0 + (tid < ntok ? tid : 0)];
    __syncthreads();
    int slot = 0;
    uint32_t aoff = (uint32_t)(rowblk + r32) * (MH / 4) + G2 * 32, boff[NPC];
#pragma unroll
    for (int k = 0; k < NPC; k++) boff[k] = (uint32_t)toks[0][(tid >> 4) + 16 * k] * MH + part * 16;
    v16i acc[NA][NF];
#pragma unroll
    for (int f = 0; f < NA; f++)
#pragma unroll
        for (int j = 0; j < NF; j++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[f][j][i] = 0;
    v4i cw[CR][NA][2];  // codes of chunk c of any item in slot c % CR
    v4i br[PA][NPC];    // activations of chunk c in slot c % PA until stored to LDS stage c % 2
#define GU_LOADC(slot_, gb_, ub_, off_, c_)                                                                     \
    {                                                                                                           \
        cw[slot_][0][0] = *(const gptr_u4 *)((gb_) + (off_) + (c_) * 64);                                      \
        cw[slot_][0][1] = *(const gptr_u4 *)((gb_) + (off_) + (c_) * 64 + 16);                                 \
        cw[slot_][1][0] = *(const gptr_u4 *)((ub_) + (off_) + (c_) * 64);                                      \
        cw[slot_][1][1] = *(const gptr_u4 *)((ub_) + (off_) + (c_) * 64 + 16);                                 \
    }
#pragma unroll
    for (int c = 0; c < PD; c++) GU_LOADC(c, gcb, ucb, aoff, c);
#pragma unroll
    for (int c = 0; c < PA; c++)
#pragma unroll
        for (int k = 0; k < NPC; k++) br[c % PA][k] = *(const gptr_u4 *)(qx + boff[k] + c * 256);
#pragma unroll
    for (int k = 0; k < NPC; k++) *(v4i *)(&bs[0][bdst + k * 16 * GU_LROW]) = br[0][k];

    while (true) {
        int nxt = cur + nbx;
        bool has_next = nxt < last;
        // next item: tile and expert now (scalar loads), its token ids into registers now and LDS at chunk 2
        Tile ntl = tiles[(has_next ? nxt : cur) / RB];
        int nrowblk = ((has_next ? nxt : cur) % RB) * 128 + wv * 32;
        const uint8_t *ngcb = eptr[ntl.u].gc, *nucb = eptr[ntl.u].uc;
        uint32_t naoff = (uint32_t)(nrowblk + r32) * (MH / 4) + G2 * 32, nboff[NPC];
        int ntk = 0;
        if (has_next && tid < TN) ntk = utok[ntl.p0 + (tid < ntl.n ? tid : 0)];
        float scv = 0.0f;   // ACT: this thread's row scale, loaded at chunk 0 and stored at chunk 4 (no wait on it)
#pragma unroll
        for (int ch = 0; ch < NCH; ch++) {
            __syncthreads();
            if (ch == 2 && tid < TN) toks[slot ^ 1][tid] = ntk;     // read after the barrier of chunk 3
            if (ACT && ch == 0) scv = (tid < 128 ? eptr[cu].gs : eptr[cu].us)[(cur % RB) * 128 + (tid & 127)];
            if (ACT && ch == 4) ssc[tid >> 7][tid & 127] = scv;   // read by the epilogue after the last barrier
            if (ch == NCH - PA && has_next) {
#pragma unroll
                for (int k = 0; k < NPC; k++) nboff[k] = (uint32_t)toks[slot ^ 1][(tid >> 4) + 16 * k] * MH + part * 16;
            }
            // prefetch codes of chunk ch + PD and activations of chunk ch + PA (of this item, or of the next one)
            if (ch + PD < NCH) GU_LOADC((ch + PD) % CR, gcb, ucb, aoff, ch + PD)
            else if (has_next) GU_LOADC((ch + PD) % CR, ngcb, nucb, naoff, (ch + PD) % NCH)
            if (ch + PA < NCH) {
#pragma unroll
                for (int k = 0; k < NPC; k++) br[ch % PA][k] = *(const gptr_u4 *)(qx + boff[k] + (ch + PA) * 256);
            } else if (has_next) {
#pragma unroll
                for (int k = 0; k < NPC; k++) br[ch % PA][k] = *(const gptr_u4 *)(qx + nboff[k] + ((ch + PA) % NCH) * 256);
            }
            gu_chunk<2>(acc, cw[ch % CR], &bs[ch % 2][0], G2, r32, ntok > 32);
            __builtin_amdgcn_sched_barrier(0);
            if (ch + 1 < NCH || has_next) {
#pragma unroll
                for (int k = 0; k < NPC; k++) *(v4i *)(&bs[(ch + 1) % 2][bdst + k * 16 * GU_LROW]) = br[(ch + 1) % PA][k];
            }
        }
        // epilogue, token r32 of each fragment, rows (i/4)*8 + G2*4 + i%4 of the wave's 32. ACT: the activation
        // SiLU(min(G,7)) * clamp(U,-7,7) with G = (float)(sum - qsum) * qs * s_gate[row] (maple.c:471-479,
        // 825-829), fp32 into out[pair][512]; else the raw int32 sums into out[pair][1024] (gate, then up).
#pragma unroll
        for (int j = 0; j < NF; j++) {
            int tk = j * 32 + r32;
            if (tk < ntok) {
                int pair = p0 + tk;
                int tok = toks[slot][tk];
                float qs = ACT ? qsx[tok] : 0.0f;
                int qsum = ACT ? qsumx[tok] : 0;
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    int row0 = rowblk + g * 8 + G2 * 4;
                    if (ACT) {
                        float4 sg = *(const float4 *)(&ssc[0][row0 - (cur % RB) * 128]), su = *(const float4 *)(&ssc[1][row0 - (cur % RB) * 128]);
                        float sgv[4] = {sg.x, sg.y, sg.z, sg.w}, suv[4] = {su.x, su.y, su.z, su.w}, o[4];
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            float gv = (float)(acc[0][j][g * 4 + i] - qsum) * qs * sgv[i];
                            float uv = (float)(acc[1][j][g * 4 + i] - qsum) * qs * suv[i];
                            float gg = gv < 7.0f ? gv : 7.0f;
                            o[i] = silu_le7(gg) * __builtin_amdgcn_fmed3f(uv, -7.0f, 7.0f);
                        }
                        *(float4 *)((float *)out + (size_t)pair * MFF + row0) = make_float4(o[0], o[1], o[2], o[3]);
                    } else {
#pragma unroll
                        for (int f = 0; f < 2; f++)
                            *(v4i *)((int *)out + (size_t)pair * 2 * MFF + f * MFF + row0) =
                                v4i{acc[f][j][g * 4], acc[f][j][g * 4 + 1], acc[f][j][g * 4 + 2], acc[f][j][g * 4 + 3]};
                    }
                }
            }
        }
        if (!has_next) break;
#pragma unroll
        for (int f = 0; f < NA; f++)
#pragma unroll
            for (int j = 0; j < NF; j++)
#pragma unroll
                for (int i = 0; i < 16; i++) acc[f][j][i] = 0;
        cur = nxt; slot ^= 1;
        p0 = ntl.p0; ntok = ntl.n; cu = ntl.u; rowblk = nrowblk;
        gcb = ngcb; ucb = nucb; aoff = naoff;
#pragma unroll
        for (int k = 0; k < NPC; k++) boff[k] = nboff[k];
    }
#undef GU_LOADC
}

// ---- dense ternary projections (attention q/k/v and o; maple.c jobB_qkv / jobB_o, 459-470, through
// tdot_multi 423-458): y[b][yoff + r] = (float)(sum_c code * q[b] - qsum[b]) * qs[b] * s[r], K = 2048 ----
struct DenseMat { const uint8_t *codes; const float *scales; int rows, yoff; };
// One workgroup = WAVES x 64 rows (wave w: rows w*64 .. +64 as two 32-row fragments) x 64 tokens, on
// v_mfma_i32_32x32x32_i8 with gu_chunk's operand mapping (the two row fragments take the places of gate and
// up). Activations pass through two padded LDS stages, codes 2 chunks ahead in registers, as k_gateup.
// grid = (sum of rows / (64 WAVES), ceil(nb / 64)); rbs[m] = first row block of matrix m (rbs[nmat] = total).
// ACC: y += the product (maple.c:724, x += o), else y = the product.
template <int WAVES, bool ACC = false>
__global__ void __launch_bounds__(WAVES * 64) k_dense(const DenseMat *__restrict__ mats, const int *__restrict__ rbs, int nmat,
                                               int nb, int ys, const int8_t *__restrict__ qx, const float *__restrict__ qsx,
                                               const int *__restrict__ qsumx, float *__restrict__ y) {
    constexpr int TN = 64, NCH = MH / 256, BB = TN * GU_LROW, NT = WAVES * 64, NPC = TN * 16 / NT, TPP = NT / 16;
    __shared__ __attribute__((aligned(16))) int8_t bs[2][BB];
    int rb = blockIdx.x, m = 0;
    while (m + 1 < nmat && rb >= rbs[m + 1]) m++;
    DenseMat M = mats[m];
    int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, G2 = l >> 5, r32 = l & 31;
    int row0 = (rb - rbs[m]) * (WAVES * 64) + wv * 64, t0 = blockIdx.y * TN, ntok = min(TN, nb - t0);
    int part = tid & 15, bdst = (tid >> 4) * GU_LROW + part * 16;
    uint32_t boff[NPC];
#pragma unroll
    for (int k = 0; k < NPC; k++) boff[k] = (uint32_t)(t0 + min((tid >> 4) + TPP * k, ntok - 1)) * MH + part * 16;
    const uint8_t *fa = M.codes + (size_t)(row0 + r32) * (MH / 4) + G2 * 32, *fb = fa + (size_t)32 * (MH / 4);
    v16i acc[2][2];
#pragma unroll
    for (int f = 0; f < 2; f++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[f][j][i] = 0;
    v4i cw[4][2][2], br[2][NPC];
#define DN2_LOADC(slot_, c_)                                                                                    \
    {                                                                                                           \
        cw[slot_][0][0] = *(const gptr_u4 *)(fa + (c_) * 64); cw[slot_][0][1] = *(const gptr_u4 *)(fa + (c_) * 64 + 16); \
        cw[slot_][1][0] = *(const gptr_u4 *)(fb + (c_) * 64); cw[slot_][1][1] = *(const gptr_u4 *)(fb + (c_) * 64 + 16); \
    }
    DN2_LOADC(0, 0); DN2_LOADC(1, 1);
#pragma unroll
    for (int c = 0; c < 2; c++)
#pragma unroll
        for (int k = 0; k < NPC; k++) br[c][k] = *(const gptr_u4 *)(qx + boff[k] + c * 256);
#pragma unroll
    for (int k = 0; k < NPC; k++) *(v4i *)(&bs[0][bdst + k * TPP * GU_LROW]) = br[0][k];
#pragma unroll
    for (int ch = 0; ch < NCH; ch++) {
        __syncthreads();
        if (ch + 2 < NCH) {
            DN2_LOADC((ch + 2) % 4, ch + 2)
#pragma unroll
            for (int k = 0; k < NPC; k++) br[ch % 2][k] = *(const gptr_u4 *)(qx + boff[k] + (ch + 2) * 256);
        }
        gu_chunk<2>(acc, cw[ch % 4], &bs[ch % 2][0], G2, r32);
        __builtin_amdgcn_sched_barrier(0);
        if (ch + 1 < NCH) {
#pragma unroll
            for (int k = 0; k < NPC; k++) *(v4i *)(&bs[(ch + 1) % 2][bdst + k * TPP * GU_LROW]) = br[(ch + 1) % 2][k];
        }
    }
#undef DN2_LOADC
    // token t0 + j*32 + r32; rows row0 + f*32 + (i/4)*8 + G2*4 + i%4. The row scales and both tokens' factors
    // are loaded together, through global-memory pointers, before the first use
    v4f sc8[2][4]; float qs2[2]; int qsum2[2];
#pragma unroll
    for (int f = 0; f < 2; f++)
#pragma unroll
        for (int g = 0; g < 4; g++) sc8[f][g] = *(const gptr_f4 *)(M.scales + row0 + f * 32 + g * 8 + G2 * 4);
#pragma unroll
    for (int j = 0; j < 2; j++) {
        int b = t0 + min(j * 32 + r32, ntok - 1);
        qs2[j] = *(const gptr_f *)(qsx + b); qsum2[j] = *(const __attribute__((address_space(1))) int *)(qsumx + b);
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
        int tk = j * 32 + r32;
        if (tk >= ntok) continue;
        int b = t0 + tk;
        float qs = qs2[j]; int qsum = qsum2[j];
#pragma unroll
        for (int f = 0; f < 2; f++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                int r = row0 + f * 32 + g * 8 + G2 * 4;
                float sv[4] = {sc8[f][g].x, sc8[f][g].y, sc8[f][g].z, sc8[f][g].w}, o[4];
#pragma unroll
                for (int i = 0; i < 4; i++) o[i] = (float)(acc[f][j][g * 4 + i] - qsum) * qs * sv[i];
                float4 *yp = (float4 *)(y + (size_t)b * ys + M.yoff + r);
                if (ACC) { v4f yv = *(const gptr_f4 *)yp; o[0] = yv.x + o[0]; o[1] = yv.y + o[1]; o[2] = yv.z + o[2]; o[3] = yv.w + o[3]; }
                *yp = make_float4(o[0], o[1], o[2], o[3]);
            }
    }
}

// Down (maple.c:498-505): D[pair][row] = (float)(sum c*qa - qsuma) * qsa * s_down[row]. Block = WAVES waves
// of RF 16-row fragments; K = 512 staged in LDS at once. Pairs of a tile are contiguous (no gather).
// 1-D grid of (token tile x row block) items in XCD order, as k_gateup.
template <int TN, int WAVES, int RF>
__global__ void __launch_bounds__(WAVES * 64) k_down(const Plan *__restrict__ plan, const Tile *__restrict__ tiles, const ExpPtr *__restrict__ eptr,
                                                      const int8_t *__restrict__ qa, const float *__restrict__ qsa,
                                                      const int *__restrict__ qsuma, float *__restrict__ down, int *__restrict__ dbg) {
    constexpr int NT = WAVES * 64;
    constexpr int NF = TN / 16;
    constexpr int LDSW = MFF + 16;
    constexpr int RB = MH / (WAVES * RF * 16);
    __shared__ __attribute__((aligned(16))) int8_t bs[TN * LDSW];
    int item = xcd_item(blockIdx.x, plan->ntile_gu * RB);
    if (item < 0) return;
    int tile = item / RB, rb = item % RB;
    Tile tl = tiles[tile];
    int p0 = tl.p0, ntok = tl.n;
    ExpPtr ex = eptr[tl.u];
    int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, G = l >> 4, r16 = l & 15;
    int rowblk = rb * (WAVES * RF * 16) + wv * RF * 16;
    const uint8_t *arow[RF];
#pragma unroll
    for (int f = 0; f < RF; f++) arow[f] = ex.dc + (size_t)(rowblk + f * 16 + r16) * (MFF / 4);
    int aoff = (G >> 1) * 32 + (G & 1) * 16;
    uint4 cw[2][RF];
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int f = 0; f < RF; f++) cw[h][f] = *(const uint4 *)(arow[f] + h * 64 + aoff);
    for (int i = tid; i < TN * (MFF / 16); i += NT) {
        int tk = i / (MFF / 16), part = i % (MFF / 16);
        uint4 v = make_uint4(0, 0, 0, 0);
        if (tk < ntok) v = *(const uint4 *)(qa + (size_t)(p0 + tk) * MFF + part * 16);
        *(uint4 *)(&bs[tk * LDSW + part * 16]) = v;
    }
    __syncthreads();
    v4i acc[RF][NF];
#pragma unroll
    for (int f = 0; f < RF; f++)
#pragma unroll
        for (int j = 0; j < NF; j++) acc[f][j] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int h = 0; h < 2; h++) {
        int boff = h * 256 + (G >> 1) * 128 + (G & 1) * 64;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            v4i bv[NF];
#pragma unroll
            for (int j = 0; j < NF; j++) bv[j] = *(const v4i *)(bs + (j * 16 + r16) * LDSW + boff + t * 16);
#pragma unroll
            for (int f = 0; f < RF; f++) {
                uint32_t w = t == 0 ? cw[h][f].x : t == 1 ? cw[h][f].y : t == 2 ? cw[h][f].z : cw[h][f].w;
                v4i av = decode_word(w);
#pragma unroll
                for (int j = 0; j < NF; j++) acc[f][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv[j], acc[f][j], 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < NF; j++) {
        int tk = j * 16 + r16;
        if (tk >= ntok) continue;
        int pair = p0 + tk;
        float qs = qsa[pair]; int qsum = qsuma[pair];
#pragma unroll
        for (int f = 0; f < RF; f++) {
            int row0 = rowblk + f * 16 + 4 * G;
            float4 sd = *(const float4 *)(ex.ds + row0);
            float sdv[4] = {sd.x, sd.y, sd.z, sd.w};
            int ad[4] = {acc[f][j].x, acc[f][j].y, acc[f][j].z, acc[f][j].w};
            float o[4];
#pragma unroll
            for (int i = 0; i < 4; i++) o[i] = (float)(ad[i] - qsum) * qs * sdv[i];
            *(float4 *)(down + (size_t)pair * MH + row0) = make_float4(o[0], o[1], o[2], o[3]);
            if (dbg) *(int4 *)(dbg + (size_t)pair * MH + row0) = make_int4(ad[0], ad[1], ad[2], ad[3]);
        }
    }
}

// Whole expert per workgroup for small batches (tiles of <= 16 pairs): gate/up with SiLU*up, the int8
// quantisation of act and down in one launch (maple.c:471-479, 498-505, 825-832). With a few pairs per expert
// these layers stream the expert's 798,720 bytes of codes and scales and do little arithmetic, so one
// workgroup per tile streams the whole expert through a register ring, as fast as a plain copy of the same
// blocks; act never leaves LDS. Block = WAVES waves (16 in use: 128 VGPRs, 4 waves per SIMD); wave w takes
// GF = 512 / (16 WAVES) gate fragments of 16 rows and the same up rows (v_mfma_i32_16x16x64_i8, operand mapping
// of k_gateup), then DF = 2048 / (16 WAVES) down fragments in passes of 8. The code loads come in groups of GL
// 16-byte loads per lane, each group whole cache lines of consecutive rows (a gate and an up fragment over
// GL / 2 chunks, or GL / 2 down fragments over both chunks; reading 64 bytes of many rows per group instead
// streamed 20% slower), RING groups deep in registers. Small groups (GL = 4, 3 deep) beat large ones (8, 3
// deep) by 8%: every workgroup issues its first loads at once, and the first group lands sooner. LDS: the
// tile's int8 input (16 rows of 2048 bytes, 16-byte parts swizzled as in k_gateup), reused for fp32 act; act
// in int8 (rows of E16_QW bytes); the tile's scales. Outputs: down[pair] as k_down, the quantised act as
// k_quant_act; with gu_d / dn_d (checks on) also the int32 sums and fp32 act.
#define E16_QW 528   // LDS bytes per quantised act row (512 + 16: rows 16 apart fall in different banks)
// Grouping inside the kernel (GRP, device routing of up to E16_GRP_MAXTOK tokens): instead of reading a plan that k_group
// wrote, every workgroup forms the grouping of maple.c:924-938 itself from the top-8 (G): per-expert counts in
// LDS, their inclusive scans (pairs, used experts, tiles of 16), its tile's expert and pair range, and the
// tile's tokens (those that picked the expert, ascending: a prefix count over tokens). It writes its pairs'
// utok, uw, sp, pu and tp (a pair's rank among its token's 8 pairs is the number of the token's experts with a
// smaller id, since pairs are ordered by expert); workgroup 0 writes the plan, tile table, expert pointers and
// eu as k_group does. The outputs equal k_group's.
#define E16_GRP_MAXTOK 256
struct GroupIn { const int *top; const float *tw; int nb; const ExpPtr *layer_tab; Plan *plan; Tile *tiles; ExpPtr *eptr_u;
                 int *eu; int *utok; float *uw; int *tp; int *sp; int *pu; };
template <int WAVES, int RING, int GRP = 0, int GL = 8>
__global__ void __launch_bounds__(WAVES * 64) k_expert16(const Plan *__restrict__ plan, const Tile *__restrict__ tiles,
                                                         const ExpPtr *__restrict__ eptr, const int *__restrict__ utok,
                                                         const int8_t *__restrict__ qx, const float *__restrict__ qsx,
                                                         const int *__restrict__ qsumx, float *__restrict__ down,
                                                         float *__restrict__ act_d, int8_t *__restrict__ qa_d,
                                                         float *__restrict__ qsa_d, int *__restrict__ qsuma_d,
                                                         int *__restrict__ gu_d, int *__restrict__ dn_d, GroupIn gi) {
    constexpr int NT = WAVES * 64;
    constexpr int GF = MFF / 16 / WAVES;       // gate (and up) fragments of 16 rows per wave
    constexpr int DF = MH / 16 / WAVES;        // down fragments per wave, in passes of 8
    // GL loads of 16 bytes per lane per group: a gate/up group is a gate and an up fragment over CPG chunks of
    // 256 columns, a down group FPG down fragments over both chunks of 256 columns
    constexpr int NFR = GL, CPG = GL / 2, GPF = 8 / CPG, FPG = GL / 2, GPP = 8 / FPG;
    constexpr int NACC = 8;                    // accumulators: 2 GF gate/up fragments, then a down pass of 8
    static_assert(GL % 2 == 0 && 8 % CPG == 0 && 2 * GF <= NACC && FPG * GPP == NACC && DF % FPG == 0, "k_expert16 group shape");
    constexpr int NGU = GF * GPF, NG = NGU + DF / FPG;
    __shared__ __attribute__((aligned(16))) int8_t xs[16 * MH];     // input rows; later fp32 act [16][512]
    __shared__ __attribute__((aligned(16))) int8_t qs8[16 * E16_QW];
    __shared__ __attribute__((aligned(16))) float sg[MFF], su[MFF], sd[MH];
    __shared__ float tqs[16], aqs[16];
    __shared__ int tqsum[16], aqsum[16], toks[16];
    int tid = threadIdx.x, l = tid & 63, G = l >> 4, r16 = l & 15;
    int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    int p0 = 0, ntok = 0, ge = 0, gti = 0;
    ExpPtr ex;
    constexpr bool GR = GRP != 0;
    __shared__ int gc[GR ? MNE : 1], gsc[GR ? MNE : 1], gsu[GR ? MNE : 1], gst[GR ? MNE : 1], gsx[GR ? MNE : 1], gwc[WAVES], gex;
    __shared__ int gslot[16];
    __shared__ __attribute__((aligned(16))) int gtl[GR ? E16_GRP_MAXTOK * MTOPK : 4];
    __shared__ __attribute__((aligned(16))) float gtw[GR ? E16_GRP_MAXTOK * MTOPK : 4], gqs[GR ? E16_GRP_MAXTOK : 1];
    __shared__ int gqsum[GR ? E16_GRP_MAXTOK : 1];
    __shared__ int gwt[4][4];
    // the grouping: the top-8 rows into LDS, counts per expert, inclusive scans over experts of pairs (gsc), used
    // experts (gsu), tiles of 16 (gst) and tiles after an expert's first (gsx); workgroup 0 publishes the plan
    auto group_scan = [&]() {
        int nb = gi.nb;
        if (tid < MNE) gc[tid] = 0;
        if (tid < nb) {   // token b's top-8, weights and quantisation scales into LDS (nb <= E16_GRP_MAXTOK), so no
                          // global load waits behind the code loads later
            const v4i *tr = (const v4i *)(gi.top + tid * MTOPK), *wr = (const v4i *)(gi.tw + tid * MTOPK);
            *(v4i *)(gtl + tid * MTOPK) = tr[0]; *(v4i *)(gtl + tid * MTOPK + 4) = tr[1];
            *(v4i *)(gtw + tid * MTOPK) = wr[0]; *(v4i *)(gtw + tid * MTOPK + 4) = wr[1];
            gqs[tid] = qsx[tid]; gqsum[tid] = qsumx[tid];
        }
        __syncthreads();
        for (int i = tid; i < nb * MTOPK; i += NT) atomicAdd(&gc[gtl[i]], 1);
        __syncthreads();
        // within each of waves 0-3 (expert = tid) by shuffles, then the totals of the waves before
        int run = 0, used = 0, nt = 0, isc = 0, isu = 0, ist = 0, isx = 0;
        if (tid < MNE) {
            run = gc[tid]; used = run > 0; nt = (run + 15) >> 4;
            isc = run; isu = used; ist = nt; isx = nt > 1 ? nt - 1 : 0;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                int a = __shfl_up(isc, o, 64), bq = __shfl_up(isu, o, 64), cq = __shfl_up(ist, o, 64), dq = __shfl_up(isx, o, 64);
                if (l >= o) { isc += a; isu += bq; ist += cq; isx += dq; }
            }
            if (l == 63) { gwt[wv][0] = isc; gwt[wv][1] = isu; gwt[wv][2] = ist; gwt[wv][3] = isx; }
        }
        __syncthreads();
        if (tid < MNE) {
            for (int w2 = 0; w2 < wv; w2++) { isc += gwt[w2][0]; isu += gwt[w2][1]; ist += gwt[w2][2]; isx += gwt[w2][3]; }
            gsc[tid] = isc; gsu[tid] = isu; gst[tid] = ist; gsx[tid] = isx;
            if (blockIdx.x == 0) {   // the plan as k_group publishes it
                int e = tid, pstart = isc - run, uidx = isu - used, tstart = ist - nt;
                gi.eu[e] = used ? uidx : -1;
                if (used) {
                    gi.plan->ue[uidx] = e; gi.plan->ustart[uidx] = pstart; gi.plan->tstart[uidx] = tstart;
                    gi.eptr_u[uidx] = gi.layer_tab[e];
                    for (int i = 0; i < nt; i++) gi.tiles[tstart + i] = Tile{uidx, pstart + i * 16, min(16, run - i * 16), 0};
                }
                if (e == MNE - 1) {
                    int nu = isu;
                    gi.plan->nu = nu; gi.plan->np = isc; gi.plan->ntile_gu = ist; gi.plan->tn = 16;
                    gi.plan->ustart[nu] = isc; gi.plan->tstart[nu] = ist;
                }
            }
        }
        __syncthreads();
    };
    // GRP == 2: workgroup e < 256 takes the first tile of expert e, so its code loads go out before the grouping
    // (wasted for unused experts: they leave after it); workgroups 256.. take the further tiles of experts with
    // more than 16 pairs, in expert order. GRP == 1: workgroup b takes the b-th tile in expert order.
    const bool first_tile = GRP == 2 && blockIdx.x < MNE;
    if (!GR) {
        int item = xcd_item(blockIdx.x, plan->ntile_gu);
        if (item < 0) return;
        Tile tl = tiles[item];
        p0 = tl.p0; ntok = tl.n;
        ex = eptr[tl.u];
    } else if (first_tile) {
        ge = blockIdx.x; gti = 0;
        ex = gi.layer_tab[ge];
    } else {
        group_scan();
        int item = GRP == 2 ? (int)blockIdx.x - MNE : (int)blockIdx.x;
        if (tid < MNE) {
            int e = tid, nt = (gc[e] + 15) >> 4;
            if (GRP == 2) { int xs0 = gsx[e] - (nt > 1 ? nt - 1 : 0); if (item >= xs0 && item < gsx[e]) gex = e; }
            else { int ts0 = gst[e] - nt; if (item >= ts0 && item < gst[e]) gex = e; }
        }
        __syncthreads();
        if (item >= (GRP == 2 ? gsx[MNE - 1] : gst[MNE - 1])) return;   // whole workgroup
        int e = __builtin_amdgcn_readfirstlane(gex);   // uniform: the expert table entry loads as scalars
        int cnt = gc[e];
        int ti = GRP == 2 ? 1 + item - (gsx[e] - (((cnt + 15) >> 4) - 1)) : item - (gst[e] - ((cnt + 15) >> 4));
        p0 = gsc[e] - cnt + 16 * ti;
        ntok = min(16, cnt - 16 * ti);
        ex = gi.layer_tab[e];
        ge = e; gti = ti;
    }
    // lane offset of its 16 code bytes: row r16 of a fragment, 16-byte part of a 64-byte chunk (as k_gateup)
    int aoff = (G >> 1) * 32 + (G & 1) * 16;
    uint32_t gl = (uint32_t)r16 * (MH / 4) + aoff, dl = (uint32_t)r16 * (MFF / 4) + aoff;
    const uint8_t *gb = ex.gc + (size_t)wv * GF * 16 * (MH / 4), *ub = ex.uc + (size_t)wv * GF * 16 * (MH / 4);
    const uint8_t *db = ex.dc + (size_t)wv * DF * 16 * (MFF / 4);
    v4i cw[RING][NFR];
    // Each group reads whole rows (8 KB contiguous per wave): gate/up group g = gate and up fragment g / 2, the
    // 4 chunks (g & 1) * 4 .. +3 (load k: up if k >= 4, chunk k & 3); down group NGU + 2 ps + q = fragments
    // 4q .. 4q+3 of pass ps (8 fragments), both chunks (load k: fragment 4q + k / 2, chunk k & 1)
    auto load_group = [&](int g, v4i (&dst)[NFR]) {
        if (g < NGU) {
            int fp = g / GPF, cb = (g % GPF) * CPG;
#pragma unroll
            for (int k = 0; k < NFR; k++)
                dst[k] = *(const gptr_u4 *)((k < CPG ? gb : ub) + fp * 16 * (MH / 4) + gl + (cb + k % CPG) * 64);
        } else {
            int ps = (g - NGU) / GPP, q = (g - NGU) % GPP;
#pragma unroll
            for (int k = 0; k < NFR; k++)
                dst[k] = *(const gptr_u4 *)(db + (ps * 128 + (FPG * q + (k >> 1)) * 16) * (MFF / 4) + dl + (k & 1) * 64);
        }
    };
#pragma unroll
    for (int g = 0; g < RING - 1; g++) load_group(g, cw[g]);
    // the expert's row scales into registers now, behind the first code loads (stored to LDS with the tile)
    static_assert(NT == 2 * MFF && NT >= MH / 4, "k_expert16 scale staging: one gate or up scale and one down float4 per thread");
    const float scg = tid < MFF ? ex.gs[tid] : ex.us[tid - MFF];
    const float4 scd = tid < MH / 4 ? *(const float4 *)(ex.ds + tid * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
    if (first_tile) {   // the grouping, with the expert's first code loads in flight
        group_scan();
        int cnt = gc[ge];
        if (cnt == 0) return;   // unused expert: the whole workgroup leaves
        p0 = gsc[ge] - cnt; ntok = min(16, cnt);
    }
    if (GR) {   // the tile's tokens (after the first code loads are in flight)
        // the tokens that picked the expert, in ascending order: entries 16 ti .. of that list
        bool has = false; int slot = 0;
        if (tid < gi.nb) {
#pragma unroll
            for (int k = 0; k < MTOPK; k++) if (gtl[tid * MTOPK + k] == ge) { has = true; slot = k; }
        }
        unsigned long long m = __ballot(has);
        if (l == 0) gwc[wv] = __popcll(m);
        __syncthreads();
        int before = __popcll(m & ((1ull << l) - 1ull));
        for (int w2 = 0; w2 < wv; w2++) before += gwc[w2];
        int r = before - 16 * gti;
        if (has && r >= 0 && r < 16) { toks[r] = tid; gslot[r] = slot; }
        __syncthreads();
        if (tid < ntok) {   // this tile's pairs in the grouping outputs
            int b = toks[tid], sl = gslot[tid], pr = p0 + tid, rank = 0;
            gi.utok[pr] = b; gi.uw[pr] = gtw[b * MTOPK + sl]; gi.pu[pr] = gsu[ge] - 1;
            if (gi.sp) gi.sp[b * MTOPK + sl] = pr;
#pragma unroll
            for (int k = 0; k < MTOPK; k++) rank += gtl[b * MTOPK + k] < ge;
            gi.tp[b * MTOPK + rank] = pr;
        }
    }
    // stage the tile: input rows (zeros for padding tokens), its quantisation scales, the expert's row scales
    if (tid < 16) {
        int tk = tid < ntok ? (GR ? toks[tid] : utok[p0 + tid]) : -1;
        toks[tid] = tk;
        tqs[tid] = tk >= 0 ? (GR ? gqs[tk] : qsx[tk]) : 0.0f;
        tqsum[tid] = tk >= 0 ? (GR ? gqsum[tk] : qsumx[tk]) : 0;
    }
    if (tid < MFF) sg[tid] = scg; else su[tid - MFF] = scg;
    if (tid < MH / 4) *(float4 *)(sd + tid * 4) = scd;
    __syncthreads();
    {   // 128 parts of 16 bytes per row; every load issued before the first store (padding rows read row 0)
        constexpr int NK = 16 * 128 / NT;
        v4i v[NK];
#pragma unroll
        for (int k = 0; k < NK; k++) {
            int i = tid + NT * k, tk = i >> 7, part = i & 127, src = toks[tk];
            v[k] = *(const gptr_u4 *)(qx + (size_t)(src >= 0 ? src : 0) * MH + part * 16);
        }
#pragma unroll
        for (int k = 0; k < NK; k++) {
            int i = tid + NT * k, tk = i >> 7, part = i & 127;
            *(v4i *)(xs + tk * MH + (part >> 4) * 256 + (((part & 15) ^ tk) * 16)) = toks[tk] >= 0 ? v[k] : v4i{0, 0, 0, 0};
        }
    }
    __syncthreads();

    v4i acc[NACC];
#pragma unroll
    for (int f = 0; f < NACC; f++) acc[f] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int g = 0; g < NG; g++) {
        if (g + RING - 1 < NG) load_group(g + RING - 1, cw[(g + RING - 1) % RING]);
        const v4i(&c)[NFR] = cw[g % RING];
        if (g < NGU) {
            int fp = g / GPF, cb = (g % GPF) * CPG;
#pragma unroll
            for (int cc = 0; cc < CPG; cc++)
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    int part = (G >> 1) * 8 + (G & 1) * 4 + t;
                    v4i bv = *(const v4i *)(xs + r16 * MH + (cb + cc) * 256 + ((part ^ r16) * 16));
                    uint32_t wg = (uint32_t)(t == 0 ? c[cc].x : t == 1 ? c[cc].y : t == 2 ? c[cc].z : c[cc].w);
                    uint32_t wu = (uint32_t)(t == 0 ? c[CPG + cc].x : t == 1 ? c[CPG + cc].y : t == 2 ? c[CPG + cc].z : c[CPG + cc].w);
                    acc[fp] = __builtin_amdgcn_mfma_i32_16x16x64_i8(decode_word(wg), bv, acc[fp], 0, 0, 0);
                    acc[GF + fp] = __builtin_amdgcn_mfma_i32_16x16x64_i8(decode_word(wu), bv, acc[GF + fp], 0, 0, 0);
                }
        } else {
            int q = (g - NGU) % GPP;
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    v4i bv = *(const v4i *)(qs8 + r16 * E16_QW + h * 256 + (G >> 1) * 128 + (G & 1) * 64 + t * 16);
#pragma unroll
                    for (int j = 0; j < FPG; j++) {
                        const v4i cj = c[2 * j + h];
                        uint32_t w = (uint32_t)(t == 0 ? cj.x : t == 1 ? cj.y : t == 2 ? cj.z : cj.w);
                        acc[FPG * q + j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(decode_word(w), bv, acc[FPG * q + j], 0, 0, 0);
                    }
                }
        }
        if (g == NGU - 1) {
            // gate/up epilogue: lane (G, n) holds rows wv*GF*16 + 16f + 4G + i of token n; act into LDS (fp32 over xs)
            __syncthreads();   // every wave is done reading xs
            float *act = (float *)xs;
            float qs = tqs[r16]; int qsum = tqsum[r16];
#pragma unroll
            for (int f = 0; f < GF; f++) {
                int row0 = wv * GF * 16 + f * 16 + 4 * G;
                float o[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    float gv = (float)(acc[f][i] - qsum) * qs * sg[row0 + i];
                    float uv = (float)(acc[GF + f][i] - qsum) * qs * su[row0 + i];
                    float gg = gv < 7.0f ? gv : 7.0f;
                    o[i] = silu_le7(gg) * __builtin_amdgcn_fmed3f(uv, -7.0f, 7.0f);
                }
                *(float4 *)(act + r16 * MFF + row0) = make_float4(o[0], o[1], o[2], o[3]);
                if (gu_d && r16 < ntok) {
                    int *gp = gu_d + (size_t)(p0 + r16) * 2 * MFF;
                    *(int4 *)(gp + row0) = make_int4(acc[f][0], acc[f][1], acc[f][2], acc[f][3]);
                    *(int4 *)(gp + MFF + row0) = make_int4(acc[GF + f][0], acc[GF + f][1], acc[GF + f][2], acc[GF + f][3]);
                    *(float4 *)(act_d + (size_t)(p0 + r16) * MFF + row0) = make_float4(o[0], o[1], o[2], o[3]);
                }
            }
            __syncthreads();
            // quantisation of act (maple.c prep on the 512-vector): half hh of wave w -> token 2w + hh
            if (wv < 8) {
                int tk = 2 * wv + (l >> 5), o = l & 31, gq = o >> 3, hq = (o >> 2) & 1, tq = o & 3;
                const float *ar = act + tk * MFF;
                float v[16];
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    float4 fv = *(const float4 *)(ar + gq * 128 + s * 32 + hq * 16 + tq * 4);
                    v[s * 4] = fv.x; v[s * 4 + 1] = fv.y; v[s * 4 + 2] = fv.z; v[s * 4 + 3] = fv.w;
                }
                quant_half<128>(v, l, qs8 + tk * E16_QW, aqs + tk, aqsum + tk);
            }
            __syncthreads();
            if (tid < 512) {   // the quantised act as k_quant_act writes it (read by callers that check it)
                int tk = tid >> 5, part = tid & 31;
                if (tk < ntok) {
                    *(v4i *)(qa_d + (size_t)(p0 + tk) * MFF + part * 16) = *(const v4i *)(qs8 + tk * E16_QW + part * 16);
                    if (part == 0) { qsa_d[p0 + tk] = aqs[tk]; qsuma_d[p0 + tk] = aqsum[tk]; }
                }
            }
#pragma unroll
            for (int f = 0; f < NACC; f++) acc[f] = v4i{0, 0, 0, 0};
        }
        if (g >= NGU && (g - NGU) % GPP == GPP - 1) {
            // down epilogue of pass ps: rows wv*DF*16 + 128ps + 16f + 4G + i of pair p0 + n
            int ps = (g - NGU) / GPP;
            if (r16 < ntok) {
                float qs = aqs[r16]; int qsum = aqsum[r16];
                float *dp = down + (size_t)(p0 + r16) * MH;
#pragma unroll
                for (int f = 0; f < NACC; f++) {
                    int row0 = wv * DF * 16 + ps * 128 + f * 16 + 4 * G;
                    float o[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) o[i] = (float)(acc[f][i] - qsum) * qs * sd[row0 + i];
                    *(float4 *)(dp + row0) = make_float4(o[0], o[1], o[2], o[3]);
                    if (dn_d) *(int4 *)(dn_d + (size_t)(p0 + r16) * MH + row0) = make_int4(acc[f][0], acc[f][1], acc[f][2], acc[f][3]);
                }
            }
#pragma unroll
            for (int f = 0; f < NACC; f++) acc[f] = v4i{0, 0, 0, 0};
        }
    }
}

// Down per tile (operand mapping as k_gateup_pk, K = 512): one workgroup takes a tile of up to 64 pairs of one expert
// and RPB row blocks of 256 down rows. The tile's activations (64 x 512 int8) are staged in LDS once (rows
// padded to DN_LROW bytes); the row blocks then run back to back, the codes of the next row block loaded
// while the current one is multiplied. Wave w owns rows w*64 .. +64 of each row block (two 32-row
// fragments) and both 32-pair fragments. grid = tiles x 8 / RPB items (XCD order as xcd_item).
// Output: D16 = false, D = (float)(sum - qsum) * qs * s_down[row] (fp32); D16 = true, d = sum - qsum as int16
// (-32768 with d in dov, int32, same index), turned into D by k_combine16 with the same operations; the int16
// results pass through a per-wave LDS tile so that each store writes 128 contiguous bytes of 8 pairs.
// QIN: the tile's act arrives in fp32 (act) and is quantised here (maple.c:832 prep, quant_half) into the LDS
// stage; the first workgroup of each tile also writes the int8 act, qs and qsum out (qa_w, qsa_w, qsuma_w) as
// k_quant_act would. This saves the separate quantisation launch at the cost of quantising each tile once per
// workgroup of the tile (MH / 256 / RPB of them).
#define DN_LROW (MFF + 16)
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
template <int RPB, bool D16, bool QIN = false>
__global__ void __launch_bounds__(256, 2) k_down_tile(const Plan *__restrict__ plan, const Tile *__restrict__ tiles,
                                                      const ExpPtr *__restrict__ eptr, const int8_t *__restrict__ qa,
                                                      const float *__restrict__ qsa, const int *__restrict__ qsuma,
                                                      float *__restrict__ down, int *__restrict__ dov, int *__restrict__ dbg,
                                                      const float *__restrict__ act = nullptr, int8_t *__restrict__ qa_w = nullptr,
                                                      float *__restrict__ qsa_w = nullptr, int *__restrict__ qsuma_w = nullptr) {
    constexpr int TN = 64, NT = 256, NF = 2, NA = 2, NSPLIT = MH / 256 / RPB;
    constexpr int NPC = TN * (MFF / 16) / NT;   // 8 pieces of 16 bytes per thread
    __shared__ __attribute__((aligned(16))) int8_t bs[TN * DN_LROW];
    __shared__ __attribute__((aligned(16))) float sds[D16 ? 4 : MH];   // the expert's down scales (fp32 output)
    constexpr int DT_LD = 72;                                       // int16 per pair row of the output tiles
    __shared__ __attribute__((aligned(16))) int16_t dtw[D16 ? 4 * 32 * DT_LD : 8];   // one [32 pairs][64 rows] tile per wave
    int item = xcd_item(blockIdx.x, plan->ntile_gu * NSPLIT);
    if (item < 0) return;
    int tile = item / NSPLIT, rb0 = (item % NSPLIT) * RPB;
    Tile tl = tiles[tile];
    int p0 = tl.p0, ntok = tl.n;
    const uint8_t *dcb = eptr[tl.u].dc;
    const float *dsb = eptr[tl.u].ds;
    int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, G2 = l >> 5, r32 = l & 31;
    uint32_t aoff = (uint32_t)(wv * 64 + r32) * (MFF / 4) + G2 * 32;   // row block 0, fragment 0
    v4i cw[2][NA][2][2];   // [row block parity][fragment][chunk][16 bytes]
#define DN_LOADC(slot_, rb_)                                                                                   \
    {                                                                                                          \
        _Pragma("unroll") for (int f = 0; f < NA; f++)                                                         \
        _Pragma("unroll") for (int c = 0; c < 2; c++) {                                                        \
            const uint8_t *ap = dcb + aoff + (uint32_t)((rb_) * 256 + f * 32) * (MFF / 4) + c * 64;            \
            cw[slot_][f][c][0] = *(const gptr_u4 *)ap;                                                         \
            cw[slot_][f][c][1] = *(const gptr_u4 *)(ap + 16);                                                  \
        }                                                                                                      \
    }
    DN_LOADC(0, rb0);
    float qs[NF]; int qsm[NF];
    __shared__ float sqs[QIN ? TN : 1];
    __shared__ int sqsum[QIN ? TN : 1];
    if (!QIN) {
#pragma unroll
        for (int j = 0; j < NF; j++) { int pr = p0 + min(j * 32 + r32, ntok - 1); qs[j] = qsa[pr]; qsm[j] = qsuma[pr]; }
#pragma unroll
        for (int k = 0; k < NPC; k++) {
            int i = tid + k * NT, tk = i >> 5, part = i & 31;
            if (tk < ntok)   // rows of absent pairs only feed outputs that are never stored
                *(v4i *)(&bs[tk * DN_LROW + part * 16]) = *(const gptr_u4 *)(qa + (size_t)(p0 + tk) * MFF + part * 16);
        }
    } else {
        // half-wave h of wave w takes pair 8k + 2w + h; lane o = l % 32 quantises the 16 values of mfma-order
        // part o (columns g*128 + s*32 + hh*16 + tq*4 + b, g = o/8, hh = o/4 % 2, tq = o % 4), as k_quant_act
        int o = l & 31, g = o >> 3, hh = (o >> 2) & 1, tq = o & 3;
#pragma unroll 2
        for (int k = 0; k < NPC; k++) {
            int tk = (tid >> 5) + 8 * k;
            float v[16];
            if (tk < ntok) {
                const float *ar = act + (size_t)(p0 + tk) * MFF + g * 128 + hh * 16 + tq * 4;
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++) {
                    float4 f = *(const float4 *)(ar + q4 * 32);
                    v[q4 * 4] = f.x; v[q4 * 4 + 1] = f.y; v[q4 * 4 + 2] = f.z; v[q4 * 4 + 3] = f.w;
                }
            } else {
#pragma unroll
                for (int q4 = 0; q4 < 16; q4++) v[q4] = 0.0f;
            }
            quant_half<128>(v, l, bs + tk * DN_LROW, &sqs[tk], &sqsum[tk]);
        }
    }
    if (!D16 && tid < RPB * 64) *(float4 *)(&sds[rb0 * 256 + tid * 4]) = *(const float4 *)(dsb + rb0 * 256 + tid * 4);
    __syncthreads();
    if (QIN) {
#pragma unroll
        for (int j = 0; j < NF; j++) { int tk = min(j * 32 + r32, ntok - 1); qs[j] = sqs[tk]; qsm[j] = sqsum[tk]; }
        if (rb0 == 0) {   // the tile's int8 act as k_quant_act writes it
#pragma unroll
            for (int k = 0; k < NPC; k++) {
                int i = tid + k * NT, tk = i >> 5, part = i & 31;
                if (tk < ntok) {
                    *(v4i *)(qa_w + (size_t)(p0 + tk) * MFF + part * 16) = *(const v4i *)(&bs[tk * DN_LROW + part * 16]);
                    if (part == 0) { qsa_w[p0 + tk] = sqs[tk]; qsuma_w[p0 + tk] = sqsum[tk]; }
                }
            }
        }
    }
#pragma unroll
    for (int rr = 0; rr < RPB; rr++) {
        int rb = rb0 + rr;
        if (rr + 1 < RPB) DN_LOADC((rr + 1) & 1, rb + 1);
        v16i acc[NA][NF];
#pragma unroll
        for (int f = 0; f < NA; f++)
#pragma unroll
            for (int j = 0; j < NF; j++)
#pragma unroll
                for (int i = 0; i < 16; i++) acc[f][j][i] = 0;
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int t = 0; t < 8; t++) {
                int part = c * 16 + G2 * 8 + t;
                v4i bv[NF];
#pragma unroll
                for (int j = 0; j < NF; j++) bv[j] = *(const v4i *)(bs + (j * 32 + r32) * DN_LROW + part * 16);
#pragma unroll
                for (int f = 0; f < NA; f++) {
                    v4i c4 = cw[rr & 1][f][c][t >> 2];
                    int tt = t & 3;
                    v4i av = decode_word((uint32_t)(tt == 0 ? c4.x : tt == 1 ? c4.y : tt == 2 ? c4.z : c4.w));
#pragma unroll
                    for (int j = 0; j < NF; j++) acc[f][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv[j], acc[f][j], 0, 0, 0);
                }
            }
        // D[pair][row] = (float)(sum - qsum) * qs * s_down[row]; lane: pair j*32 + r32, rows (i/4)*8 + G2*4 + i%4
        if (D16) {
            // d = sum - qsum as int16 into the wave's LDS tile [32 pairs][64 rows], one pair fragment at a time,
            // then out as 8 pairs x 128 bytes per store (lane: pair l/8 + 8k, 16-byte piece l%8)
            // range check of the live pairs' 64 values per lane at once (sum within qsum +- 32767); only a wave
            // holding a value outside takes the per-value path (marker -32768 and the int32 side entry)
            int16_t *tw = dtw + wv * (32 * DT_LD);
            bool bad = false;
#pragma unroll
            for (int j = 0; j < NF; j++) {
                int mn = acc[0][j][0], mx = mn;
#pragma unroll
                for (int f = 0; f < NA; f++)
#pragma unroll
                    for (int i = 0; i < 16; i++) { mn = min(mn, acc[f][j][i]); mx = max(mx, acc[f][j][i]); }
                bad |= j * 32 + r32 < ntok && (mn < qsm[j] - 32767 || mx > qsm[j] + 32767);
            }
            const bool wbad = __ballot(bad) != 0;
            u16x2 qsm2[NF];
#pragma unroll
            for (int j = 0; j < NF; j++) qsm2[j] = u16x2{(uint16_t)qsm[j], (uint16_t)qsm[j]};
#pragma unroll
            for (int j = 0; j < NF; j++) {
#pragma unroll
                for (int f = 0; f < NA; f++)
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        int rl = f * 32 + g * 8 + G2 * 4, tk = j * 32 + r32;
                        uint32_t w2[2];
#pragma unroll
                        for (int h = 0; h < 2; h++) {   // low halves of two sums, minus qsum mod 2^16 in each half
                            uint32_t pk = __builtin_amdgcn_perm((uint32_t)acc[f][j][g * 4 + 2 * h + 1], (uint32_t)acc[f][j][g * 4 + 2 * h], 0x05040100u);
                            w2[h] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, pk) - qsm2[j]);
                        }
                        if (wbad) {
#pragma unroll
                            for (int i = 0; i < 4; i++) {
                                int d = acc[f][j][g * 4 + i] - qsm[j];
                                if (d >= -32767 && d <= 32767) continue;
                                if (tk < ntok) dov[(size_t)(p0 + tk) * MH + rb * 256 + wv * 64 + rl + i] = d;
                                w2[i >> 1] = (w2[i >> 1] & (0xffff0000u >> (16 * (i & 1)))) | (0x8000u << (16 * (i & 1)));
                            }
                        }
                        *(uint2 *)(tw + r32 * DT_LD + rl) = make_uint2(w2[0], w2[1]);
                    }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    int pl = k * 8 + (l >> 3), pc = l & 7, tk = j * 32 + pl;
                    uint4 v = *(const uint4 *)(tw + pl * DT_LD + pc * 8);
                    if (tk < ntok) *(uint4 *)((int16_t *)down + (size_t)(p0 + tk) * MH + rb * 256 + wv * 64 + pc * 8) = v;
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");   // the tile is rewritten next
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
            continue;
        }
#pragma unroll
        for (int j = 0; j < NF; j++) {
            int tk = j * 32 + r32;
            if (tk >= ntok) continue;
            int pair = p0 + tk;
#pragma unroll
            for (int f = 0; f < NA; f++)
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    int row0 = rb * 256 + wv * 64 + f * 32 + g * 8 + G2 * 4;
                    float4 sd = *(const float4 *)(&sds[row0]);
                    float sdv[4] = {sd.x, sd.y, sd.z, sd.w};
                    int ad[4]; float o[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) { ad[i] = acc[f][j][g * 4 + i]; o[i] = (float)(ad[i] - qsm[j]) * qs[j] * sdv[i]; }
                    *(float4 *)(down + (size_t)pair * MH + row0) = make_float4(o[0], o[1], o[2], o[3]);
                    if (dbg) *(int4 *)(dbg + (size_t)pair * MH + row0) = make_int4(ad[0], ad[1], ad[2], ad[3]);
                }
        }
    }
#undef DN_LOADC
}

// =====================================================================================================
// Combine, flag bits of mode: 1 = start from x (else from 0), 2 = slot order (sp/tw, else ascending pair
// order tp/uw), 4 = add the chain to x at the end (else store it).
//   step_batch maple.c:834            mode 1: x[b] = fma(uw[a], D[a], x[b]) over b's pairs in ascending order
//   gpre_moe cmb gpu_pre.m:158-163    mode 0: y[b] = the same FMA chain from 0
//   gfull_moe cmba gpu_full.metal:212 mode 4: x[b] += (FMA chain from 0)
//   step maple.c:664                  mode 6: y = FMA chain over slots 0..7 from 0, x[b] += y
// Thread = 4 columns of one token.
// =====================================================================================================
// Combine from int16 down results (k_down_tile<., true>): block = one token, 256 threads x 8 columns. The
// token's 8 pairs (tp/sp order as k_combine), their weights, qs and down-scale rows are looked up once into
// LDS; then D = (float)d * qs * s_down[row] (k_down_tile's operations) and the same FMA chain as k_combine.
__global__ void __launch_bounds__(256) k_combine16(const int16_t *__restrict__ down, const float *__restrict__ uw,
                                                   const int *__restrict__ tp, const int *__restrict__ sp,
                                                   const float *__restrict__ tw, int nb, float *__restrict__ x, int mode,
                                                   const int *__restrict__ pu, const ExpPtr *__restrict__ eptr,
                                                   const float *__restrict__ qsa, const int *__restrict__ dov,
                                                   int *__restrict__ hz, int hzn) {
    if (hz && (int)(blockIdx.x * 256 + threadIdx.x) < hzn) hz[blockIdx.x * 256 + threadIdx.x] = 0;   // k_group's counts, for the next call
    __shared__ int sa[MTOPK];
    __shared__ float sw[MTOPK], sq[MTOPK];
    __shared__ const float *sds[MTOPK];
    int b = blockIdx.x, t = threadIdx.x, c = t * 8;
    if (t < MTOPK) {
        int a = (mode & 2) ? sp[b * MTOPK + t] : tp[b * MTOPK + t];
        sa[t] = a; sw[t] = (mode & 2) ? tw[b * MTOPK + t] : uw[a];
        sq[t] = qsa[a]; sds[t] = eptr[pu[a]].ds;
    }
    float *xp = x + (size_t)b * MH + c;
    float acc[8];
    if (mode & 1) {
        float4 x0 = *(const float4 *)xp, x1 = *(const float4 *)(xp + 4);
        acc[0] = x0.x; acc[1] = x0.y; acc[2] = x0.z; acc[3] = x0.w; acc[4] = x1.x; acc[5] = x1.y; acc[6] = x1.z; acc[7] = x1.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) acc[i] = 0.0f;
    }
    __syncthreads();
    // the 8 pairs in two groups of 4, each group's loads issued together (the barrier keeps the second group's
    // loads from being hoisted: about 80 VGPRs, so three waves share a SIMD instead of one)
#pragma unroll
    for (int jg = 0; jg < MTOPK; jg += 4) {
        uint4 dv[4];
        v4f s0[4], s1[4];
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            // global (not generic) loads: a generic load also counts in the LDS counter, so the wait for the next
            // pointer read from LDS would wait for it too and serialise the four rows
            const gptr_f4 *ds = (const gptr_f4 *)(sds[jg + jj] + c);
            s0[jj] = ds[0]; s1[jj] = ds[1];
        }
#pragma unroll
        for (int jj = 0; jj < 4; jj++) dv[jj] = *(const uint4 *)(down + (size_t)sa[jg + jj] * MH + c);
        bool ovf = false;   // any -32768 marker (its d is in dov): rare, handled by a compact loop
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            uint32_t w4[4] = {dv[jj].x, dv[jj].y, dv[jj].z, dv[jj].w};
#pragma unroll
            for (int k = 0; k < 4; k++) ovf |= ((w4[k] & 0xffffu) == 0x8000u) | ((w4[k] >> 16) == 0x8000u);
        }
        // one path for both cases (the scale rows are used unconditionally, so their loads stay with the int16
        // loads); an entry marked -32768 takes its int32 value from dov (rare)
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            int j = jg + jj;
            float sdv[8] = {s0[jj].x, s0[jj].y, s0[jj].z, s0[jj].w, s1[jj].x, s1[jj].y, s1[jj].z, s1[jj].w};
            uint32_t wd[4] = {dv[jj].x, dv[jj].y, dv[jj].z, dv[jj].w};
            int d[8];
#pragma unroll
            for (int i = 0; i < 8; i++) d[i] = (int16_t)(wd[i >> 1] >> (16 * (i & 1)));
            if (ovf) {
#pragma unroll 1
                for (int i = 0; i < 8; i++)
                    if (d[i] == -32768) d[i] = dov[(size_t)sa[j] * MH + c + i];
            }
            float qs = sq[j], wgt = sw[j];
#pragma unroll
            for (int i = 0; i < 8; i++) acc[i] = __builtin_fmaf(wgt, (float)d[i] * qs * sdv[i], acc[i]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    if (mode & 4) {
        float4 x0 = *(const float4 *)xp, x1 = *(const float4 *)(xp + 4);
        float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int i = 0; i < 8; i++) acc[i] = xv[i] + acc[i];
    }
    *(float4 *)xp = make_float4(acc[0], acc[1], acc[2], acc[3]);
    *(float4 *)(xp + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
}

__global__ void __launch_bounds__(256) k_combine(const float *__restrict__ down, const float *__restrict__ uw,
                                                 const int *__restrict__ tp, const int *__restrict__ sp,
                                                 const float *__restrict__ tw, int nb, float *__restrict__ x, int mode,
                                                 int *__restrict__ hz = nullptr, int hzn = 0) {
    int gid = blockIdx.x * 256 + threadIdx.x;
    if (hz && gid < hzn) hz[gid] = 0;   // k_group's counts, for the next call
    int b = gid / (MH / 4), c = (gid % (MH / 4)) * 4;
    if (b >= nb) return;
    float4 *xp = (float4 *)(x + (size_t)b * MH + c);
    float4 acc = (mode & 1) ? *xp : make_float4(0.f, 0.f, 0.f, 0.f);
    // the token's 8 pair ids, then their weights and down rows, each level's loads issued together
    int a[MTOPK]; float w[MTOPK]; float4 d[MTOPK];
#pragma unroll
    for (int j = 0; j < MTOPK; j++) a[j] = (mode & 2) ? sp[b * MTOPK + j] : tp[b * MTOPK + j];
#pragma unroll
    for (int j = 0; j < MTOPK; j++) {
        w[j] = (mode & 2) ? tw[b * MTOPK + j] : uw[a[j]];
        d[j] = *(const float4 *)(down + (size_t)a[j] * MH + c);
    }
#pragma unroll
    for (int j = 0; j < MTOPK; j++) {
        acc.x = __builtin_fmaf(w[j], d[j].x, acc.x); acc.y = __builtin_fmaf(w[j], d[j].y, acc.y);
        acc.z = __builtin_fmaf(w[j], d[j].z, acc.z); acc.w = __builtin_fmaf(w[j], d[j].w, acc.w);
    }
    if (mode & 4) { float4 xv = *xp; acc.x = xv.x + acc.x; acc.y = xv.y + acc.y; acc.z = xv.z + acc.z; acc.w = xv.w + acc.w; }
    *xp = acc;
}
