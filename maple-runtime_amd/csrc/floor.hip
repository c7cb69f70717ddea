// floor.hip -- libmaplefloor: the measured floor under the decode path's three dependent kernels per layer.
//
// Bench tooling, not part of the MoE path (bench.py --floor). It replays, as one HIP graph, 24 "layers" of three
// dependent kernels with the decode kernels' grid shapes (k_dec_route: 64 blocks of 64 threads; k_dec_gateup:
// 64 x 8 blocks of 256; k_dec_down: 256 blocks of 256), in three forms:
//   0  empty kernels: the dependent-launch cost alone;
//   1  every thread reads one 4-byte value the previous kernel wrote and writes one for the next: launch plus
//      a load round trip on data another kernel just produced (as logits -> top-8, act -> down);
//   2  as 1, then a second, dependent 16-byte load from a 1 GiB buffer at an address derived from the first
//      value (cold lines, as the expert codes a decode kernel fetches after reading the routing).
// The result is microseconds per layer (three kernels), averaged over `replays` graph replays.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#define FL_COLD_BYTES (1ull << 30)

template <int FORM>
__global__ void k_floor(const int *__restrict__ in, int *__restrict__ out, const uint4 *__restrict__ cold, uint32_t salt) {
    if (FORM == 0) return;
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    int v = in[i & 4095];
    if (FORM == 2) {
        uint32_t line = ((uint32_t)v * 2654435761u + salt + (uint32_t)i * 40503u) % (uint32_t)(FL_COLD_BYTES / 16);
        uint4 c = cold[line];
        v += (int)(c.x ^ c.w);
    }
    if ((i & 4095) == i) out[i] = v + 1;
}

static hipStream_t g_st;
static int *g_a, *g_b;
static uint4 *g_cold;

extern "C" double floor_layer_us(int form, int layers, int replays) {
    if (form < 0 || form > 2 || layers < 1 || replays < 1) return -1.0;
    if (!g_st) {
        if (hipStreamCreateWithFlags(&g_st, hipStreamNonBlocking) != hipSuccess) return -1.0;
        if (hipMalloc(&g_a, 4096 * 4) != hipSuccess || hipMalloc(&g_b, 4096 * 4) != hipSuccess) return -1.0;
        if (hipMalloc(&g_cold, FL_COLD_BYTES) != hipSuccess) return -1.0;
        if (hipMemsetAsync(g_a, 0, 4096 * 4, g_st) != hipSuccess || hipMemsetAsync(g_b, 0, 4096 * 4, g_st) != hipSuccess ||
            hipMemsetAsync(g_cold, 1, FL_COLD_BYTES, g_st) != hipSuccess || hipStreamSynchronize(g_st) != hipSuccess)
            return -1.0;
    }
    void (*k)(const int *, int *, const uint4 *, uint32_t) = form == 0 ? k_floor<0> : form == 1 ? k_floor<1> : k_floor<2>;
    hipGraph_t g;
    hipGraphExec_t ge;
    if (hipStreamBeginCapture(g_st, hipStreamCaptureModeThreadLocal) != hipSuccess) return -1.0;
    for (int L = 0; L < layers; L++) {
        hipLaunchKernelGGL(k, dim3(64), dim3(64), 0, g_st, g_a, g_b, g_cold, (uint32_t)(3 * L));
        hipLaunchKernelGGL(k, dim3(64, 8), dim3(256), 0, g_st, g_b, g_a, g_cold, (uint32_t)(3 * L + 1));
        hipLaunchKernelGGL(k, dim3(256), dim3(256), 0, g_st, g_a, g_b, g_cold, (uint32_t)(3 * L + 2));
    }
    if (hipStreamEndCapture(g_st, &g) != hipSuccess) return -1.0;
    if (hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) != hipSuccess) return -1.0;
    (void)hipGraphDestroy(g);
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -1.0;
    for (int i = 0; i < 3; i++) (void)hipGraphLaunch(ge, g_st);   // warm-up
    (void)hipEventRecord(e0, g_st);
    for (int i = 0; i < replays; i++) (void)hipGraphLaunch(ge, g_st);
    (void)hipEventRecord(e1, g_st);
    float ms = -1.0f;
    if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess) ms = -1.0f;
    (void)hipGraphExecDestroy(ge);
    (void)hipEventDestroy(e0); (void)hipEventDestroy(e1);
    return ms < 0 ? -1.0 : (double)ms * 1e3 / replays / layers;
}
