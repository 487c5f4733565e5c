// Sustained f16 MFMA rate of the GPU the library runs on, for the benchmark's
// roofline: every SIMD runs four waves of independent
// v_mfma_f32_32x32x16_f16 (eight accumulators per wave, no memory traffic in
// the loop) on operands that are either all zero or pseudo-random in
// [-1, 1).  The MI355X lowers its core clock under a sustained matrix load
// by an amount that depends on the operand bits (the switching activity of
// the multipliers), so the rate an MFMA-bound kernel can reach is the one
// measured with random operands, below the published peak that assumes the
// full boost clock.  The core clock seen by one wave is read from the shader
// cycle counter (s_memtime) against the 100 MHz constant clock
// (s_memrealtime) over the loop.
#include "tpmd.h"
#include "tpmd_device.h"

namespace tpmd {

constexpr int PROBE_WG = 1024;   // workgroups of 4 waves: four waves on each of the 1024 SIMDs

// f16 in [-1, 1) from a 32-bit hash of (lane, slot)
__device__ __forceinline__ half_t probe_operand(unsigned lane, unsigned slot) {
    unsigned h = lane * 0x9E3779B1u ^ (slot + 0x7F4A7C15u) * 0x85EBCA77u;
    h ^= h >> 15;
    h *= 0x2C1B3C6Du;
    h ^= h >> 12;
    return (half_t) ((float) (h >> 8) * (2.0f / 16777216.0f) - 1.0f);
}

__global__ __launch_bounds__(256) void mfma_probe_kernel(int random, int iters, float *out,
                                                         unsigned long long *clk) {
    const unsigned l = threadIdx.x & 63;
    half8 a0, a1, b0, b1;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        a0[e] = random ? probe_operand(l, e) : (half_t) 0.0f;
        a1[e] = random ? probe_operand(l, 8 + e) : (half_t) 0.0f;
        b0[e] = random ? probe_operand(l, 16 + e) : (half_t) 0.0f;
        b1[e] = random ? probe_operand(l, 24 + e) : (half_t) 0.0f;
    }
    floatx16 c[8];
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
        for (int v = 0; v < 16; v++) c[j][v] = 0.0f;
    const unsigned long long t0 = __builtin_amdgcn_s_memtime();
    const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; it++) {
        c[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b0, c[0], 0, 0, 0);
        c[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b0, c[1], 0, 0, 0);
        c[2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b1, c[2], 0, 0, 0);
        c[3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b1, c[3], 0, 0, 0);
        c[4] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b0, a0, c[4], 0, 0, 0);
        c[5] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b1, a0, c[5], 0, 0, 0);
        c[6] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b0, a1, c[6], 0, 0, 0);
        c[7] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b1, a1, c[7], 0, 0, 0);
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime();
    const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
        for (int v = 0; v < 16; v++) s += c[j][v];
    out[blockIdx.x * 256 + threadIdx.x] = s;   // keeps the MFMAs live
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        clk[0] = t1 - t0;
        clk[1] = r1 - r0;
    }
}

}  // namespace tpmd

extern "C" int tpmd_probe_mfma_f16(int random_operands, int iters, float *tflops, float *core_ghz) {
    using namespace tpmd;
    if (iters < 1 || iters > (1 << 20) || !tflops || !core_ghz) return -1;
    float *out = nullptr;
    unsigned long long *clk = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    constexpr int timed = 10;
    bool ok = hipMalloc(&out, (size_t) PROBE_WG * 256 * sizeof(float)) == hipSuccess &&
              hipMalloc(&clk, 2 * sizeof(unsigned long long)) == hipSuccess &&
              hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess;
    float ms = 0.0f;
    unsigned long long c[2] = {0, 0};
    if (ok) {
        for (int k = 0; k < 3 + timed && ok; k++) {
            if (k == 3) ok = hipEventRecord(e0, nullptr) == hipSuccess;
            hipLaunchKernelGGL(mfma_probe_kernel, dim3(PROBE_WG), dim3(256), 0, nullptr, random_operands ? 1 : 0,
                               iters, out, clk);
            ok = ok && hipGetLastError() == hipSuccess;
        }
        ok = ok && hipEventRecord(e1, nullptr) == hipSuccess && hipEventSynchronize(e1) == hipSuccess &&
             hipEventElapsedTime(&ms, e0, e1) == hipSuccess &&
             hipMemcpy(c, clk, sizeof(c), hipMemcpyDeviceToHost) == hipSuccess;
    }
    if (e0) (void) hipEventDestroy(e0);
    if (e1) (void) hipEventDestroy(e1);
    if (out) (void) hipFree(out);
    if (clk) (void) hipFree(clk);
    if (!ok || ms <= 0.0f || c[1] == 0) return -1;
    const double flop = (double) timed * PROBE_WG * 4 * (double) iters * 8 * 32768.0;
    *tflops = (float) (flop / (ms * 1e-3) * 1e-12);
    *core_ghz = (float) ((double) c[0] / ((double) c[1] / 100e6) * 1e-9);
    return 0;
}
