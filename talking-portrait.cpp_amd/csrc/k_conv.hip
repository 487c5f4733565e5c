// Modulated 3x3 convolution as an MFMA implicit GEMM for gfx950.
//
// One kernel template serves both decoder convolutions of a stage:
//   MODE_DENSE : ModulatedConv2d 3x3 pad 1 (styled_conv, src/motion_dec.cpp:357-373)
//   MODE_SUBPIX: the composed sub-pixel up-conv — conv_transpose(3x3, s2) o
//                Blur(4x4) folded into one 3x3 pad-1 conv with 4*OC outputs,
//                one per output parity class (styled_conv_up + subpix_lrelu_cl,
//                src/motion_dec.cpp:397-433, patch :980-994)
//
// GEMM view (channels-first im2col fused into the B-operand loader, never
// materialised):  Y[m][n] = sum_k A[m][k] * X(k, n)
//   m : output channel (MODE_SUBPIX: q = k*OC + o, parity k = 2*by + bx)
//   n : input pixel (frame, y, x), flattened over the batch
//   k : tap*IC + ic  (tap = 3*kh + kw), the reference's cf row order
//       r = ic + IC*(kw + 3*kh)
//   X(k, n) = x[frame][y+kh-1][x+kw-1][ic], zero outside the map.
// Style modulation is applied to the input activation by its producer (the
// stored activation is x * s for this conv), so A is shared by every frame of
// the batch and streamed once per tile row; demodulation (1/den), the
// FusedLeakyReLU bias + leaky and the NEXT conv's style are fused into the
// epilogue.
//
// Tiling: BM x BN block tile, BK-wide k tiles staged through LDS
// (double-buffered, 16-byte rows padded to 144 B so every 32x32 MFMA operand
// read is one bank-conflict-free ds_read_b128), WM x WN waves each owning a
// (BM/WM) x (BN/WN) tile of 32x32 MFMA accumulators.
//   f16: v_mfma_f32_32x32x16_f16 (f16 in, f32 accumulate)
//   f32: v_mfma_f32_32x32x2_f32, four per 16-byte operand read; the lane's k
//        assignment is a permutation shared by A and B, so every product pairs
//        A[m][k] with X(k, n) exactly once.
#include "tpmd_device.h"
#include "tpmd_launch.h"

namespace tpmd {

enum { MODE_DENSE = 0, MODE_SUBPIX = 1 };

template <typename TA>
struct mfma_op;

template <>
struct mfma_op<half_t> {
    __device__ __forceinline__ static void run(const uint4 &a, const uint4 &b, floatx16 &c) {
        c = __builtin_amdgcn_mfma_f32_32x32x16_f16(*(const half8 *) &a, *(const half8 *) &b, c, 0, 0,
                                                   0);
    }
};

template <>
struct mfma_op<float> {
    __device__ __forceinline__ static void run(const uint4 &a, const uint4 &b, floatx16 &c) {
        const floatx4 av = *(const floatx4 *) &a, bv = *(const floatx4 *) &b;
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(av[0], bv[0], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(av[1], bv[1], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(av[2], bv[2], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(av[3], bv[3], c, 0, 0, 0);
    }
};

template <typename T> __device__ __forceinline__ void store4(T *p, float a, float b, float c, float d);
template <> __device__ __forceinline__ void store4<float>(float *p, float a, float b, float c, float d) {
    *(floatx4 *) p = floatx4{a, b, c, d};
}
template <> __device__ __forceinline__ void store4<half_t>(half_t *p, float a, float b, float c, float d) {
    *(half4 *) p = half4{(half_t) a, (half_t) b, (half_t) c, (half_t) d};
}

// RB: bytes of one k tile row (128 or 64); BK = RB / sizeof(act) must divide IC
template <typename TA, typename TO, int BM, int BN, int WM, int WN, int MODE, int RB>
__global__ __launch_bounds__(WM *WN * 64) void modconv3x3_kernel(
    const TA *__restrict__ A,        // [M][9*IC]
    const TA *__restrict__ X,        // CL input, frame stride x_bstride elements
    TO *__restrict__ Y,              // CL output
    const float *__restrict__ inv_den,   // [B][OC]
    const float *__restrict__ bias,      // [OC]
    const float *__restrict__ out_scale, // [B][OC] or null
    int N, int H, int W, int IC, int OC, int64_t x_bstride) {
    constexpr int NT = WM * WN * 64;
    constexpr int kRowBytes = RB;
    constexpr int kRowStride = RB + 16;           // padded LDS row (bytes)
    constexpr int BK = RB / (int) sizeof(TA);     // elements per k tile
    constexpr int VEC = 16 / sizeof(TA);          // elements per 16-byte chunk
    constexpr int CR = kRowBytes / 16;            // chunks per LDS row
    constexpr int A_PER = (BM * CR + NT - 1) / NT;  // A chunks per thread
    constexpr int B_PER = (BN * CR + NT - 1) / NT;  // B chunks per thread
    constexpr bool A_PART = BM * CR < NT;         // only the first BM*CR threads load A
    constexpr bool B_PART = BN * CR < NT;
    constexpr int ROWS_PER_PASS = NT / CR;
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    static_assert((BM * CR) % NT == 0 || A_PART, "A tile/threads");
    static_assert((BN * CR) % NT == 0 || B_PART, "B tile/threads");
    static_assert(TM >= 1 && TN >= 1, "wave tile");

    __shared__ __attribute__((aligned(16))) char smem[2 * (BM + BN) * kRowStride];
    // buffer b: A tile at smem + b*(BM+BN)*kRowStride, B tile right after it
    constexpr int kBufBytes = (BM + BN) * kRowStride;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wid = tid >> 6;
    const int wm = wid / WN, wn = wid % WN;
    const int m0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * BN;
    const int K = 9 * IC;
    const int HW = H * W;
    const int kc = tid % CR;         // this thread's 16-byte chunk within a row
    const int prow = tid / CR;       // first row this thread loads

    // B-loader pixel bookkeeping (fixed across the k loop)
    int py[B_PER], px[B_PER];
    int64_t pbase[B_PER];            // element offset of (frame, 0, 0)
    bool pval[B_PER];
#pragma unroll
    for (int i = 0; i < B_PER; i++) {
        const int n = n0 + prow + i * ROWS_PER_PASS;
        pval[i] = n < N;
        const int nn = pval[i] ? n : 0;
        const int b = nn / HW, rem = nn - b * HW;
        py[i] = rem / W;
        px[i] = rem - py[i] * W;
        pbase[i] = (int64_t) b * x_bstride;
    }

    uint4 ra[A_PER], rb[B_PER];
    const int kt_per_tap = IC / BK;
    const int T = 9 * kt_per_tap;

    auto load_tiles = [&](int t) {
        const int tap = t / kt_per_tap;
        const int ic0 = (t - tap * kt_per_tap) * BK;
        const int dy = tap / 3 - 1, dx = tap % 3 - 1;
        const int kofs = t * BK + kc * VEC;
#pragma unroll
        for (int i = 0; i < A_PER; i++) {
            if (A_PART && prow >= BM) continue;
            const int m = m0 + prow + i * ROWS_PER_PASS;
            ra[i] = *(const uint4 *) (A + (int64_t) m * K + kofs);
        }
#pragma unroll
        for (int i = 0; i < B_PER; i++) {
            if (B_PART && prow >= BN) continue;
            const int iy = py[i] + dy, ix = px[i] + dx;
            if (pval[i] && iy >= 0 && iy < H && ix >= 0 && ix < W) {
                rb[i] = *(const uint4 *) (X + pbase[i] + (int64_t) (iy * W + ix) * IC + ic0 + kc * VEC);
            } else {
                rb[i] = uint4{0u, 0u, 0u, 0u};
            }
        }
    };
    auto store_tiles = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_PER; i++)
            if (!A_PART || prow < BM)
                *(uint4 *) (smem + buf * kBufBytes + (prow + i * ROWS_PER_PASS) * kRowStride + kc * 16) = ra[i];
#pragma unroll
        for (int i = 0; i < B_PER; i++)
            if (!B_PART || prow < BN)
                *(uint4 *) (smem + buf * kBufBytes + BM * kRowStride + (prow + i * ROWS_PER_PASS) * kRowStride + kc * 16) = rb[i];
    };

    floatx16 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; a++)
#pragma unroll
        for (int b = 0; b < TN; b++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[a][b][v] = 0.0f;

    load_tiles(0);
    store_tiles(0);
    __syncthreads();

    const int lrow = lane & 31;
    const int lk = (lane >> 5) * 16;  // byte offset of this lane's k chunk
    for (int t = 0; t < T; t++) {
        const int cur = t & 1;
        if (t + 1 < T) load_tiles(t + 1);
#pragma unroll
        for (int ks = 0; ks < kRowBytes / 32; ks++) {
            uint4 af[TM], bf[TN];
#pragma unroll
            for (int a = 0; a < TM; a++)
                af[a] = *(const uint4 *) (smem + cur * kBufBytes + (wm * WTM + a * 32 + lrow) * kRowStride + ks * 32 + lk);
#pragma unroll
            for (int b = 0; b < TN; b++)
                bf[b] = *(const uint4 *) (smem + cur * kBufBytes + BM * kRowStride + (wn * WTN + b * 32 + lrow) * kRowStride + ks * 32 + lk);
#pragma unroll
            for (int a = 0; a < TM; a++)
#pragma unroll
                for (int b = 0; b < TN; b++) mfma_op<TA>::run(af[a], bf[b], acc[a][b]);
        }
        if (t + 1 < T) store_tiles(cur ^ 1);
        __syncthreads();
    }

    // epilogue: 1/den, + bias, leaky, * next style, store (4 channels / lane)
#pragma unroll
    for (int b = 0; b < TN; b++) {
        const int n = n0 + wn * WTN + b * 32 + lrow;
        if (n >= N) continue;
        const int fr = n / HW, rem = n - fr * HW;
        const int y = rem / W, x = rem - y * W;
#pragma unroll
        for (int a = 0; a < TM; a++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = m0 + wm * WTM + a * 32 + i * 8 + (lane >> 5) * 4;
                int o;
                int64_t opix;
                if (MODE == MODE_DENSE) {
                    o = m;
                    opix = n;
                } else {
                    const int cls = m / OC;
                    o = m - cls * OC;
                    opix = (int64_t) fr * 4 * HW + (int64_t) (2 * y + (cls >> 1)) * (2 * W) + 2 * x + (cls & 1);
                }
                const floatx4 id = *(const floatx4 *) (inv_den + (int64_t) fr * OC + o);
                const floatx4 bb = *(const floatx4 *) (bias + o);
                float v[4];
#pragma unroll
                for (int j = 0; j < 4; j++) v[j] = leaky(acc[a][b][i * 4 + j] * id[j] + bb[j]);
                if (out_scale) {
                    const floatx4 sc = *(const floatx4 *) (out_scale + (int64_t) fr * OC + o);
#pragma unroll
                    for (int j = 0; j < 4; j++) v[j] *= sc[j];
                }
                store4<TO>(Y + opix * OC + o, v[0], v[1], v[2], v[3]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// launch: pick the tile shape from M (= OC or 4*OC)

template <typename TA, typename TO, int BM, int BN, int WM, int WN, int RB>
static hipError_t launch_cfg_rb(int mode, const TA *A, const TA *X, TO *Y, const float *inv_den,
                                const float *bias, const float *out_scale, int N, int H, int W,
                                int IC, int OC, int64_t x_bstride, hipStream_t st) {
    const int M = mode == MODE_DENSE ? OC : 4 * OC;
    dim3 grid((N + BN - 1) / BN, M / BM);
    dim3 block(WM * WN * 64);
    if (mode == MODE_DENSE)
        hipLaunchKernelGGL((modconv3x3_kernel<TA, TO, BM, BN, WM, WN, MODE_DENSE, RB>), grid, block,
                           0, st, A, X, Y, inv_den, bias, out_scale, N, H, W, IC, OC, x_bstride);
    else
        hipLaunchKernelGGL((modconv3x3_kernel<TA, TO, BM, BN, WM, WN, MODE_SUBPIX, RB>), grid, block,
                           0, st, A, X, Y, inv_den, bias, out_scale, N, H, W, IC, OC, x_bstride);
    return hipGetLastError();
}

template <typename TA, typename TO, int BM, int BN, int WM, int WN>
static hipError_t launch_cfg(int mode, const TA *A, const TA *X, TO *Y, const float *inv_den,
                             const float *bias, const float *out_scale, int N, int H, int W,
                             int IC, int OC, int64_t x_bstride, hipStream_t st) {
    if ((IC * (int) sizeof(TA)) % 128 == 0)
        return launch_cfg_rb<TA, TO, BM, BN, WM, WN, 128>(mode, A, X, Y, inv_den, bias, out_scale, N,
                                                          H, W, IC, OC, x_bstride, st);
    return launch_cfg_rb<TA, TO, BM, BN, WM, WN, 64>(mode, A, X, Y, inv_den, bias, out_scale, N, H,
                                                     W, IC, OC, x_bstride, st);
}

template <typename TA, typename TO>
static hipError_t launch_modconv_typed(int mode, const TA *A, const TA *X, TO *Y,
                                       const float *inv_den, const float *bias,
                                       const float *out_scale, int nframes, int H, int W, int IC,
                                       int OC, int64_t x_bstride, hipStream_t st) {
    const int M = mode == MODE_DENSE ? OC : 4 * OC;
    const int N = nframes * H * W;
    if (M % 128 == 0)
        return launch_cfg<TA, TO, 128, 128, 2, 2>(mode, A, X, Y, inv_den, bias, out_scale, N, H, W,
                                                  IC, OC, x_bstride, st);
    if (M % 64 == 0)
        return launch_cfg<TA, TO, 64, 128, 1, 4>(mode, A, X, Y, inv_den, bias, out_scale, N, H, W,
                                                 IC, OC, x_bstride, st);
    return launch_cfg<TA, TO, 32, 256, 1, 4>(mode, A, X, Y, inv_den, bias, out_scale, N, H, W, IC,
                                             OC, x_bstride, st);
}

// IC must be a multiple of this (the 64-byte k tile)
int modconv_k_align(bool f16) { return f16 ? 32 : 16; }

hipError_t launch_modconv(int mode, bool f16, bool out_f16, const void *A, const void *X, void *Y,
                          const float *inv_den, const float *bias, const float *out_scale,
                          int nframes, int H, int W, int IC, int OC, int64_t x_bstride,
                          hipStream_t st) {
    if (f16) {
        if (out_f16)
            return launch_modconv_typed<half_t, half_t>(mode, (const half_t *) A, (const half_t *) X,
                                                        (half_t *) Y, inv_den, bias, out_scale,
                                                        nframes, H, W, IC, OC, x_bstride, st);
        return launch_modconv_typed<half_t, float>(mode, (const half_t *) A, (const half_t *) X,
                                                   (float *) Y, inv_den, bias, out_scale, nframes,
                                                   H, W, IC, OC, x_bstride, st);
    }
    return launch_modconv_typed<float, float>(mode, (const float *) A, (const float *) X,
                                              (float *) Y, inv_den, bias, out_scale, nframes, H, W,
                                              IC, OC, x_bstride, st);
}

}  // namespace tpmd
