// LIA motion encoder (src/motion_enc.cpp:50-160, graph helpers
// src/ops_common.h:12-42), once per portrait: the EncoderApp pyramid on
// channel-last maps, the fc chain and the Direction product.
//
//   enc_stem_kernel   EqualConv2d(3, C0, 1) + FusedLeakyReLU on the CHW image
//   enc_blur_kernel   4x4 FIR with zero padding (ggml_pad_ext + conv_2d_dw_direct)
//   enc_conv_kernel   KxK conv, any stride / padding, as an implicit GEMM on
//                     MFMA (f16 or f32 operands, f32 accumulation), epilogue
//                     bias + leaky + residual, f32 output plus an optional
//                     copy in the next conv's operand type
//   enc_linear_kernel y = W x (+ b): the final 4x4 conv on the 4x4 map, the
//                     fc chain and motion = Q lambda
#include "tpmd_conv.h"
#include "tpmd_enc.h"

namespace tpmd {

// tanh-approximated GELU (ggml_gelu's formula): 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))
__device__ __forceinline__ float gelu_tanh(float x) {
    return 0.5f * x * (1.0f + tanhf(0.7978845608028654f * (x + 0.044715f * x * x * x)));
}

template <typename T> __device__ __forceinline__ T enc_cast(float v);
template <> __device__ __forceinline__ float enc_cast<float>(float v) { return v; }
template <> __device__ __forceinline__ half_t enc_cast<half_t>(float v) { return (half_t) v; }

template <typename TA>
__global__ __launch_bounds__(256) void enc_stem_kernel(const float *__restrict__ img, const float *__restrict__ w,
                                                       const float *__restrict__ b, int64_t HW, int C0,
                                                       float *__restrict__ y, TA *__restrict__ ya) {
    const int64_t total = HW * C0;
    for (int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t) gridDim.x * 256) {
        const int64_t p = i / C0;
        const int o = (int) (i - p * C0);
        float acc = w[o * 3] * img[p];
        acc = __builtin_fmaf(w[o * 3 + 1], img[HW + p], acc);
        acc = __builtin_fmaf(w[o * 3 + 2], img[2 * HW + p], acc);
        const float v = leaky(acc + b[o]);
        y[i] = v;
        if (ya) ya[i] = enc_cast<TA>(v);
    }
}

// one thread per output pixel and 4 consecutive channels (C % 4 == 0): one
// 16-byte load per tap and 32-bit index arithmetic; each channel's taps are
// summed in (row, column) order, out-of-map taps skipped
template <typename TO>
__global__ __launch_bounds__(256) void enc_blur_kernel(const float *__restrict__ x, const float *__restrict__ k,
                                                       int H, int W, int C, int pad, int OH, int OW,
                                                       TO *__restrict__ y) {
    const unsigned C4 = (unsigned) C >> 2;
    const unsigned total = (unsigned) OH * (unsigned) OW * C4;
    float kk[16];
#pragma unroll
    for (int t = 0; t < 16; t++) kk[t] = k[t];
    for (unsigned i = blockIdx.x * 256u + threadIdx.x; i < total; i += gridDim.x * 256u) {
        const unsigned pix = i / C4, c = (i - pix * C4) * 4u;
        const int oy = (int) (pix / (unsigned) OW), ox = (int) (pix - (unsigned) oy * (unsigned) OW);
        floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const int iy = oy + a - pad;
            if ((unsigned) iy >= (unsigned) H) continue;
#pragma unroll
            for (int bb = 0; bb < 4; bb++) {
                const int ix = ox + bb - pad;
                if ((unsigned) ix >= (unsigned) W) continue;
                const floatx4 v = *(const floatx4 *) (x + ((unsigned) (iy * W + ix) * (unsigned) C + c));
#pragma unroll
                for (int j = 0; j < 4; j++) acc[j] = __builtin_fmaf(kk[a * 4 + bb], v[j], acc[j]);
            }
        }
        TO *o = y + (size_t) pix * (size_t) C + c;
        if constexpr (sizeof(TO) == 4) {
            *(floatx4 *) o = acc;
        } else {
            store4<TO>(o, acc[0], acc[1], acc[2], acc[3]);
        }
    }
}

// bias, activation, gate, residual; f32 store and operand-type copy of 4
// consecutive outputs o..o+3 of pixel n
__device__ __forceinline__ void enc_epilogue(const EncConvParams &p, int n, int o, const float acc[4]) {
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        float a = acc[j];
        if (p.bias) a = a + p.bias[o + j];
        if (p.leaky == 1) a = leaky(a);
        else if (p.leaky == 2) a = gelu_tanh(a);
        if (p.gate) a = p.gate[(int64_t) n * p.gstride + o + j] * a;
        v[j] = a;
    }
    const int64_t off = (int64_t) n * p.OC + o;
    if (p.res) {
        const floatx4 r = *(const floatx4 *) (p.res + off);
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = r[j] + v[j];
    }
    if (p.Y) *(floatx4 *) (p.Y + off) = floatx4{v[0], v[1], v[2], v[3]};
    if (p.Ya) {
        if (p.ya_f16) store4<half_t>((half_t *) p.Ya + off, v[0], v[1], v[2], v[3]);
        else store4<float>((float *) p.Ya + off, v[0], v[1], v[2], v[3]);
    }
}

// 64 output channels x 64 output pixels per workgroup, k tiles of 32 input
// channels of one tap; 4 waves of 32 x 32 (one 32x32 MFMA accumulator each);
// operand rows in LDS padded by 16 bytes (conflict-free fragment reads); the
// next k tile is loaded into registers while the current one multiplies
template <typename TA>
__global__ __launch_bounds__(256) void enc_conv_kernel(EncConvParams p) {
    constexpr int BM = 64, BN = 64, BK = 32;
    constexpr int RB = BK * (int) sizeof(TA);       // bytes of a k-tile row
    constexpr int RS = RB + 16;                     // padded LDS row
    constexpr int CH = RB / 16;                     // 16-byte chunks per row
    constexpr int PT = BM * CH / 256;               // chunks per thread per operand
    constexpr int EPC = 16 / (int) sizeof(TA);      // elements per chunk
    constexpr int KS = RB / 32;                     // MFMA steps per k tile (16-byte fragments)
    __shared__ __attribute__((aligned(16))) char As[2][BM * RS];
    __shared__ __attribute__((aligned(16))) char Bs[2][BN * RS];

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid >> 1, wn = wid & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int IC = p.IC, OC = p.OC, N = p.OH * p.OW;
    const int K = p.KH * p.KW * IC;
    const int cpt = IC / BK;                        // k tiles per tap
    const int TT = p.KH * p.KW * cpt;
    const int ks_n = p.ksplit > 1 ? p.ksplit : 1, split = (int) blockIdx.z;
    const int t_begin = (int) ((int64_t) split * TT / ks_n), t_end = (int) ((int64_t) (split + 1) * TT / ks_n);
    const TA *A = (const TA *) p.A, *X = (const TA *) p.X;

    // this thread's chunks: chunk u = tid + i*256 -> row u / CH, chunk u % CH
    int arow[PT], brow_y[PT], brow_x[PT], cq[PT];
    bool bok[PT];
#pragma unroll
    for (int i = 0; i < PT; i++) {
        const int u = tid + i * 256;
        const int r = u / CH;
        cq[i] = u - r * CH;
        const int m = m0 + r;
        arow[i] = m < OC ? m : OC - 1;              // rows past OC: loaded, never stored
        const int n = n0 + r;
        bok[i] = n < N;
        const int nn = n < N ? n : N - 1;
        const int oy = nn / p.OW, ox = nn - oy * p.OW;
        brow_y[i] = oy * p.stride - p.pad;
        brow_x[i] = ox * p.stride - p.pad;
    }
    u32x4 ra[PT], rb[PT];
    auto load = [&](int t) {
        const int tap = t / cpt, ic0 = (t - tap * cpt) * BK;
        const int kh = tap / p.KW, kw = tap - kh * p.KW;
#pragma unroll
        for (int i = 0; i < PT; i++) {
            ra[i] = *(const u32x4 *) (A + (int64_t) arow[i] * K + (int64_t) tap * IC + ic0 + cq[i] * EPC);
            const int iy = brow_y[i] + kh, ix = brow_x[i] + kw;
            rb[i] = u32x4{0u, 0u, 0u, 0u};
            if (bok[i] && (unsigned) iy < (unsigned) p.H && (unsigned) ix < (unsigned) p.W)
                rb[i] = *(const u32x4 *) (X + ((int64_t) iy * p.W + ix) * IC + ic0 + cq[i] * EPC);
        }
    };
    auto store = [&](int s) {
#pragma unroll
        for (int i = 0; i < PT; i++) {
            const int u = tid + i * 256;
            const int r = u / CH;
            *(u32x4 *) (As[s] + r * RS + cq[i] * 16) = ra[i];
            *(u32x4 *) (Bs[s] + r * RS + cq[i] * 16) = rb[i];
        }
    };

    floatx16 acc;
#pragma unroll
    for (int v = 0; v < 16; v++) acc[v] = 0.0f;
    const int lrow = lane & 31, khalf = lane >> 5;
    load(t_begin);
    store(0);
    __syncthreads();
    for (int t = t_begin; t < t_end; t++) {
        const int s = (t - t_begin) & 1;
        if (t + 1 < t_end) load(t + 1);
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const int kc = ks * 2 + khalf;
            const u32x4 af = *(const u32x4 *) (As[s] + (wm * 32 + lrow) * RS + kc * 16);
            const u32x4 bf = *(const u32x4 *) (Bs[s] + (wn * 32 + lrow) * RS + kc * 16);
            mfma_op<TA>::run(af, bf, acc);
        }
        if (t + 1 < t_end) {
            store(s ^ 1);
            __syncthreads();
        }
    }

    // accumulator v: row (v/4)*8 + (lane/32)*4 + v%4, column lane%32
    const int n = n0 + wn * 32 + lrow;
    if (n >= N) return;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int o = m0 + wm * 32 + i * 8 + khalf * 4;
        if (o >= OC) continue;
        const float q[4] = {acc[i * 4], acc[i * 4 + 1], acc[i * 4 + 2], acc[i * 4 + 3]};
        if (ks_n > 1) *(floatx4 *) (p.ws + ((int64_t) split * N + n) * OC + o) = floatx4{q[0], q[1], q[2], q[3]};
        else enc_epilogue(p, n, o, q);
    }
}

// split-K second pass: the partials summed in split order, then the epilogue
__global__ __launch_bounds__(256) void enc_splitk_kernel(EncConvParams p) {
    const int N = p.OH * p.OW, OQ = p.OC / 4;
    const int64_t total = (int64_t) N * OQ;
    for (int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t) gridDim.x * 256) {
        const int n = (int) (i / OQ), o = (int) (i - (int64_t) n * OQ) * 4;
        floatx4 a = *(const floatx4 *) (p.ws + (int64_t) n * p.OC + o);
        for (int s = 1; s < p.ksplit; s++) {
            const floatx4 b = *(const floatx4 *) (p.ws + ((int64_t) s * N + n) * p.OC + o);
#pragma unroll
            for (int j = 0; j < 4; j++) a[j] = a[j] + b[j];
        }
        const float q[4] = {a[0], a[1], a[2], a[3]};
        enc_epilogue(p, n, o, q);
    }
}

// one wave per output: y[o] = sum_i W[o][i] x[i] (+ b[o]); x rounded to f16
// first when W is an f16 tensor (ggml's vec_dot / GEMM operand conversion)
__global__ __launch_bounds__(256) void enc_linear_kernel(const float *__restrict__ W, const float *__restrict__ b,
                                                         const float *__restrict__ x, int O, int I, int round16,
                                                         float *__restrict__ y) {
    const int lane = threadIdx.x & 63;
    const int o = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (o >= O) return;  // whole wave
    const float *w = W + (int64_t) o * I;
    float acc = 0.0f;
    for (int i = lane; i < I; i += 64) {
        const float xv = round16 ? (float) (half_t) x[i] : x[i];
        acc = __builtin_fmaf(w[i], xv, acc);
    }
    acc = group_sum<64>(acc);
    if (lane == 0) y[o] = b ? acc + b[o] : acc;
}

static unsigned grid_1d(int64_t total) {
    int64_t nb = (total + 255) / 256;
    if (nb > 65536) nb = 65536;
    return (unsigned) (nb < 1 ? 1 : nb);
}

hipError_t launch_enc_stem(const float *img, const float *w, const float *b, int64_t HW, int C0, float *y,
                           void *ya, bool ya_f16, hipStream_t st) {
    if (ya_f16)
        hipLaunchKernelGGL(enc_stem_kernel<half_t>, dim3(grid_1d(HW * C0)), dim3(256), 0, st, img, w, b, HW, C0, y,
                           (half_t *) ya);
    else
        hipLaunchKernelGGL(enc_stem_kernel<float>, dim3(grid_1d(HW * C0)), dim3(256), 0, st, img, w, b, HW, C0, y,
                           (float *) ya);
    return hipGetLastError();
}

hipError_t launch_enc_blur(const float *x, const float *k, int H, int W, int C, int pad, void *y, bool y_f16,
                           hipStream_t st) {
    const int OH = H + 2 * pad - 3, OW = W + 2 * pad - 3;
    if (OH < 1 || OW < 1 || C % 4 != 0 || (int64_t) H * W * C >= (int64_t) 1 << 31) return hipErrorInvalidValue;
    const unsigned g = grid_1d((int64_t) OH * OW * (C / 4));
    if (y_f16)
        hipLaunchKernelGGL(enc_blur_kernel<half_t>, dim3(g), dim3(256), 0, st, x, k, H, W, C, pad, OH, OW,
                           (half_t *) y);
    else
        hipLaunchKernelGGL(enc_blur_kernel<float>, dim3(g), dim3(256), 0, st, x, k, H, W, C, pad, OH, OW,
                           (float *) y);
    return hipGetLastError();
}

hipError_t launch_enc_conv(EncConvParams p, bool f16, hipStream_t st) {
    if (p.IC % 32 != 0 || p.OC % 4 != 0 || p.OH < 1 || p.OW < 1) return hipErrorInvalidValue;
    const int T = p.KH * p.KW * p.IC / 32;
    if (p.ksplit < 1) p.ksplit = 1;
    if (p.ksplit > T || (p.ksplit > 1 && !p.ws)) return hipErrorInvalidValue;
    dim3 grid((unsigned) ((p.OH * p.OW + 63) / 64), (unsigned) ((p.OC + 63) / 64), (unsigned) p.ksplit);
    if (f16) hipLaunchKernelGGL(enc_conv_kernel<half_t>, grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL(enc_conv_kernel<float>, grid, dim3(256), 0, st, p);
    if (p.ksplit > 1) {
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(enc_splitk_kernel, dim3(grid_1d((int64_t) p.OH * p.OW * (p.OC / 4))), dim3(256), 0, st,
                           p);
    }
    return hipGetLastError();
}

hipError_t launch_enc_epilogue(EncConvParams p, hipStream_t st) {
    if (p.OC % 4 != 0 || p.OH < 1 || p.OW < 1 || !p.ws) return hipErrorInvalidValue;
    p.ksplit = 1;
    hipLaunchKernelGGL(enc_splitk_kernel, dim3(grid_1d((int64_t) p.OH * p.OW * (p.OC / 4))), dim3(256), 0, st, p);
    return hipGetLastError();
}

hipError_t launch_enc_linear(const float *W, const float *b, const float *x, int O, int I, bool round16, float *y,
                             hipStream_t st) {
    hipLaunchKernelGGL(enc_linear_kernel, dim3((unsigned) ((O + 3) / 4)), dim3(256), 0, st, W, b, x, O, I,
                       round16 ? 1 : 0, y);
    return hipGetLastError();
}

}  // namespace tpmd
