// Flow-matching transformer pieces (src/fmt.cpp:44-205, src/pipeline.cpp:38-91)
// around the MFMA GEMM of k_enc.hip (a linear layer is its 1x1 conv over a
// row of tokens):
//
//   fmt_convert_kernel   f32 rows -> GEMM operand type, zero-padding K
//   fmt_tfreq_kernel     the GLIDE timestep features
//   fmt_silu_kernel      in place, the t-embedder's hidden layer
//   fmt_cond_kernel      silu(c_embed + t_embed) in the adaLN GEMMs' operand type
//   fmt_xpos_kernel      x = x_embed + pos, replicated over the CFG branches
//   fmt_ln_mod_kernel    LayerNorm (no affine) then adaLN modulate: n*scale + n + shift,
//                        optionally after the gated residual update of the linear before it
//   fmt_attn_kernel      banded multi-head attention (softmax(q k / sqrt(hd) + mask) v)
//   fmt_euler_kernel     CFG combination of the three branches and the Euler step
#include "tpmd_conv.h"
#include "tpmd_fmt.h"

namespace tpmd {

template <typename T> __device__ __forceinline__ T fmt_cast(float v);
template <> __device__ __forceinline__ float fmt_cast<float>(float v) { return v; }
template <> __device__ __forceinline__ half_t fmt_cast<half_t>(float v) { return (half_t) v; }

__device__ __forceinline__ float fmt_silu(float x) { return x / (1.0f + expf(-x)); }

template <typename TO>
__global__ __launch_bounds__(256) void fmt_convert_kernel(const float *__restrict__ x, int rows, int cols, int ld,
                                                          TO *__restrict__ y) {
    const int64_t total = (int64_t) rows * ld;
    for (int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t) gridDim.x * 256) {
        const int64_t r = i / ld;
        const int c = (int) (i - r * ld);
        y[i] = fmt_cast<TO>(c < cols ? x[r * cols + c] : 0.0f);
    }
}

// [cos(t f_k), sin(t f_k)], k < half (the product rounded to f32 first, as the reference)
__global__ __launch_bounds__(256) void fmt_tfreq_kernel(const float *__restrict__ fk, float t, int half,
                                                        float *__restrict__ y) {
    const int k = blockIdx.x * 256 + threadIdx.x;
    if (k < half) {
        const float a = t * fk[k];
        y[k] = cosf(a);
        y[half + k] = sinf(a);
    }
}

__global__ __launch_bounds__(256) void fmt_silu_kernel(float *__restrict__ x, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] = fmt_silu(x[i]);
}

template <typename TO>
__global__ __launch_bounds__(256) void fmt_cond_kernel(const float *__restrict__ clin, const float *__restrict__ temb,
                                                       int rows, int H, TO *__restrict__ y) {
    const int64_t total = (int64_t) rows * H;
    for (int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t) gridDim.x * 256) {
        const int c = (int) (i % H);
        y[i] = fmt_cast<TO>(fmt_silu(clin[i] + temb[c]));
    }
}

__global__ __launch_bounds__(256) void fmt_xpos_kernel(const float *__restrict__ x1, const float *__restrict__ pos,
                                                       int T, int H, int B, float *__restrict__ x) {
    const int64_t per = (int64_t) T * H, total = per * B;
    for (int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t) gridDim.x * 256) {
        const int64_t j = i % per;
        x[i] = x1[j] + pos[j];
    }
}

// one workgroup per row of H: mean, then the variance of the centred values
// (two passes over registers), n = (x - mean) / sqrt(var + eps),
// h = n * scale + n + shift
// RES: first the residual update of the linear before it, whose f32
// product P (no bias) is given: x += gate * (P + b), stored back to x, as
// the linear's own epilogue pass computes it; then the norm of the new x
template <typename TO, bool RES>
// (x and xout alias: RES updates x in place, each element read and then
// written by one thread)
__global__ __launch_bounds__(256) void fmt_ln_mod_kernel(const float *x, const float *__restrict__ mod,
                                                         int64_t mstride, int shift_off, int scale_off, int H,
                                                         float eps, TO *__restrict__ y, const float *__restrict__ prod,
                                                         const float *__restrict__ bias, const float *__restrict__ gate,
                                                         int64_t gstride, float *xout) {
    constexpr int MAXV = 16;  // H <= 4096
    __shared__ float red[4];
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const float *xr = x + (int64_t) row * H;
    float v[MAXV];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < MAXV; k++) {
        const int i = tid + k * 256;
        v[k] = i < H ? xr[i] : 0.0f;
        if constexpr (RES) {
            if (i < H) {
                float a = prod[(int64_t) row * H + i];
                if (bias) a = a + bias[i];
                a = gate[(int64_t) row * gstride + i] * a;
                v[k] = v[k] + a;
                xout[(int64_t) row * H + i] = v[k];
            }
        }
        s += v[k];
    }
    auto block_sum = [&](float a) {
        a = group_sum<64>(a);
        __syncthreads();
        if (lane == 0) red[wid] = a;
        __syncthreads();
        return red[0] + red[1] + red[2] + red[3];
    };
    const float mean = block_sum(s) / (float) H;
    float s2 = 0.0f;
#pragma unroll
    for (int k = 0; k < MAXV; k++) {
        const int i = tid + k * 256;
        if (i < H) {
            v[k] = v[k] - mean;
            s2 += v[k] * v[k];
        }
    }
    const float var = block_sum(s2) / (float) H;
    const float inv = 1.0f / sqrtf(var + eps);
    const float *mr = mod + (int64_t) row * mstride;
    TO *yr = y + (int64_t) row * H;
#pragma unroll
    for (int k = 0; k < MAXV; k++) {
        const int i = tid + k * 256;
        if (i < H) {
            const float n = v[k] * inv;
            yr[i] = fmt_cast<TO>((n * mr[scale_off + i] + n) + mr[shift_off + i]);
        }
    }
}

// one wave per (branch, head, query): the keys |tq - tk| <= w only (the
// band mask's -inf elsewhere contributes exp(-inf) = 0), lanes over the
// head dimension
template <typename TO>
__global__ __launch_bounds__(256) void fmt_attn_kernel(const float *__restrict__ qkv, int B, int T, int H, int nh,
                                                       int w, float scale, TO *__restrict__ o) {
    constexpr int MAXK = 15, MAXD = 4;  // 2w + 1 keys, head dim <= 256
    const int lane = threadIdx.x & 63;
    const int g = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (g >= B * nh * T) return;  // whole wave
    const int tq = g % T, hh = (g / T) % nh, b = g / (T * nh);
    const int hd = H / nh;
    const int64_t rs = 3 * (int64_t) H;
    const float *qr = qkv + ((int64_t) b * T + tq) * rs + hh * hd;
    float q[MAXD];
#pragma unroll
    for (int k = 0; k < MAXD; k++) q[k] = lane + 64 * k < hd ? qr[lane + 64 * k] : 0.0f;
    const int k0 = tq - w > 0 ? tq - w : 0, k1 = tq + w < T - 1 ? tq + w : T - 1;
    // every key and value row of the band is requested before any is used,
    // and the 2w+1 dot products are reduced together (independent chains)
    float kv[MAXK][MAXD], vv[MAXK][MAXD];
#pragma unroll
    for (int j = 0; j < MAXK; j++) {
        const int tk = k0 + j <= k1 ? k0 + j : k1;
        const float *kr = qkv + ((int64_t) b * T + tk) * rs + H + hh * hd;
        const float *vr = kr + H;
#pragma unroll
        for (int k = 0; k < MAXD; k++) {
            kv[j][k] = lane + 64 * k < hd ? kr[lane + 64 * k] : 0.0f;
            vv[j][k] = lane + 64 * k < hd ? vr[lane + 64 * k] : 0.0f;
        }
    }
    float sc[MAXK];
#pragma unroll
    for (int j = 0; j < MAXK; j++) {
        float a = 0.0f;
#pragma unroll
        for (int k = 0; k < MAXD; k++) a = __builtin_fmaf(q[k], kv[j][k], a);
        sc[j] = a;
    }
#pragma unroll
    for (int j = 0; j < MAXK; j++) sc[j] = group_sum<64>(sc[j]) * scale;
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < MAXK; j++)
        if (k0 + j <= k1) mx = sc[j] > mx ? sc[j] : mx;
    float den = 0.0f;
#pragma unroll
    for (int j = 0; j < MAXK; j++) {
        sc[j] = k0 + j <= k1 ? expf(sc[j] - mx) : 0.0f;
        den += sc[j];
    }
    float acc[MAXD] = {};
#pragma unroll
    for (int j = 0; j < MAXK; j++) {
        if (k0 + j <= k1) {
#pragma unroll
            for (int k = 0; k < MAXD; k++) acc[k] = __builtin_fmaf(sc[j], vv[j][k], acc[k]);
        }
    }
    TO *orow = o + ((int64_t) b * T + tq) * H + hh * hd;
#pragma unroll
    for (int k = 0; k < MAXD; k++)
        if (lane + 64 * k < hd) orow[lane + 64 * k] = fmt_cast<TO>(acc[k] / den);
}

// vc = (u + a_cfg (a - u)) + e_cfg (fu - a) for the chunk's rows, x += dt vc
__global__ __launch_bounds__(256) void fmt_euler_kernel(const float *__restrict__ v, float *__restrict__ x60, int T,
                                                        int P, int D, float a_cfg, float e_cfg, float dt) {
    const int64_t n = (int64_t) (T - P) * D;
    const int64_t per = (int64_t) T * D;
    for (int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t) gridDim.x * 256) {
        const int64_t j = (int64_t) P * D + i;
        const float u = v[j], fu = v[per + j], a = v[2 * per + j];
        const float vc = (u + a_cfg * (a - u)) + e_cfg * (fu - a);
        x60[j] = x60[j] + dt * vc;
    }
}

static unsigned fmt_grid(int64_t total) {
    int64_t nb = (total + 255) / 256;
    if (nb > 65536) nb = 65536;
    return (unsigned) (nb < 1 ? 1 : nb);
}

hipError_t launch_fmt_convert(const float *x, int rows, int cols, int ld, void *y, bool f16, hipStream_t st) {
    const unsigned g = fmt_grid((int64_t) rows * ld);
    if (f16) hipLaunchKernelGGL(fmt_convert_kernel<half_t>, dim3(g), dim3(256), 0, st, x, rows, cols, ld, (half_t *) y);
    else hipLaunchKernelGGL(fmt_convert_kernel<float>, dim3(g), dim3(256), 0, st, x, rows, cols, ld, (float *) y);
    return hipGetLastError();
}

hipError_t launch_fmt_tfreq(const float *fk, float t, int half, float *y, hipStream_t st) {
    hipLaunchKernelGGL(fmt_tfreq_kernel, dim3((unsigned) ((half + 255) / 256)), dim3(256), 0, st, fk, t, half, y);
    return hipGetLastError();
}

hipError_t launch_fmt_silu(float *x, int n, hipStream_t st) {
    hipLaunchKernelGGL(fmt_silu_kernel, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, st, x, n);
    return hipGetLastError();
}

hipError_t launch_fmt_cond(const float *clin, const float *temb, int rows, int H, void *y, bool f16, hipStream_t st) {
    const unsigned g = fmt_grid((int64_t) rows * H);
    if (f16) hipLaunchKernelGGL(fmt_cond_kernel<half_t>, dim3(g), dim3(256), 0, st, clin, temb, rows, H, (half_t *) y);
    else hipLaunchKernelGGL(fmt_cond_kernel<float>, dim3(g), dim3(256), 0, st, clin, temb, rows, H, (float *) y);
    return hipGetLastError();
}

hipError_t launch_fmt_xpos(const float *x1, const float *pos, int T, int H, int B, float *x, hipStream_t st) {
    hipLaunchKernelGGL(fmt_xpos_kernel, dim3(fmt_grid((int64_t) T * H * B)), dim3(256), 0, st, x1, pos, T, H, B, x);
    return hipGetLastError();
}

hipError_t launch_fmt_ln_mod(const float *x, const float *mod, int64_t mstride, int shift_off, int scale_off,
                             int rows, int H, float eps, void *y, bool f16, hipStream_t st) {
    if (H > 16 * 256) return hipErrorInvalidValue;
    if (f16)
        hipLaunchKernelGGL((fmt_ln_mod_kernel<half_t, false>), dim3((unsigned) rows), dim3(256), 0, st, x, mod,
                           mstride, shift_off, scale_off, H, eps, (half_t *) y, nullptr, nullptr, nullptr, 0, nullptr);
    else
        hipLaunchKernelGGL((fmt_ln_mod_kernel<float, false>), dim3((unsigned) rows), dim3(256), 0, st, x, mod,
                           mstride, shift_off, scale_off, H, eps, (float *) y, nullptr, nullptr, nullptr, 0, nullptr);
    return hipGetLastError();
}

hipError_t launch_fmt_res_ln_mod(const float *prod, const float *bias, const float *gate, int64_t gstride, float *x,
                                 const float *mod, int64_t mstride, int shift_off, int scale_off, int rows, int H,
                                 float eps, void *y, bool f16, hipStream_t st) {
    if (H > 16 * 256 || !prod || !gate || !x) return hipErrorInvalidValue;
    if (f16)
        hipLaunchKernelGGL((fmt_ln_mod_kernel<half_t, true>), dim3((unsigned) rows), dim3(256), 0, st, x, mod,
                           mstride, shift_off, scale_off, H, eps, (half_t *) y, prod, bias, gate, gstride, x);
    else
        hipLaunchKernelGGL((fmt_ln_mod_kernel<float, true>), dim3((unsigned) rows), dim3(256), 0, st, x, mod,
                           mstride, shift_off, scale_off, H, eps, (float *) y, prod, bias, gate, gstride, x);
    return hipGetLastError();
}

hipError_t launch_fmt_attn(const float *qkv, int B, int T, int H, int nh, int w, void *o, bool f16, hipStream_t st) {
    if (H % nh != 0 || H / nh > 256 || 2 * w + 1 > 15 || w < 0) return hipErrorInvalidValue;
    const float scale = 1.0f / sqrtf((float) (H / nh));
    const unsigned g = (unsigned) ((B * nh * T + 3) / 4);
    if (f16) hipLaunchKernelGGL(fmt_attn_kernel<half_t>, dim3(g), dim3(256), 0, st, qkv, B, T, H, nh, w, scale, (half_t *) o);
    else hipLaunchKernelGGL(fmt_attn_kernel<float>, dim3(g), dim3(256), 0, st, qkv, B, T, H, nh, w, scale, (float *) o);
    return hipGetLastError();
}

hipError_t launch_fmt_euler(const float *v, float *x60, int T, int P, int D, float a_cfg, float e_cfg, float dt,
                            hipStream_t st) {
    hipLaunchKernelGGL(fmt_euler_kernel, dim3(fmt_grid((int64_t) (T - P) * D)), dim3(256), 0, st, v, x60, T, P, D,
                       a_cfg, e_cfg, dt);
    return hipGetLastError();
}

}  // namespace tpmd
