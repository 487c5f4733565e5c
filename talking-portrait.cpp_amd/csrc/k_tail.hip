// Fused per-stage tail of the motion decoder: everything that follows the
// dense modulated conv of stage j, for every pixel of every frame, in ONE
// pass over the stage output (src/motion_dec.cpp:1077-1108 channel-last
// stages; :1012-1064 spatial stages — same arithmetic):
//
//   fl   = (Wf * s_f) . out + b_f  [+ upfirdn2x(fl_prev)]        ToFlow + skip
//   gx   = tanh(fl0) + lin[x],  gy = tanh(fl1) + lin[y],  m = sigmoid(fl2)
//   smp  = grid_sample(feat_j, gx, gy)   bilinear, zeros, align_corners=False
//   warp = smp * m ;  trunk = warp + out * (1 - m)
//   rgb  = leaky(Wr . warp + b1) + b_rgb  [+ upfirdn2x(rgb_prev)]  ToRGB + skip
//
// Layout: G lanes own one pixel and 8 channels each (C = 8*G); the two 3-row
// dot products (ToFlow, ToRGB) finish with a butterfly over the G lanes, so
// every lane holds the pixel's flow/mask and can run its slice of the gather.
// The feature map is channel-last, so the 4 taps of a pixel are 4 contiguous
// channel runs read by the G lanes together.  trunk is written pre-multiplied
// by the next up-conv's style (that conv's B operand); the last stage writes
// only rgb, straight into the CHW output frame.
#include "tpmd_device.h"
#include "tpmd_launch.h"

namespace tpmd {

template <typename T> struct load8;
template <> struct load8<float> {
    __device__ __forceinline__ static void run(const float *p, float v[8]) {
        const floatx4 a = *(const floatx4 *) p, b = *(const floatx4 *) (p + 4);
        v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
        v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
    }
};
template <> struct load8<half_t> {
    __device__ __forceinline__ static void run(const half_t *p, float v[8]) {
        const half8 a = *(const half8 *) p;
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = (float) a[e];
    }
};
template <typename T> __device__ __forceinline__ void store8(T *p, const float v[8]);
template <> __device__ __forceinline__ void store8<float>(float *p, const float v[8]) {
    *(floatx4 *) p = floatx4{v[0], v[1], v[2], v[3]};
    *(floatx4 *) (p + 4) = floatx4{v[4], v[5], v[6], v[7]};
}
template <> __device__ __forceinline__ void store8<half_t>(half_t *p, const float v[8]) {
    half8 h;
#pragma unroll
    for (int e = 0; e < 8; e++) h[e] = (half_t) v[e];
    *(half8 *) p = h;
}

template <typename TF, typename TOUT, typename TT, int G>
__global__ __launch_bounds__(256) void stage_tail_kernel(TailArgs a) {
    // one rounding per operation everywhere; the two dot products use explicit fma
#pragma clang fp contract(off)
    constexpr int PPW = 64 / G;  // pixels per wave
    const int lane = threadIdx.x & 63;
    const int gl = lane % G, grp = lane / G;
    const int c0 = gl * 8;
    const int r = a.r, C = a.C, rh = r >> 1;
    const int64_t RR = (int64_t) r * r;
    const int64_t P = (int64_t) a.nframes * RR;
    const int64_t wave = (int64_t) blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t nwaves = (int64_t) gridDim.x * (blockDim.x >> 6);

    // per-lane constant weight slices
    float wf[3][8], wr[3][8];
#pragma unroll
    for (int k = 0; k < 3; k++) {
        load8<float>::run(a.wflow + k * C + c0, wf[k]);
        load8<float>::run(a.wrgb + k * C + c0, wr[k]);
    }

    for (int64_t base = wave * PPW; base < P; base += nwaves * PPW) {
        const int64_t p = base + grp;
        const bool valid = p < P;
        const int64_t pp = valid ? p : P - 1;
        const int fr = (int) (pp / RR);
        const int pix = (int) (pp - (int64_t) fr * RR);
        const int y = pix / r, x = pix - y * r;

        float ov[8];
        load8<TOUT>::run((const TOUT *) a.out + pp * C + c0, ov);

        // ---- ToFlow: (Wf * s_f) . out, folded weight rounded like gemm_weight
        float sf[8];
        load8<float>::run(a.sflow + (int64_t) fr * C + c0, sf);
        float fl[3];
#pragma unroll
        for (int k = 0; k < 3; k++) {
            float acc = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float w = wf[k][e] * sf[e];
                acc = __builtin_fmaf(w, ov[e], acc);
            }
            fl[k] = group_sum<G>(acc);
        }
        {
#pragma unroll
            for (int k = 0; k < 3; k++) {
                fl[k] = fl[k] + a.fbias[k];
                if (a.flow_prev)
                    fl[k] = fl[k] + upfirdn2x_at(a.flow_prev + ((int64_t) fr * 3 + k) * rh * rh, rh, rh,
                                                 a.fup, x, y);
            }
        }
        if (a.flow_cur && valid && gl < 3) {
            const float v = gl == 0 ? fl[0] : (gl == 1 ? fl[1] : fl[2]);
            a.flow_cur[((int64_t) fr * 3 + gl) * RR + pix] = v;
        }

        // ---- flow head + gather
        float gx, gy, m;
        {
            gx = tanhf(fl[0]) + a.lin[x];
            gy = tanhf(fl[1]) + a.lin[y];
            m = 1.0f / (1.0f + expf(-fl[2]));
        }
        const taps4 t = gather_geometry(gx, gy, r, r);
        float smp[8];
#pragma unroll
        for (int e = 0; e < 8; e++) smp[e] = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int cx = t.x0 + (k & 1), cy = t.y0 + (k >> 1);
            if (cx < 0 || cx >= r || cy < 0 || cy >= r) continue;
            const float w = tap_weight(t, k);
            float fv[8];
            load8<TF>::run((const TF *) a.feat + (int64_t) (cy * r + cx) * C + c0, fv);
#pragma unroll
            for (int e = 0; e < 8; e++) smp[e] += w * fv[e];
        }

        // ---- warp / trunk
        float warp[8], trunk[8];
        {
            const float one_m = 1.0f - m;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                warp[e] = smp[e] * m;
                trunk[e] = warp[e] + ov[e] * one_m;
            }
        }
        if (valid && a.warp_tap) store8<float>(a.warp_tap + pp * C + c0, warp);
        if (valid && a.trunk) {
            if (a.s_next) {
                float sn[8];
                load8<float>::run(a.s_next + (int64_t) fr * C + c0, sn);
#pragma unroll
                for (int e = 0; e < 8; e++) trunk[e] = trunk[e] * sn[e];
            }
            store8<TT>((TT *) a.trunk + pp * C + c0, trunk);
        }

        // ---- ToRGB
        float rgb[3];
#pragma unroll
        for (int k = 0; k < 3; k++) {
            float acc = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) acc = __builtin_fmaf(wr[k][e], warp[e], acc);
            rgb[k] = group_sum<G>(acc);
        }
        if (valid && gl < 3) {
            const int k = gl;
            const float rv = k == 0 ? rgb[0] : (k == 1 ? rgb[1] : rgb[2]);
            float v = leaky(rv + a.rlb[k]);
            v = v + a.rbias[k];
            if (a.rgb_prev)
                v = v + upfirdn2x_at(a.rgb_prev + ((int64_t) fr * 3 + k) * rh * rh, rh, rh, a.rup, x, y);
            a.rgb_cur[((int64_t) fr * 3 + k) * RR + pix] = v;
        }
    }
}

template <typename TF, typename TOUT, typename TT>
static hipError_t launch_tail_typed(const TailArgs &a, hipStream_t st) {
    const int G = a.C / 8;
    const int64_t P = (int64_t) a.nframes * a.r * a.r;
    const int ppb = 4 * (64 / G);
    int64_t nb = (P + ppb - 1) / ppb;
    if (nb > 16384) nb = 16384;
    if (nb < 1) nb = 1;
#define TPMD_T(g)                                                                                \
    case g:                                                                                      \
        hipLaunchKernelGGL((stage_tail_kernel<TF, TOUT, TT, g>), dim3((unsigned) nb), dim3(256), 0, \
                           st, a);                                                               \
        break;
    switch (G) {
        TPMD_T(4) TPMD_T(8) TPMD_T(16) TPMD_T(32) TPMD_T(64)
        default: return hipErrorInvalidValue;
    }
#undef TPMD_T
    return hipGetLastError();
}

hipError_t launch_stage_tail(const TailArgs &a, bool feat_f16, bool out_f16, bool trunk_f16,
                             hipStream_t st) {
    if (a.nframes <= 0) return hipSuccess;
    if (feat_f16) {
        if (out_f16) {
            if (trunk_f16) return launch_tail_typed<half_t, half_t, half_t>(a, st);
            return launch_tail_typed<half_t, half_t, float>(a, st);
        }
        if (trunk_f16) return launch_tail_typed<half_t, float, half_t>(a, st);
        return launch_tail_typed<half_t, float, float>(a, st);
    }
    if (out_f16) return hipErrorInvalidValue;
    if (trunk_f16) return hipErrorInvalidValue;
    return launch_tail_typed<float, float, float>(a, st);
}

}  // namespace tpmd
