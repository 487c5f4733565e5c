// Per-pixel stage tail of the motion decoder, shared by the standalone tail
// kernel (k_tail.hip) and the dense conv's fused epilogue (k_conv.hip).
//
// Everything that follows the dense modulated conv of stage j, for one pixel
// (src/motion_dec.cpp:1077-1108 channel-last stages; :1012-1064 spatial
// stages, same arithmetic):
//
//   fl   = (Wf * s_f) . out + b_f  [+ upfirdn2x(fl_prev)]        ToFlow + skip
//   gx   = tanh(fl0) + lin[x],  gy = tanh(fl1) + lin[y],  m = sigmoid(fl2)
//   smp  = grid_sample(feat_j, gx, gy)   bilinear, zeros, align_corners=False
//   warp = smp * m ;  trunk = warp + out * (1 - m)
//   rgb  = leaky(Wr . warp + b1) + b_rgb  [+ upfirdn2x(rgb_prev)]  ToRGB + skip
//
// G lanes own one pixel, 8 channels each (C = 8*G); the two 3-row dot
// products finish with a butterfly over the G lanes, so every lane holds the
// pixel's flow and mask and gathers its own 8 channels of the 4 taps (the
// feature map is channel-last: each tap is one contiguous run read by the G
// lanes together).  trunk is stored pre-multiplied by the next up-conv's
// style (that conv's operand); the last stage writes only rgb, straight into
// the CHW output frame.
#pragma once

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

// per-lane slices of the ToFlow / ToRGB weights (channels c0 .. c0+7)
struct TailWeights {
    float wf[3][8], wr[3][8];
};

__device__ __forceinline__ void load_tail_weights(const TailArgs &a, int c0, TailWeights &w) {
#pragma unroll
    for (int k = 0; k < 3; k++) {
        load8<float>::run(a.wflow + k * a.C + c0, w.wf[k]);
        load8<float>::run(a.wrgb + k * a.C + c0, w.wr[k]);
    }
}

// One pixel pp = frame * r*r + y*r + x of the batch; `valid` false for the
// padding lanes of the last group (they take part in the butterflies and
// store nothing).  ov: this lane's 8 dense-conv output channels (f32).
template <typename TF, typename TT, int G>
__device__ __forceinline__ void tail_pixel(const TailArgs &a, int64_t pp, bool valid, int gl,
                                           const float ov[8], const TailWeights &w) {
    // one rounding per operation everywhere; the two dot products use explicit fma
#pragma clang fp contract(off)
    const int c0 = gl * 8;
    const int r = a.r, C = a.C, rh = r >> 1;
    const int64_t RR = (int64_t) r * r;
    const int fr = (int) (pp / RR);
    const int pix = (int) (pp - (int64_t) fr * RR);
    const int y = pix / r, x = pix - y * r;

    // ---- ToFlow: (Wf * s_f) . out, folded weight rounded like gemm_weight
    float sf[8];
    load8<float>::run(a.sflow + (int64_t) fr * C + c0, sf);
    float fl[3];
#pragma unroll
    for (int k = 0; k < 3; k++) {
        float acc = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float wv = w.wf[k][e] * sf[e];
            acc = __builtin_fmaf(wv, ov[e], acc);
        }
        fl[k] = group_sum<G>(acc);
    }
#pragma unroll
    for (int k = 0; k < 3; k++) {
        fl[k] = fl[k] + a.fbias[k];
        if (a.flow_prev)
            fl[k] = fl[k] + upfirdn2x_at(a.flow_prev + ((int64_t) fr * 3 + k) * rh * rh, rh, rh, a.fup, x, y);
    }
    if (a.flow_cur && valid && gl < 3) {
        const float v = gl == 0 ? fl[0] : (gl == 1 ? fl[1] : fl[2]);
        a.flow_cur[((int64_t) fr * 3 + gl) * RR + pix] = v;
    }

    // ---- flow head + gather
    const float gx = tanhf(fl[0]) + a.lin[x];
    const float gy = tanhf(fl[1]) + a.lin[y];
    const float m = 1.0f / (1.0f + expf(-fl[2]));
    const taps4 t = gather_geometry(gx, gy, r, r);
    float fv[4][8];
    bool in[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {  // issue the four tap loads together
        const int cx = t.x0 + (k & 1), cy = t.y0 + (k >> 1);
        in[k] = cx >= 0 && cx < r && cy >= 0 && cy < r;
        if (in[k]) load8<TF>::run((const TF *) a.feat + (int64_t) (cy * r + cx) * C + c0, fv[k]);
    }
    float smp[8];
#pragma unroll
    for (int e = 0; e < 8; e++) smp[e] = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        if (!in[k]) continue;
        const float wk = tap_weight(t, k);
#pragma unroll
        for (int e = 0; e < 8; e++) smp[e] += wk * fv[k][e];
    }

    // ---- warp / trunk
    float warp[8], trunk[8];
    const float one_m = 1.0f - m;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        warp[e] = smp[e] * m;
        trunk[e] = warp[e] + ov[e] * one_m;
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
        for (int e = 0; e < 8; e++) acc = __builtin_fmaf(w.wr[k][e], warp[e], acc);
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

}  // namespace tpmd
