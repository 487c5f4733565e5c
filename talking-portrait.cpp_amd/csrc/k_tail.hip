// Standalone stage-tail kernel (the per-pixel body is tail_pixel in
// tpmd_tail.h): one pass over a dense-conv output `out` held in HBM.  The
// decoder uses it for the wide stages (C >= 256), where one conv tile does
// not hold all channels of a pixel; narrower stages run the same body inside
// the dense conv's epilogue (k_conv.hip).
#include "tpmd_tail.h"

namespace tpmd {

template <typename TF, typename TOUT, typename TT, int G, bool FGR>
__global__ __launch_bounds__(256) void stage_tail_kernel(TailArgs a) {
    constexpr int PPW = 64 / G;  // pixels per wave
    const int lane = threadIdx.x & 63;
    const int gl = lane % G, grp = lane / G;
    const int64_t P = (int64_t) a.nframes * a.r * a.r;
    const int64_t wave = (int64_t) blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t nwaves = (int64_t) gridDim.x * (blockDim.x >> 6);
    TailWeights w;
    load_tail_weights<FGR>(a, gl * 8, w);
    for (int64_t base = wave * PPW; base < P; base += nwaves * PPW) {
        const int64_t p = base + grp;
        const bool valid = p < P;
        const int64_t pp = valid ? p : P - 1;
        float ov[8];
        load8<TOUT>::run((const TOUT *) a.out + pp * a.C + gl * 8, ov);
        tail_pixel<TF, TT, G, FGR>(a, pp, valid, gl, ov, w);
    }
}

template <typename TF, typename TOUT, typename TT>
static hipError_t launch_tail_typed(const TailArgs &a, hipStream_t st) {
    const int G = a.C / 8;
    const int64_t P = (int64_t) a.nframes * a.r * a.r;
    const int ppb = 4 * (64 / G);
    int64_t nb = (P + ppb - 1) / ppb;
    if (nb > 65536) nb = 65536;
    if (nb < 1) nb = 1;
#define TPMD_T(g)                                                                                       \
    case g:                                                                                             \
        if (a.featg)                                                                                    \
            hipLaunchKernelGGL((stage_tail_kernel<TF, TOUT, TT, g, true>), dim3((unsigned) nb), dim3(256), 0, \
                               st, a);                                                                  \
        else                                                                                            \
            hipLaunchKernelGGL((stage_tail_kernel<TF, TOUT, TT, g, false>), dim3((unsigned) nb), dim3(256), 0, \
                               st, a);                                                                  \
        break;
    switch (G) {
        TPMD_T(4) TPMD_T(8) TPMD_T(16) TPMD_T(32) TPMD_T(64)
        default: return hipErrorInvalidValue;
    }
#undef TPMD_T
    return hipGetLastError();
}

// ToRGB weight . feature, per feature pixel: the last stage's ToRGB sum as a
// bilinear sample of 3 values instead of C (tile_tail, tpmd_tail.h)
template <typename TF>
__global__ __launch_bounds__(256) void feat_rgb_kernel(const TF *__restrict__ feat, const float *__restrict__ wrgb,
                                                       int C, int64_t npix, float *__restrict__ g) {
    for (int64_t p = (int64_t) blockIdx.x * 256 + threadIdx.x; p < npix; p += (int64_t) gridDim.x * 256) {
        float acc[3] = {0.0f, 0.0f, 0.0f};
        for (int c = 0; c < C; c++) {
            const float f = (float) feat[p * C + c];
#pragma unroll
            for (int k = 0; k < 3; k++) acc[k] = __builtin_fmaf(wrgb[k * C + c], f, acc[k]);
        }
        *(floatx4 *) (g + p * 4) = floatx4{acc[0], acc[1], acc[2], 0.0f};
    }
}

hipError_t launch_feat_rgb(bool feat_f16, const void *feat, const float *wrgb, int C, int64_t npix, float *g,
                           hipStream_t st) {
    if (npix <= 0) return hipSuccess;
    const int64_t nb = (npix + 255) / 256 > 8192 ? 8192 : (npix + 255) / 256;
    if (feat_f16)
        hipLaunchKernelGGL(feat_rgb_kernel<half_t>, dim3((unsigned) nb), dim3(256), 0, st, (const half_t *) feat,
                           wrgb, C, npix, g);
    else
        hipLaunchKernelGGL(feat_rgb_kernel<float>, dim3((unsigned) nb), dim3(256), 0, st, (const float *) feat,
                           wrgb, C, npix, g);
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
