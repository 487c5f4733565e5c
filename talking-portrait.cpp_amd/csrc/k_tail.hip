// Standalone stage-tail kernel (the per-pixel body is tail_pixel in
// tpmd_tail.h): one pass over a dense-conv output `out` held in HBM.  The
// decoder uses it for the wide stages (C >= 256), where one conv tile does
// not hold all channels of a pixel; narrower stages run the same body inside
// the dense conv's epilogue (k_conv.hip).
#include "tpmd_tail.h"

namespace tpmd {

template <typename TF, typename TOUT, typename TT, int G>
__global__ __launch_bounds__(256) void stage_tail_kernel(TailArgs a) {
    constexpr int PPW = 64 / G;  // pixels per wave
    const int lane = threadIdx.x & 63;
    const int gl = lane % G, grp = lane / G;
    const int64_t P = (int64_t) a.nframes * a.r * a.r;
    const int64_t wave = (int64_t) blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t nwaves = (int64_t) gridDim.x * (blockDim.x >> 6);
    TailWeights w;
    load_tail_weights(a, gl * 8, w);
    for (int64_t base = wave * PPW; base < P; base += nwaves * PPW) {
        const int64_t p = base + grp;
        const bool valid = p < P;
        const int64_t pp = valid ? p : P - 1;
        float ov[8];
        load8<TOUT>::run((const TOUT *) a.out + pp * a.C + gl * 8, ov);
        tail_pixel<TF, TT, G>(a, pp, valid, gl, ov, w);
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
