// Motion-encoder kernel launchers (k_enc.hip), internal.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tpmd {

// y[n][o] = gate[n][o] * act(sum_k A[o][k] X(k, n) + bias[o]) + res[n][o] over channel-last
// maps: A [OC][KH][KW][IC] (tap-major k = (kh*KW + kw)*IC + ic), X [H][W][IC],
// y [OH][OW][OC] f32, OH = (H + 2 pad - KH) / stride + 1
struct EncConvParams {
    const void *A;          // operand type (f16 or f32)
    const void *X;          // operand type
    float *Y;               // f32 output, or null (Ya only)
    void *Ya;               // optional copy of Y in the next conv's operand type
    int ya_f16;             // Ya is f16 (else f32)
    const float *bias;      // [OC] or null
    const float *res;       // [OH][OW][OC] f32 added after the activation, or null
    int leaky;              // activation after the bias: 0 none, 1 leaky_relu 0.2, 2 tanh-GELU
    const float *gate;      // gate[n * gstride + o] multiplies the activation, or null
    int64_t gstride;
    int ksplit;             // > 1: k split over gridDim.z, partials in ws, epilogue in a second pass
    float *ws;              // [ksplit][OH*OW][OC] f32 (ksplit > 1)
    int H, W, IC, OC, KH, KW, stride, pad, OH, OW;
};

hipError_t launch_enc_stem(const float *img, const float *w, const float *b, int64_t HW, int C0, float *y,
                           void *ya, bool ya_f16, hipStream_t st);
hipError_t launch_enc_blur(const float *x, const float *k, int H, int W, int C, int pad, void *y, bool y_f16,
                           hipStream_t st);
hipError_t launch_enc_conv(EncConvParams p, bool f16, hipStream_t st);
// the conv's epilogue alone, on the f32 product [OH*OW][OC] already in p.ws
// (p.ksplit ignored): bias, activation, gate, residual, Y and Ya as above
hipError_t launch_enc_epilogue(EncConvParams p, hipStream_t st);
hipError_t launch_enc_linear(const float *W, const float *b, const float *x, int O, int I, bool round16, float *y,
                             hipStream_t st);

}  // namespace tpmd
