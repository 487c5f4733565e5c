// Flow-matching transformer kernel launchers (k_fmt.hip), internal.  The
// linear layers run on the MFMA GEMM of k_enc.hip (launch_enc_conv, 1x1).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tpmd_enc.h"

namespace tpmd {

hipError_t launch_fmt_convert(const float *x, int rows, int cols, int ld, void *y, bool f16, hipStream_t st);
hipError_t launch_fmt_tfreq(const float *fk, float t, int half, float *y, hipStream_t st);
hipError_t launch_fmt_silu(float *x, int n, hipStream_t st);
hipError_t launch_fmt_cond(const float *clin, const float *temb, int rows, int H, void *y, bool f16, hipStream_t st);
hipError_t launch_fmt_xpos(const float *x1, const float *pos, int T, int H, int B, float *x, hipStream_t st);
hipError_t launch_fmt_ln_mod(const float *x, const float *mod, int64_t mstride, int shift_off, int scale_off,
                             int rows, int H, float eps, void *y, bool f16, hipStream_t st);
// x += gate * (prod + bias) per row (the gated residual update of a linear
// whose f32 product is prod, [rows][H]; bias may be null), then the norm and
// modulation of launch_fmt_ln_mod on the new x, in one launch
hipError_t launch_fmt_res_ln_mod(const float *prod, const float *bias, const float *gate, int64_t gstride, float *x,
                                 const float *mod, int64_t mstride, int shift_off, int scale_off, int rows, int H,
                                 float eps, void *y, bool f16, hipStream_t st);
hipError_t launch_fmt_attn(const float *qkv, int B, int T, int H, int nh, int w, void *o, bool f16, hipStream_t st);
hipError_t launch_fmt_euler(const float *v, float *x60, int T, int P, int D, float a_cfg, float e_cfg, float dt,
                            hipStream_t st);

}  // namespace tpmd
