// Pieces shared by the two MFMA implicit-GEMM conv kernels (k_conv.hip,
// k_conv_halo.hip): operand types, the MFMA step, the launch parameters and
// the store epilogue (1/den, FusedLeakyReLU bias + leaky, next style).
#pragma once

#include <utility>

#include "tpmd_tail.h"

namespace tpmd {

// f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>): compile-time
// indices, so register arrays indexed inside never go to scratch
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

enum { MODE_DENSE = 0, MODE_SUBPIX = 1 };
enum { EPI_STORE = 0, EPI_PARTIAL = 1, EPI_TAIL = 2 };

template <typename TA>
struct mfma_op;

template <>
struct mfma_op<half_t> {
    __device__ __forceinline__ static void run(const u32x4 &a, const u32x4 &b, floatx16 &c) {
        c = __builtin_amdgcn_mfma_f32_32x32x16_f16(*(const half8 *) &a, *(const half8 *) &b, c, 0, 0,
                                                   0);
    }
};

template <>
struct mfma_op<float> {
    __device__ __forceinline__ static void run(const u32x4 &a, const u32x4 &b, floatx16 &c) {
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

struct ConvParams {
    const void *A;          // [M][9*IC]
    const void *X;          // CL input, frame stride x_bstride elements
    void *Y;                // CL output (EPI_STORE)
    const float *inv_den;   // [frame][OC]
    const float *bias;      // [OC]
    const float *out_scale; // [frame][OC] or null
    float *ws;              // [split][N][M] (EPI_PARTIAL)
    int N, H, W, IC, OC, M;
    int MT;                 // M tiles
    int T;                  // k tiles (9 * IC / BK)
    int64_t x_bstride;
    int a_img;              // A is stored as the k-tile DMA's LDS image (A_ORDER_RING_TAP)
};

// hardware hands workgroup ids to the 8 XCDs round robin; renumber so each
// XCD processes a contiguous range of `total` tiles
__device__ __forceinline__ int xcd_remap(int L, int total) {
    const int per = total >> 3, rem = total & 7;
    const int xcd = L & 7, slot = L >> 3;
    return xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
}

// Input halo of a TH x TW pixel block (top-left y0, x0) of one frame Xf
// (channel-last, IC f16 channels, CPP = IC / 8 16-byte chunks per pixel,
// HWD = TW + 2 halo pixels per row, HCH chunks in all) into registers: chunk
// tid + i*NT of the halo in hv[i].  The loads go through a buffer resource
// over the frame, so offsets are 32-bit and a pixel outside the map (or a
// chunk past the halo) reads at an offset past the extent, which the hardware
// answers with zeros: no branch and no 64-bit address per load.
template <int PF, int NT, int CPP, int HWD, int HCH, int IC>
__device__ __forceinline__ void halo_load(const half_t *Xf, int H, int W, int y0, int x0, int tid, u32x4 (&hv)[PF]) {
    const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(Xf, (int64_t) H * W * IC * 2);
    static_for<PF>([&](auto i) {
        const int ch = tid + i * NT;
        const int px = ch / CPP, c = ch - px * CPP;
        const int hy = px / HWD, hx = px - hy * HWD;
        const int iy = y0 - 1 + hy, ix = x0 - 1 + hx;
        const bool ok = ch < HCH && (unsigned) iy < (unsigned) H && (unsigned) ix < (unsigned) W;
        const unsigned off = ok ? (unsigned) ((iy * W + ix) * IC * 2 + c * 16) : 0x80000000u;
        hv[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0));
    });
}

// activation of 4 consecutive GEMM rows m..m+3 of column n, stored to Y
template <typename TO, int MODE>
__device__ __forceinline__ void epi_store_quad(const ConvParams &p, const float acc[4], int m, int n) {
    const int HW = p.H * p.W;
    const int fr = n / HW;
    int o;
    int64_t opix;
    if (MODE == MODE_DENSE) {
        o = m;
        opix = n;
    } else {
        const int rem = n - fr * HW;
        const int y = rem / p.W, x = rem - y * p.W;
        const int cls = m / p.OC;
        o = m - cls * p.OC;
        opix = (int64_t) fr * 4 * HW + (int64_t) (2 * y + (cls >> 1)) * (2 * p.W) + 2 * x + (cls & 1);
    }
    const floatx4 id = *(const floatx4 *) (p.inv_den + (int64_t) fr * p.OC + o);
    const floatx4 bb = *(const floatx4 *) (p.bias + o);
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = leaky(acc[j] * id[j] + bb[j]);
    if (p.out_scale) {
        const floatx4 sc = *(const floatx4 *) (p.out_scale + (int64_t) fr * p.OC + o);
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] *= sc[j];
    }
    store4<TO>((TO *) p.Y + opix * p.OC + o, v[0], v[1], v[2], v[3]);
}

// k_conv_halo.hip: the A-stationary halo-tile kernel for IC in {32, 64}
bool modconv_halo_ok(bool f16, int mode, int IC, int OC, int H, int W, bool tail);
hipError_t launch_modconv_halo(const ConvParams &p, int mode, bool out_f16, hipStream_t st);

// k_conv_async.hip: f16 store / split-K convs with LDS-DMA operand loads into
// a 4-stage ring; bm = 256 (256 x 256 tiles, 8 waves) or 128 (128 x 128,
// 4 waves); M % bm == 0, IC % 32 == 0
hipError_t launch_modconv_async(const ConvParams &p, int mode, int epi, int nsplit, bool out_f16, int bm,
                                hipStream_t st);
// k_conv_async.hip: f16 dense conv + fused stage tail for OC in {32, 64, 128,
// 256} (tiles of 256, 128, 128, 128 pixels of one frame) with the same ring
bool modconv_tail_async_ok(int OC, int r);
// k_conv_hfrag_tail.hip: f16 dense conv + fused stage tail for IC = OC = 128 or 256 on
// the halo conv (4 x 32 pixel blocks, A in A_ORDER_FRAG)
bool modconv_hfrag_tail_ok(bool f16, int IC, int OC, int H, int W);
hipError_t launch_modconv_hfrag_tail(const ConvParams &p, const TailArgs &ta, bool trunk_f16, hipStream_t st);
// 256- or 128-row tiles over 8 x 32 or 16 x 16 pixel blocks with the input
// halo in LDS and A read from L2 in fragment order (k_conv_hfrag.hip,
// A_ORDER_FRAG); f16 output, or f32 output of a dense conv
bool modconv_hfrag_ok(bool f16, bool out_f16, int mode, int IC, int OC, int H, int W);
hipError_t launch_modconv_hfrag(ConvParams p, int mode, bool out_f16, hipStream_t st);
// k_conv_up.hip: f16 composed sub-pixel up-conv 64 -> 32 channels with f16
// output, on 4 x 32 halo tiles (H % 4 == 0, W % 32 == 0)
bool modconv_up64_ok(bool f16, bool out_f16, int mode, int IC, int OC, int H, int W);
// frag: p.A in A_ORDER_FRAG order (else tap-major)
hipError_t launch_modconv_up64(const ConvParams &p, bool frag, hipStream_t st);
// k_conv_fused.hip: f16 dense conv + fused stage tail for IC = OC = 32 on
// halo tiles of 8 x 32 pixels (r % 32 == 0)
bool modconv_fused32_ok(bool f16, int IC, int OC, int r);
// frag: p.A in A_ORDER_FRAG order (else tap-major)
hipError_t launch_modconv_fused32(const ConvParams &p, const TailArgs &ta, bool trunk_f16, bool frag,
                                  hipStream_t st);
// ... and for IC = OC = 64 on 4 x 32 halo tiles, A streamed through LDS per tap
bool modconv_fused64_ok(bool f16, int IC, int OC, int r);
hipError_t launch_modconv_fused64(const ConvParams &p, const TailArgs &ta, bool trunk_f16, bool frag,
                                  hipStream_t st);
hipError_t launch_modconv_tail_async(const ConvParams &p, const TailArgs &ta, bool trunk_f16, hipStream_t st);

}  // namespace tpmd
