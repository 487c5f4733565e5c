// Composed sub-pixel up-conv (conv_transpose 3x3 s2 o Blur 4x4 as one 3x3
// pad-1 conv with four output parity classes, styled_conv_up +
// subpix_lrelu_cl, src/motion_dec.cpp:397-433 and :980-994) for the
// 64 -> 32 channel stage (IC = 64, OC = 32, GEMM rows M = 4 * 32), f16
// operands and f16 output:
//
//   * a workgroup owns a TH x 32 block of low-resolution pixels of one frame;
//     its (TH+2) x 34 input halo (zero outside the map) is staged in LDS once
//     (144-byte pixel rows: conflict-free 32-pixel fragment reads);
//   * wave w computes parity class w (GEMM rows 32w .. 32w+31) for every
//     pixel of the block; its A fragments are read from L2 two taps ahead of
//     the MFMAs (four per tap), so the wave holds no full copy of A.  With A
//     in fragment order (FRAG) each of those reads is one contiguous 1 KB
//     (8 cache lines); tap-major A scatters it over 32 rows of A, 32 bytes
//     per line, which keeps the CU's address unit as busy as the MFMAs
//     (measured on MI355X at 16 frames: 226 -> 178 us for the r512 up-conv);
//   * the store epilogue (1/den, FusedLeakyReLU bias + leaky, next style) goes
//     through LDS: the four classes interleave into 2*TH output rows of 64
//     pixels, which are written as whole 16-byte chunks of contiguous
//     memory instead of 8-byte pieces two pixels apart.
#include "tpmd_conv.h"

namespace tpmd {

template <int TH>
struct up64_cfg {
    static constexpr int IC = 64, OC = 32, M = 4 * OC, NT = 256, TW = 32;
    static constexpr int HWD = TW + 2, HPX = (TH + 2) * HWD;
    static constexpr int PXB = IC * 2 + 16;            // padded halo pixel (bytes)
    static constexpr int CPP = IC * 2 / 16;            // 16-byte chunks per pixel
    static constexpr int HCH = HPX * CPP;
    static constexpr int PF = (HCH + NT - 1) / NT;
    static constexpr int KS = IC / 16;                 // MFMA k steps per tap
    static constexpr int OPX = 2 * TW;                 // output pixels per staged row
    static constexpr int OPB = OC * 2 + 16;            // padded staged output pixel (bytes)
    static constexpr int HALO = HPX * PXB;
    static constexpr int STAGE = 2 * TH * OPX * OPB;
    static constexpr int LDS = HALO > STAGE ? HALO : STAGE;
    static constexpr int OCH = 2 * TH * OPX * (OC * 2 / 16);  // 16-byte output chunks
    static_assert(OCH % NT == 0, "store pass");
};

// Four waves per SIMD (128 registers: the accumulators in VGPRs, no AGPRs),
// so four workgroups share a CU, as many as its LDS holds: measured at 16
// frames 178 -> 163 us against three per SIMD (160 registers).  Two waves of
// two classes each (each B fragment read from LDS feeding two MFMAs, 204
// registers, two waves per SIMD) measured no faster than three per SIMD.
template <int TH, bool FRAG>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void upconv64_kernel(ConvParams p,
                                                                                             int tiles_x,
                                                                                             int tiles_frame) {
    typedef half_t TA;
    typedef up64_cfg<TH> F;
    constexpr int IC = F::IC, OC = F::OC, NT = F::NT, TW = F::TW, HWD = F::HWD, PXB = F::PXB;
    constexpr int CPP = F::CPP, HCH = F::HCH, PF = F::PF, KS = F::KS, OPX = F::OPX, OPB = F::OPB;
    constexpr int K = 9 * IC;
    __shared__ __attribute__((aligned(16))) char smem[F::LDS];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wid = tid >> 6;
    const int lrow = lane & 31, khalf = lane >> 5;
    const int tile = xcd_remap((int) blockIdx.x, (int) gridDim.x);
    const int fr = tile / tiles_frame;
    const int trem = tile - fr * tiles_frame;
    const int ty = trem / tiles_x, tx = trem - ty * tiles_x;
    const int H = p.H, W = p.W;
    const int y0 = ty * TH, x0 = tx * TW;

    // halo -> registers, and the first tap's A fragments
    const TA *Xf = (const TA *) p.X + (int64_t) fr * p.x_bstride;
    u32x4 hv[PF];
    halo_load<PF, NT, CPP, HWD, HCH, IC>(Xf, H, W, y0, x0, tid, hv);
    // A fragment (tap, step): rows 32*wid + lane%32, k = tap*IC + step*16 + (lane/32)*8 .. +8
    const TA *arow = FRAG ? (const TA *) p.A + (wid * 64 + lane) * 8
                          : (const TA *) p.A + (int64_t) (wid * 32 + lrow) * K + khalf * 8;
    // FRAG: A through a buffer resource, this lane's byte offset fixed and
    // the fragment's offset scalar, so the loads need no VALU address
    // arithmetic (measured at 16 frames beside the library: 197 -> 193 us)
    const __amdgpu_buffer_rsrc_t ars =
        __builtin_amdgcn_make_buffer_rsrc((void *) p.A, (short) 0, (int) (F::M * K * 2), 0x00020000);
    const unsigned avoff = (unsigned) ((wid * 64 + lane) * 16);
    auto afrag = [&](int tap, int s) -> u32x4 {
        if constexpr (FRAG)
            return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 ars, avoff, (int) ((tap * KS + s) * (4 * 64 * 8) * 2), 0));
        return *(const u32x4 *) (arow + tap * IC + s * 16);
    };
    u32x4 af[3][KS];   // tap t's fragments in set t % 3, requested two taps ahead
    static_for<KS>([&](auto s) { af[0][s] = afrag(0, s); });
    static_for<KS>([&](auto s) { af[1][s] = afrag(1, s); });
    static_for<PF>([&](auto i) {
        const int ch = tid + i * NT;
        if (ch < HCH) {
            const int px = ch / CPP, c = ch - px * CPP;
            *(u32x4 *) (smem + px * PXB + c * 16) = hv[i];
        }
    });
    __syncthreads();

    // conv: acc[b] = class wid's 32 rows x the 32 pixels of block row b
    floatx16 acc[TH];
    static_for<TH>([&](auto b) {
#pragma unroll
        for (int v = 0; v < 16; v++) acc[b][v] = 0.0f;
    });
    static_for<9>([&](auto tap) {
        constexpr int dy = tap / 3, dx = tap % 3;  // halo offsets of the tap
        constexpr int cur = tap % 3;
        if constexpr (tap + 2 < 9)
            static_for<KS>([&](auto s) { af[(tap + 2) % 3][s] = afrag(tap + 2, s); });
        static_for<KS>([&](auto s) {
            static_for<TH>([&](auto b) {
                const u32x4 bf =
                    *(const u32x4 *) (smem + ((b + dy) * HWD + lrow + dx) * PXB + (s * 2 + khalf) * 16);
                mfma_op<TA>::run(af[cur][s], bf, acc[b]);
            });
            __builtin_amdgcn_sched_barrier(0);  // bound the reads in flight (registers)
        });
    });
    __syncthreads();  // halo reads done: the LDS becomes the output stage

    // epilogue: class (by, bx) = (wid >> 1, wid & 1) of low-res pixel (y0+b, x0+lrow) is
    // output pixel (2(y0+b)+by, 2(x0+lrow)+bx); channels i*8 + khalf*4 .. +4
    const int by = wid >> 1, bx = wid & 1;
    static_for<4>([&](auto i) {
        const int o = i * 8 + khalf * 4;
        const floatx4 id = *(const floatx4 *) (p.inv_den + (int64_t) fr * OC + o);
        const floatx4 bb = *(const floatx4 *) (p.bias + o);
        floatx4 sc = {1.0f, 1.0f, 1.0f, 1.0f};
        if (p.out_scale) sc = *(const floatx4 *) (p.out_scale + (int64_t) fr * OC + o);
        static_for<TH>([&](auto b) {
            half4 h;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float v = leaky(acc[b][i * 4 + j] * id[j] + bb[j]);
                if (p.out_scale) v *= sc[j];
                h[j] = (half_t) v;
            }
            *(half4 *) (smem + ((2 * b + by) * OPX + 2 * lrow + bx) * OPB + o * 2) = h;
        });
    });
    __syncthreads();

    // store pass: 2*TH output rows of 64 pixels x 64 bytes, contiguous in Y
    half_t *Yf = (half_t *) p.Y + (int64_t) fr * 4 * H * W * OC;
    static_for<F::OCH / NT>([&](auto j) {
        const int c = tid + j * NT;
        const int row = c / (OPX * 4), rem = c - row * (OPX * 4);
        const int px = rem >> 2, part = rem & 3;
        const u32x4 v = *(const u32x4 *) (smem + (row * OPX + px) * OPB + part * 16);
        *(u32x4 *) (Yf + ((int64_t) (2 * y0 + row) * (2 * W) + 2 * x0 + px) * OC + part * 8) = v;
    });
}

// block rows: 4 keeps the accumulators at 64 registers
constexpr int UP64_TH = 4;

bool modconv_up64_ok(bool f16, bool out_f16, int mode, int IC, int OC, int H, int W) {
    return f16 && out_f16 && mode == MODE_SUBPIX && IC == 64 && OC == 32 && W % 32 == 0 && H % UP64_TH == 0;
}

hipError_t launch_modconv_up64(const ConvParams &p, bool frag, hipStream_t st) {
    constexpr int TH = UP64_TH;
    if (p.IC != 64 || p.OC != 32 || p.M != 128 || p.W % 32 != 0 || p.H % TH != 0) return hipErrorInvalidValue;
    // the input halo is read through a buffer resource over one frame (32-bit offsets)
    if ((int64_t) p.H * p.W * p.IC * 2 >= ((int64_t) 1 << 31)) return hipErrorInvalidValue;
    const int tiles_x = p.W / 32, tiles_frame = tiles_x * (p.H / TH);
    const int nframes = p.N / (p.H * p.W);
    if (frag)
        hipLaunchKernelGGL((upconv64_kernel<TH, true>), dim3((unsigned) (nframes * tiles_frame)), dim3(256), 0, st,
                           p, tiles_x, tiles_frame);
    else
        hipLaunchKernelGGL((upconv64_kernel<TH, false>), dim3((unsigned) (nframes * tiles_frame)), dim3(256), 0,
                           st, p, tiles_x, tiles_frame);
    return hipGetLastError();
}

}  // namespace tpmd
