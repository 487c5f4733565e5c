// Modulated 3x3 convolution for the high-resolution, few-channel stages
// (input channels IC in {32, 64}, GEMM rows M in {32, 64, 128}; f16 operands):
// the same implicit GEMM as k_conv.hip, Y[m][n] = sum_k A[m][k] X(k, n) with
// k = tap*IC + ic, organised so that neither operand is re-read per tap:
//
//   * A stationary in registers.  Each wave owns 32 GEMM rows and keeps
//     their 9*IC columns as MFMA A fragments for the whole kernel (72 VGPRs
//     for IC = 32, 144 for IC = 64).
//   * B as a halo tile in LDS.  A workgroup computes a TH x 32 block of
//     output pixels of one frame; the (TH+2) x 34 input pixels around it (all
//     IC channels, zero outside the map) are staged in LDS once, and each tap
//     reads its B fragments as a shifted window of that tile — the im2col of
//     the reference (src/motion_dec.cpp:340-354) is never formed, and every
//     input byte leaves L2 about (TH+2)*34 / (TH*32) times instead of 9.
//   * Persistent workgroups.  Each workgroup walks tiles t, t + grid, ...;
//     the next tile's halo is loaded into registers while the current one is
//     multiplied, so a tile costs one LDS commit and two barriers.
//
// Epilogue: the store epilogue of k_conv.hip (dense or composed sub-pixel
// up-conv store, 1/den + bias + leaky + next style).  With the stage tail the
// A fragments keep one workgroup per CU and the tail's gather latency is
// exposed, so the fused conv + tail stages use the other kernels.
//
// MFMA: v_mfma_f32_32x32x16_f16; a 32-column block of the output is one row
// of the tile (32 consecutive pixels), lane % 32 its column.
#include "tpmd_conv.h"

namespace tpmd {

template <int IC, int M>
struct halo_cfg {
    static constexpr int NT = 256;
    static constexpr int WM = M / 32, WN = 4 / WM;       // waves along M / along tile rows
    static constexpr int TH = M == 128 ? 4 : 8;
    static constexpr int TW = 32;
    static constexpr int TN = TH / WN;                  // tile rows per wave
    static constexpr int BN = TH * TW;                  // pixels per tile
    static constexpr int HWD = TW + 2, HPX = (TH + 2) * HWD;
    static constexpr int ROWB = IC * 2 + 16;            // padded halo pixel (bytes)
    static constexpr int CPP = IC * 2 / 16;             // 16-byte chunks per pixel
    static constexpr int HCH = HPX * CPP;
    static constexpr int PF = (HCH + NT - 1) / NT;      // prefetch chunks per thread
    static constexpr int KS = IC / 16;                  // MFMA k steps per tap
    static constexpr int NAF = 9 * KS;                  // A fragments per wave
    static constexpr int HALO_BYTES = HPX * ROWB;
    static constexpr int LDS = HALO_BYTES;
    static_assert(WM * WN == 4 && TN * WN == TH, "wave layout");
};

template <int IC, int M, int MODE, typename TO>
__global__ __launch_bounds__(256) void modconv_halo_kernel(ConvParams p, int tiles_x,
                                                           int tiles_y, int ntiles) {
    typedef halo_cfg<IC, M> C;
    typedef half_t TA;
    constexpr int NT = C::NT, TW = C::TW, TN = C::TN, HWD = C::HWD, ROWB = C::ROWB;
    constexpr int CPP = C::CPP, HCH = C::HCH, PF = C::PF, KS = C::KS, NAF = C::NAF;
    __shared__ __attribute__((aligned(16))) char smem[C::LDS];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wid = tid >> 6;
    const int wm = wid / C::WN, wn = wid % C::WN;
    const int lrow = lane & 31;
    const int lk = (lane >> 5) * 16;
    const int H = p.H, W = p.W;
    const int K = 9 * IC;

    // this wave's A rows wm*32 + lane%32, all 9*IC columns: fragment f holds
    // k = f*16 + (lane/32)*8 .. +8 (f = tap*KS + ks)
    u32x4 af[NAF];
    {
        const TA *arow = (const TA *) p.A + (int64_t) (wm * 32 + lrow) * K + (lane >> 5) * 8;
        static_for<NAF>([&](auto f) { af[f] = *(const u32x4 *) (arow + f * 16); });
    }

    auto origin = [&](int t, int &b, int &y0, int &x0) {
        x0 = (t % tiles_x) * TW;
        const int q = t / tiles_x;
        y0 = (q % tiles_y) * C::TH;
        b = q / tiles_y;
    };
    u32x4 pf[PF];
    auto prefetch = [&](int t) {
        int b, y0, x0;
        origin(t, b, y0, x0);
        const TA *xb = (const TA *) p.X + (int64_t) b * p.x_bstride;
        static_for<PF>([&](auto i) {
            const int c = tid + i * NT;
            pf[i] = u32x4{0u, 0u, 0u, 0u};
            if (c < HCH) {
                const int px = c / CPP, kc = c - px * CPP;
                const int hy = px / HWD, hx = px - hy * HWD;
                const int iy = y0 + hy - 1, ix = x0 + hx - 1;
                if ((unsigned) iy < (unsigned) H && (unsigned) ix < (unsigned) W)
                    pf[i] = *(const u32x4 *) (xb + (int64_t) (iy * W + ix) * IC + kc * 8);
            }
        });
    };
    auto commit = [&]() {
        static_for<PF>([&](auto i) {
            const int c = tid + i * NT;
            if (c < HCH) {
                const int px = c / CPP, kc = c - px * CPP;
                *(u32x4 *) (smem + px * ROWB + kc * 16) = pf[i];
            }
        });
    };

    // workgroup ids reach the 8 XCDs round robin: the workgroups of one XCD
    // walk one contiguous range of tiles, so neighbouring tiles share an L2
    const int G = (int) gridDim.x;
    const int xcd = (int) blockIdx.x & 7, slot = (int) blockIdx.x >> 3;
    const int nx = (G - xcd + 7) >> 3;                      // workgroups on this XCD
    const int per = (ntiles + 7) >> 3;                      // tiles per XCD
    const int tbeg = xcd * per, tend = tbeg + per < ntiles ? tbeg + per : ntiles;
    int t = tbeg + slot;
    if (t < tend) prefetch(t);
    for (; t < tend; t += nx) {
        commit();
        __syncthreads();
        if (t + nx < tend) prefetch(t + nx);  // lands during the MFMAs

        floatx16 acc[TN];
#pragma unroll
        for (int b = 0; b < TN; b++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[b][v] = 0.0f;
        static_for<9>([&](auto tap_c) {
            constexpr int tap = decltype(tap_c)::value;
            constexpr int dy = tap / 3 - 1, dx = tap % 3 - 1;
            static_for<KS>([&](auto ks_c) {
                constexpr int ks = decltype(ks_c)::value;
#pragma unroll
                for (int b = 0; b < TN; b++) {
                    const int hy = wn * TN + b + dy + 1;
                    const u32x4 bf = *(const u32x4 *) (smem + (hy * HWD + lrow + dx + 1) * ROWB + ks * 32 + lk);
                    mfma_op<TA>::run(af[tap * KS + ks], bf, acc[b]);
                }
            });
        });

        int b0, y0, x0;
        origin(t, b0, y0, x0);
        const int n0 = (b0 * H + y0) * W + x0;  // top-left pixel of the tile
#pragma unroll
        for (int b = 0; b < TN; b++) {
            const int n = n0 + (wn * TN + b) * W + lrow;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = wm * 32 + i * 8 + (lane >> 5) * 4;
                const float q[4] = {acc[b][i * 4], acc[b][i * 4 + 1], acc[b][i * 4 + 2], acc[b][i * 4 + 3]};
                epi_store_quad<TO, MODE>(p, q, m, n);
            }
        }
        __syncthreads();  // halo reads done before the next commit
    }
}

// ---------------------------------------------------------------------------
// host side

bool modconv_halo_ok(bool f16, int mode, int IC, int OC, int H, int W, bool tail) {
    const int M = mode == MODE_DENSE ? OC : 4 * OC;
    if (!f16 || tail || (IC != 32 && IC != 64) || (M != 32 && M != 64 && M != 128)) return false;
    if (mode == MODE_SUBPIX && M != 128) return false;
    const int th = M == 128 ? 4 : 8;  // halo_cfg::TH
    return W % 32 == 0 && H % th == 0;
}

static int cu_count() {
    static int n = 0;
    if (!n) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
    }
    return n;
}

template <int IC, int M, int MODE, typename TO>
static hipError_t launch_halo_k(const ConvParams &p, hipStream_t st) {
    typedef halo_cfg<IC, M> C;
    const int tiles_x = p.W / C::TW, tiles_y = p.H / C::TH;
    const int nframes = p.N / (p.H * p.W);
    const int ntiles = tiles_x * tiles_y * nframes;
    auto kern = modconv_halo_kernel<IC, M, MODE, TO>;
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, C::NT, 0) != hipSuccess || occ < 1) occ = 1;
    int grid = cu_count() * occ;
    if (grid > ntiles) grid = ntiles;
    hipLaunchKernelGGL(kern, dim3((unsigned) grid), dim3(C::NT), 0, st, p, tiles_x, tiles_y, ntiles);
    return hipGetLastError();
}

template <int IC, int M, typename TO>
static hipError_t launch_halo_m(const ConvParams &p, int mode, hipStream_t st) {
    if (mode == MODE_DENSE) return launch_halo_k<IC, M, MODE_DENSE, TO>(p, st);
    if constexpr (M == 128) return launch_halo_k<IC, M, MODE_SUBPIX, TO>(p, st);
    return hipErrorInvalidValue;
}

template <typename TO>
static hipError_t launch_halo_t(const ConvParams &p, int mode, hipStream_t st) {
    const int M = p.M;
    if (p.IC == 32) {
        if (M == 32) return launch_halo_m<32, 32, TO>(p, mode, st);
        if (M == 64) return launch_halo_m<32, 64, TO>(p, mode, st);
        return launch_halo_m<32, 128, TO>(p, mode, st);
    }
    if (M == 32) return launch_halo_m<64, 32, TO>(p, mode, st);
    if (M == 64) return launch_halo_m<64, 64, TO>(p, mode, st);
    return launch_halo_m<64, 128, TO>(p, mode, st);
}

// f16 operands; out_f16: stored activation type
hipError_t launch_modconv_halo(const ConvParams &p, int mode, bool out_f16, hipStream_t st) {
    if (out_f16) return launch_halo_t<half_t>(p, mode, st);
    return launch_halo_t<float>(p, mode, st);
}

}  // namespace tpmd
