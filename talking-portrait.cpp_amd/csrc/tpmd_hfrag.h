// The halo conv kernel (modconv3x3_hfrag_kernel) and its launch for one
// chunk count NC, instantiated per NC in k_conv_hfrag*.hip so the large
// unrolled kernels compile in parallel.
#pragma once

#include "tpmd_halo.h"

namespace tpmd {

// Halo convs (f16 operands, every tile inside one frame): a tile is BM GEMM
// rows x a TH x TW block of pixels of one frame, and the k order is
// channel-chunk major, k tile t = c*9 + tap (32 channels c*32 .. +31 of tap
// `tap`).  Per chunk the (TH+2) x (TW+2) halo of those 32 channels sits in
// one of two LDS halo buffers (80-byte pixels: 4 chunks of 8 channels + a pad
// chunk, so 32 consecutive pixels read at any offset hit distinct banks), and
// its 9 taps read it shifted by (dy, dx): the B bytes moved per chunk drop
// from 9 x 16 KB of im2col rows to one halo of at most 32 KB.
//
// A is read by every wave straight from L2 in MFMA fragment order
// (A_ORDER_FRAG: each fragment is one contiguous 1 KB), not through LDS.
// NW waves, each 32*TM rows x 32*TN pixels (WM = BM/(32*TM) wave rows, WN =
// NW/WM wave columns): per 16-wide k step a wave reads TM A fragments and TN
// B fragments for TM*TN MFMAs.  The waves that share A rows read the same
// lines and find them in L1.  The LDS holds only the two halo buffers, so the
// one barrier per 32-channel chunk (9 k tiles) is the halo hand-over; A needs
// no barrier.
//   * A fragments are requested two k tiles ahead into three register sets
//     (k tile t in set t % 3; 9 taps per chunk keep the set of a tap fixed);
//   * the B fragments of the next k step are read from LDS while the
//     current step's MFMAs run;
//   * the halo of chunk c+1 is loaded into registers early in chunk c and
//     written to the other LDS buffer late in it; one barrier ends the chunk.
// Configurations (hfrag_config):
//   * 256 rows x 8 x 32 pixels (the r64 and r128 up-convs): eight waves of
//     64 x 128 (two per SIMD), and for IC = 512 (the r64 up-conv) four waves
//     of 128 x 128 (one per SIMD, 16 MFMAs per 4 A and 4 B fragments: half
//     the A requests per MFMA; 137 -> 132 us per 16-frame launch in the
//     decoder; the r128 up-conv measured the same either way);
//   * 128 rows x 8 x 32 pixels on four waves of 64 x 128 for IC = 128 (the
//     r256 up-conv): at most 256 registers and 68 KB of LDS, so two
//     workgroups share a CU and one's prologue and store epilogue run under
//     the other's MFMAs (155.3 -> 150.8 us per 16-frame launch against the
//     one-per-CU 256-row form);
//   * 128 rows x 8 x 32 or x 16 x 16 pixels where 256 rows leave fewer than
//     256 tiles at 16 frames (the r32 convs: a 32 x 32 map, a 16 x 16 up-conv
//     input): eight waves of 64 x 64, and for IC = 512 four waves of 64 x 128:
//     the up-conv on 16 x 16 blocks (the r32 up-conv, 76 -> 72 us) and the
//     dense conv with f32 output (the r32 dense conv, whose f32 stage then
//     goes out in two passes of 128 pixels, 67.6 KB, two workgroups per CU:
//     78 -> 76 us);
// f16 output, or f32 output of a dense conv on 128 rows.  The output goes
// through an LDS stage ([pixel][row], f16 or f32) and is written as whole
// 16-byte chunks of contiguous memory.

template <int BM_, int TH_, int TW_, int NW_ = 8, int TM_ = 2>
struct hfrag_cfg {
    static constexpr int BM = BM_, TH = TH_, TW = TW_, BN = TH * TW;
    static constexpr int NW = NW_, NT = NW * 64;
    static constexpr int TM = TM_, WM = BM / (32 * TM), WN = NW / WM;    // wave grid
    static constexpr int TN = BN / 32 / WN;
    static constexpr int HWD = TW + 2, HPX = (TH + 2) * HWD;
    static constexpr int LPH = HR_HBUF / 1024 / NW;      // halo units of 1 KB per wave per chunk
    static_assert(WM * WN == NW && TN * 32 * WN == BN && BN == 256, "wave grid");
    static_assert(HPX * HR_PXB <= HR_HBUF, "halo buffer");
};

// WPE: waves per SIMD the registers must allow (2: at most 256 registers, so
// two four-wave workgroups share a CU)
template <int MODE, int NC, int BM, int TH, int TW, typename TO, int NW_ = 8, int TM_ = 2, int WPE = 1>
__global__ __launch_bounds__(NW_ * 64) __attribute__((amdgpu_waves_per_eu(WPE))) void modconv3x3_hfrag_kernel(
    ConvParams p, int tiles_x, int tiles_frame) {
    typedef half_t TA;
    typedef hfrag_cfg<BM, TH, TW, NW_, TM_> F;
    constexpr int NW = F::NW, NT = F::NT, WN = F::WN, BN = F::BN, TM = F::TM, TN = F::TN;
    constexpr int HWD = F::HWD, HPX = F::HPX, LPH = F::LPH;
    // staged output, one padded row per pixel; f32 output of four waves goes
    // through in two passes of half the pixels (each pass the tile of half
    // the wave columns), so its stage fits beside a second workgroup
    constexpr int ORS = BM * (int) sizeof(TO) + 16;
    constexpr int NP = sizeof(TO) == 4 && NW == 4 && WN % 2 == 0 ? 2 : 1, BNP = BN / NP, OUT = BNP * ORS;
    constexpr int LDS = 2 * HR_HBUF > OUT ? 2 * HR_HBUF : OUT;
    __shared__ __attribute__((aligned(16))) char smem[LDS];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wid = tid >> 6;
    const int wm = wid / WN, wn = wid % WN;
    const int tile = xcd_remap((int) blockIdx.x, (int) gridDim.x);
    const int mt = tile % p.MT, nt = tile / p.MT;
    const int fr = nt / tiles_frame;
    const int trem = nt - fr * tiles_frame;
    const int ty = trem / tiles_x;
    const int y0 = ty * TH, x0 = (trem - ty * tiles_x) * TW;
    const int m0 = mt * BM;
    constexpr int IC = NC * 32, KSA = IC / 16;
    const int H = p.H, W = p.W;
    const int MB = p.M / 32;

    // A fragment (tap, ks) of row block w = m0/32 + wm*TM + a: 1 KB at
    // ((tap*KSA + ks)*MB + w) KB; this lane's 16 bytes of it.
    // A is read through a buffer resource: this lane's byte offset in the
    // fragment is fixed (vector offset), the fragment's own offset is the
    // same for every lane (scalar offset), so no per-load 64-bit address
    // arithmetic runs on the VALU (measured at 16 frames: r64 / r128 / r256
    // up-convs 141 / 151 / 168 -> 136 / 145 / 167 us beside the library)
    const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(
        (void *) p.A, (short) 0, (int) ((int64_t) p.M * 9 * IC * (int) sizeof(TA)), 0x00020000);
    const unsigned avoff = (unsigned) (((m0 / 32 + wm * TM) * 512 + lane * 8) * (int) sizeof(TA));
    auto afrag = [&](int tap, int ks, int a) -> u32x4 {
        return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             ars, avoff, (int) (((tap * KSA + ks) * MB + a) * 1024), 0));
    };
    u32x4 af[3][TM][2];
    auto load_a = [&](int c, int tap, u32x4 (&dst)[TM][2]) {
        static_for<2>([&](auto s) { static_for<TM>([&](auto a) { dst[a][s] = afrag(tap, 2 * c + s, a); }); });
    };

    // halo unit u = (wid*LPH + h)*64 + lane of a halo buffer: halo pixel u / 5,
    // channel chunk u % 5 (4: the pad), read through a buffer resource over
    // the input: the unit's byte offset as the vector offset (2^31, past the
    // extent, for pads, units past the halo and pixels outside the map, which
    // the hardware answers with zeros) and the chunk's offset as the scalar one
    const int64_t xbytes = (int64_t) (p.N / (H * W)) * p.x_bstride * (int) sizeof(TA);
    const __amdgpu_buffer_rsrc_t xrs =
        __builtin_amdgcn_make_buffer_rsrc((void *) p.X, (short) 0, (int) xbytes, 0x00020000);
    unsigned hvo[LPH];
#pragma unroll
    for (int h = 0; h < LPH; h++) {
        const int u = (wid * LPH + h) * 64 + lane;
        const int hp = u / 5, q = u - hp * 5;
        const int hy = hp / HWD, hx = hp - hy * HWD;
        const int iy = y0 - 1 + hy, ix = x0 - 1 + hx;
        const bool ok = q < 4 && hp < HPX && (unsigned) iy < (unsigned) H && (unsigned) ix < (unsigned) W;
        hvo[h] = ok ? (unsigned) (((int64_t) fr * p.x_bstride + ((int64_t) iy * W + ix) * IC + q * 8) *
                                  (int) sizeof(TA))
                    : 0x80000000u;
    }
    // the halo goes through registers rather than the LDS DMA path: the
    // compiler then counts every load exactly, while after an LDS DMA it
    // waits for all loads in flight before the next MFMA
    u32x4 hreg[LPH];
    auto load_h = [&](int c) {
        static_for<LPH>([&](auto h) {
            hreg[h] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, hvo[h], c * 64, 0));
        });
    };
    auto store_h = [&](int c) {
        char *buf = smem + (c & 1) * HR_HBUF;
        static_for<LPH>([&](auto h) { *(u32x4 *) (buf + (wid * LPH + h) * 1024 + lane * 16) = hreg[h]; });
    };

    floatx16 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; a++)
#pragma unroll
        for (int b = 0; b < TN; b++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[a][b][v] = 0.0f;

    const int lrow = lane & 31, khalf = lane >> 5;
    // this lane's halo pixel for tap (0, 0) of fragment b: block pixel
    // (wn*TN + b)*32 + lrow
    int hoff[TN];
    static_for<TN>([&](auto b) {
        const int n = (wn * TN + b) * 32 + lrow;
        hoff[b] = ((n / TW) * HWD + n % TW) * HR_PXB + khalf * 16;
    });
    auto read_b = [&](const char *hb, int tap, int s, u32x4 (&bf)[TN]) {
        const int dy = tap / 3, dx = tap - dy * 3;
        const char *q = hb + (dy * HWD + dx) * HR_PXB + s * 32;
        static_for<TN>([&](auto b) { bf[b] = *(const u32x4 *) (q + hoff[b]); });
    };

    load_h(0);
    load_a(0, 0, af[0]);
    load_a(0, 1, af[1]);
    store_h(0);
    __syncthreads();
    // the chunks unrolled (NC is a template argument), so the compiler's
    // memory-counter waits are exact: no wait drains the loads in flight
    static_for<NC>([&](auto cc) {
        constexpr int c = decltype(cc)::value;
        const char *hb = smem + (c & 1) * HR_HBUF;
        u32x4 bcur[TN];
        read_b(hb, 0, 0, bcur);
        static_for<18>([&](auto q) {
            constexpr int u = q / 2, s = q % 2;
            // requests first (A of k tile t + 2, B of the next step), then the MFMAs
            if constexpr (s == 0) {
                if constexpr (u + 2 < 9) load_a(c, u + 2, af[(u + 2) % 3]);
                else if constexpr (c + 1 < NC) load_a(c + 1, u + 2 - 9, af[(u + 2) % 3]);
            }
            u32x4 bnext[TN];
            if constexpr (q + 1 < 18) read_b(hb, (q + 1) / 2, (q + 1) % 2, bnext);
            __builtin_amdgcn_sched_barrier(0);
            static_for<TM>([&](auto a) {
                static_for<TN>([&](auto b) { mfma_op<TA>::run(af[u % 3][a][s], bcur[b], acc[a][b]); });
            });
            if constexpr (q + 1 < 18) static_for<TN>([&](auto b) { bcur[b] = bnext[b]; });
            __builtin_amdgcn_sched_barrier(0);
            // the next chunk's halo: requested after the first step, written
            // (into the buffer whose last reads, chunk c-1's, ended before
            // the barrier) after the 13th, when it has long arrived
            if constexpr (q == 0 && c + 1 < NC) load_h(c + 1);
            if constexpr (q == 12 && c + 1 < NC) store_h(c + 1);
        });
        if constexpr (c + 1 < NC) __syncthreads();   // halo c+1 written, chunk c's reads done
    });

    // store epilogue: the tile is staged in LDS as [pixel][row] (ORS-byte
    // rows) and written back as whole 16-byte chunks of contiguous output,
    // in NP passes of BNP pixels (pass h: the waves of wave columns
    // h*WN/NP ..)
    constexpr int EPC = 16 / (int) sizeof(TO);           // output elements per 16-byte chunk
    constexpr int CPR = BM / EPC, NCH = BNP * CPR, STEP = NT / CPR;
    static_assert(NCH % NT == 0 && NT % CPR == 0 && WN % NP == 0, "store pass");
    const int mc = tid % CPR;
    const int m = m0 + mc * EPC;
    int cls = 0, o = m;
    if constexpr (MODE == MODE_SUBPIX) {
        cls = m / p.OC;
        o = m - cls * p.OC;
    }
    const int64_t HW = (int64_t) H * W;
    TO *Yp = (TO *) p.Y;
    static_for<NP>([&](auto hh) {
        constexpr int h = decltype(hh)::value;
        __syncthreads();   // the halo's (h = 0) or the previous pass's reads are done
        if (wn / (WN / NP) == h) {
            static_for<TN>([&](auto b) {
                const int nl = (wn * TN + b) * 32 + lrow - h * BNP;
                static_for<TM>([&](auto a) {
                    static_for<4>([&](auto i) {
                        const int ml = (wm * TM + a) * 32 + i * 8 + khalf * 4;
                        const int mr = m0 + ml;
                        const int orow = MODE == MODE_DENSE ? mr : mr % p.OC;
                        const floatx4 id = *(const floatx4 *) (p.inv_den + (int64_t) fr * p.OC + orow);
                        const floatx4 bb = *(const floatx4 *) (p.bias + orow);
                        floatx4 sc = {1.0f, 1.0f, 1.0f, 1.0f};
                        if (p.out_scale) sc = *(const floatx4 *) (p.out_scale + (int64_t) fr * p.OC + orow);
                        floatx4 v;
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            v[j] = leaky(acc[a][b][i * 4 + j] * id[j] + bb[j]);
                            if (p.out_scale) v[j] *= sc[j];
                        }
                        if constexpr (sizeof(TO) == 2) {
                            half4 hv;
#pragma unroll
                            for (int j = 0; j < 4; j++) hv[j] = (half_t) v[j];
                            *(half4 *) (smem + nl * ORS + ml * 2) = hv;
                        } else {
                            *(floatx4 *) (smem + nl * ORS + ml * 4) = v;
                        }
                    });
                });
            });
        }
        __syncthreads();
        static_for<NCH / NT>([&](auto j) {
            const int nq = tid / CPR + j * STEP;   // pixel of this pass
            const int nl = h * BNP + nq;
            const int y = y0 + nl / TW, x = x0 + nl % TW;
            int64_t opix;
            if constexpr (MODE == MODE_DENSE) opix = fr * HW + (int64_t) y * W + x;
            else opix = fr * 4 * HW + (int64_t) (2 * y + (cls >> 1)) * (2 * W) + 2 * x + (cls & 1);
            const u32x4 v = *(const u32x4 *) (smem + nq * ORS + mc * 16);
            *(u32x4 *) (Yp + opix * p.OC + o) = v;
        });
    });
}

// launch of a conv with IC = 32 * NC on halo configuration cfg (1 = 256 rows
// x 8 x 32 pixels, 2 = 128 rows x 8 x 32, 3 = 128 rows x 16 x 16); p.MT and
// p.T set by the caller
template <int NC>
hipError_t launch_hfrag_nc(const ConvParams &p, int cfg, int mode, bool out_f16, int tiles_x, int tiles_frame,
                           dim3 grid, hipStream_t st) {
    auto go = [&](auto bm, auto th, auto tw) {
        constexpr int B = decltype(bm)::value;
        constexpr int T_H = decltype(th)::value, T_W = decltype(tw)::value;
        if constexpr (NC == 16 && B == 256) {
            if (mode == MODE_SUBPIX) {
                hipLaunchKernelGGL((modconv3x3_hfrag_kernel<MODE_SUBPIX, NC, B, T_H, T_W, half_t, 4, 4>), grid,
                                   dim3(256), 0, st, p, tiles_x, tiles_frame);
                return hipGetLastError();
            }
        }
        if constexpr (NC == 4 && B == 128 && T_H == 8) {
            if (mode == MODE_SUBPIX) {
                hipLaunchKernelGGL((modconv3x3_hfrag_kernel<MODE_SUBPIX, NC, B, T_H, T_W, half_t, 4, 2, 2>), grid,
                                   dim3(256), 0, st, p, tiles_x, tiles_frame);
                return hipGetLastError();
            }
        }
        if constexpr (NC == 16 && B == 128 && T_H == 16) {
            if (mode == MODE_SUBPIX) {
                hipLaunchKernelGGL((modconv3x3_hfrag_kernel<MODE_SUBPIX, NC, B, T_H, T_W, half_t, 4, 2>), grid,
                                   dim3(256), 0, st, p, tiles_x, tiles_frame);
                return hipGetLastError();
            }
        }
        if constexpr (NC == 16 && B == 128) {
            if (mode == MODE_DENSE && !out_f16) {
                hipLaunchKernelGGL((modconv3x3_hfrag_kernel<MODE_DENSE, NC, B, T_H, T_W, float, 4, 2>), grid,
                                   dim3(256), 0, st, p, tiles_x, tiles_frame);
                return hipGetLastError();
            }
        }
        if (mode == MODE_SUBPIX)
            hipLaunchKernelGGL((modconv3x3_hfrag_kernel<MODE_SUBPIX, NC, B, T_H, T_W, half_t>), grid, dim3(512), 0,
                               st, p, tiles_x, tiles_frame);
        else if (out_f16)
            hipLaunchKernelGGL((modconv3x3_hfrag_kernel<MODE_DENSE, NC, B, T_H, T_W, half_t>), grid, dim3(512), 0,
                               st, p, tiles_x, tiles_frame);
        else if constexpr (B == 128)   // a 256-row f32 stage would not fit the LDS
            hipLaunchKernelGGL((modconv3x3_hfrag_kernel<MODE_DENSE, NC, B, T_H, T_W, float>), grid, dim3(512), 0,
                               st, p, tiles_x, tiles_frame);
        else
            return hipErrorInvalidValue;
        return hipGetLastError();
    };
    if (cfg == 1)
        return go(std::integral_constant<int, 256>{}, std::integral_constant<int, 8>{},
                  std::integral_constant<int, 32>{});
    if (cfg == 2)
        return go(std::integral_constant<int, 128>{}, std::integral_constant<int, 8>{},
                  std::integral_constant<int, 32>{});
    return go(std::integral_constant<int, 128>{}, std::integral_constant<int, 16>{},
              std::integral_constant<int, 16>{});
}

// instantiated in k_conv_hfrag.hip (NC = 1, 2, 4), k_conv_hfrag8.hip, k_conv_hfrag16.hip
#define TPMD_HFRAG_NC(NC)                                                                                  \
    template hipError_t launch_hfrag_nc<NC>(const ConvParams &, int, int, bool, int, int, dim3, hipStream_t)
extern TPMD_HFRAG_NC(8);
extern TPMD_HFRAG_NC(16);

}  // namespace tpmd
