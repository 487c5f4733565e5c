// Dense 3x3 modulated conv + stage tail for the 32-channel stage
// (IC = OC = 32, f16 operands; src/motion_dec.cpp:357-373 then :1077-1108):
// the implicit GEMM of k_conv.hip on a halo tile, so every input pixel is
// fetched once per tile instead of once per tap:
//
//   * a workgroup owns a TH x 32 block of output pixels of one frame; the
//     (TH+2) x 34 input pixels around it (zero outside the map) go through
//     registers to LDS with a 16-byte pad per pixel (conflict-free 32-pixel
//     fragment reads); FRAG (A stored in MFMA fragment order, A_ORDER_FRAG:
//     18 fragments of 1 KB): every wave reads the 32 x 288 weight matrix
//     from L2 straight into registers, each tap's two fragments two taps
//     ahead of its MFMAs, so the LDS holds only the halo (49.5 KB: three
//     workgroups per CU at six waves per SIMD, 80 registers, against two when
//     A sat in LDS too; measured at r512, 16 frames: 194.6 -> 184.1 us on
//     synthetic operands, bit-identical); tap-major A goes global -> LDS by
//     the DMA path instead (one fragment of 32 rows x 16 bytes per DMA);
//   * wave w computes rows w*RPW .. of the block (RPW = 2): for each tap (dy, dx) and
//     16-channel step, the B fragment is the halo row shifted by (dy, dx);
//   * the activated tile goes to LDS over the halo and the two-phase stage
//     tail of tpmd_tail.h runs on it (the tail's skips and the folded ToFlow
//     weights are fetched with the halo, in one round trip).
// One global round trip for the conv instead of one per tap.
#include "tpmd_conv.h"

namespace tpmd {

// FG (the stage's warp feeds ToRGB alone, TailArgs::featg): each lane finishes
// its own pixel from the accumulators (the ToFlow dot in registers, halves
// joined across the two 32-lane halves), so the activated tile never goes to
// LDS and the workgroup needs only the halo, A and the ToFlow weights;
// F32_SWZ: 64-byte halo pixels, the 16-byte chunk index XORed with bits 2-3
// of the pixel index (16 consecutive pixels' reads of one chunk still hit
// distinct banks) instead of a 16-byte pad per pixel.
// Measured on MI355X, r512 at 16 frames (FG): 8 x 32 blocks of 4 waves,
// three per CU, 222 us; the same with F32_SWZ (four per CU) 184 us;
// 16 x 32 blocks of 8 waves (two per CU: A loaded once per 512 pixels, 18
// halo rows per 16) 175 us, 183 us with F32_SWZ.  The non-FG form keeps the
// same blocks (its activated tile takes 90 KB of LDS: one per CU).  A
// persistent form (each workgroup walking a run of tiles, A loaded once, the
// next tile's halo, skips and ToFlow weights requested under the current
// tile's conv) needs 200+ registers, two waves per SIMD: 213-221 us against
// 171; capped at four waves per SIMD it spills (531 us).
constexpr int F32_NT = 512;
constexpr bool F32_SWZ = false;

template <int TH, bool FG = false, bool AREG = false>
struct fused32_cfg {
    static constexpr int C = 32, NT = F32_NT, TW = 32, BN = TH * TW;
    static constexpr int HWD = TW + 2, HPX = (TH + 2) * HWD;
    static constexpr bool SWZ = FG && F32_SWZ;
    static constexpr int PXB = SWZ ? C * 2 : C * 2 + 16;  // halo pixel (bytes)
    static constexpr int CPP = C * 2 / 16;              // 16-byte chunks per pixel
    static constexpr int HCH = HPX * CPP;
    static constexpr int PF = (HCH + NT - 1) / NT;      // halo chunks per thread
    static constexpr int KS = C / 16;                   // MFMA k steps per tap
    static constexpr int NAF = 9 * KS;                  // A fragments
    static constexpr int RPW = TH / (NT / 64);          // output rows per wave
    typedef tile_tail_lds<C, BN> L;
    static constexpr int HALO = HPX * PXB;
    static constexpr int AOFF = (HALO + 255) / 256 * 256;  // A fragments, fragment-major
    static constexpr int CONV = AOFF + (AREG ? 0 : NAF * 1024);  // conv-phase LDS
    static constexpr int TAIL = FG ? 0 : L::WFS0 * 4;       // so + prm, over the conv's LDS
    // FG: the block's skip windows after the halo (after A when A sits in
    // LDS), then the ToFlow weights: 53.7 KB with A in registers, three
    // workgroups per CU at any LDS allocation granule up to 1280 bytes
    typedef skip_lds<TH, TW, NT> SK;
    static constexpr int SKOFF = FG ? (AREG ? (HALO + 15) / 16 * 16 : CONV) : 0;
    static constexpr int WFS = FG ? SKOFF + SK::FLOATS * 4 : (CONV > TAIL ? CONV : TAIL);
    static constexpr int LDS = WFS + 3 * C * 4;
    static_assert(TH % (NT / 64) == 0 && (FG ? BN == NT : BN % NT == 0), "rows per wave");
    static_assert(!FG || RPW == 2, "FG: a lane's two block rows are its pixel and its partner's");
    __device__ static int hoff(int px, int c) { return px * PXB + (SWZ ? (c ^ ((px >> 2) & 3)) : c) * 16; }
};

template <typename TF, typename TT, int TH, bool FRAG, bool FG>
__global__ __launch_bounds__(F32_NT) __attribute__((amdgpu_waves_per_eu(6))) void conv32_tail_kernel(
    ConvParams p, TailArgs ta, int tiles_x, int tiles_frame) {
    typedef half_t TA;
    constexpr bool AREG = FRAG;                 // A fragments from L2 into registers
    typedef fused32_cfg<TH, FG, AREG> F;
    typedef typename F::L L;
    constexpr int C = F::C, NT = F::NT, TW = F::TW, BN = F::BN, HWD = F::HWD, PXB = F::PXB;
    constexpr int CPP = F::CPP, HCH = F::HCH, PF = F::PF, KS = F::KS, NAF = F::NAF, RPW = F::RPW;
    constexpr int K = 9 * C;
    __shared__ __attribute__((aligned(16))) char smem[F::LDS];
    float *so = (float *) smem, *prm = so + L::PRM0, *wfs = (float *) (smem + F::WFS);

    const int tid = threadIdx.x;
    const int lane = tid & 63, wid = tid >> 6;
    const int tile = xcd_remap((int) blockIdx.x, (int) gridDim.x);
    const int fr = tile / tiles_frame;
    const int trem = tile - fr * tiles_frame;
    const int ty = trem / tiles_x, tx = trem - ty * tiles_x;
    const int H = p.H, W = p.W;
    const int y0 = ty * TH, x0 = tx * TW;
    const int n0 = (fr * H + y0) * W + x0;  // top-left pixel of the block

    // memory order, bounded by registers: the tail's skips and the halo are
    // requested together; once the skips are summed (the halo still in
    // flight) the A fragments and the frame's ToFlow weights follow.  FG: the
    // block's skip windows go to LDS with the halo instead (a few values per
    // thread), and each pixel sums its skips after the conv
    const TA *Xf = (const TA *) p.X + (int64_t) fr * p.x_bstride;
    u32x4 hv[PF];
    tail_skip sk{};
    float skv[F::SK::NV];
    float lx = 0.0f, ly = 0.0f;
    if constexpr (FG) {
        skip_window_load<TH, TW, NT>(ta, fr, y0, x0, tid, skv);
        lx = ta.lin[x0 + tid % TW];
        ly = ta.lin[y0 + tid / TW];
        halo_load<PF, NT, CPP, HWD, HCH, C>(Xf, H, W, y0, x0, tid, hv);
    } else {
        sk = tile_tail_skips_then<BN, TW>(ta, n0, tid, [&]() {
            halo_load<PF, NT, CPP, HWD, HCH, C>(Xf, H, W, y0, x0, tid, hv);
        });
    }
    const int lrow = lane & 31, khalf = lane >> 5;
    // A fragment f = tap*KS + step: lane l holds A[l%32][f*16 + (l/32)*8 .. +8]
    u32x4 areg[3][KS];   // AREG: tap t's fragments in set t % 3, requested two taps ahead
    // (through a buffer resource: this lane's byte offset fixed, the
    // fragment's offset scalar)
    const __amdgpu_buffer_rsrc_t ars =
        __builtin_amdgcn_make_buffer_rsrc((void *) p.A, (short) 0, (int) (C * K * 2), 0x00020000);
    auto load_a = [&](int tap, u32x4 (&dst)[KS]) {
        static_for<KS>([&](auto s) {
            dst[s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                   ars, (unsigned) (lane * 16), (int) ((tap * KS + s) * 1024), 0));
        });
    };
    if constexpr (AREG) {
        load_a(0, areg[0]);
        load_a(1, areg[1]);
    } else {
        const TA *arow = (const TA *) p.A + (int64_t) lrow * K + khalf * 8;
        for (int f = wid; f < NAF; f += NT / 64)
            __builtin_amdgcn_global_load_lds((const void *) (arow + f * 16),
                                             (__attribute__((address_space(3))) void *) (smem + F::AOFF + f * 1024),
                                             16, 0, 0);
    }
    const tail_wfs_regs<C, NT> wr = tile_tail_wfs_load<C, NT>(ta, fr, tid);
    static_for<PF>([&](auto i) {
        const int ch = tid + i * NT;
        if (ch < HCH) {
            const int px = ch / CPP, c = ch - px * CPP;
            *(u32x4 *) (smem + F::hoff(px, c)) = hv[i];
        }
    });
    tile_tail_wfs_store<C, NT>(wfs, tid, wr);
    if constexpr (FG) skip_window_store<TH, TW, NT>((float *) (smem + F::SKOFF), tid, skv);
    __syncthreads();  // (waits for the A fragments' DMA too, when A goes through LDS)

    // conv: acc[b] = 32 channels x the 32 pixels of output row wid*RPW + b
    floatx16 acc[RPW];
    static_for<RPW>([&](auto b) {
#pragma unroll
        for (int v = 0; v < 16; v++) acc[b][v] = 0.0f;
    });
    static_for<9>([&](auto tap) {
        constexpr int dy = tap / 3, dx = tap % 3;  // halo offsets of the tap
        if constexpr (AREG && tap + 2 < 9) load_a(tap + 2, areg[(tap + 2) % 3]);
        static_for<KS>([&](auto ks) {
            static_for<RPW>([&](auto b) {
                const int hrow = wid * RPW + b + dy;
                const u32x4 bf = *(const u32x4 *) (smem + F::hoff(hrow * HWD + lrow + dx, ks * 2 + khalf));
                u32x4 af;
                if constexpr (AREG) af = areg[tap % 3][ks];
                else af = *(const u32x4 *) (smem + F::AOFF + (tap * KS + ks) * 1024 + lane * 16);
                mfma_op<TA>::run(af, bf, acc[b]);
            });
        });
        __builtin_amdgcn_sched_barrier(0);  // bound the fragments in flight (registers)
    });

    // accumulator (b, v): channel (v/4)*8 + (lane/32)*4 + v%4, tile pixel (wid*RPW + b)*32 + lane%32
    if constexpr (FG) {
        // ToFlow dot over this lane's 16 channels of both block rows (the
        // c % 8 < 4 chain of the tile tail for khalf 0, the other for
        // khalf 1, same order); the lane keeps row khalf (tile pixel
        // wid*64 + lane = tid, whose skips it holds) and trades the other
        // row's sum with lane ^ 32
        float part[RPW][3];
        static_for<RPW>([&](auto b) {
#pragma unroll
            for (int k = 0; k < 3; k++) part[b][k] = 0.0f;
        });
        static_for<4>([&](auto i) {
            const int row = i * 8 + khalf * 4;
            // 1/den and bias of the frame's channels as scalar loads, each
            // lane half taking its four: no vector load (and no memory
            // round trip) after the conv
            floatx4 id, bb;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float d0 = ld_uniform(p.inv_den + (int64_t) fr * C, i * 8 + j);
                const float d1 = ld_uniform(p.inv_den + (int64_t) fr * C, i * 8 + 4 + j);
                const float b0 = ld_uniform(p.bias, i * 8 + j), b1 = ld_uniform(p.bias, i * 8 + 4 + j);
                id[j] = khalf ? d1 : d0;
                bb[j] = khalf ? b1 : b0;
            }
            floatx4 w[3];
#pragma unroll
            for (int k = 0; k < 3; k++) w[k] = *(const floatx4 *) (wfs + k * C + row);
            static_for<RPW>([&](auto b) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float v = leaky(acc[b][i * 4 + j] * id[j] + bb[j]);
#pragma unroll
                    for (int k = 0; k < 3; k++) part[b][k] = __builtin_fmaf(w[k][j], v, part[b][k]);
                }
            });
        });
        float fl[3];
#pragma unroll
        for (int k = 0; k < 3; k++) {
            const float mine = khalf ? part[1][k] : part[0][k];
            const float give = khalf ? part[0][k] : part[1][k];
            const float got = __shfl_xor(give, 32);
            fl[k] = khalf ? got + mine : mine + got;
        }
        const int pix = tile_pix<TW>(n0 - fr * (H * W), W, tid);
        const tail_skip skw =
            skip_from_window<TH, TW, NT>(ta, (const float *) (smem + F::SKOFF), y0, x0, x0 + tid % TW, y0 + tid / TW,
                                         lx, ly);
        taps4 t;
        float m;
        tail_flow_head(ta, fl, fr, pix, skw, t, m);
        tail_featg_rgb(ta, t, m, fr, pix, skw);
        return;
    }
    __syncthreads();  // halo reads done: the LDS becomes the activated tile
    static_for<RPW>([&](auto b) {
        const int col = (wid * RPW + b) * TW + lrow;
        static_for<4>([&](auto i) {
            const int row = i * 8 + khalf * 4;
            const floatx4 id = *(const floatx4 *) (p.inv_den + (int64_t) fr * C + row);
            const floatx4 bb = *(const floatx4 *) (p.bias + row);
            floatx4 v;
#pragma unroll
            for (int j = 0; j < 4; j++) v[j] = leaky(acc[b][i * 4 + j] * id[j] + bb[j]);
            *(floatx4 *) (so + col * L::SOS + row) = v;
        });
    });
    __syncthreads();
    tile_tail<TF, TT, C, BN, NT, TW>(ta, so, prm, wfs, n0, tid, sk);
}

// ---------------------------------------------------------------------------
// The 64-channel stage (IC = OC = 64): 4 x 32 blocks (the tail's 128
// pixels), four waves.  The halo goes to LDS through registers as above.  The
// two row blocks of 32 weight rows are split over the waves: wave w computes
// row block w&1 for block rows 2*(w>>1) .. +1.  Every wave reads its A
// fragments (C/16 of 1 KB per tap) straight from L2 into registers, two taps
// ahead of the MFMAs: no LDS for A and no barrier inside the conv, so the taps
// do not wait on one another's memory round trips.  LDS: the halo, then the
// activated tile (40 KB: four workgroups per CU).  FRAG: A in fragment order
// (A_ORDER_FRAG), each fragment one contiguous 1 KB.  The 128- and
// 256-channel stages run on modconv3x3_hfrag_tail_kernel (k_conv_hfrag_tail.hip:
// eight waves of 64 rows x 64 pixels, A per 32-channel k tile), which at
// C = 128 keeps four waves per SIMD against two for this form (r128 at 16
// frames: 115 -> 108 us).
template <int C_>
struct fusedh_cfg {
    static constexpr int C = C_, NT = 256, TH = 4, TW = 32, BN = TH * TW;
    static constexpr int HWD = TW + 2, HPX = (TH + 2) * HWD;
    static constexpr int PXB = C * 2 + 16;
    static constexpr int CPP = C * 2 / 16;
    static constexpr int HCH = HPX * CPP;
    static constexpr int PF = (HCH + NT - 1) / NT;
    static constexpr int KS = C / 16;                   // MFMA k steps per tap
    static constexpr int MBK = C / 32;                  // 32-row blocks of A
    static constexpr int RG = (NT / 64) / MBK;          // wave groups along the block rows
    static constexpr int RPW = TH / RG;                 // block rows per wave
    typedef tile_tail_lds<C, BN> L;
    static constexpr int HALO = HPX * PXB;
    static constexpr int CONV = (HALO + 255) / 256 * 256;
    static constexpr int TAIL = L::WFS0 * 4;
    static constexpr int WFS = CONV > TAIL ? CONV : TAIL;
    static constexpr int LDS = WFS + 3 * C * 4;
    static_assert(RG * MBK == NT / 64 && RG * RPW == TH, "wave grid");
};

// s_waitcnt immediate: vmcnt(n), expcnt and lgkmcnt not waited on
constexpr int fused_waitcnt_vm(int n) { return (n & 0xF) | (0x7 << 4) | (0xF << 8) | ((n >> 4) << 14); }

template <typename TF, typename TT, int C_, bool FRAG>
__global__ __launch_bounds__(256) void convh_tail_kernel(ConvParams p, TailArgs ta, int tiles_x,
                                                         int tiles_frame) {
    typedef half_t TA;
    typedef fusedh_cfg<C_> F;
    typedef typename F::L L;
    constexpr int C = F::C, NT = F::NT, TW = F::TW, BN = F::BN, HWD = F::HWD, PXB = F::PXB;
    constexpr int CPP = F::CPP, HCH = F::HCH, PF = F::PF, KS = F::KS, MBK = F::MBK, RPW = F::RPW;
    constexpr int K = 9 * C;
    __shared__ __attribute__((aligned(16))) char smem[F::LDS];
    float *so = (float *) smem, *prm = so + L::PRM0, *wfs = (float *) (smem + F::WFS);

    const int tid = threadIdx.x;
    const int lane = tid & 63, wid = tid >> 6;
    const int mb = wid % MBK, rg = wid / MBK;
    const int lrow = lane & 31, khalf = lane >> 5;
    const int tile = xcd_remap((int) blockIdx.x, (int) gridDim.x);
    const int fr = tile / tiles_frame;
    const int trem = tile - fr * tiles_frame;
    const int ty = trem / tiles_x, tx = trem - ty * tiles_x;
    const int H = p.H, W = p.W;
    const int y0 = ty * F::TH, x0 = tx * TW;
    const int n0 = (fr * H + y0) * W + x0;

    // A fragment (tap t, step s) of this wave's row block mb: lane l holds
    // A[32*mb + l%32][t*C + s*16 + (l/32)*8 .. +8] (fragment order: fragment
    // (t*KS + s)*MBK + mb); tap t's fragments go to register set t % 3
    const TA *Ab = (const TA *) p.A;
    const TA *arow = FRAG ? Ab + (mb * 64 + lane) * 8 : Ab + (int64_t) (mb * 32 + lrow) * K + khalf * 8;
    // FRAG: through a buffer resource, this lane's byte offset fixed and the
    // fragment's offset scalar
    const __amdgpu_buffer_rsrc_t ars =
        __builtin_amdgcn_make_buffer_rsrc((void *) p.A, (short) 0, (int) (C * K * 2), 0x00020000);
    const unsigned avoff = (unsigned) ((mb * 64 + lane) * 16);
    u32x4 af[3][KS];
    auto load_a = [&](int t, u32x4 (&dst)[KS]) {
        static_for<KS>([&](auto st) {
            constexpr int s = decltype(st)::value;
            if constexpr (FRAG)
                dst[s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                       ars, avoff, (int) ((t * KS + s) * MBK * 1024), 0));
            else
                dst[s] = *(const u32x4 *) (arow + t * C + s * 16);
        });
    };

    // memory order: skips + halo, then taps 0 and 1 of A and the ToFlow weights
    const TA *Xf = (const TA *) p.X + (int64_t) fr * p.x_bstride;
    u32x4 hv[PF];
    const tail_skip sk = tile_tail_skips_then<BN, TW>(ta, n0, tid, [&]() {
        halo_load<PF, NT, CPP, HWD, HCH, C>(Xf, H, W, y0, x0, tid, hv);
    });
    load_a(0, af[0]);
    load_a(1, af[1]);
    const tail_wfs_regs<C, NT> wr = tile_tail_wfs_load<C, NT>(ta, fr, tid);
    static_for<PF>([&](auto i) {
        const int ch = tid + i * NT;
        if (ch < HCH) {
            const int px = ch / CPP, c = ch - px * CPP;
            *(u32x4 *) (smem + px * PXB + c * 16) = hv[i];
        }
    });
    tile_tail_wfs_store<C, NT>(wfs, tid, wr);
    __syncthreads();  // halo and wfs in place

    floatx16 acc[RPW];
    static_for<RPW>([&](auto b) {
#pragma unroll
        for (int v = 0; v < 16; v++) acc[b][v] = 0.0f;
    });
    static_for<9>([&](auto tp) {
        constexpr int tap = decltype(tp)::value;
        constexpr int dy = tap / 3, dx = tap % 3;
        if constexpr (tap + 2 < 9) load_a(tap + 2, af[(tap + 2) % 3]);
        static_for<KS>([&](auto s) {
            static_for<RPW>([&](auto b) {
                const int hrow = rg * RPW + b + dy;
                const u32x4 bf =
                    *(const u32x4 *) (smem + (hrow * HWD + lrow + dx) * PXB + (s * 2 + khalf) * 16);
                mfma_op<TA>::run(af[tap % 3][s], bf, acc[b]);
            });
        });
        __builtin_amdgcn_sched_barrier(0);
    });
    __syncthreads();  // halo reads done: the LDS becomes the activated tile

    // accumulator (b, v): channel mb*32 + (v/4)*8 + (lane/32)*4 + v%4, tile pixel (rg*2 + b)*32 + lane%32
    static_for<RPW>([&](auto b) {
        const int col = (rg * RPW + b) * TW + lrow;
        static_for<4>([&](auto i) {
            const int row = mb * 32 + i * 8 + khalf * 4;
            const floatx4 id = *(const floatx4 *) (p.inv_den + (int64_t) fr * C + row);
            const floatx4 bb = *(const floatx4 *) (p.bias + row);
            floatx4 v;
#pragma unroll
            for (int j = 0; j < 4; j++) v[j] = leaky(acc[b][i * 4 + j] * id[j] + bb[j]);
            *(floatx4 *) (so + col * L::SOS + row) = v;
        });
    });
    __syncthreads();
    tile_tail<TF, TT, C, BN, NT, TW>(ta, so, prm, wfs, n0, tid, sk);
}

bool modconv_fused64_ok(bool f16, int IC, int OC, int r) { return f16 && IC == 64 && OC == 64 && r % 32 == 0; }

hipError_t launch_modconv_fused64(const ConvParams &p, const TailArgs &ta, bool trunk_f16, bool frag,
                                  hipStream_t st) {
    constexpr int TH = fusedh_cfg<64>::TH;
    if (p.IC != 64 || p.OC != 64 || p.M != 64 || p.W % 32 != 0 || p.H % TH != 0) return hipErrorInvalidValue;
    // the input halo is read through a buffer resource over one frame (32-bit offsets)
    if ((int64_t) p.H * p.W * p.IC * 2 >= ((int64_t) 1 << 31)) return hipErrorInvalidValue;
    const int tiles_x = p.W / 32, tiles_frame = tiles_x * (p.H / TH);
    const int nframes = p.N / (p.H * p.W);
    const dim3 grid((unsigned) (nframes * tiles_frame));
    auto go = [&](auto c) {
        constexpr int C = decltype(c)::value;
#define TPMD_L(TT, FR)                                                                                       \
    hipLaunchKernelGGL((convh_tail_kernel<half_t, TT, C, FR>), grid, dim3(256), 0, st, p, ta, tiles_x, \
                       tiles_frame)
        if (trunk_f16) {
            if (frag) TPMD_L(half_t, true);
            else TPMD_L(half_t, false);
        } else {
            if (frag) TPMD_L(float, true);
            else TPMD_L(float, false);
        }
#undef TPMD_L
    };
    go(std::integral_constant<int, 64>{});
    return hipGetLastError();
}

bool modconv_fused32_ok(bool f16, int IC, int OC, int r) { return f16 && IC == 32 && OC == 32 && r % 32 == 0; }

hipError_t launch_modconv_fused32(const ConvParams &p, const TailArgs &ta, bool trunk_f16, bool frag,
                                  hipStream_t st) {
    constexpr int TH = 16;
    if (p.IC != 32 || p.OC != 32 || p.M != 32 || p.W % 32 != 0 || p.H % TH != 0) return hipErrorInvalidValue;
    // the input halo is read through a buffer resource over one frame (32-bit offsets)
    if ((int64_t) p.H * p.W * p.IC * 2 >= ((int64_t) 1 << 31)) return hipErrorInvalidValue;
    const int tiles_x = p.W / 32, tiles_frame = tiles_x * (p.H / TH);
    const int nframes = p.N / (p.H * p.W);
    const dim3 grid((unsigned) (nframes * tiles_frame));
#define TPMD_L2(TT, FR, FG) \
    hipLaunchKernelGGL((conv32_tail_kernel<half_t, TT, TH, FR, FG>), grid, dim3(F32_NT), 0, st, p, ta, tiles_x, \
                       tiles_frame)
#define TPMD_L(TT, FR)                               \
    do {                                             \
        if (ta.featg && !ta.trunk && !ta.warp_tap) TPMD_L2(TT, FR, true); \
        else TPMD_L2(TT, FR, false);                 \
    } while (0)
    if (trunk_f16) {
        if (frag) TPMD_L(half_t, true);
        else TPMD_L(half_t, false);
    } else {
        if (frag) TPMD_L(float, true);
        else TPMD_L(float, false);
    }
#undef TPMD_L
#undef TPMD_L2
    return hipGetLastError();
}

}  // namespace tpmd
