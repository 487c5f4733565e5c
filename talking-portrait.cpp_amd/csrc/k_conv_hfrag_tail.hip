// Dense conv + stage tail for C = 128 and 256 (the r128 and r64 stages) on
// the halo conv of k_conv_hfrag.hip.
#include "tpmd_halo.h"

namespace tpmd {

// The conv (A fragments from L2, each 32-channel chunk's input halo in LDS,
// chunk-major k) runs on 4 x 32 pixel blocks, 256 rows = every channel of the block, eight
// waves of 64 rows x 64 pixels; the activated 256 x 128 tile then goes to LDS
// as f32 and the two-phase tile tail runs on it.  The tail's skips, the
// ToFlow weights and the first chunk's halo are requested together.
// the C = 256 and C = 128 dense conv + tail on this kernel (else on the
// im2col ring and the register-staged tiles of k_conv.hip)
constexpr bool HFRAG_TAIL = true, HFRAG_TAIL128 = true;

constexpr int HT_TH = 4, HT_TW = 32, HT_HWD = HT_TW + 2, HT_HPX = (HT_TH + 2) * HT_HWD;
constexpr int HT_HBUF = 16 * 1024;      // one halo buffer: 16 units of 1 KB
static_assert(HT_HPX * HR_PXB <= HT_HBUF, "halo buffer");

template <int C_>
struct hfrag_tail_cfg {
    static constexpr int C = C_, NW = 8, NT = 512, BN = HT_TH * HT_TW;
    static constexpr int WM = 4, WN = 2, TM = C / 32 / WM, TN = BN / 32 / WN;
    static constexpr int LPH = HT_HBUF / 1024 / NW;
    typedef tile_tail_lds<C, BN> L;
    static constexpr int CONV = 2 * HT_HBUF;
    static constexpr int TAIL = L::WFS0 * 4;             // so + prm, over the conv's LDS
    static constexpr int WFS = CONV > TAIL ? CONV : TAIL;
    static constexpr int LDS = WFS + 3 * C * 4;
    static_assert(TM >= 1 && TN >= 1 && HT_HPX * 5 <= LPH * 64 * NW, "wave grid");
};

template <typename TF, typename TT, int C>
__global__ __launch_bounds__(512) void modconv3x3_hfrag_tail_kernel(ConvParams p, TailArgs ta, int tiles_x,
                                                                    int tiles_frame) {
    typedef half_t TA;
    typedef hfrag_tail_cfg<C> F;
    typedef typename F::L L;
    constexpr int NT = F::NT, WN = F::WN, BN = F::BN, TM = F::TM, TN = F::TN, LPH = F::LPH;
    constexpr int NC = C / 32, KSA = C / 16, MB = C / 32;
    __shared__ __attribute__((aligned(16))) char smem[F::LDS];
    float *so = (float *) smem, *prm = so + L::PRM0, *wfs = (float *) (smem + F::WFS);

    const int tid = threadIdx.x;
    const int lane = tid & 63, wid = tid >> 6;
    const int wm = wid / WN, wn = wid % WN;
    const int lrow = lane & 31, khalf = lane >> 5;
    const int tile = xcd_remap((int) blockIdx.x, (int) gridDim.x);
    const int fr = tile / tiles_frame;
    const int trem = tile - fr * tiles_frame;
    const int ty = trem / tiles_x;
    const int y0 = ty * HT_TH, x0 = (trem - ty * tiles_x) * HT_TW;
    const int H = p.H, W = p.W;
    const int n0 = (fr * H + y0) * W + x0;  // top-left pixel of the block

    // A fragment (tap, ks) of row block w = wm*TM + a: 1 KB at ((tap*KSA + ks)*MB + w) KB
    // A through a buffer resource: this lane's byte offset fixed, the
    // fragment's offset scalar (no VALU address arithmetic per load)
    const __amdgpu_buffer_rsrc_t ars =
        __builtin_amdgcn_make_buffer_rsrc((void *) p.A, (short) 0, (int) (C * 9 * C * 2), 0x00020000);
    const unsigned avoff = (unsigned) (((wm * TM) * 512 + lane * 8) * 2);
    auto afrag = [&](int tap, int ks, int a) -> u32x4 {
        return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             ars, avoff, (int) (((tap * KSA + ks) * MB + a) * 1024), 0));
    };
    u32x4 af[3][TM][2];
    auto load_a = [&](int c, int tap, u32x4 (&dst)[TM][2]) {
        static_for<2>([&](auto s) { static_for<TM>([&](auto a) { dst[a][s] = afrag(tap, 2 * c + s, a); }); });
    };

    // halo unit u = (wid*LPH + h)*64 + lane: halo pixel u / 5, chunk u % 5 (4: the pad),
    // through a buffer resource over the input: this lane's unit's byte
    // offset (past the extent for a unit outside the map, which the hardware
    // answers with zeros) and the chunk's offset as the scalar offset
    const int64_t xbytes = (int64_t) (p.N / (H * W)) * p.x_bstride * (int) sizeof(TA);
    const __amdgpu_buffer_rsrc_t xrs =
        __builtin_amdgcn_make_buffer_rsrc((void *) p.X, (short) 0, (int) xbytes, 0x00020000);
    unsigned hvo[LPH];
#pragma unroll
    for (int h = 0; h < LPH; h++) {
        const int u = (wid * LPH + h) * 64 + lane;
        const int hp = u / 5, q = u - hp * 5;
        const int hy = hp / HT_HWD, hx = hp - hy * HT_HWD;
        const int iy = y0 - 1 + hy, ix = x0 - 1 + hx;
        const bool ok = q < 4 && hp < HT_HPX && (unsigned) iy < (unsigned) H && (unsigned) ix < (unsigned) W;
        hvo[h] = ok ? (unsigned) (((int64_t) fr * p.x_bstride + ((int64_t) iy * W + ix) * C + q * 8) *
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
        char *buf = smem + (c & 1) * HT_HBUF;
        static_for<LPH>([&](auto h) { *(u32x4 *) (buf + (wid * LPH + h) * 1024 + lane * 16) = hreg[h]; });
    };

    // memory order: skips + the first halo chunk, then A and the ToFlow weights
    const tail_skip sk = tile_tail_skips_then<BN, HT_TW>(ta, n0, tid, [&]() { load_h(0); });
    load_a(0, 0, af[0]);
    load_a(0, 1, af[1]);
    const tail_wfs_regs<C, NT> wr = tile_tail_wfs_load<C, NT>(ta, fr, tid);
    store_h(0);
    tile_tail_wfs_store<C, NT>(wfs, tid, wr);
    __syncthreads();

    floatx16 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; a++)
#pragma unroll
        for (int b = 0; b < TN; b++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[a][b][v] = 0.0f;
    // this lane's halo pixel for tap (0, 0) of fragment b: block pixel (wn*TN + b)*32 + lrow
    int hoff[TN];
    static_for<TN>([&](auto b) {
        const int n = (wn * TN + b) * 32 + lrow;
        hoff[b] = ((n / HT_TW) * HT_HWD + n % HT_TW) * HR_PXB + khalf * 16;
    });
    auto read_b = [&](const char *hb, int tap, int s, u32x4 (&bf)[TN]) {
        const int dy = tap / 3, dx = tap - dy * 3;
        const char *q = hb + (dy * HT_HWD + dx) * HR_PXB + s * 32;
        static_for<TN>([&](auto b) { bf[b] = *(const u32x4 *) (q + hoff[b]); });
    };
    static_for<NC>([&](auto cc) {
        constexpr int c = decltype(cc)::value;
        const char *hb = smem + (c & 1) * HT_HBUF;
        u32x4 bcur[TN];
        read_b(hb, 0, 0, bcur);
        static_for<18>([&](auto q) {
            constexpr int u = q / 2, s = q % 2;
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
            if constexpr (q == 0 && c + 1 < NC) load_h(c + 1);
            if constexpr (q == 12 && c + 1 < NC) store_h(c + 1);
        });
        if constexpr (c + 1 < NC) __syncthreads();
    });
    __syncthreads();  // halo reads done: the LDS becomes the activated tile

    // accumulator (a, b, v): channel (wm*TM + a)*32 + (v/4)*8 + (lane/32)*4 + v%4,
    // tile pixel (wn*TN + b)*32 + lane%32
    static_for<TN>([&](auto b) {
        const int col = (wn * TN + b) * 32 + lrow;
        static_for<TM>([&](auto a) {
            static_for<4>([&](auto i) {
                const int row = (wm * TM + a) * 32 + i * 8 + khalf * 4;
                const floatx4 id = *(const floatx4 *) (p.inv_den + (int64_t) fr * C + row);
                const floatx4 bb = *(const floatx4 *) (p.bias + row);
                floatx4 v;
#pragma unroll
                for (int j = 0; j < 4; j++) v[j] = leaky(acc[a][b][i * 4 + j] * id[j] + bb[j]);
                *(floatx4 *) (so + col * L::SOS + row) = v;
            });
        });
    });
    __syncthreads();
    tile_tail<TF, TT, C, BN, NT, HT_TW>(ta, so, prm, wfs, n0, tid, sk);
}

bool modconv_hfrag_tail_ok(bool f16, int IC, int OC, int H, int W) {
    return HFRAG_TAIL && f16 && IC == OC && (OC == 256 || (OC == 128 && HFRAG_TAIL128)) && H % HT_TH == 0 &&
           W % HT_TW == 0;
}

hipError_t launch_modconv_hfrag_tail(const ConvParams &p, const TailArgs &ta, bool trunk_f16, hipStream_t st) {
    if (p.IC != p.OC || (p.OC != 256 && p.OC != 128) || p.M != p.OC || p.H % HT_TH != 0 || p.W % HT_TW != 0)
        return hipErrorInvalidValue;
    const int tiles_x = p.W / HT_TW, tiles_frame = tiles_x * (p.H / HT_TH);
    const int nframes = p.N / (p.H * p.W);
    // the input is read through a buffer resource (32-bit byte extent)
    if ((int64_t) nframes * p.x_bstride * 2 >= ((int64_t) 1 << 31)) return hipErrorInvalidValue;
    const dim3 grid((unsigned) (nframes * tiles_frame));
    auto go = [&](auto c) {
        constexpr int CC = decltype(c)::value;
        if (trunk_f16)
            hipLaunchKernelGGL((modconv3x3_hfrag_tail_kernel<half_t, half_t, CC>), grid, dim3(512), 0, st, p, ta,
                               tiles_x, tiles_frame);
        else
            hipLaunchKernelGGL((modconv3x3_hfrag_tail_kernel<half_t, float, CC>), grid, dim3(512), 0, st, p, ta,
                               tiles_x, tiles_frame);
    };
    if (p.OC == 256) go(std::integral_constant<int, 256>{});
    else go(std::integral_constant<int, 128>{});
    return hipGetLastError();
}

}  // namespace tpmd
