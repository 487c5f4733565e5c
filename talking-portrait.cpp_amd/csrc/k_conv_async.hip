// Modulated 3x3 convolution, f16 operands: the implicit GEMM of k_conv.hip
// (Y[m][n] = sum_k A[m][k] X(k, n), k = tap*IC + ic, the reference's cf
// order; store / split-K epilogues of tpmd_conv.h) with the operand tiles
// moved by the LDS DMA path instead of through registers:
//
//   * every k tile (64-byte rows: 32 channels of one tap) is fetched with
//     global_load_lds_dwordx4 straight into one stage of an S-stage LDS ring,
//     two to three tiles ahead of the one being multiplied;
//   * the operand fragments of each 16-wide k step are read from LDS while
//     the previous step's MFMAs run (two fragment sets in registers);
//   * a DMA writes 16 bytes per lane to consecutive LDS addresses, so rows
//     cannot be padded: LDS slot j of row r holds k chunk j ^ swz(r), with
//     swz(r) = ((r >> 2) ^ (r >> 3)) & 3, the permutation that measured
//     fastest on gfx950 for the 32x32 MFMA operand reads (32 consecutive
//     rows, one 16-byte chunk each): 220 B/clk per CU, against 186 for rows
//     padded to 80 bytes and 63 for unpermuted 64-byte rows;
//   * taps outside the map read 16 bytes from a zero block in device
//     memory, so the zero padding needs no branch in LDS;
//   * one counted vmcnt wait and one barrier per k tile; the barrier carries
//     no memory fence (a fence would drain the tiles in flight).
// 256 x 256 tiles over 8 waves (2 x 4, 128 x 64 per wave), 128 KiB of LDS.
#include "tpmd_conv.h"

namespace tpmd {

// 16 zero bytes: the source of every out-of-map im2col chunk
__device__ __attribute__((aligned(16))) unsigned int g_zero16[4];

#define TPMD_LDS(p) ((__attribute__((address_space(3))) void *) (p))

__device__ __forceinline__ int swz(int row) { return ((row >> 2) ^ (row >> 3)) & 3; }

// s_waitcnt immediate: vmcnt(n), expcnt and lgkmcnt not waited on
constexpr int waitcnt_vm(int n) { return (n & 0xF) | (0x7 << 4) | (0xF << 8) | ((n >> 4) << 14); }

template <int BM, int BN, int S>
struct async_cfg {
    static constexpr int RB = 64;                    // bytes per k-tile row
    static constexpr int STAGE = (BM + BN) * RB;     // bytes per stage
    static constexpr int RING = S * STAGE;
    static constexpr int ORS = BM * 2 + 16;          // staged f16 output row (one pixel), padded
    static constexpr int OUT = BN * ORS;
    static constexpr int LDS = RING > OUT ? RING : OUT;
};

template <typename TO, int BM, int BN, int WM, int WN, int S, int MODE, int EPI>
__global__ __launch_bounds__(WM *WN * 64) void modconv3x3_async_kernel(ConvParams p) {
    typedef half_t TA;
    typedef async_cfg<BM, BN, S> C;
    constexpr int NT = WM * WN * 64, NW = WM * WN;
    constexpr int RB = C::RB, BK = RB / 2;           // 32 halves per row
    constexpr int KS = RB / 32;                      // 16-element MFMA k steps per tile
    constexpr int LPA = BM / 16 / NW, LPB = BN / 16 / NW;  // DMA instructions per wave per tile
    constexpr int LPW = LPA + LPB;
    constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / 32, TN = WTN / 32;
    static_assert(BM % (16 * NW) == 0 && BN % (16 * NW) == 0, "row groups per wave");
    static_assert(TM >= 1 && TN >= 1, "wave tile");
    static_assert(S >= 3, "stages");
    static_assert(KS == 2, "two MFMA k steps per tile");

    __shared__ __attribute__((aligned(16))) char smem[C::LDS];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wid = tid >> 6;
    const int wm = wid / WN, wn = wid % WN;
    const int tile = xcd_remap((int) blockIdx.x, (int) gridDim.x);
    const int mt = tile % p.MT, nt = tile / p.MT;
    const int m0 = mt * BM, n0 = nt * BN;
    const int IC = p.IC, H = p.H, W = p.W;
    const int K = 9 * IC;
    const int HW = H * W;
    const int kpt = IC / BK;

    // this lane's DMA rows: instruction j of a wave moves 16 rows of A
    // (j < LPA) or of B; lane i carries chunk (i % 4) ^ swz(row) of row i / 4
    const int lrow16 = lane >> 2, lpos = lane & 3;
    const TA *Ap = (const TA *) p.A, *Xp = (const TA *) p.X;
    const TA *asrc[LPA];     // A row + chunk; + t * BK per tile
    const TA *bsrc[LPB];     // pixel + chunk; + tap offset + ic0 per tile
    unsigned bmask[LPB];     // bit tap: that tap of the pixel lies inside the map
#pragma unroll
    for (int j = 0; j < LPA; j++) {
        const int row = (wid * LPA + j) * 16 + lrow16;
        asrc[j] = Ap + (int64_t) (m0 + row) * K + (lpos ^ swz(row)) * 8;
    }
#pragma unroll
    for (int j = 0; j < LPB; j++) {
        const int row = BM + (wid * LPB + j) * 16 + lrow16;
        const int n = n0 + row - BM;
        bmask[j] = 0;
        bsrc[j] = Xp;
        if (n < p.N) {
            const int b = n / HW, rem = n - b * HW;
            const int y = rem / W, x = rem - y * W;
            bsrc[j] = Xp + (int64_t) b * p.x_bstride + (int64_t) rem * IC + (lpos ^ swz(row)) * 8;
#pragma unroll
            for (int tap = 0; tap < 9; tap++) {
                const int iy = y + tap / 3 - 1, ix = x + tap % 3 - 1;
                if ((unsigned) iy < (unsigned) H && (unsigned) ix < (unsigned) W) bmask[j] |= 1u << tap;
            }
        }
    }
    const void *zero = (const void *) g_zero16;

    const int nsplit = (int) gridDim.y, split = (int) blockIdx.y;
    const int t_begin = (int) ((int64_t) split * p.T / nsplit);
    const int t_end = (int) ((int64_t) (split + 1) * p.T / nsplit);

    // next tile to issue: k tile t = tap * kpt + ic0 / BK, walked in order
    int q_t = t_begin, q_tap = t_begin / kpt, q_ic0 = (t_begin - q_tap * kpt) * BK;
    auto issue = [&]() {
        const int dy = q_tap / 3 - 1, dx = q_tap - (q_tap / 3) * 3 - 1;
        const int boff = (dy * W + dx) * IC + q_ic0;
        char *stage = smem + ((q_t - t_begin) % S) * C::STAGE;
        static_for<LPA>([&](auto j) {
            __builtin_amdgcn_global_load_lds((const void *) (asrc[j] + q_t * BK),
                                             TPMD_LDS(stage + (wid * LPA + j) * 16 * RB), 16, 0, 0);
        });
        static_for<LPB>([&](auto j) {
            const void *g = (bmask[j] >> q_tap) & 1u ? (const void *) (bsrc[j] + boff) : zero;
            __builtin_amdgcn_global_load_lds(g, TPMD_LDS(stage + (BM + (wid * LPB + j) * 16) * RB), 16, 0,
                                             0);
        });
        q_t++;
        q_ic0 += BK;
        if (q_ic0 == IC) {
            q_ic0 = 0;
            q_tap++;
        }
    };

    floatx16 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; a++)
#pragma unroll
        for (int b = 0; b < TN; b++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[a][b][v] = 0.0f;

    const int lrow = lane & 31;
    const int khalf = lane >> 5;  // which 16-byte half of a 32-byte k step the lane holds
    // operand fragments of k step ks (0 or 1) of the tile in stage st
    auto read_frags = [&](const char *st, int ks, u32x4 (&af)[TM], u32x4 (&bf)[TN]) {
        const int kc = ks * 2 + khalf;
        static_for<TM>([&](auto a) {
            const int row = wm * WTM + a * 32 + lrow;
            af[a] = *(const u32x4 *) (st + row * RB + ((kc ^ swz(row)) << 4));
        });
        static_for<TN>([&](auto b) {
            const int row = BM + wn * WTN + b * 32 + lrow;
            bf[b] = *(const u32x4 *) (st + row * RB + ((kc ^ swz(row)) << 4));
        });
    };
    auto mfmas = [&](const u32x4 (&af)[TM], const u32x4 (&bf)[TN]) {
        static_for<TM>([&](auto a) { static_for<TN>([&](auto b) { mfma_op<TA>::run(af[a], bf[b], acc[a][b]); }); });
    };
    auto stage_of = [&](int t) { return smem + ((t - t_begin) % S) * C::STAGE; };

    // Software pipeline over k steps (two per tile).  Iteration t:
    //   reads of (t, 1)             | MFMAs of (t, 0)
    //   wait: tile t+1 landed; barrier: every wave is done with tile t-1
    //   DMA of tile t+S-1 into the stage of tile t-1
    //   reads of (t+1, 0)           | MFMAs of (t, 1)
    // The fragments of a step are read while the previous step multiplies.
    if (t_begin < t_end) {
        // prologue: tiles t_begin .. t_begin+S-2 in flight, wait for the first
#pragma unroll
        for (int s = 0; s < S - 1; s++)
            if (t_begin + s < t_end) issue();
        if (t_begin + S - 2 < t_end) __builtin_amdgcn_s_waitcnt(waitcnt_vm((S - 2) * LPW));
        else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    }
    u32x4 a0[TM], b0[TN], a1[TM], b1[TN];
    if (t_begin < t_end) read_frags(stage_of(t_begin), 0, a0, b0);
    for (int t = t_begin; t < t_end; t++) {
        read_frags(stage_of(t), 1, a1, b1);
        mfmas(a0, b0);
        if (t + 1 < t_end) {
            // tile t+1 landed (this wave's part): tiles t+2 .. t+S-2 may be in flight
            if (t + S - 2 < t_end) __builtin_amdgcn_s_waitcnt(waitcnt_vm((S - 3) * LPW));
            else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
            __builtin_amdgcn_s_barrier();  // every wave's part landed, tile t-1 consumed
            asm volatile("" ::: "memory");  // no LDS access crosses the barrier
            if (t + S - 1 < t_end) issue();
            read_frags(stage_of(t + 1), 0, a0, b0);
        }
        mfmas(a1, b1);
    }

    // accumulator (a, b, v): row = a*32 + (v/4)*8 + (lane/32)*4 + v%4, col = b*32 + lane%32
    if constexpr (EPI == EPI_STORE && sizeof(TO) == 2) {
        // f16 store epilogue through LDS: the activated tile is staged as
        // [pixel][row] and written back as whole 16-byte chunks, so a wave
        // store covers 1 KB of contiguous output instead of 8-byte pieces
        __syncthreads();  // every wave is done with the ring
        static_for<TN>([&](auto b) {
            const int nl = wn * WTN + b * 32 + lrow;
            const int n = n0 + nl < p.N ? n0 + nl : p.N - 1;
            const int fr = n / HW;
            static_for<TM>([&](auto a) {
                static_for<4>([&](auto i) {
                    const int ml = wm * WTM + a * 32 + i * 8 + (lane >> 5) * 4;
                    const int m = m0 + ml;
                    const int o = MODE == MODE_DENSE ? m : m % p.OC;
                    const floatx4 id = *(const floatx4 *) (p.inv_den + (int64_t) fr * p.OC + o);
                    const floatx4 bb = *(const floatx4 *) (p.bias + o);
                    floatx4 sc = {1.0f, 1.0f, 1.0f, 1.0f};
                    if (p.out_scale) sc = *(const floatx4 *) (p.out_scale + (int64_t) fr * p.OC + o);
                    half4 h;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        float v = leaky(acc[a][b][i * 4 + j] * id[j] + bb[j]);
                        if (p.out_scale) v *= sc[j];
                        h[j] = (half_t) v;
                    }
                    *(half4 *) (smem + nl * C::ORS + ml * 2) = h;
                });
            });
        });
        __syncthreads();
        // chunk c: pixel n0 + c / (BM/8), rows (c % (BM/8)) * 8 .. +8 of the tile
        constexpr int CPR = BM / 8, NCH = BN * CPR, STEP = NT / CPR;
        static_assert(NCH % NT == 0 && NT % CPR == 0, "store pass");
        const int mc = tid % CPR;
        const int m = m0 + mc * 8;
        int cls = 0, o = m;
        if constexpr (MODE == MODE_SUBPIX) {
            cls = m / p.OC;
            o = m - cls * p.OC;
        }
        // pixel of this thread's first chunk, then STEP pixels further per pass
        int nl = tid / CPR;
        int n = n0 + nl;
        int fr = n / HW, rem = n - fr * HW;
        int y = rem / W, x = rem - y * W;
        half_t *Yp = (half_t *) p.Y;
        static_for<NCH / NT>([&](auto j) {
            if (n < p.N) {
                int64_t opix;
                if constexpr (MODE == MODE_DENSE) opix = n;
                else opix = (int64_t) fr * 4 * HW + (int64_t) (2 * y + (cls >> 1)) * (2 * W) + 2 * x + (cls & 1);
                const u32x4 v = *(const u32x4 *) (smem + nl * C::ORS + mc * 16);
                *(u32x4 *) (Yp + opix * p.OC + o) = v;
            }
            nl += STEP;
            n += STEP;
            x += STEP;
            while (x >= W) {
                x -= W;
                if (++y == H) {
                    y = 0;
                    fr++;
                }
            }
        });
    } else {
        static_for<TN>([&](auto b) {
            const int n = n0 + wn * WTN + b * 32 + lrow;
            if (n < p.N) {
                static_for<TM>([&](auto a) {
                    static_for<4>([&](auto i) {
                        const int m = m0 + wm * WTM + a * 32 + i * 8 + (lane >> 5) * 4;
                        const float q[4] = {acc[a][b][i * 4], acc[a][b][i * 4 + 1], acc[a][b][i * 4 + 2],
                                            acc[a][b][i * 4 + 3]};
                        if constexpr (EPI == EPI_STORE) {
                            epi_store_quad<TO, MODE>(p, q, m, n);
                        } else {
                            float *w = p.ws + ((int64_t) split * p.N + n) * p.M + m;
                            *(floatx4 *) w = floatx4{q[0], q[1], q[2], q[3]};
                        }
                    });
                });
            }
        });
    }
}

// ---------------------------------------------------------------------------
// Dense conv + stage tail (OC = BM in {32, 64, 128}, one frame per tile of BN
// pixels): the same DMA ring and fragment pipeline, then the activated tile
// goes to LDS and the two-phase stage tail of tpmd_tail.h runs on it.  The
// (BM + BN) / 16 row groups of a k tile are dealt to the waves round robin;
// a wave that moves fewer groups than another waits on the smaller count,
// which only waits longer.  The tail's skips and the frame's folded ToFlow
// weights are fetched before the k loop.
template <int C, int BN, int S>
struct tail_async_cfg {
    static constexpr int RB = 64;
    static constexpr int STAGE = (C + BN) * RB;
    static constexpr int RING = S * STAGE;
    typedef tile_tail_lds<C, BN> L;
    static constexpr int TAIL = L::WFS0 * 4;                   // so + prm, over the ring
    static constexpr int WFS = RING > TAIL ? RING : TAIL;       // byte offset of wfs
    static constexpr int LDS = WFS + 3 * C * 4;
};

template <typename TF, typename TT, int BM, int BN, int WM, int WN, int S>
__global__ __launch_bounds__(WM *WN * 64) void modconv3x3_tail_async_kernel(ConvParams p, TailArgs ta) {
    typedef half_t TA;
    typedef tail_async_cfg<BM, BN, S> C;
    typedef typename C::L L;
    constexpr int NT = WM * WN * 64, NW = WM * WN;
    constexpr int RB = C::RB, BK = RB / 2, KS = RB / 32;
    constexpr int NG = (BM + BN) / 16;                 // 16-row DMA groups per k tile
    constexpr int SLOTS = (NG + NW - 1) / NW, LPW = NG / NW;
    constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / 32, TN = WTN / 32;
    static_assert(BM % 16 == 0 && BN % 16 == 0 && LPW >= 1, "row groups");
    static_assert(TM >= 1 && TN >= 1, "wave tile");
    static_assert(S >= 3 && KS == 2, "pipeline");

    __shared__ __attribute__((aligned(16))) char smem[C::LDS];
    float *so = (float *) smem, *prm = so + L::PRM0, *wfs = (float *) (smem + C::WFS);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wid / WN, wn = wid % WN;
    const int n0 = xcd_remap((int) blockIdx.x, (int) gridDim.x) * BN;
    const int IC = p.IC, H = p.H, W = p.W;
    const int K = 9 * IC;
    const int HW = H * W;
    const int fr = n0 / HW;
    const int T = p.T;

    // conv-independent tail inputs first
    const tail_skip sk = tile_tail_skips<BN, 0>(ta, n0, tid);
    tile_tail_wfs<BM, NT>(ta, wfs, fr, tid);

    // DMA slots: slot j of wave w moves row group g = j * NW + w
    const int lrow16 = lane >> 2, lpos = lane & 3;
    const TA *Ap = (const TA *) p.A, *Xp = (const TA *) p.X;
    const TA *src[SLOTS];
    unsigned smask[SLOTS];  // taps whose source lies in the map (all for A rows)
#pragma unroll
    for (int j = 0; j < SLOTS; j++) {
        const int row = (j * NW + wid) * 16 + lrow16;
        const int chunk = (lpos ^ swz(row)) * 8;
        src[j] = Xp;
        smask[j] = 0;
        if (row < BM) {
            // (a_img: row group g's k tile t is the 1 KB block (g*T + t) of A)
            src[j] = p.a_img ? Ap + (int64_t) (row >> 4) * T * 512 + lane * 8 : Ap + (int64_t) row * K + chunk;
            smask[j] = 0x1FFu;
        } else if (row < BM + BN) {
            const int rem = n0 - fr * HW + row - BM;
            const int y = rem / W, x = rem - y * W;
            src[j] = Xp + (int64_t) fr * p.x_bstride + (int64_t) rem * IC + chunk;
#pragma unroll
            for (int tap = 0; tap < 9; tap++) {
                const int iy = y + tap / 3 - 1, ix = x + tap % 3 - 1;
                if ((unsigned) iy < (unsigned) H && (unsigned) ix < (unsigned) W) smask[j] |= 1u << tap;
            }
        }
    }
    const void *zero = (const void *) g_zero16;

    int q_t = 0, q_tap = 0, q_ic0 = 0;  // next k tile to issue
    auto issue = [&]() {
        const int dy = q_tap / 3 - 1, dx = q_tap - (q_tap / 3) * 3 - 1;
        const int boff = (dy * W + dx) * IC + q_ic0;
        char *stage = smem + (q_t % S) * C::STAGE;
        static_for<SLOTS>([&](auto j) {
            const int g = j * NW + wid;
            if (g < NG) {
                const int off = g < BM / 16 ? q_t * (p.a_img ? 512 : BK) : boff;
                const void *gp = (smask[j] >> q_tap) & 1u ? (const void *) (src[j] + off) : zero;
                __builtin_amdgcn_global_load_lds(gp, TPMD_LDS(stage + g * 16 * RB), 16, 0, 0);
            }
        });
        q_t++;
        q_ic0 += BK;
        if (q_ic0 == IC) {
            q_ic0 = 0;
            q_tap++;
        }
    };

    floatx16 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; a++)
#pragma unroll
        for (int b = 0; b < TN; b++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[a][b][v] = 0.0f;

    const int lrow = lane & 31;
    const int khalf = lane >> 5;
    auto read_frags = [&](const char *st, int ks, u32x4 (&af)[TM], u32x4 (&bf)[TN]) {
        const int kc = ks * 2 + khalf;
        static_for<TM>([&](auto a) {
            const int row = wm * WTM + a * 32 + lrow;
            af[a] = *(const u32x4 *) (st + row * RB + ((kc ^ swz(row)) << 4));
        });
        static_for<TN>([&](auto b) {
            const int row = BM + wn * WTN + b * 32 + lrow;
            bf[b] = *(const u32x4 *) (st + row * RB + ((kc ^ swz(row)) << 4));
        });
    };
    auto mfmas = [&](const u32x4 (&af)[TM], const u32x4 (&bf)[TN]) {
        static_for<TM>([&](auto a) { static_for<TN>([&](auto b) { mfma_op<TA>::run(af[a], bf[b], acc[a][b]); }); });
    };
    auto stage_of = [&](int t) { return smem + (t % S) * C::STAGE; };

#pragma unroll
    for (int s = 0; s < S - 1; s++)
        if (s < T) issue();
    if (S - 2 < T) __builtin_amdgcn_s_waitcnt(waitcnt_vm((S - 2) * LPW));
    else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    u32x4 a0[TM], b0[TN], a1[TM], b1[TN];
    read_frags(stage_of(0), 0, a0, b0);
    for (int t = 0; t < T; t++) {
        read_frags(stage_of(t), 1, a1, b1);
        mfmas(a0, b0);
        if (t + 1 < T) {
            if (t + S - 2 < T) __builtin_amdgcn_s_waitcnt(waitcnt_vm((S - 3) * LPW));
            else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if (t + S - 1 < T) issue();
            read_frags(stage_of(t + 1), 0, a0, b0);
        }
        mfmas(a1, b1);
    }
    __syncthreads();  // every wave is done with the ring: it becomes the activated tile

    // accumulator (a, b, v): channel a*32 + (v/4)*8 + (lane/32)*4 + v%4, pixel b*32 + lane%32
    static_for<TN>([&](auto b) {
        const int col = wn * WTN + b * 32 + lrow;
        static_for<TM>([&](auto a) {
            static_for<4>([&](auto i) {
                const int row = wm * WTM + a * 32 + i * 8 + (lane >> 5) * 4;
                const floatx4 id = *(const floatx4 *) (p.inv_den + (int64_t) fr * p.OC + row);
                const floatx4 bb = *(const floatx4 *) (p.bias + row);
                floatx4 v;
#pragma unroll
                for (int j = 0; j < 4; j++) v[j] = leaky(acc[a][b][i * 4 + j] * id[j] + bb[j]);
                *(floatx4 *) (so + col * L::SOS + row) = v;
            });
        });
    });
    __syncthreads();
    tile_tail<TF, TT, BM, BN, NT, 0>(ta, so, prm, wfs, n0, tid, sk);
}

// ---------------------------------------------------------------------------
// host side: p.MT, p.T are set here

template <typename TO, int BM, int BN, int WM, int WN, int S>
static hipError_t launch_async_cfg(ConvParams p, int mode, int epi, int nsplit, hipStream_t st) {
    p.MT = p.M / BM;
    p.T = 9 * p.IC * 2 / async_cfg<BM, BN, S>::RB;
    if (nsplit > p.T) return hipErrorInvalidValue;
    dim3 grid((unsigned) (p.MT * ((p.N + BN - 1) / BN)), (unsigned) nsplit);
    dim3 block(WM * WN * 64);
#define TPMD_A(MODE_, EPI_)                                                                            \
    hipLaunchKernelGGL((modconv3x3_async_kernel<TO, BM, BN, WM, WN, S, MODE_, EPI_>), grid, block, 0, st, p)
    if (epi == EPI_PARTIAL) {
        if (mode == MODE_DENSE) TPMD_A(MODE_DENSE, EPI_PARTIAL);
        else TPMD_A(MODE_SUBPIX, EPI_PARTIAL);
    } else {
        if (mode == MODE_DENSE) TPMD_A(MODE_DENSE, EPI_STORE);
        else TPMD_A(MODE_SUBPIX, EPI_STORE);
    }
#undef TPMD_A
    return hipGetLastError();
}

hipError_t launch_modconv_async(const ConvParams &p, int mode, int epi, int nsplit, bool out_f16, int bm,
                                hipStream_t st) {
    if ((bm != 256 && bm != 128) || p.M % bm != 0 || p.IC % 32 != 0) return hipErrorInvalidValue;
    if (bm == 256) {
        if (out_f16) return launch_async_cfg<half_t, 256, 256, 2, 4, 4>(p, mode, epi, nsplit, st);
        return launch_async_cfg<float, 256, 256, 2, 4, 4>(p, mode, epi, nsplit, st);
    }
    if (out_f16) return launch_async_cfg<half_t, 128, 128, 2, 2, 4>(p, mode, epi, nsplit, st);
    return launch_async_cfg<float, 128, 128, 2, 2, 4>(p, mode, epi, nsplit, st);
}

template <typename TT, int BM, int BN, int WM, int WN>
static hipError_t launch_tail_cfg(ConvParams p, const TailArgs &ta, hipStream_t st) {
    constexpr int S = 4;
    p.MT = 1;
    p.T = 9 * p.IC * 2 / tail_async_cfg<BM, BN, S>::RB;
    if (p.M != BM || p.N % BN != 0 || (p.H * p.W) % BN != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL((modconv3x3_tail_async_kernel<half_t, TT, BM, BN, WM, WN, S>), dim3((unsigned) (p.N / BN)),
                       dim3(WM * WN * 64), 0, st, p, ta);
    return hipGetLastError();
}

// measured: the ring pays at OC = 64; at OC = 128 the register-staged
// k_conv.hip kernel (three workgroups per CU) is faster
bool modconv_tail_async_ok(int OC, int r) {
    if (OC == 32) return (r * r) % 256 == 0;
    if (OC == 64 || OC == 256) return (r * r) % 128 == 0;
    return false;
}

hipError_t launch_modconv_tail_async(const ConvParams &p, const TailArgs &ta, bool trunk_f16, hipStream_t st) {
    if (p.IC % 32 != 0) return hipErrorInvalidValue;
    if (p.M == 32) {
        if (trunk_f16) return launch_tail_cfg<half_t, 32, 256, 1, 4>(p, ta, st);
        return launch_tail_cfg<float, 32, 256, 1, 4>(p, ta, st);
    }
    if (p.M == 64) {
        if (trunk_f16) return launch_tail_cfg<half_t, 64, 128, 1, 4>(p, ta, st);
        return launch_tail_cfg<float, 64, 128, 1, 4>(p, ta, st);
    }
    if (p.M == 128) {
        if (trunk_f16) return launch_tail_cfg<half_t, 128, 128, 2, 2>(p, ta, st);
        return launch_tail_cfg<float, 128, 128, 2, 2>(p, ta, st);
    }
    if (p.M == 256) {
        if (trunk_f16) return launch_tail_cfg<half_t, 256, 128, 4, 2>(p, ta, st);
        return launch_tail_cfg<float, 256, 128, 4, 2>(p, ta, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace tpmd