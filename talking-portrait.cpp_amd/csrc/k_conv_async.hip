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
// Eight waves, each 64 rows x BN/WN pixels (WM = BM/64 wave rows, WN = 8/WM
// wave columns): per 16-wide k step a wave reads 2 A fragments and TN B
// fragments for 2*TN MFMAs.  The waves that share A rows read the same lines
// and find them in L1.  The LDS holds only the two halo buffers, so the one
// barrier per 32-channel chunk (9 k tiles) is the halo hand-over; A needs no
// barrier.
//   * A fragments are requested two k tiles ahead into three register sets
//     (k tile t in set t % 3; 9 taps per chunk keep the set of a tap fixed);
//   * the B fragments of the next k step are read from LDS while the
//     current step's MFMAs run;
//   * the halo of chunk c+1 is loaded into registers early in chunk c and
//     written to the other LDS buffer late in it; one barrier ends the chunk.
// Configurations (hfrag_config): 256 rows x 8 x 32 pixels (the r64 - r256
// up-convs); 128 rows x 8 x 32 or x 16 x 16 pixels where 256 rows leave fewer
// than 256 tiles at 16 frames (the r32 convs: a 32 x 32 map, a 16 x 16 up-conv
// input).  The output goes through an LDS stage ([pixel][row], f16 or f32)
// and is written as whole 16-byte chunks of contiguous memory.
constexpr int HR_PXB = 80;              // halo pixel: 64 bytes of channels + 16-byte pad
constexpr int HR_HBUF = 32 * 1024;      // one halo buffer: 32 units of 1 KB per wave-set
// the C = 256 dense conv + tail on the halo conv (else on the im2col ring)
constexpr bool HFRAG_TAIL = true, HFRAG_TAIL128 = true;

template <int BM_, int TH_, int TW_>
struct hfrag_cfg {
    static constexpr int BM = BM_, TH = TH_, TW = TW_, BN = TH * TW;
    static constexpr int NW = 8, NT = NW * 64;
    static constexpr int WM = BM / 64, WN = NW / WM;    // wave grid
    static constexpr int TM = 2, TN = BN / 32 / WN;      // 64 x 32*TN per wave
    static constexpr int HWD = TW + 2, HPX = (TH + 2) * HWD;
    static constexpr int LPH = HR_HBUF / 1024 / NW;      // halo units of 1 KB per wave per chunk
    static_assert(WM * WN == NW && TN * 32 * WN == BN && BN == 256, "wave grid");
    static_assert(HPX * HR_PXB <= HR_HBUF, "halo buffer");
};

template <int MODE, int NC, int BM, int TH, int TW, typename TO>
__global__ __launch_bounds__(512) void modconv3x3_hfrag_kernel(ConvParams p, int tiles_x, int tiles_frame) {
    typedef half_t TA;
    typedef hfrag_cfg<BM, TH, TW> F;
    constexpr int NW = F::NW, NT = F::NT, WN = F::WN, BN = F::BN, TM = F::TM, TN = F::TN;
    constexpr int HWD = F::HWD, HPX = F::HPX, LPH = F::LPH;
    constexpr int ORS = BM * (int) sizeof(TO) + 16, OUT = BN * ORS;  // staged output, one padded row per pixel
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
    // ((tap*KSA + ks)*MB + w) KB; this lane's 16 bytes of it
    const TA *abase = (const TA *) p.A + ((int64_t) (m0 / 32 + wm * TM)) * 512 + lane * 8;
    auto afrag = [&](int tap, int ks, int a) -> u32x4 {
        return *(const u32x4 *) (abase + ((int64_t) (tap * KSA + ks) * MB + a) * 512);
    };
    u32x4 af[3][TM][2];
    auto load_a = [&](int c, int tap, u32x4 (&dst)[TM][2]) {
        static_for<2>([&](auto s) { static_for<TM>([&](auto a) { dst[a][s] = afrag(tap, 2 * c + s, a); }); });
    };

    // halo unit u = (wid*LPH + h)*64 + lane of a halo buffer: halo pixel u / 5,
    // channel chunk u % 5 (4: the pad); units past the halo, pads and pixels
    // outside the map read zeros
    const TA *Xf = (const TA *) p.X + (int64_t) fr * p.x_bstride;
    const TA *hsrc[LPH];
    bool hok[LPH];
#pragma unroll
    for (int h = 0; h < LPH; h++) {
        const int u = (wid * LPH + h) * 64 + lane;
        const int hp = u / 5, q = u - hp * 5;
        const int hy = hp / HWD, hx = hp - hy * HWD;
        const int iy = y0 - 1 + hy, ix = x0 - 1 + hx;
        hok[h] = q < 4 && hp < HPX && (unsigned) iy < (unsigned) H && (unsigned) ix < (unsigned) W;
        hsrc[h] = hok[h] ? Xf + ((int64_t) iy * W + ix) * IC + q * 8 : Xf;
    }
    // the halo goes through registers rather than the LDS DMA path: the
    // compiler then counts every load exactly, while after an LDS DMA it
    // waits for all loads in flight before the next MFMA
    const u32x4 *zero = (const u32x4 *) g_zero16;
    u32x4 hreg[LPH];
    auto load_h = [&](int c) {
        static_for<LPH>([&](auto h) { hreg[h] = *(hok[h] ? (const u32x4 *) (hsrc[h] + c * 32) : zero); });
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
    // rows) and written back as whole 16-byte chunks of contiguous output
    __syncthreads();
    static_for<TN>([&](auto b) {
        const int nl = (wn * TN + b) * 32 + lrow;
        static_for<TM>([&](auto a) {
            static_for<4>([&](auto i) {
                const int ml = (wm * TM + a) * 32 + i * 8 + khalf * 4;
                const int m = m0 + ml;
                const int o = MODE == MODE_DENSE ? m : m % p.OC;
                const floatx4 id = *(const floatx4 *) (p.inv_den + (int64_t) fr * p.OC + o);
                const floatx4 bb = *(const floatx4 *) (p.bias + o);
                floatx4 sc = {1.0f, 1.0f, 1.0f, 1.0f};
                if (p.out_scale) sc = *(const floatx4 *) (p.out_scale + (int64_t) fr * p.OC + o);
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
    __syncthreads();
    constexpr int EPC = 16 / (int) sizeof(TO);           // output elements per 16-byte chunk
    constexpr int CPR = BM / EPC, NCH = BN * CPR, STEP = NT / CPR;
    static_assert(NCH % NT == 0 && NT % CPR == 0, "store pass");
    const int mc = tid % CPR;
    const int m = m0 + mc * EPC;
    int cls = 0, o = m;
    if constexpr (MODE == MODE_SUBPIX) {
        cls = m / p.OC;
        o = m - cls * p.OC;
    }
    const int64_t HW = (int64_t) H * W;
    TO *Yp = (TO *) p.Y;
    static_for<NCH / NT>([&](auto j) {
        const int nl = tid / CPR + j * STEP;
        const int y = y0 + nl / TW, x = x0 + nl % TW;
        int64_t opix;
        if constexpr (MODE == MODE_DENSE) opix = fr * HW + (int64_t) y * W + x;
        else opix = fr * 4 * HW + (int64_t) (2 * y + (cls >> 1)) * (2 * W) + 2 * x + (cls & 1);
        const u32x4 v = *(const u32x4 *) (smem + nl * ORS + mc * 16);
        *(u32x4 *) (Yp + opix * p.OC + o) = v;
    });
}

// ---------------------------------------------------------------------------
// Dense conv + stage tail for C = 256 (the r64 stage): the halo conv above
// (A fragments from L2, each 32-channel chunk's input halo in LDS, chunk-major
// k) on 4 x 32 pixel blocks, 256 rows = every channel of the block, eight
// waves of 64 rows x 64 pixels; the activated 256 x 128 tile then goes to LDS
// as f32 and the two-phase tile tail runs on it.  The tail's skips, the
// ToFlow weights and the first chunk's halo are requested together.
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
    const TA *abase = (const TA *) p.A + (wm * TM) * 512 + lane * 8;
    auto afrag = [&](int tap, int ks, int a) -> u32x4 {
        return *(const u32x4 *) (abase + ((tap * KSA + ks) * MB + a) * 512);
    };
    u32x4 af[3][TM][2];
    auto load_a = [&](int c, int tap, u32x4 (&dst)[TM][2]) {
        static_for<2>([&](auto s) { static_for<TM>([&](auto a) { dst[a][s] = afrag(tap, 2 * c + s, a); }); });
    };

    // halo unit u = (wid*LPH + h)*64 + lane: halo pixel u / 5, chunk u % 5 (4: the pad)
    const TA *Xf = (const TA *) p.X + (int64_t) fr * p.x_bstride;
    const TA *hsrc[LPH];
    bool hok[LPH];
#pragma unroll
    for (int h = 0; h < LPH; h++) {
        const int u = (wid * LPH + h) * 64 + lane;
        const int hp = u / 5, q = u - hp * 5;
        const int hy = hp / HT_HWD, hx = hp - hy * HT_HWD;
        const int iy = y0 - 1 + hy, ix = x0 - 1 + hx;
        hok[h] = q < 4 && hp < HT_HPX && (unsigned) iy < (unsigned) H && (unsigned) ix < (unsigned) W;
        hsrc[h] = hok[h] ? Xf + ((int64_t) iy * W + ix) * C + q * 8 : Xf;
    }
    const u32x4 *zero = (const u32x4 *) g_zero16;
    u32x4 hreg[LPH];
    auto load_h = [&](int c) {
        static_for<LPH>([&](auto h) { hreg[h] = *(hok[h] ? (const u32x4 *) (hsrc[h] + c * 32) : zero); });
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

// the halo kernel configuration of a conv shape: 1 = 256 rows x 8 x 32
// pixels, 2 = 128 rows x 8 x 32, 3 = 128 rows x 16 x 16, 0 = none.  f16
// operands, IC a power of two from 32 to 512, and the first configuration
// (in that order) that gives every CU a tile at 16 frames; a function of the
// per-frame shape only
static int hfrag_config(bool f16, int mode, int IC, int H, int W, int M) {
    if (!f16 || (IC != 32 && IC != 64 && IC != 128 && IC != 256 && IC != 512)) return 0;
    auto tiles = [&](int bm, int th, int tw) -> int64_t {
        if (M % bm != 0 || H % th != 0 || W % tw != 0) return 0;
        return (int64_t) (M / bm) * 16 * (H / th) * (W / tw);
    };
    if (tiles(256, 8, 32) >= 256) return 1;
    if (tiles(128, 8, 32) >= 256) return 2;
    if (tiles(128, 16, 16) >= 256) return 3;
    return 0;
}

// f16 output, or f32 output of a dense conv on 128-row tiles
bool modconv_hfrag_ok(bool f16, bool out_f16, int mode, int IC, int OC, int H, int W) {
    const int M = mode == MODE_DENSE ? OC : 4 * OC;
    const int cfg = hfrag_config(f16, mode, IC, H, W, M);
    return cfg != 0 && (out_f16 || (mode == MODE_DENSE && cfg != 1));
}

hipError_t launch_modconv_hfrag(ConvParams p, int mode, bool out_f16, hipStream_t st) {
    const int cfg = hfrag_config(true, mode, p.IC, p.H, p.W, p.M);
    if (cfg == 0 || (!out_f16 && (mode != MODE_DENSE || cfg == 1))) return hipErrorInvalidValue;
    const int BM = cfg == 1 ? 256 : 128, TH = cfg == 3 ? 16 : 8, TW = cfg == 3 ? 16 : 32;
    const int64_t HW = (int64_t) p.H * p.W;
    if (p.N % HW != 0) return hipErrorInvalidValue;
    p.MT = p.M / BM;
    p.T = 9 * p.IC / 32;
    const int tiles_x = p.W / TW, tiles_frame = tiles_x * (p.H / TH);
    const dim3 grid((unsigned) ((int64_t) p.MT * (p.N / HW) * tiles_frame));
    auto go = [&](auto nc, auto bm, auto th, auto tw) {
        constexpr int NC = decltype(nc)::value, B = decltype(bm)::value;
        constexpr int T_H = decltype(th)::value, T_W = decltype(tw)::value;
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
    auto by_cfg = [&](auto nc) {
        if (cfg == 1)
            return go(nc, std::integral_constant<int, 256>{}, std::integral_constant<int, 8>{},
                      std::integral_constant<int, 32>{});
        if (cfg == 2)
            return go(nc, std::integral_constant<int, 128>{}, std::integral_constant<int, 8>{},
                      std::integral_constant<int, 32>{});
        return go(nc, std::integral_constant<int, 128>{}, std::integral_constant<int, 16>{},
                  std::integral_constant<int, 16>{});
    };
    switch (p.IC) {
        case 32: return by_cfg(std::integral_constant<int, 1>{});
        case 64: return by_cfg(std::integral_constant<int, 2>{});
        case 128: return by_cfg(std::integral_constant<int, 4>{});
        case 256: return by_cfg(std::integral_constant<int, 8>{});
        case 512: return by_cfg(std::integral_constant<int, 16>{});
        default: return hipErrorInvalidValue;
    }
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
