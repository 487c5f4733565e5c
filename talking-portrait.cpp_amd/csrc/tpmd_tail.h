// Per-pixel stage tail of the motion decoder, shared by the standalone tail
// kernel (k_tail.hip) and the dense conv's fused epilogue (k_conv.hip).
//
// Everything that follows the dense modulated conv of stage j, for one pixel
// (src/motion_dec.cpp:1077-1108 channel-last stages; :1012-1064 spatial
// stages, same arithmetic):
//
//   fl   = (Wf * s_f) . out + b_f  [+ upfirdn2x(fl_prev)]        ToFlow + skip
//   gx   = tanh(fl0) + lin[x],  gy = tanh(fl1) + lin[y],  m = sigmoid(fl2)
//   smp  = grid_sample(feat_j, gx, gy)   bilinear, zeros, align_corners=False
//   warp = smp * m ;  trunk = warp + out * (1 - m)
//   rgb  = leaky(Wr . warp + b1) + b_rgb  [+ upfirdn2x(rgb_prev)]  ToRGB + skip
//
// G lanes own one pixel, 8 channels each (C = 8*G); the two 3-row dot
// products finish with a butterfly over the G lanes, so every lane holds the
// pixel's flow and mask and gathers its own 8 channels of the 4 taps (the
// feature map is channel-last: each tap is one contiguous run read by the G
// lanes together).  trunk is stored pre-multiplied by the next up-conv's
// style (that conv's operand); the last stage writes only rgb, straight into
// the CHW output frame.
#pragma once

#include "tpmd_device.h"
#include "tpmd_launch.h"

namespace tpmd {

template <typename T> struct load8;
template <> struct load8<float> {
    __device__ __forceinline__ static void run(const float *p, float v[8]) {
        const floatx4 a = *(const floatx4 *) p, b = *(const floatx4 *) (p + 4);
        v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
        v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
    }
};
template <> struct load8<half_t> {
    __device__ __forceinline__ static void run(const half_t *p, float v[8]) {
        const half8 a = *(const half8 *) p;
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = (float) a[e];
    }
};
template <typename T> __device__ __forceinline__ void store8(T *p, const float v[8]);
template <> __device__ __forceinline__ void store8<float>(float *p, const float v[8]) {
    *(floatx4 *) p = floatx4{v[0], v[1], v[2], v[3]};
    *(floatx4 *) (p + 4) = floatx4{v[4], v[5], v[6], v[7]};
}
template <> __device__ __forceinline__ void store8<half_t>(half_t *p, const float v[8]) {
    half8 h;
#pragma unroll
    for (int e = 0; e < 8; e++) h[e] = (half_t) v[e];
    *(half8 *) p = h;
}

// per-lane slices of the ToFlow / ToRGB weights (channels c0 .. c0+7)
struct TailWeights {
    float wf[3][8], wr[3][8];
};

// (FGR: the ToRGB sum comes from TailArgs::featg, the ToRGB slice is not needed)
template <bool FGR>
__device__ __forceinline__ void load_tail_weights(const TailArgs &a, int c0, TailWeights &w) {
#pragma unroll
    for (int k = 0; k < 3; k++) {
        load8<float>::run(a.wflow + k * a.C + c0, w.wf[k]);
        if constexpr (!FGR) load8<float>::run(a.wrgb + k * a.C + c0, w.wr[k]);
    }
}

}  // namespace tpmd

namespace tpmd {

// ---------------------------------------------------------------------------
// Stage tail of a tile of BN consecutive pixels of ONE frame whose dense-conv
// output (after bias + leaky) sits in LDS, run by the NT threads of a
// workgroup in two phases (same arithmetic as tail_pixel):
//   phase 1, one thread per pixel: ToFlow dot (the style-folded weights
//     Wf * s_f of the tile's frame are staged in LDS), flow skip, flow head,
//     bilinear tap geometry; the per-pixel results go to LDS;
//   phase 2, G = C/8 lanes per pixel: gather of the feature taps, warp,
//     trunk (* next style, stored).
// The ToRGB sum is Wr . (m * sum_k w_k feat_k) = m * sum_k w_k (Wr . feat_k)
// from the per-feature-pixel Wr . feat (TailArgs::featg), taken in phase 1:
// 3 values per tap instead of C channels and a butterfly over the G lanes,
// the ToRGB dot of phase 2 (measured at r256, 16 frames: 174 -> 167 us);
// phase 2 then runs only for the trunk or the warp tap.
// Per-pixel scalar work runs once instead of on each of the G lanes.  The
// flow / rgb skips do not depend on the conv output: tile_tail_skips loads
// them before the conv runs, so their latency hides behind it.
template <int C, int BN>
struct tile_tail_lds {
    static constexpr int SOS = C + 4;                 // out row stride (floats)
    static constexpr int PRM = 8;                     // per-pixel record (floats)
    static constexpr int OUT = BN * SOS;              // offsets in floats
    static constexpr int PRM0 = OUT;
    static constexpr int WFS0 = PRM0 + BN * PRM;
    static constexpr int FLOATS = WFS0 + 3 * C;
};

// The tile's pixels: p = 0..BN-1 -> frame pixel pix0 + p (TWC = 0: a run of
// consecutive pixels starting at batch pixel n0) or pix0 + (p / TWC) * r +
// p % TWC (TWC > 0: a TWC-wide block of rows whose top-left pixel is n0).  Every
// pixel of the tile exists (the caller's tiling guarantees it).
template <int TWC>
__device__ __forceinline__ int tile_pix(int pix0, int r, int p) {
    if constexpr (TWC > 0) return pix0 + (p / TWC) * r + p % TWC;
    return pix0 + p;
}

// upfirdn2x skips of the flow and rgb heads and the identity-grid
// coordinates of tile pixel tid (tid < BN)
struct tail_skip {
    float fl[3], rgb[3];
    float lx, ly;
};

// ... with more loads (`issue`) requested between the skip taps and their sums
template <int BN, int TWC, typename F>
__device__ __forceinline__ tail_skip tile_tail_skips_then(const TailArgs &a, int n0, int tid, F &&issue);

template <int BN, int TWC>
__device__ __forceinline__ tail_skip tile_tail_skips(const TailArgs &a, int n0, int tid) {
    return tile_tail_skips_then<BN, TWC>(a, n0, tid, []() {});
}

template <int BN, int TWC, typename F>
__device__ __forceinline__ tail_skip tile_tail_skips_then(const TailArgs &a, int n0, int tid, F &&issue) {
#pragma clang fp contract(off)
    tail_skip sk;
#pragma unroll
    for (int k = 0; k < 3; k++) sk.fl[k] = sk.rgb[k] = 0.0f;
    sk.lx = sk.ly = 0.0f;
    if (tid < BN) {
        const int r = a.r, rh = r >> 1, RR = r * r;
        const int fr = n0 / RR;
        const int pix0 = n0 - fr * RR;
        int y, x;
        if constexpr (TWC > 0) {
            // the block's first row and column are the same for every lane
            // (scalar division); the lane's offsets in the block follow
            const int py0 = pix0 / r;
            y = py0 + tid / TWC;
            x = pix0 - py0 * r + tid % TWC;
        } else {
            y = (pix0 + tid) / r;
            x = pix0 + tid - y * r;
        }
        sk.lx = a.lin[x];
        sk.ly = a.lin[y];
        // every tap of the six planes is requested before any sum is formed
        // (through buffer resources over the skip arrays: 32-bit offsets)
        const int64_t sbytes = (int64_t) a.nframes * 3 * rh * rh * 4;
        const __amdgpu_buffer_rsrc_t frs = buffer_rsrc(a.flow_prev, sbytes), rrs = buffer_rsrc(a.rgb_prev, sbytes);
        // the kernel taps once per kernel, shared by its three planes
        upfirdn_k kf{}, kr{};
        if (a.flow_prev) kf = upfirdn2x_weights(a.fup, x, y);
        if (a.rgb_prev) kr = upfirdn2x_weights(a.rup, x, y);
        upfirdn_taps tf[3], tr[3];
#pragma unroll
        for (int k = 0; k < 3; k++) {
            const unsigned plane0 = (unsigned) ((fr * 3 + k) * rh * rh);
            if (a.flow_prev) upfirdn2x_load(frs, plane0, rh, rh, kf, x, y, tf[k]);
            if (a.rgb_prev) upfirdn2x_load(rrs, plane0, rh, rh, kr, x, y, tr[k]);
        }
        issue();
#pragma unroll
        for (int k = 0; k < 3; k++) {
            if (a.flow_prev) sk.fl[k] = upfirdn2x_sum(tf[k]);
            if (a.rgb_prev) sk.rgb[k] = upfirdn2x_sum(tr[k]);
        }
    } else {
        issue();
    }
    return sk;
}

// The skips of a whole TH x TW output block (TH, TW even; top-left y0, x0
// even) staged in LDS: the 2x upfirdn taps of its pixels lie in rows
// y0/2 - 1 .. y0/2 + TH/2 and columns x0/2 - 1 .. x0/2 + TW/2 of the
// half-resolution planes, SKH x SKW values per plane (source indices clamped
// into the plane, as upfirdn2x_load clamps them; a tap outside the plane is
// skipped by the sum all the same).  The workgroup requests the six planes'
// windows together, one value per thread and step (instead of 24 single
// loads per pixel, most of them shared with the neighbours), stores them
// with the halo, and each pixel reads its taps back when it needs them:
// the same values summed in the same order as tile_tail_skips.
template <int TH, int TW, int NT>
struct skip_lds {
    static constexpr int SKH = TH / 2 + 2, SKW = TW / 2 + 2, PL = SKH * SKW;
    static constexpr int FLOATS = 6 * PL;            // flow planes 0-2, rgb planes 3-5
    static constexpr int NV = (FLOATS + NT - 1) / NT;  // values per thread
};
template <int TH, int TW, int NT>
__device__ __forceinline__ void skip_window_load(const TailArgs &a, int fr, int y0, int x0, int tid,
                                                 float (&v)[skip_lds<TH, TW, NT>::NV]) {
    typedef skip_lds<TH, TW, NT> S;
    const int rh = a.r >> 1;
    const int64_t sbytes = (int64_t) a.nframes * 3 * rh * rh * 4;
    const __amdgpu_buffer_rsrc_t frs = buffer_rsrc(a.flow_prev, sbytes), rrs = buffer_rsrc(a.rgb_prev, sbytes);
#pragma unroll
    for (int j = 0; j < S::NV; j++) {
        const int i = tid + j * NT;
        const int pl = i / S::PL, rem = i - pl * S::PL;
        const int wr = rem / S::SKW, wc = rem - wr * S::SKW;
        int sy = (y0 >> 1) - 1 + wr, sx = (x0 >> 1) - 1 + wc;
        sy = sy < 0 ? 0 : (sy >= rh ? rh - 1 : sy);
        sx = sx < 0 ? 0 : (sx >= rh ? rh - 1 : sx);
        const int k = pl < 3 ? pl : pl - 3;
        const unsigned off = (unsigned) (((fr * 3 + k) * rh + sy) * rh + sx) * 4u;
        // past the extent (zeros) for the steps past the six windows and for absent skips
        const bool rgb = pl >= 3;
        const bool have = i < S::FLOATS && (rgb ? a.rgb_prev != nullptr : a.flow_prev != nullptr);
        const unsigned o = have ? off : 0x80000000u;
        v[j] = rgb ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rrs, o, 0, 0))
                   : __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(frs, o, 0, 0));
    }
}
template <int TH, int TW, int NT>
__device__ __forceinline__ void skip_window_store(float *lds, int tid, const float (&v)[skip_lds<TH, TW, NT>::NV]) {
    typedef skip_lds<TH, TW, NT> S;
#pragma unroll
    for (int j = 0; j < S::NV; j++) {
        const int i = tid + j * NT;
        if (i < S::FLOATS) lds[i] = v[j];
    }
}
// the skips of output pixel (x, y) of the block from the staged windows;
// lx, ly: its identity-grid coordinates lin[x], lin[y] (loaded earlier)
template <int TH, int TW, int NT>
__device__ __forceinline__ tail_skip skip_from_window(const TailArgs &a, const float *lds, int y0, int x0, int x,
                                                      int y, float lx, float ly) {
#pragma clang fp contract(off)
    typedef skip_lds<TH, TW, NT> S;
    tail_skip sk;
#pragma unroll
    for (int k = 0; k < 3; k++) sk.fl[k] = sk.rgb[k] = 0.0f;
    sk.lx = lx;
    sk.ly = ly;
    const int rh = a.r >> 1;
    const int i0 = x & 1, j0 = y & 1;
    const int sx0 = (x + i0 - 2) >> 1, sy0 = (y + j0 - 2) >> 1;
    const int w0 = (sy0 - ((y0 >> 1) - 1)) * S::SKW + sx0 - ((x0 >> 1) - 1);  // window index of tap (0, 0)
    bool in[4];
#pragma unroll
    for (int jj = 0; jj < 2; jj++)
#pragma unroll
        for (int ii = 0; ii < 2; ii++)
            in[2 * jj + ii] = (unsigned) (sy0 + jj) < (unsigned) rh && (unsigned) (sx0 + ii) < (unsigned) rh;
    auto plane = [&](int pl, const upfirdn_k &kw) {
        upfirdn_taps t;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            t.v[q] = lds[pl * S::PL + w0 + (q >> 1) * S::SKW + (q & 1)];
            t.k[q] = kw.k[q];
            t.in[q] = in[q];
        }
        return upfirdn2x_sum(t);
    };
    if (a.flow_prev) {
        const upfirdn_k kf = upfirdn2x_weights(a.fup, x, y);
#pragma unroll
        for (int k = 0; k < 3; k++) sk.fl[k] = plane(k, kf);
    }
    if (a.rgb_prev) {
        const upfirdn_k kr = upfirdn2x_weights(a.rup, x, y);
#pragma unroll
        for (int k = 0; k < 3; k++) sk.rgb[k] = plane(3 + k, kr);
    }
    return sk;
}

// park tile pixel tid's skips in its LDS record (prm, [BN][8] floats) while
// the conv runs, and take them back before phase 1 overwrites the record
template <int BN>
__device__ __forceinline__ void tile_tail_stash(float *prm, int tid, const tail_skip &sk) {
    if (tid < BN) {
        *(floatx4 *) (prm + tid * 8) = floatx4{sk.fl[0], sk.fl[1], sk.fl[2], sk.lx};
        *(floatx4 *) (prm + tid * 8 + 4) = floatx4{sk.ly, sk.rgb[0], sk.rgb[1], sk.rgb[2]};
    }
}
template <int BN>
__device__ __forceinline__ tail_skip tile_tail_unstash(const float *prm, int tid) {
    tail_skip sk{};
    if (tid < BN) {
        const floatx4 a = *(const floatx4 *) (prm + tid * 8), b = *(const floatx4 *) (prm + tid * 8 + 4);
        sk.fl[0] = a[0]; sk.fl[1] = a[1]; sk.fl[2] = a[2]; sk.lx = a[3];
        sk.ly = b[0]; sk.rgb[0] = b[1]; sk.rgb[1] = b[2]; sk.rgb[2] = b[3];
    }
    return sk;
}

// folded ToFlow weights of frame fr (gemm_weight: W * s rounded to f32),
// in two halves so that the loads can join an earlier memory round trip
template <int C, int NT>
struct tail_wfs_regs {
    static constexpr int N = (3 * C + NT - 1) / NT;
    float w[N], s[N];
};
template <int C, int NT>
__device__ __forceinline__ tail_wfs_regs<C, NT> tile_tail_wfs_load(const TailArgs &a, int fr, int tid) {
    tail_wfs_regs<C, NT> r;
#pragma unroll
    for (int j = 0; j < r.N; j++) {
        const int i = tid + j * NT;
        r.w[j] = i < 3 * C ? a.wflow[i] : 0.0f;
        r.s[j] = i < 3 * C ? a.sflow[(int64_t) fr * C + i % C] : 0.0f;
    }
    return r;
}
template <int C, int NT>
__device__ __forceinline__ void tile_tail_wfs_store(float *wfs, int tid, const tail_wfs_regs<C, NT> &r) {
#pragma unroll
    for (int j = 0; j < r.N; j++) {
        const int i = tid + j * NT;
        if (i < 3 * C) wfs[i] = r.w[j] * r.s[j];
    }
}
template <int C, int NT>
__device__ __forceinline__ void tile_tail_wfs(const TailArgs &a, float *wfs, int fr, int tid) {
    tile_tail_wfs_store<C, NT>(wfs, tid, tile_tail_wfs_load<C, NT>(a, fr, tid));
}

// 8 channels of one feature tap, kept in the stored type until used
template <typename T> struct feat8;
template <> struct feat8<half_t> {
    half8 h;
    __device__ __forceinline__ void load(const half_t *p) { h = *(const half8 *) p; }
    // at byte offset off of a buffer resource over the feature map
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, unsigned off) {
        h = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    }
    __device__ __forceinline__ float operator[](int e) const { return (float) h[e]; }
};
template <> struct feat8<float> {
    floatx4 lo, hi;
    __device__ __forceinline__ void load(const float *p) {
        lo = *(const floatx4 *) p;
        hi = *(const floatx4 *) (p + 4);
    }
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, unsigned off) {
        lo = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
        hi = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16u, 0, 0));
    }
    __device__ __forceinline__ float operator[](int e) const { return e < 4 ? lo[e] : hi[e - 4]; }
};

// Runs after the activated tile `so` ([BN][SOS] f32) and `wfs` are written
// and a barrier has made them visible; prm is [BN][PRM] scratch.
// Phase 1 of one pixel, part 1: the ToFlow bias and skip, the flow output,
// and the warp's sampling taps and mask (fl: the ToFlow dot, bias not added)
__device__ __forceinline__ void tail_flow_head(const TailArgs &a, float fl[3], int fr, int pix,
                                               const tail_skip &sk, taps4 &t, float &m) {
#pragma clang fp contract(off)
    const int r = a.r, RR = r * r;
#pragma unroll
    for (int k = 0; k < 3; k++) {
        fl[k] = fl[k] + ld_uniform(a.fbias, k);
        if (a.flow_prev) fl[k] = fl[k] + sk.fl[k];
    }
    if (a.flow_cur) {
#pragma unroll
        for (int k = 0; k < 3; k++) a.flow_cur[((int64_t) fr * 3 + k) * RR + pix] = fl[k];
    }
    const float gx = tanhf(fl[0]) + sk.lx;
    const float gy = tanhf(fl[1]) + sk.ly;
    m = 1.0f / (1.0f + expf(-fl[2]));
    t = gather_geometry(gx, gy, r, r);
}

// the ToRGB sum from featg: Wr . (m * sum_k w_k feat_k) = m * sum_k w_k
// (Wr . feat_k), with Wr . feat stored per feature pixel; a tap outside the
// map reads the zero pad after it.  Load the four taps' values ...
__device__ __forceinline__ void tail_featg_load(const TailArgs &a, const taps4 &t, floatx4 gv[4]) {
    const int r = a.r, RR = r * r;
    // through a buffer resource over featg and its pad: 32-bit offsets
    const __amdgpu_buffer_rsrc_t grs = buffer_rsrc(a.featg, (int64_t) RR * 16 + TAIL_FEATG_PAD);
    const unsigned gpad = (unsigned) RR * 16u;
    const bool inx[2] = {(unsigned) t.x0 < (unsigned) r, (unsigned) t.x0 + 1u < (unsigned) r};
    const bool iny[2] = {(unsigned) t.y0 < (unsigned) r, (unsigned) t.y0 + 1u < (unsigned) r};
    const unsigned base = (unsigned) (t.y0 * r + t.x0) * 16u;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const unsigned off = base + (unsigned) (((k >> 1) * r + (k & 1)) * 16);
        gv[k] = __builtin_bit_cast(
            floatx4, __builtin_amdgcn_raw_buffer_load_b128(grs, inx[k & 1] && iny[k >> 1] ? off : gpad, 0, 0));
    }
}
// ... then form and store the pixel's rgb
__device__ __forceinline__ void tail_featg_finish(const TailArgs &a, const taps4 &t, float m, int fr, int pix,
                                                  const float skr[3], const floatx4 gv[4]) {
#pragma clang fp contract(off)
    const int RR = a.r * a.r;
    float rgb[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float wk = tap_weight(t, k);
#pragma unroll
        for (int q = 0; q < 3; q++) rgb[q] = __builtin_fmaf(wk, gv[k][q], rgb[q]);
    }
    float *rgbf = a.rgb_cur + (int64_t) fr * 3 * RR;
#pragma unroll
    for (int q = 0; q < 3; q++) {
        float v = leaky(rgb[q] * m + ld_uniform(a.rlb, q));
        v = v + ld_uniform(a.rbias, q);
        if (a.rgb_prev) v = v + skr[q];
        rgbf[(unsigned) (q * RR + pix)] = v;
    }
}
__device__ __forceinline__ void tail_featg_rgb(const TailArgs &a, const taps4 &t, float m, int fr, int pix,
                                               const tail_skip &sk) {
    floatx4 gv[4];
    tail_featg_load(a, t, gv);
    tail_featg_finish(a, t, m, fr, pix, sk.rgb, gv);
}

// s_waitcnt immediate: lgkmcnt(0), vmcnt and expcnt not waited on
constexpr int tail_waitcnt_lgkm0 = 0xF | (0x7 << 4) | (0x3 << 14);
// the fused tile tail's phase 2: pixels whose feature taps are requested
// together (f16 / f32 features), and whether the featg values of phase 1's
// pixels stay in flight through phase 2
constexpr int TAIL_NB16 = 4, TAIL_NB32 = 2;
constexpr bool TAIL_FEATG_OVERLAP = false;

// Runs after the activated tile `so` ([BN][SOS] f32) and `wfs` are written
// and a barrier has made them visible; prm is [BN][PRM] scratch.  a.featg
// must be set: the ToRGB sum is taken from it in phase 1.
template <typename TF, typename TT, int C, int BN, int NT, int TWC>
__device__ __forceinline__ void tile_tail(const TailArgs &a, const float *so, float *prm, const float *wfs,
                                          int n0, int tid, const tail_skip &sk) {
#pragma clang fp contract(off)
    typedef tile_tail_lds<C, BN> L;
    constexpr int G = C / 8;
    constexpr int PPW = 64 / G;
    constexpr int PPB = (NT / 64) * PPW;
    static_assert(BN % PPB == 0, "tail pass");
    const int r = a.r;
    const int RR = r * r;
    const int fr = n0 / RR;                          // the tile lies in one frame
    const int pix0 = n0 - fr * RR;
    // phase 2 gathers the warp channel by channel, for the trunk or the warp tap
    const bool p2 = a.trunk || a.warp_tap;

    // ---- phase 1: one thread per pixel
    taps4 gt{};
    float gm = 0.0f;
    floatx4 gv[4];
    if (tid < BN) {
        const int p = tid;
        const int pix = tile_pix<TWC>(pix0, r, p);
        // ToFlow dot as two chains, over channels c with c % 8 < 4 and over
        // the rest, each in channel order, then added: the order in which
        // the MFMA accumulator layout leaves the channels split over a
        // lane pair, so a kernel finishing pixels in registers gets the
        // same bits as this one
        float fl[3], fh[3];
#pragma unroll
        for (int k = 0; k < 3; k++) fl[k] = fh[k] = 0.0f;
#pragma unroll
        for (int c = 0; c < C; c += 8) {
            const floatx4 o = *(const floatx4 *) (so + p * L::SOS + c);
            const floatx4 q = *(const floatx4 *) (so + p * L::SOS + c + 4);
#pragma unroll
            for (int k = 0; k < 3; k++) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    fl[k] = __builtin_fmaf(wfs[k * C + c + j], o[j], fl[k]);
                    fh[k] = __builtin_fmaf(wfs[k * C + c + 4 + j], q[j], fh[k]);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < 3; k++) fl[k] = fl[k] + fh[k];
        taps4 t;
        float m;
        tail_flow_head(a, fl, fr, pix, sk, t, m);
        if (p2) *(floatx4 *) (prm + p * L::PRM) = floatx4{__int_as_float(t.x0), __int_as_float(t.y0), t.wx, t.wy};
        if (p2) prm[p * L::PRM + 4] = m;
        if (TAIL_FEATG_OVERLAP && p2) {
            tail_featg_load(a, t, gv);
            gt = t;
            gm = m;
        } else {
            tail_featg_rgb(a, t, m, fr, pix, sk);
        }
    }
    if (!p2) return;  // (uniform) nothing is left for phase 2
    if constexpr (TAIL_FEATG_OVERLAP) {
        // the records are in LDS for every wave; a bare barrier, so the
        // featg loads stay in flight
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(tail_waitcnt_lgkm0);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    } else {
        __syncthreads();
    }

    // ---- phase 2: G lanes per pixel, 8 channels each; the feature taps of
    // NB pixels are requested together, then used
    constexpr int ITER = BN / PPB;
    constexpr int NBMAX = sizeof(TF) == 2 ? TAIL_NB16 : TAIL_NB32;
    constexpr int NB = ITER < NBMAX ? ITER : NBMAX;
    static_assert(ITER % NB == 0, "tail batch");
    const int lane = tid & 63, wid = tid >> 6;
    const int gl = lane % G, grp = lane / G;
    const int c0 = gl * 8;
    float sn[8];
    if (a.s_next) load8<float>::run(a.s_next + (int64_t) fr * C + c0, sn);
    // 32-bit byte offsets from per-frame bases; a tap outside the map reads
    // the zero pad that follows the feature map (TAIL_FEAT_PAD bytes), whose
    // product w * 0 = +0 leaves the running sum unchanged, as skipping it does
    const unsigned pad_off = (unsigned) RR * C * (unsigned) sizeof(TF);
    const __amdgpu_buffer_rsrc_t featrs = buffer_rsrc(a.feat, (int64_t) pad_off + TAIL_FEAT_PAD);
    char *trunkb = a.trunk ? (char *) a.trunk + (int64_t) fr * RR * C * (int64_t) sizeof(TT) : nullptr;
    float *warpf = a.warp_tap ? a.warp_tap + (int64_t) fr * RR * C : nullptr;
    for (int it0 = 0; it0 < ITER; it0 += NB) {
        taps4 t[NB];
        float m[NB];
        feat8<TF> fv[NB][4];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const int lp = (it0 + b) * PPB + wid * PPW + grp;
            const floatx4 q0 = *(const floatx4 *) (prm + lp * L::PRM);
            t[b].x0 = __float_as_int(q0[0]);
            t[b].y0 = __float_as_int(q0[1]);
            t[b].wx = q0[2];
            t[b].wy = q0[3];
            m[b] = prm[lp * L::PRM + 4];
            const bool inx[2] = {(unsigned) t[b].x0 < (unsigned) r, (unsigned) t[b].x0 + 1u < (unsigned) r};
            const bool iny[2] = {(unsigned) t[b].y0 < (unsigned) r, (unsigned) t[b].y0 + 1u < (unsigned) r};
            const unsigned base = ((unsigned) (t[b].y0 * r + t[b].x0) * C + c0) * (unsigned) sizeof(TF);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const unsigned off = base + (unsigned) (((k >> 1) * r + (k & 1)) * C * (int) sizeof(TF));
                fv[b][k].load(featrs, inx[k & 1] && iny[k >> 1] ? off : pad_off);
            }
        }
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const int lp = (it0 + b) * PPB + wid * PPW + grp;
            const int pix = tile_pix<TWC>(pix0, r, lp);
            // taps and weights exactly as the reference selects them; the
            // weighted sum as one fused multiply-add per channel and tap
            float smp[8];
#pragma unroll
            for (int e = 0; e < 8; e++) smp[e] = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float wk = tap_weight(t[b], k);
#pragma unroll
                for (int e = 0; e < 8; e++) smp[e] = __builtin_fmaf(wk, fv[b][k][e], smp[e]);
            }
            float warp[8];
#pragma unroll
            for (int e = 0; e < 8; e++) warp[e] = smp[e] * m[b];
            const unsigned po = (unsigned) pix * C + c0;
            if (warpf) store8<float>(warpf + po, warp);
            if (trunkb) {
                const floatx4 x0 = *(const floatx4 *) (so + lp * L::SOS + c0);
                const floatx4 x1 = *(const floatx4 *) (so + lp * L::SOS + c0 + 4);
                const float ov[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
                const float one_m = 1.0f - m[b];
                float trunk[8];
#pragma unroll
                for (int e = 0; e < 8; e++) trunk[e] = warp[e] + ov[e] * one_m;
                if (a.s_next) {
#pragma unroll
                    for (int e = 0; e < 8; e++) trunk[e] = trunk[e] * sn[e];
                }
                store8<TT>((TT *) (trunkb + po * (unsigned) sizeof(TT)), trunk);
            }
        }
    }
    if (TAIL_FEATG_OVERLAP && tid < BN) {
        const float skr[3] = {sk.rgb[0], sk.rgb[1], sk.rgb[2]};
        tail_featg_finish(a, gt, gm, fr, tile_pix<TWC>(pix0, r, tid), skr, gv);
    }
}

// One pixel pp = frame * r*r + y*r + x of the batch; `valid` false for the
// padding lanes of the last group (they take part in the butterflies and
// store nothing).  ov: this lane's 8 dense-conv output channels (f32).
template <typename TF, typename TT, int G, bool FGR>
__device__ __forceinline__ void tail_pixel(const TailArgs &a, int64_t pp, bool valid, int gl,
                                           const float ov[8], const TailWeights &w) {
    // one rounding per operation everywhere; the two dot products use explicit fma
#pragma clang fp contract(off)
    const int c0 = gl * 8;
    const int r = a.r, C = a.C, rh = r >> 1;
    const int64_t RR = (int64_t) r * r;
    const int fr = (int) (pp / RR);
    const int pix = (int) (pp - (int64_t) fr * RR);
    const int y = pix / r, x = pix - y * r;

    // ---- ToFlow: (Wf * s_f) . out, folded weight rounded like gemm_weight
    float sf[8];
    load8<float>::run(a.sflow + (int64_t) fr * C + c0, sf);
    float fl[3];
#pragma unroll
    for (int k = 0; k < 3; k++) {
        float acc = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float wv = w.wf[k][e] * sf[e];
            acc = __builtin_fmaf(wv, ov[e], acc);
        }
        fl[k] = group_sum<G>(acc);
    }
#pragma unroll
    for (int k = 0; k < 3; k++) {
        fl[k] = fl[k] + a.fbias[k];
        if (a.flow_prev)
            fl[k] = fl[k] + upfirdn2x_at(a.flow_prev + ((int64_t) fr * 3 + k) * rh * rh, rh, rh, a.fup, x, y);
    }
    if (a.flow_cur && valid && gl < 3) {
        const float v = gl == 0 ? fl[0] : (gl == 1 ? fl[1] : fl[2]);
        a.flow_cur[((int64_t) fr * 3 + gl) * RR + pix] = v;
    }

    // ---- flow head + gather
    const float gx = tanhf(fl[0]) + a.lin[x];
    const float gy = tanhf(fl[1]) + a.lin[y];
    const float m = 1.0f / (1.0f + expf(-fl[2]));
    const taps4 t = gather_geometry(gx, gy, r, r);
    feat8<TF> fv[4];  // kept in the stored type until used
    bool in[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {  // issue the four tap loads together
        in[k] = tap_inside(t, k, r, r);
        if (in[k]) fv[k].load((const TF *) a.feat + (int64_t) ((t.y0 + (k >> 1)) * r + t.x0 + (k & 1)) * C + c0);
    }
    float smp[8];
#pragma unroll
    for (int e = 0; e < 8; e++) smp[e] = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        if (!in[k]) continue;
        const float wk = tap_weight(t, k);
#pragma unroll
        for (int e = 0; e < 8; e++) smp[e] += wk * fv[k][e];
    }

    // ---- warp / trunk
    float warp[8], trunk[8];
    const float one_m = 1.0f - m;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        warp[e] = smp[e] * m;
        trunk[e] = warp[e] + ov[e] * one_m;
    }
    if (valid && a.warp_tap) store8<float>(a.warp_tap + pp * C + c0, warp);
    if (valid && a.trunk) {
        if (a.s_next) {
            float sn[8];
            load8<float>::run(a.s_next + (int64_t) fr * C + c0, sn);
#pragma unroll
            for (int e = 0; e < 8; e++) trunk[e] = trunk[e] * sn[e];
        }
        store8<TT>((TT *) a.trunk + pp * C + c0, trunk);
    }

    // ---- ToRGB: from the per-feature-pixel Wr . feat (FGR, TailArgs::featg
    // set: lane 0 stores the pixel's three values), else a dot over the G
    // lanes' channels
    if constexpr (FGR) {
        if (valid && gl == 0) {
            tail_skip sk{};
            if (a.rgb_prev) {
#pragma unroll
                for (int k = 0; k < 3; k++)
                    sk.rgb[k] = upfirdn2x_at(a.rgb_prev + ((int64_t) fr * 3 + k) * rh * rh, rh, rh, a.rup, x, y);
            }
            tail_featg_rgb(a, t, m, fr, pix, sk);
        }
        return;
    }
    float rgb[3];
#pragma unroll
    for (int k = 0; k < 3; k++) {
        float acc = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) acc = __builtin_fmaf(w.wr[k][e], warp[e], acc);
        rgb[k] = group_sum<G>(acc);
    }
    if (valid && gl < 3) {
        const int k = gl;
        const float rv = k == 0 ? rgb[0] : (k == 1 ? rgb[1] : rgb[2]);
        float v = leaky(rv + a.rlb[k]);
        v = v + a.rbias[k];
        if (a.rgb_prev)
            v = v + upfirdn2x_at(a.rgb_prev + ((int64_t) fr * 3 + k) * rh * rh, rh, rh, a.rup, x, y);
        a.rgb_cur[((int64_t) fr * 3 + k) * RR + pix] = v;
    }
}

}  // namespace tpmd
