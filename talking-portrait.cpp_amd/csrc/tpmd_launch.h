// Host-callable kernel launchers of the motion-decoder library (internal).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tpmd {

constexpr int kMaxSeg = 32;

// style GEMV: global row -> (conv segment, row within it, output offset)
struct SegTable {
    int n;                    // segments
    int row0[kMaxSeg + 1];    // first global row of each segment; row0[n] = total
    int width[kMaxSeg];       // rows of the segment (= channels of the style)
    int64_t out0[kMaxSeg];    // element offset of the segment's [frame][width] block
};

// demodulation: global row -> (demod conv, output channel)
struct DemodTable {
    int n;
    int row0[kMaxSeg + 1];
    int ic[kMaxSeg], oc[kMaxSeg];
    int64_t saug0[kMaxSeg];   // element offset of the conv's S_aug: [OC][IC], then [OC]
    int64_t s0[kMaxSeg];      // element offset of its style block [frame][IC]
    int64_t d0[kMaxSeg];      // element offset of its 1/den block [frame][OC]
};

// zero bytes that follow every warp feature map and its ToRGB projection:
// the fused stage tail reads them for the bilinear taps outside the map
constexpr int TAIL_FEAT_PAD = 64;
constexpr int TAIL_FEATG_PAD = 64;

struct TailArgs {
    const void *out;          // CL [frame][r*r][C] dense-conv output (TOUT)
    const void *feat;         // [r*r][C] warp features (TF), then TAIL_FEAT_PAD zero bytes
    const float *wflow;       // [3][C] ToFlow weight (scale-folded)
    const float *sflow;       // [frame][C] ToFlow style
    const float *fbias;       // [3]
    const float *fup;         // [16] upsample kernel (x4 gain)
    const float *flow_prev;   // SP [frame][3][r/2][r/2] or null
    float *flow_cur;          // SP [frame][3][r][r] or null
    const float *lin;         // [r] identity grid coordinates
    const float *wrgb;        // [3][C] ToRGB weight (scale-folded)
    const float *rlb;         // [3] ToRGB FusedLeakyReLU bias (x sqrt2)
    const float *rbias;       // [3] ToRGB output bias
    const float *rup;         // [16]
    const float *rgb_prev;    // SP [frame][3][r/2][r/2] or null
    float *rgb_cur;           // SP [frame][3][r][r]
    const float *s_next;      // [frame][C] style of the next up-conv, or null
    void *trunk;              // CL [frame][r*r][C] (TT) or null
    float *warp_tap;          // CL [frame][r*r][C] f32 or null (tests)
    // [r*r][4] f32: ToRGB weight . feat of each feature pixel (4th value 0),
    // then TAIL_FEATG_PAD zero bytes, or null; when set, the fused tile
    // tails take the ToRGB sum from it instead of from the warp (the
    // standalone per-pixel tail always sums the warp)
    const float *featg;
    int nframes, r, C;
};

// g[p] = (wrgb[0] . feat[p], wrgb[1] . feat[p], wrgb[2] . feat[p], 0), p < npix
hipError_t launch_feat_rgb(bool feat_f16, const void *feat, const float *wrgb, int C, int64_t npix, float *g,
                           hipStream_t st);
hipError_t launch_gather(const void *feat, bool feat_f16, const float *grid, float *dst, int C,
                         int W, int H, int64_t N, int planar, int sp, hipStream_t st);
hipError_t launch_gather_taps(const float *grid, int W, int H, int64_t N, int planar, int32_t *x0,
                              int32_t *y0, float *wx, float *wy, hipStream_t st);
hipError_t launch_upfirdn2x(const float *x, const float *k4, float *y, int W, int H, int64_t CB,
                            hipStream_t st);
// CHW f32 frames -> interleaved RGB24 (tp-cli's conversion)
hipError_t launch_rgb24(const float *chw, int n, int R, uint8_t *rgb, hipStream_t st);
hipError_t launch_flow_grid(const float *fl, const float *xs, float *y, int64_t N,
                            hipStream_t st);

// one modulated 3x3 conv launch (k_conv.hip)
struct ConvArgs {
    int mode = 0;               // 0 dense, 1 composed sub-pixel up-conv
    bool f16 = false;           // operands f16 (else f32)
    bool out_f16 = false;       // stored activation f16 (f16 mode only)
    const void *A = nullptr;    // [M][9*IC], M = OC or 4*OC
    const void *A_perm = nullptr;   // the same in the order modconv_a_order names, or null
    const void *X = nullptr;    // CL input [frame][H][W][IC], frame stride x_bstride
    void *Y = nullptr;          // CL output [frame][H'][W'][OC]
    const float *inv_den = nullptr;    // [frame][OC]
    const float *bias = nullptr;       // [OC]
    const float *out_scale = nullptr;  // [frame][OC] or null
    int nframes = 0, H = 0, W = 0, IC = 0, OC = 0;
    int64_t x_bstride = 0;
    float *ws = nullptr;        // split-K workspace, ws_elems floats
    int64_t ws_elems = 0;
    // fused stage tail (dense conv with OC in {32, 64, 128}): the conv output
    // stays on chip; Y is unused and the tail's outputs are written instead
    const TailArgs *tail = nullptr;
    bool trunk_f16 = false;
};

int modconv_k_align(bool f16);
// the order in which the kernel chosen for a conv shape reads A best
// (ConvArgs::A_perm holds that copy; a function of the per-frame shape only):
//   A_ORDER_TAP    [M][9][IC], A itself (no copy);
//   A_ORDER_FRAG   [9][IC/16][M/32][64][8], MFMA fragment order: fragment
//                  (tap, ks) of row block w at lane l holds row 32w + l%32,
//                  k = tap*IC + ks*16 + (l/32)*8 .. +8 (the halo up-convs,
//                  the 64 -> 32 up-conv and the fused 32- to 128-channel
//                  dense convs), so a wave reads each fragment as one
//                  contiguous 1 KB;
//   A_ORDER_RING_TAP  [M/16][9*IC/32][64][8], the LDS image of each block of
//                  16 rows x one tap-major k tile of 32 channels (lane i =
//                  row 16g + i/4, k chunk (i%4) ^ ((row>>2 ^ row>>3) & 3)),
//                  so each A DMA instruction of the fused 256-channel dense
//                  conv's LDS ring (r64) reads 1 KB of contiguous memory.
enum { A_ORDER_TAP = 0, A_ORDER_FRAG = 2, A_ORDER_RING_TAP = 3 };
int modconv_a_order(bool f16, bool out_f16, int mode, int IC, int OC, int H, int W);
// whether the dense conv of an r x r stage with OC channels fuses the tail
bool modconv_fusable(int OC, int r, bool f16);
// split-K factor of a conv (depends on the per-frame shape only)
int modconv_splits(int mode, int H, int W, int IC, int OC, bool f16);
// workspace floats a conv needs for nframes frames (0 = no split)
int64_t modconv_ws_elems(int mode, int nframes, int H, int W, int IC, int OC, bool f16);
hipError_t launch_modconv(const ConvArgs &c, hipStream_t st);

hipError_t launch_stage_tail(const TailArgs &a, bool feat_f16, bool out_f16, bool trunk_f16,
                             hipStream_t st);

hipError_t launch_style_gemv(const float *Wm, const float *bm, const float *lat, float *s,
                             const SegTable &seg, int nframes, hipStream_t st);
hipError_t launch_demod(const float *saug, const float *s, float *inv_den, const DemodTable &t,
                        int nframes, hipStream_t st);
hipError_t launch_prescale_input(bool f16, const float *in, const float *s, void *xs, int C,
                                 int nframes, hipStream_t st);
hipError_t launch_prescale_map(bool f16, const float *x, const float *s, void *xs, int C,
                               int64_t npix_per_frame, int nframes, hipStream_t st);

}  // namespace tpmd
