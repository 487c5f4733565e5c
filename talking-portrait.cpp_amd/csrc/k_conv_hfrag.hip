// Halo convs (the kernel is in tpmd_hfrag.h): the shape -> configuration
// rule and the launch for every chunk count.
#include "tpmd_hfrag.h"

namespace tpmd {

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
    // the 128-channel up-conv (r256): 128-row tiles on four waves, two
    // workgroups per CU
    if (IC == 128 && mode == MODE_SUBPIX && tiles(128, 8, 32) >= 256) return 2;
    if (tiles(256, 8, 32) >= 256) return 1;
    if (tiles(128, 8, 32) >= 256) return 2;
    if (tiles(128, 16, 16) >= 256) return 3;
    return 0;
}

// f16 output, or f32 output of a dense conv on 128-row tiles
bool modconv_hfrag_ok(bool f16, bool out_f16, int mode, int IC, int OC, int H, int W) {
    const int M = mode == MODE_DENSE ? OC : 4 * OC;
    const int cfg = hfrag_config(f16, mode, IC, H, W, M);
    return cfg != 0 && (out_f16 || (mode == MODE_DENSE && cfg != 1)) && (int64_t) M * 9 * IC * 2 < ((int64_t) 1 << 31);
}

TPMD_HFRAG_NC(1);
TPMD_HFRAG_NC(2);
TPMD_HFRAG_NC(4);

hipError_t launch_modconv_hfrag(ConvParams p, int mode, bool out_f16, hipStream_t st) {
    const int cfg = hfrag_config(true, mode, p.IC, p.H, p.W, p.M);
    if (cfg == 0 || (!out_f16 && (mode != MODE_DENSE || cfg == 1))) return hipErrorInvalidValue;
    const int BM = cfg == 1 ? 256 : 128, TH = cfg == 3 ? 16 : 8, TW = cfg == 3 ? 16 : 32;
    const int64_t HW = (int64_t) p.H * p.W;
    if (p.N % HW != 0) return hipErrorInvalidValue;
    // A and the input are read through buffer resources, whose extents are
    // 32-bit byte counts (a halo unit outside the map reads at 2^31)
    if ((int64_t) p.M * 9 * p.IC * 2 >= ((int64_t) 1 << 31) ||
        (p.N / HW) * p.x_bstride * 2 >= ((int64_t) 1 << 31))
        return hipErrorInvalidValue;
    p.MT = p.M / BM;
    p.T = 9 * p.IC / 32;
    const int tiles_x = p.W / TW, tiles_frame = tiles_x * (p.H / TH);
    const dim3 grid((unsigned) ((int64_t) p.MT * (p.N / HW) * tiles_frame));
    switch (p.IC) {
        case 32: return launch_hfrag_nc<1>(p, cfg, mode, out_f16, tiles_x, tiles_frame, grid, st);
        case 64: return launch_hfrag_nc<2>(p, cfg, mode, out_f16, tiles_x, tiles_frame, grid, st);
        case 128: return launch_hfrag_nc<4>(p, cfg, mode, out_f16, tiles_x, tiles_frame, grid, st);
        case 256: return launch_hfrag_nc<8>(p, cfg, mode, out_f16, tiles_x, tiles_frame, grid, st);
        case 512: return launch_hfrag_nc<16>(p, cfg, mode, out_f16, tiles_x, tiles_frame, grid, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace tpmd
