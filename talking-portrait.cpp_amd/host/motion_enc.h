// tp::motion_enc over the MI355X encoder entry points (tpme_*, include/tpmd.h).
//
// Keeps the reference's motion_enc interface (src/motion_enc.h:10-30): one
// run(be, image, menc_result, tap, err) per portrait, whose result feeds
// motion_dec::set_feats (src/pipeline.cpp:113-115).  The weights come from
// the same weight_source as the decoder's (the motion_ae checkpoint holds
// enc.* and dec.direction.Q next to dec.*).  The channel plan follows the
// decoder's: feats j must have stage_oc[j] channels, so ResBlock i outputs
// stage_oc[n-2-i] channels and the stem stage_oc[n-1] (the reference's
// {32 -> 64,128,256,512,512,512,512} for the reference decoder).
#pragma once

#include <string>
#include <vector>

#include "motion_dec.h"

namespace tp {

struct menc_result {
    std::vector<float> appearance;  // s_r [512]
    std::vector<float> lambda;      // [20]
    std::vector<float> motion;      // r_s [512] = Q lambda
    // pyramid features for decoder warping, host copies, pixel-major [r*r][C]
    // (index j: stage r = 8 << j warps feats[j] = menc conv{6-j})
    std::vector<std::vector<float>> feats;
    std::vector<int> feat_ch, feat_res;
};

struct motion_enc {
    const weight_source *w = nullptr;  // borrowed (the reference's weights_t *)

    tpme_ctx *ctx = nullptr;
    bool built = false;

    // image: [3][512][512] f32 CHW in [-1, 1] (host).  Taps come from the
    // reference's tap plan, which this library does not run: a run that asks
    // for taps fails.
    template <class Tap>
    bool run(hip_backend &be, const float *image, menc_result &out, Tap &tap, std::string &err) {
        if (tap) {
            err = "motion_enc: taps need the reference's tap plan, which the HIP encoder does not run";
            return false;
        }
        return run(be, image, out, err);
    }
    bool run(hip_backend &be, const float *image, menc_result &out, std::string &err);
    // device addresses of the last run's feats (tpme_feat), for
    // tpmd_set_feats_device without a host round trip
    std::vector<const float *> device_feats() const;

    void release();
    ~motion_enc() { release(); }

  private:
    bool fail(std::string &err, const char *what);
};

}  // namespace tp
