// tp::motion_enc over tpme_* (see motion_enc.h).
#include "motion_enc.h"

namespace tp {

bool motion_enc::fail(std::string &err, const char *what) {
    err = std::string(what) + ": " + (ctx ? tpme_last_error(ctx) : "no context");
    return false;
}

bool motion_enc::run(hip_backend &be, const float *image, menc_result &out, std::string &err) {
    if (!w) {
        err = "motion_enc: no weights";
        return false;
    }
    if (!built) {
        // channel plan from the decoder's (see motion_enc.h)
        const int n = be.n_stages;
        std::vector<int> cin, cout;
        if (!be.stage_oc.empty()) {
            if ((int) be.stage_oc.size() != n || n != 7) {
                err = "motion_enc: the encoder needs the 7-stage decoder plan";
                return false;
            }
            cout.resize(7);
            cin.resize(7);
            for (int i = 0; i < 6; i++) cout[(size_t) i] = be.stage_oc[(size_t) (5 - i)];
            cout[6] = be.stage_oc[0];
            cin[0] = be.stage_oc[6];
            for (int i = 1; i < 7; i++) cin[(size_t) i] = cout[(size_t) (i - 1)];
        }
        release();
        ctx = tpme_create(be.device, be.ftype.c_str(), 7, cin.empty() ? nullptr : cin.data(),
                          cout.empty() ? nullptr : cout.data());
        if (!ctx) {
            err = "motion_enc: tpme_create failed";
            return false;
        }
        std::vector<float> v;
        for (int i = 0;; i++) {
            int64_t ne = 0;
            const char *name = tpme_weight_name(ctx, i, &ne, nullptr);
            if (!name) break;
            bool f16 = false;
            if (!w->get(name, v, f16)) continue;  // prepare names the first missing tensor
            if (tpme_set_weight(ctx, name, v.data(), (int64_t) v.size(), f16 ? TPMD_W_F16_FILE : 0) != 0)
                return fail(err, "set_weight");
        }
        if (tpme_prepare(ctx) != 0) return fail(err, "prepare");
        built = true;
    }
    if (tpme_run(ctx, image, 0) != 0) return fail(err, "run");
    out.appearance.assign(512, 0.0f);
    out.lambda.assign(20, 0.0f);
    out.motion.assign(512, 0.0f);
    if (tpme_result(ctx, out.appearance.data(), out.lambda.data(), out.motion.data()) != 0)
        return fail(err, "result");
    out.feats.assign(7, {});
    out.feat_ch.assign(7, 0);
    out.feat_res.assign(7, 0);
    for (int j = 0; j < 7; j++) {
        const int l = 6 - j;  // pyramid level of feats j
        const int64_t n = tpme_level(ctx, l, nullptr);
        if (n < 0) return fail(err, "feats");
        out.feats[(size_t) j].resize((size_t) n);
        if (tpme_level(ctx, l, out.feats[(size_t) j].data()) != n) return fail(err, "feats");
        int C = 0, r = 0;
        tpme_feat(ctx, j, &C, &r);
        out.feat_ch[(size_t) j] = C;
        out.feat_res[(size_t) j] = r;
    }
    return true;
}

std::vector<const float *> motion_enc::device_feats() const {
    std::vector<const float *> v;
    for (int j = 0; ctx && j < 7; j++) v.push_back(tpme_feat(ctx, j, nullptr, nullptr));
    return v;
}

void motion_enc::release() {
    if (ctx) tpme_destroy(ctx);
    ctx = nullptr;
    built = false;
}

}  // namespace tp
