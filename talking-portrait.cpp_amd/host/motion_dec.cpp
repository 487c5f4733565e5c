// tp::motion_dec over the C ABI of include/tpmd.h (see motion_dec.h).
#include "motion_dec.h"

#include <cstdlib>

namespace tp {

namespace {

tpmd_ctx *create_ctx(const hip_backend &be) {
    const bool custom = !be.stage_ic.empty();
    if (custom && ((int) be.stage_ic.size() < be.n_stages || (int) be.stage_oc.size() < be.n_stages))
        return nullptr;
    return tpmd_create(be.device, be.ftype.c_str(), be.n_stages, custom ? be.stage_ic.data() : nullptr,
                       custom ? be.stage_oc.data() : nullptr);
}

}  // namespace

bool motion_dec::fail(std::string &err, const char *what) {
    err = std::string(what) + ": " + tpmd_last_error(ctx);
    return false;
}

std::vector<std::string> motion_dec_host_tensors(const hip_backend &be) {
    std::vector<std::string> v;
    tpmd_ctx *c = create_ctx(be);
    if (!c) return v;
    for (int i = 0;; i++) {
        const char *n = tpmd_weight_name(c, i, nullptr, nullptr);
        if (!n) break;
        v.push_back(n);
    }
    tpmd_destroy(c);
    return v;
}

// src/motion_dec.cpp:31-226: every decoder tensor is handed over raw; the
// library folds the load-time scales and derives S_aug / composed kernels
bool motion_dec::prepare(hip_backend &be, std::string &err) {
    release();
    if (!w) {
        err = "motion_dec: no weights";
        return false;
    }
    ctx = create_ctx(be);
    if (!ctx) {
        err = "motion_dec: tpmd_create failed (device / ftype / channel plan)";
        return false;
    }
    if (be.stream && tpmd_set_stream(ctx, be.stream) != 0) return fail(err, "set_stream");
    std::vector<float> data;
    for (int i = 0;; i++) {
        int64_t n = 0;
        int is_matrix = 0;
        const char *name = tpmd_weight_name(ctx, i, &n, &is_matrix);
        if (!name) break;
        bool f16_file = false;
        data.clear();
        if (!w->get(name, data, f16_file)) {
            err = std::string("missing tensor ") + name;
            return false;
        }
        if ((int64_t) data.size() != n) {
            err = std::string("motion_dec: bad element count for ") + name;
            return false;
        }
        if (tpmd_set_weight(ctx, name, data.data(), n, f16_file ? TPMD_W_F16_FILE : 0) != 0)
            return fail(err, "set_weight");
    }
    if (tpmd_prepare(ctx) != 0) return fail(err, "prepare");
    res = tpmd_out_res(ctx);
    static const int REF_OC[7] = {512, 512, 512, 256, 128, 64, 32};
    feat_sizes.clear();
    for (int j = 0; j < be.n_stages; j++) {
        const size_t r = (size_t) 8 << j;
        feat_sizes.push_back(r * r * (size_t) (be.stage_oc.empty() ? REF_OC[j] : be.stage_oc[(size_t) j]));
    }
    return true;
}

bool motion_dec::build(hip_backend &be, bool with_taps, std::string &err) {
    (void) be;
    if (!ctx) {
        err = "motion_dec: build before prepare";
        return false;
    }
    int b = 8;
    if (const char *e = std::getenv("TP_MDEC_BATCH")) b = std::atoi(e);
    if (b < 1) b = 1;
    if (b > MAX_BATCH) b = MAX_BATCH;
    if (tpmd_build(ctx, b) != 0) return fail(err, "build");
    batch = tpmd_batch(ctx);
    img_chunks = 1;
    // the tap plan (decode with a tap sink) runs beside the batched plan on
    // the same buffers, so asking for it changes nothing else
    taps_in_graph = with_taps;
    built = true;
    return true;
}

// src/motion_dec.cpp:1137-1160
bool motion_dec::set_feats_vec(const std::vector<std::vector<float>> &feats, std::string &err) {
    if (!built) {
        err = "decoder not built";
        return false;
    }
    if (feats.size() < feat_sizes.size()) {
        err = "feat size mismatch";
        return false;
    }
    std::vector<const float *> p(feat_sizes.size());
    for (size_t j = 0; j < feat_sizes.size(); j++) {
        if (feats[j].size() != feat_sizes[j]) {
            err = "feat size mismatch";
            return false;
        }
        p[j] = feats[j].data();
    }
    if (tpmd_set_feats(ctx, p.data()) != 0) return fail(err, "set_feats");
    return true;
}

// src/motion_dec.cpp:1162-1188 (one frame; the reference replicates the style
// across its fixed batch, the library decodes n = 1 directly)
bool motion_dec::decode(hip_backend &be, const float *style, float *img_out, std::string &err) {
    (void) be;
    if (!built) {
        err = "decoder not built";
        return false;
    }
    if (tpmd_decode_batch(ctx, style, 1, img_out, 0) != 0) return fail(err, "decode");
    return true;
}

// src/motion_dec.cpp:1190-1220
bool motion_dec::decode_batch(hip_backend &be, const float *styles, float *imgs_out, std::string &err) {
    (void) be;
    if (!built) {
        err = "decoder not built";
        return false;
    }
    if (tpmd_decode_batch(ctx, styles, batch, imgs_out, 0) != 0) return fail(err, "decode_batch");
    return true;
}

void motion_dec::release() {
    if (ctx) tpmd_destroy(ctx);
    ctx = nullptr;
    built = false;
    img_chunks = 0;
    batch = 1;
    feat_sizes.clear();
}

}  // namespace tp
