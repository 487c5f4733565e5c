// Motion-encoder context behind the tpme_* C ABI: the reference's
// tp::motion_enc (src/motion_enc.h:20-30) with its weights_t slice (enc.*
// tensors and dec.direction.Q), prepare-time operand layout and the run
// (src/motion_enc.cpp:50-184) on the k_enc.hip kernels.  Host code only.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <map>
#include <string>
#include <vector>

#include "tpmd_guard.h"
#include "tpmd.h"
#include "tpmd_enc.h"

using namespace tpmd;

namespace {

std::string efmt(const char *f, ...) __attribute__((format(printf, 1, 2)));
std::string efmt(const char *f, ...) {
    char b[512];
    va_list ap;
    va_start(ap, f);
    vsnprintf(b, sizeof b, f, ap);
    va_end(ap);
    return b;
}

struct ETensor {
    std::vector<float> data;  // scale-folded f32
    int flags = 0;
};

// motion_ae_scale for the encoder tensors and dec.direction.Q
// (src/motion_enc.cpp:14-45); ne is the ggml order (reversed torch shape)
double enc_scale(const std::string &name, const std::vector<int64_t> &ne) {
    const double SQRT2 = 1.4142135623730951;
    auto ends_with = [&](const char *s) {
        size_t n = strlen(s);
        return name.size() >= n && name.compare(name.size() - n, n, s) == 0;
    };
    if (name == "enc.net_app.convs.0.1.bias" || ends_with(".conv1.1.bias") || ends_with(".activate.bias"))
        return SQRT2;
    if (!ends_with(".weight")) return 1.0;
    if (name.rfind("dec.direction", 0) == 0 || ends_with("noise.weight")) return 1.0;
    if (ends_with("modulation.weight")) return 1.0 / sqrt((double) ne[0]);
    if (name.rfind("enc.fc.", 0) == 0) return 1.0 / sqrt((double) ne[0]);
    const double conv = 1.0 / sqrt((double) (ne[0] * ne[1] * ne[2]));
    if (name == "enc.net_app.convs.0.0.weight" || ends_with(".conv1.0.weight")) return conv * SQRT2;
    if (ends_with(".conv2.1.weight")) return conv;
    if (ends_with(".skip.1.weight")) return conv / SQRT2;
    if (name.rfind("enc.net_app.convs.", 0) == 0) return conv;  // the final 4x4 conv
    return 1.0;
}

}  // namespace

struct tpme_ctx {
    int device = 0;
    bool f16 = false;
    int nb = 7;
    int cin[8] = {}, cout[8] = {};
    int res = 512;
    std::string err;
    hipStream_t stream = nullptr;

    std::vector<std::pair<std::string, std::vector<int64_t>>> tensors;
    std::map<std::string, ETensor> host;
    bool prepared = false, ran = false;
    std::vector<void *> allocs;

    struct Conv {
        void *A = nullptr;  // [OC][KH][KW][IC], f16 when kept f16
        bool f16 = false;
        int ic = 0, oc = 0, k = 0;
    };
    struct Block {
        Conv c1, c2, sk;
        float *b1 = nullptr, *b2 = nullptr, *k2 = nullptr, *ks = nullptr;
    } blk[8];
    float *stem_w = nullptr, *stem_b = nullptr;
    float *w_last = nullptr;  // the final 4x4 conv as [512][16*C] f32 values
    bool last16 = false;
    float *fc_w[5] = {}, *fc_b[5] = {}, *q = nullptr;
    bool fc16[5] = {}, q16 = false;
    int dim = 512, n_motion = 20;

    // activations
    float *img = nullptr;
    float *lvl[9] = {};          // menc.conv<l>, CL f32
    void *xa = nullptr;          // next conv1's operand copy (f16 mode)
    float *x1 = nullptr, *sk = nullptr;
    void *xb = nullptr, *sb = nullptr;
    float *app = nullptr, *fch[5] = {}, *motion = nullptr;
    float *ws = nullptr;         // split-K partials of the deep levels' convs

    bool hip_ok(hipError_t e, const char *what) {
        if (e == hipSuccess) return true;
        err = efmt("%s: %s", what, hipGetErrorString(e));
        return false;
    }
    void *dalloc(size_t bytes) {
        void *p = nullptr;
        if (hipMalloc(&p, bytes < 256 ? 256 : bytes) != hipSuccess) {
            err = efmt("hipMalloc of %zu bytes failed", bytes);
            return nullptr;
        }
        allocs.push_back(p);
        return p;
    }
    template <typename T>
    T *upload(const std::vector<T> &v) {
        T *p = (T *) dalloc(v.size() * sizeof(T));
        if (!p) return nullptr;
        if (!hip_ok(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice), "upload")) return nullptr;
        return p;
    }
    const ETensor *need(const std::string &name) {
        auto it = host.find(name);
        if (it == host.end()) {
            if (err.empty()) err = "missing tensor " + name;
            return nullptr;
        }
        return &it->second;
    }
    // kept f16 under the keep rule (src/gguf_load.cpp:149-153)
    bool kept16(const ETensor &t) const { return f16 && (t.flags & TPMD_W_F16_FILE) && t.data.size() >= 4096; }
    std::vector<float> dev_value(const ETensor &t) const {
        std::vector<float> v = t.data;
        if (kept16(t))
            for (auto &x : v) x = (float) (_Float16) x;
        return v;
    }
    int level_res(int l) const { return res >> l; }
    int level_ch(int l) const { return l == 0 ? cin[0] : cout[l - 1]; }
    void free_all() {
        for (void *p : allocs) (void) hipFree(p);
        allocs.clear();
    }
    ~tpme_ctx() {
        if (device >= 0) (void) hipSetDevice(device);
        free_all();
        if (stream) (void) hipStreamDestroy(stream);
    }
};

namespace {

bool check(tpme_ctx *c) {
    if (!c) return false;
    c->err.clear();
    if (hipSetDevice(c->device) != hipSuccess) {
        c->err = "hipSetDevice failed";
        return false;
    }
    return true;
}

void make_tensor_list(tpme_ctx *c) {
    auto &v = c->tensors;
    const std::string b0 = "enc.net_app.convs";
    v.push_back({b0 + ".0.0.weight", {c->cin[0], 3, 1, 1}});
    v.push_back({b0 + ".0.1.bias", {c->cin[0]}});
    for (int i = 1; i <= c->nb; i++) {
        const int64_t ci = c->cin[i - 1], co = c->cout[i - 1];
        const std::string b = efmt("%s.%d", b0.c_str(), i);
        v.push_back({b + ".conv1.0.weight", {ci, ci, 3, 3}});
        v.push_back({b + ".conv1.1.bias", {ci}});
        v.push_back({b + ".conv2.0.kernel", {4, 4}});
        v.push_back({b + ".conv2.1.weight", {co, ci, 3, 3}});
        v.push_back({b + ".conv2.2.bias", {co}});
        v.push_back({b + ".skip.0.kernel", {4, 4}});
        v.push_back({b + ".skip.1.weight", {co, ci, 1, 1}});
    }
    v.push_back({efmt("%s.%d.weight", b0.c_str(), c->nb + 1), {c->dim, c->cout[c->nb - 1], 4, 4}});
    for (int i = 0; i < 5; i++) {
        const int64_t o = i == 4 ? c->n_motion : c->dim;
        v.push_back({efmt("enc.fc.%d.weight", i), {o, c->dim}});
        v.push_back({efmt("enc.fc.%d.bias", i), {o}});
    }
    v.push_back({"dec.direction.Q", {c->dim, c->n_motion}});
}

// torch [OC][IC][KH][KW] -> tap-major [OC][KH][KW][IC]
std::vector<float> tap_major(const std::vector<float> &w, int OC, int IC, int K) {
    std::vector<float> a(w.size());
    for (int o = 0; o < OC; o++)
        for (int i = 0; i < IC; i++)
            for (int t = 0; t < K * K; t++)
                a[((size_t) o * K * K + t) * IC + i] = w[((size_t) o * IC + i) * K * K + t];
    return a;
}

bool make_conv(tpme_ctx *c, tpme_ctx::Conv &cv, const std::string &name, int ic, int oc, int k) {
    const ETensor *t = c->need(name);
    if (!t) return false;
    cv.ic = ic;
    cv.oc = oc;
    cv.k = k;
    cv.f16 = c->kept16(*t);
    const std::vector<float> a = tap_major(c->dev_value(*t), oc, ic, k);
    if (cv.f16) {
        std::vector<_Float16> h(a.size());
        for (size_t i = 0; i < a.size(); i++) h[i] = (_Float16) a[i];
        cv.A = c->upload(h);
    } else {
        cv.A = c->upload(a);
    }
    return cv.A != nullptr;
}

float *upload_value(tpme_ctx *c, const std::string &name, bool *is16 = nullptr) {
    const ETensor *t = c->need(name);
    if (!t) return nullptr;
    if (is16) *is16 = c->kept16(*t);
    return c->upload(c->dev_value(*t));
}

}  // namespace

extern "C" {

static tpme_ctx *tpme_create_body(int device, const char *ftype, int n_blocks, const int *ch_in, const int *ch_out) {
    static const int REF_IN[7] = {32, 64, 128, 256, 512, 512, 512};
    static const int REF_OUT[7] = {64, 128, 256, 512, 512, 512, 512};
    if (!ftype || (strcmp(ftype, "f32") != 0 && strcmp(ftype, "f16") != 0)) {
        fprintf(stderr, "tpme_create: ftype must be f32 or f16\n");
        return nullptr;
    }
    if (n_blocks < 1 || n_blocks > 7 || (!ch_in != !ch_out) || (!ch_in && n_blocks != 7)) {
        fprintf(stderr, "tpme_create: n_blocks 1..7 with channel lists (7 for the reference widths)\n");
        return nullptr;
    }
    tpme_ctx *c = new tpme_ctx();
    c->device = device;
    c->f16 = strcmp(ftype, "f16") == 0;
    c->nb = n_blocks;
    c->res = 4 << n_blocks;
    for (int i = 0; i < n_blocks; i++) {
        c->cin[i] = ch_in ? ch_in[i] : REF_IN[i];
        c->cout[i] = ch_out ? ch_out[i] : REF_OUT[i];
        if (c->cin[i] <= 0 || c->cin[i] % 32 != 0 || c->cout[i] <= 0 || c->cout[i] % 32 != 0 ||
            (i > 0 && c->cin[i] != c->cout[i - 1])) {
            fprintf(stderr, "tpme_create: channel lists must be multiples of 32 with ch_in[i+1] == ch_out[i]\n");
            c->device = -1;
            delete c;
            return nullptr;
        }
    }
    if (hipSetDevice(device) != hipSuccess ||
        hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        fprintf(stderr, "tpme_create: no HIP device %d\n", device);
        c->device = -1;
        delete c;
        return nullptr;
    }
    make_tensor_list(c);
    return c;
}

void tpme_destroy(tpme_ctx *c) { delete c; }

const char *tpme_last_error(const tpme_ctx *c) { return c ? c->err.c_str() : "no context"; }

const char *tpme_weight_name(const tpme_ctx *c, int i, int64_t *n, int *is_matrix) {
    if (!c || i < 0 || i >= (int) c->tensors.size()) return nullptr;
    const auto &t = c->tensors[(size_t) i];
    int64_t e = 1;
    for (auto d : t.second) e *= d;
    if (n) *n = e;
    if (is_matrix) *is_matrix = t.second.size() >= 2 ? 1 : 0;
    return t.first.c_str();
}

static int tpme_set_weight_body(tpme_ctx *c, const char *name, const float *data, int64_t n, int flags) {
    if (!check(c)) return -1;
    if (!name || !data || n <= 0) {
        c->err = "tpme_set_weight: null name/data or empty tensor";
        return -1;
    }
    const std::vector<int64_t> *shape = nullptr;
    for (const auto &t : c->tensors)
        if (t.first == name) shape = &t.second;
    if (!shape) {
        c->err = efmt("tpme_set_weight: unknown encoder tensor %s", name);
        return -1;
    }
    int64_t want = 1;
    for (auto d : *shape) want *= d;
    if (want != n) {
        c->err = efmt("tpme_set_weight: %s has %lld elements, expected %lld", name, (long long) n, (long long) want);
        return -1;
    }
    std::vector<int64_t> ne(shape->rbegin(), shape->rend());
    while (ne.size() < 4) ne.push_back(1);
    ETensor t;
    t.data.assign(data, data + n);
    t.flags = flags;
    if (!(flags & TPMD_W_FOLDED)) {
        const double s = enc_scale(name, ne);
        if (s != 1.0) {
            const float fs = (float) s;
            for (auto &v : t.data) v *= fs;
        }
    }
    c->host[name] = std::move(t);
    c->prepared = false;
    c->ran = false;
    return 0;
}

// split-K factor of an encoder conv: the deep levels' convs have few 64 x 64
// output tiles (8 at 8 x 8 with 512 channels) against a long k loop (up to
// 9 * 512 / 32 = 144 k tiles), so their k range is split to give about 256
// workgroups; the partials are summed in split order by a second pass
static int enc_splits(int OH, int OW, int OC, int KH, int KW, int IC) {
    const int tiles = ((OH * OW + 63) / 64) * ((OC + 63) / 64);
    const int T = KH * KW * IC / 32;
    return std::max(1, std::min(256 / std::max(tiles, 1), T / 4));
}

static int tpme_prepare_body(tpme_ctx *c) {
    if (!check(c)) return -1;
    c->free_all();
    c->prepared = c->ran = false;
    for (auto &b : c->blk) b = tpme_ctx::Block{};
    const std::string b0 = "enc.net_app.convs";
    c->stem_w = upload_value(c, b0 + ".0.0.weight");
    c->stem_b = upload_value(c, b0 + ".0.1.bias");
    if (!c->stem_w || !c->stem_b) return -1;
    for (int i = 1; i <= c->nb; i++) {
        tpme_ctx::Block &B = c->blk[i - 1];
        const int ci = c->cin[i - 1], co = c->cout[i - 1];
        const std::string b = efmt("%s.%d", b0.c_str(), i);
        if (!make_conv(c, B.c1, b + ".conv1.0.weight", ci, ci, 3) ||
            !make_conv(c, B.c2, b + ".conv2.1.weight", ci, co, 3) ||
            !make_conv(c, B.sk, b + ".skip.1.weight", ci, co, 1))
            return -1;
        B.b1 = upload_value(c, b + ".conv1.1.bias");
        B.b2 = upload_value(c, b + ".conv2.2.bias");
        B.k2 = upload_value(c, b + ".conv2.0.kernel");
        B.ks = upload_value(c, b + ".skip.0.kernel");
        if (!B.b1 || !B.b2 || !B.k2 || !B.ks) return -1;
    }
    {
        const std::string nl = efmt("%s.%d.weight", b0.c_str(), c->nb + 1);
        const ETensor *t = c->need(nl);
        if (!t) return -1;
        c->last16 = c->kept16(*t);
        c->w_last = c->upload(tap_major(c->dev_value(*t), c->dim, c->cout[c->nb - 1], 4));
        if (!c->w_last) return -1;
    }
    for (int i = 0; i < 5; i++) {
        c->fc_w[i] = upload_value(c, efmt("enc.fc.%d.weight", i), &c->fc16[i]);
        c->fc_b[i] = upload_value(c, efmt("enc.fc.%d.bias", i));
        if (!c->fc_w[i] || !c->fc_b[i]) return -1;
    }
    c->q = upload_value(c, "dec.direction.Q", &c->q16);
    if (!c->q) return -1;

    // activations: the pyramid levels stay (feats and taps); the rest is
    // sized for the largest block
    const int R = c->res;
    c->img = (float *) c->dalloc((size_t) 3 * R * R * 4);
    if (!c->img) return -1;
    size_t x1b = 0, xbb = 0, sbb = 0, skb = 0, xab = 0, wsb = 0;
    for (int l = 0; l <= c->nb; l++) {
        const size_t r = (size_t) c->level_res(l);
        c->lvl[l] = (float *) c->dalloc(r * r * c->level_ch(l) * 4);
        if (!c->lvl[l]) return -1;
        if (l < c->nb) {
            const size_t C = (size_t) c->cin[l];
            x1b = std::max(x1b, r * r * C * 4);
            xbb = std::max(xbb, (r + 1) * (r + 1) * C * 4);
            sbb = std::max(sbb, (r - 1) * (r - 1) * C * 4);
            skb = std::max(skb, (r / 2) * (r / 2) * (size_t) c->cout[l] * 4);
            xab = std::max(xab, r * r * C * 4);
            const int ri = (int) r, Ci = (int) C, Co = c->cout[l];
            wsb = std::max(wsb, (size_t) enc_splits(ri, ri, Ci, 3, 3, Ci) * r * r * C * 4);
            wsb = std::max(wsb, (size_t) enc_splits(ri / 2, ri / 2, Co, 1, 1, Ci) * (r / 2) * (r / 2) * Co * 4);
            wsb = std::max(wsb, (size_t) enc_splits(ri / 2, ri / 2, Co, 3, 3, Ci) * (r / 2) * (r / 2) * Co * 4);
        }
    }
    c->ws = (float *) c->dalloc(wsb < 256 ? 256 : wsb);
    if (!c->ws) return -1;
    c->x1 = (float *) c->dalloc(x1b);
    c->xb = c->dalloc(xbb);
    c->sb = c->dalloc(sbb);
    c->sk = (float *) c->dalloc(skb);
    c->xa = c->dalloc(xab);
    c->app = (float *) c->dalloc((size_t) c->dim * 4);
    for (int i = 0; i < 5; i++) c->fch[i] = (float *) c->dalloc((size_t) c->dim * 4);
    c->motion = (float *) c->dalloc((size_t) c->dim * 4);
    if (!c->x1 || !c->xb || !c->sb || !c->sk || !c->xa || !c->app || !c->motion) return -1;
    for (int i = 0; i < 5; i++)
        if (!c->fch[i]) return -1;
    c->prepared = true;
    return 0;
}

static int tpme_run_body(tpme_ctx *c, const float *image, int on_device) {
    if (!check(c)) return -1;
    if (!c->prepared) {
        c->err = "encoder not prepared";
        return -1;
    }
    if (!image) {
        c->err = "tpme_run: null image";
        return -1;
    }
    c->ran = false;
    hipStream_t st = c->stream;
    const int R = c->res;
    const size_t ib = (size_t) 3 * R * R * 4;
    if (!c->hip_ok(hipMemcpyAsync(c->img, image, ib, on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, st),
                   "image upload"))
        return -1;
    // stem; conv1 of block 1 reads the map itself (f32) or its f16 copy
    const bool a16 = c->blk[0].c1.f16;
    if (!c->hip_ok(launch_enc_stem(c->img, c->stem_w, c->stem_b, (int64_t) R * R, c->cin[0], c->lvl[0],
                                   a16 ? c->xa : nullptr, true, st),
                   "stem"))
        return -1;
    for (int i = 1; i <= c->nb; i++) {
        const tpme_ctx::Block &B = c->blk[i - 1];
        const int r = c->level_res(i - 1), C = c->cin[i - 1], Co = c->cout[i - 1];
        EncConvParams p{};
        // x1 = leaky(conv3x3(x) + b1)
        p.A = B.c1.A;
        p.X = B.c1.f16 ? c->xa : (const void *) c->lvl[i - 1];
        p.Y = c->x1;
        p.bias = B.b1;
        p.leaky = 1;
        p.H = p.W = r;
        p.IC = C;
        p.OC = C;
        p.KH = p.KW = 3;
        p.stride = 1;
        p.pad = 1;
        p.OH = p.OW = r;
        p.ksplit = enc_splits(r, r, C, 3, 3, C);
        p.ws = c->ws;
        if (!c->hip_ok(launch_enc_conv(p, B.c1.f16, st), "conv1")) return -1;
        // skip: conv1x1 stride 2 of blur(x, pad 1)
        if (!c->hip_ok(launch_enc_blur(c->lvl[i - 1], B.ks, r, r, C, 1, c->sb, B.sk.f16, st), "skip blur")) return -1;
        p = EncConvParams{};
        p.A = B.sk.A;
        p.X = c->sb;
        p.Y = c->sk;
        p.H = p.W = r - 1;
        p.IC = C;
        p.OC = Co;
        p.KH = p.KW = 1;
        p.stride = 2;
        p.pad = 0;
        p.OH = p.OW = r / 2;
        p.ksplit = enc_splits(r / 2, r / 2, Co, 1, 1, C);
        p.ws = c->ws;
        if (!c->hip_ok(launch_enc_conv(p, B.sk.f16, st), "skip")) return -1;
        // x = leaky(conv3x3 stride 2 of blur(x1, pad 2) + b2) + skip
        if (!c->hip_ok(launch_enc_blur(c->x1, B.k2, r, r, C, 2, c->xb, B.c2.f16, st), "blur")) return -1;
        const bool next16 = i < c->nb && c->blk[i].c1.f16;
        p = EncConvParams{};
        p.A = B.c2.A;
        p.X = c->xb;
        p.Y = c->lvl[i];
        p.Ya = next16 ? c->xa : nullptr;
        p.ya_f16 = 1;
        p.bias = B.b2;
        p.res = c->sk;
        p.leaky = 1;
        p.H = p.W = r + 1;
        p.IC = C;
        p.OC = Co;
        p.KH = p.KW = 3;
        p.stride = 2;
        p.pad = 0;
        p.OH = p.OW = r / 2;
        p.ksplit = enc_splits(r / 2, r / 2, Co, 3, 3, C);
        p.ws = c->ws;
        if (!c->hip_ok(launch_enc_conv(p, B.c2.f16, st), "conv2")) return -1;
    }
    // appearance = the final 4x4 conv on the 4x4 map (one output pixel)
    const int Cl = c->cout[c->nb - 1];
    if (!c->hip_ok(launch_enc_linear(c->w_last, nullptr, c->lvl[c->nb], c->dim, 16 * Cl, c->last16, c->app, st),
                   "appearance"))
        return -1;
    const float *h = c->app;
    for (int i = 0; i < 5; i++) {
        const int O = i == 4 ? c->n_motion : c->dim;
        if (!c->hip_ok(launch_enc_linear(c->fc_w[i], c->fc_b[i], h, O, c->dim, c->fc16[i], c->fch[i], st), "fc"))
            return -1;
        h = c->fch[i];
    }
    if (!c->hip_ok(launch_enc_linear(c->q, nullptr, h, c->dim, c->n_motion, c->q16, c->motion, st), "motion"))
        return -1;
    if (!c->hip_ok(hipStreamSynchronize(st), "encoder sync")) return -1;
    c->ran = true;
    return 0;
}

int tpme_result(const tpme_ctx *cc, float *appearance, float *lambda, float *motion) {
    tpme_ctx *c = const_cast<tpme_ctx *>(cc);
    if (!check(c)) return -1;
    if (!c->ran) {
        c->err = "encoder has not run";
        return -1;
    }
    if (appearance && !c->hip_ok(hipMemcpy(appearance, c->app, (size_t) c->dim * 4, hipMemcpyDeviceToHost), "copy"))
        return -1;
    if (lambda && !c->hip_ok(hipMemcpy(lambda, c->fch[4], (size_t) c->n_motion * 4, hipMemcpyDeviceToHost), "copy"))
        return -1;
    if (motion && !c->hip_ok(hipMemcpy(motion, c->motion, (size_t) c->dim * 4, hipMemcpyDeviceToHost), "copy"))
        return -1;
    return 0;
}

const float *tpme_feat(const tpme_ctx *c, int j, int *C, int *r) {
    if (!c || !c->ran || j < 0 || j >= c->nb) return nullptr;
    const int l = c->nb - 1 - j;
    if (C) *C = c->level_ch(l);
    if (r) *r = c->level_res(l);
    return c->lvl[l];
}

static int64_t tpme_level_body(tpme_ctx *c, int level, float *dst) {
    if (!check(c)) return -1;
    if (level < 0 || level > c->nb) {
        c->err = "tpme_level: bad level";
        return -1;
    }
    const int64_t r = c->level_res(level), n = r * r * c->level_ch(level);
    if (!dst) return n;
    if (!c->ran) {
        c->err = "encoder has not run";
        return -1;
    }
    if (!c->hip_ok(hipMemcpy(dst, c->lvl[level], (size_t) n * 4, hipMemcpyDeviceToHost), "copy")) return -1;
    return n;
}


// ---- entry points that allocate host memory, exception-safe

tpme_ctx *tpme_create(int device, const char *ftype, int n_blocks, const int *ch_in, const int *ch_out) {
    return guarded((void *) nullptr, [&] { return tpme_create_body(device, ftype, n_blocks, ch_in, ch_out); });
}

int tpme_set_weight(tpme_ctx *c, const char *name, const float *data, int64_t n, int flags) {
    return guarded(c, [&] { return tpme_set_weight_body(c, name, data, n, flags); });
}

int tpme_prepare(tpme_ctx *c) {
    return guarded(c, [&] { return tpme_prepare_body(c); });
}

int tpme_run(tpme_ctx *c, const float *image, int on_device) {
    return guarded(c, [&] { return tpme_run_body(c, image, on_device); });
}

int64_t tpme_level(tpme_ctx *c, int level, float *dst) {
    return guarded(c, [&] { return tpme_level_body(c, level, dst); });
}

}  // extern "C"
