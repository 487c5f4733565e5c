// shim_check — drives tp::motion_dec (host/motion_dec.h) the way the
// reference's generation loop does (src/pipeline.cpp:153-185): prepare,
// build, set_feats, then decode_batch over a clip in `batch`-frame launches
// with the tail padded by repeating the last frame, plus one single-frame
// decode().  Inputs come from a little-endian blob file:
//
//   "TPMDBLOB" u32 n_stages, i32 ic[n], i32 oc[n], u32 ftype_f16,
//   u32 n_tensors, { u32 len, name, u8 f16_in_file, u64 n, f32 data[n] }...,
//   feats j < n_stages: f32 [r_j*r_j*OC_j],
//   u32 n_frames, f32 styles[n_frames][512]
//
// Output file: f32 frames [n_frames][3][R][R], then the single-frame decode
// of frame 0 [3][R][R].  Exit status 0 on success; errors on stderr.
//
//   shim_check <blob> <out> [device] [gguf] [image]
//
// With a GGUF path the weights come from that checkpoint through
// tp::gguf_weight_source (the reference's tp_load flow, src/tp.cpp:13-41)
// and the blob's weight section is ignored.  With an image file too (f32
// [3][512][512] CHW), tp::motion_enc runs on it and its menc_result replaces
// the blob's feats (the generation flow, src/pipeline.cpp:113-115); the
// output then ends with appearance [512], lambda [20] and motion [512].
//
// TPMD_SHIM_ALLOCS=<frames> in the environment: after the above, count the
// heap allocations (malloc / calloc / realloc, operator new included) that
// this thread makes in steady state, the way the reference's zero-allocation
// check does (bench/tp-allocproof.cpp:121-150): two warm-up decode() calls,
// then <frames> single-frame decode() calls, counted one by one; then two
// warm-up and 20 counted decode_batch() calls.  Printed as "allocs ..." lines.
#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "gguf.h"
#include "motion_dec.h"
#include "motion_enc.h"

// ---- counting allocator: allocations of the main thread while counting
// is on; every call goes on to glibc's own allocator
extern "C" void *__libc_malloc(size_t);
extern "C" void *__libc_calloc(size_t, size_t);
extern "C" void *__libc_realloc(void *, size_t);
extern "C" void __libc_free(void *);

namespace {
std::atomic<bool> g_counting{false};
std::atomic<long> g_allocs{0};
thread_local bool t_counted = false;
inline void note_alloc() {
    if (t_counted && g_counting.load(std::memory_order_relaxed)) g_allocs.fetch_add(1, std::memory_order_relaxed);
}
}  // namespace

extern "C" void *malloc(size_t n) {
    note_alloc();
    return __libc_malloc(n);
}
extern "C" void *calloc(size_t n, size_t m) {
    note_alloc();
    return __libc_calloc(n, m);
}
extern "C" void *realloc(void *p, size_t n) {
    note_alloc();
    return __libc_realloc(p, n);
}
extern "C" void free(void *p) { __libc_free(p); }

namespace {

struct reader {
    std::vector<uint8_t> b;
    size_t p = 0;
    bool ok = true;
    template <typename T>
    T get() {
        T v{};
        if (p + sizeof(T) > b.size()) {
            ok = false;
            return v;
        }
        memcpy(&v, b.data() + p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    bool bytes(void *dst, size_t n) {
        if (p + n > b.size()) return ok = false;
        memcpy(dst, b.data() + p, n);
        p += n;
        return true;
    }
};

struct blob_weights : tp::weight_source {
    struct t {
        std::vector<float> v;
        bool f16;
    };
    std::map<std::string, t> m;
    bool get(const std::string &name, std::vector<float> &data, bool &f16) const override {
        auto it = m.find(name);
        if (it == m.end()) return false;
        data = it->second.v;
        f16 = it->second.f16;
        return true;
    }
};

struct menc_like {  // the member of menc_result that set_feats reads
    std::vector<std::vector<float>> feats;
};

struct no_taps {
    explicit operator bool() const { return false; }
};

// the reference's tap_writer / tap_sink pair (src/dump.h:13-24,
// src/tp_internal.h:131-142) reduced to what motion_dec::decode uses: one raw
// little-endian .f32 file per tap and a line "name d0 d1 ..." per tap in
// meta.txt
struct dir_writer {
    std::string dir, err;
    FILE *meta = nullptr;
    bool add_f32(const std::string &name, const float *data, const std::vector<int64_t> &shape) {
        int64_t n = 1;
        for (int64_t d : shape) n *= d;
        FILE *f = fopen((dir + "/" + name + ".f32").c_str(), "wb");
        if (!f || fwrite(data, 4, (size_t) n, f) != (size_t) n) {
            err = "cannot write tap " + name;
            if (f) fclose(f);
            return false;
        }
        fclose(f);
        fprintf(meta, "%s", name.c_str());
        for (int64_t d : shape) fprintf(meta, " %lld", (long long) d);
        fprintf(meta, "\n");
        return true;
    }
};
struct dir_sink {
    dir_writer *wr = nullptr;
    std::string prefix;
    explicit operator bool() const { return wr != nullptr; }
};

}  // namespace

int main(int argc, char **argv) {
    if (argc < 3) {
        fprintf(stderr, "usage: shim_check <blob> <out> [device] [gguf] [image]\n");
        return 2;
    }
    reader r;
    {
        FILE *f = fopen(argv[1], "rb");
        if (!f) {
            fprintf(stderr, "cannot open %s\n", argv[1]);
            return 1;
        }
        fseek(f, 0, SEEK_END);
        r.b.resize((size_t) ftell(f));
        fseek(f, 0, SEEK_SET);
        if (fread(r.b.data(), 1, r.b.size(), f) != r.b.size()) r.ok = false;
        fclose(f);
    }
    char magic[8];
    if (!r.bytes(magic, 8) || memcmp(magic, "TPMDBLOB", 8) != 0) {
        fprintf(stderr, "bad blob\n");
        return 1;
    }
    tp::hip_backend be;
    be.device = argc > 3 ? atoi(argv[3]) : 0;
    be.n_stages = (int) r.get<uint32_t>();
    if (be.n_stages < 1 || be.n_stages > 7) return 1;
    be.stage_ic.resize((size_t) be.n_stages);
    be.stage_oc.resize((size_t) be.n_stages);
    for (auto &v : be.stage_ic) v = r.get<int32_t>();
    for (auto &v : be.stage_oc) v = r.get<int32_t>();
    be.ftype = r.get<uint32_t>() ? "f16" : "f32";
    blob_weights w;
    const uint32_t nt = r.get<uint32_t>();
    for (uint32_t i = 0; i < nt && r.ok; i++) {
        std::string name(r.get<uint32_t>(), '\0');
        r.bytes(&name[0], name.size());
        blob_weights::t t;
        t.f16 = r.get<uint8_t>() != 0;
        t.v.resize(r.get<uint64_t>());
        r.bytes(t.v.data(), t.v.size() * 4);
        w.m[name] = std::move(t);
    }
    menc_like m;
    for (int j = 0; j < be.n_stages; j++) {
        const size_t r2 = (size_t) (8 << j) * (8 << j);
        m.feats.emplace_back(r2 * (size_t) be.stage_oc[(size_t) j]);
        r.bytes(m.feats.back().data(), m.feats.back().size() * 4);
    }
    const uint32_t nf = r.get<uint32_t>();
    std::vector<float> styles((size_t) nf * 512);
    r.bytes(styles.data(), styles.size() * 4);
    if (!r.ok || nf == 0) {
        fprintf(stderr, "truncated blob\n");
        return 1;
    }

    tp::motion_dec dec;
    dec.w = &w;
    std::string err;
    tp::gguf_file gf;
    tp::gguf_weight_source gw;
    if (argc > 4) {
        if (!gf.open(argv[4], "float-motion-ae", err)) {
            fprintf(stderr, "shim_check: %s\n", err.c_str());
            return 1;
        }
        gw.f = &gf;
        dec.w = &gw;
    }
    tp::menc_result mr;
    const bool with_enc = argc > 5;
    if (with_enc) {
        std::vector<float> img((size_t) 3 * 512 * 512);
        FILE *fi = fopen(argv[5], "rb");
        if (!fi || fread(img.data(), 4, img.size(), fi) != img.size()) {
            fprintf(stderr, "cannot read image %s\n", argv[5]);
            return 1;
        }
        fclose(fi);
        tp::motion_enc enc;
        enc.w = dec.w;
        no_taps et;
        if (!enc.run(be, img.data(), mr, et, err)) {
            fprintf(stderr, "shim_check: %s\n", err.c_str());
            return 1;
        }
    }
    if (!dec.prepare(be, err) || !dec.build(be, false, err) ||
        !(with_enc ? dec.set_feats(mr, err) : dec.set_feats(m, err))) {
        fprintf(stderr, "shim_check: %s\n", err.c_str());
        return 1;
    }
    const int BQ = dec.batch;
    const size_t fsz = (size_t) 3 * dec.res * dec.res;
    std::vector<float> out((size_t) nf * fsz + fsz), bst((size_t) BQ * 512), bimg((size_t) BQ * fsz);
    for (uint32_t t0 = 0; t0 < nf; t0 += (uint32_t) BQ) {
        for (int b = 0; b < BQ; b++) {
            const uint32_t t = t0 + (uint32_t) b < nf ? t0 + (uint32_t) b : nf - 1;
            memcpy(bst.data() + (size_t) b * 512, styles.data() + (size_t) t * 512, 512 * 4);
        }
        if (!dec.decode_batch(be, bst.data(), bimg.data(), err)) {
            fprintf(stderr, "shim_check: %s\n", err.c_str());
            return 1;
        }
        const uint32_t nb = nf - t0 < (uint32_t) BQ ? nf - t0 : (uint32_t) BQ;
        memcpy(out.data() + (size_t) t0 * fsz, bimg.data(), (size_t) nb * fsz * 4);
    }
    no_taps tap;
    if (!dec.decode(be, styles.data(), out.data() + (size_t) nf * fsz, tap, err)) {
        fprintf(stderr, "shim_check: %s\n", err.c_str());
        return 1;
    }
    if (const char *na = std::getenv("TPMD_SHIM_ALLOCS")) {
        const int frames = atoi(na) > 0 ? atoi(na) : 100;
        std::vector<float> img(fsz);
        t_counted = true;
        auto counted = [&](auto &&call, long &total, long &worst) {
            g_allocs = 0;
            g_counting = true;
            const bool ok = call();
            g_counting = false;
            const long a = g_allocs.load();
            total += a;
            worst = a > worst ? a : worst;
            return ok;
        };
        long d_total = 0, d_worst = 0, b_total = 0, b_worst = 0, warm = 0, warm_worst = 0;
        bool ok = true;
        for (int f = 0; f < frames + 2 && ok; f++) {
            const float *st = styles.data() + (size_t) (f % (int) nf) * 512;
            auto call = [&] { return dec.decode(be, st, img.data(), tap, err); };
            ok = f < 2 ? counted(call, warm, warm_worst) : counted(call, d_total, d_worst);
        }
        const int calls = 20;
        for (int k = 0; k < calls + 2 && ok; k++) {
            auto call = [&] { return dec.decode_batch(be, bst.data(), bimg.data(), err); };
            ok = k < 2 ? counted(call, warm, warm_worst) : counted(call, b_total, b_worst);
        }
        t_counted = false;
        if (!ok) {
            fprintf(stderr, "shim_check allocs: %s\n", err.c_str());
            return 1;
        }
        printf("allocs decode: %ld over %d frames, max %ld per frame\n", d_total, frames, d_worst);
        printf("allocs decode_batch: %ld over %d calls of %d frames, max %ld per call\n", b_total, calls, BQ,
               b_worst);
    }
    // TPMD_SHIM_TAPS=<dir>: the tap plan of the first style, as tools/tp-parity
    // asks for it (build with taps, then decode with a tap sink), its taps in
    // <dir> and its frame appended to the output
    if (const char *tdir = std::getenv("TPMD_SHIM_TAPS")) {
        dir_writer wr;
        wr.dir = tdir;
        wr.meta = fopen((wr.dir + "/meta.txt").c_str(), "w");
        dir_sink ts;
        ts.wr = &wr;
        ts.prefix = "mdec.f0.";
        std::vector<float> timg(fsz);
        if (!wr.meta || !dec.build(be, true, err) || !dec.set_feats(m, err) ||
            !dec.decode(be, styles.data(), timg.data(), ts, err)) {
            fprintf(stderr, "shim_check taps: %s\n", wr.meta ? err.c_str() : "cannot open meta.txt");
            return 1;
        }
        fclose(wr.meta);
        out.insert(out.end(), timg.begin(), timg.end());
    }
    if (with_enc) {
        out.insert(out.end(), mr.appearance.begin(), mr.appearance.end());
        out.insert(out.end(), mr.lambda.begin(), mr.lambda.end());
        out.insert(out.end(), mr.motion.begin(), mr.motion.end());
    }
    FILE *f = fopen(argv[2], "wb");
    if (!f || fwrite(out.data(), 4, out.size(), f) != out.size()) {
        fprintf(stderr, "cannot write %s\n", argv[2]);
        return 1;
    }
    fclose(f);
    printf("shim_check: %u frames in batches of %d, %d stages, ftype %s\n", nf, BQ, be.n_stages,
           be.ftype.c_str());
    return 0;
}
