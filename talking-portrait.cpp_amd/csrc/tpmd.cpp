// Host side of the MI355X motion decoder: the C ABI of include/tpmd.h.
//
// Mirrors the reference's motion_dec lifecycle (src/motion_dec.h:34-47):
//   set_weight* -> prepare -> build -> set_feats -> decode_batch ...
// prepare() restates src/motion_dec.cpp:31-226 (S_aug, composed sub-pixel
// kernels, cf GEMM matrices) and the load-time folding of
// src/motion_enc.cpp:14-45 / src/gguf_load.cpp:146-194; decode_batch()
// enqueues the whole batched decoder on one HIP stream:
//   style GEMV, demod, conv1 input, conv1,
//   then per stage j: sub-pixel up-conv, dense conv, fused tail.
#include "tpmd_guard.h"
#include "tpmd.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <new>
#include <atomic>
#include <condition_variable>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include <sched.h>

#include "tpmd_launch.h"

using namespace tpmd;

// The scratch of tpmd_modconv_static, one array per GPU, held by every GPU the
// library runs on until the process ends.  On the host the name is only a
// stand-in for the symbol: each device's address comes from
// hipGetSymbolAddress (static_scratch_of), and only that address is used.
static __device__ __align__(256) char scratch[TPMD_STATIC_SCRATCH_BYTES];

namespace {

// the device address of `scratch` on `device`, which must be current;
// resolved on the first call for each device and kept (null + reason in err
// on failure)
constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void *scratch_dev[kMaxDevices] = {};
void *static_scratch_of(int device, std::string &err) {
    if (device < 0 || device >= kMaxDevices) {
        err = "device ordinal out of range";
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(scratch_mu);
    if (!scratch_dev[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            err = std::string("hipGetSymbolAddress: ") + hipGetErrorString(e);
            return nullptr;
        }
        scratch_dev[device] = p;
    }
    return scratch_dev[device];
}

const int REF_IC[7] = {512, 512, 512, 512, 256, 128, 64};
const int REF_OC[7] = {512, 512, 512, 256, 128, 64, 32};

struct HostTensor {
    std::vector<float> data;  // scale-folded f32
    int flags = 0;
};

// helper threads for the frame path's host copies out of the pinned slots
// (one thread copies ~5-10 GB/s, less than the decoder produces frames; the
// pool takes the CPUs of the process's affinity, up to 16 with the caller):
// made by the first tpmd_decode_frames call and kept by the context, so later
// calls allocate nothing; a copy is split in parts that the helpers and the
// calling thread take in turn
struct CopyPool {
    std::vector<std::thread> th;
    std::mutex m;
    std::condition_variable go, done;
    char *dst = nullptr;
    const char *src = nullptr;
    size_t bytes = 0, part = 0;
    int nparts = 0, finished = 0;
    std::atomic<int> next{0};
    unsigned gen = 0;
    bool quit = false;

    explicit CopyPool(int n) {
        for (int i = 0; i < n; i++) th.emplace_back([this] { loop(); });
    }
    ~CopyPool() {
        {
            std::lock_guard<std::mutex> lk(m);
            quit = true;
        }
        go.notify_all();
        for (auto &t : th) t.join();
    }
    void work() {
        for (;;) {
            const int i = next.fetch_add(1);
            if (i >= nparts) return;
            const size_t b0 = (size_t) i * part;
            memcpy(dst + b0, src + b0, std::min(part, bytes - b0));
        }
    }
    void loop() {
        unsigned seen = 0;
        std::unique_lock<std::mutex> lk(m);
        for (;;) {
            go.wait(lk, [&] { return quit || gen != seen; });
            if (quit) return;
            seen = gen;
            lk.unlock();
            work();
            lk.lock();
            if (++finished == (int) th.size()) done.notify_one();
        }
    }
    void copy(char *d, const char *s_, size_t n) {
        if (th.empty() || n < ((size_t) 2 << 20)) {
            memcpy(d, s_, n);
            return;
        }
        {
            std::lock_guard<std::mutex> lk(m);
            dst = d;
            src = s_;
            bytes = n;
            part = (n / (th.size() + 1) + 4095) & ~(size_t) 4095;
            nparts = (int) ((n + part - 1) / part);
            next = 0;
            finished = 0;
            ++gen;
        }
        go.notify_all();
        work();
        std::unique_lock<std::mutex> lk(m);
        done.wait(lk, [&] { return finished == (int) th.size(); });
    }
};

struct ConvW {
    int ic = 0, oc = 0;
    bool up = false;
    void *A = nullptr;         // act [M][9*IC], M = oc or 4*oc
    void *A_perm = nullptr;    // act: A in the order modconv_a_order names for the decode shape, or null
    float *bias = nullptr;     // [oc] activate.bias (x sqrt2)
    int64_t saug_off = 0;      // into saug_all, [oc][ic+1]
    int seg = 0;               // style segment
    int64_t s_off = 0, d_off = 0;  // [batch][ic] / [batch][oc] blocks (set at build)
};

struct StageW {
    float *wflow = nullptr, *fbias = nullptr, *fup = nullptr;
    float *wrgb = nullptr, *rlb = nullptr, *rbias = nullptr, *rup = nullptr;
    float *lin = nullptr;
    void *feat = nullptr;      // act [r*r][oc]
    float *featg = nullptr;    // [r*r][4] ToRGB weight . feat
    int seg = 0;
    int64_t s_off = 0;
};

std::string fmt(const char *f, ...) __attribute__((format(printf, 1, 2)));
std::string fmt(const char *f, ...) {
    char b[512];
    va_list ap;
    va_start(ap, f);
    vsnprintf(b, sizeof b, f, ap);
    va_end(ap);
    return b;
}

float round_f16(float v) { return (float) (_Float16) v; }

}  // namespace

struct tpmd_ctx {
    int device = 0;
    bool f16 = false;
    int ns = 7;
    int ic[7] = {}, oc[7] = {};
    std::string err;
    hipStream_t stream = nullptr;     // the stream all work is enqueued on
    hipStream_t own_stream = nullptr; // created by tpmd_create

    std::map<std::string, HostTensor> host;
    std::vector<std::pair<std::string, std::vector<int64_t>>> tensors;  // expected inputs
    bool prepared = false, built = false, feats_set = false;
    std::vector<void *> allocs;      // weights / constants
    std::vector<void *> batch_allocs;

    ConvW conv[15];
    StageW st[7];
    int nconv = 0;
    float *wmod = nullptr, *bmod = nullptr;  // [R][512], [R]
    int seg_width[kMaxSeg] = {};
    int nseg = 0, R_total = 0;
    float *input_cl = nullptr;        // [16][C0]
    float *saug_all = nullptr;
    SegTable seg{};
    DemodTable dem{};

    int batch = 0;
    // per-batch buffers of one launch chain.  Device-resident decodes on the
    // library's own stream rotate over kLanes lanes, each with its own
    // buffers and stream, so consecutive batches overlap on the GPU
    // (measured at 16 frames: 2 lanes 9.9k frames/s, 3 lanes 10.05k, 4 lanes 9.8k;
    // with later kernels 3 lanes 12.36k, 4 lanes 11.98k, 5 lanes 11.77k)
    static constexpr int kLanes = 3;
    struct Lane {
        float *lat = nullptr, *s_all = nullptr, *den_all = nullptr;
        void *xs0 = nullptr, *c1 = nullptr, *trunk = nullptr;
        float *outb = nullptr, *flow[2] = {}, *rgb[2] = {}, *img = nullptr;
        float *ws = nullptr;          // split-K partials of the low-resolution convs
        int64_t ws_elems = 0;
    } lane[kLanes];
    Lane *L = &lane[0];               // the lane the enqueued work uses
    hipStream_t lane_stream[kLanes] = {};  // lanes 1.. (lane 0 runs on `stream`)
    int next_lane = 0;
    // ordering of the lanes' device-resident decodes:
    //   ev_in[k]   recorded on the null stream as a call starts; lane k waits
    //              for it before reading the latents (prior null-stream
    //              writers of the latents come first)
    //   ev_read[k] lane k has copied the call's latents; the null stream
    //              waits for it (later null-stream writers of that buffer
    //              come after the read)
    //   ev_done[k] lane k's launch chain has finished (frames written); a
    //              call whose frame buffer overlaps lane k's last one waits
    //              for it before writing frames
    hipEvent_t ev_in[kLanes] = {}, ev_read[kLanes] = {}, ev_done[kLanes] = {};
    struct OutRange {
        const char *lo = nullptr, *hi = nullptr;
    } lane_out[kLanes];

    // device copies of the decode chain's intermediate buffers
    // (tpmd_set_tap), index [kind][stage + 1]
    struct Tap {
        void *dst = nullptr;
        int64_t bytes = 0;
    } taps[TPMD_TAP_KINDS][TPMD_MAX_STAGES + 1];
    bool any_tap = false;

    // scratch for the per-stage entry points (grow-only)
    void *scr[13] = {};
    size_t scr_sz[13] = {};
    // this device's static scratch (tpmd_modconv_static), or null + reason
    void *static_scratch = nullptr;
    std::string static_scratch_err;

    bool profile = false;

    // each lane's launch chain captured as HIP graphs, one per (frames,
    // frame buffer) in use, replayed with one launch; kGraphs per lane, the
    // least recently used replaced (TPMD_GRAPHS=0 in the environment, or
    // tpmd_set_graphs, turns them off)
    bool use_graphs = true;
    static constexpr int kGraphs = 4;
    struct Graph {
        hipGraphExec_t exec = nullptr;
        int n = 0;
        const float *dst = nullptr;
        uint64_t used = 0;
    } graphs[kLanes][kGraphs];
    uint64_t graph_clock = 0;
    void drop_graphs() {
        for (auto &lg : graphs)
            for (auto &g : lg) {
                if (g.exec) (void) hipGraphExecDestroy(g.exec);
                g = Graph{};
            }
    }

    // frame streaming (tpmd_decode_frames): one device frame slot per lane,
    // pinned host staging, a copy stream and events; made by the first call
    struct {
        hipStream_t copy = nullptr;
        hipEvent_t computed[kLanes] = {}, copied[kLanes] = {};
        void *dev[kLanes] = {}, *host[kLanes] = {};
        size_t bytes = 0;  // per slot
        std::unique_ptr<CopyPool> pool;
    } fs;
    std::vector<hipEvent_t> ev;
    std::vector<float> times;

    size_t act_size() const { return f16 ? 2 : 4; }
    int out_res() const { return 8 << (ns - 1); }

    bool hip_ok(hipError_t e, const char *what) {
        if (e == hipSuccess) return true;
        err = fmt("%s: %s", what, hipGetErrorString(e));
        return false;
    }
    void *dalloc(size_t bytes, std::vector<void *> &list) {
        void *p = nullptr;
        if (hipMalloc(&p, bytes < 256 ? 256 : bytes) != hipSuccess) {
            err = fmt("hipMalloc of %zu bytes failed", bytes);
            return nullptr;
        }
        list.push_back(p);
        return p;
    }
    template <typename T>
    T *upload(const std::vector<T> &v) {
        T *p = (T *) dalloc(v.size() * sizeof(T), allocs);
        if (!p) return nullptr;
        if (!hip_ok(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice), "upload"))
            return nullptr;
        return p;
    }
    // f32 values -> device act tensor (f16 RNE in f16 mode)
    void *upload_act(const std::vector<float> &v) {
        if (!f16) return upload(v);
        std::vector<_Float16> h(v.size());
        for (size_t i = 0; i < v.size(); i++) h[i] = (_Float16) v[i];
        return upload(h);
    }
    const HostTensor *need(const std::string &name) {
        auto it = host.find(name);
        if (it == host.end()) {
            if (err.empty()) err = "missing tensor " + name;
            return nullptr;
        }
        return &it->second;
    }
    // device value of a tensor under the f16 keep rule (src/gguf_load.cpp:149-153)
    std::vector<float> dev_value(const HostTensor &t) const {
        std::vector<float> v = t.data;
        if (f16 && (t.flags & TPMD_W_F16_FILE) && v.size() >= 4096)
            for (auto &x : v) x = round_f16(x);
        return v;
    }
    void *scratch(int i, size_t bytes) {
        if (scr_sz[i] < bytes) {
            if (scr[i]) (void) hipFree(scr[i]);
            scr[i] = nullptr;
            scr_sz[i] = 0;
            if (hipMalloc(&scr[i], bytes) != hipSuccess) {
                err = fmt("hipMalloc of %zu bytes failed", bytes);
                return nullptr;
            }
            scr_sz[i] = bytes;
        }
        return scr[i];
    }

    std::string conv_name(int L) const {
        return L == 0 ? std::string("dec.conv1") : fmt("dec.convs.%d", L - 1);
    }

    ~tpmd_ctx() {
        if (device >= 0) (void) hipSetDevice(device);
        for (hipStream_t ls : lane_stream)
            if (ls) (void) hipStreamSynchronize(ls);
        if (own_stream) (void) hipStreamSynchronize(own_stream);
        drop_graphs();
        for (auto e : ev) (void) hipEventDestroy(e);
        for (void *p : allocs) (void) hipFree(p);
        for (void *p : batch_allocs) (void) hipFree(p);
        for (void *p : scr)
            if (p) (void) hipFree(p);
        for (int i = 0; i < kLanes; i++) {
            if (fs.dev[i]) (void) hipFree(fs.dev[i]);
            if (fs.host[i]) (void) hipHostFree(fs.host[i]);
            if (fs.computed[i]) (void) hipEventDestroy(fs.computed[i]);
            if (fs.copied[i]) (void) hipEventDestroy(fs.copied[i]);
        }
        if (fs.copy) (void) hipStreamDestroy(fs.copy);
        for (int i = 0; i < kLanes; i++)
            for (hipEvent_t e : {ev_in[i], ev_read[i], ev_done[i]})
                if (e) (void) hipEventDestroy(e);
        if (own_stream) (void) hipStreamDestroy(own_stream);
        for (hipStream_t ls : lane_stream)
            if (ls) (void) hipStreamDestroy(ls);
    }
};

namespace {

// motion_ae_scale restricted to dec.* tensors (src/motion_enc.cpp:14-45);
// ne is the ggml order (reversed torch shape)
double motion_ae_scale(const std::string &name, const std::vector<int64_t> &ne) {
    const double SQRT2 = 1.4142135623730951;
    auto ends_with = [&](const char *s) {
        size_t n = strlen(s);
        return name.size() >= n && name.compare(name.size() - n, n, s) == 0;
    };
    if (ends_with(".activate.bias") || (name.rfind("dec.to_rgbs.", 0) == 0 && ends_with(".conv.1.bias")))
        return SQRT2;
    if (!ends_with(".weight")) return 1.0;
    if (name.rfind("dec.direction", 0) == 0 || ends_with("noise.weight")) return 1.0;
    if (ends_with("modulation.weight")) return 1.0 / sqrt((double) ne[0]);
    const double conv = 1.0 / sqrt((double) (ne[0] * ne[1] * ne[2]));
    if (name.rfind("dec.to_rgbs.", 0) == 0 && ends_with(".conv.0.weight")) return conv * SQRT2;
    if (ends_with(".conv.weight")) return conv;
    return 1.0;
}

// every decoder tensor of this config with its torch shape, in GGUF names
// (src/motion_dec.cpp:17-29, :249-261; shapes as tests/test_gguf.cpp:54-58)
std::vector<std::pair<std::string, std::vector<int64_t>>> tensor_list(const tpmd_ctx *c) {
    std::vector<std::pair<std::string, std::vector<int64_t>>> v;
    const int64_t C0 = c->ic[0];
    v.push_back({"dec.input.input", {1, C0, 4, 4}});
    v.push_back({"dec.conv1.conv.weight", {1, C0, C0, 3, 3}});
    v.push_back({"dec.conv1.conv.modulation.weight", {C0, 512}});
    v.push_back({"dec.conv1.conv.modulation.bias", {C0}});
    v.push_back({"dec.conv1.activate.bias", {C0}});
    for (int j = 0; j < c->ns; j++) {
        for (int i = 2 * j; i <= 2 * j + 1; i++) {
            const int64_t cin = (i % 2 == 0) ? c->ic[j] : c->oc[j], cout = c->oc[j];
            const std::string b = fmt("dec.convs.%d", i);
            v.push_back({b + ".conv.weight", {1, cout, cin, 3, 3}});
            v.push_back({b + ".conv.modulation.weight", {cin, 512}});
            v.push_back({b + ".conv.modulation.bias", {cin}});
            v.push_back({b + ".activate.bias", {cout}});
            if (i % 2 == 0) v.push_back({b + ".conv.blur.kernel", {4, 4}});
        }
        const int64_t C = c->oc[j];
        const std::string f = fmt("dec.to_flows.%d", j), r = fmt("dec.to_rgbs.%d", j);
        v.push_back({f + ".conv.weight", {1, 3, C, 1, 1}});
        v.push_back({f + ".conv.modulation.weight", {C, 512}});
        v.push_back({f + ".conv.modulation.bias", {C}});
        v.push_back({f + ".bias", {1, 3, 1, 1}});
        v.push_back({f + ".upsample.kernel", {4, 4}});
        v.push_back({r + ".conv.0.weight", {3, C, 1, 1}});
        v.push_back({r + ".conv.1.bias", {3}});
        v.push_back({r + ".bias", {1, 3, 1, 1}});
        v.push_back({r + ".upsample.kernel", {4, 4}});
    }
    return v;
}

bool expected_shape(const tpmd_ctx *c, const std::string &name, std::vector<int64_t> &shape) {
    for (const auto &t : c->tensors)
        if (t.first == name) {
            shape = t.second;
            return true;
        }
    return false;
}

// dense cf GEMM matrix A[o][ic + IC*(kw + 3*kh)] (src/motion_dec.cpp:132-143)
std::vector<float> make_acf(const std::vector<float> &W, int OC, int IC) {
    const size_t R = (size_t) IC * 9;
    std::vector<float> a((size_t) OC * R);
    for (int o = 0; o < OC; o++)
        for (int i = 0; i < IC; i++)
            for (int kh = 0; kh < 3; kh++)
                for (int kw = 0; kw < 3; kw++)
                    a[(size_t) o * R + i + (size_t) IC * (kw + 3 * kh)] =
                        W[((size_t) o * IC + i) * 9 + kh * 3 + kw];
    return a;
}

// conv_transpose(3x3, s2) o Blur(4x4) as four 3x3 pad-1 kernels, one per
// output parity class (by, bx); rows q = (2*by + bx)*OC + o, columns cf
// ordered; double accumulation (src/motion_dec.cpp:144-186)
std::vector<float> make_tsub(const std::vector<float> &W, const std::vector<float> &BK, int OC,
                             int IC) {
    const size_t R = (size_t) IC * 9;
    std::vector<float> t((size_t) 4 * OC * R, 0.0f);
    for (int o = 0; o < OC; o++)
        for (int i = 0; i < IC; i++) {
            const float *w = W.data() + ((size_t) o * IC + i) * 9;
            for (int by = 0; by < 2; by++)
                for (int bx = 0; bx < 2; bx++) {
                    float *dst = t.data() + (size_t) ((2 * by + bx) * OC + o) * R;
                    for (int ty = 0; ty < 3; ty++)
                        for (int tx = 0; tx < 3; tx++) {
                            const int dy = 1 - ty, dx = 1 - tx;
                            double acc = 0;
                            for (int cy = 0; cy < 3; cy++) {
                                const int ay = 3 - by - 2 * dy - cy;
                                if (ay < 0 || ay > 3) continue;
                                for (int cx = 0; cx < 3; cx++) {
                                    const int ax = 3 - bx - 2 * dx - cx;
                                    if (ax < 0 || ax > 3) continue;
                                    // flipped weight V[cy][cx] = W[2-cy][2-cx]
                                    acc += (double) w[(2 - cy) * 3 + (2 - cx)] * (double) BK[ay * 4 + ax];
                                }
                            }
                            dst[i + (size_t) IC * (tx + 3 * ty)] = (float) acc;
                        }
                }
        }
    return t;
}

// S_aug (src/motion_dec.cpp:113-122): [OC][IC] 0.5*sum_k W^2 (double), then
// the [OC] last column 0.5e-8 (folds the FusedLeakyReLU sqrt2 into 1/den);
// rows of IC floats keep every row 16-byte aligned for the demod kernel
std::vector<float> make_saug(const std::vector<float> &W, int OC, int IC) {
    std::vector<float> s((size_t) OC * (IC + 1));
    for (int o = 0; o < OC; o++) {
        for (int i = 0; i < IC; i++) {
            double a = 0;
            const float *w = W.data() + ((size_t) o * IC + i) * 9;
            for (int k = 0; k < 9; k++) a += (double) w[k] * w[k];
            s[(size_t) o * IC + i] = (float) (a * 0.5);
        }
        s[(size_t) OC * IC + o] = 0.5e-8f;
    }
    return s;
}

// A [M][K = 9*IC] (tap-major k) -> the LDS ring's DMA order [M/16][T = K/32][64][8]:
// block (g, t), lane i = row 16g + i/4, chunk (i%4) ^ swz(row) of k tile t
// (the row-swizzled LDS image the DMA writes)
std::vector<float> dma_image(const std::vector<float> &ck, int M, int IC) {
    const size_t K = (size_t) 9 * IC;
    const int T = 9 * IC / 32;
    std::vector<float> out(ck.size());
    for (int g = 0; g < M / 16; g++)
        for (int t = 0; t < T; t++)
            for (int i = 0; i < 64; i++) {
                const int row = g * 16 + i / 4;
                const int chunk = (i % 4) ^ (((row >> 2) ^ (row >> 3)) & 3);
                for (int e = 0; e < 8; e++)
                    out[(((size_t) g * T + t) * 64 + i) * 8 + e] = ck[row * K + (size_t) t * 32 + chunk * 8 + e];
            }
    return out;
}

// A [M][9*IC] (k = tap*IC + ic) -> MFMA fragment order [9][IC/16][M/32][64][8]:
// fragment (tap, ks) of row block w, lane l = row 32w + l%32, k = tap*IC + ks*16 + (l/32)*8 + e
std::vector<float> fragment_order(const std::vector<float> &A, int M, int IC) {
    const size_t K = (size_t) 9 * IC;
    const int KS = IC / 16, MB = M / 32;
    std::vector<float> out(A.size());
    for (int tap = 0; tap < 9; tap++)
        for (int ks = 0; ks < KS; ks++)
            for (int w = 0; w < MB; w++)
                for (int l = 0; l < 64; l++)
                    for (int e = 0; e < 8; e++)
                        out[((((size_t) tap * KS + ks) * MB + w) * 64 + l) * 8 + e] =
                            A[(size_t) (w * 32 + l % 32) * K + (size_t) tap * IC + ks * 16 + (l / 32) * 8 + e];
    return out;
}

bool check_ctx(tpmd_ctx *c) {
    if (!c) return false;
    c->err.clear();
    if (hipSetDevice(c->device) != hipSuccess) {
        c->err = "hipSetDevice failed";
        return false;
    }
    return true;
}

// dense convs whose output channels fit one conv tile run the stage tail in
// their epilogue (the stage output never goes to HBM)
bool fused_tail(const tpmd_ctx *c, int oc, int r) { return modconv_fusable(oc, r, c->f16); }

// work of the other lanes finished (before anything that rewrites shared
// state or hands results back through lane 0 alone)
bool drain_lanes(tpmd_ctx *c) {
    for (hipStream_t ls : c->lane_stream)
        if (ls && !c->hip_ok(hipStreamSynchronize(ls), "lane sync")) return false;
    return true;
}

// every lane finished, lane 0's own stream included (before work moves to
// another stream, which then uses lane 0's buffers)
bool drain_all(tpmd_ctx *c) {
    return drain_lanes(c) && c->hip_ok(hipStreamSynchronize(c->own_stream), "lane sync");
}

// stage entry points run on the caller's stream; NULL is HIP's null stream
hipStream_t pick_stream(tpmd_ctx *, void *s) { return (hipStream_t) s; }

}  // namespace

// ===========================================================================
extern "C" {

int tpmd_abi_version(void) { return TPMD_ABI_VERSION; }

static tpmd_ctx *tpmd_create_body(int device, const char *ftype, int n_stages, const int *stage_ic,
                      const int *stage_oc) {
    const std::string ft = ftype ? ftype : "f32";
    if (ft != "f32" && ft != "f16") {
        fprintf(stderr, "tpmd_create: ftype must be f32 or f16\n");
        return nullptr;
    }
    if (n_stages < 1 || n_stages > TPMD_MAX_STAGES) {
        fprintf(stderr, "tpmd_create: n_stages must be 1..7\n");
        return nullptr;
    }
    if ((stage_ic == nullptr) != (stage_oc == nullptr)) {
        fprintf(stderr, "tpmd_create: give both stage_ic and stage_oc or neither\n");
        return nullptr;
    }
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev) {
        fprintf(stderr, "tpmd_create: no HIP device %d\n", device);
        return nullptr;
    }
    tpmd_ctx *c = new (std::nothrow) tpmd_ctx();
    if (!c) return nullptr;
    c->device = device;
    c->f16 = ft == "f16";
    c->ns = n_stages;
    for (int j = 0; j < 7; j++) {
        c->ic[j] = stage_ic ? (j < n_stages ? stage_ic[j] : 0) : REF_IC[j];
        c->oc[j] = stage_oc ? (j < n_stages ? stage_oc[j] : 0) : REF_OC[j];
    }
    const int kal = modconv_k_align(c->f16);
    for (int j = 0; j < n_stages; j++) {
        const int C = c->oc[j];
        const bool c_ok = C == 32 || C == 64 || C == 128 || C == 256 || C == 512;
        const bool ic_ok = c->ic[j] % kal == 0 && c->ic[j] % 32 == 0 && c->ic[j] >= 32;
        const bool chain_ok = j == 0 || c->ic[j] == c->oc[j - 1];
        if (!c_ok || !ic_ok || !chain_ok) {
            fprintf(stderr,
                    "tpmd_create: stage %d channels %d->%d unsupported (OC in {32..512} powers of "
                    "two, IC multiple of 32, IC[j] == OC[j-1])\n",
                    j, c->ic[j], c->oc[j]);
            delete c;
            return nullptr;
        }
    }
    c->tensors = tensor_list(c);
    bool streams = hipSetDevice(device) == hipSuccess &&
                   hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking) == hipSuccess;
    for (int i = 1; i < tpmd_ctx::kLanes && streams; i++)
        streams = hipStreamCreateWithFlags(&c->lane_stream[i], hipStreamNonBlocking) == hipSuccess;
    for (int i = 0; i < tpmd_ctx::kLanes && streams; i++)
        streams = hipEventCreateWithFlags(&c->ev_in[i], hipEventDisableTiming) == hipSuccess &&
                  hipEventCreateWithFlags(&c->ev_read[i], hipEventDisableTiming) == hipSuccess &&
                  hipEventCreateWithFlags(&c->ev_done[i], hipEventDisableTiming) == hipSuccess;
    if (!streams) {
        fprintf(stderr, "tpmd_create: stream or event creation failed\n");
        delete c;
        return nullptr;
    }
    c->stream = c->own_stream;
    c->static_scratch = static_scratch_of(device, c->static_scratch_err);
    if (const char *g = std::getenv("TPMD_GRAPHS")) c->use_graphs = std::strcmp(g, "0") != 0;
    return c;
}

void tpmd_destroy(tpmd_ctx *c) { delete c; }

const char *tpmd_last_error(const tpmd_ctx *c) { return c ? c->err.c_str() : "no context"; }

static int tpmd_set_weight_body(tpmd_ctx *c, const char *name, const float *data, int64_t n, int flags) {
    if (!check_ctx(c)) return -1;
    if (!name || !data || n <= 0) {
        c->err = "tpmd_set_weight: null name/data or empty tensor";
        return -1;
    }
    std::vector<int64_t> shape;
    if (!expected_shape(c, name, shape)) {
        c->err = fmt("tpmd_set_weight: unknown decoder tensor %s", name);
        return -1;
    }
    int64_t want = 1;
    for (auto d : shape) want *= d;
    if (want != n) {
        c->err = fmt("tpmd_set_weight: %s has %lld elements, expected %lld", name, (long long) n,
                     (long long) want);
        return -1;
    }
    std::vector<int64_t> ne(shape.rbegin(), shape.rend());
    // the loader drops unit dims beyond 4 (src/gguf_load.cpp:111-124)
    while (ne.size() > 4 && ne.back() == 1) ne.pop_back();
    while (ne.size() < 4) ne.push_back(1);
    HostTensor t;
    t.data.assign(data, data + n);
    t.flags = flags;
    if (!(flags & TPMD_W_FOLDED)) {
        const double s = motion_ae_scale(name, ne);
        if (s != 1.0) {
            const float fs = (float) s;
            for (auto &v : t.data) v *= fs;
        }
    }
    c->host[name] = std::move(t);
    c->prepared = false;
    return 0;
}

const char *tpmd_weight_name(const tpmd_ctx *c, int i, int64_t *n, int *is_matrix) {
    if (!c || i < 0 || i >= (int) c->tensors.size()) return nullptr;
    const auto &t = c->tensors[(size_t) i];
    int64_t e = 1;
    for (auto d : t.second) e *= d;
    if (n) *n = e;
    if (is_matrix) *is_matrix = t.second.size() >= 2 ? 1 : 0;
    return t.first.c_str();
}

static int tpmd_prepare_body(tpmd_ctx *c) {
    if (!check_ctx(c)) return -1;
    if (!drain_all(c)) return -1;
    c->drop_graphs();
    for (void *p : c->allocs) (void) hipFree(p);
    c->allocs.clear();
    c->prepared = false;
    const int ns = c->ns, C0 = c->ic[0];

    // ---- convs: conv1 + 2 per stage
    c->nconv = 1 + 2 * ns;
    std::vector<float> saug_all, wmod, bmod;
    int seg = 0;
    c->R_total = 0;
    auto add_style = [&](const std::string &base, int width) -> int {
        const HostTensor *mw = c->need(base + ".modulation.weight");
        const HostTensor *mb = c->need(base + ".modulation.bias");
        if (!mw || !mb) return -1;
        std::vector<float> v = c->dev_value(*mw);
        wmod.insert(wmod.end(), v.begin(), v.end());
        bmod.insert(bmod.end(), mb->data.begin(), mb->data.end());
        c->seg_width[seg] = width;
        c->R_total += width;
        return seg++;
    };
    for (int L = 0; L < c->nconv; L++) {
        ConvW &cv = c->conv[L];
        const std::string base = c->conv_name(L);
        const int j = (L - 1) / 2;
        cv.up = L > 0 && (L - 1) % 2 == 0;
        cv.ic = L == 0 ? C0 : (cv.up ? c->ic[j] : c->oc[j]);
        cv.oc = L == 0 ? C0 : c->oc[j];
        const HostTensor *W = c->need(base + ".conv.weight");
        const HostTensor *ab = c->need(base + ".activate.bias");
        if (!W || !ab) return -1;
        cv.seg = add_style(base + ".conv", cv.ic);
        if (cv.seg < 0) return -1;
        std::vector<float> sa = make_saug(W->data, cv.oc, cv.ic);
        cv.saug_off = (int64_t) saug_all.size();
        saug_all.insert(saug_all.end(), sa.begin(), sa.end());
        std::vector<float> A;
        if (cv.up) {
            const HostTensor *bk = c->need(base + ".conv.blur.kernel");
            if (!bk) return -1;
            A = make_tsub(W->data, bk->data, cv.oc, cv.ic);
        } else {
            // conv1 uses its weight tensor as stored (f16-kept values); the
            // dense convs use the derived acf (f16 whenever ftype is f16)
            std::vector<float> wv = L == 0 ? c->dev_value(*W) : W->data;
            A = make_acf(wv, cv.oc, cv.ic);
        }
        cv.A = c->upload_act(A);
        // input map of the conv: 4 x 4 for conv1, r/2 for stage j's up-conv, r for its dense conv
        const int hin = L == 0 ? 4 : (cv.up ? 4 << j : 8 << j);
        const int order = modconv_a_order(c->f16, true, cv.up ? 1 : 0, cv.ic, cv.oc, hin, hin);
        if (order != A_ORDER_TAP) {
            const int M = cv.up ? 4 * cv.oc : cv.oc;
            cv.A_perm = c->upload_act(order == A_ORDER_RING_TAP ? dma_image(A, M, cv.ic) : fragment_order(A, M, cv.ic));
            if (!cv.A_perm) return -1;
        }
        cv.bias = c->upload(ab->data);
        if (!cv.A || !cv.bias) return -1;
    }
    for (int j = 0; j < ns; j++) {
        StageW &s = c->st[j];
        const int C = c->oc[j], r = 8 << j;
        const std::string f = fmt("dec.to_flows.%d", j), rb = fmt("dec.to_rgbs.%d", j);
        const HostTensor *fw = c->need(f + ".conv.weight"), *fb = c->need(f + ".bias"),
                         *fu = c->need(f + ".upsample.kernel"), *rw = c->need(rb + ".conv.0.weight"),
                         *rl = c->need(rb + ".conv.1.bias"), *rbs = c->need(rb + ".bias"),
                         *ru = c->need(rb + ".upsample.kernel");
        if (!fw || !fb || !fu || !rw || !rl || !rbs || !ru) return -1;
        s.seg = add_style(f + ".conv", C);
        if (s.seg < 0) return -1;
        s.wflow = c->upload(c->dev_value(*fw));
        s.fbias = c->upload(fb->data);
        s.fup = c->upload(fu->data);
        s.wrgb = c->upload(c->dev_value(*rw));
        s.rlb = c->upload(rl->data);
        s.rbias = c->upload(rbs->data);
        s.rup = c->upload(ru->data);
        std::vector<float> lin((size_t) r);
        for (int i = 0; i < r; i++) lin[(size_t) i] = (float) (-1.0 + 2.0 * i / (r - 1));
        s.lin = c->upload(lin);
        if (!s.wflow || !s.fbias || !s.fup || !s.wrgb || !s.rlb || !s.rbias || !s.rup || !s.lin)
            return -1;
        (void) C;
    }
    c->nseg = seg;
    {
        const HostTensor *in = c->need("dec.input.input");
        if (!in) return -1;
        std::vector<float> v = c->dev_value(*in), cl((size_t) 16 * C0);
        for (int ch = 0; ch < C0; ch++)
            for (int p = 0; p < 16; p++) cl[(size_t) p * C0 + ch] = v[(size_t) ch * 16 + p];
        c->input_cl = c->upload(cl);
    }
    c->wmod = c->upload(wmod);
    c->bmod = c->upload(bmod);
    c->saug_all = c->upload(saug_all);
    if (!c->input_cl || !c->wmod || !c->bmod || !c->saug_all) return -1;
    c->prepared = true;
    c->built = false;
    c->feats_set = false;
    return 0;
}

static int tpmd_build_body(tpmd_ctx *c, int max_batch) {
    if (!check_ctx(c)) return -1;
    if (!drain_all(c)) return -1;
    c->drop_graphs();
    if (!c->prepared) {
        c->err = "decoder not prepared";
        return -1;
    }
    if (max_batch < 1 || max_batch > 256) {
        c->err = "max_batch must be 1..256";
        return -1;
    }
    for (void *p : c->batch_allocs) (void) hipFree(p);
    c->batch_allocs.clear();
    c->built = false;
    c->feats_set = false;
    const int B = max_batch, ns = c->ns, C0 = c->ic[0];
    c->batch = B;

    // style segment table: block [B][width] per segment
    SegTable &sg = c->seg;
    sg.n = c->nseg;
    int64_t off = 0;
    int row = 0;
    for (int i = 0; i < c->nseg; i++) {
        sg.row0[i] = row;
        sg.width[i] = c->seg_width[i];
        sg.out0[i] = off;
        row += c->seg_width[i];
        off += (int64_t) B * c->seg_width[i];
    }
    sg.row0[c->nseg] = row;
    const int64_t s_total = off;
    DemodTable &dt = c->dem;
    dt.n = c->nconv;
    int64_t doff = 0;
    row = 0;
    for (int L = 0; L < c->nconv; L++) {
        ConvW &cv = c->conv[L];
        cv.s_off = sg.out0[cv.seg];
        cv.d_off = doff;
        dt.row0[L] = row;
        dt.ic[L] = cv.ic;
        dt.oc[L] = cv.oc;
        dt.saug0[L] = cv.saug_off;
        dt.s0[L] = cv.s_off;
        dt.d0[L] = doff;
        row += cv.oc;
        doff += (int64_t) B * cv.oc;
    }
    dt.row0[c->nconv] = row;
    for (int j = 0; j < ns; j++) c->st[j].s_off = sg.out0[c->st[j].seg];

    size_t act_max = (size_t) 16 * C0, out_max = 0, skip_max = 1;
    int64_t ws_max = 0;
    for (int L = 0; L < c->nconv; L++) {
        const ConvW &cv = c->conv[L];
        const int j = (L - 1) / 2;
        const int H = L == 0 ? 4 : (cv.up ? 4 << j : 8 << j);
        ws_max = std::max(ws_max, modconv_ws_elems(cv.up ? 1 : 0, B, H, H, cv.ic, cv.oc, c->f16));
    }
    for (int j = 0; j < ns; j++) {
        const size_t r = (size_t) 8 << j;
        act_max = std::max(act_max, r * r * c->oc[j]);
        if (!fused_tail(c, c->oc[j], (int) r)) out_max = std::max(out_max, r * r * c->oc[j]);
        if (j + 1 < ns) skip_max = std::max(skip_max, 3 * r * r);
    }
    const size_t R = (size_t) c->out_res();
    auto A = [&](size_t bytes) { return c->dalloc(bytes, c->batch_allocs); };
    for (int li = tpmd_ctx::kLanes - 1; li >= 0; li--) {
    c->L = &c->lane[li];
    c->L->lat = (float *) A((size_t) B * 512 * 4);
    c->L->s_all = (float *) A((size_t) s_total * 4);
    c->L->den_all = (float *) A((size_t) doff * 4);
    c->L->xs0 = A((size_t) B * 16 * C0 * c->act_size());
    c->L->c1 = A((size_t) B * act_max * c->act_size());
    c->L->trunk = A((size_t) B * act_max * c->act_size());
    c->L->outb = (float *) A((size_t) B * std::max<size_t>(out_max, 1) * 4);
    c->L->ws_elems = ws_max;
    c->L->ws = ws_max > 0 ? (float *) A((size_t) ws_max * 4) : nullptr;
    if (ws_max > 0 && !c->L->ws) return -1;
    for (int i = 0; i < 2; i++) {
        c->L->flow[i] = (float *) A((size_t) B * skip_max * 4);
        c->L->rgb[i] = (float *) A((size_t) B * skip_max * 4);
    }
    c->L->img = (float *) A((size_t) B * 3 * R * R * 4);
    if (!c->L->lat || !c->L->s_all || !c->L->den_all || !c->L->xs0 || !c->L->c1 || !c->L->trunk || !c->L->outb ||
        !c->L->flow[0] || !c->L->flow[1] || !c->L->rgb[0] || !c->L->rgb[1] || !c->L->img)
        return -1;
    }  // lanes; c->L is lane 0 again
    for (int j = 0; j < ns; j++) {
        const size_t r = (size_t) 8 << j;
        const size_t fb = r * r * c->oc[j] * c->act_size() + TAIL_FEAT_PAD;  // + zero pad
        c->st[j].feat = A(fb);
        if (!c->st[j].feat) return -1;
        if (!c->hip_ok(hipMemset(c->st[j].feat, 0, fb), "memset")) return -1;
        const size_t gb = r * r * 16 + TAIL_FEATG_PAD;
        c->st[j].featg = (float *) A(gb);
        if (!c->st[j].featg) return -1;
        if (!c->hip_ok(hipMemset(c->st[j].featg, 0, gb), "memset")) return -1;
    }
    c->built = true;
    return 0;
}

int tpmd_batch(const tpmd_ctx *c) { return c ? c->batch : 0; }
int tpmd_out_res(const tpmd_ctx *c) { return c ? c->out_res() : 0; }

static int set_feats_impl(tpmd_ctx *c, const float *const *feats, bool dev) {
    if (!check_ctx(c)) return -1;
    if (!drain_lanes(c)) return -1;
    if (!c->built) {
        c->err = "decoder not built";
        return -1;
    }
    if (!feats) {
        c->err = "feat size mismatch";
        return -1;
    }
    for (int j = 0; j < c->ns; j++) {
        if (!feats[j]) {
            c->err = "feat size mismatch";
            return -1;
        }
        const size_t r = (size_t) 8 << j, n = r * r * c->oc[j];
        float *tmp = (float *) c->scratch(0, n * 4);
        if (!tmp) return -1;
        if (!c->hip_ok(hipMemcpyAsync(tmp, feats[j], n * 4, dev ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                                      c->stream), "feat upload"))
            return -1;
        if (!c->hip_ok(launch_prescale_map(c->f16, tmp, nullptr, c->st[j].feat, c->oc[j], (int64_t) r * r, 1,
                                           c->stream), "feat convert"))
            return -1;
        if (!c->hip_ok(launch_feat_rgb(c->f16, c->st[j].feat, c->st[j].wrgb, c->oc[j], (int64_t) r * r,
                                       c->st[j].featg, c->stream), "feat rgb"))
            return -1;
        if (!c->hip_ok(hipStreamSynchronize(c->stream), "feat sync")) return -1;
    }
    c->feats_set = true;
    return 0;
}

int tpmd_set_feats(tpmd_ctx *c, const float *const *feats) { return set_feats_impl(c, feats, false); }
int tpmd_set_feats_device(tpmd_ctx *c, const float *const *feats) { return set_feats_impl(c, feats, true); }

// tail arguments of stage j for frames [0, n) of the decode buffers
static TailArgs stage_tail_args(tpmd_ctx *c, int j, int n, float *img_dst) {
    const StageW &s = c->st[j];
    const bool last = j + 1 == c->ns;
    TailArgs a{};
    a.out = c->L->outb;
    a.feat = s.feat;
    a.wflow = s.wflow;
    a.sflow = c->L->s_all + s.s_off;
    a.fbias = s.fbias;
    a.fup = s.fup;
    a.flow_prev = j > 0 ? c->L->flow[(j - 1) & 1] : nullptr;
    a.flow_cur = last ? nullptr : c->L->flow[j & 1];
    a.lin = s.lin;
    a.wrgb = s.wrgb;
    a.rlb = s.rlb;
    a.rbias = s.rbias;
    a.rup = s.rup;
    a.rgb_prev = j > 0 ? c->L->rgb[(j - 1) & 1] : nullptr;
    a.rgb_cur = last ? img_dst : c->L->rgb[j & 1];
    a.s_next = last ? nullptr : c->L->s_all + c->conv[3 + 2 * j].s_off;
    a.trunk = last ? nullptr : c->L->trunk;
    a.warp_tap = nullptr;
    a.featg = s.featg;
    a.nframes = n;
    a.r = 8 << j;
    a.C = c->oc[j];
    return a;
}

static ConvArgs conv_args(tpmd_ctx *c, const ConvW &cv, int n, int H, const void *X, void *Y,
                          const float *out_scale, bool out_f16) {
    ConvArgs a;
    a.mode = cv.up ? 1 : 0;
    a.f16 = c->f16;
    a.out_f16 = out_f16;
    a.A = cv.A;
    a.A_perm = cv.A_perm;
    a.X = X;
    a.Y = Y;
    a.inv_den = c->L->den_all + cv.d_off;
    a.bias = cv.bias;
    a.out_scale = out_scale;
    a.nframes = n;
    a.H = H;
    a.W = H;
    a.IC = cv.ic;
    a.OC = cv.oc;
    a.x_bstride = (int64_t) H * H * cv.ic;
    a.ws = c->L->ws;
    a.ws_elems = c->L->ws_elems;
    return a;
}

// bytes per frame of a tap (tpmd_set_tap), or -1 when the decode chain does
// not hold that buffer
static int64_t tap_frame_bytes(const tpmd_ctx *c, int kind, int stage) {
    const int ns = c->ns;
    if (stage < -1 || stage >= ns) return -1;
    const int r = stage < 0 ? 4 : 8 << stage;
    const int C = stage < 0 ? c->ic[0] : c->oc[stage];
    const int64_t px = (int64_t) r * r;
    switch (kind) {
    case TPMD_TAP_TRUNK:
        return stage < ns - 1 ? px * C * (int64_t) c->act_size() : -1;
    case TPMD_TAP_C1:
        return stage >= 0 ? px * C * (int64_t) c->act_size() : -1;
    case TPMD_TAP_OUT:
        return stage >= 0 && !fused_tail(c, C, r) ? px * C * 4 : -1;
    case TPMD_TAP_FLOW:
        return stage >= 0 ? px * 3 * 4 : -1;
    case TPMD_TAP_RGB:
        return stage >= 0 && stage < ns - 1 ? px * 3 * 4 : -1;
    default:
        return -1;
    }
}

// copy frames [0, n) of a chain buffer to its registered tap, if any
static bool tap_copy(tpmd_ctx *c, int kind, int stage, const void *src, int n, hipStream_t st) {
    const tpmd_ctx::Tap &t = c->taps[kind][stage + 1];
    if (!t.dst) return true;
    const int64_t bytes = tap_frame_bytes(c, kind, stage) * n;
    if (bytes > t.bytes) {
        c->err = fmt("tap %d of stage %d holds %lld bytes, the decode needs %lld", kind, stage,
                     (long long) t.bytes, (long long) bytes);
        return false;
    }
    return c->hip_ok(hipMemcpyAsync(t.dst, src, (size_t) bytes, hipMemcpyDeviceToDevice, st), "tap copy");
}

// the whole batched decoder for frames [0, n) of the current lane on its
// stream; the launch that writes img_dst (the last stage's tail) first waits
// for `frames_after` when given
static bool enqueue_decode(tpmd_ctx *c, int n, float *img_dst, hipEvent_t frames_after = nullptr) {
    hipStream_t st = c->stream;
    const bool f16 = c->f16;
    const int ns = c->ns, C0 = c->ic[0];
    int slot = 0;
    auto mark = [&]() {
        if (c->profile) (void) hipEventRecord(c->ev[(size_t) slot++], st);
    };
    mark();
    if (!c->hip_ok(launch_style_gemv(c->wmod, c->bmod, c->L->lat, c->L->s_all, c->seg, n, st), "style")) return false;
    if (!c->hip_ok(launch_demod(c->saug_all, c->L->s_all, c->L->den_all, c->dem, n, st), "demod")) return false;
    const ConvW &k1 = c->conv[0];
    if (!c->hip_ok(launch_prescale_input(f16, c->input_cl, c->L->s_all + k1.s_off, c->L->xs0, C0, n, st), "prescale"))
        return false;
    // conv1 -> trunk (pre-scaled by the stage-0 up-conv style)
    if (!c->hip_ok(launch_modconv(conv_args(c, k1, n, 4, c->L->xs0, c->L->trunk, c->L->s_all + c->conv[1].s_off, f16), st),
                   "conv1"))
        return false;
    if (c->any_tap && !tap_copy(c, TPMD_TAP_TRUNK, -1, c->L->trunk, n, st)) return false;
    for (int j = 0; j < ns; j++) {
        const int r = 8 << j, rh = r / 2, C = c->oc[j];
        const bool last = j + 1 == ns;
        const ConvW &up = c->conv[1 + 2 * j], &dn = c->conv[2 + 2 * j];
        mark();
        if (!c->hip_ok(launch_modconv(conv_args(c, up, n, rh, c->L->trunk, c->L->c1, c->L->s_all + dn.s_off, f16), st),
                       "up-conv"))
            return false;
        if (c->any_tap && !tap_copy(c, TPMD_TAP_C1, j, c->L->c1, n, st)) return false;
        mark();
        TailArgs ta = stage_tail_args(c, j, n, img_dst);
        // the last stage keeps no flow map; a flow tap there is written by
        // the tail itself
        const tpmd_ctx::Tap &lf = c->taps[TPMD_TAP_FLOW][j + 1];
        if (last && lf.dst) {
            if (lf.bytes < tap_frame_bytes(c, TPMD_TAP_FLOW, j) * n) {
                c->err = fmt("tap %d of stage %d is too small", TPMD_TAP_FLOW, j);
                return false;
            }
            ta.flow_cur = (float *) lf.dst;
        }
        if (last && frames_after && !c->hip_ok(hipStreamWaitEvent(st, frames_after, 0), "wait")) return false;
        if (fused_tail(c, C, r)) {
            ConvArgs ca = conv_args(c, dn, n, r, c->L->c1, nullptr, nullptr, false);
            ca.tail = &ta;
            ca.trunk_f16 = f16;
            if (!c->hip_ok(launch_modconv(ca, st), "conv+tail")) return false;
            mark();
        } else {
            if (!c->hip_ok(launch_modconv(conv_args(c, dn, n, r, c->L->c1, c->L->outb, nullptr, false), st), "conv"))
                return false;
            if (c->any_tap && !tap_copy(c, TPMD_TAP_OUT, j, c->L->outb, n, st)) return false;
            mark();
            if (!c->hip_ok(launch_stage_tail(ta, f16, false, f16, st), "tail")) return false;
        }
        if (c->any_tap && !last &&
            (!tap_copy(c, TPMD_TAP_TRUNK, j, c->L->trunk, n, st) || !tap_copy(c, TPMD_TAP_FLOW, j, ta.flow_cur, n, st) ||
             !tap_copy(c, TPMD_TAP_RGB, j, ta.rgb_cur, n, st)))
            return false;
    }
    mark();
    return true;
}

// enqueue_decode as one graph launch: the current lane's chain for (n,
// img_dst) is captured on first use and replayed after that.  The graph
// holds kernel launches only (no memsets, no copies).  Per-stage profiling,
// taps, a stream that is itself being captured, or graphs turned off
// enqueue the launches directly; `frames_after` then orders the whole graph
// instead of its last stage.
static bool run_chain(tpmd_ctx *c, int n, float *img_dst, hipEvent_t frames_after = nullptr) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (!c->use_graphs || c->profile || c->any_tap || !c->stream ||
        hipStreamIsCapturing(c->stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
        return enqueue_decode(c, n, img_dst, frames_after);
    auto &lg = c->graphs[c->L - c->lane];
    tpmd_ctx::Graph *g = nullptr, *lru = &lg[0];
    for (auto &e : lg) {
        if (e.exec && e.n == n && e.dst == img_dst) g = &e;
        if (e.used < lru->used) lru = &e;
    }
    if (!g) {
        g = lru;
        if (g->exec) (void) hipGraphExecDestroy(g->exec);
        *g = tpmd_ctx::Graph{};
        if (!c->hip_ok(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal), "graph capture"))
            return false;
        const bool ok = enqueue_decode(c, n, img_dst);
        hipGraph_t graph = nullptr;
        const hipError_t e = hipStreamEndCapture(c->stream, &graph);
        hipGraphExec_t exec = nullptr;
        const bool made = ok && c->hip_ok(e, "graph capture") &&
                          c->hip_ok(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "graph instantiate");
        if (graph) (void) hipGraphDestroy(graph);
        if (!made) return false;
        g->exec = exec;
        g->n = n;
        g->dst = img_dst;
    }
    g->used = ++c->graph_clock;
    if (frames_after && !c->hip_ok(hipStreamWaitEvent(c->stream, frames_after, 0), "wait")) return false;
    return c->hip_ok(hipGraphLaunch(g->exec, c->stream), "graph launch");
}

static int decode_batch_lane(tpmd_ctx *c, const float *styles, int n, float *imgs, int on_device,
                             int lane = -1);

static int tpmd_decode_batch_body(tpmd_ctx *c, const float *styles, int n, float *imgs, int on_device) {
    if (!check_ctx(c)) return -1;
    // device-resident decodes on the library's own stream rotate over the lanes;
    // every other form (host buffers, a caller's stream, per-stage
    // profiling, taps) runs on lane 0 after the other lanes have drained
    const bool multi = on_device && imgs && !c->profile && !c->any_tap && c->stream == c->own_stream &&
                       tpmd_ctx::kLanes > 1;
    if (!multi) {
        if (!drain_lanes(c)) return -1;
        for (auto &o : c->lane_out) o = tpmd_ctx::OutRange{};
        return decode_batch_lane(c, styles, n, imgs, on_device);
    }
    const int k = c->next_lane;
    c->next_lane = (c->next_lane + 1) % tpmd_ctx::kLanes;
    hipStream_t keep = c->stream;
    c->L = &c->lane[k];
    if (k > 0) c->stream = c->lane_stream[k];
    const int rc = decode_batch_lane(c, styles, n, imgs, on_device, k);
    c->L = &c->lane[0];
    c->stream = keep;
    return rc;
}

// lane >= 0: a device-resident decode on that lane's stream, ordered against
// the null stream for its latents and against the other lanes for its frames
static int decode_batch_lane(tpmd_ctx *c, const float *styles, int n, float *imgs, int on_device, int lane) {
    if (!c->built) {
        c->err = "decoder not built";
        return -1;
    }
    if (!c->feats_set) {
        c->err = "feats not set";
        return -1;
    }
    if (!styles || n < 1 || n > c->batch) {
        c->err = fmt("decode_batch: need 1..%d styles", c->batch);
        return -1;
    }
    const size_t R = (size_t) c->out_res();
    const hipMemcpyKind k_in = on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
    // the latents are read after the caller's earlier null-stream work, and
    // the null stream's later work waits for that read
    if (lane >= 0 && !(c->hip_ok(hipEventRecord(c->ev_in[lane], nullptr), "event") &&
                       c->hip_ok(hipStreamWaitEvent(c->stream, c->ev_in[lane], 0), "wait")))
        return -1;
    if (!c->hip_ok(hipMemcpyAsync(c->L->lat, styles, (size_t) n * 512 * 4, k_in, c->stream), "style upload"))
        return -1;
    if (lane >= 0 && !(c->hip_ok(hipEventRecord(c->ev_read[lane], c->stream), "event") &&
                       c->hip_ok(hipStreamWaitEvent(nullptr, c->ev_read[lane], 0), "wait")))
        return -1;
    if (c->profile) {
        const size_t need = (size_t) 2 + 3 * c->ns;
        while (c->ev.size() < need) {
            hipEvent_t e;
            if (!c->hip_ok(hipEventCreate(&e), "event")) return -1;
            c->ev.push_back(e);
        }
    }
    float *dst = (on_device && imgs) ? imgs : c->L->img;
    // frames written into a buffer that another lane's in-flight call writes
    // too land after that call's (a caller may reuse one frame buffer)
    hipEvent_t after = nullptr;
    const char *lo = (const char *) dst, *hi = lo + (size_t) n * 3 * R * R * 4;
    if (lane >= 0) {
        for (int l = 0; l < tpmd_ctx::kLanes; l++) {
            const tpmd_ctx::OutRange &o = c->lane_out[l];
            if (l == lane || !o.lo || hi <= o.lo || o.hi <= lo) continue;
            if (after && !c->hip_ok(hipStreamWaitEvent(c->stream, after, 0), "wait")) return -1;
            after = c->ev_done[l];
        }
    }
    if (!run_chain(c, n, dst, after)) return -1;
    if (lane >= 0) {
        if (!c->hip_ok(hipEventRecord(c->ev_done[lane], c->stream), "event")) return -1;
        c->lane_out[lane] = {lo, hi};
    }
    if (!on_device) {
        if (imgs && !c->hip_ok(hipMemcpyAsync(imgs, c->L->img, (size_t) n * 3 * R * R * 4, hipMemcpyDeviceToHost,
                                              c->stream), "image download"))
            return -1;
        if (!c->hip_ok(hipStreamSynchronize(c->stream), "decode")) return -1;
    }
    if (c->profile) {
        if (!c->hip_ok(hipStreamSynchronize(c->stream), "decode")) return -1;
        const size_t ns = (size_t) 1 + 3 * c->ns;
        c->times.assign(ns, 0.0f);
        for (size_t i = 0; i < ns; i++) {
            float ms = 0;
            (void) hipEventElapsedTime(&ms, c->ev[i], c->ev[i + 1]);
            c->times[i] = ms * 1000.0f;
        }
    }
    return 0;
}

// slot buffers of the frame stream, grow-only
static bool frame_slots(tpmd_ctx *c, size_t bytes) {
    auto &f = c->fs;
    if (!f.copy) {
        if (!c->hip_ok(hipStreamCreateWithFlags(&f.copy, hipStreamNonBlocking), "copy stream")) return false;
        for (int i = 0; i < tpmd_ctx::kLanes; i++)
            if (!c->hip_ok(hipEventCreateWithFlags(&f.computed[i], hipEventDisableTiming), "event") ||
                !c->hip_ok(hipEventCreateWithFlags(&f.copied[i], hipEventDisableTiming), "event"))
                return false;
    }
    if (!f.pool) {
        // helpers: the CPUs this process may run on, less the calling thread,
        // at most 15 (measured on a 16-CPU share, f32 frames into a reused
        // pageable buffer: 7 helpers 9.3k, 11 9.6k, 15 9.7k frames/s)
        unsigned ncpu = std::thread::hardware_concurrency();
        cpu_set_t cs;
        CPU_ZERO(&cs);
        if (sched_getaffinity(0, sizeof(cs), &cs) == 0) ncpu = (unsigned) CPU_COUNT(&cs);
        f.pool.reset(new (std::nothrow) CopyPool((int) std::min(15u, ncpu > 1 ? ncpu - 1 : 0u)));
        if (!f.pool) {
            c->err = "frame copy threads: out of memory";
            return false;
        }
    }
    if (f.bytes >= bytes) return true;
    for (int i = 0; i < tpmd_ctx::kLanes; i++) {
        if (f.dev[i]) (void) hipFree(f.dev[i]);
        if (f.host[i]) (void) hipHostFree(f.host[i]);
        f.dev[i] = f.host[i] = nullptr;
    }
    f.bytes = 0;
    for (int i = 0; i < tpmd_ctx::kLanes; i++) {
        if (!c->hip_ok(hipMalloc(&f.dev[i], bytes), "frame slot") ||
            !c->hip_ok(hipHostMalloc(&f.host[i], bytes, hipHostMallocDefault), "pinned frame slot"))
            return false;
    }
    f.bytes = bytes;
    return true;
}

static int64_t tpmd_decode_frames_body(tpmd_ctx *c, const float *styles, int64_t n_frames, int format, void *out,
                           tpmd_frame_cb cb, void *ud) {
    if (!check_ctx(c)) return -1;
    if (!drain_lanes(c)) return -1;
    if (!c->built || !c->feats_set) {
        c->err = !c->built ? "decoder not built" : "feats not set";
        return -1;
    }
    if (!styles || n_frames < 1 || (format != TPMD_FRAME_F32 && format != TPMD_FRAME_RGB24)) {
        c->err = "tpmd_decode_frames: bad arguments";
        return -1;
    }
    const size_t R = (size_t) c->out_res();
    const size_t fsz = format == TPMD_FRAME_F32 ? 3 * R * R * 4 : 3 * R * R;
    const int B = c->batch;
    if (!frame_slots(c, (size_t) B * fsz)) return -1;
    const bool prof = c->profile;
    c->profile = false;  // no per-stage events inside the stream
    auto &f = c->fs;
    const int64_t nb = (n_frames + B - 1) / B;
    bool ok = true, stopped = false;
    // on the library's own stream, batch k runs on lane k % kLanes (its own
    // buffers and stream) with frame slot k % kLanes; on a caller's stream,
    // every batch runs on lane 0 in that stream
    constexpr int NS = tpmd_ctx::kLanes;
    const bool multi = c->stream == c->own_stream;
    hipStream_t keep = c->stream;
    // a pinned caller buffer takes the downloads directly (no staging copy)
    bool direct = false;
    if (out) {
        hipPointerAttribute_t pa{};
        direct = hipPointerGetAttributes(&pa, out) == hipSuccess && pa.type == hipMemoryTypeHost;
        (void) hipGetLastError();  // a pageable buffer is reported as an error: clear it
    }
    // frames of batch k, from its pinned slot, to the caller
    auto deliver = [&](int64_t k) {
        const int s = (int) (k % NS);
        const int64_t t0 = k * B;
        const int64_t nk = std::min<int64_t>(B, n_frames - t0);
        if (!c->hip_ok(hipEventSynchronize(f.copied[s]), "frame copy")) return ok = false;
        const char *src = direct ? (const char *) out + (size_t) t0 * fsz : (const char *) f.host[s];
        if (out && !direct) f.pool->copy((char *) out + (size_t) t0 * fsz, src, (size_t) nk * fsz);
        if (cb)
            for (int64_t i = 0; i < nk; i++)
                if (cb(t0 + i, src + (size_t) i * fsz, ud)) return !(stopped = true);
        return true;
    };
    for (int64_t k = 0; k < nb && ok && !stopped; k++) {
        const int s = (int) (k % NS);
        const int64_t t0 = k * B;
        const int nk = (int) std::min<int64_t>(B, n_frames - t0);
        const int li = multi ? s : 0;
        c->L = &c->lane[li];
        c->stream = li == 0 ? keep : c->lane_stream[li];
        // slot s is free once the copy of batch k-NS has finished
        if (k >= NS && !c->hip_ok(hipStreamWaitEvent(c->stream, f.copied[s], 0), "wait")) ok = false;
        ok = ok && c->hip_ok(hipMemcpyAsync(c->L->lat, styles + (size_t) t0 * 512, (size_t) nk * 512 * 4,
                                            hipMemcpyHostToDevice, c->stream),
                             "style upload");
        if (format == TPMD_FRAME_F32) {
            ok = ok && run_chain(c, nk, (float *) f.dev[s]);
        } else {
            ok = ok && run_chain(c, nk, c->L->img) &&
                 c->hip_ok(launch_rgb24(c->L->img, nk, (int) R, (uint8_t *) f.dev[s], c->stream), "rgb24");
        }
        ok = ok && c->hip_ok(hipEventRecord(f.computed[s], c->stream), "event") &&
             c->hip_ok(hipStreamWaitEvent(f.copy, f.computed[s], 0), "wait") &&
             c->hip_ok(hipMemcpyAsync(direct ? (char *) out + (size_t) t0 * fsz : f.host[s], f.dev[s],
                                      (size_t) nk * fsz, hipMemcpyDeviceToHost, f.copy),
                       "frame download") &&
             c->hip_ok(hipEventRecord(f.copied[s], f.copy), "event");
        c->L = &c->lane[0];
        c->stream = keep;
        if (ok && k >= 1) deliver(k - 1);  // batch k decodes while batch k-1 is handed over
        if (ok && !stopped && k == nb - 1) deliver(k);
    }
    c->L = &c->lane[0];
    c->stream = keep;
    // leave every stream idle: the slots may be reused by the next call
    const bool drained = c->hip_ok(hipStreamSynchronize(f.copy), "drain") && drain_lanes(c) &&
                         c->hip_ok(hipStreamSynchronize(c->stream), "drain");
    for (auto &o : c->lane_out) o = tpmd_ctx::OutRange{};
    c->profile = prof;
    return ok && drained ? n_frames : -1;
}

int tpmd_decode(tpmd_ctx *c, const float *style, float *img) {
    return tpmd_decode_batch(c, style, 1, img, 0);
}

int tpmd_set_stream(tpmd_ctx *c, void *stream) {
    if (!check_ctx(c)) return -1;
    // lane 0's buffers move to the new stream: nothing may still use them on
    // the library's streams or on the previous caller stream
    if (!drain_all(c)) return -1;
    if (c->stream != c->own_stream && !c->hip_ok(hipStreamSynchronize(c->stream), "stream sync")) return -1;
    for (auto &o : c->lane_out) o = tpmd_ctx::OutRange{};
    c->stream = (hipStream_t) stream;
    return 0;
}

int tpmd_set_graphs(tpmd_ctx *c, int enable) {
    if (!check_ctx(c)) return -1;
    if (!drain_all(c)) return -1;
    c->drop_graphs();
    c->use_graphs = enable != 0;
    return 0;
}

int tpmd_sync(tpmd_ctx *c) {
    if (!check_ctx(c)) return -1;
    return drain_all(c) && c->hip_ok(hipStreamSynchronize(c->stream), "sync") ? 0 : -1;
}

int tpmd_profile_stages(tpmd_ctx *c, int enable) {
    if (!check_ctx(c)) return -1;
    c->profile = enable != 0;
    return 1 + 3 * c->ns;
}

int tpmd_stage_times(const tpmd_ctx *c, float *us, int max_slots) {
    if (!c || !us) return -1;
    const int n = (int) c->times.size() < max_slots ? (int) c->times.size() : max_slots;
    for (int i = 0; i < n; i++) us[i] = c->times[(size_t) i];
    return n;
}

int64_t tpmd_tap_frame_bytes(const tpmd_ctx *c, int kind, int stage) {
    return c ? tap_frame_bytes(c, kind, stage) : -1;
}

static int tpmd_set_tap_body(tpmd_ctx *c, int kind, int stage, void *dst, int64_t bytes) {
    if (!check_ctx(c)) return -1;
    if (kind < 0 || kind >= TPMD_TAP_KINDS || stage < -1 || stage >= c->ns) {
        c->err = "tpmd_set_tap: bad kind or stage";
        return -1;
    }
    if (dst && tap_frame_bytes(c, kind, stage) < 0) {
        c->err = fmt("tpmd_set_tap: the decode chain holds no buffer of kind %d at stage %d", kind, stage);
        return -1;
    }
    if (dst && bytes < 0) {
        c->err = "tpmd_set_tap: negative size";
        return -1;
    }
    // a call with taps runs on lane 0 after the other lanes drain: none of
    // them may still write a tap buffer being replaced
    if (!drain_lanes(c)) return -1;
    c->taps[kind][stage + 1] = {dst, dst ? bytes : 0};
    c->any_tap = false;
    for (const auto &row : c->taps)
        for (const auto &t : row) c->any_tap = c->any_tap || t.dst;
    return 0;
}

// argument checks of tpmd_modconv / tpmd_modconv_static
static bool modconv_args_ok(tpmd_ctx *c, const char *who, int conv, const float *x, int n, int H, int W,
                            const float *s, const float *y) {
    if (!c->prepared) {
        c->err = "decoder not prepared";
        return false;
    }
    if (conv < 0 || conv >= c->nconv || !x || !s || !y || n < 1 || H < 1 || W < 1) {
        c->err = std::string(who) + ": bad arguments";
        return false;
    }
    return true;
}

// device scratch of one tpmd_modconv call: the input multiplied by the style
// (the conv's operand type), 1/den, and the split-K partial sums (0 bytes
// when the conv shape runs unsplit)
struct ModconvScratch {
    size_t xs = 0, den = 0, ws = 0;
    static size_t up256(size_t b) { return (b + 255) & ~(size_t) 255; }
    size_t total() const { return up256(xs) + up256(den) + up256(ws); }
};
static ModconvScratch modconv_scratch(const tpmd_ctx *c, const ConvW &cv, int n, int H, int W) {
    ModconvScratch m;
    m.xs = (size_t) n * H * W * cv.ic * c->act_size();
    m.den = (size_t) n * cv.oc * 4;
    m.ws = (size_t) modconv_ws_elems(cv.up ? 1 : 0, n, H, W, cv.ic, cv.oc, c->f16) * 4;
    return m;
}

// demodulation, style multiply and the conv of tpmd_modconv on given scratch
static int modconv_run(tpmd_ctx *c, const ConvW &cv, const float *x, int n, int H, int W, const float *s, float *y,
                       hipStream_t st, void *xs, float *den, float *ws) {
    const int64_t npix = (int64_t) H * W;
    DemodTable t{};
    t.n = 1;
    t.row0[0] = 0;
    t.row0[1] = cv.oc;
    t.ic[0] = cv.ic;
    t.oc[0] = cv.oc;
    t.saug0[0] = cv.saug_off;
    t.s0[0] = 0;
    t.d0[0] = 0;
    if (!c->hip_ok(launch_demod(c->saug_all, s, den, t, n, st), "demod")) return -1;
    if (!c->hip_ok(launch_prescale_map(c->f16, x, s, xs, cv.ic, npix, n, st), "prescale")) return -1;
    ConvArgs ca;
    ca.mode = cv.up ? 1 : 0;
    ca.f16 = c->f16;
    ca.A = cv.A;
    ca.A_perm = cv.A_perm;
    ca.X = xs;
    ca.Y = y;
    ca.inv_den = den;
    ca.bias = cv.bias;
    ca.nframes = n;
    ca.H = H;
    ca.W = W;
    ca.IC = cv.ic;
    ca.OC = cv.oc;
    ca.x_bstride = npix * cv.ic;
    ca.ws_elems = modconv_ws_elems(ca.mode, n, H, W, cv.ic, cv.oc, c->f16);
    ca.ws = ca.ws_elems > 0 ? ws : nullptr;
    return c->hip_ok(launch_modconv(ca, st), "modconv") ? 0 : -1;
}

static int tpmd_modconv_body(tpmd_ctx *c, int conv, const float *x, int n, int H, int W, const float *s, float *y,
                             void *stream) {
    if (!check_ctx(c) || !modconv_args_ok(c, "tpmd_modconv", conv, x, n, H, W, s, y)) return -1;
    const ConvW &cv = c->conv[conv];
    const ModconvScratch m = modconv_scratch(c, cv, n, H, W);
    void *xs = c->scratch(1, m.xs);
    float *den = (float *) c->scratch(2, m.den);
    float *ws = m.ws ? (float *) c->scratch(3, m.ws) : nullptr;
    if (!xs || !den || (m.ws && !ws)) return -1;
    return modconv_run(c, cv, x, n, H, W, s, y, pick_stream(c, stream), xs, den, ws);
}

static int tpmd_modconv_static_body(tpmd_ctx *c, int conv, const float *x, int n, int H, int W, const float *s,
                                    float *y, void *stream) {
    if (!check_ctx(c) || !modconv_args_ok(c, "tpmd_modconv_static", conv, x, n, H, W, s, y)) return -1;
    if (!c->static_scratch) {
        c->err = "tpmd_modconv_static: the static scratch of this device is unavailable (" +
                 c->static_scratch_err + ")";
        return -1;
    }
    const ConvW &cv = c->conv[conv];
    const ModconvScratch m = modconv_scratch(c, cv, n, H, W);
    if (m.total() > TPMD_STATIC_SCRATCH_BYTES) {
        c->err = fmt("tpmd_modconv_static: this call needs %zu bytes of scratch, the static scratch holds %zu",
                     m.total(), (size_t) TPMD_STATIC_SCRATCH_BYTES);
        return -1;
    }
    char *base = (char *) c->static_scratch;
    void *xs = base;
    float *den = (float *) (base + ModconvScratch::up256(m.xs));
    float *ws = m.ws ? (float *) (base + ModconvScratch::up256(m.xs) + ModconvScratch::up256(m.den)) : nullptr;
    return modconv_run(c, cv, x, n, H, W, s, y, pick_stream(c, stream), xs, den, ws);
}

// tpmd_decode_taps: one frame through the unfused f32 chain (the per-stage
// entry points' kernels: styled convs with f32 output, the standalone stage
// tail storing trunk, warp, flow and rgb), every tap copied to the host in the
// reference's tap layout
static int tpmd_decode_taps_body(tpmd_ctx *c, const float *style, float *img, tpmd_tap_cb cb, void *ud) {
    if (!check_ctx(c)) return -1;
    if (!c->built || !c->feats_set) {
        c->err = !c->built ? "decoder not built" : "feats not set";
        return -1;
    }
    if (!style || !cb) {
        c->err = "tpmd_decode_taps: null style or callback";
        return -1;
    }
    if (!drain_lanes(c)) return -1;
    for (auto &o : c->lane_out) o = tpmd_ctx::OutRange{};
    hipStream_t st = c->stream;
    tpmd_ctx::Lane &L = c->lane[0];
    const int ns = c->ns, C0 = c->ic[0];
    size_t mx = (size_t) 16 * C0;
    for (int j = 0; j < ns; j++) mx = std::max(mx, (size_t) (8 << j) * (8 << j) * c->oc[j]);
    const size_t R = (size_t) c->out_res(), skip = 3 * R * R;
    // grid: the flow head's [3][r*r] output, then the identity grid [2][r*r]
    float *buf[3], *warp = (float *) c->scratch(7, mx * 4), *grid = (float *) c->scratch(8, 5 * R * R * 4);
    if (!warp || !grid) return -1;
    for (int i = 0; i < 3; i++)
        if (!(buf[i] = (float *) c->scratch(4 + i, mx * 4))) return -1;
    // flow and rgb maps of every stage up to the last, 3 x R x R each (the
    // lane's skip buffers hold only the stages before the last)
    float *flow[2], *rgb[2];
    for (int i = 0; i < 2; i++) {
        flow[i] = (float *) c->scratch(9 + i, skip * 4);
        rgb[i] = (float *) c->scratch(11 + i, skip * 4);
        if (!flow[i] || !rgb[i]) return -1;
    }
    if (!c->hip_ok(hipMemcpyAsync(L.lat, style, 512 * 4, hipMemcpyHostToDevice, st), "style upload") ||
        !c->hip_ok(launch_style_gemv(c->wmod, c->bmod, L.lat, L.s_all, c->seg, 1, st), "style") ||
        !c->hip_ok(launch_demod(c->saug_all, L.s_all, L.den_all, c->dem, 1, st), "demod"))
        return -1;
    // the convs' scratch at its largest up front: no slot is reallocated while
    // an earlier launch of this call may still read it
    {
        ModconvScratch big;
        for (int L_ = 0; L_ < c->nconv; L_++) {
            const ConvW &cv = c->conv[L_];
            const int j = (L_ - 1) / 2;
            const int H = L_ == 0 ? 4 : (cv.up ? 4 << j : 8 << j);
            const ModconvScratch m = modconv_scratch(c, cv, 1, H, H);
            big.xs = std::max(big.xs, m.xs);
            big.den = std::max(big.den, m.den);
            big.ws = std::max(big.ws, m.ws);
        }
        if (!c->scratch(1, big.xs) || !c->scratch(2, big.den) || (big.ws && !c->scratch(3, big.ws))) return -1;
    }
    std::vector<float> h((size_t) mx), t((size_t) mx);
    // device CL [r*r][C] (or SP when sp) -> host, SP [1][C][r][r] -> callback
    auto emit = [&](const char *name, const float *d, int C, int r, bool sp, std::vector<int64_t> shape) {
        const size_t n = (size_t) r * r * C;
        if (!c->hip_ok(hipMemcpyAsync(h.data(), d, n * 4, hipMemcpyDeviceToHost, st), "tap download") ||
            !c->hip_ok(hipStreamSynchronize(st), "tap sync"))
            return false;
        const float *src = h.data();
        if (!sp) {
            for (size_t p = 0; p < (size_t) r * r; p++)
                for (int ch = 0; ch < C; ch++) t[(size_t) ch * r * r + p] = h[p * C + ch];
            src = t.data();
        }
        if (cb(name, src, (int) shape.size(), shape.data(), ud) != 0) {
            if (c->err.empty()) c->err = std::string("tap callback stopped at ") + name;
            return false;
        }
        return true;
    };
    auto conv = [&](int L_, const float *x, int H, float *y) {
        const ConvW &cv = c->conv[L_];
        const ModconvScratch m = modconv_scratch(c, cv, 1, H, H);
        void *xs = c->scratch(1, m.xs);
        float *den = (float *) c->scratch(2, m.den);
        float *ws = m.ws ? (float *) c->scratch(3, m.ws) : nullptr;
        if (!xs || !den || (m.ws && !ws)) return false;
        return modconv_run(c, cv, x, 1, H, H, L.s_all + cv.s_off, y, st, xs, den, ws) == 0;
    };
    if (!conv(0, c->input_cl, 4, buf[0]) || !emit("conv1_4", buf[0], C0, 4, false, {1, C0, 4, 4})) return -1;
    std::vector<float> xs;
    char nm[32];
    for (int j = 0; j < ns; j++) {
        const int r = 8 << j, C = c->oc[j];
        const int64_t r64 = r, C64 = C;
        float *c1 = buf[1], *out = buf[2], *trunk = buf[0];
        if (!conv(1 + 2 * j, buf[0], r / 2, c1)) return -1;
        snprintf(nm, sizeof nm, "r%d.conv1", r);
        if (!emit(nm, c1, C, r, false, {1, C64, r64, r64})) return -1;
        if (!conv(2 + 2 * j, c1, r, out)) return -1;
        snprintf(nm, sizeof nm, "r%d.conv2", r);
        if (!emit(nm, out, C, r, false, {1, C64, r64, r64})) return -1;
        const StageW &sw = c->st[j];
        TailArgs a{};
        a.out = out;
        a.feat = sw.feat;
        a.wflow = sw.wflow;
        a.sflow = L.s_all + sw.s_off;
        a.fbias = sw.fbias;
        a.fup = sw.fup;
        a.flow_prev = j > 0 ? flow[(j - 1) & 1] : nullptr;
        a.flow_cur = flow[j & 1];
        a.lin = sw.lin;
        a.wrgb = sw.wrgb;
        a.rlb = sw.rlb;
        a.rbias = sw.rbias;
        a.rup = sw.rup;
        a.rgb_prev = j > 0 ? rgb[(j - 1) & 1] : nullptr;
        a.rgb_cur = rgb[j & 1];
        a.trunk = trunk;      // overwrites the stage input, read by the up-conv only
        a.warp_tap = warp;
        a.nframes = 1;
        a.r = r;
        a.C = C;
        if (!c->hip_ok(launch_stage_tail(a, c->f16, false, false, st), "tail")) return -1;
        snprintf(nm, sizeof nm, "r%d.flowmap", r);
        if (!emit(nm, flow[j & 1], 3, r, true, {1, 3, r64, r64})) return -1;
        // grid: the flow head on the identity grid (planar gx, gy), interleaved
        xs.resize((size_t) 2 * r * r);
        for (int y = 0; y < r; y++)
            for (int x = 0; x < r; x++) {
                xs[(size_t) y * r + x] = (float) (-1.0 + 2.0 * x / (r - 1));
                xs[(size_t) r * r + (size_t) y * r + x] = (float) (-1.0 + 2.0 * y / (r - 1));
            }
        float *xs_d = grid + skip;
        if (!c->hip_ok(hipMemcpyAsync(xs_d, xs.data(), xs.size() * 4, hipMemcpyHostToDevice, st), "grid upload") ||
            !c->hip_ok(launch_flow_grid(flow[j & 1], xs_d, grid, (int64_t) r * r, st), "flow head"))
            return -1;
        // [3][r*r] planar -> [r*r][2] interleaved is the CL view of the first two planes
        if (!c->hip_ok(hipMemcpyAsync(h.data(), grid, (size_t) 2 * r * r * 4, hipMemcpyDeviceToHost, st), "tap download") ||
            !c->hip_ok(hipStreamSynchronize(st), "tap sync"))
            return -1;
        for (size_t p = 0; p < (size_t) r * r; p++) {
            t[2 * p] = h[p];
            t[2 * p + 1] = h[(size_t) r * r + p];
        }
        snprintf(nm, sizeof nm, "r%d.grid", r);
        const int64_t gshape[4] = {1, r64, r64, 2};
        if (cb(nm, t.data(), 4, gshape, ud) != 0) {
            if (c->err.empty()) c->err = std::string("tap callback stopped at ") + nm;
            return -1;
        }
        snprintf(nm, sizeof nm, "r%d.warp", r);
        if (!emit(nm, warp, C, r, false, {1, C64, r64, r64})) return -1;
        snprintf(nm, sizeof nm, "r%d.out", r);
        if (!emit(nm, trunk, C, r, false, {1, C64, r64, r64})) return -1;
        snprintf(nm, sizeof nm, "r%d.rgb", r);
        if (!emit(nm, rgb[j & 1], 3, r, true, {1, 3, r64, r64})) return -1;
    }
    if (img) {
        if (!c->hip_ok(hipMemcpyAsync(img, rgb[(ns - 1) & 1], skip * 4, hipMemcpyDeviceToHost, st), "image download"))
            return -1;
    }
    return c->hip_ok(hipStreamSynchronize(st), "decode") ? 0 : -1;
}

static int tpmd_stage_tail_body(tpmd_ctx *c, int j, const float *out, int n, const float *s_flow, const float *flow_prev,
                    const float *rgb_prev, float *flow, float *trunk, float *rgb, float *warp,
                    void *stream) {
    if (!check_ctx(c)) return -1;
    if (!c->built || !c->feats_set) {
        c->err = "decoder not built / feats not set";
        return -1;
    }
    if (j < 0 || j >= c->ns || !out || !s_flow || !rgb || n < 1) {
        c->err = "tpmd_stage_tail: bad arguments";
        return -1;
    }
    if (j > 0 && (!flow_prev || !rgb_prev)) {
        c->err = "tpmd_stage_tail: stages > 0 need flow_prev and rgb_prev";
        return -1;
    }
    const StageW &s = c->st[j];
    TailArgs a{};
    a.out = out;
    a.feat = s.feat;
    a.wflow = s.wflow;
    a.sflow = s_flow;
    a.fbias = s.fbias;
    a.fup = s.fup;
    a.flow_prev = j > 0 ? flow_prev : nullptr;
    a.flow_cur = flow;
    a.lin = s.lin;
    a.wrgb = s.wrgb;
    a.rlb = s.rlb;
    a.rbias = s.rbias;
    a.rup = s.rup;
    a.rgb_prev = j > 0 ? rgb_prev : nullptr;
    a.rgb_cur = rgb;
    a.s_next = nullptr;
    a.trunk = trunk;
    a.warp_tap = warp;
    a.featg = s.featg;
    a.nframes = n;
    a.r = 8 << j;
    a.C = c->oc[j];
    return c->hip_ok(launch_stage_tail(a, c->f16, false, false, pick_stream(c, stream)), "tail") ? 0 : -1;
}

static int tpmd_stage_conv_tail_body(tpmd_ctx *c, int j, const float *c1, int n, const float *s_conv, const float *s_flow,
                         const float *flow_prev, const float *rgb_prev, float *flow, float *trunk, float *rgb,
                         float *warp, void *stream) {
    if (!check_ctx(c)) return -1;
    if (!c->built || !c->feats_set) {
        c->err = "decoder not built / feats not set";
        return -1;
    }
    if (j < 0 || j >= c->ns || !c1 || !s_conv || !s_flow || !rgb || n < 1) {
        c->err = "tpmd_stage_conv_tail: bad arguments";
        return -1;
    }
    if (j > 0 && (!flow_prev || !rgb_prev)) {
        c->err = "tpmd_stage_conv_tail: stages > 0 need flow_prev and rgb_prev";
        return -1;
    }
    hipStream_t st = pick_stream(c, stream);
    const ConvW &cv = c->conv[2 + 2 * j];
    const int r = 8 << j, C = c->oc[j];
    const int64_t npix = (int64_t) r * r;
    void *xs = c->scratch(1, (size_t) n * npix * C * c->act_size());
    float *den = (float *) c->scratch(2, (size_t) n * C * 4);
    if (!xs || !den) return -1;
    DemodTable t{};
    t.n = 1;
    t.row0[0] = 0;
    t.row0[1] = cv.oc;
    t.ic[0] = cv.ic;
    t.oc[0] = cv.oc;
    t.saug0[0] = cv.saug_off;
    if (!c->hip_ok(launch_demod(c->saug_all, s_conv, den, t, n, st), "demod")) return -1;
    if (!c->hip_ok(launch_prescale_map(c->f16, c1, s_conv, xs, C, npix, n, st), "prescale")) return -1;
    TailArgs a{};
    a.feat = c->st[j].feat;
    a.wflow = c->st[j].wflow;
    a.sflow = s_flow;
    a.fbias = c->st[j].fbias;
    a.fup = c->st[j].fup;
    a.flow_prev = j > 0 ? flow_prev : nullptr;
    a.flow_cur = flow;
    a.lin = c->st[j].lin;
    a.wrgb = c->st[j].wrgb;
    a.rlb = c->st[j].rlb;
    a.rbias = c->st[j].rbias;
    a.rup = c->st[j].rup;
    a.rgb_prev = j > 0 ? rgb_prev : nullptr;
    a.rgb_cur = rgb;
    a.trunk = trunk;
    a.warp_tap = warp;
    a.featg = c->st[j].featg;
    a.nframes = n;
    a.r = r;
    a.C = C;
    ConvArgs ca;
    ca.mode = 0;
    ca.f16 = c->f16;
    ca.A = cv.A;
    ca.A_perm = cv.A_perm;
    ca.X = xs;
    ca.inv_den = den;
    ca.bias = cv.bias;
    ca.nframes = n;
    ca.H = r;
    ca.W = r;
    ca.IC = C;
    ca.OC = C;
    ca.x_bstride = npix * C;
    ca.ws_elems = modconv_ws_elems(0, n, r, r, C, C, c->f16);
    if (ca.ws_elems > 0) {
        ca.ws = (float *) c->scratch(3, (size_t) ca.ws_elems * 4);
        if (!ca.ws) return -1;
    }
    if (fused_tail(c, C, r)) {
        ca.tail = &a;
        return c->hip_ok(launch_modconv(ca, st), "conv+tail") ? 0 : -1;
    }
    float *out = (float *) c->scratch(0, (size_t) n * npix * C * 4);
    if (!out) return -1;
    ca.Y = out;
    if (!c->hip_ok(launch_modconv(ca, st), "conv")) return -1;
    a.out = out;
    return c->hip_ok(launch_stage_tail(a, c->f16, false, false, st), "tail") ? 0 : -1;
}

// ---- op-level

int tpmd_gather(const void *feat, int feat_f16, int C, int W, int H, const float *grid, int64_t N,
                int planar, int sp, float *dst, void *stream) {
    if (C < 1 || W < 1 || H < 1 || N < 0) return -1;
    if (N == 0) return 0;  // nothing to sample (empty tensors may carry null pointers)
    if (!feat || !grid || !dst) return -1;
    return launch_gather(feat, feat_f16 != 0, grid, dst, C, W, H, N, planar, sp, (hipStream_t) stream) ==
                   hipSuccess
               ? 0
               : -1;
}

int tpmd_gather_taps(const float *grid, int W, int H, int64_t N, int planar, int32_t *x0, int32_t *y0,
                     float *wx, float *wy, void *stream) {
    if (W < 1 || H < 1 || N < 0) return -1;
    if (N == 0) return 0;
    if (!grid || !x0 || !y0 || !wx || !wy) return -1;
    return launch_gather_taps(grid, W, H, N, planar, x0, y0, wx, wy, (hipStream_t) stream) == hipSuccess ? 0
                                                                                                      : -1;
}

int tpmd_frames_to_rgb24(const float *chw, int n, int R, uint8_t *rgb, void *stream) {
    if (n < 0 || R < 1 || (R * R) % 4 != 0) return -1;
    if (n == 0) return 0;
    if (!chw || !rgb) return -1;
    return launch_rgb24(chw, n, R, rgb, (hipStream_t) stream) == hipSuccess ? 0 : -1;
}

int tpmd_upfirdn2x(const float *x, const float *k4, float *y, int W, int H, int64_t CB, void *stream) {
    if (!x || !k4 || !y || W < 1 || H < 1 || CB < 0) return -1;
    return launch_upfirdn2x(x, k4, y, W, H, CB, (hipStream_t) stream) == hipSuccess ? 0 : -1;
}

int tpmd_flow_grid(const float *fl, const float *xs, float *y, int64_t N, void *stream) {
    if (!fl || !xs || !y || N < 0) return -1;
    return launch_flow_grid(fl, xs, y, N, (hipStream_t) stream) == hipSuccess ? 0 : -1;
}


// ---- entry points that allocate host memory, exception-safe

tpmd_ctx *tpmd_create(int device, const char *ftype, int n_stages, const int *stage_ic,
                      const int *stage_oc) {
    return guarded((void *) nullptr, [&] { return tpmd_create_body(device, ftype, n_stages, stage_ic, stage_oc); });
}

int tpmd_set_weight(tpmd_ctx *c, const char *name, const float *data, int64_t n, int flags) {
    return guarded(c, [&] { return tpmd_set_weight_body(c, name, data, n, flags); });
}

int tpmd_prepare(tpmd_ctx *c) {
    return guarded(c, [&] { return tpmd_prepare_body(c); });
}

int tpmd_build(tpmd_ctx *c, int max_batch) {
    return guarded(c, [&] { return tpmd_build_body(c, max_batch); });
}

int tpmd_decode_batch(tpmd_ctx *c, const float *styles, int n, float *imgs, int on_device) {
    return guarded(c, [&] { return tpmd_decode_batch_body(c, styles, n, imgs, on_device); });
}

int64_t tpmd_decode_frames(tpmd_ctx *c, const float *styles, int64_t n_frames, int format, void *out,
                           tpmd_frame_cb cb, void *ud) {
    return guarded(c, [&] { return tpmd_decode_frames_body(c, styles, n_frames, format, out, cb, ud); });
}

int tpmd_set_tap(tpmd_ctx *c, int kind, int stage, void *dst, int64_t bytes) {
    return guarded(c, [&] { return tpmd_set_tap_body(c, kind, stage, dst, bytes); });
}

int tpmd_modconv(tpmd_ctx *c, int conv, const float *x, int n, int H, int W, const float *s, float *y,
                 void *stream) {
    return guarded(c, [&] { return tpmd_modconv_body(c, conv, x, n, H, W, s, y, stream); });
}

int tpmd_decode_taps(tpmd_ctx *c, const float *style, float *img, tpmd_tap_cb cb, void *ud) {
    return guarded(c, [&] { return tpmd_decode_taps_body(c, style, img, cb, ud); });
}

int tpmd_modconv_static(tpmd_ctx *c, int conv, const float *x, int n, int H, int W, const float *s, float *y,
                        void *stream) {
    return guarded(c, [&] { return tpmd_modconv_static_body(c, conv, x, n, H, W, s, y, stream); });
}

int tpmd_stage_tail(tpmd_ctx *c, int j, const float *out, int n, const float *s_flow, const float *flow_prev,
                    const float *rgb_prev, float *flow, float *trunk, float *rgb, float *warp,
                    void *stream) {
    return guarded(c, [&] { return tpmd_stage_tail_body(c, j, out, n, s_flow, flow_prev, rgb_prev, flow, trunk, rgb, warp, stream); });
}

int tpmd_stage_conv_tail(tpmd_ctx *c, int j, const float *c1, int n, const float *s_conv, const float *s_flow,
                         const float *flow_prev, const float *rgb_prev, float *flow, float *trunk, float *rgb,
                         float *warp, void *stream) {
    return guarded(c, [&] { return tpmd_stage_conv_tail_body(c, j, c1, n, s_conv, s_flow, flow_prev, rgb_prev, flow, trunk, rgb, warp, stream); });
}

}  // extern "C"
