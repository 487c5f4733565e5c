// tp::motion_dec over the MI355X decoder library (include/tpmd.h).
//
// Keeps the reference's motion_dec interface (src/motion_dec.h:10-49) method
// for method, so the generation loop (src/pipeline.cpp:153-185), tp-bench's
// mdec row (bench/tp-bench.cpp:133-152) and tp_ctx (src/tp_ctx.h:11-21) call
// it unchanged:
//
//   prepare(be, err)                  once after the weights are loaded
//   build(be, with_taps, err)         persistent buffers, `batch` frames/call
//   set_feats(menc_result, err)       once per portrait
//   decode(be, style, img, tap, err)  one frame
//   decode_batch(be, styles, imgs, err)   `batch` frames
//   release()
//
// The ggml types of the reference signatures are replaced by what this
// library needs from them:
//   backend_t   -> hip_backend   (device ordinal + ftype, src/backend.cpp:9-57)
//   weights_t   -> weight_source (name -> raw f32 values, src/gguf_load.cpp)
//   tap_sink    -> any type with the reference's tap_sink members `wr` (a
//                  tap_writer with add_f32(name, data, torch_shape) and `err`,
//                  src/dump.h:13-24) and `prefix`, and its bool test: a
//                  decode that asks for taps runs the library's tap plan
//                  (tpmd_decode_taps) and writes the reference's tap names
//                  (src/motion_dec.cpp:805-883) through it.
// Error contract as the reference: false + err, no exceptions.
#pragma once

#include <string>
#include <type_traits>
#include <utility>
#include <vector>

#include "tpmd.h"

namespace tp {

// decoder weights by GGUF name: f32 values in torch layout as stored in the
// file (before the load-time scale folding), plus whether the file holds
// the tensor in f16.  The adapter in the reference tree implements this over
// weights_t (ggml_backend_tensor_get + the f16 type of the GGUF tensor).
struct weight_source {
    virtual ~weight_source() = default;
    virtual bool get(const std::string &name, std::vector<float> &data, bool &f16_in_file) const = 0;
};

// the device the decoder runs on.  stage_ic/stage_oc empty = the reference's
// channel plan (src/motion_dec.cpp:12-13); n_stages < 7 truncates the
// pyramid like TP_MDEC_STAGES (src/motion_dec.cpp:787-792).
struct hip_backend {
    int device = 0;
    std::string ftype = "f16";
    int n_stages = 7;
    std::vector<int> stage_ic, stage_oc;
    void *stream = nullptr;  // hipStream_t to enqueue on; null = the library's own
};

struct motion_dec {
    const weight_source *w = nullptr;  // borrowed, like the reference's weights_t *

    tpmd_ctx *ctx = nullptr;
    bool built = false;
    bool taps_in_graph = false;  // build(be, true) was asked for (decode then serves taps)
    int batch = 1;               // frames per decode_batch call
    int img_chunks = 0;          // 1 once the batched plan is built
    int res = 512;

    static const int N_STAGES = 7;
    static const int MAX_BATCH = 256;

    bool prepare(hip_backend &be, std::string &err);
    // batch = TP_MDEC_BATCH (default 8, as src/motion_dec.cpp:752-762), 1..MAX_BATCH
    bool build(hip_backend &be, bool with_taps, std::string &err);
    // m.feats[j]: [OC_j * r_j * r_j] pixel-major channel-fastest (menc_result)
    template <class Menc>
    bool set_feats(const Menc &m, std::string &err) {
        return set_feats_vec(m.feats, err);
    }
    bool set_feats_vec(const std::vector<std::vector<float>> &feats, std::string &err);
    bool decode(hip_backend &be, const float *style, float *img_out, std::string &err);
    template <class Tap>
    bool decode(hip_backend &be, const float *style, float *img_out, Tap &tap, std::string &err) {
        if (!tap) return decode(be, style, img_out, err);
        if constexpr (!has_tap_writer<Tap>::value) {
            err = "motion_dec: taps need a sink with a tap writer (wr->add_f32) and a prefix";
            return false;
        } else {
            return decode_taps(style, img_out, tap, err);
        }
    }
    bool decode_batch(hip_backend &be, const float *styles, float *imgs_out, std::string &err);

    void release();
    ~motion_dec() { release(); }

  private:
    // Tap has the reference tap_sink's `wr` (with add_f32 and err) and `prefix`
    template <class T, class = void>
    struct has_tap_writer : std::false_type {};
    template <class T>
    struct has_tap_writer<T, std::void_t<decltype(std::declval<T &>().wr->add_f32(
                                 std::declval<T &>().prefix + "", (const float *) nullptr,
                                 std::vector<int64_t>()))>> : std::true_type {};
    template <class Tap>
    bool decode_taps(const float *style, float *img_out, Tap &tap, std::string &err) {
        if (!ctx || !built) {
            err = "decoder not built";
            return false;
        }
        struct sink_t {
            Tap *tap;
            std::string err;
        } sink{&tap, {}};
        auto put = [](const char *name, const float *data, int ndim, const int64_t *shape, void *ud) -> int {
            sink_t *s = (sink_t *) ud;
            const std::vector<int64_t> sh(shape, shape + ndim);
            if (s->tap->wr->add_f32(s->tap->prefix + name, data, sh)) return 0;
            s->err = s->tap->wr->err;
            return 1;
        };
        if (tpmd_decode_taps(ctx, style, img_out, put, &sink) != 0) {
            err = !sink.err.empty() ? sink.err : tpmd_last_error(ctx);
            return false;
        }
        return true;
    }

    std::vector<size_t> feat_sizes;  // elements of feats[j] for this channel plan
    bool fail(std::string &err, const char *what);
};

// weight names whose host copies prepare() reads (src/motion_dec.cpp:17-29):
// here every decoder tensor, since prepare() uploads everything itself
std::vector<std::string> motion_dec_host_tensors(const hip_backend &be);

}  // namespace tp
