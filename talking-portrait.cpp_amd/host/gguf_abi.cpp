// The C entry points of include/tpmd.h that read GGUF files:
// tpmd_load_gguf / tpme_load_gguf / tpfm_read_config / tpfm_load_gguf /
// tpmd_gguf_read_tensor.  No exception leaves an entry point: a failed host
// allocation or any other C++ exception becomes a -1 return with a message.
#include <cstdio>
#include <cstring>
#include <new>
#include <stdexcept>

#include "gguf.h"
#include "tpmd.h"

// ---------------------------------------------------------------------------
namespace {

using put_fn = void (*)(char *, size_t, const std::string &);
void put_err(char *err, size_t err_size, const std::string &m) {
    if (err && err_size) snprintf(err, err_size, "%s", m.c_str());
}

// an entry point's body with every C++ exception turned into -1 + message
template <typename F>
int64_t guarded(char *err, size_t err_size, F &&body) {
    try {
        return body();
    } catch (const std::bad_alloc &) {
        put_err(err, err_size, "out of host memory");
    } catch (const std::exception &e) {
        put_err(err, err_size, std::string("internal error: ") + e.what());
    }
    return -1;
}

// every tensor a context lists (name_of(i) until null) that the file holds,
// handed to set(name, data, n, flags); missing ones are left for prepare()
// to name.  Returns 0, or -1 with the message in err.
template <typename NameOf, typename Set, typename LastErr>
int load_listed(const tp::gguf_file &f, const char *path, NameOf name_of, Set set, LastErr last_error,
                char *err, size_t err_size) {
    std::vector<float> v;
    std::string e;
    for (int i = 0;; i++) {
        int64_t n = 0;
        const char *name = name_of(i, &n);
        if (!name) return 0;
        if (!f.find(name)) continue;
        bool f16 = false;
        if (!f.read(name, v, f16, e)) {
            put_err(err, err_size, e);
            return -1;
        }
        if ((int64_t) v.size() != n) {
            put_err(err, err_size, std::string(path) + ": tensor " + name + " has " + std::to_string(v.size()) +
                                       " elements, expected " + std::to_string(n));
            return -1;
        }
        if (set(name, v.data(), n, f16 ? TPMD_W_F16_FILE : 0) != 0) {
            put_err(err, err_size, last_error());
            return -1;
        }
    }
}

}  // namespace

extern "C" {

int tpmd_load_gguf(tpmd_ctx *ctx, const char *path, char *err, size_t err_size) {
    return (int) guarded(err, err_size, [&]() -> int64_t {
        if (!ctx || !path) return put_err(err, err_size, "tpmd_load_gguf: null context or path"), -1;
        tp::gguf_file f;
        std::string e;
        if (!f.open(path, "float-motion-ae", e)) return put_err(err, err_size, e), -1;
        return load_listed(
            f, path, [&](int i, int64_t *n) { return tpmd_weight_name(ctx, i, n, nullptr); },
            [&](const char *nm, const float *d, int64_t n, int fl) { return tpmd_set_weight(ctx, nm, d, n, fl); },
            [&] { return std::string(tpmd_last_error(ctx)); }, err, err_size);
    });
}

int tpme_load_gguf(tpme_ctx *ctx, const char *path, char *err, size_t err_size) {
    return (int) guarded(err, err_size, [&]() -> int64_t {
        if (!ctx || !path) return put_err(err, err_size, "tpme_load_gguf: null context or path"), -1;
        tp::gguf_file f;
        std::string e;
        if (!f.open(path, "float-motion-ae", e)) return put_err(err, err_size, e), -1;
        return load_listed(
            f, path, [&](int i, int64_t *n) { return tpme_weight_name(ctx, i, n, nullptr); },
            [&](const char *nm, const float *d, int64_t n, int fl) { return tpme_set_weight(ctx, nm, d, n, fl); },
            [&] { return std::string(tpme_last_error(ctx)); }, err, err_size);
    });
}

int tpfm_read_config(const char *path, tpfm_config *cfg, char *err, size_t err_size) {
    return (int) guarded(err, err_size, [&]() -> int64_t {
        if (!path || !cfg) return put_err(err, err_size, "tpfm_read_config: null path or config"), -1;
        tp::gguf_file f;
        std::string e;
        if (!f.open(path, "float-fmt", e)) return put_err(err, err_size, e), -1;
        tpfm_default_config(cfg);
        auto num = [&](const char *key, double def) {
            auto it = f.kv_num.find(std::string("float.fmt.") + key);
            return it == f.kv_num.end() ? def : it->second;
        };
        // the float.fmt.* hyper-parameters over the defaults (src/fmt.cpp:10-26)
        struct { const char *key; int *v; } ints[] = {
            {"dim_h", &cfg->dim_h}, {"depth", &cfg->depth}, {"n_heads", &cfg->n_heads},
            {"dim_w", &cfg->dim_w}, {"dim_a", &cfg->dim_a}, {"dim_e", &cfg->dim_e},
            {"chunk_frames", &cfg->chunk_frames}, {"prev_frames", &cfg->prev_frames},
            {"attn_window", &cfg->attn_window}, {"t_freq_dim", &cfg->t_freq_dim}, {"nfe", &cfg->nfe}};
        for (auto &k : ints) *k.v = (int) num(k.key, *k.v);
        struct { const char *key; float *v; } flts[] = {
            {"a_cfg_scale", &cfg->a_cfg}, {"e_cfg_scale", &cfg->e_cfg}, {"r_cfg_scale", &cfg->r_cfg},
            {"ln_eps", &cfg->ln_eps}, {"mlp_ratio", &cfg->mlp_ratio}};
        for (auto &k : flts) *k.v = (float) num(k.key, *k.v);
        const double total = num("num_total_frames", cfg->chunk_frames + cfg->prev_frames);
        if ((int) total != cfg->chunk_frames + cfg->prev_frames)
            return put_err(err, err_size, std::string(path) + ": num_total_frames != chunk_frames + prev_frames"),
                   -1;
        return 0;
    });
}

int tpfm_load_gguf(tpfm_ctx *ctx, const char *path, char *err, size_t err_size) {
    return (int) guarded(err, err_size, [&]() -> int64_t {
        if (!ctx || !path) return put_err(err, err_size, "tpfm_load_gguf: null context or path"), -1;
        tp::gguf_file f;
        std::string e;
        if (!f.open(path, "float-fmt", e)) return put_err(err, err_size, e), -1;
        return load_listed(
            f, path, [&](int i, int64_t *n) { return tpfm_weight_name(ctx, i, n, nullptr); },
            [&](const char *nm, const float *d, int64_t n, int fl) { return tpfm_set_weight(ctx, nm, d, n, fl); },
            [&] { return std::string(tpfm_last_error(ctx)); }, err, err_size);
    });
}

int64_t tpmd_gguf_read_tensor(const char *path, const char *name, float *out, int64_t cap, int *is_f16,
                              char *err, size_t err_size) {
    return guarded(err, err_size, [&]() -> int64_t {
        if (!path || !name) return put_err(err, err_size, "tpmd_gguf_read_tensor: null path or name"), -1;
        tp::gguf_file f;
        std::string e;
        if (!f.open(path, nullptr, e)) return put_err(err, err_size, e), -1;
        const tp::gguf_file::tensor *t = f.find(name);
        if (!t) return put_err(err, err_size, std::string("missing tensor ") + name), -1;
        if (is_f16) *is_f16 = t->type == 1 ? 1 : 0;
        if (!out) return t->n;
        if (cap < t->n) return put_err(err, err_size, "tpmd_gguf_read_tensor: buffer too small"), -1;
        std::vector<float> v;
        bool f16 = false;
        if (!f.read(name, v, f16, e)) return put_err(err, err_size, e), -1;
        if (!v.empty()) memcpy(out, v.data(), v.size() * 4);
        return (int64_t) v.size();
    });
}

}  // extern "C"
