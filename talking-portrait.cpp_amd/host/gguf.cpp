// GGUF v3 reader (see gguf.h) and the C entry points tpmd_load_gguf /
// tpme_load_gguf / tpfm_read_config / tpfm_load_gguf / tpmd_gguf_read_tensor
// of include/tpmd.h.
#include "gguf.h"

#include <cstdio>
#include <cstring>

#include "tpmd.h"

namespace tp {

namespace {

struct cursor {
    const uint8_t *p, *end;
    bool ok = true;
    template <typename T>
    T get() {
        T v{};
        if ((size_t) (end - p) < sizeof(T)) {
            ok = false;
            return v;
        }
        memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!ok || n > (uint64_t) (end - p) || n > (1u << 20)) {
            ok = false;
            return {};
        }
        std::string s((const char *) p, (size_t) n);
        p += n;
        return s;
    }
};

bool read_all(const std::string &path, std::vector<uint8_t> &out, std::string &err) {
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) {
        err = path + ": cannot open";
        return false;
    }
    bool ok = fseek(f, 0, SEEK_END) == 0;
    const long sz = ok ? ftell(f) : -1;
    ok = ok && sz >= 0 && fseek(f, 0, SEEK_SET) == 0;
    if (ok) {
        out.resize((size_t) sz);
        ok = fread(out.data(), 1, out.size(), f) == out.size();
    }
    fclose(f);
    if (!ok) err = path + ": read error";
    return ok;
}

}  // namespace

float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {  // subnormal: m * 2^-24, normalised
            int sh = 0;
            uint32_t mm = m;
            while (!(mm & 0x400u)) {
                mm <<= 1;
                sh++;
            }
            x = sign | ((uint32_t) (113 - sh) << 23) | ((mm & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

bool gguf_file::open(const std::string &path, const char *expect_arch, std::string &err) {
    path_ = path;
    kv_num.clear();
    kv_str.clear();
    tensors.clear();
    index.clear();
    if (!read_all(path, data_, err)) return false;
    cursor c{data_.data(), data_.data() + data_.size()};
    char magic[4];
    for (char &ch : magic) ch = (char) c.get<uint8_t>();
    if (!c.ok || memcmp(magic, "GGUF", 4) != 0) {
        err = path + ": not a GGUF file";
        return false;
    }
    if (c.get<uint32_t>() != 3) {
        err = path + ": unsupported GGUF version";
        return false;
    }
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    if (!c.ok || n_tensors > 100000 || n_kv > 100000) {
        err = path + ": corrupt header";
        return false;
    }
    for (uint64_t i = 0; i < n_kv && c.ok; i++) {
        const std::string key = c.str();
        const uint32_t vt = c.get<uint32_t>();
        switch (vt) {
            case 4: kv_num[key] = c.get<uint32_t>(); break;
            case 5: kv_num[key] = c.get<int32_t>(); break;
            case 6: kv_num[key] = c.get<float>(); break;
            case 7: kv_num[key] = c.get<uint8_t>() ? 1 : 0; break;
            case 8: kv_str[key] = c.str(); break;
            default:
                err = path + ": unsupported KV type " + std::to_string(vt) + " for " + key;
                return false;
        }
    }
    if (!c.ok) {
        err = path + ": truncated KV section";
        return false;
    }
    if (expect_arch) {
        auto it = kv_str.find("general.architecture");
        if (it == kv_str.end() || it->second != expect_arch) {
            err = path + ": unexpected architecture '" + (it == kv_str.end() ? "<none>" : it->second) +
                  "', want " + expect_arch;
            return false;
        }
    }
    tensors.resize((size_t) n_tensors);
    for (auto &t : tensors) {
        t.name = c.str();
        const uint32_t nd = c.get<uint32_t>();
        if (!c.ok || nd > 8) {
            err = path + ": corrupt tensor info";
            return false;
        }
        for (uint32_t j = 0; j < nd; j++) {
            const uint64_t d = c.get<uint64_t>();
            if (d > (1ull << 40)) c.ok = false;
            t.dims.push_back(d);
            t.n *= (int64_t) (d ? d : 1);
        }
        t.type = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        if (c.ok && t.type > 1) {
            err = path + ": tensor " + t.name + " has unsupported type";
            return false;
        }
        if (!c.ok) break;
    }
    if (!c.ok) {
        err = path + ": truncated tensor info section";
        return false;
    }
    uint64_t align = 32;
    auto al = kv_num.find("general.alignment");
    if (al != kv_num.end() && al->second >= 1 && al->second <= 4096) align = (uint64_t) al->second;
    const size_t pre = (size_t) (c.p - data_.data());
    data_off_ = (size_t) ((pre + align - 1) / align * align);
    for (size_t i = 0; i < tensors.size(); i++) {
        const tensor &t = tensors[i];
        const size_t esz = t.type == 0 ? 4 : 2;
        if (t.offset > data_.size() || data_off_ + t.offset + (size_t) t.n * esz > data_.size()) {
            err = path + ": tensor " + t.name + " out of bounds";
            return false;
        }
        index[t.name] = i;
    }
    return true;
}

const gguf_file::tensor *gguf_file::find(const std::string &name) const {
    auto it = index.find(name);
    return it == index.end() ? nullptr : &tensors[it->second];
}

bool gguf_file::read(const std::string &name, std::vector<float> &out, bool &f16, std::string &err) const {
    const tensor *t = find(name);
    if (!t) {
        err = "missing tensor " + name;
        return false;
    }
    const uint8_t *src = data_.data() + data_off_ + t->offset;
    out.resize((size_t) t->n);
    f16 = t->type == 1;
    if (!f16) {
        memcpy(out.data(), src, (size_t) t->n * 4);
    } else {
        for (int64_t j = 0; j < t->n; j++) {
            uint16_t h;
            memcpy(&h, src + 2 * j, 2);
            out[(size_t) j] = half_to_float(h);
        }
    }
    return true;
}

bool gguf_weight_source::get(const std::string &name, std::vector<float> &data, bool &f16_in_file) const {
    std::string err;
    return f && f->read(name, data, f16_in_file, err);
}

}  // namespace tp

// ---------------------------------------------------------------------------
extern "C" {

int tpmd_load_gguf(tpmd_ctx *ctx, const char *path, char *err, size_t err_size) {
    auto fail = [&](const std::string &m) {
        if (err && err_size) snprintf(err, err_size, "%s", m.c_str());
        return -1;
    };
    if (!ctx || !path) return fail("tpmd_load_gguf: null context or path");
    tp::gguf_file f;
    std::string e;
    if (!f.open(path, "float-motion-ae", e)) return fail(e);
    std::vector<float> v;
    for (int i = 0;; i++) {
        int64_t n = 0;
        const char *name = tpmd_weight_name(ctx, i, &n, nullptr);
        if (!name) break;
        if (!f.find(name)) continue;  // prepare() names the first missing tensor
        bool f16 = false;
        if (!f.read(name, v, f16, e)) return fail(e);
        if ((int64_t) v.size() != n)
            return fail(std::string(path) + ": tensor " + name + " has " + std::to_string(v.size()) +
                        " elements, expected " + std::to_string(n));
        if (tpmd_set_weight(ctx, name, v.data(), n, f16 ? TPMD_W_F16_FILE : 0) != 0)
            return fail(tpmd_last_error(ctx));
    }
    return 0;
}

int tpme_load_gguf(tpme_ctx *ctx, const char *path, char *err, size_t err_size) {
    auto fail = [&](const std::string &m) {
        if (err && err_size) snprintf(err, err_size, "%s", m.c_str());
        return -1;
    };
    if (!ctx || !path) return fail("tpme_load_gguf: null context or path");
    tp::gguf_file f;
    std::string e;
    if (!f.open(path, "float-motion-ae", e)) return fail(e);
    std::vector<float> v;
    for (int i = 0;; i++) {
        int64_t n = 0;
        const char *name = tpme_weight_name(ctx, i, &n, nullptr);
        if (!name) break;
        if (!f.find(name)) continue;  // prepare() names the first missing tensor
        bool f16 = false;
        if (!f.read(name, v, f16, e)) return fail(e);
        if ((int64_t) v.size() != n)
            return fail(std::string(path) + ": tensor " + name + " has " + std::to_string(v.size()) +
                        " elements, expected " + std::to_string(n));
        if (tpme_set_weight(ctx, name, v.data(), n, f16 ? TPMD_W_F16_FILE : 0) != 0)
            return fail(tpme_last_error(ctx));
    }
    return 0;
}

int tpfm_read_config(const char *path, tpfm_config *cfg, char *err, size_t err_size) {
    auto fail = [&](const std::string &m) {
        if (err && err_size) snprintf(err, err_size, "%s", m.c_str());
        return -1;
    };
    if (!path || !cfg) return fail("tpfm_read_config: null path or config");
    tp::gguf_file f;
    std::string e;
    if (!f.open(path, "float-fmt", e)) return fail(e);
    tpfm_default_config(cfg);
    auto num = [&](const char *key, double def) {
        auto it = f.kv_num.find(std::string("float.fmt.") + key);
        return it == f.kv_num.end() ? def : it->second;
    };
    // src/fmt.cpp:10-26
    cfg->dim_h = (int) num("dim_h", cfg->dim_h);
    cfg->depth = (int) num("depth", cfg->depth);
    cfg->n_heads = (int) num("n_heads", cfg->n_heads);
    cfg->dim_w = (int) num("dim_w", cfg->dim_w);
    cfg->dim_a = (int) num("dim_a", cfg->dim_a);
    cfg->dim_e = (int) num("dim_e", cfg->dim_e);
    cfg->chunk_frames = (int) num("chunk_frames", cfg->chunk_frames);
    cfg->prev_frames = (int) num("prev_frames", cfg->prev_frames);
    cfg->attn_window = (int) num("attn_window", cfg->attn_window);
    cfg->t_freq_dim = (int) num("t_freq_dim", cfg->t_freq_dim);
    cfg->nfe = (int) num("nfe", cfg->nfe);
    cfg->a_cfg = (float) num("a_cfg_scale", cfg->a_cfg);
    cfg->e_cfg = (float) num("e_cfg_scale", cfg->e_cfg);
    cfg->r_cfg = (float) num("r_cfg_scale", cfg->r_cfg);
    cfg->ln_eps = (float) num("ln_eps", cfg->ln_eps);
    cfg->mlp_ratio = (float) num("mlp_ratio", cfg->mlp_ratio);
    const double total = num("num_total_frames", cfg->chunk_frames + cfg->prev_frames);
    if ((int) total != cfg->chunk_frames + cfg->prev_frames)
        return fail(std::string(path) + ": num_total_frames != chunk_frames + prev_frames");
    return 0;
}

int tpfm_load_gguf(tpfm_ctx *ctx, const char *path, char *err, size_t err_size) {
    auto fail = [&](const std::string &m) {
        if (err && err_size) snprintf(err, err_size, "%s", m.c_str());
        return -1;
    };
    if (!ctx || !path) return fail("tpfm_load_gguf: null context or path");
    tp::gguf_file f;
    std::string e;
    if (!f.open(path, "float-fmt", e)) return fail(e);
    std::vector<float> v;
    for (int i = 0;; i++) {
        int64_t n = 0;
        const char *name = tpfm_weight_name(ctx, i, &n, nullptr);
        if (!name) break;
        if (!f.find(name)) continue;  // prepare() names the first missing tensor
        bool f16 = false;
        if (!f.read(name, v, f16, e)) return fail(e);
        if ((int64_t) v.size() != n)
            return fail(std::string(path) + ": tensor " + name + " has " + std::to_string(v.size()) +
                        " elements, expected " + std::to_string(n));
        if (tpfm_set_weight(ctx, name, v.data(), n, f16 ? TPMD_W_F16_FILE : 0) != 0)
            return fail(tpfm_last_error(ctx));
    }
    return 0;
}

int64_t tpmd_gguf_read_tensor(const char *path, const char *name, float *out, int64_t cap, int *is_f16,
                              char *err, size_t err_size) {
    auto fail = [&](const std::string &m) -> int64_t {
        if (err && err_size) snprintf(err, err_size, "%s", m.c_str());
        return -1;
    };
    if (!path || !name) return fail("tpmd_gguf_read_tensor: null path or name");
    tp::gguf_file f;
    std::string e;
    if (!f.open(path, nullptr, e)) return fail(e);
    std::vector<float> v;
    bool f16 = false;
    if (!f.read(name, v, f16, e)) return fail(e);
    if (is_f16) *is_f16 = f16 ? 1 : 0;
    if (out) {
        if (cap < (int64_t) v.size()) return fail("tpmd_gguf_read_tensor: buffer too small");
        memcpy(out, v.data(), v.size() * 4);
    }
    return (int64_t) v.size();
}

}  // extern "C"
