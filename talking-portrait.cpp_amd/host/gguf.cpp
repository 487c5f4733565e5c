// GGUF v3 reader (see gguf.h).  Plain C++ with no device code: the library
// links it, and host/Makefile.sanitize builds it with AddressSanitizer and
// UndefinedBehaviorSanitizer under the gguf_check driver.
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>

namespace tp {

namespace {

// metadata value types of the format
enum : uint32_t {
    GT_U8 = 0, GT_I8, GT_U16, GT_I16, GT_U32, GT_I32, GT_F32, GT_BOOL, GT_STRING, GT_ARRAY,
    GT_U64, GT_I64, GT_F64,
};

// bytes of a fixed-size value type; 0 for string and array, -1 unknown
int fixed_bytes(uint32_t t) {
    switch (t) {
        case GT_U8: case GT_I8: case GT_BOOL: return 1;
        case GT_U16: case GT_I16: return 2;
        case GT_U32: case GT_I32: case GT_F32: return 4;
        case GT_U64: case GT_I64: case GT_F64: return 8;
        case GT_STRING: case GT_ARRAY: return 0;
        default: return -1;
    }
}

template <typename T>
T load_le(const uint8_t *p) {
    T v;
    memcpy(&v, p, sizeof v);  // the format and the host are little-endian
    return v;
}

// a fixed-size scalar as a double (bool as 0 / 1)
double number_of(uint32_t t, const uint8_t *p) {
    switch (t) {
        case GT_U8: return p[0];
        case GT_I8: return (int8_t) p[0];
        case GT_BOOL: return p[0] ? 1.0 : 0.0;
        case GT_U16: return load_le<uint16_t>(p);
        case GT_I16: return load_le<int16_t>(p);
        case GT_U32: return load_le<uint32_t>(p);
        case GT_I32: return load_le<int32_t>(p);
        case GT_F32: return load_le<float>(p);
        case GT_U64: return (double) load_le<uint64_t>(p);
        case GT_I64: return (double) load_le<int64_t>(p);
        default: return load_le<double>(p);
    }
}

// bounds-checked sequential reads over the mapped file; a read that would
// run past the end fails and the parse stops there
class span_reader {
  public:
    span_reader(const uint8_t *b, uint64_t n) : b_(b), n_(n) {}
    uint64_t pos() const { return pos_; }
    bool take(uint64_t len, const uint8_t *&p) {
        if (len > n_ - pos_) return false;
        p = b_ + pos_;
        pos_ += len;
        return true;
    }
    template <typename T>
    bool scalar(T &v) {
        const uint8_t *p;
        if (!take(sizeof(T), p)) return false;
        v = load_le<T>(p);
        return true;
    }
    bool text(std::string &s) {
        uint64_t len;
        const uint8_t *p;
        if (!scalar(len) || !take(len, p)) return false;
        s.assign((const char *) p, (size_t) len);
        return true;
    }

  private:
    const uint8_t *b_;
    uint64_t n_, pos_ = 0;
};

enum class walk { ok, truncated, bad_type };

// one metadata value of type t: scalars into *num, strings into *str,
// arrays (of any element type, nested up to 4 deep) walked and dropped
walk walk_value(span_reader &r, uint32_t t, int depth, double *num, std::string *str) {
    const int fb = fixed_bytes(t);
    if (fb < 0) return walk::bad_type;
    if (fb > 0) {
        const uint8_t *p;
        if (!r.take((uint64_t) fb, p)) return walk::truncated;
        if (num) *num = number_of(t, p);
        return walk::ok;
    }
    if (t == GT_STRING) {
        std::string s;
        if (!r.text(s)) return walk::truncated;
        if (str) *str = std::move(s);
        return walk::ok;
    }
    uint32_t et;
    uint64_t count;
    if (!r.scalar(et) || !r.scalar(count)) return walk::truncated;
    const int efb = fixed_bytes(et);
    if (efb < 0 || (et == GT_ARRAY && depth >= 4)) return walk::bad_type;
    if (efb > 0) {
        uint64_t bytes;
        const uint8_t *p;
        if (__builtin_mul_overflow(count, (uint64_t) efb, &bytes) || !r.take(bytes, p)) return walk::truncated;
        return walk::ok;
    }
    // strings / arrays: each element takes at least 8 bytes, so a count
    // beyond the file ends at the first truncated element
    for (uint64_t i = 0; i < count; i++) {
        const walk w = walk_value(r, et, depth + 1, nullptr, nullptr);
        if (w != walk::ok) return w;
    }
    return walk::ok;
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

void gguf_file::unmap() {
    if (base_ && size_) munmap((void *) base_, (size_t) size_);
    base_ = nullptr;
    size_ = 0;
}

bool gguf_file::open(const std::string &path, const char *expect_arch, std::string &err) {
    unmap();
    path_ = path;
    kv_num.clear();
    kv_str.clear();
    tensors.clear();
    index_.clear();
    auto bad = [&](const std::string &what) {
        err = path + ": " + what;
        return false;
    };
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return bad("cannot open");
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 0) {
        ::close(fd);
        return bad("cannot stat");
    }
    size_ = (uint64_t) st.st_size;
    if (size_ > 0) {
        void *m = mmap(nullptr, (size_t) size_, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            ::close(fd);
            size_ = 0;
            return bad("cannot map");
        }
        base_ = (const uint8_t *) m;
    }
    ::close(fd);

    span_reader r(base_, size_);
    const uint8_t *magic;
    if (!r.take(4, magic) || memcmp(magic, "GGUF", 4) != 0) return bad("not a GGUF file");
    uint32_t version;
    if (!r.scalar(version) || version != 3) return bad("unsupported GGUF version");
    uint64_t n_tensors, n_kv;
    // a metadata pair takes at least 12 bytes and a tensor record 24
    if (!r.scalar(n_tensors) || !r.scalar(n_kv) || n_kv > size_ / 12 || n_tensors > size_ / 24)
        return bad("corrupt header");

    for (uint64_t i = 0; i < n_kv; i++) {
        std::string key;
        uint32_t vt;
        if (!r.text(key) || !r.scalar(vt)) return bad("truncated KV section");
        double num = 0;
        std::string str;
        const bool scalar = fixed_bytes(vt) > 0;
        const walk w = walk_value(r, vt, 0, scalar ? &num : nullptr, vt == GT_STRING ? &str : nullptr);
        if (w == walk::truncated) return bad("truncated KV section");
        if (w == walk::bad_type) return bad("unsupported KV type " + std::to_string(vt) + " for " + key);
        if (scalar) kv_num[key] = num;
        if (vt == GT_STRING) kv_str[key] = std::move(str);
    }
    if (expect_arch) {
        auto it = kv_str.find("general.architecture");
        if (it == kv_str.end() || it->second != expect_arch)
            return bad("unexpected architecture '" + (it == kv_str.end() ? std::string("<none>") : it->second) +
                       "', want " + expect_arch);
    }
    uint64_t align = 32;
    if (auto al = kv_num.find("general.alignment"); al != kv_num.end()) {
        const double a = al->second;
        if (!(a >= 1 && a <= 65536) || a != (double) (uint64_t) a || ((uint64_t) a & ((uint64_t) a - 1)))
            return bad("corrupt header (general.alignment)");
        align = (uint64_t) a;
    }

    tensors.resize((size_t) n_tensors);
    for (size_t i = 0; i < tensors.size(); i++) {
        tensor &t = tensors[i];
        uint32_t nd;
        if (!r.text(t.name) || !r.scalar(nd)) return bad("truncated tensor info section");
        if (nd > 8) return bad("corrupt tensor info");
        uint64_t n = 1;
        bool too_big = false;
        t.dims.resize(nd);
        for (auto &d : t.dims) {
            if (!r.scalar(d)) return bad("truncated tensor info section");
            too_big = too_big || __builtin_mul_overflow(n, d, &n);
        }
        if (!r.scalar(t.type) || !r.scalar(t.offset)) return bad("truncated tensor info section");
        if (t.type > 1) return bad("tensor " + t.name + " has unsupported type");
        // 2^60 elements of at most 4 bytes keep every byte count below 2^64
        if (too_big || n > ((uint64_t) 1 << 60)) return bad("tensor " + t.name + " out of bounds");
        t.n = (int64_t) n;
        if (!index_.emplace(t.name, i).second) return bad("duplicate tensor " + t.name);
    }
    // the data section starts at the next multiple of the alignment
    data_start_ = (r.pos() + align - 1) / align * align;
    const uint64_t avail = size_ > data_start_ ? size_ - data_start_ : 0;
    for (const tensor &t : tensors) {
        const uint64_t bytes = (uint64_t) t.n * (t.type == 0 ? 4 : 2);
        if (t.offset > avail || bytes > avail - t.offset) return bad("tensor " + t.name + " out of bounds");
    }
    return true;
}

const gguf_file::tensor *gguf_file::find(const std::string &name) const {
    auto it = index_.find(name);
    return it == index_.end() ? nullptr : &tensors[it->second];
}

bool gguf_file::read(const std::string &name, std::vector<float> &out, bool &f16, std::string &err) const {
    const tensor *t = find(name);
    if (!t) {
        err = "missing tensor " + name;
        return false;
    }
    const uint8_t *src = base_ + data_start_ + t->offset;  // in bounds: checked by open()
    out.resize((size_t) t->n);
    f16 = t->type == 1;
    if (!f16) {
        if (t->n) memcpy(out.data(), src, (size_t) t->n * 4);
    } else {
        for (int64_t j = 0; j < t->n; j++) out[(size_t) j] = half_to_float(load_le<uint16_t>(src + 2 * j));
    }
    return true;
}

bool gguf_weight_source::get(const std::string &name, std::vector<float> &data, bool &f16_in_file) const {
    std::string err;
    return f && f->read(name, data, f16_in_file, err);
}

}  // namespace tp

