// GGUF v3 reader for the decoder's checkpoints (motion_ae_{f32,f16}.gguf,
// float-fmt .gguf), written from the GGUF v3 format description:
//
//   header    "GGUF" u32 version (3) u64 tensor_count u64 kv_count
//   kv        string key, u32 value type, value  (types 0..12: u8, i8, u16,
//             i16, u32, i32, f32, bool, string, array, u64, i64, f64; an
//             array is u32 element type, u64 count, elements)
//   tensors   string name, u32 n_dims, u64 dims[n_dims] (ggml order, the
//             reversed torch shape), u32 ggml type, u64 offset
//   padding   to general.alignment (32 when absent)
//   data      tensor bytes at data_start + offset
//
// The file is memory-mapped, so only the tensors read are paged in.  Every
// well-formed metadata value is walked (scalars kept, strings kept, arrays
// skipped); tensors must be F32 (type 0) or F16 (type 1), the checkpoint
// types the reference's loader reads (src/gguf_load.cpp:51-197).  Defects
// are reported with the reference loader's wording ("not a GGUF file",
// "unsupported GGUF version", "tensor <name> out of bounds", ...).  Values
// come back as stored (f16 widened exactly to f32); the load-time scale
// folding and the f16 keep rule are tpmd_set_weight's.
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "motion_dec.h"

namespace tp {

class gguf_file {
  public:
    struct tensor {
        std::string name;
        std::vector<uint64_t> dims;  // ggml order
        uint32_t type = 0;           // 0 = F32, 1 = F16
        uint64_t offset = 0;         // from the start of the data section
        int64_t n = 1;               // elements
    };
    std::map<std::string, double> kv_num;      // numeric and bool scalars
    std::map<std::string, std::string> kv_str;
    std::vector<tensor> tensors;

    gguf_file() = default;
    gguf_file(const gguf_file &) = delete;
    gguf_file &operator=(const gguf_file &) = delete;
    ~gguf_file() { unmap(); }

    // map the file and parse its header and tensor directory; expect_arch
    // (or null) must equal general.architecture.  Errors name the file.
    bool open(const std::string &path, const char *expect_arch, std::string &err);
    // one tensor's values as f32 (exact for f16); f16 = stored as F16
    bool read(const std::string &name, std::vector<float> &out, bool &f16, std::string &err) const;
    const tensor *find(const std::string &name) const;

  private:
    void unmap();
    std::string path_;
    const uint8_t *base_ = nullptr;  // the mapping
    uint64_t size_ = 0;
    uint64_t data_start_ = 0;
    std::map<std::string, size_t> index_;
};

// the decoder's weights from a GGUF file, for motion_dec::prepare
struct gguf_weight_source : weight_source {
    const gguf_file *f = nullptr;
    bool get(const std::string &name, std::vector<float> &data, bool &f16_in_file) const override;
};

// IEEE binary16 -> binary32, exact
float half_to_float(uint16_t h);

}  // namespace tp
