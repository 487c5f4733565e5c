// GGUF v3 reader for the decoder's checkpoint (motion_ae_{f32,f16}.gguf).
//
// Follows the format conventions of the reference's loader
// (src/gguf_load.cpp:51-197): little-endian "GGUF" v3 header, KV values of
// type u32 / i32 / f32 / bool / string only, tensor dims stored in ggml order
// (reversed torch shape), tensor types F32 (0) or F16 (1), data section
// aligned to 32 bytes (or general.alignment when present), offsets relative
// to it.  Values are returned as stored in the file (f16 widened exactly to
// f32); the load-time scale folding and the f16 keep rule are applied by
// tpmd_set_weight, as the reference's weights_t::load does after reading.
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "motion_dec.h"

namespace tp {

struct gguf_file {
    struct tensor {
        std::string name;
        std::vector<uint64_t> dims;  // ggml order
        uint32_t type = 0;           // 0 = F32, 1 = F16
        uint64_t offset = 0;         // relative to the data section
        int64_t n = 1;               // elements
    };
    std::map<std::string, double> kv_num;
    std::map<std::string, std::string> kv_str;
    std::vector<tensor> tensors;
    std::map<std::string, size_t> index;

    // parse the header and tensor directory; expect_arch (or null) must match
    // general.architecture.  Errors name the file and the defect.
    bool open(const std::string &path, const char *expect_arch, std::string &err);
    // one tensor's values as f32 (exact for f16); f16 = stored as F16
    bool read(const std::string &name, std::vector<float> &out, bool &f16, std::string &err) const;
    const tensor *find(const std::string &name) const;

  private:
    std::string path_;
    std::vector<uint8_t> data_;
    size_t data_off_ = 0;
};

// the decoder's weights from a GGUF file, for motion_dec::prepare
struct gguf_weight_source : weight_source {
    const gguf_file *f = nullptr;
    bool get(const std::string &name, std::vector<float> &data, bool &f16_in_file) const override;
};

// IEEE binary16 -> binary32, exact
float half_to_float(uint16_t h);

}  // namespace tp
