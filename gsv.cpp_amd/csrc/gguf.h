// Minimal GGUF (v2/v3) reader: header, key/values and tensor directory, data read on demand.
// Only what the AR and BERT loaders need (u32/i32/f32 keys; F32, F16, Q8_0 and I8 tensors).
#pragma once

#include <cstdint>
#include <cstdio>
#include <map>
#include <string>
#include <vector>

namespace gsvk {

enum GgmlType : uint32_t { GGML_F32 = 0, GGML_F16 = 1, GGML_Q8_0 = 8, GGML_I8 = 24 };

struct GgufTensor {
    std::string name;
    std::vector<int64_t> ne;   // ggml order: ne[0] is the contiguous dimension
    uint32_t type = 0;
    uint64_t offset = 0;       // absolute file offset of the data
    uint64_t nbytes = 0;
    int64_t rows() const {     // product of ne[1..]
        int64_t r = 1;
        for (size_t i = 1; i < ne.size(); i++) r *= ne[i];
        return r;
    }
};

class GgufFile {
public:
    ~GgufFile();
    // Returns false with a message in err on any problem; io_error tells an unreadable file
    // from a malformed one.
    bool open(const std::string & path, std::string & err, bool * io_error = nullptr);
    const GgufTensor * tensor(const std::string & name) const;
    bool get_u32(const std::string & key, uint32_t & out) const;
    bool get_f32(const std::string & key, float & out) const;
    bool read(const GgufTensor & t, void * dst) const;
    const std::vector<GgufTensor> & tensors() const { return tensors_; }

private:
    FILE * f_ = nullptr;
    uint64_t size_ = 0;
    std::map<std::string, uint64_t> u32_;
    std::map<std::string, float> f32_;
    std::vector<GgufTensor> tensors_;
    std::map<std::string, size_t> index_;
};

}  // namespace gsvk
