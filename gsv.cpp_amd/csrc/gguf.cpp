// Minimal GGUF reader (format: ggml's gguf.h / docs/gguf.md; written by
// tools/export_gguf/convert_ar.py through gguf-py).
#include "gguf.h"

#include <cstring>

namespace gsvk {

namespace {

enum : uint32_t {
    T_U8 = 0, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64
};

struct Reader {
    FILE * f;
    uint64_t size;
    bool bad = false;

    bool bytes(void * dst, size_t n) {
        if (bad) return false;
        if (fread(dst, 1, n, f) != n) bad = true;
        return !bad;
    }
    uint32_t u32() { uint32_t v = 0; bytes(&v, 4); return v; }
    uint64_t u64() { uint64_t v = 0; bytes(&v, 8); return v; }
    bool str(std::string & s) {
        const uint64_t n = u64();
        if (bad || n > (1u << 20)) { bad = true; return false; }
        s.resize(n);
        return n == 0 || bytes(&s[0], n);
    }
    bool skip(uint64_t n) {
        if (bad) return false;
        if (fseeko(f, (off_t) n, SEEK_CUR) != 0) bad = true;
        return !bad;
    }
    static uint64_t scalar_size(uint32_t t) {
        switch (t) {
            case T_U8: case T_I8: case T_BOOL: return 1;
            case T_U16: case T_I16: return 2;
            case T_U32: case T_I32: case T_F32: return 4;
            case T_U64: case T_I64: case T_F64: return 8;
            default: return 0;
        }
    }
    bool skip_value(uint32_t t, int depth = 0) {
        if (t == T_STR) { std::string s; return str(s); }
        if (t == T_ARR) {
            if (depth > 2) { bad = true; return false; }
            const uint32_t et = u32();
            const uint64_t n = u64();
            if (bad) return false;
            const uint64_t es = scalar_size(et);
            if (es) return skip(es * n);
            for (uint64_t i = 0; i < n && !bad; i++) skip_value(et, depth + 1);
            return !bad;
        }
        const uint64_t s = scalar_size(t);
        if (!s) { bad = true; return false; }
        return skip(s);
    }
};

uint64_t tensor_bytes(uint32_t type, int64_t nelem) {
    switch (type) {
        case GGML_F32: return (uint64_t) nelem * 4;
        case GGML_F16: return (uint64_t) nelem * 2;
        case GGML_Q8_0: return nelem % 32 ? 0 : (uint64_t) (nelem / 32) * 34;
        case GGML_I8: return (uint64_t) nelem;
        default: return 0;
    }
}

}  // namespace

GgufFile::~GgufFile() {
    if (f_) fclose(f_);
}

bool GgufFile::open(const std::string & path, std::string & err, bool * io_error) {
    if (io_error) *io_error = false;
    f_ = fopen(path.c_str(), "rb");
    if (!f_) {
        err = "cannot open " + path;
        if (io_error) *io_error = true;
        return false;
    }
    fseeko(f_, 0, SEEK_END);
    size_ = (uint64_t) ftello(f_);
    fseeko(f_, 0, SEEK_SET);
    Reader r{f_, size_};
    char magic[4];
    if (!r.bytes(magic, 4) || memcmp(magic, "GGUF", 4) != 0) { err = path + ": not a GGUF file"; return false; }
    const uint32_t version = r.u32();
    if (version < 2 || version > 3) { err = path + ": unsupported GGUF version"; return false; }
    const uint64_t n_tensors = r.u64();
    const uint64_t n_kv = r.u64();
    if (r.bad || n_tensors > 100000 || n_kv > 100000) { err = path + ": corrupt header"; return false; }
    uint32_t alignment = 32;
    for (uint64_t i = 0; i < n_kv && !r.bad; i++) {
        std::string key;
        r.str(key);
        const uint32_t t = r.u32();
        if (t == T_U32 || t == T_I32) {
            const uint32_t v = r.u32();
            u32_[key] = v;
            if (key == "general.alignment") alignment = v;
        } else if (t == T_F32) {
            const uint32_t v = r.u32();
            float f;
            memcpy(&f, &v, 4);
            f32_[key] = f;
        } else {
            r.skip_value(t);
        }
    }
    if (alignment == 0 || (alignment & (alignment - 1))) { err = path + ": bad alignment"; return false; }
    tensors_.resize(n_tensors);
    for (uint64_t i = 0; i < n_tensors && !r.bad; i++) {
        GgufTensor & t = tensors_[i];
        r.str(t.name);
        const uint32_t nd = r.u32();
        if (nd < 1 || nd > 4) { r.bad = true; break; }
        t.ne.resize(nd);
        int64_t nel = 1;
        for (uint32_t d = 0; d < nd; d++) {
            t.ne[d] = (int64_t) r.u64();
            if (t.ne[d] <= 0 || t.ne[d] > (1ll << 32)) r.bad = true;
            nel *= t.ne[d];
        }
        t.type = r.u32();
        t.offset = r.u64();
        t.nbytes = tensor_bytes(t.type, nel);
        index_[t.name] = i;
    }
    if (r.bad) { err = path + ": truncated or corrupt tensor directory"; return false; }
    const uint64_t pos = (uint64_t) ftello(f_);
    const uint64_t data = (pos + alignment - 1) / alignment * alignment;
    for (GgufTensor & t : tensors_) {
        t.offset += data;
        if (t.nbytes && t.offset + t.nbytes > size_) {
            err = path + ": tensor " + t.name + " extends past the end of the file";
            return false;
        }
    }
    return true;
}

const GgufTensor * GgufFile::tensor(const std::string & name) const {
    auto it = index_.find(name);
    return it == index_.end() ? nullptr : &tensors_[it->second];
}

bool GgufFile::get_u32(const std::string & key, uint32_t & out) const {
    auto it = u32_.find(key);
    if (it == u32_.end()) return false;
    out = (uint32_t) it->second;
    return true;
}

bool GgufFile::get_f32(const std::string & key, float & out) const {
    auto it = f32_.find(key);
    if (it == f32_.end()) return false;
    out = it->second;
    return true;
}

bool GgufFile::read(const GgufTensor & t, void * dst) const {
    if (!t.nbytes) return false;
    if (fseeko(f_, (off_t) t.offset, SEEK_SET) != 0) return false;
    return fread(dst, 1, t.nbytes, f_) == t.nbytes;
}

}  // namespace gsvk
