// The reference's GGUF reader interface (src/gguf.hpp:20-88: GgmlType, TypeInfo, Tensor, Gguf) over the C ABI, so a
// loader written against fnx::Gguf keeps its shape: t() and i()/f()/s() throw std::runtime_error when missing.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>

#include "../../../include/sfnx_moe.h"

namespace sfnx {

struct TypeInfo {
    int block;   // elements per block
    int bytes;   // bytes per block
};
inline TypeInfo type_info(uint32_t t) {
    TypeInfo ti{};
    if (sfnx_gguf_type_info(t, &ti.block, &ti.bytes) != 0) throw std::runtime_error(sfnx_last_error());
    return ti;
}

struct Tensor {
    std::string name;
    uint32_t type = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    int n_dims = 0;
    const uint8_t* data = nullptr;   // in the mapping
    size_t nbytes = 0;
    int shard = -1;
    size_t row_bytes() const { return (size_t) (ne[0] / type_info(type).block) * type_info(type).bytes; }
    int64_t nrows() const { return ne[1] * ne[2] * ne[3]; }
};

class Gguf {
public:
    explicit Gguf(const std::string& first_shard) {
        if (sfnx_gguf_open(first_shard.c_str(), &g_) != 0) throw std::runtime_error(sfnx_last_error());
    }
    ~Gguf() { sfnx_gguf_close(g_); }
    Gguf(const Gguf&) = delete;
    Gguf& operator=(const Gguf&) = delete;
    const sfnx_gguf* handle() const { return g_; }
    // the tensor, or false when missing
    bool find(const std::string& name, Tensor& t) const {
        sfnx_gguf_tensor info;
        const int r = sfnx_gguf_find(g_, name.c_str(), &info);
        if (r < 0) throw std::runtime_error(sfnx_last_error());
        if (r == 0) return false;
        t.name = name;
        t.type = info.type;
        t.n_dims = info.n_dims;
        for (int d = 0; d < 4; ++d) t.ne[d] = info.ne[d];
        t.data = (const uint8_t*) info.data;
        t.nbytes = info.nbytes;
        t.shard = info.shard;
        return true;
    }
    Tensor t(const std::string& name) const {
        Tensor x;
        if (!find(name, x)) throw std::runtime_error("gguf: tensor " + name + " is missing");
        return x;
    }
    bool has(const std::string& key) const {
        int64_t i;
        double f;
        const char* s;
        return sfnx_gguf_int(g_, key.c_str(), &i) == 1 || sfnx_gguf_float(g_, key.c_str(), &f) == 1 ||
               sfnx_gguf_str(g_, key.c_str(), &s) == 1;
    }
    int64_t i(const std::string& key) const {
        int64_t v;
        if (sfnx_gguf_int(g_, key.c_str(), &v) != 1) throw std::runtime_error("gguf: no integer key " + key);
        return v;
    }
    double f(const std::string& key) const {
        double v;
        if (sfnx_gguf_float(g_, key.c_str(), &v) != 1) throw std::runtime_error("gguf: no number key " + key);
        return v;
    }
    double num(const std::string& key) const { return f(key); }
    std::string s(const std::string& key) const {
        const char* v;
        if (sfnx_gguf_str(g_, key.c_str(), &v) != 1) throw std::runtime_error("gguf: no string key " + key);
        return v;
    }
    int n_tensors() const { return sfnx_gguf_n_tensors(g_); }

private:
    sfnx_gguf* g_ = nullptr;
};

}  // namespace sfnx
