// GGUF model files on the host: a read-only mapping of every shard, the tensor index and the metadata, and the loader
// that slices one layer's expert tensors and router into the device store (src/gguf.hpp:20-88, src/gguf.cpp,
// src/model.cpp:554-606 and 766-809).  Host code only: the device work is a copy and sfnx_store_pack.
//
// The file format (GGUF v2/v3, little-endian): "GGUF", version u32, tensor count u64, key/value count u64; each key is a
// string (u64 length + bytes) with a u32 value type and its value (arrays: element type u32, count u64, elements); each
// tensor is a name, n_dims u32, ne[n_dims] u64, ggml type u32 and a data offset u64; the data section starts at the
// next multiple of general.alignment (32 when absent) after the tensor list.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <memory>
#include <regex>
#include <string>
#include <vector>

#include <hip/hip_runtime.h>

#include "common.hpp"

namespace sfnx {
void set_error(const std::string& msg);
}

struct sfnx_gguf {
    struct Map {
        void* base = nullptr;
        size_t size = 0;
        int fd = -1;
    };
    struct Tensor {
        std::string name;
        sfnx_gguf_tensor info{};
    };
    std::vector<Map> maps;
    std::vector<Tensor> tensors;
    std::map<std::string, size_t> index;
    std::map<std::string, int64_t> ints;
    std::map<std::string, double> floats;
    std::map<std::string, std::string> strs;
    ~sfnx_gguf() {
        for (Map& m : maps) {
            if (m.base) munmap(m.base, m.size);
            if (m.fd >= 0) close(m.fd);
        }
    }
};

namespace sfnx {
namespace {

enum : uint32_t {
    G_U8 = 0, G_I8 = 1, G_U16 = 2, G_I16 = 3, G_U32 = 4, G_I32 = 5, G_F32 = 6, G_BOOL = 7, G_STR = 8, G_ARR = 9,
    G_U64 = 10, G_I64 = 11, G_F64 = 12,
};

// elements a block and bytes a block of the ggml types a GGUF can hold (the GGUF format's own table)
bool type_info(uint32_t t, int& block, int& bytes) {
    switch (t) {
        case 0: block = 1, bytes = 4; return true;        // F32
        case 1: block = 1, bytes = 2; return true;        // F16
        case 30: block = 1, bytes = 2; return true;       // BF16
        case 2: block = 32, bytes = 18; return true;      // Q4_0
        case 3: block = 32, bytes = 20; return true;      // Q4_1
        case 6: block = 32, bytes = 22; return true;      // Q5_0
        case 7: block = 32, bytes = 24; return true;      // Q5_1
        case 8: block = 32, bytes = 34; return true;      // Q8_0
        case 9: block = 32, bytes = 36; return true;      // Q8_1
        case 10: block = 256, bytes = 84; return true;    // Q2_K
        case 11: block = 256, bytes = 110; return true;   // Q3_K
        case 12: block = 256, bytes = 144; return true;   // Q4_K
        case 13: block = 256, bytes = 176; return true;   // Q5_K
        case 14: block = 256, bytes = 210; return true;   // Q6_K
        case 15: block = 256, bytes = 292; return true;   // Q8_K
        case 20: block = 32, bytes = 18; return true;     // IQ4_NL
    }
    return false;
}

struct Reader {
    const uint8_t* p;
    const uint8_t* end;
    template <typename T> T get() {
        require(p + sizeof(T) <= end, "gguf: truncated header");
        T v;
        std::memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        require(n <= (uint64_t) (end - p), "gguf: truncated string");
        std::string s((const char*) p, n);
        p += n;
        return s;
    }
    void skip(uint64_t n) {
        require(n <= (uint64_t) (end - p), "gguf: truncated value");
        p += n;
    }
};

size_t scalar_bytes(uint32_t t) {
    switch (t) {
        case G_U8: case G_I8: case G_BOOL: return 1;
        case G_U16: case G_I16: return 2;
        case G_U32: case G_I32: case G_F32: return 4;
        case G_U64: case G_I64: case G_F64: return 8;
    }
    throw std::runtime_error("gguf: unknown value type " + std::to_string(t));
}

int64_t read_int(Reader& r, uint32_t t) {
    switch (t) {
        case G_U8: return r.get<uint8_t>();
        case G_I8: return r.get<int8_t>();
        case G_BOOL: return r.get<uint8_t>() != 0;
        case G_U16: return r.get<uint16_t>();
        case G_I16: return r.get<int16_t>();
        case G_U32: return r.get<uint32_t>();
        case G_I32: return r.get<int32_t>();
        case G_U64: return (int64_t) r.get<uint64_t>();
        case G_I64: return r.get<int64_t>();
    }
    throw std::runtime_error("gguf: not an integer type");
}

// one shard: map it, read its header; the first shard's metadata is kept
void load_shard(sfnx_gguf& g, const std::string& path, bool meta) {
    sfnx_gguf::Map m;
    m.fd = open(path.c_str(), O_RDONLY);
    require(m.fd >= 0, ("gguf: cannot open " + path).c_str());
    struct stat st;
    if (fstat(m.fd, &st) != 0) {
        close(m.fd);
        throw std::runtime_error("gguf: cannot stat " + path);
    }
    m.size = (size_t) st.st_size;
    if (m.size > 0) {
        m.base = mmap(nullptr, m.size, PROT_READ, MAP_SHARED, m.fd, 0);
        if (m.base == MAP_FAILED) {
            close(m.fd);
            throw std::runtime_error("gguf: cannot map " + path);
        }
    }
    g.maps.push_back(m);
    const int shard = (int) g.maps.size() - 1;
    const uint8_t* base = (const uint8_t*) m.base;
    Reader r{base, base + m.size};
    require(m.size >= 4 && std::memcmp(base, "GGUF", 4) == 0, ("gguf: " + path + " is not a GGUF file").c_str());
    r.p += 4;
    const uint32_t version = r.get<uint32_t>();
    require(version == 2 || version == 3, "gguf: only versions 2 and 3 are read");
    const uint64_t nt = r.get<uint64_t>(), nkv = r.get<uint64_t>();
    require(nt < (1u << 24) && nkv < (1u << 24), "gguf: implausible tensor or key count");
    uint64_t align = 32;
    for (uint64_t k = 0; k < nkv; ++k) {
        const std::string key = r.str();
        const uint32_t t = r.get<uint32_t>();
        if (t == G_STR) {
            std::string v = r.str();
            if (meta) g.strs[key] = std::move(v);
        } else if (t == G_ARR) {
            const uint32_t et = r.get<uint32_t>();
            const uint64_t n = r.get<uint64_t>();
            if (et == G_STR) {
                for (uint64_t i = 0; i < n; ++i) r.str();
            } else {
                const size_t eb = scalar_bytes(et);
                require(n <= (uint64_t) (r.end - r.p) / eb, "gguf: truncated array");
                r.skip(n * eb);
            }
        } else if (t == G_F32 || t == G_F64) {
            const double v = t == G_F32 ? (double) r.get<float>() : r.get<double>();
            if (meta) g.floats[key] = v;
        } else {
            const int64_t v = read_int(r, t);
            if (key == "general.alignment") align = (uint64_t) v;
            if (meta) g.ints[key] = v;
        }
    }
    require(align > 0 && (align & (align - 1)) == 0, "gguf: general.alignment is not a power of two");
    std::vector<sfnx_gguf::Tensor> local;
    std::vector<uint64_t> offs;
    for (uint64_t i = 0; i < nt; ++i) {
        sfnx_gguf::Tensor t;
        t.name = r.str();
        const uint32_t nd = r.get<uint32_t>();
        require(nd >= 1 && nd <= 4, ("gguf: " + t.name + " has more than 4 dimensions").c_str());
        t.info.n_dims = (int) nd;
        for (int d = 0; d < 4; ++d) t.info.ne[d] = 1;
        for (uint32_t d = 0; d < nd; ++d) {
            const uint64_t v = r.get<uint64_t>();
            require(v > 0 && v < (1ull << 40), ("gguf: " + t.name + " has an implausible dimension").c_str());
            t.info.ne[d] = (int64_t) v;
        }
        t.info.type = r.get<uint32_t>();
        int block, bytes;
        require(type_info(t.info.type, block, bytes), ("gguf: " + t.name + " has an unknown ggml type").c_str());
        require(t.info.ne[0] % block == 0, ("gguf: " + t.name + "'s rows are not whole blocks").c_str());
        // the byte count with every product checked: each dimension may be up to 2^40, so a crafted header's
        // product can wrap 64 bits and pass a bounds check it should fail
        uint64_t nb = (uint64_t) (t.info.ne[0] / block), prod = 0;
        bool wrap = __builtin_mul_overflow(nb, (uint64_t) bytes, &nb);
        for (int d = 1; d < 4; ++d) wrap |= __builtin_mul_overflow(nb, (uint64_t) t.info.ne[d], &prod), nb = prod;
        require(!wrap && nb <= m.size, ("gguf: " + t.name + "'s data is larger than the file").c_str());
        t.info.nbytes = (size_t) nb;
        t.info.shard = shard;
        offs.push_back(r.get<uint64_t>());
        local.push_back(std::move(t));
    }
    const uint64_t data0 = ((uint64_t) (r.p - base) + align - 1) / align * align;
    for (size_t i = 0; i < local.size(); ++i) {
        sfnx_gguf::Tensor& t = local[i];
        // step by step, so that no sum can wrap: data0 <= size, then offs <= size - data0, then nbytes <= the rest
        require(data0 <= m.size && offs[i] <= m.size - data0 && t.info.nbytes <= m.size - data0 - offs[i],
                ("gguf: " + t.name + "'s data runs past the end of " + path).c_str());
        t.info.data = base + data0 + offs[i];
        require(g.index.count(t.name) == 0, ("gguf: tensor " + t.name + " appears twice").c_str());
        g.index[t.name] = g.tensors.size();
        g.tensors.push_back(std::move(t));
    }
}

const sfnx_gguf_tensor* find(const sfnx_gguf* g, const std::string& name) {
    const auto it = g->index.find(name);
    return it == g->index.end() ? nullptr : &g->tensors[it->second].info;
}
const sfnx_gguf_tensor& need(const sfnx_gguf* g, const std::string& name) {
    const sfnx_gguf_tensor* t = find(g, name);
    require(t != nullptr, ("gguf: tensor " + name + " is missing").c_str());
    return *t;
}
size_t row_bytes_of(const sfnx_gguf_tensor& t) {
    int block, bytes;
    type_info(t.type, block, bytes);
    return (size_t) (t.ne[0] / block) * bytes;
}

}  // namespace
}  // namespace sfnx

using namespace sfnx;

extern "C" int sfnx_gguf_type_info(uint32_t type, int* block, int* bytes) {
    return guarded_host("sfnx_gguf_type_info", [&] {
        int b, n;
        require(type_info(type, b, n), "unknown ggml type");
        if (block) *block = b;
        if (bytes) *bytes = n;
    });
}

extern "C" int sfnx_gguf_open(const char* path, sfnx_gguf** out) {
    return guarded_host("sfnx_gguf_open", [&] {
        require(path != nullptr && out != nullptr, "null argument");
        *out = nullptr;
        auto g = std::make_unique<sfnx_gguf>();
        const std::string p(path);
        // a split model: "<stem>-0000N-of-0000M.gguf" maps every shard, the first one's metadata kept
        static const std::regex split("(.*)-([0-9]{5})-of-([0-9]{5})\\.gguf");
        std::smatch sm;
        if (std::regex_match(p, sm, split)) {
            const int n = std::stoi(sm[3].str());
            require(n >= 1 && n <= 9999, "gguf: implausible shard count");
            for (int i = 1; i <= n; ++i) {
                char num[16];
                std::snprintf(num, sizeof num, "%05d", i);
                load_shard(*g, sm[1].str() + "-" + num + "-of-" + sm[3].str() + ".gguf", i == 1);
            }
        } else {
            load_shard(*g, p, true);
        }
        *out = g.release();
    });
}

extern "C" void sfnx_gguf_close(sfnx_gguf* g) { delete g; }

extern "C" int sfnx_gguf_n_tensors(const sfnx_gguf* g) { return g ? (int) g->tensors.size() : -1; }

extern "C" int sfnx_gguf_tensor_at(const sfnx_gguf* g, int i, const char** name, sfnx_gguf_tensor* info) {
    return guarded_host("sfnx_gguf_tensor_at", [&] {
        require(g != nullptr && i >= 0 && i < (int) g->tensors.size(), "tensor index out of range");
        if (name) *name = g->tensors[(size_t) i].name.c_str();
        if (info) *info = g->tensors[(size_t) i].info;
    });
}

extern "C" int sfnx_gguf_find(const sfnx_gguf* g, const char* name, sfnx_gguf_tensor* info) {
    int found = 0;
    const int st = guarded_host("sfnx_gguf_find", [&] {
        require(g != nullptr && name != nullptr, "null argument");
        const sfnx_gguf_tensor* t = find(g, name);
        if (t) {
            found = 1;
            if (info) *info = *t;
        }
    });
    return st != 0 ? st : found;
}

extern "C" int sfnx_gguf_int(const sfnx_gguf* g, const char* key, int64_t* v) {
    int found = 0;
    const int st = guarded_host("sfnx_gguf_int", [&] {
        require(g != nullptr && key != nullptr, "null argument");
        const auto it = g->ints.find(key);
        if (it != g->ints.end()) {
            found = 1;
            if (v) *v = it->second;
        }
    });
    return st != 0 ? st : found;
}

extern "C" int sfnx_gguf_float(const sfnx_gguf* g, const char* key, double* v) {
    int found = 0;
    const int st = guarded_host("sfnx_gguf_float", [&] {
        require(g != nullptr && key != nullptr, "null argument");
        const auto it = g->floats.find(key);
        const auto ii = g->ints.find(key);
        if (it != g->floats.end()) {
            found = 1;
            if (v) *v = it->second;
        } else if (ii != g->ints.end()) {   // writers differ on whether a number is stored as an integer
            found = 1;
            if (v) *v = (double) ii->second;
        }
    });
    return st != 0 ? st : found;
}

extern "C" int sfnx_gguf_str(const sfnx_gguf* g, const char* key, const char** v) {
    int found = 0;
    const int st = guarded_host("sfnx_gguf_str", [&] {
        require(g != nullptr && key != nullptr, "null argument");
        const auto it = g->strs.find(key);
        if (it != g->strs.end()) {
            found = 1;
            if (v) *v = it->second.c_str();
        }
    });
    return st != 0 ? st : found;
}

namespace {
// sh_gu null: the shared expert (when present, of the routed types) is expert E of gu / dn.  Else the shared expert
// must be present and Q8_0 (src/model.cpp:807-809 throws otherwise) and goes to sh_gu [2 ffs][H] / sh_dn [H][ffs] in
// the split layout (src/model.cpp:384-440 q8split).
void moe_layer(const sfnx_gguf* g, int layer, int ff0, int ff1, void* gu, size_t gu_stride, size_t gu_cap, void* dn,
               size_t dn_stride, size_t dn_cap, float* W, int w_rows, const sfnx_q8s* sh_gu, const sfnx_q8s* sh_dn,
               int* info, void* st) {
    require(g != nullptr && gu != nullptr && dn != nullptr && W != nullptr, "null argument");
    const bool q8s = sh_gu != nullptr;
    require(!q8s || (sh_dn != nullptr && sh_gu->q && sh_gu->d && sh_dn->q && sh_dn->d), "null argument");
    const std::string L = "blk." + std::to_string(layer) + ".";
    const sfnx_gguf_tensor& tg = need(g, L + "ffn_gate_exps.weight");
    const sfnx_gguf_tensor& tu = need(g, L + "ffn_up_exps.weight");
    const sfnx_gguf_tensor& td = need(g, L + "ffn_down_exps.weight");
    const sfnx_gguf_tensor& ti = need(g, L + "ffn_gate_inp.weight");
    const uint32_t type = tg.type, dtype = td.type;   // gate|up stack into one store; down is its own (src/model.cpp:540-606)
    require(expert_type_ok(type) && expert_type_ok(dtype), "expert tensors must be Q4_0, Q5_1, Q8_0, Q4_K or Q5_K");
    require(tu.type == type, "gate and up experts differ in type (they stack into one matrix)");
    const int64_t H = tg.ne[0], FF = tg.ne[1], E = tg.ne[2];
    require(tu.ne[0] == H && tu.ne[1] == FF && tu.ne[2] == E, "up experts differ in shape from gate experts");
    require(td.ne[0] == FF && td.ne[1] == H && td.ne[2] == E, "down experts are not [FF][H] a expert");
    const int cb = block_values(dtype);   // a column slice of the down rows is whole blocks
    require(0 <= ff0 && ff0 < ff1 && ff1 <= FF && ff0 % cb == 0 && (ff1 - ff0) % 512 == 0,
            "FF slice must start on a whole block and span a multiple of 512 (the store's runs)");
    require(H % 512 == 0, "the hidden size must be a multiple of 512 (the store's runs)");
    require(ti.type == 0 && ti.ne[0] == H && ti.ne[1] == E, "ffn_gate_inp must be f32 [E][H]");
    const int ffs = ff1 - ff0;
    const size_t rb_in = row_bytes(type, (int) H), rb_ff = row_bytes(dtype, ffs);
    require(gu_stride >= 2 * (size_t) ffs * rb_in && dn_stride >= (size_t) H * rb_ff, "strides smaller than a matrix");
    const sfnx_gguf_tensor* sg = find(g, L + "ffn_gate_shexp.weight");
    const sfnx_gguf_tensor* su = find(g, L + "ffn_up_shexp.weight");
    const sfnx_gguf_tensor* sd = find(g, L + "ffn_down_shexp.weight");
    const sfnx_gguf_tensor* sgi = find(g, L + "ffn_gate_inp_shexp.weight");
    const bool shared = sg && su && sd && sgi;
    require(shared || !q8s, "the layer has no shared expert (ffn_{gate,up,down,gate_inp}_shexp)");
    // the shared expert's types: Q8_0 for the dense path, else those of the routed stores it joins
    const uint32_t stype = q8s ? (uint32_t) SFNX_Q8_0 : type, sdtype = q8s ? (uint32_t) SFNX_Q8_0 : dtype;
    if (shared) {
        if (q8s)
            require(sg->type == SFNX_Q8_0 && su->type == SFNX_Q8_0 && sd->type == SFNX_Q8_0, "the shared expert is not Q8_0");
        else
            require(sg->type == type && su->type == type && sd->type == dtype,
                    "the shared expert's types differ from the routed experts' (it is one more expert of their stores)");
        require(sg->ne[0] == H && sg->ne[1] == FF && su->ne[0] == H && su->ne[1] == FF && sd->ne[0] == FF &&
                    sd->ne[1] == H, "the shared expert's shape differs from a routed expert's");
        require(sgi->type == 0 && sgi->ne[0] == H && sgi->ne[1] == 1, "ffn_gate_inp_shexp must be f32 [1][H]");
    }
    const int64_t NE = E + (shared && !q8s ? 1 : 0);   // experts the routed stores receive
    // the caller's buffers, checked against what the file holds before anything is written
    require((uint64_t) (NE - 1) * gu_stride + 2 * (size_t) ffs * rb_in <= gu_cap,
            "gu buffer too small for the layer's experts (E from the file, plus the shared expert when it joins)");
    require((uint64_t) (NE - 1) * dn_stride + (size_t) H * rb_ff <= dn_cap,
            "dn buffer too small for the layer's experts (E from the file, plus the shared expert when it joins)");
    require((int64_t) w_rows >= E + 1, "W holds fewer than E + 1 router rows");
    hipStream_t s = stream_of(st);
    // one expert's matrices at a time in GGUF layout through a pinned host buffer and a device buffer, then packed
    const size_t gu_bytes = 2 * (size_t) ffs * rb_in, dn_bytes = (size_t) H * rb_ff;
    const size_t sgu_bytes = 2 * (size_t) ffs * row_bytes(stype, (int) H), sdn_bytes = (size_t) H * row_bytes(sdtype, ffs);
    const size_t stage = std::max(gu_bytes, sgu_bytes) + std::max(dn_bytes, sdn_bytes);
    void *host = nullptr, *dev = nullptr;
    check(hipHostMalloc(&host, stage, hipHostMallocDefault), "hipHostMalloc");
    const hipError_t ea = hipMalloc(&dev, stage);
    if (ea != hipSuccess) {
        (void) hipHostFree(host);
        check(ea, "hipMalloc");
    }
    auto cleanup = [&] {
        (void) hipStreamSynchronize(s);
        (void) hipFree(dev);
        (void) hipHostFree(host);
    };
    try {
        uint8_t* h = (uint8_t*) host;
        for (int64_t e = 0; e < E + (shared ? 1 : 0); ++e) {
            const bool sh = e == E;
            const uint32_t gt = sh ? stype : type, dt = sh ? sdtype : dtype;
            const size_t rbi = row_bytes(gt, (int) H), rbf = row_bytes(dt, ffs), rb_full_dn = row_bytes(dt, (int) FF);
            const size_t col0 = row_bytes(dt, ff0), gub = 2 * (size_t) ffs * rbi;
            const uint8_t* g0 = (const uint8_t*) (sh ? sg->data : tg.data) + (sh ? 0 : e * FF * rbi);
            const uint8_t* u0 = (const uint8_t*) (sh ? su->data : tu.data) + (sh ? 0 : e * FF * rbi);
            const uint8_t* d0 = (const uint8_t*) (sh ? sd->data : td.data) + (sh ? 0 : e * H * rb_full_dn);
            check(hipStreamSynchronize(s), "hipStreamSynchronize");   // the buffers are free again
            // gate rows ff0..ff1, then up rows ff0..ff1 (src/model.cpp:554-576)
            std::memcpy(h, g0 + (size_t) ff0 * rbi, (size_t) ffs * rbi);
            std::memcpy(h + (size_t) ffs * rbi, u0 + (size_t) ff0 * rbi, (size_t) ffs * rbi);
            // every down row, columns ff0..ff1 (src/model.cpp:586-606)
            for (int64_t r = 0; r < H; ++r) std::memcpy(h + gub + r * rbf, d0 + r * rb_full_dn + col0, rbf);
            check(hipMemcpyAsync(dev, host, gub + (size_t) H * rbf, hipMemcpyHostToDevice, s), "hipMemcpyAsync");
            if (sh && q8s) {   // the dense shared expert: the reference's split planes
                if (sfnx_q8s_split(dev, 2 * ffs, (int) H, sh_gu, st) != 0) throw std::runtime_error(sfnx_last_error());
                if (sfnx_q8s_split((uint8_t*) dev + gub, (int) H, ffs, sh_dn, st) != 0) throw std::runtime_error(sfnx_last_error());
                continue;
            }
            void* gdst = (uint8_t*) gu + e * gu_stride;
            void* ddst = (uint8_t*) dn + e * dn_stride;
            if (sfnx_store_pack(gt, dev, gdst, 1, 2 * ffs, (int) H, st) != 0) throw std::runtime_error(sfnx_last_error());
            if (sfnx_store_pack(dt, (uint8_t*) dev + gub, ddst, 1, (int) H, ffs, st) != 0) throw std::runtime_error(sfnx_last_error());
        }
        // router rows, then the shared expert's gate row (src/model.cpp:766-773)
        check(hipMemcpyAsync(W, ti.data, (size_t) E * H * 4, hipMemcpyHostToDevice, s), "hipMemcpyAsync");
        if (shared) check(hipMemcpyAsync(W + E * H, sgi->data, (size_t) H * 4, hipMemcpyHostToDevice, s), "hipMemcpyAsync");
        check(hipStreamSynchronize(s), "hipStreamSynchronize");
    } catch (...) {
        cleanup();
        throw;
    }
    cleanup();
    if (info) {
        info[0] = (int) type;
        info[1] = (int) H;
        info[2] = (int) E;
        info[3] = ffs;
        info[4] = shared ? 1 : 0;
        info[5] = (int) dtype;
    }
}
}  // namespace

extern "C" int sfnx_gguf_moe_layer(const sfnx_gguf* g, int layer, int ff0, int ff1, void* gu, size_t gu_stride,
                                   size_t gu_bytes, void* dn, size_t dn_stride, size_t dn_bytes, float* W, int w_rows,
                                   int* info, void* st) {
    return guarded("sfnx_gguf_moe_layer", [&] {
        moe_layer(g, layer, ff0, ff1, gu, gu_stride, gu_bytes, dn, dn_stride, dn_bytes, W, w_rows, nullptr, nullptr, info, st);
    });
}

extern "C" int sfnx_gguf_moe_layer_q8s(const sfnx_gguf* g, int layer, int ff0, int ff1, void* gu, size_t gu_stride,
                                       size_t gu_bytes, void* dn, size_t dn_stride, size_t dn_bytes, float* W,
                                       int w_rows, const sfnx_q8s* sh_gu, const sfnx_q8s* sh_dn, int* info, void* st) {
    return guarded("sfnx_gguf_moe_layer_q8s", [&] {
        require(sh_gu != nullptr && sh_dn != nullptr, "null argument");
        moe_layer(g, layer, ff0, ff1, gu, gu_stride, gu_bytes, dn, dn_stride, dn_bytes, W, w_rows, sh_gu, sh_dn, info, st);
    });
}
