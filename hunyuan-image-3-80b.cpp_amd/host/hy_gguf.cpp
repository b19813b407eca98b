// hy_gguf.cpp -- GGUF reader (see hy_gguf.hpp) and its C ABI entry points.
#include "hy_gguf.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>

#include "../../include/hy_moe.h"

namespace hy {

int set_last_error(int code, const std::string& msg);  // hy_capi.hip

uint64_t ggml_row_bytes(int32_t type, uint64_t n) {
    auto blocks = [&](uint64_t bytes_per_block) -> uint64_t {
        return n % 32 == 0 ? n / 32 * bytes_per_block : 0;
    };
    switch (type) {
    case GGML_F32: return n * 4;
    case GGML_F16:
    case GGML_BF16: return n * 2;
    case GGML_Q4_0: return blocks(18);
    case GGML_Q4_1: return blocks(20);
    case GGML_Q5_0: return blocks(22);
    case GGML_Q5_1: return blocks(24);
    case GGML_Q8_0: return blocks(34);
    case GGML_Q8_1: return blocks(36);
    default: return 0;
    }
}

float fp16_bits_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0x1f) {
        bits = sign | 0x7f800000u | (m << 13);   // inf / NaN
    } else if (e != 0) {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0) {
        bits = sign;
    } else {  // subnormal: m * 2^-24, normalised
        int sh = 0;
        uint32_t mm = m;
        while (!(mm & 0x400u)) {
            mm <<= 1;
            sh++;
        }
        bits = sign | ((uint32_t)(113 - sh) << 23) | ((mm & 0x3ffu) << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

float bf16_bits_to_f32(uint16_t b) {
    const uint32_t bits = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

bool tensor_to_f32(const GgufTensor& t, float* out) {
    if (!t.data) return false;
    const uint64_t n = t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3];
    const uint8_t* p = t.data;
    auto u16 = [](const uint8_t* q) { return (uint16_t)(q[0] | (q[1] << 8)); };
    switch (t.type) {
    case GGML_F32:
        std::memcpy(out, p, n * 4);
        return true;
    case GGML_F16:
        for (uint64_t i = 0; i < n; i++) out[i] = fp16_bits_to_f32(u16(p + 2 * i));
        return true;
    case GGML_BF16:
        for (uint64_t i = 0; i < n; i++) out[i] = bf16_bits_to_f32(u16(p + 2 * i));
        return true;
    case GGML_Q8_0:
        for (uint64_t b = 0; b < n / 32; b++, p += 34) {
            const float d = fp16_bits_to_f32(u16(p));
            for (int j = 0; j < 32; j++) out[32 * b + j] = d * (float)(int8_t)p[2 + j];
        }
        return true;
    case GGML_Q4_0:
        for (uint64_t b = 0; b < n / 32; b++, p += 18) {
            const float d = fp16_bits_to_f32(u16(p));
            for (int j = 0; j < 16; j++) {
                out[32 * b + j] = d * (float)((int)(p[2 + j] & 0x0f) - 8);
                out[32 * b + 16 + j] = d * (float)((int)(p[2 + j] >> 4) - 8);
            }
        }
        return true;
    default:
        return false;
    }
}

void q4_0_to_q8_0(const uint8_t* src, uint8_t* dst, uint64_t n_blocks) {
    for (uint64_t b = 0; b < n_blocks; b++, src += 18, dst += 34) {
        dst[0] = src[0];
        dst[1] = src[1];
        for (int j = 0; j < 16; j++) {
            dst[2 + j] = (uint8_t)(int8_t)((int)(src[2 + j] & 0x0f) - 8);
            dst[2 + 16 + j] = (uint8_t)(int8_t)((int)(src[2 + j] >> 4) - 8);
        }
    }
}

GgufFile::~GgufFile() {
    if (map_) munmap(const_cast<uint8_t*>(map_), size);
    if (fd_ >= 0) close(fd_);
}

int GgufFile::open(const char* path, std::string* err) {
    if (!path) {
        *err = "null path";
        return HY_ERR_INVALID;
    }
    fd_ = ::open(path, O_RDONLY);
    if (fd_ < 0) {
        *err = std::string("cannot open ") + path + ": " + strerror(errno);
        return HY_ERR_INVALID;
    }
    struct stat st;
    if (fstat(fd_, &st) != 0 || st.st_size <= 0) {
        *err = std::string("cannot stat ") + path;
        return HY_ERR_INVALID;
    }
    size = (size_t)st.st_size;
    void* m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (m == MAP_FAILED) {
        map_ = nullptr;
        *err = std::string("cannot map ") + path + ": " + strerror(errno);
        return HY_ERR_INVALID;
    }
    map_ = static_cast<const uint8_t*>(m);
    const int rc = parse(err);
    if (rc != HY_OK) *err = std::string(path) + ": " + *err;
    return rc;
}

namespace {

// bounds-checked little-endian cursor over the mapping
struct Cursor {
    const uint8_t* p;
    size_t n, at = 0;
    bool ok = true;
    bool need(size_t k) {
        if (!ok || k > n - at) ok = false;
        return ok;
    }
    template <typename T>
    T get() {
        T v{};
        if (need(sizeof(T))) {
            memcpy(&v, p + at, sizeof(T));
            at += sizeof(T);
        }
        return v;
    }
    std::string str() {
        const uint64_t len = get<uint64_t>();
        if (!need(len)) return {};
        std::string s(reinterpret_cast<const char*>(p + at), (size_t)len);
        at += (size_t)len;
        return s;
    }
    void skip(uint64_t k) {
        if (need(k)) at += (size_t)k;
    }
};

size_t scalar_size(uint32_t t) {
    switch (t) {
    case GGUF_U8: case GGUF_I8: case GGUF_BOOL: return 1;
    case GGUF_U16: case GGUF_I16: return 2;
    case GGUF_U32: case GGUF_I32: case GGUF_F32: return 4;
    case GGUF_U64: case GGUF_I64: case GGUF_F64: return 8;
    default: return 0;
    }
}

bool read_scalar(Cursor& c, uint32_t t, GgufValue& v) {
    switch (t) {
    case GGUF_U8: v.u = c.get<uint8_t>(); break;
    case GGUF_BOOL: v.u = c.get<uint8_t>() != 0; break;
    case GGUF_I8: v.i = c.get<int8_t>(); break;
    case GGUF_U16: v.u = c.get<uint16_t>(); break;
    case GGUF_I16: v.i = c.get<int16_t>(); break;
    case GGUF_U32: v.u = c.get<uint32_t>(); break;
    case GGUF_I32: v.i = c.get<int32_t>(); break;
    case GGUF_U64: v.u = c.get<uint64_t>(); break;
    case GGUF_I64: v.i = c.get<int64_t>(); break;
    case GGUF_F32: v.f = c.get<float>(); break;
    case GGUF_F64: v.f = c.get<double>(); break;
    case GGUF_STRING: v.s = c.str(); break;
    default: return false;
    }
    return c.ok;
}

}  // namespace

int GgufFile::parse(std::string* err) {
    Cursor c{map_, size};
    const uint32_t magic = c.get<uint32_t>();
    if (!c.ok || magic != 0x46554747u) {  // "GGUF" little-endian
        *err = "not a GGUF file (bad magic)";
        return HY_ERR_INVALID;
    }
    version = c.get<uint32_t>();
    if (version != 2 && version != 3) {
        *err = "unsupported GGUF version " + std::to_string(version);
        return HY_ERR_UNSUPPORTED;
    }
    const uint64_t n_tensors = c.get<uint64_t>();
    const uint64_t n_kv = c.get<uint64_t>();
    // every key/value and tensor info takes at least 8 + 4 bytes: counts beyond the
    // file are corrupt
    if (!c.ok || n_tensors > size / 12 || n_kv > size / 12) {
        *err = "corrupt header counts";
        return HY_ERR_INVALID;
    }
    for (uint64_t i = 0; i < n_kv; i++) {
        const std::string key = c.str();
        GgufValue v;
        v.type = c.get<uint32_t>();
        if (!c.ok) break;
        if (v.type == GGUF_ARRAY) {
            v.arr_type = c.get<uint32_t>();
            v.arr_n = c.get<uint64_t>();
            if (!c.ok) break;
            if (v.arr_type == GGUF_STRING) {
                for (uint64_t j = 0; j < v.arr_n && c.ok; j++) c.skip(c.get<uint64_t>());
            } else {
                const size_t es = scalar_size(v.arr_type);
                if (es == 0 || v.arr_n > (size - c.at) / es) {
                    *err = "bad array in key " + key;
                    return HY_ERR_INVALID;
                }
                c.skip(v.arr_n * es);
            }
        } else if (!read_scalar(c, v.type, v)) {
            *err = "bad value for key " + key;
            return HY_ERR_INVALID;
        }
        kv_[key] = std::move(v);
    }
    if (!c.ok) {
        *err = "truncated key/value section";
        return HY_ERR_INVALID;
    }
    auto al = kv_.find("general.alignment");
    if (al != kv_.end()) {
        if (al->second.type != GGUF_U32 || al->second.u == 0 || (al->second.u & (al->second.u - 1)) != 0) {
            *err = "general.alignment must be a power-of-two u32";
            return HY_ERR_INVALID;
        }
        alignment = (uint32_t)al->second.u;
    }
    tensors.resize((size_t)n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        GgufTensor& t = tensors[(size_t)i];
        t.name = c.str();
        t.n_dims = c.get<uint32_t>();
        if (!c.ok || t.n_dims == 0 || t.n_dims > 4) {
            *err = "bad tensor info #" + std::to_string(i);
            return HY_ERR_INVALID;
        }
        for (uint32_t d = 0; d < t.n_dims; d++) t.ne[d] = c.get<uint64_t>();
        t.type = (int32_t)c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        if (!c.ok) break;
        tindex_[t.name] = (size_t)i;
    }
    if (!c.ok) {
        *err = "truncated tensor infos";
        return HY_ERR_INVALID;
    }
    data_offset = (c.at + alignment - 1) / alignment * alignment;
    if (data_offset > size) {
        *err = "no data section";
        return HY_ERR_INVALID;
    }
    const uint64_t data_size = size - data_offset;
    for (auto& t : tensors) {
        uint64_t rows = 1;
        for (uint32_t d = 1; d < t.n_dims; d++) {
            if (t.ne[d] != 0 && rows > UINT64_MAX / t.ne[d]) {
                *err = "tensor " + t.name + ": dims overflow";
                return HY_ERR_INVALID;
            }
            rows *= t.ne[d];
        }
        const uint64_t rb = ggml_row_bytes(t.type, t.ne[0]);
        if (rb == 0) continue;  // a type this reader does not size: left unmapped
        if (rows != 0 && rb > UINT64_MAX / rows) {
            *err = "tensor " + t.name + ": size overflow";
            return HY_ERR_INVALID;
        }
        t.nbytes = rb * rows;
        if (t.offset % alignment != 0 || t.offset > data_size || t.nbytes > data_size - t.offset) {
            *err = "tensor " + t.name + ": data outside the file or misaligned";
            return HY_ERR_INVALID;
        }
        t.data = map_ + data_offset + t.offset;
    }
    return HY_OK;
}

const GgufTensor* GgufFile::find(const std::string& name) const {
    auto it = tindex_.find(name);
    return it == tindex_.end() ? nullptr : &tensors[it->second];
}

const GgufValue* GgufFile::kv(const std::string& key) const {
    auto it = kv_.find(key);
    return it == kv_.end() ? nullptr : &it->second;
}

}  // namespace hy

struct hy_gguf {
    hy::GgufFile f;
};

extern "C" {

int hy_gguf_open(const char* path, hy_gguf** out) {
    if (!out) return hy::set_last_error(HY_ERR_INVALID, "null out");
    *out = nullptr;
    hy_gguf* g = new hy_gguf();
    std::string err;
    const int rc = g->f.open(path, &err);
    if (rc != HY_OK) {
        delete g;
        return hy::set_last_error(rc, err);
    }
    *out = g;
    return HY_OK;
}

int hy_gguf_close(hy_gguf* g) {
    delete g;
    return HY_OK;
}

int hy_gguf_n_tensors(const hy_gguf* g, uint64_t* n) {
    if (!g || !n) return hy::set_last_error(HY_ERR_INVALID, "null argument");
    *n = g->f.tensors.size();
    return HY_OK;
}

int hy_gguf_tensor(const hy_gguf* g, const char* name, int32_t* type, uint32_t* n_dims, uint64_t* ne,
                   uint64_t* nbytes, const void** data) {
    if (!g || !name) return hy::set_last_error(HY_ERR_INVALID, "null argument");
    const hy::GgufTensor* t = g->f.find(name);
    if (!t) return hy::set_last_error(HY_ERR_INVALID, std::string("no tensor ") + name);
    if (type) *type = t->type;
    if (n_dims) *n_dims = t->n_dims;
    if (ne)
        for (int d = 0; d < 4; d++) ne[d] = t->ne[d];
    if (nbytes) *nbytes = t->nbytes;
    if (data) *data = t->data;
    return HY_OK;
}

int hy_gguf_tensor_f32(const hy_gguf* g, const char* name, float* out, uint64_t n) {
    if (!g || !name || !out) return hy::set_last_error(HY_ERR_INVALID, "null argument");
    const hy::GgufTensor* t = g->f.find(name);
    if (!t) return hy::set_last_error(HY_ERR_INVALID, std::string("no tensor ") + name);
    const uint64_t count = t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3];
    if (n != count)
        return hy::set_last_error(HY_ERR_INVALID, std::string("tensor ") + name + " has " + std::to_string(count) +
                                                      " elements, the buffer " + std::to_string(n));
    if (!hy::tensor_to_f32(*t, out))
        return hy::set_last_error(HY_ERR_UNSUPPORTED, std::string("tensor ") + name + " has ggml type " +
                                                          std::to_string(t->type) +
                                                          "; F32, F16, BF16, Q8_0 or Q4_0 expected");
    return HY_OK;
}

int hy_gguf_get_u32(const hy_gguf* g, const char* key, uint32_t* out) {
    if (!g || !key || !out) return hy::set_last_error(HY_ERR_INVALID, "null argument");
    const hy::GgufValue* v = g->f.kv(key);
    if (!v) return hy::set_last_error(HY_ERR_INVALID, std::string("no key ") + key);
    switch (v->type) {
    case hy::GGUF_U8: case hy::GGUF_U16: case hy::GGUF_U32: case hy::GGUF_BOOL:
        *out = (uint32_t)v->u;
        return HY_OK;
    case hy::GGUF_U64:
        if (v->u > UINT32_MAX) break;
        *out = (uint32_t)v->u;
        return HY_OK;
    case hy::GGUF_I8: case hy::GGUF_I16: case hy::GGUF_I32: case hy::GGUF_I64:
        if (v->i < 0 || v->i > (int64_t)UINT32_MAX) break;
        *out = (uint32_t)v->i;
        return HY_OK;
    default: break;
    }
    return hy::set_last_error(HY_ERR_INVALID, std::string("key ") + key + " is not an unsigned 32-bit value");
}

int hy_gguf_get_f32(const hy_gguf* g, const char* key, float* out) {
    if (!g || !key || !out) return hy::set_last_error(HY_ERR_INVALID, "null argument");
    const hy::GgufValue* v = g->f.kv(key);
    if (!v) return hy::set_last_error(HY_ERR_INVALID, std::string("no key ") + key);
    if (v->type != hy::GGUF_F32 && v->type != hy::GGUF_F64)
        return hy::set_last_error(HY_ERR_INVALID, std::string("key ") + key + " is not a float");
    *out = (float)v->f;
    return HY_OK;
}

}  // extern "C"

namespace hy {
const GgufFile& gguf_file(const hy_gguf* g) { return g->f; }
}  // namespace hy
