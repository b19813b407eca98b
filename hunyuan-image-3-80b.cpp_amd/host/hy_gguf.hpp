// hy_gguf.hpp -- a reader for GGUF files (format versions 2 and 3), written from the
// public GGUF layout: header (magic "GGUF", version, tensor count, key/value count),
// typed key/value metadata, tensor infos (name, dims, ggml type, data offset), then
// the tensor data, aligned to general.alignment (default 32).  The file is memory
// mapped read-only; tensor data pointers point into the mapping.
//
// It replaces, for the MoE tensors, the gguf_* calls of the reference's loader
// (src/hunyuan_gguf_loader.cpp:84-158) and load_layer_weights (:229-280), without
// dequantizing: GGUF Q8_0 / Q4_0 blocks go to the device as they are.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace hy {

// ggml type numbers the reader knows the sizes of
enum GgmlType : int32_t {
    GGML_F32 = 0,
    GGML_F16 = 1,
    GGML_Q4_0 = 2,
    GGML_Q4_1 = 3,
    GGML_Q5_0 = 6,
    GGML_Q5_1 = 7,
    GGML_Q8_0 = 8,
    GGML_Q8_1 = 9,
    GGML_BF16 = 30,
};

// bytes of a row of n elements of a ggml type; 0 for an unknown type or an n that is
// not a whole number of blocks
uint64_t ggml_row_bytes(int32_t type, uint64_t n);

struct GgufTensor {
    std::string name;
    int32_t type = 0;
    uint32_t n_dims = 0;
    uint64_t ne[4] = {1, 1, 1, 1};  // ne[0] = elements per row (innermost)
    uint64_t offset = 0;            // from the start of the data section
    uint64_t nbytes = 0;            // 0: type without a known size
    const uint8_t* data = nullptr;  // into the mapping (null when nbytes == 0)
};

// GGUF value types
enum GgufValueType : uint32_t {
    GGUF_U8 = 0, GGUF_I8 = 1, GGUF_U16 = 2, GGUF_I16 = 3, GGUF_U32 = 4, GGUF_I32 = 5,
    GGUF_F32 = 6, GGUF_BOOL = 7, GGUF_STRING = 8, GGUF_ARRAY = 9, GGUF_U64 = 10,
    GGUF_I64 = 11, GGUF_F64 = 12,
};

struct GgufValue {
    uint32_t type = 0;
    uint64_t u = 0;  // unsigned and bool values
    int64_t i = 0;   // signed values
    double f = 0.0;  // float values
    std::string s;   // string values
    uint32_t arr_type = 0;  // arrays: element type and count (elements are skipped)
    uint64_t arr_n = 0;
};

class GgufFile {
public:
    GgufFile() = default;
    ~GgufFile();
    GgufFile(const GgufFile&) = delete;
    GgufFile& operator=(const GgufFile&) = delete;

    // 0 on success, else a negative hy_status with a message in *err
    int open(const char* path, std::string* err);

    const GgufTensor* find(const std::string& name) const;
    const GgufValue* kv(const std::string& key) const;

    uint32_t version = 0;
    uint32_t alignment = 32;
    uint64_t data_offset = 0;
    size_t size = 0;
    std::vector<GgufTensor> tensors;

private:
    int parse(std::string* err);
    std::unordered_map<std::string, size_t> tindex_;
    std::unordered_map<std::string, GgufValue> kv_;
    int fd_ = -1;
    const uint8_t* map_ = nullptr;
};

}  // namespace hy
