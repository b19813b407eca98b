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

// IEEE binary16 / bfloat16 bit patterns to f32 (subnormals, infinities and NaNs kept)
float fp16_bits_to_f32(uint16_t h);
float bf16_bits_to_f32(uint16_t b);

struct GgufTensor;

// The tensor's values as f32, row-major as stored (ne0 innermost), for F32, F16,
// BF16 and the GGUF block formats Q8_0 (fp16 d + 32 int8 q: d*q) and Q4_0 (fp16 d +
// 16 bytes, element j in the low nibble of byte j and element j+16 in the high one:
// d*(nibble-8)).  This is what the reference loader's read_tensor_data does for every
// tensor it reads (src/hunyuan_gguf_loader.cpp:167-222), with two deliberate
// differences: fp16 subnormal scales are kept rather than flushed to zero, and Q4_0
// follows the GGUF nibble order (the reference's decoder reads element i from byte
// i/2, which real GGUF files do not use).  Returns false for any other type.
bool tensor_to_f32(const GgufTensor& t, float* out);

// Q4_0 blocks re-encoded as Q8_0 blocks with the same scale: q = nibble - 8 is an
// int8, so the values are unchanged.  n_blocks blocks of 18 bytes -> 34 bytes.
void q4_0_to_q8_0(const uint8_t* src, uint8_t* dst, uint64_t n_blocks);

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
