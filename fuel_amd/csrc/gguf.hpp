// GGUF container reader (host only): the header parse of fuel's
// fuel_formats::gguf::Content::read (fuel-formats/src/gguf.rs:378-461) over a
// read-only memory map of the file, as fuel-core's MmapedContent does
// (fuel-core/src/quantized/gguf_mmap.rs:44-79).  Tensor bytes are slices of
// the map: elem_count / block_size * type_size bytes at
// tensor_data_offset + offset (fuel-core/src/lazy_quantized_llama.rs:251-260).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

namespace frq {
namespace gguf {

// ValueType codes of the format (gguf.rs:125-143).
enum ValueType : int {
    VT_U8 = 0, VT_I8 = 1, VT_U16 = 2, VT_I16 = 3, VT_U32 = 4, VT_I32 = 5, VT_F32 = 6,
    VT_BOOL = 7, VT_STRING = 8, VT_ARRAY = 9, VT_U64 = 10, VT_I64 = 11, VT_F64 = 12,
};

struct Value {
    int type = VT_U8;
    uint64_t u = 0;  // U8 / U16 / U32 / U64 / Bool
    int64_t i = 0;   // I8 / I16 / I32 / I64
    double f = 0.0;  // F32 (exactly widened) / F64
    std::string s;   // String
    std::vector<Value> a;  // Array
};

struct TensorInfo {
    std::string name;
    int ggml_dtype = 0;
    std::vector<uint64_t> dims;  // outermost first (the file's order reversed)
    uint64_t offset = 0;         // relative to tensor_data_offset
    uint64_t nbytes = 0;         // elem_count / block_size * type_size
};

struct File {
    int version = 0;  // 1, 2 or 3
    // metadata in first-appearance order; a repeated key replaces the value
    std::vector<std::pair<std::string, Value>> metadata;
    std::unordered_map<std::string, size_t> meta_index;
    std::vector<TensorInfo> tensors;  // first-appearance order, repeated names replaced
    std::unordered_map<std::string, size_t> tensor_index;
    uint64_t tensor_data_offset = 0;
    const uint8_t* map = nullptr;
    size_t map_bytes = 0;
    ~File();
};

// Block geometry of a GgmlDType code (fuel-ir/src/quantized.rs:60-104);
// 0 for a code GgmlDType::from_u32 rejects.
size_t dtype_block_size(int ggml_dtype);
size_t dtype_type_size(int ggml_dtype);

// Map `path` and parse its header.  On failure returns null and sets `err`
// to a message in the reference's words.
std::unique_ptr<File> open(const char* path, std::string& err);

}  // namespace gguf
}  // namespace frq
