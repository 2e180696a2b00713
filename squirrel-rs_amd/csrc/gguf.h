// GGUF v3 reader (mmap) and writer.
//
// Reader semantics follow the reference's file parser (src/file_parser/):
// the magic is not validated (gguf_header.rs:13-24), metadata values are
// typed and arrays recursive (gguf_metadata_value.rs:49-80), an unknown
// value or GGML type id, a bool other than 0/1, invalid UTF-8 or a truncated
// file is an error, and tensor data starts at the next multiple of 32
// regardless of `general.alignment` (gguf_file.rs:10,44-46).
#pragma once
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace sq {

enum GGUFType : uint32_t {
    GT_U8 = 0, GT_I8 = 1, GT_U16 = 2, GT_I16 = 3, GT_U32 = 4, GT_I32 = 5, GT_F32 = 6,
    GT_BOOL = 7, GT_STRING = 8, GT_ARRAY = 9, GT_U64 = 10, GT_I64 = 11, GT_F64 = 12,
};

struct GGUFValue {
    uint32_t type = 0;
    uint64_t u = 0;   // unsigned scalars and bool
    int64_t i = 0;    // signed scalars
    double f = 0.0;   // F32 / F64 (F32 stored exactly)
    float f32 = 0.0f;
    std::string s;
    uint32_t arr_type = 0;
    std::vector<GGUFValue> arr;
};

struct GGUFTensorInfo {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t ggml_type = 0;
    uint64_t offset = 0;
    uint64_t numel = 0;
};

// Elements and bytes per storage block for the types the path supports
// (ggml_type.rs:45-62); false for every other type.
bool ggml_block(uint32_t ggml_type, uint64_t* elems, uint64_t* bytes);
bool ggml_type_known(uint32_t ggml_type);

class GGUFFile {
   public:
    GGUFFile() = default;
    ~GGUFFile();
    GGUFFile(const GGUFFile&) = delete;
    GGUFFile& operator=(const GGUFFile&) = delete;

    // 0 or SQ_ERR_IO / SQ_ERR_FORMAT (message via sq_last_error).
    int open(const std::string& path);
    int parse(const uint8_t* data, size_t size);  // over caller-owned bytes

    // tensor_bytes_size (gguf_tensor_info.rs:52-65): SQ_ERR_UNSUPPORTED for
    // types other than F32/BF16/Q8_0/Q4_0 or a partial block.
    int tensor_bytes(const GGUFTensorInfo& t, uint64_t* out) const;
    // Pointer to a tensor's bytes, or null (with status) when missing,
    // unsupported or out of bounds.
    const uint8_t* tensor_data(const std::string& name, int* status) const;

    uint32_t magic = 0, version = 0;
    std::unordered_map<std::string, GGUFValue> meta;
    std::unordered_map<std::string, GGUFTensorInfo> tensors;
    uint64_t data_offset = 0;
    uint64_t alignment = 32;  // general.alignment when present
    const uint8_t* base = nullptr;
    size_t size = 0;

   private:
    void* map_ = nullptr;
    size_t map_len_ = 0;
};

// Minimal writer: metadata in insertion order, tensors at 32-aligned offsets.
class GGUFWriter {
   public:
    void add_u32(const std::string& k, uint32_t v);
    void add_f32(const std::string& k, float v);
    void add_string(const std::string& k, const std::string& v);
    // `data` must stay alive until write().
    void add_tensor(const std::string& name, const std::vector<uint64_t>& dims, uint32_t ggml_type,
                    const void* data, uint64_t bytes);
    int write(const std::string& path) const;

   private:
    struct KV {
        std::string key;
        uint32_t type;
        uint32_t u;
        float f;
        std::string s;
    };
    struct T {
        std::string name;
        std::vector<uint64_t> dims;
        uint32_t type;
        const void* data;
        uint64_t bytes;
    };
    std::vector<KV> kvs_;
    std::vector<T> ts_;
};

}  // namespace sq
