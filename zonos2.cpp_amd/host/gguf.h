// gguf.h — minimal GGUF v2/v3 reader and v3 writer (host side).
//
// Container layout (public GGUF format; the reference reads it through ggml's gguf API,
// src/zonos2.cpp:15-124): magic "GGUF", u32 version, u64 n_tensors, u64 n_kv, the KV pairs
// (string key, u32 type, value), the tensor infos (name, u32 n_dims, u64 ne[n_dims], u32 type,
// u64 offset), padding to `general.alignment` (default 32), then the tensor data.
#pragma once
#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace z2 {

enum gguf_vtype : uint32_t {
    GV_U8 = 0, GV_I8 = 1, GV_U16 = 2, GV_I16 = 3, GV_U32 = 4, GV_I32 = 5, GV_F32 = 6, GV_BOOL = 7,
    GV_STR = 8, GV_ARR = 9, GV_U64 = 10, GV_I64 = 11, GV_F64 = 12,
};

struct gguf_value {
    uint32_t type = GV_U32;
    uint32_t arr_type = 0;          // element type when type == GV_ARR
    std::vector<uint8_t> raw;       // scalar / array payload (little endian), strings excluded
    std::string str;                // GV_STR
    std::vector<std::string> strs;  // array of strings
    uint64_t n = 1;                 // array length
    double as_f64() const;
    int64_t as_i64() const;
};

struct gguf_tensor_info {
    std::string name;
    std::vector<int64_t> ne;        // ggml order, ne0 fastest
    int32_t type = 0;
    uint64_t offset = 0;            // relative to the data section
    uint64_t nbytes = 0;
};

struct gguf_file {
    uint32_t version = 3;
    uint64_t alignment = 32;
    std::map<std::string, gguf_value> kv;
    std::vector<std::string> kv_order;
    std::vector<gguf_tensor_info> tensors;
    uint64_t data_offset = 0;       // absolute file offset of the data section

    const gguf_value * find(const std::string & k) const;
    const gguf_tensor_info * tensor(const std::string & n) const;
};

// Parse header + tensor table. Returns false with a message on malformed input.
bool gguf_read_header(const std::string & path, gguf_file & out, std::string & err);
// Read one tensor's bytes.
bool gguf_read_tensor(const std::string & path, const gguf_file & f, const gguf_tensor_info & t,
                      std::vector<uint8_t> & out, std::string & err);

struct gguf_writer {
    std::vector<std::pair<std::string, gguf_value>> kv;
    struct item { gguf_tensor_info info; const void * data; };
    std::vector<item> tensors;
    void add_u32(const std::string & k, uint32_t v);
    void add_f32(const std::string & k, float v);
    void add_str(const std::string & k, const std::string & v);
    void add_i32_array(const std::string & k, const std::vector<int32_t> & v);
    void add_tensor(const std::string & name, int32_t type, const std::vector<int64_t> & ne, const void * data);
    bool write(const std::string & path, std::string & err) const;
};

int64_t gguf_tensor_nbytes(int32_t type, const std::vector<int64_t> & ne);

} // namespace z2
