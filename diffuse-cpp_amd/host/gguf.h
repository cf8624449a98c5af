// gguf.h — GGUF v2/v3 reader (mmap) and writer.
//
// Format: "GGUF" magic, u32 version, u64 n_tensors, u64 n_kv, typed key/value
// pairs, tensor infos {name, u32 n_dims, u64 ne[n_dims], u32 type, u64 offset},
// then tensor data aligned to general.alignment (default 32).  This is the file
// format diffuse-cpp loads through GGML's gguf_init_from_file
// (src/diffuse-model.cpp:86-95) and writes through gguf_write_to_file
// (tools/quantize.cpp:336).
#pragma once
#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace gguf {

enum value_type : uint32_t {
    T_U8 = 0, T_I8 = 1, T_U16 = 2, T_I16 = 3, T_U32 = 4, T_I32 = 5, T_F32 = 6, T_BOOL = 7,
    T_STRING = 8, T_ARRAY = 9, T_U64 = 10, T_I64 = 11, T_F64 = 12,
};

struct value {
    value_type type = T_U32;
    uint64_t u = 0;      // unsigned integers and bool
    int64_t  i = 0;      // signed integers
    double   f = 0;      // floats
    std::string s;
    value_type arr_type = T_U8;
    std::vector<value> arr;
};

struct tensor_info {
    std::string name;
    int         type = 0;
    int64_t     ne[4] = {1, 1, 1, 1};
    int         n_dims = 0;
    uint64_t    offset = 0;   // relative to the data section
    uint64_t    nbytes = 0;
    const uint8_t * data = nullptr;   // into the mapping (reader)
};

// GGML block geometry (elements per block, bytes per block); {0,0} if unknown.
void type_geometry(int type, int64_t & block, int64_t & bytes);
int64_t row_bytes(int type, int64_t n);   // -1 if n is not a block multiple / unknown type
const char * type_name(int type);

class reader {
public:
    ~reader();
    // Returns false with err set on failure.
    bool open(const std::string & path, std::string & err);
    const value * find(const std::string & key) const;
    bool get_u32(const std::string & key, uint32_t & out) const;   // any integer type
    bool get_f32(const std::string & key, float & out) const;      // any float type
    bool get_str(const std::string & key, std::string & out) const;
    const tensor_info * tensor(const std::string & name) const;
    const std::vector<tensor_info> & tensors() const { return tensors_; }
    const std::vector<std::pair<std::string, value>> & kvs() const { return kv_; }
    uint32_t version() const { return version_; }
    uint32_t alignment() const { return alignment_; }

private:
    void * map_ = nullptr;
    size_t size_ = 0;
    uint32_t version_ = 0, alignment_ = 32;
    std::vector<std::pair<std::string, value>> kv_;
    std::map<std::string, size_t> kv_index_;
    std::vector<tensor_info> tensors_;
    std::map<std::string, size_t> tensor_index_;
};

class writer {
public:
    void set_u32(const std::string & key, uint32_t v);
    void set_f32(const std::string & key, float v);
    void set_str(const std::string & key, const std::string & v);
    void set_value(const std::string & key, const value & v);   // copy a parsed value
    // data must stay valid until write(); ne[0] is the contiguous dimension.
    void add_tensor(const std::string & name, int type, int n_dims, const int64_t * ne, const void * data,
                    uint64_t nbytes);
    bool write(const std::string & path, std::string & err) const;

private:
    std::vector<std::pair<std::string, value>> kv_;
    struct pending { tensor_info info; const void * data; };
    std::vector<pending> tensors_;
};

}  // namespace gguf
