// gguf.cpp — GGUF reader (mmap) and writer.
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>

namespace gguf {

void type_geometry(int type, int64_t & block, int64_t & bytes) {
    switch (type) {
        case 0:  block = 1;   bytes = 4;   return;   // F32
        case 1:  block = 1;   bytes = 2;   return;   // F16
        case 2:  block = 32;  bytes = 18;  return;   // Q4_0
        case 3:  block = 32;  bytes = 20;  return;   // Q4_1
        case 6:  block = 32;  bytes = 22;  return;   // Q5_0
        case 7:  block = 32;  bytes = 24;  return;   // Q5_1
        case 8:  block = 32;  bytes = 34;  return;   // Q8_0
        case 9:  block = 32;  bytes = 36;  return;   // Q8_1
        case 10: block = 256; bytes = 84;  return;   // Q2_K
        case 11: block = 256; bytes = 110; return;   // Q3_K
        case 12: block = 256; bytes = 144; return;   // Q4_K
        case 13: block = 256; bytes = 176; return;   // Q5_K
        case 14: block = 256; bytes = 210; return;   // Q6_K
        case 15: block = 256; bytes = 292; return;   // Q8_K
        case 24: block = 1;   bytes = 1;   return;   // I8
        case 25: block = 1;   bytes = 2;   return;   // I16
        case 26: block = 1;   bytes = 4;   return;   // I32
        case 27: block = 1;   bytes = 8;   return;   // I64
        case 28: block = 1;   bytes = 8;   return;   // F64
        case 30: block = 1;   bytes = 2;   return;   // BF16
    }
    block = 0;
    bytes = 0;
}

int64_t row_bytes(int type, int64_t n) {
    int64_t b, s;
    type_geometry(type, b, s);
    if (b <= 0 || n % b) return -1;
    return n / b * s;
}

const char * type_name(int type) {
    switch (type) {
        case 0: return "F32";   case 1: return "F16";   case 2: return "Q4_0"; case 3: return "Q4_1";
        case 6: return "Q5_0";  case 7: return "Q5_1";  case 8: return "Q8_0"; case 9: return "Q8_1";
        case 10: return "Q2_K"; case 11: return "Q3_K"; case 12: return "Q4_K"; case 13: return "Q5_K";
        case 14: return "Q6_K"; case 15: return "Q8_K"; case 30: return "BF16";
    }
    return "?";
}

// ---------------------------------------------------------------------------
// reader
// ---------------------------------------------------------------------------
namespace {
struct cursor {
    const uint8_t * p;
    const uint8_t * end;
    bool ok = true;
    bool take(void * dst, size_t n) {
        if (!ok || (size_t)(end - p) < n) { ok = false; return false; }
        memcpy(dst, p, n);
        p += n;
        return true;
    }
    template <typename T> T get() {
        T v{};
        take(&v, sizeof(T));
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!ok || (uint64_t)(end - p) < n) { ok = false; return {}; }
        std::string s((const char *)p, (size_t)n);
        p += n;
        return s;
    }
};

bool read_value(cursor & c, value_type t, value & v, int depth) {
    v.type = t;
    switch (t) {
        case T_U8:   v.u = c.get<uint8_t>(); break;
        case T_I8:   v.i = c.get<int8_t>(); break;
        case T_U16:  v.u = c.get<uint16_t>(); break;
        case T_I16:  v.i = c.get<int16_t>(); break;
        case T_U32:  v.u = c.get<uint32_t>(); break;
        case T_I32:  v.i = c.get<int32_t>(); break;
        case T_F32:  v.f = c.get<float>(); break;
        case T_BOOL: v.u = c.get<uint8_t>(); break;
        case T_STRING: v.s = c.str(); break;
        case T_U64:  v.u = c.get<uint64_t>(); break;
        case T_I64:  v.i = c.get<int64_t>(); break;
        case T_F64:  v.f = c.get<double>(); break;
        case T_ARRAY: {
            if (depth > 2) return false;
            v.arr_type = (value_type)c.get<uint32_t>();
            const uint64_t n = c.get<uint64_t>();
            if (!c.ok || n > (uint64_t)(c.end - c.p)) return false;
            v.arr.resize((size_t)n);
            for (uint64_t k = 0; k < n && c.ok; k++)
                if (!read_value(c, v.arr_type, v.arr[k], depth + 1)) return false;
            break;
        }
        default: return false;
    }
    return c.ok;
}
}  // namespace

reader::~reader() {
    if (map_) munmap(map_, size_);
}

bool reader::open(const std::string & path, std::string & err) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) { err = "cannot open " + path; return false; }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        ::close(fd);
        err = "cannot stat or too small: " + path;
        return false;
    }
    size_ = (size_t)st.st_size;
    map_ = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (map_ == MAP_FAILED) { map_ = nullptr; err = "mmap failed: " + path; return false; }

    cursor c{(const uint8_t *)map_, (const uint8_t *)map_ + size_};
    const uint32_t magic = c.get<uint32_t>();
    if (magic != 0x46554747u) { err = "not a GGUF file: " + path; return false; }
    version_ = c.get<uint32_t>();
    if (version_ < 2 || version_ > 3) { err = "unsupported GGUF version " + std::to_string(version_); return false; }
    const uint64_t n_tensors = c.get<uint64_t>();
    const uint64_t n_kv = c.get<uint64_t>();
    if (!c.ok || n_tensors > (1u << 24) || n_kv > (1u << 24)) { err = "corrupt GGUF header"; return false; }
    for (uint64_t k = 0; k < n_kv; k++) {
        std::string key = c.str();
        const value_type t = (value_type)c.get<uint32_t>();
        value v;
        if (!c.ok || !read_value(c, t, v, 0)) { err = "corrupt GGUF key/value at key '" + key + "'"; return false; }
        kv_index_[key] = kv_.size();
        kv_.emplace_back(std::move(key), std::move(v));
    }
    const value * al = find("general.alignment");
    if (al && (al->type == T_U32 || al->type == T_U64) && al->u > 0) alignment_ = (uint32_t)al->u;
    for (uint64_t k = 0; k < n_tensors; k++) {
        tensor_info ti;
        ti.name = c.str();
        ti.n_dims = (int)c.get<uint32_t>();
        if (!c.ok || ti.n_dims < 1 || ti.n_dims > 4) { err = "corrupt tensor info for '" + ti.name + "'"; return false; }
        for (int d = 0; d < ti.n_dims; d++) ti.ne[d] = (int64_t)c.get<uint64_t>();
        ti.type = (int)c.get<uint32_t>();
        ti.offset = c.get<uint64_t>();
        if (!c.ok) { err = "truncated tensor infos"; return false; }
        tensor_index_[ti.name] = tensors_.size();
        tensors_.push_back(ti);
    }
    const size_t pos = (size_t)(c.p - (const uint8_t *)map_);
    const size_t data0 = (pos + alignment_ - 1) / alignment_ * alignment_;
    for (auto & ti : tensors_) {
        const int64_t rb = row_bytes(ti.type, ti.ne[0]);
        if (rb < 0) { ti.nbytes = 0; continue; }   // unknown type: usable only if never read
        ti.nbytes = (uint64_t)rb * ti.ne[1] * ti.ne[2] * ti.ne[3];
        if (data0 + ti.offset + ti.nbytes > size_) { err = "tensor '" + ti.name + "' runs past end of file"; return false; }
        ti.data = (const uint8_t *)map_ + data0 + ti.offset;
    }
    return true;
}

const value * reader::find(const std::string & key) const {
    auto it = kv_index_.find(key);
    return it == kv_index_.end() ? nullptr : &kv_[it->second].second;
}

bool reader::get_u32(const std::string & key, uint32_t & out) const {
    const value * v = find(key);
    if (!v) return false;
    switch (v->type) {
        case T_U8: case T_U16: case T_U32: case T_U64: case T_BOOL: out = (uint32_t)v->u; return true;
        case T_I8: case T_I16: case T_I32: case T_I64: out = (uint32_t)v->i; return true;
        default: return false;
    }
}

bool reader::get_f32(const std::string & key, float & out) const {
    const value * v = find(key);
    if (!v) return false;
    if (v->type == T_F32 || v->type == T_F64) { out = (float)v->f; return true; }
    return false;
}

bool reader::get_str(const std::string & key, std::string & out) const {
    const value * v = find(key);
    if (!v || v->type != T_STRING) return false;
    out = v->s;
    return true;
}

const tensor_info * reader::tensor(const std::string & name) const {
    auto it = tensor_index_.find(name);
    return it == tensor_index_.end() ? nullptr : &tensors_[it->second];
}

// ---------------------------------------------------------------------------
// writer
// ---------------------------------------------------------------------------
void writer::set_value(const std::string & key, const value & v) {
    for (auto & kv : kv_)
        if (kv.first == key) { kv.second = v; return; }
    kv_.emplace_back(key, v);
}
void writer::set_u32(const std::string & key, uint32_t x) {
    value v;
    v.type = T_U32;
    v.u = x;
    set_value(key, v);
}
void writer::set_f32(const std::string & key, float x) {
    value v;
    v.type = T_F32;
    v.f = x;
    set_value(key, v);
}
void writer::set_str(const std::string & key, const std::string & s) {
    value v;
    v.type = T_STRING;
    v.s = s;
    set_value(key, v);
}

void writer::add_tensor(const std::string & name, int type, int n_dims, const int64_t * ne, const void * data,
                        uint64_t nbytes) {
    pending p;
    p.info.name = name;
    p.info.type = type;
    p.info.n_dims = n_dims;
    for (int d = 0; d < 4; d++) p.info.ne[d] = d < n_dims ? ne[d] : 1;
    p.info.nbytes = nbytes;
    p.data = data;
    tensors_.push_back(p);
}

namespace {
struct out_file {
    FILE * f;
    bool ok = true;
    void put(const void * p, size_t n) {
        if (ok && n && fwrite(p, 1, n, f) != n) ok = false;
    }
    template <typename T> void put(T v) { put(&v, sizeof(T)); }
    void str(const std::string & s) {
        put<uint64_t>(s.size());
        put(s.data(), s.size());
    }
    void val(const value & v) {
        switch (v.type) {
            case T_U8: put<uint8_t>((uint8_t)v.u); break;
            case T_I8: put<int8_t>((int8_t)v.i); break;
            case T_U16: put<uint16_t>((uint16_t)v.u); break;
            case T_I16: put<int16_t>((int16_t)v.i); break;
            case T_U32: put<uint32_t>((uint32_t)v.u); break;
            case T_I32: put<int32_t>((int32_t)v.i); break;
            case T_F32: put<float>((float)v.f); break;
            case T_BOOL: put<uint8_t>((uint8_t)v.u); break;
            case T_STRING: str(v.s); break;
            case T_U64: put<uint64_t>(v.u); break;
            case T_I64: put<int64_t>(v.i); break;
            case T_F64: put<double>(v.f); break;
            case T_ARRAY:
                put<uint32_t>(v.arr_type);
                put<uint64_t>(v.arr.size());
                for (const auto & e : v.arr) val(e);
                break;
        }
    }
};
}  // namespace

bool writer::write(const std::string & path, std::string & err) const {
    const uint32_t align = 32;
    FILE * f = fopen(path.c_str(), "wb");
    if (!f) { err = "cannot create " + path; return false; }
    out_file o{f};
    o.put<uint32_t>(0x46554747u);
    o.put<uint32_t>(3);
    o.put<uint64_t>(tensors_.size());
    o.put<uint64_t>(kv_.size());
    for (const auto & kv : kv_) {
        o.str(kv.first);
        o.put<uint32_t>(kv.second.type);
        o.val(kv.second);
    }
    uint64_t off = 0;
    for (const auto & t : tensors_) {
        o.str(t.info.name);
        o.put<uint32_t>((uint32_t)t.info.n_dims);
        for (int d = 0; d < t.info.n_dims; d++) o.put<uint64_t>((uint64_t)t.info.ne[d]);
        o.put<uint32_t>((uint32_t)t.info.type);
        o.put<uint64_t>(off);
        off += (t.info.nbytes + align - 1) / align * align;
    }
    static const uint8_t zeros[64] = {0};
    long pos = ftell(f);
    if (pos % align) o.put(zeros, align - pos % align);
    for (const auto & t : tensors_) {
        o.put(t.data, t.info.nbytes);
        const uint64_t pad = (align - t.info.nbytes % align) % align;
        o.put(zeros, pad);
    }
    const bool ok = o.ok && fclose(f) == 0;
    if (!ok) err = "write failed: " + path;
    return ok;
}

}  // namespace gguf
