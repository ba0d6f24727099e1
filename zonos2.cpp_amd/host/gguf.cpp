// gguf.cpp — minimal GGUF reader/writer (see gguf.h for the container layout).
#include "gguf.h"
#include "z2_formats.h"

#include <cstdio>
#include <cstring>
#include <memory>

namespace z2 {

namespace {

size_t scalar_size(uint32_t t) {
    switch (t) {
        case GV_U8: case GV_I8: case GV_BOOL: return 1;
        case GV_U16: case GV_I16: return 2;
        case GV_U32: case GV_I32: case GV_F32: return 4;
        case GV_U64: case GV_I64: case GV_F64: return 8;
    }
    return 0;
}

struct reader {
    FILE * f = nullptr;
    bool ok = true;
    template <class T> T get() { T v{}; if (fread(&v, sizeof(T), 1, f) != 1) ok = false; return v; }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!ok || n > (1ull << 30)) { ok = false; return {}; }
        std::string s(n, '\0');
        if (n && fread(&s[0], 1, n, f) != n) ok = false;
        return s;
    }
    void bytes(std::vector<uint8_t> & out, size_t n) {
        out.resize(n);
        if (n && fread(out.data(), 1, n, f) != n) ok = false;
    }
};

struct writer {
    FILE * f = nullptr;
    bool ok = true;
    void put(const void * p, size_t n) { if (n && fwrite(p, 1, n, f) != n) ok = false; }
    template <class T> void val(T v) { put(&v, sizeof(T)); }
    void str(const std::string & s) { val<uint64_t>(s.size()); put(s.data(), s.size()); }
};

void write_value(writer & w, const gguf_value & v) {
    w.val<uint32_t>(v.type);
    if (v.type == GV_STR) { w.str(v.str); return; }
    if (v.type == GV_ARR) {
        w.val<uint32_t>(v.arr_type);
        w.val<uint64_t>(v.n);
        if (v.arr_type == GV_STR) for (auto & s : v.strs) w.str(s);
        else w.put(v.raw.data(), v.raw.size());
        return;
    }
    w.put(v.raw.data(), v.raw.size());
}

} // namespace

int64_t gguf_tensor_nbytes(int32_t type, const std::vector<int64_t> & ne) {
    if (!type_known(type) || ne.empty() || ne[0] % type_block(type)) return -1;
    int64_t rows = 1;
    for (size_t i = 1; i < ne.size(); ++i) rows *= ne[i];
    return row_bytes(type, ne[0]) * rows;
}

double gguf_value::as_f64() const {
    if (type == GV_STR || type == GV_ARR || raw.empty()) return 0.0;
    switch (type) {
        case GV_F32: { float x; std::memcpy(&x, raw.data(), 4); return x; }
        case GV_F64: { double x; std::memcpy(&x, raw.data(), 8); return x; }
        default: return (double) as_i64();
    }
}

int64_t gguf_value::as_i64() const {
    if (type == GV_STR || type == GV_ARR || raw.empty()) return 0;
    switch (type) {
        case GV_U8: return raw[0];
        case GV_I8: return (int8_t) raw[0];
        case GV_BOOL: return raw[0] != 0;
        case GV_U16: { uint16_t x; std::memcpy(&x, raw.data(), 2); return x; }
        case GV_I16: { int16_t x; std::memcpy(&x, raw.data(), 2); return x; }
        case GV_U32: { uint32_t x; std::memcpy(&x, raw.data(), 4); return x; }
        case GV_I32: { int32_t x; std::memcpy(&x, raw.data(), 4); return x; }
        case GV_U64: { uint64_t x; std::memcpy(&x, raw.data(), 8); return (int64_t) x; }
        case GV_I64: { int64_t x; std::memcpy(&x, raw.data(), 8); return x; }
        case GV_F32: { float x; std::memcpy(&x, raw.data(), 4); return (int64_t) x; }
        case GV_F64: { double x; std::memcpy(&x, raw.data(), 8); return (int64_t) x; }
    }
    return 0;
}

const gguf_value * gguf_file::find(const std::string & k) const {
    auto it = kv.find(k);
    return it == kv.end() ? nullptr : &it->second;
}

const gguf_tensor_info * gguf_file::tensor(const std::string & n) const {
    for (auto & t : tensors) if (t.name == n) return &t;
    return nullptr;
}

bool gguf_read_header(const std::string & path, gguf_file & out, std::string & err) {
    std::unique_ptr<FILE, int (*)(FILE *)> fp(fopen(path.c_str(), "rb"), fclose);
    if (!fp) { err = "cannot open " + path; return false; }
    reader r{fp.get()};
    char magic[4];
    if (fread(magic, 1, 4, r.f) != 4 || std::memcmp(magic, "GGUF", 4) != 0) { err = "bad magic"; return false; }
    out = gguf_file();
    out.version = r.get<uint32_t>();
    if (out.version < 2 || out.version > 3) { err = "unsupported GGUF version"; return false; }
    const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
    if (!r.ok || n_tensors > (1u << 24) || n_kv > (1u << 24)) { err = "bad counts"; return false; }
    for (uint64_t i = 0; i < n_kv && r.ok; ++i) {
        std::string key = r.str();
        gguf_value v;
        v.type = r.get<uint32_t>();
        if (v.type == GV_STR) v.str = r.str();
        else if (v.type == GV_ARR) {
            v.arr_type = r.get<uint32_t>();
            v.n = r.get<uint64_t>();
            if (v.arr_type == GV_STR) { for (uint64_t j = 0; j < v.n && r.ok; ++j) v.strs.push_back(r.str()); }
            else {
                const size_t es = scalar_size(v.arr_type);
                if (!es || v.n > (1ull << 32)) { err = "bad array in " + key; return false; }
                r.bytes(v.raw, es * v.n);
            }
        } else {
            const size_t es = scalar_size(v.type);
            if (!es) { err = "bad kv type in " + key; return false; }
            r.bytes(v.raw, es);
        }
        out.kv_order.push_back(key);
        out.kv[key] = std::move(v);
    }
    if (auto * a = out.find("general.alignment")) out.alignment = (uint64_t) a->as_i64();
    if (out.alignment == 0 || (out.alignment & (out.alignment - 1))) { err = "bad alignment"; return false; }
    for (uint64_t i = 0; i < n_tensors && r.ok; ++i) {
        gguf_tensor_info t;
        t.name = r.str();
        const uint32_t nd = r.get<uint32_t>();
        if (nd == 0 || nd > 4) { err = "bad n_dims for " + t.name; return false; }
        for (uint32_t j = 0; j < nd; ++j) t.ne.push_back((int64_t) r.get<uint64_t>());
        t.type = (int32_t) r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
        const int64_t nb = gguf_tensor_nbytes(t.type, t.ne);
        if (nb < 0) { err = "unsupported tensor type/shape for " + t.name; return false; }
        t.nbytes = (uint64_t) nb;
        out.tensors.push_back(std::move(t));
    }
    if (!r.ok) { err = "truncated header"; return false; }
    const uint64_t pos = (uint64_t) ftello(r.f);
    out.data_offset = (pos + out.alignment - 1) / out.alignment * out.alignment;
    return true;
}

bool gguf_read_tensor(const std::string & path, const gguf_file & f, const gguf_tensor_info & t,
                      std::vector<uint8_t> & out, std::string & err) {
    std::unique_ptr<FILE, int (*)(FILE *)> fp(fopen(path.c_str(), "rb"), fclose);
    if (!fp) { err = "cannot open " + path; return false; }
    if (fseeko(fp.get(), (off_t) (f.data_offset + t.offset), SEEK_SET) != 0) { err = "seek failed"; return false; }
    out.resize(t.nbytes);
    if (t.nbytes && fread(out.data(), 1, t.nbytes, fp.get()) != t.nbytes) { err = "read failed for " + t.name; return false; }
    return true;
}

void gguf_writer::add_u32(const std::string & k, uint32_t v) {
    gguf_value x; x.type = GV_U32; x.raw.resize(4); std::memcpy(x.raw.data(), &v, 4); kv.emplace_back(k, x);
}
void gguf_writer::add_f32(const std::string & k, float v) {
    gguf_value x; x.type = GV_F32; x.raw.resize(4); std::memcpy(x.raw.data(), &v, 4); kv.emplace_back(k, x);
}
void gguf_writer::add_str(const std::string & k, const std::string & v) {
    gguf_value x; x.type = GV_STR; x.str = v; kv.emplace_back(k, x);
}
void gguf_writer::add_i32_array(const std::string & k, const std::vector<int32_t> & v) {
    gguf_value x; x.type = GV_ARR; x.arr_type = GV_I32; x.n = v.size();
    x.raw.resize(v.size() * 4); if (!v.empty()) std::memcpy(x.raw.data(), v.data(), v.size() * 4);
    kv.emplace_back(k, x);
}
void gguf_writer::add_tensor(const std::string & name, int32_t type, const std::vector<int64_t> & ne, const void * data) {
    item it; it.info.name = name; it.info.type = type; it.info.ne = ne;
    it.info.nbytes = (uint64_t) gguf_tensor_nbytes(type, ne); it.data = data;
    tensors.push_back(it);
}

bool gguf_writer::write(const std::string & path, std::string & err) const {
    std::unique_ptr<FILE, int (*)(FILE *)> fp(fopen(path.c_str(), "wb"), fclose);
    if (!fp) { err = "cannot create " + path; return false; }
    writer w{fp.get()};
    const uint64_t align = 32;
    w.put("GGUF", 4);
    w.val<uint32_t>(3);
    w.val<uint64_t>(tensors.size());
    w.val<uint64_t>(kv.size());
    for (auto & p : kv) { w.str(p.first); write_value(w, p.second); }
    uint64_t off = 0;
    std::vector<uint64_t> offs;
    for (auto & t : tensors) {
        w.str(t.info.name);
        w.val<uint32_t>((uint32_t) t.info.ne.size());
        for (int64_t n : t.info.ne) w.val<uint64_t>((uint64_t) n);
        w.val<uint32_t>((uint32_t) t.info.type);
        w.val<uint64_t>(off);
        offs.push_back(off);
        off += (t.info.nbytes + align - 1) / align * align;
    }
    const uint64_t pos = (uint64_t) ftello(fp.get());
    const uint64_t data_off = (pos + align - 1) / align * align;
    static const uint8_t zeros[64] = {0};
    w.put(zeros, data_off - pos);
    for (size_t i = 0; i < tensors.size(); ++i) {
        w.put(tensors[i].data, tensors[i].info.nbytes);
        const uint64_t pad = (tensors[i].info.nbytes + align - 1) / align * align - tensors[i].info.nbytes;
        w.put(zeros, pad);
    }
    if (!w.ok) { err = "write failed"; return false; }
    return true;
}

} // namespace z2
