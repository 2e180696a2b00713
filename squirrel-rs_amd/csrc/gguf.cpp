#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>

#include "../../include/squirrel_hip.h"

namespace sq {

int set_error(int code, const std::string& msg);

namespace {

constexpr uint64_t kAlign = 32;  // GGUF_DEFAULT_ALIGNMENT, gguf_file.rs:10

struct Cursor {
    const uint8_t* p;
    size_t size;
    size_t pos = 0;
    std::string err;

    bool take(void* out, size_t n) {
        if (pos + n > size || pos + n < pos) {
            err = "unexpected end of file";
            return false;
        }
        memcpy(out, p + pos, n);
        pos += n;
        return true;
    }
    template <typename T>
    bool get(T* v) { return take(v, sizeof(T)); }

    // UTF-8 validity as String::from_utf8 requires (binary_reader_common.rs:76-83).
    static bool utf8_ok(const std::string& s) {
        const unsigned char* b = (const unsigned char*)s.data();
        const size_t n = s.size();
        size_t i = 0;
        while (i < n) {
            const unsigned c = b[i];
            int extra;
            uint32_t cp;
            if (c < 0x80) {
                i++;
                continue;
            } else if ((c >> 5) == 6) {
                extra = 1;
                cp = c & 0x1F;
            } else if ((c >> 4) == 14) {
                extra = 2;
                cp = c & 0x0F;
            } else if ((c >> 3) == 30) {
                extra = 3;
                cp = c & 0x07;
            } else {
                return false;
            }
            if (i + extra >= n) return false;
            for (int k = 1; k <= extra; k++) {
                if ((b[i + k] & 0xC0) != 0x80) return false;
                cp = (cp << 6) | (b[i + k] & 0x3F);
            }
            const uint32_t min_cp = extra == 1 ? 0x80 : extra == 2 ? 0x800 : 0x10000;
            if (cp < min_cp || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
            i += extra + 1;
        }
        return true;
    }

    bool str(std::string* s) {
        uint64_t n;
        if (!get(&n)) return false;
        if (n > size - pos) {
            err = "unexpected end of file";
            return false;
        }
        s->assign((const char*)p + pos, n);
        pos += n;
        if (!utf8_ok(*s)) {
            err = "invalid utf-8 string";
            return false;
        }
        return true;
    }

    bool value(uint32_t t, GGUFValue* v, int depth = 0) {
        v->type = t;
        switch (t) {
            case GT_U8: { uint8_t x; if (!get(&x)) return false; v->u = x; return true; }
            case GT_I8: { int8_t x; if (!get(&x)) return false; v->i = x; return true; }
            case GT_U16: { uint16_t x; if (!get(&x)) return false; v->u = x; return true; }
            case GT_I16: { int16_t x; if (!get(&x)) return false; v->i = x; return true; }
            case GT_U32: { uint32_t x; if (!get(&x)) return false; v->u = x; return true; }
            case GT_I32: { int32_t x; if (!get(&x)) return false; v->i = x; return true; }
            case GT_U64: { uint64_t x; if (!get(&x)) return false; v->u = x; return true; }
            case GT_I64: { int64_t x; if (!get(&x)) return false; v->i = x; return true; }
            case GT_F32: { float x; if (!get(&x)) return false; v->f32 = x; v->f = x; return true; }
            case GT_F64: { double x; if (!get(&x)) return false; v->f = x; return true; }
            case GT_BOOL: {
                uint8_t x;
                if (!get(&x)) return false;
                if (x > 1) { err = "Invalid bool data!"; return false; }
                v->u = x;
                return true;
            }
            case GT_STRING: return str(&v->s);
            case GT_ARRAY: {
                uint32_t at;
                uint64_t n;
                if (!get(&at)) return false;
                if (at > GT_F64) { err = "Invalid GGUF array type!"; return false; }
                if (!get(&n)) return false;
                if (depth > 8) { err = "array nesting too deep"; return false; }
                v->arr_type = at;
                // Each element takes at least one byte: a cheap bound before reserving.
                if (n > size - pos) { err = "unexpected end of file"; return false; }
                v->arr.resize(n);
                for (uint64_t k = 0; k < n; k++)
                    if (!value(at, &v->arr[k], depth + 1)) return false;
                return true;
            }
            default:
                err = "Invalid GGUF Type!";
                return false;
        }
    }
};

}  // namespace

bool ggml_type_known(uint32_t t) {
    static const uint32_t known[] = {0, 1, 2, 3, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18,
                                     19, 20, 21, 22, 23, 24, 25, 26, 27, 28, 29, 30, 34, 35, 39};
    for (uint32_t k : known)
        if (k == t) return true;
    return false;
}

bool ggml_block(uint32_t t, uint64_t* elems, uint64_t* bytes) {
    switch (t) {
        case 0: *elems = 1; *bytes = 4; return true;    // F32
        case 30: *elems = 1; *bytes = 2; return true;   // BF16
        case 8: *elems = 32; *bytes = 34; return true;  // Q8_0
        case 2: *elems = 32; *bytes = 18; return true;  // Q4_0
        default: return false;
    }
}

GGUFFile::~GGUFFile() {
    if (map_) munmap(map_, map_len_);
}

int GGUFFile::open(const std::string& path) {
    int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) return set_error(SQ_ERR_IO, "cannot open " + path);
    struct stat st;
    if (fstat(fd, &st) != 0) {
        ::close(fd);
        return set_error(SQ_ERR_IO, "cannot stat " + path);
    }
    size_t len = (size_t)st.st_size;
    void* m = nullptr;
    if (len > 0) {
        m = mmap(nullptr, len, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            ::close(fd);
            return set_error(SQ_ERR_IO, "cannot mmap " + path);
        }
    }
    ::close(fd);
    map_ = m;
    map_len_ = len;
    return parse((const uint8_t*)m, len);
}

int GGUFFile::parse(const uint8_t* data, size_t sz) {
    base = data;
    size = sz;
    Cursor c{data, sz};
    uint64_t n_tensors = 0, n_kv = 0;
    if (!c.get(&magic) || !c.get(&version) || !c.get(&n_tensors) || !c.get(&n_kv))
        return set_error(SQ_ERR_FORMAT, "gguf header: " + c.err);
    for (uint64_t k = 0; k < n_kv; k++) {
        std::string key;
        uint32_t t;
        if (!c.str(&key) || !c.get(&t)) return set_error(SQ_ERR_FORMAT, "gguf metadata: " + c.err);
        if (t > GT_F64) return set_error(SQ_ERR_FORMAT, "gguf metadata: Invalid GGUF Type!");
        GGUFValue v;
        if (!c.value(t, &v)) return set_error(SQ_ERR_FORMAT, "gguf metadata " + key + ": " + c.err);
        meta[key] = std::move(v);
    }
    for (uint64_t k = 0; k < n_tensors; k++) {
        GGUFTensorInfo ti;
        uint32_t nd;
        if (!c.str(&ti.name) || !c.get(&nd)) return set_error(SQ_ERR_FORMAT, "gguf tensor info: " + c.err);
        if (nd > 8) return set_error(SQ_ERR_FORMAT, "gguf tensor info: too many dimensions");
        ti.numel = 1;
        for (uint32_t d = 0; d < nd; d++) {
            uint64_t v;
            if (!c.get(&v)) return set_error(SQ_ERR_FORMAT, "gguf tensor info: " + c.err);
            ti.dims.push_back(v);
            ti.numel *= v;
        }
        if (!c.get(&ti.ggml_type)) return set_error(SQ_ERR_FORMAT, "gguf tensor info: " + c.err);
        if (!ggml_type_known(ti.ggml_type))
            return set_error(SQ_ERR_FORMAT, "unknown GGML type id " + std::to_string(ti.ggml_type) +
                                                " in tensor \"" + ti.name + "\"");
        if (!c.get(&ti.offset)) return set_error(SQ_ERR_FORMAT, "gguf tensor info: " + c.err);
        std::string name = ti.name;
        tensors[name] = std::move(ti);
    }
    // The reference always pads to 32 bytes (gguf_file.rs:10,44-46); llama.cpp
    // writes general.alignment (a power-of-two u32, 32 unless chosen
    // otherwise) and pads the data section and every tensor to it.  Honouring
    // the key reads every file the reference reads (alignment 32) and also
    // files written with another alignment.
    uint64_t align = kAlign;
    auto al = meta.find("general.alignment");
    if (al != meta.end()) {
        const uint64_t a = al->second.u;
        if (al->second.type != GT_U32 || a == 0 || (a & (a - 1)) != 0)
            return set_error(SQ_ERR_FORMAT, "general.alignment must be a power-of-two u32");
        align = a;
    }
    alignment = align;
    data_offset = (c.pos + align - 1) & ~(align - 1);
    return 0;
}

int GGUFFile::tensor_bytes(const GGUFTensorInfo& t, uint64_t* out) const {
    uint64_t e, b;
    if (!ggml_block(t.ggml_type, &e, &b) || t.numel % e != 0)
        return set_error(SQ_ERR_UNSUPPORTED, "UnsupportedQuantScheme(type " + std::to_string(t.ggml_type) +
                                                 ") for tensor " + t.name);
    *out = t.numel / e * b;
    return 0;
}

const uint8_t* GGUFFile::tensor_data(const std::string& name, int* status) const {
    auto it = tensors.find(name);
    if (it == tensors.end()) {
        *status = set_error(SQ_ERR_WEIGHTS, "MissingTensor(" + name + ")");
        return nullptr;
    }
    uint64_t nb;
    if ((*status = tensor_bytes(it->second, &nb)) != 0) return nullptr;
    uint64_t start = data_offset + it->second.offset;
    if (start > size || nb > size - start) {
        *status = set_error(SQ_ERR_FORMAT, "tensor " + name + " runs past the end of the file");
        return nullptr;
    }
    *status = 0;
    return base + start;
}

void GGUFWriter::add_u32(const std::string& k, uint32_t v) { kvs_.push_back({k, GT_U32, v, 0.f, {}}); }
void GGUFWriter::add_f32(const std::string& k, float v) { kvs_.push_back({k, GT_F32, 0, v, {}}); }
void GGUFWriter::add_string(const std::string& k, const std::string& v) {
    kvs_.push_back({k, GT_STRING, 0, 0.f, v});
}
void GGUFWriter::add_tensor(const std::string& name, const std::vector<uint64_t>& dims, uint32_t type,
                            const void* data, uint64_t bytes) {
    ts_.push_back({name, dims, type, data, bytes});
}

int GGUFWriter::write(const std::string& path) const {
    FILE* f = fopen(path.c_str(), "wb");
    if (!f) return set_error(SQ_ERR_IO, "cannot create " + path);
    std::vector<uint8_t> h;
    auto put = [&](const void* p, size_t n) { h.insert(h.end(), (const uint8_t*)p, (const uint8_t*)p + n); };
    auto put_u32 = [&](uint32_t v) { put(&v, 4); };
    auto put_u64 = [&](uint64_t v) { put(&v, 8); };
    auto put_str = [&](const std::string& s) { put_u64(s.size()); put(s.data(), s.size()); };
    put_u32(0x46554747u);  // "GGUF"
    put_u32(3);
    put_u64(ts_.size());
    put_u64(kvs_.size());
    for (const KV& kv : kvs_) {
        put_str(kv.key);
        put_u32(kv.type);
        if (kv.type == GT_U32) put_u32(kv.u);
        else if (kv.type == GT_F32) put(&kv.f, 4);
        else put_str(kv.s);
    }
    uint64_t off = 0;
    std::vector<uint64_t> offs;
    for (const T& t : ts_) {
        put_str(t.name);
        put_u32((uint32_t)t.dims.size());
        for (uint64_t d : t.dims) put_u64(d);
        put_u32(t.type);
        put_u64(off);
        offs.push_back(off);
        off = (off + t.bytes + kAlign - 1) & ~(kAlign - 1);
    }
    while (h.size() % kAlign) h.push_back(0);
    bool ok = fwrite(h.data(), 1, h.size(), f) == h.size();
    static const uint8_t zeros[kAlign] = {0};
    for (size_t i = 0; ok && i < ts_.size(); i++) {
        ok = fwrite(ts_[i].data, 1, ts_[i].bytes, f) == ts_[i].bytes;
        uint64_t pad = ((ts_[i].bytes + kAlign - 1) & ~(kAlign - 1)) - ts_[i].bytes;
        if (ok && pad && i + 1 < ts_.size()) ok = fwrite(zeros, 1, pad, f) == pad;
    }
    if (fclose(f) != 0) ok = false;
    if (!ok) return set_error(SQ_ERR_IO, "write failed: " + path);
    return 0;
}

}  // namespace sq
