// gguf.cpp -- read-only GGUF reader (include/kernelcore/gguf.h): the file mapped with mmap, the
// metadata and tensor directory parsed with every length checked against the bytes left.
//
// Follows the reference reader's layout handling (llm/gguf.cpp:87-141): magic "GGUF", version >= 2,
// n_tensors and n_kv as u64, key/value pairs (scalars, strings, arrays of either), then per tensor
// name, n_dims, ne[n_dims] (u64), ggml type, offset; the data section starts at the header's end
// rounded up to general.alignment (32 when absent) and each tensor at data start + offset; bytes of
// a tensor = values / block values * block bytes, 0 for a type without a known block size (listed,
// not readable). Different from the reference: POSIX mmap instead of the Windows file mapping,
// string arrays (a tokenizer's vocabulary) are skipped with their count kept rather than copied,
// and offsets, sizes and counts are checked for overflow as well as for the end of the file.
#include "kernelcore/gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <map>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "internal.hpp"

namespace kcamd {
namespace gguf {

// Bytes per block and values per block of the ggml types with a known block size.
bool blockInfo(uint32_t t, size_t* bb, size_t* bv) {
    switch (t) {
        case KC_GGML_F32: *bb = 4, *bv = 1; return true;
        case KC_GGML_F16:
        case KC_GGML_BF16: *bb = 2, *bv = 1; return true;
        case KC_GGML_Q4_0: *bb = 18, *bv = 32; return true;
        case KC_GGML_Q4_1: *bb = 20, *bv = 32; return true;
        case KC_GGML_Q5_0: *bb = 22, *bv = 32; return true;
        case KC_GGML_Q5_1: *bb = 24, *bv = 32; return true;
        case KC_GGML_Q8_0: *bb = 34, *bv = 32; return true;
        case KC_GGML_Q2_K: *bb = 84, *bv = 256; return true;
        case KC_GGML_Q3_K: *bb = 110, *bv = 256; return true;
        case KC_GGML_Q4_K: *bb = 144, *bv = 256; return true;
        case KC_GGML_Q5_K: *bb = 176, *bv = 256; return true;
        case KC_GGML_Q6_K: *bb = 210, *bv = 256; return true;
        case KC_GGML_Q8_K: *bb = 292, *bv = 256; return true;
        default: return false;
    }
}

struct Entry {
    uint32_t type = 0;         // GGUF value type
    double num = 0;            // numeric scalars
    const char* str = nullptr; // strings: in the map
    size_t len = 0;
    uint32_t elem = 0;         // arrays: element type and count
    uint64_t count = 0;
};

struct Tensor {
    std::string name;
    int n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint32_t type = 0;
    uint64_t offset = 0;
    size_t bytes = 0;
    const uint8_t* data = nullptr;
};

struct Error {
    std::string what;
};

struct Reader {
    const uint8_t* p;
    const uint8_t* end;
    void need(uint64_t n) const {
        if (uint64_t(end - p) < n) throw Error{"truncated file"};
    }
    template <class T>
    T get() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, p, sizeof v);
        p += sizeof v;
        return v;
    }
    void str(const char** s, size_t* n) {
        const uint64_t len = get<uint64_t>();
        need(len);
        *s = reinterpret_cast<const char*>(p);
        *n = size_t(len);
        p += len;
    }
    // a scalar of value type t as a double (GGUF: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32,
    // 7 bool, 10 u64, 11 i64, 12 f64)
    double number(uint32_t t) {
        switch (t) {
            case 0: return get<uint8_t>();
            case 1: return get<int8_t>();
            case 2: return get<uint16_t>();
            case 3: return get<int16_t>();
            case 4: return get<uint32_t>();
            case 5: return get<int32_t>();
            case 6: return get<float>();
            case 7: return get<uint8_t>();
            case 10: return double(get<uint64_t>());
            case 11: return double(get<int64_t>());
            case 12: return get<double>();
            default: throw Error{"unknown value type " + std::to_string(t)};
        }
    }
    static size_t scalarBytes(uint32_t t) {
        switch (t) {
            case 0: case 1: case 7: return 1;
            case 2: case 3: return 2;
            case 4: case 5: case 6: return 4;
            case 10: case 11: case 12: return 8;
            default: return 0;
        }
    }
};

}  // namespace gguf
}  // namespace kcamd

struct kcGguf_st {
    int fd = -1;
    const uint8_t* base = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    size_t alignment = 32;
    std::map<std::string, kcamd::gguf::Entry> meta;
    std::vector<kcamd::gguf::Tensor> tensors;
    std::map<std::string, size_t> by_name;
    ~kcGguf_st() {
        if (base) munmap(const_cast<uint8_t*>(base), size);
        if (fd >= 0) close(fd);
    }
};

namespace {

using E = kcError_t;
constexpr E ok = kc::Error::Success;
using namespace kcamd::gguf;

E bad(const char* fmt, const std::string& s) {
    kcamd::setDetail(fmt, s.c_str());
    return kc::Error::InvalidValue;
}

void parse(kcGguf_st& g) {
    Reader r{g.base, g.base + g.size};
    if (r.get<uint32_t>() != 0x46554747u) throw Error{"bad magic (not a GGUF file)"};  // "GGUF"
    g.version = r.get<uint32_t>();
    if (g.version < 2 || g.version > 3) throw Error{"unsupported version " + std::to_string(g.version)};
    const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
    // every key/value and tensor entry takes at least 12 / 24 bytes: counts beyond that are corrupt
    if (n_kv > g.size / 12 || n_tensors > g.size / 24) throw Error{"implausible counts in the header"};
    for (uint64_t i = 0; i < n_kv; ++i) {
        const char* ks = nullptr;
        size_t kn = 0;
        r.str(&ks, &kn);
        Entry e;
        e.type = r.get<uint32_t>();
        if (e.type == 8) {
            r.str(&e.str, &e.len);
        } else if (e.type == 9) {
            e.elem = r.get<uint32_t>();
            e.count = r.get<uint64_t>();
            if (e.elem == 8) {
                for (uint64_t j = 0; j < e.count; ++j) {
                    const char* s;
                    size_t n;
                    r.str(&s, &n);
                }
            } else {
                const size_t eb = Reader::scalarBytes(e.elem);
                if (!eb) throw Error{"unsupported array element type " + std::to_string(e.elem)};
                if (e.count > uint64_t(r.end - r.p) / eb) throw Error{"truncated file"};
                r.p += e.count * eb;
            }
        } else {
            e.num = r.number(e.type);
        }
        g.meta[std::string(ks, kn)] = e;
    }
    g.tensors.resize(size_t(n_tensors));
    for (auto& t : g.tensors) {
        const char* ns;
        size_t nn;
        r.str(&ns, &nn);
        t.name.assign(ns, nn);
        const uint32_t nd = r.get<uint32_t>();
        if (nd < 1 || nd > 4) throw Error{"tensor " + t.name + ": " + std::to_string(nd) + " dimensions"};
        t.n_dims = int(nd);
        for (uint32_t d = 0; d < nd; ++d) {
            const uint64_t v = r.get<uint64_t>();
            if (v == 0 || v > (uint64_t(1) << 40)) throw Error{"tensor " + t.name + ": bad dimension"};
            t.ne[d] = int64_t(v);
        }
        t.type = r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
    }
    auto al = g.meta.find("general.alignment");
    if (al != g.meta.end()) {
        if (al->second.type == 8 || al->second.type == 9 || !(al->second.num >= 1) || al->second.num > 65536)
            throw Error{"bad general.alignment"};
        g.alignment = size_t(al->second.num);
    }
    const size_t header = size_t(r.p - g.base);
    const size_t data_start = (header + g.alignment - 1) / g.alignment * g.alignment;
    for (size_t i = 0; i < g.tensors.size(); ++i) {
        Tensor& t = g.tensors[i];
        size_t bb = 0, bv = 0;
        if (blockInfo(t.type, &bb, &bv)) {
            uint64_t n = 1;
            for (int d = 0; d < t.n_dims; ++d) {
                if (n > (uint64_t(1) << 50) / uint64_t(t.ne[d])) throw Error{"tensor " + t.name + ": too large"};
                n *= uint64_t(t.ne[d]);
            }
            if (n % bv) throw Error{"tensor " + t.name + ": size not a whole number of blocks"};
            t.bytes = size_t(n / bv * bb);
        }
        if (data_start > g.size || t.offset > g.size - data_start || t.bytes > g.size - data_start - t.offset)
            throw Error{"tensor past the end of the file: " + t.name};
        t.data = g.base + data_start + t.offset;
        if (!g.by_name.emplace(t.name, i).second) throw Error{"duplicate tensor name " + t.name};
    }
}

const Entry* findKey(kcGguf_t g, const char* key) {
    if (!key) return nullptr;
    auto it = g->meta.find(key);
    return it == g->meta.end() ? nullptr : &it->second;
}

}  // namespace

kcError_t kcGgufOpen(const char* path, kcGguf_t* out) noexcept {
    if (!out) return kc::Error::InvalidValue;
    *out = nullptr;
    if (!path) return bad("%s", "path is null");
    try {
        auto g = std::unique_ptr<kcGguf_st>(new kcGguf_st);
        g->fd = open(path, O_RDONLY | O_CLOEXEC);
        if (g->fd < 0) return bad("gguf: cannot open %s", path);
        struct stat st {};
        if (fstat(g->fd, &st) != 0 || st.st_size < 24) return bad("gguf: %s is too short to be a GGUF file", path);
        g->size = size_t(st.st_size);
        void* p = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
        if (p == MAP_FAILED) return bad("gguf: cannot map %s", path);
        g->base = static_cast<const uint8_t*>(p);
        parse(*g);
        *out = g.release();
        return ok;
    } catch (const Error& e) {
        return bad("gguf: %s", e.what);
    } catch (const std::bad_alloc&) {
        kcamd::setDetail("gguf: out of host memory");
        return kc::Error::OutOfMemory;
    } catch (...) {
        kcamd::setDetail("gguf: internal error");
        return kc::Error::InternalError;
    }
}

kcError_t kcGgufClose(kcGguf_t g) noexcept {
    delete g;
    return ok;
}

kcError_t kcGgufVersion(kcGguf_t g, int* version, int* alignment) noexcept {
    if (!g) return kc::Error::InvalidValue;
    if (version) *version = int(g->version);
    if (alignment) *alignment = int(g->alignment);
    return ok;
}

kcError_t kcGgufGetNum(kcGguf_t g, const char* key, double* value) noexcept {
    if (!g || !value) return kc::Error::InvalidValue;
    const Entry* e = findKey(g, key);
    if (!e || e->type == 8 || e->type == 9) return bad("gguf: no numeric key %s", key ? key : "(null)");
    *value = e->num;
    return ok;
}

kcError_t kcGgufGetStr(kcGguf_t g, const char* key, const char** str, size_t* len) noexcept {
    if (!g || !str || !len) return kc::Error::InvalidValue;
    const Entry* e = findKey(g, key);
    if (!e || e->type != 8) return bad("gguf: no string key %s", key ? key : "(null)");
    *str = e->str;
    *len = e->len;
    return ok;
}

kcError_t kcGgufGetArray(kcGguf_t g, const char* key, int64_t* count, int* elem_type) noexcept {
    if (!g) return kc::Error::InvalidValue;
    const Entry* e = findKey(g, key);
    if (!e || e->type != 9) return bad("gguf: no array key %s", key ? key : "(null)");
    if (count) *count = int64_t(e->count);
    if (elem_type) *elem_type = int(e->elem);
    return ok;
}

kcError_t kcGgufTensorCount(kcGguf_t g, int* count) noexcept {
    if (!g || !count) return kc::Error::InvalidValue;
    *count = int(g->tensors.size());
    return ok;
}

kcError_t kcGgufTensorName(kcGguf_t g, int i, const char** name) noexcept {
    if (!g || !name || i < 0 || size_t(i) >= g->tensors.size()) return kc::Error::InvalidValue;
    *name = g->tensors[size_t(i)].name.c_str();
    return ok;
}

kcError_t kcGgufTensorInfo(kcGguf_t g, const char* name, int* type, int* n_dims, int64_t ne[4], size_t* bytes,
                           const void** data) noexcept {
    if (!g || !name) return kc::Error::InvalidValue;
    auto it = g->by_name.find(name);
    if (it == g->by_name.end()) return bad("gguf: no tensor %s", name);
    const Tensor& t = g->tensors[it->second];
    if (type) *type = int(t.type);
    if (n_dims) *n_dims = t.n_dims;
    if (ne)
        for (int d = 0; d < 4; ++d) ne[d] = t.ne[d];
    if (bytes) *bytes = t.bytes;
    if (data) *data = t.data;
    return ok;
}
