// GGUF reader on the host and the file -> HBM upload of its tensors.
//
// The file is mapped read-only (the page cache is the loader; only the pages
// a caller touches become resident) and its header, metadata and tensor
// index are parsed with a bounds-checked little-endian cursor (format:
// src/gguf.cpp:150-354 and engine/gguf.py:166-233 of the reference):
//
//   "GGUF" | u32 version (2, 3) | u64 n_tensors | u64 n_kv
//   n_kv x (string key, u32 value type, value)
//   n_tensors x (string name, u32 n_dims, u64 dims[n_dims], u32 ggml type,
//                u64 offset relative to the data section)
//   padding to general.alignment (default 32), then the tensor data.
//
// A string is a u64 length and its bytes; an array is a u32 element type, a
// u64 count and the elements. Scalars take their natural width (u16/i16 two
// bytes, as the format and the reference's Python reader read them).
//
// Uploads read the file with pread from four threads, each into two pinned
// host buffers in turn, and queue each buffer's copy to HBM while the next
// read runs; the call returns once the bytes are in HBM.
#include "aero_hip.h"
#include "common.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <atomic>
#include <cerrno>
#include <cmath>
#include <cstring>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <unordered_map>
#include <utility>
#include <vector>

namespace aero {
namespace {

// GGUF metadata value types
enum : uint32_t {
    GV_U8 = 0, GV_I8, GV_U16, GV_I16, GV_U32, GV_I32, GV_F32, GV_BOOL, GV_STRING,
    GV_ARRAY, GV_U64, GV_I64, GV_F64,
};

// ggml tensor types: (bytes, values) per block; 0 for a type this table does
// not know (its bytes cannot be located, so it cannot be read).
void ggml_block(uint32_t t, int64_t& bytes, int64_t& values) {
    bytes = 0;
    values = 0;
    switch (t) {
    case 0: bytes = 4; values = 1; break;      // F32
    case 1: bytes = 2; values = 1; break;      // F16
    case 30: bytes = 2; values = 1; break;     // BF16
    case 2: bytes = 18; values = 32; break;    // Q4_0
    case 3: bytes = 20; values = 32; break;    // Q4_1
    case 6: bytes = 22; values = 32; break;    // Q5_0
    case 7: bytes = 24; values = 32; break;    // Q5_1
    case 8: bytes = 34; values = 32; break;    // Q8_0
    case 10: bytes = 84; values = 256; break;  // Q2_K
    case 11: bytes = 110; values = 256; break; // Q3_K
    case 12: bytes = 144; values = 256; break; // Q4_K
    case 13: bytes = 176; values = 256; break; // Q5_K
    case 14: bytes = 210; values = 256; break; // Q6_K
    case 23: bytes = 136; values = 256; break; // IQ4_XS
    default: break;
    }
}

struct Cursor {
    const uint8_t* p;
    const uint8_t* end;
    void need(uint64_t n) const {
        if (n > (uint64_t)(end - p)) throw std::runtime_error("truncated file");
    }
    template <typename T>
    T get() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        need(n);
        std::string s(reinterpret_cast<const char*>(p), (size_t)n);
        p += n;
        return s;
    }
};

// One metadata value. Scalars keep their GGUF type; arrays keep their
// elements (nested arrays are values too).
struct Value {
    uint32_t type = GV_U8;
    uint64_t u = 0;     // unsigned scalars and bool
    int64_t i = 0;      // signed scalars
    double f = 0.0;     // floats
    std::string s;
    uint32_t elem = 0;  // array element type
    std::vector<Value> arr;
};

// Fewest bytes a value of this type takes in the file (0: unknown type).
uint64_t value_min_bytes(uint32_t type) {
    switch (type) {
    case GV_U8: case GV_I8: case GV_BOOL: return 1;
    case GV_U16: case GV_I16: return 2;
    case GV_U32: case GV_I32: case GV_F32: return 4;
    case GV_U64: case GV_I64: case GV_F64: case GV_STRING: return 8;
    case GV_ARRAY: return 12;
    default: return 0;
    }
}

void read_value(Cursor& c, uint32_t type, Value& v, int depth) {
    v.type = type;
    switch (type) {
    case GV_U8: v.u = c.get<uint8_t>(); break;
    case GV_I8: v.i = c.get<int8_t>(); break;
    case GV_U16: v.u = c.get<uint16_t>(); break;
    case GV_I16: v.i = c.get<int16_t>(); break;
    case GV_U32: v.u = c.get<uint32_t>(); break;
    case GV_I32: v.i = c.get<int32_t>(); break;
    case GV_F32: v.f = c.get<float>(); break;
    case GV_BOOL: v.u = c.get<uint8_t>() != 0; break;
    case GV_STRING: v.s = c.str(); break;
    case GV_U64: v.u = c.get<uint64_t>(); break;
    case GV_I64: v.i = c.get<int64_t>(); break;
    case GV_F64: v.f = c.get<double>(); break;
    case GV_ARRAY: {
        if (depth > 8) throw std::runtime_error("arrays nested too deeply");
        v.elem = c.get<uint32_t>();
        const uint64_t n = c.get<uint64_t>();
        // a count whose smallest encoding runs past the file's end is corrupt,
        // not a large array
        const uint64_t min_bytes = value_min_bytes(v.elem);
        if (min_bytes == 0) throw std::runtime_error("unknown array element type");
        if (n > (uint64_t)(c.end - c.p) / min_bytes) throw std::runtime_error("truncated file");
        v.arr.resize((size_t)n);
        for (uint64_t k = 0; k < n; ++k) read_value(c, v.elem, v.arr[(size_t)k], depth + 1);
        break;
    }
    default: throw std::runtime_error("unknown metadata value type " + std::to_string(type));
    }
}

bool value_int(const Value& v, int64_t& out) {
    switch (v.type) {
    case GV_U8: case GV_U16: case GV_U32: case GV_U64: case GV_BOOL:
        out = (int64_t)v.u;
        return true;
    case GV_I8: case GV_I16: case GV_I32: case GV_I64:
        out = v.i;
        return true;
    default: return false;
    }
}

bool value_float(const Value& v, double& out) {
    int64_t i;
    if (v.type == GV_F32 || v.type == GV_F64) {
        out = v.f;
        return true;
    }
    if (v.type == GV_BOOL) return false;
    if (value_int(v, i)) {
        out = v.type == GV_U64 ? (double)v.u : (double)i;
        return true;
    }
    return false;
}

struct Tensor {
    std::string name;
    std::vector<int64_t> dims;  // GGUF order: fastest-varying first
    uint32_t type = 0;
    int64_t offset = 0;         // relative to the data section
    int64_t n_elements = 0;
    int64_t nbytes = -1;        // -1: a type without a known block size
};

// Pinned staging for uploads, made on first use on the device current then:
// kWorkers reader threads, each with two chunk buffers so a buffer's copy to
// HBM overlaps the next read into the other.
struct Staging {
    static constexpr size_t kChunk = 8u << 20;
    static constexpr int kWorkers = 4;
    struct Slot {
        void* buf = nullptr;
        hipEvent_t done = nullptr;
        bool used = false;
    };
    Slot slot[kWorkers][2];
    int device = -1;

    bool ensure() {
        int dev = 0;
        if (!hip_ok(hipGetDevice(&dev), "hipGetDevice")) return false;
        if (slot[0][0].buf != nullptr && dev == device) return true;
        release();
        for (auto& w : slot)
            for (auto& sl : w)
                if (!hip_ok(hipHostMalloc(&sl.buf, kChunk, hipHostMallocDefault), "hipHostMalloc") ||
                    !hip_ok(hipEventCreateWithFlags(&sl.done, hipEventDisableTiming),
                            "hipEventCreate")) {
                    release();
                    return false;
                }
        device = dev;
        return true;
    }
    // wait for every copy still reading from the buffers
    bool drain() {
        bool ok = true;
        for (auto& w : slot)
            for (auto& sl : w) {
                if (sl.used && !hip_ok(hipEventSynchronize(sl.done), "hipEventSynchronize"))
                    ok = false;
                sl.used = false;
            }
        return ok;
    }
    void release() {
        for (auto& w : slot)
            for (auto& sl : w) {
                if (sl.used && sl.done) (void)hipEventSynchronize(sl.done);
                if (sl.done) (void)hipEventDestroy(sl.done);
                if (sl.buf) (void)hipHostFree(sl.buf);
                sl = Slot{};
            }
        device = -1;
    }
};

class GgufFile {
public:
    explicit GgufFile(const std::string& path) : path_(path) {
        try {
            fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
            if (fd_ < 0)
                throw std::runtime_error("cannot open " + path + ": " + std::strerror(errno));
            struct stat st {};
            if (::fstat(fd_, &st) != 0) throw std::runtime_error("fstat failed");
            size_ = (int64_t)st.st_size;
            if (size_ < 24) throw std::runtime_error("file too short for a GGUF header");
            void* m = ::mmap(nullptr, (size_t)size_, PROT_READ, MAP_PRIVATE, fd_, 0);
            if (m == MAP_FAILED) throw std::runtime_error("mmap failed");
            base_ = static_cast<const uint8_t*>(m);
            parse();
        } catch (...) {
            unmap();
            throw;
        }
    }
    ~GgufFile() {
        staging_.release();
        unmap();
    }
    GgufFile(const GgufFile&) = delete;
    GgufFile& operator=(const GgufFile&) = delete;

    // metadata in file order, and the lookup map of the reference's C++
    // reader: every key, and also the part after its first dot unless it is
    // a "tokenizer…" or "general." key; the first entry for a name wins
    std::vector<std::pair<std::string, Value>> kv;
    std::unordered_map<std::string, size_t> lookup;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> tensor_index;
    std::string arch;
    uint32_t version = 0;
    int64_t alignment = 32;
    int64_t data_offset = 0;
    std::string json;  // metadata as JSON, made on first request
    Staging staging_;

    int64_t size() const { return size_; }
    const uint8_t* base() const { return base_; }
    int fd() const { return fd_; }

    const Value* find(const char* key) const {
        auto it = lookup.find(key);
        return it == lookup.end() ? nullptr : &kv[it->second].second;
    }
    const Tensor* tensor(const char* name) const {
        auto it = tensor_index.find(name);
        return it == tensor_index.end() ? nullptr : &tensors[it->second];
    }

private:
    void unmap() {
        if (base_) ::munmap(const_cast<uint8_t*>(base_), (size_t)size_);
        if (fd_ >= 0) ::close(fd_);
        base_ = nullptr;
        fd_ = -1;
    }

    void parse() {
        Cursor c{base_, base_ + size_};
        if (std::memcmp(base_, "GGUF", 4) != 0) throw std::runtime_error("bad magic");
        c.p += 4;
        version = c.get<uint32_t>();
        if (version < 2 || version > 3)
            throw std::runtime_error("unsupported GGUF version " + std::to_string(version));
        const uint64_t n_tensors = c.get<uint64_t>();
        const uint64_t n_kv = c.get<uint64_t>();
        for (uint64_t k = 0; k < n_kv; ++k) {
            std::string key = c.str();
            const uint32_t type = c.get<uint32_t>();
            Value v;
            read_value(c, type, v, 0);
            const size_t at = kv.size();
            const size_t dot = key.find('.');
            if (dot != std::string::npos && key.compare(0, 9, "tokenizer") != 0 &&
                key.compare(0, 8, "general.") != 0)
                lookup.emplace(key.substr(dot + 1), at);
            lookup.emplace(key, at);
            if (key == "general.architecture" && v.type == GV_STRING) arch = v.s;
            kv.emplace_back(std::move(key), std::move(v));
        }
        if (const Value* a = find("general.alignment")) {
            int64_t al = 0;
            if (!value_int(*a, al) || al <= 0 || (al & (al - 1)) != 0)
                throw std::runtime_error("bad general.alignment (must be a power of two)");
            alignment = al;
        }
        int64_t max_end = 0;
        for (uint64_t k = 0; k < n_tensors; ++k) {
            Tensor t;
            t.name = c.str();
            const uint32_t nd = c.get<uint32_t>();
            if (nd > 4) throw std::runtime_error("tensor " + t.name + ": bad n_dims");
            t.dims.resize(nd);
            int64_t n = 1;
            for (uint32_t d = 0; d < nd; ++d) {
                const uint64_t dim = c.get<uint64_t>();
                if (dim > ((uint64_t)1 << 40)) throw std::runtime_error("tensor " + t.name + ": bad dim");
                t.dims[d] = (int64_t)dim;
                // bound the product before forming it: n <= 2^48 and dim <= 2^40
                // could overflow int64 (and wrap to a small count) otherwise
                constexpr int64_t kMaxElements = (int64_t)1 << 48;
                if (dim != 0 && n > kMaxElements / (int64_t)dim)
                    throw std::runtime_error("tensor " + t.name + ": too large");
                n *= (int64_t)dim;
            }
            t.n_elements = n;
            t.type = c.get<uint32_t>();
            const uint64_t off = c.get<uint64_t>();
            if (off > (uint64_t)size_) throw std::runtime_error("tensor " + t.name + ": offset past end");
            t.offset = (int64_t)off;
            int64_t bb, bv;
            ggml_block(t.type, bb, bv);
            if (bv > 0) {
                if (n % bv != 0)
                    throw std::runtime_error("tensor " + t.name +
                                             ": element count is not a whole number of blocks");
                t.nbytes = (n / bv) * bb;
                max_end = std::max(max_end, t.offset + t.nbytes);
            }
            tensor_index.emplace(t.name, tensors.size());
            tensors.push_back(std::move(t));
        }
        const int64_t here = (int64_t)(c.p - base_);
        data_offset = (here + alignment - 1) / alignment * alignment;
        if (data_offset + max_end > size_)
            throw std::runtime_error("tensor data runs past the end of the file");
    }

    std::string path_;
    int fd_ = -1;
    const uint8_t* base_ = nullptr;
    int64_t size_ = 0;
};

// ----------------------------------------------------------- JSON export
void json_str(std::string& o, const std::string& s) {
    // bytes >= 0x80 as \u00XX (one code point per byte): the reader turns
    // them back into bytes and decodes them as UTF-8 itself
    static const char* hex = "0123456789abcdef";
    o += '"';
    for (unsigned char ch : s) {
        if (ch == '"' || ch == '\\') {
            o += '\\';
            o += (char)ch;
        } else if (ch < 0x20 || ch >= 0x80) {
            o += "\\u00";
            o += hex[ch >> 4];
            o += hex[ch & 15];
        } else {
            o += (char)ch;
        }
    }
    o += '"';
}

void json_value(std::string& o, const Value& v) {
    char b[40];
    switch (v.type) {
    case GV_U8: case GV_U16: case GV_U32: case GV_U64:
        std::snprintf(b, sizeof b, "%llu", (unsigned long long)v.u);
        o += b;
        break;
    case GV_I8: case GV_I16: case GV_I32: case GV_I64:
        std::snprintf(b, sizeof b, "%lld", (long long)v.i);
        o += b;
        break;
    case GV_BOOL: o += v.u ? "true" : "false"; break;
    case GV_F32: case GV_F64:
        if (std::isnan(v.f)) o += "NaN";
        else if (std::isinf(v.f)) o += v.f > 0 ? "Infinity" : "-Infinity";
        else {
            std::snprintf(b, sizeof b, "%.17g", v.f);
            o += b;
        }
        break;
    case GV_STRING: json_str(o, v.s); break;
    case GV_ARRAY:
        o += '[';
        for (size_t k = 0; k < v.arr.size(); ++k) {
            if (k) o += ',';
            json_value(o, v.arr[k]);
        }
        o += ']';
        break;
    default: o += "null"; break;
    }
}

GgufFile* handle(void* h) {
    if (h == nullptr) set_error("gguf: null handle");
    return static_cast<GgufFile*>(h);
}

const Tensor* need_tensor(GgufFile* f, const char* name) {
    if (f == nullptr) return nullptr;
    const Tensor* t = name ? f->tensor(name) : nullptr;
    if (t == nullptr) set_error("gguf: no tensor named %s", name ? name : "(null)");
    return t;
}

// bytes [byte0, byte0 + n) of a tensor with a known size
bool tensor_range(const Tensor* t, int64_t byte0, int64_t n) {
    if (t->nbytes < 0) {
        set_error("gguf: tensor %s has ggml type %u, whose block size is not known",
                  t->name.c_str(), t->type);
        return false;
    }
    if (byte0 < 0 || n < 0 || byte0 > t->nbytes || n > t->nbytes - byte0) {
        set_error("gguf: bytes [%lld, +%lld) outside tensor %s (%lld bytes)", (long long)byte0,
                  (long long)n, t->name.c_str(), (long long)t->nbytes);
        return false;
    }
    return true;
}

bool pread_all(int fd, void* dst, size_t n, int64_t off) {
    uint8_t* d = static_cast<uint8_t*>(dst);
    while (n > 0) {
        const ssize_t r = ::pread(fd, d, n, (off_t)off);
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) {
            set_error("gguf: read failed at offset %lld: %s", (long long)off,
                      r < 0 ? std::strerror(errno) : "end of file");
            return false;
        }
        d += r;
        n -= (size_t)r;
        off += r;
    }
    return true;
}

}  // namespace
}  // namespace aero

using aero::GgufFile;
using aero::Tensor;
using aero::Value;

extern "C" {

void* aero_gguf_open(const char* path) {
    aero::clear_error();
    if (path == nullptr) {
        aero::set_error("gguf: null path");
        return nullptr;
    }
    try {
        return new GgufFile(path);
    } catch (const std::exception& e) {
        aero::set_error("gguf: %s: %s", path, e.what());
        return nullptr;
    } catch (...) {
        aero::set_error("gguf: %s: parse failed", path);
        return nullptr;
    }
}

void aero_gguf_close(void* h) { delete static_cast<GgufFile*>(h); }

int64_t aero_gguf_file_size(void* h) {
    GgufFile* f = aero::handle(h);
    return f ? f->size() : -1;
}

int aero_gguf_version(void* h) {
    GgufFile* f = aero::handle(h);
    return f ? (int)f->version : -1;
}

int64_t aero_gguf_alignment(void* h) {
    GgufFile* f = aero::handle(h);
    return f ? f->alignment : -1;
}

int64_t aero_gguf_data_offset(void* h) {
    GgufFile* f = aero::handle(h);
    return f ? f->data_offset : -1;
}

const char* aero_gguf_arch(void* h) {
    GgufFile* f = aero::handle(h);
    return f ? f->arch.c_str() : nullptr;
}

int64_t aero_gguf_n_kv(void* h) {
    GgufFile* f = aero::handle(h);
    return f ? (int64_t)f->kv.size() : -1;
}

const char* aero_gguf_kv_key(void* h, int64_t i) {
    GgufFile* f = aero::handle(h);
    if (f == nullptr || i < 0 || i >= (int64_t)f->kv.size()) return nullptr;
    return f->kv[(size_t)i].first.c_str();
}

int aero_gguf_kv_type(void* h, const char* key) {
    GgufFile* f = aero::handle(h);
    const Value* v = (f && key) ? f->find(key) : nullptr;
    return v ? (int)v->type : -1;
}

int aero_gguf_get_int(void* h, const char* key, int64_t* out) {
    GgufFile* f = aero::handle(h);
    const Value* v = (f && key) ? f->find(key) : nullptr;
    int64_t x;
    if (v == nullptr || out == nullptr || !aero::value_int(*v, x)) return 0;
    *out = x;
    return 1;
}

int aero_gguf_get_float(void* h, const char* key, double* out) {
    GgufFile* f = aero::handle(h);
    const Value* v = (f && key) ? f->find(key) : nullptr;
    double x;
    if (v == nullptr || out == nullptr || !aero::value_float(*v, x)) return 0;
    *out = x;
    return 1;
}

const char* aero_gguf_get_str(void* h, const char* key, int64_t* len) {
    GgufFile* f = aero::handle(h);
    const Value* v = (f && key) ? f->find(key) : nullptr;
    if (v == nullptr || v->type != aero::GV_STRING) return nullptr;
    if (len) *len = (int64_t)v->s.size();
    return v->s.c_str();
}

int64_t aero_gguf_array_len(void* h, const char* key) {
    GgufFile* f = aero::handle(h);
    const Value* v = (f && key) ? f->find(key) : nullptr;
    return (v && v->type == aero::GV_ARRAY) ? (int64_t)v->arr.size() : -1;
}

int64_t aero_gguf_array_ints(void* h, const char* key, int64_t* out, int64_t n) {
    GgufFile* f = aero::handle(h);
    const Value* v = (f && key) ? f->find(key) : nullptr;
    if (v == nullptr || v->type != aero::GV_ARRAY || (n > 0 && out == nullptr)) return -1;
    int64_t k = 0;
    for (; k < (int64_t)v->arr.size() && k < n; ++k)
        if (!aero::value_int(v->arr[(size_t)k], out[k])) return -1;
    return k;
}

int64_t aero_gguf_array_floats(void* h, const char* key, double* out, int64_t n) {
    GgufFile* f = aero::handle(h);
    const Value* v = (f && key) ? f->find(key) : nullptr;
    if (v == nullptr || v->type != aero::GV_ARRAY || (n > 0 && out == nullptr)) return -1;
    int64_t k = 0;
    for (; k < (int64_t)v->arr.size() && k < n; ++k)
        if (!aero::value_float(v->arr[(size_t)k], out[k])) return -1;
    return k;
}

const char* aero_gguf_array_str(void* h, const char* key, int64_t i, int64_t* len) {
    GgufFile* f = aero::handle(h);
    const Value* v = (f && key) ? f->find(key) : nullptr;
    if (v == nullptr || v->type != aero::GV_ARRAY || i < 0 || i >= (int64_t)v->arr.size() ||
        v->arr[(size_t)i].type != aero::GV_STRING)
        return nullptr;
    if (len) *len = (int64_t)v->arr[(size_t)i].s.size();
    return v->arr[(size_t)i].s.c_str();
}

const char* aero_gguf_kv_json(void* h, int64_t* len) {
    GgufFile* f = aero::handle(h);
    if (f == nullptr) return nullptr;
    if (f->json.empty()) {
        std::string o = "[";
        for (size_t k = 0; k < f->kv.size(); ++k) {
            if (k) o += ',';
            o += '[';
            aero::json_str(o, f->kv[k].first);
            o += ',';
            char b[16];
            std::snprintf(b, sizeof b, "%u", f->kv[k].second.type);
            o += b;
            o += ',';
            aero::json_value(o, f->kv[k].second);
            o += ']';
        }
        o += ']';
        f->json = std::move(o);
    }
    if (len) *len = (int64_t)f->json.size();
    return f->json.c_str();
}

int64_t aero_gguf_n_tensors(void* h) {
    GgufFile* f = aero::handle(h);
    return f ? (int64_t)f->tensors.size() : -1;
}

const char* aero_gguf_tensor_name(void* h, int64_t i) {
    GgufFile* f = aero::handle(h);
    if (f == nullptr || i < 0 || i >= (int64_t)f->tensors.size()) return nullptr;
    return f->tensors[(size_t)i].name.c_str();
}

int64_t aero_gguf_tensor_info(void* h, const char* name, int* type, int* n_dims, int64_t* dims,
                              int64_t* offset, int64_t* nbytes) {
    aero::clear_error();
    GgufFile* f = aero::handle(h);
    const Tensor* t = aero::need_tensor(f, name);
    if (t == nullptr) return -1;
    if (type) *type = (int)t->type;
    if (n_dims) *n_dims = (int)t->dims.size();
    if (dims)
        for (size_t d = 0; d < 4; ++d) dims[d] = d < t->dims.size() ? t->dims[d] : 0;
    if (offset) *offset = t->offset;
    if (nbytes) *nbytes = t->nbytes;
    return (int64_t)f->tensor_index.at(t->name);
}

const void* aero_gguf_tensor_data(void* h, const char* name) {
    aero::clear_error();
    GgufFile* f = aero::handle(h);
    const Tensor* t = aero::need_tensor(f, name);
    if (t == nullptr || !aero::tensor_range(t, 0, 0)) return nullptr;
    return f->base() + f->data_offset + t->offset;
}

int aero_gguf_read(void* h, const char* name, int64_t byte0, int64_t nbytes, void* dst) {
    aero::clear_error();
    GgufFile* f = aero::handle(h);
    const Tensor* t = aero::need_tensor(f, name);
    if (t == nullptr || !aero::tensor_range(t, byte0, nbytes)) return 0;
    if (nbytes > 0 && dst == nullptr) {
        aero::set_error("gguf: null destination");
        return 0;
    }
    std::memcpy(dst, f->base() + f->data_offset + t->offset + byte0, (size_t)nbytes);
    return 1;
}

int aero_gguf_upload(void* h, const char* name, int64_t byte0, int64_t nbytes, void* dst_dev,
                     void* stream) {
    aero::clear_error();
    GgufFile* f = aero::handle(h);
    const Tensor* t = aero::need_tensor(f, name);
    if (t == nullptr || !aero::tensor_range(t, byte0, nbytes)) return 0;
    if (nbytes == 0) return 1;
    if (dst_dev == nullptr) {
        aero::set_error("gguf: null device destination");
        return 0;
    }
    using aero::Staging;
    Staging& st = f->staging_;
    if (!st.ensure()) return 0;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t file0 = f->data_offset + t->offset + byte0;
    uint8_t* dst = static_cast<uint8_t*>(dst_dev);
    const int64_t chunks = (nbytes + (int64_t)Staging::kChunk - 1) / (int64_t)Staging::kChunk;
    const int nw = (int)std::min<int64_t>(Staging::kWorkers, chunks);
    std::atomic<int64_t> next{0};
    std::atomic<bool> ok{true};
    std::mutex err_mu;
    std::string err;
    // worker w takes the next chunk index until none is left: read it into
    // one of its two buffers (after that buffer's previous copy has left),
    // queue the copy to HBM, record when the copy is done
    auto work = [&](int w) {
        const bool own_thread = nw > 1;
        if (own_thread && !aero::hip_ok(hipSetDevice(st.device), "hipSetDevice")) ok = false;
        int k = 0;
        while (ok) {
            const int64_t i = next.fetch_add(1);
            if (i >= chunks) break;
            Staging::Slot& sl = st.slot[w][k];
            const int64_t off = i * (int64_t)Staging::kChunk;
            const size_t n = (size_t)std::min<int64_t>(Staging::kChunk, nbytes - off);
            bool good = !sl.used || aero::hip_ok(hipEventSynchronize(sl.done), "hipEventSynchronize");
            sl.used = false;
            good = good && aero::pread_all(f->fd(), sl.buf, n, file0 + off) &&
                   aero::hip_ok(hipMemcpyAsync(dst + off, sl.buf, n, hipMemcpyHostToDevice, s),
                                "hipMemcpyAsync") &&
                   aero::hip_ok(hipEventRecord(sl.done, s), "hipEventRecord");
            if (!good) {
                ok = false;
                break;
            }
            sl.used = true;
            k ^= 1;
        }
        if (!ok && own_thread) {
            // errors are per thread: hand this one to the caller's
            std::lock_guard<std::mutex> g(err_mu);
            if (err.empty()) err = aero_hip_last_error();
        }
    };
    if (nw == 1) {
        work(0);
    } else {
        std::vector<std::thread> threads;
        threads.reserve((size_t)nw);
        for (int w = 0; w < nw; ++w) threads.emplace_back(work, w);
        for (auto& th : threads) th.join();
    }
    const bool drained = st.drain();
    if (!ok) {
        if (!err.empty()) aero::set_error("%s", err.c_str());
        return 0;
    }
    return drained ? 1 : 0;
}

}  // extern "C"
