// TEST INFRASTRUCTURE (oracle): a C binding of the reference's own GGUF
// reader class (include/aero/gguf.hpp:75-137, src/gguf.cpp:150-379), built
// with the reference's src/gguf.cpp and src/kernels.cpp where they lie into
// oracle/_ref/libref_gguf.so by `make -C oracle ref`. The class has no C ABI;
// these functions call its public members one for one so tests can compare
// the library's parser with the reference's on the same files.
#include "aero/gguf.hpp"

#include <cstring>
#include <exception>

using aero::GgufReader;
using aero::TensorInfo;

extern "C" {

// NULL when the reference's constructor throws (its refusal).
void* rg_open(const char* path, char* err, int err_cap) {
    try {
        return new GgufReader(path);
    } catch (const std::exception& e) {
        if (err && err_cap > 0) {
            std::strncpy(err, e.what(), (size_t)err_cap - 1);
            err[err_cap - 1] = '\0';
        }
        return nullptr;
    }
}

void rg_close(void* h) { delete static_cast<GgufReader*>(h); }

const char* rg_arch(void* h) { return static_cast<GgufReader*>(h)->arch().c_str(); }

int64_t rg_file_size(void* h) { return static_cast<GgufReader*>(h)->file_size(); }

int rg_has(void* h, const char* key) { return static_cast<GgufReader*>(h)->has(key) ? 1 : 0; }

int64_t rg_get_int(void* h, const char* key, int64_t def) {
    return static_cast<GgufReader*>(h)->get_int(key, def);
}

double rg_get_float(void* h, const char* key, double def) {
    return static_cast<GgufReader*>(h)->get_float(key, def);
}

// Copies the string value (or def) into buf; returns its length.
int64_t rg_get_str(void* h, const char* key, char* buf, int64_t cap) {
    const std::string s = static_cast<GgufReader*>(h)->get_str(key, "");
    if (buf && cap > 0) {
        const size_t n = std::min((size_t)cap, s.size());
        std::memcpy(buf, s.data(), n);
    }
    return (int64_t)s.size();
}

int64_t rg_int_array(void* h, const char* key, int64_t* out, int64_t cap) {
    const std::vector<int64_t> v = static_cast<GgufReader*>(h)->get_int_array(key);
    for (size_t i = 0; i < v.size() && (int64_t)i < cap; ++i) out[i] = v[i];
    return (int64_t)v.size();
}

int64_t rg_str_array_len(void* h, const char* key) {
    return (int64_t)static_cast<GgufReader*>(h)->get_str_array(key).size();
}

int64_t rg_str_array_item(void* h, const char* key, int64_t i, char* buf, int64_t cap) {
    const std::vector<std::string> v = static_cast<GgufReader*>(h)->get_str_array(key);
    if (i < 0 || i >= (int64_t)v.size()) return -1;
    const std::string& s = v[(size_t)i];
    if (buf && cap > 0) std::memcpy(buf, s.data(), std::min((size_t)cap, s.size()));
    return (int64_t)s.size();
}

int64_t rg_n_tensors(void* h) { return (int64_t)static_cast<GgufReader*>(h)->tensors().size(); }

// type, n_dims, dims (GGUF order), offset, bytes; 0 when absent.
int rg_tensor(void* h, const char* name, int* type, int* n_dims, int64_t* dims, int64_t* offset,
              int64_t* nbytes) {
    const GgufReader* r = static_cast<GgufReader*>(h);
    const TensorInfo* t = r->find(name);
    if (t == nullptr) return 0;
    *type = (int)t->type;
    *n_dims = (int)t->dims.size();
    for (size_t d = 0; d < 4; ++d) dims[d] = d < t->dims.size() ? t->dims[d] : 0;
    *offset = t->offset;
    *nbytes = r->tensor_bytes(*t);
    return 1;
}

const void* rg_tensor_data(void* h, const char* name) {
    const GgufReader* r = static_cast<GgufReader*>(h);
    const TensorInfo* t = r->find(name);
    return t ? r->tensor_data(*t) : nullptr;
}

}  // extern "C"
