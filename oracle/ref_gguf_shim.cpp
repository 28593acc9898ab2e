// C entry points over the reference's own GGUF reader (cpp/src/gguf.cpp,
// cpp/include/gguf.h), compiled where it lies under the reference tree (see
// Makefile, target ref).  Test infrastructure only: it checks the parser of
// the product (libvbhip's vb_gguf_*), which never loads this.
#include <cstdint>
#include <cstring>
#include <exception>
#include <string>
#include "gguf.h"

using vibeblade::GGUFFile;

namespace {
thread_local std::string g_err;

int put(const std::string& s, char* buf, int64_t cap) {
    if (buf && cap > 0) {
        const size_t n = s.size() < static_cast<size_t>(cap - 1) ? s.size() : static_cast<size_t>(cap - 1);
        std::memcpy(buf, s.data(), n);
        buf[n] = 0;
    }
    return static_cast<int>(s.size());
}
}  // namespace

extern "C" {

const char* ref_gguf_error(void) { return g_err.c_str(); }

// GGUFFile::GGUFFile (gguf.h:30); nullptr (message in ref_gguf_error) if it throws.
void* ref_gguf_open(const char* path) {
    try {
        return new GGUFFile(path);
    } catch (const std::exception& e) {
        g_err = e.what();
        return nullptr;
    }
}

void ref_gguf_close(void* h) { delete static_cast<GGUFFile*>(h); }

int64_t ref_gguf_n_tensors(void* h) { return static_cast<int64_t>(static_cast<GGUFFile*>(h)->tensors().size()); }

// tensors()[i] (gguf.h:20-27, :55)
int ref_gguf_tensor(void* h, int64_t i, char* name, int64_t cap, int32_t* n_dims, int64_t* dims, int32_t* type,
                    uint64_t* offset, uint64_t* size) {
    const auto& t = static_cast<GGUFFile*>(h)->tensors().at(static_cast<size_t>(i));
    put(t.name, name, cap);
    *n_dims = t.n_dims;
    for (int d = 0; d < 4; d++) dims[d] = t.dims[d];
    *type = static_cast<int32_t>(t.type);
    *offset = t.offset;
    *size = t.size;
    return 0;
}

// tensor_data (gguf.h:38): copies up to cap bytes; -1 if absent or it throws.
int64_t ref_gguf_tensor_bytes(void* h, const char* name, void* out, int64_t cap) {
    try {
        auto* f = static_cast<GGUFFile*>(h);
        const auto* ti = f->tensor_info(name);
        const void* p = f->tensor_data(name);
        if (!ti || !p) return -1;
        const size_t n = ti->size < static_cast<size_t>(cap) ? ti->size : static_cast<size_t>(cap);
        std::memcpy(out, p, n);
        return static_cast<int64_t>(ti->size);
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

// meta_* accessors (gguf.h:44-52)
int64_t ref_gguf_meta_int(void* h, const char* key, int64_t def) { return static_cast<GGUFFile*>(h)->meta_int(key, def); }
float ref_gguf_meta_float(void* h, const char* key, float def) { return static_cast<GGUFFile*>(h)->meta_float(key, def); }
int ref_gguf_meta_bool(void* h, const char* key, int def) { return static_cast<GGUFFile*>(h)->meta_bool(key, def != 0); }
int ref_gguf_meta_string(void* h, const char* key, char* buf, int64_t cap) {
    return put(static_cast<GGUFFile*>(h)->meta_string(key), buf, cap);
}
int64_t ref_gguf_meta_int_array(void* h, const char* key, int64_t* out, int64_t cap) {
    const auto v = static_cast<GGUFFile*>(h)->meta_int_array(key);
    for (size_t j = 0; j < v.size() && static_cast<int64_t>(j) < cap; j++) out[j] = v[j];
    return static_cast<int64_t>(v.size());
}
int64_t ref_gguf_meta_float_array(void* h, const char* key, float* out, int64_t cap) {
    const auto v = static_cast<GGUFFile*>(h)->meta_float_array(key);
    for (size_t j = 0; j < v.size() && static_cast<int64_t>(j) < cap; j++) out[j] = v[j];
    return static_cast<int64_t>(v.size());
}
// element j of a string array; -1 when absent
int ref_gguf_meta_string_array(void* h, const char* key, int64_t j, char* buf, int64_t cap) {
    const auto v = static_cast<GGUFFile*>(h)->meta_string_array(key);
    if (j < 0 || static_cast<size_t>(j) >= v.size()) return -1;
    return put(v[static_cast<size_t>(j)], buf, cap);
}
int64_t ref_gguf_meta_string_array_len(void* h, const char* key) {
    return static_cast<int64_t>(static_cast<GGUFFile*>(h)->meta_string_array(key).size());
}

}
