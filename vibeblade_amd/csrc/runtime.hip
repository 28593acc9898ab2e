// Runtime part of the C ABI: error text, device selection, buffers, streams.
// The op entry points live next to their kernels (dequant.hip, gemv.hip, ...).
#include <cstdarg>
#include <cstring>

#include "vb_common.hpp"
#include "../../include/vbhip.h"

namespace vb {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error.assign(buf);
}

const char* last_error() { return g_last_error.c_str(); }

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
        return E_HIP;
    }
    return OK;
}

}  // namespace vb

using namespace vb;

#define VB_HIP(call)                                                          \
    do {                                                                      \
        const hipError_t e_ = (call);                                         \
        if (e_ != hipSuccess) {                                               \
            set_error("%s: %s", #call, hipGetErrorString(e_));                \
            return E_HIP;                                                     \
        }                                                                     \
    } while (0)

extern "C" {

const char* vb_last_error(void) { return last_error(); }

int vb_version(void) { return VB_ABI_VERSION; }

int64_t vb_row_bytes(int32_t ggml_type, int64_t k) { return row_bytes(ggml_type, k); }

int vb_init(int device) {
    int n = 0;
    VB_HIP(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) {
        set_error("vb_init: device %d out of range (%d devices)", device, n);
        return E_INVAL;
    }
    VB_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    VB_HIP(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_error("vb_init: device %d is %s; this library is built for gfx950", device,
                  prop.gcnArchName);
        return E_UNSUPPORTED;
    }
    return OK;
}

int vb_malloc(void** ptr, size_t bytes) {
    if (!ptr) { set_error("vb_malloc: null out pointer"); return E_INVAL; }
    VB_HIP(hipMalloc(ptr, bytes));
    return OK;
}

int vb_free(void* ptr) {
    VB_HIP(hipFree(ptr));
    return OK;
}

int vb_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    VB_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)));
    return OK;
}

int vb_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    VB_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)));
    return OK;
}

int vb_stream_create(void** stream) {
    if (!stream) { set_error("vb_stream_create: null out pointer"); return E_INVAL; }
    hipStream_t s;
    VB_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
    return OK;
}

int vb_stream_sync(void* stream) {
    VB_HIP(hipStreamSynchronize(as_stream(stream)));
    return OK;
}

int vb_stream_destroy(void* stream) {
    VB_HIP(hipStreamDestroy(as_stream(stream)));
    return OK;
}

}  // extern "C"
