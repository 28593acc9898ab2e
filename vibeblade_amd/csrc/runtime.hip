// Runtime part of the C ABI: error text, device selection, buffers, streams.
// The op entry points live next to their kernels (dequant.hip, gemv.hip, ...).
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "vb_common.hpp"
#include "vb_internal.hpp"
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

namespace {
Knobs read_knobs() {
    Knobs k;
    if (const char* e = std::getenv("VB_GEMV_RING")) {
        const int d = std::atoi(e);
        if (d >= 1 && d <= 6) k.gemv_ring = d;  // the general kernel takes 1..4
    }
    if (const char* e = std::getenv("VB_GEMV_DMA")) k.gemv_dma = std::atoi(e) != 0;
    if (const char* e = std::getenv("VB_GEMV_CFG")) {
        int a = 0, b = 0;
        if (std::sscanf(e, "%d,%d", &a, &b) == 2 && a >= 1 && b >= 1) {
            k.gemv_cfg_wpg = a;
            k.gemv_cfg_rpg = b;
        }
    }
    if (const char* e = std::getenv("VB_GEMV_Q4K_PATH")) {
        k.gemv_q4k_mfma = std::strcmp(e, "mfma") == 0;
        k.gemv_q4k_general = std::strcmp(e, "dot") == 0;
    }
    if (const char* e = std::getenv("VB_GEMV_Q6K_PATH")) k.gemv_q6k_general = std::strcmp(e, "dot") == 0;
    if (const char* e = std::getenv("VB_GEMV_Q8_PATH")) k.gemv_q8_general = std::strcmp(e, "dot") == 0;
    if (const char* e = std::getenv("VB_GEMV_MFMA_CFG")) {
        int a = 0, b = 0;
        if (std::sscanf(e, "%d,%d", &a, &b) == 2 && a >= 1 && b >= 1) {
            k.gemv_mfma_wpg = a;
            k.gemv_mfma_ks = b;
        }
    }
    if (const char* e = std::getenv("VB_GEMM_NF")) {
        const int v = std::atoi(e);
        if (v == 6 || v == 8) k.gemm_nf = v;
    }
    if (const char* e = std::getenv("VB_GEMM_TILE")) {
        int a = 0, b = 0, c = 0, d = 1;
        const int got = std::sscanf(e, "%d,%d,%d,%d", &a, &b, &c, &d);
        if ((got == 3 || got == 4) && (a == 1 || a == 2 || a == 4) && (b == 2 || b == 4) &&
            (c == 4 || c == 6 || c == 8) && c % b == 0 && (d == 1 || d == 2)) {
            k.gemm_tile_wm = a;
            k.gemm_tile_wn = b;
            k.gemm_tile_nf = c;
            k.gemm_tile_ks = d;
        }
    }
    if (const char* e = std::getenv("VB_GEMV_SPLIT")) {
        int a = 0, b = 0;
        if (std::sscanf(e, "%d,%d", &a, &b) == 2 && (a == 2 || a == 4 || a == 8) && b >= 1 && b <= 4) {
            k.gemv_split_sl = a;
            k.gemv_split_d = b;
        }
    }
    if (const char* e = std::getenv("VB_GEMM_SPLIT_MIN_M")) {
        const int v = std::atoi(e);
        if (v >= 0) k.gemm_split_min_m = v;
    }
    if (const char* e = std::getenv("VB_GEMM_ZSPLIT")) {
        const int v = std::atoi(e);
        if (v >= 1 && v <= 8) k.gemm_zsplit = v;
    }
    if (const char* e = std::getenv("VB_GEMM_XR_KQ")) k.gemm_xr_kq = std::atoi(e) != 0;
    if (const char* e = std::getenv("VB_SPARSE_FUSED")) k.sparse_fused = e[0] != '0';
    if (const char* e = std::getenv("VB_SPARSE_NPW")) k.sparse_npw = e[0] == '2' ? 2 : (e[0] == '1' ? 1 : 0);
    return k;
}

constexpr int kMaxDevices = 64;
std::atomic<int> g_num_cus[kMaxDevices];
}  // namespace

// The current overrides: an immutable snapshot behind an atomic pointer,
// replaced (never freed: a few bytes per reload) by vb_tuning_reload.
std::atomic<const Knobs*> g_knobs{nullptr};

const Knobs& knobs() {
    const Knobs* k = g_knobs.load(std::memory_order_acquire);
    if (!k) {
        const Knobs* fresh = new Knobs(read_knobs());
        if (g_knobs.compare_exchange_strong(k, fresh, std::memory_order_acq_rel)) {
            k = fresh;
        } else {
            delete fresh;  // another thread published first; k holds its snapshot
        }
    }
    return *k;
}

int num_cus() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    int n = g_num_cus[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    g_num_cus[dev].store(n, std::memory_order_relaxed);
    return n;
}

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
    (void)knobs();
    (void)num_cus();
    void* scratch_dev = nullptr;  // the allocation-free entry point's scratch on this device
    return sparse_scratch_ptr(&scratch_dev);
}

int vb_tuning_reload(void) {
    g_knobs.store(new Knobs(read_knobs()), std::memory_order_release);
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
