// C entry points over the reference's own dequant.cpp / fp16_compat.cpp,
// compiled where they lie under the reference tree (see Makefile, target ref).
// Test and CPU-baseline infrastructure only: the product never loads this.
#include <cstdint>
#include <exception>
#include "dequant.h"
#include "fp16_compat.h"

extern "C" {

// vibeblade::dequantize_row (cpp/include/dequant.h:11); returns -1 if it throws.
int ref_dequantize_row(const void* row, float* out, int64_t n, int32_t type) {
    try {
        vibeblade::dequantize_row(row, out, n, (vibeblade::ggml_type)type);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// vibeblade::gemv_dequant (cpp/include/dequant.h:27-35).
int ref_gemv_dequant(const float* x, const void* w, float* out, int64_t K, int64_t N,
                     int32_t type, float* scratch) {
    try {
        vibeblade::gemv_dequant(x, w, out, K, N, (vibeblade::ggml_type)type, scratch);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// vibeblade::f16_to_f32 (cpp/src/fp16_compat.cpp:13-35).
float ref_f16_to_f32(uint16_t h) { return vibeblade::f16_to_f32(h); }

}
