// Read-only stream of GGUF rows with the launch shape and the load pattern
// of the short-row Q4_K GEMV (gemv_q4k.hip): how fast one launch can read
// the bytes that GEMV reads, with nothing computed from them.  A
// measurement utility with no counterpart in the reference; the bench's
// floor table times it beside the GEMV.
//
// Shape: one 8-wave workgroup per CU slot, rows per wave as the GEMV takes
// them (n / (CUs x 8), rounded up), each row read as contiguous 16-byte
// non-temporal pieces (lane L: slots L, 64 + L, ... of the row; lanes past
// the row's end re-read an in-row slot), `ring` rows loaded ahead of the
// row being consumed (the GEMV's ring is 3).  Each lane folds what it
// reads into an xor and stores it to the caller's 4-byte sink only when it
// equals one fixed value, so the loads stay in the program and a launch
// writes at most a few dwords of the sink (rarely: by chance).
#include "vb_common.hpp"
#include "vb_internal.hpp"
#include "../../include/vbhip.h"

namespace vb {
namespace {

constexpr int PROBE_WPG = 8;
constexpr int PROBE_PIECES = 4;  // rows up to 4 KB

template <int RPW, int NS>
__global__ void __launch_bounds__(64 * PROBE_WPG) stream_read_kernel(const uint8_t* __restrict__ w,
                                                                     uint32_t* __restrict__ sink, int n,
                                                                     uint32_t rb) {
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int row0 = (static_cast<int>(blockIdx.x) * PROBE_WPG + wave) * RPW;
    const int rlast = n - 1;
    const int rbase = row0 < rlast ? row0 : rlast;
    const uint8_t* wb = w + static_cast<int64_t>(rbase) * rb;
    const int64_t span64 = static_cast<int64_t>(n - rbase) * rb;
    const uint32_t span = span64 < 0xFFFFFFFFll ? static_cast<uint32_t>(span64) : 0xFFFFFFFFu;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(wb, span);
    const int slots = static_cast<int>(rb >> 4);
    const int npieces = (slots + 63) >> 6;
    uint32_t voff[PROBE_PIECES];
#pragma unroll
    for (int p = 0; p < PROBE_PIECES; p++) {
        const int sl = 64 * p + lane;
        voff[p] = 16u * static_cast<uint32_t>(sl < slots ? sl : lane % (slots < 8 ? slots : 8));
    }
    auto soff = [&](int s) -> uint32_t {
        int r = row0 + s;
        r = r < rlast ? r : rlast;
        return static_cast<uint32_t>(r - rbase) * rb;
    };
    u32x4 ring[NS][PROBE_PIECES];
    auto issue = [&](int slot, int s) {
        const uint32_t so = soff(s);
#pragma unroll
        for (int p = 0; p < PROBE_PIECES; p++)
            if (p < npieces)
                ring[slot][p] = __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(voff[p]),
                                                                     static_cast<int>(so), 2);
    };
    uint32_t acc = 0;
#pragma unroll
    for (int s = 0; s < NS - 1 && s < RPW; s++) issue(s, s);
#pragma unroll
    for (int s = 0; s < RPW; s++) {
        if (s + NS - 1 < RPW) issue((s + NS - 1) % NS, s + NS - 1);
#pragma unroll
        for (int p = 0; p < PROBE_PIECES; p++)
            if (p < npieces) {
                const u32x4 v = ring[s % NS][p];
                acc ^= v.x ^ v.y ^ v.z ^ v.w;
            }
        __builtin_amdgcn_sched_barrier(0);
    }
    if (acc == 0x5EEDF00Du) sink[0] = acc;
}

template <int NS>
void launch_probe(int rpw, const void* w, uint32_t* sink, int n, uint32_t rb, hipStream_t st) {
    const dim3 grid(static_cast<uint32_t>((n + PROBE_WPG * rpw - 1) / (PROBE_WPG * rpw)));
    const dim3 block(64 * PROBE_WPG);
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    switch (rpw) {
    case 1: stream_read_kernel<1, NS><<<grid, block, 0, st>>>(wb, sink, n, rb); break;
    case 2: stream_read_kernel<2, NS><<<grid, block, 0, st>>>(wb, sink, n, rb); break;
    case 3: stream_read_kernel<3, NS><<<grid, block, 0, st>>>(wb, sink, n, rb); break;
    case 4: stream_read_kernel<4, NS><<<grid, block, 0, st>>>(wb, sink, n, rb); break;
    case 5: stream_read_kernel<5, NS><<<grid, block, 0, st>>>(wb, sink, n, rb); break;
    case 6: stream_read_kernel<6, NS><<<grid, block, 0, st>>>(wb, sink, n, rb); break;
    case 7: stream_read_kernel<7, NS><<<grid, block, 0, st>>>(wb, sink, n, rb); break;
    default: stream_read_kernel<8, NS><<<grid, block, 0, st>>>(wb, sink, n, rb); break;
    }
}

}  // namespace
}  // namespace vb

extern "C" int vb_stream_read(const void* w, int64_t n, int64_t row_bytes, int32_t ring, uint32_t* sink,
                              void* stream) {
    using namespace vb;
    if (!w || !sink || n < 1 || n > INT32_MAX || row_bytes < 16 || row_bytes % 16 != 0 ||
        row_bytes > 16 * 64 * PROBE_PIECES || ring < 0 || ring > 8) {
        set_error("vb_stream_read: bad arguments (n=%lld row_bytes=%lld ring=%d)", static_cast<long long>(n),
                  static_cast<long long>(row_bytes), ring);
        return E_INVAL;
    }
    if (reinterpret_cast<uintptr_t>(w) % 16) {
        set_error("vb_stream_read: w must be 16-byte aligned");
        return E_INVAL;
    }
    const int64_t cus = num_cus();
    const int64_t rpw64 = (n + cus * PROBE_WPG - 1) / (cus * PROBE_WPG);
    if (rpw64 > 8) {
        set_error("vb_stream_read: %lld rows is more than 8 per wave", static_cast<long long>(n));
        return E_INVAL;
    }
    const int rpw = static_cast<int>(rpw64);
    // ring 0: every row of a wave in flight at once
    const int r = ring == 0 ? rpw : ring;
    const hipStream_t st = as_stream(stream);
    const int ni = static_cast<int>(n);
    const uint32_t rb = static_cast<uint32_t>(row_bytes);
    switch (r) {
    case 1: launch_probe<2>(rpw, w, sink, ni, rb, st); break;
    case 2: launch_probe<3>(rpw, w, sink, ni, rb, st); break;
    case 3: launch_probe<4>(rpw, w, sink, ni, rb, st); break;
    case 4: launch_probe<5>(rpw, w, sink, ni, rb, st); break;
    case 5: launch_probe<6>(rpw, w, sink, ni, rb, st); break;
    case 6: launch_probe<7>(rpw, w, sink, ni, rb, st); break;
    case 7: launch_probe<8>(rpw, w, sink, ni, rb, st); break;
    default: launch_probe<9>(rpw, w, sink, ni, rb, st); break;
    }
    return check_launch("vb_stream_read");
}
