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
// row being consumed (the GEMV's register ring is 3).  With a negative ring
// the rows land in LDS by DMA (buffer_load ... lds, one __shared__ array per
// ring slot, as the GEMV's DMA kernel loads them; its ring is 2) and each
// lane reads its pieces back from LDS.  Each lane folds what it
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

// DMA variant: slot k of the ring is its own __shared__ array (NP KB a
// wave); NP = the 1 KB pieces of a row
template <int RPW, int NS, int NP>
__global__ void __launch_bounds__(64 * PROBE_WPG) stream_read_dma_kernel(const uint8_t* __restrict__ w,
                                                                         uint32_t* __restrict__ sink, int n,
                                                                         uint32_t rb) {
    static_assert(NS >= 2 && NS <= 4 && NP >= 1 && NP <= PROBE_PIECES, "ring of 1..3 rows ahead");
    constexpr int SL = 64 * NP;
    __shared__ u32x4 s0[PROBE_WPG][SL], s1[PROBE_WPG][SL], s2[PROBE_WPG][SL], s3[PROBE_WPG][SL];
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
    uint32_t voff[NP];
#pragma unroll
    for (int p = 0; p < NP; p++) {
        const int sl = 64 * p + lane;
        voff[p] = 16u * static_cast<uint32_t>(sl < slots ? sl : lane % (slots < 8 ? slots : 8));
    }
    auto base = [&](auto k_c) __attribute__((always_inline)) -> u32x4* {
        constexpr int k = decltype(k_c)::value;
        if constexpr (k == 0) return s0[wave];
        else if constexpr (k == 1) return s1[wave];
        else if constexpr (k == 2) return s2[wave];
        else return s3[wave];
    };
    auto issue = [&](auto k_c, int s) __attribute__((always_inline)) {
        int r = row0 + s;
        r = r < rlast ? r : rlast;
        const uint32_t so = static_cast<uint32_t>(r - rbase) * rb;
        u32x4* b = base(k_c);
        typedef __attribute__((address_space(3))) void* lds_ptr;
#pragma unroll
        for (int p = 0; p < NP; p++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(b + 64 * p), 16, static_cast<int>(voff[p]),
                                                     static_cast<int>(so), 0, 2);
    };
    uint32_t acc = 0;
    if constexpr (NS - 1 >= 1) issue(std::integral_constant<int, 0>{}, 0);
    if constexpr (NS - 1 >= 2) if (1 < RPW) issue(std::integral_constant<int, 1>{}, 1);
    if constexpr (NS - 1 >= 3) if (2 < RPW) issue(std::integral_constant<int, 2>{}, 2);
    auto step = [&](auto s_c) __attribute__((always_inline)) {
        constexpr int s = decltype(s_c)::value;
        if constexpr (s < RPW) {
            if constexpr (s + NS - 1 < RPW) issue(std::integral_constant<int, (s + NS - 1) % NS>{}, s + NS - 1);
            // loads retire in order: row s is in once at most the later rows' loads remain
            constexpr int later = NP * (s + NS - 1 < RPW ? NS - 1 : RPW - 1 - s);
            static_assert(later < 16, "vmcnt field");
            __builtin_amdgcn_s_waitcnt(0x0F70 | later);
            const u32x4* b = base(std::integral_constant<int, s % NS>{});
#pragma unroll
            for (int p = 0; p < NP; p++) {
                const u32x4 v = b[64 * p + lane];
                acc ^= v.x ^ v.y ^ v.z ^ v.w;
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    step(std::integral_constant<int, 0>{});
    step(std::integral_constant<int, 1>{});
    step(std::integral_constant<int, 2>{});
    step(std::integral_constant<int, 3>{});
    step(std::integral_constant<int, 4>{});
    step(std::integral_constant<int, 5>{});
    step(std::integral_constant<int, 6>{});
    step(std::integral_constant<int, 7>{});
    if (acc == 0x5EEDF00Du) sink[0] = acc;
}

template <int NS, int NP>
void launch_probe_dma(int rpw, const void* w, uint32_t* sink, int n, uint32_t rb, hipStream_t st) {
    const dim3 grid(static_cast<uint32_t>((n + PROBE_WPG * rpw - 1) / (PROBE_WPG * rpw)));
    const dim3 block(64 * PROBE_WPG);
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    switch (rpw) {
    case 1: stream_read_dma_kernel<1, NS, NP><<<grid, block, 0, st>>>(wb, sink, n, rb); break;
    case 2: stream_read_dma_kernel<2, NS, NP><<<grid, block, 0, st>>>(wb, sink, n, rb); break;
    case 3: stream_read_dma_kernel<3, NS, NP><<<grid, block, 0, st>>>(wb, sink, n, rb); break;
    case 4: stream_read_dma_kernel<4, NS, NP><<<grid, block, 0, st>>>(wb, sink, n, rb); break;
    case 5: stream_read_dma_kernel<5, NS, NP><<<grid, block, 0, st>>>(wb, sink, n, rb); break;
    case 6: stream_read_dma_kernel<6, NS, NP><<<grid, block, 0, st>>>(wb, sink, n, rb); break;
    case 7: stream_read_dma_kernel<7, NS, NP><<<grid, block, 0, st>>>(wb, sink, n, rb); break;
    default: stream_read_dma_kernel<8, NS, NP><<<grid, block, 0, st>>>(wb, sink, n, rb); break;
    }
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
        row_bytes > 16 * 64 * PROBE_PIECES || ring < -3 || ring > 8) {
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
    if (ring < 0) {
        // 3 rows ahead hold 4 x 8 x 3 KB of LDS at most
        const int np = static_cast<int>((rb / 16 + 63) / 64);
        if (np * (1 - ring) * 8 > 128) {
            set_error("vb_stream_read: a DMA ring of %d rows of %u bytes does not fit in LDS", -ring, rb);
            return E_INVAL;
        }
        auto go = [&](auto np_c) {
            constexpr int NP = decltype(np_c)::value;
            if (ring == -1) launch_probe_dma<2, NP>(rpw, w, sink, ni, rb, st);
            else if (ring == -2) launch_probe_dma<3, NP>(rpw, w, sink, ni, rb, st);
            else launch_probe_dma<4, NP>(rpw, w, sink, ni, rb, st);
        };
        if (np == 1) go(std::integral_constant<int, 1>{});
        else if (np == 2) go(std::integral_constant<int, 2>{});
        else if (np == 3) go(std::integral_constant<int, 3>{});
        else go(std::integral_constant<int, 4>{});
        return check_launch("vb_stream_read");
    }
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
