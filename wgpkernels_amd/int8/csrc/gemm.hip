// INT8 x INT8 GEMM on gfx950 matrix cores (v_mfma_i32_32x32x32_i8), all modes of the reference's gemm_s8
// (wgpkernels/int8/int8_gemm.cu, K8:528-986):
//   row     Y = float(A.B) * sa[r] * sb[c] + bias
//   exact   two activation operands hi / lo:   (float(hi.B) + float(lo.B) / 254) * sa[r] * sb[c] + bias
//   block   sa per token and 128-element K block: the exact INT32 sums of each block are scaled into FP32
//   +g      weight scales per channel and 128-element K block (block and exact modes)
// then Y = R + rscale * Y (optional residual, may alias Y), one rounding to BF16 / FP16.
// Kernels: gemm_pingpong (gemm_pingpong.h) for the long tiles of every mode but block in the reference order, gemm_ring
// (gemm_ring.h) for those and the short tiles.
// C ABI below.
#include "gemm_ring.h"
#include "gemm_pingpong.h"
#include "wq8_abi.h"
#include <mutex>

namespace wq8 {

// ---- variants: the reference's variant ids keep their mode (K8:1417-1432); the tiles are this library's -------
// long: row 256 tokens x 256 channels, block (biased fold) and block with weight groups 256 x 192, hi/lo 128 x 256 or
// 128 x 192, hi/lo with weight groups 128 x 192, all on two groups of 4 waves in ping-pong (gemm_pingpong.h).
// short: 64 x 128 (hi/lo 32 x 128) on 4 waves, for inputs of few tokens. Variant 10 folds block sums with the
// single-FMA biased form; 11 and the weight-group variants fold in the reference's order.
enum { TILE_LONG = 0, TILE_SHORT = 1 };
struct Variant { int mode; bool wgroup; int tile; bool biased; };
static bool variant_info(int v, Variant& out) {
    switch (v) {
        case 0: case 2: out = {MODE_ROW, false, TILE_LONG, false}; return true;
        case 6: out = {MODE_ROW, false, TILE_SHORT, false}; return true;
        case 1: out = {MODE_EXACT, false, TILE_LONG, false}; return true;
        case 7: out = {MODE_EXACT, false, TILE_SHORT, false}; return true;
        case 10: out = {MODE_BLOCK, false, TILE_LONG, true}; return true;
        case 11: out = {MODE_BLOCK, false, TILE_SHORT, false}; return true;
        case 12: out = {MODE_BLOCK, true, TILE_LONG, false}; return true;
        case 13: out = {MODE_BLOCK, true, TILE_SHORT, false}; return true;
        case 14: out = {MODE_EXACT, true, TILE_LONG, false}; return true;
    }
    return false;
}

template <int BM, int BN, int WAVES_N, int WAVES_M, int MODE, bool WG, bool BIASED, int DT, bool SUMS, bool SEG, int BK = 128, int STAGES = 3>
static int launch_ring(GemmArgs& g, hipStream_t stream) {
    g.tiles_m = (g.m + BM - 1) / BM;
    g.tiles_n = (g.n + BN - 1) / BN;
    g.n_first = 0;
    gemm_ring<BM, BN, WAVES_N, WAVES_M, BK, STAGES, MODE, WG, BIASED, DT, SUMS, SEG><<<g.tiles_m * g.tiles_n, 64 * WAVES_N * WAVES_M, 0, stream>>>(g);
    return int(hipGetLastError());
}

// channels [n_first, n_first + n_count) of the output (all of them by default)
template <int BM, int BN, int WAVES_N, int WAVES_M, int MODE, bool WG, bool BIASED, int DT, bool SEG>
static int launch_pingpong(GemmArgs& g, hipStream_t stream, int n_first = 0, int n_count = -1) {
    g.tiles_m = (g.m + BM - 1) / BM;
    g.tiles_n = ((n_count < 0 ? g.n : n_count) + BN - 1) / BN;
    g.n_first = n_first;
    // K % 128 == 0: the copies need no K-tail select (one VALU compare-select fewer per copy)
    if (g.k % 128 == 0) gemm_pingpong<BM, BN, WAVES_N, WAVES_M, MODE, WG, BIASED, DT, SEG, false><<<g.tiles_m * g.tiles_n, 512, 0, stream>>>(g);
    else gemm_pingpong<BM, BN, WAVES_N, WAVES_M, MODE, WG, BIASED, DT, SEG><<<g.tiles_m * g.tiles_n, 512, 0, stream>>>(g);
    return int(hipGetLastError());
}

// The kernels address operands with 32-bit buffer offsets: each operand (plus a tile of rows) below 2^31 bytes.
static bool offsets_fit(const GemmArgs& g) {
    const int64_t lim = int64_t(1) << 31;
    const int64_t rows_b = g.seg_rows ? int64_t(g.seg_rows) : int64_t(g.n);
    return (int64_t(g.m) + 256) * g.k < lim && (rows_b + 256) * g.k < lim && (int64_t(g.m) + 256) * g.kblocks * 4 < lim &&
           (int64_t(g.n) + 256) * g.kblocks * 4 < lim;
}

// Tile area times the waves of workgroups a bm x bn tiling runs (one workgroup per CU at a time): the padded work of the
// launch, including the idle CUs of its last wave.
static int64_t padded_work(const GemmArgs& g, int bm, int bn) {
    const int64_t tiles = int64_t((g.m + bm - 1) / bm) * ((g.n + bn - 1) / bn), cus = g.sms > 0 ? g.sms : 256;
    return (tiles + cus - 1) / cus * bm * bn;
}

// Channel split of the long biased block tiles: the number of channels (a multiple of 192) run as 256 x 192 tiles, the
// rest as 256 x 128 tiles, or 0 for one launch. Chosen when the estimated time, in waves of 256 x 192 workgroups with a
// 256 x 128 one counted as 0.8 of one (measured: 256 x 128 tiles alone ran 15% slower than 256 x 192 at K = 13824,
// N = 5120, which is 0.805 per tile), beats one launch by more than 2%.
static int block_channel_split(const GemmArgs& g) {
    const int64_t cus = g.sms > 0 ? g.sms : 256, tm = (g.m + 255) / 256;
    auto waves = [&](int64_t tiles) { return (tiles + cus - 1) / cus; };
    const double one = double(waves(tm * ((g.n + 191) / 192)));
    double best = one * 0.98;
    int split = 0;
    for (int c = g.n / 192; c > 0 && c >= g.n / 192 - 8; --c) {
        const int rest = g.n - 192 * c;
        if (rest <= 0 || rest % 128) continue;
        const double t = double(waves(tm * c)) + 0.8 * double(waves(tm * (rest / 128)));
        if (t < best) {
            best = t;
            split = 192 * c;
        }
    }
    return split;
}

template <int MODE, bool WG, bool BIASED, int DT, bool SEG>
static int launch_tiles(GemmArgs& g, int tile, hipStream_t stream) {
    constexpr bool HILO = MODE == MODE_EXACT;
    if (tile == TILE_SHORT) {
        if constexpr (HILO) return launch_ring<32, 128, 4, 1, MODE, WG, BIASED, DT, false, SEG>(g, stream);
        else return launch_ring<64, 128, 4, 1, MODE, WG, BIASED, DT, false, SEG>(g, stream);
    }
    // hi/lo: 128 x 256 or 128 x 192 ping-pong (waves of 32 tokens x 128 or 96 channels, two INT32 accumulators per
    // tile), 128 x 192 when its last wave of workgroups is fuller; a stage holds the 128 tokens' hi and lo rows. 10-12%
    // faster than the 2-stage ring at config 4 (M = 4096, N = 3 x 5120 through the segments entry point: 533-542 against
    // 603-652 us, the same bits); the two tiles measure within 2% of each other there.
    if constexpr (HILO && !WG) {
        if (padded_work(g, 128, 192) < padded_work(g, 128, 256)) return launch_pingpong<128, 192, 2, 4, MODE, false, false, DT, SEG>(g, stream);
        return launch_pingpong<128, 256, 2, 4, MODE, false, false, DT, SEG>(g, stream);
    }
    // hi/lo with weight groups: 128 x 192 ping-pong (waves of 32 tokens x 96 channels). 23% faster than the 128 x 128
    // ring at M = 8192, N = 12288, K = 3072 (652 against 803 us), the same bits.
    else if constexpr (HILO && !SEG) return launch_pingpong<128, 192, 2, 4, MODE, true, false, DT, false>(g, stream);
    else if constexpr (HILO) return launch_ring<128, 128, 2, 4, MODE, WG, BIASED, DT, false, SEG>(g, stream);
    // row: 256 x 256 ping-pong (waves of 64 tokens x 128 channels); block with the biased fold: 256 x 192 ping-pong
    // (waves of 64 tokens x 96 channels, whose FP32 accumulators, fragments and fold chain fit 256 registers); block in the
    // reference's fold order and weight groups: 128 x 256 ring
    else if constexpr (MODE == MODE_ROW) return launch_pingpong<256, 256, 2, 4, MODE, false, false, DT, SEG>(g, stream);
    else if constexpr (MODE == MODE_BLOCK && BIASED && !WG) {
        // When the last wave of 256 x 192 workgroups would be at most half full, the channels split in two launches:
        // 256 x 192 tiles over a range that fills whole waves and 256 x 128 tiles over the rest (K = 13824, N = 5120:
        // 12 + 2 waves instead of 13.5 in 14). The tiles are the same tiles, so are the bits.
        const int split = block_channel_split(g);
        if (split > 0) {
            if (const int rc = launch_pingpong<256, 192, 2, 4, MODE, false, true, DT, SEG>(g, stream, 0, split)) return rc;
            return launch_pingpong<256, 128, 2, 4, MODE, false, true, DT, SEG>(g, stream, split, g.n - split);
        }
        return launch_pingpong<256, 192, 2, 4, MODE, false, true, DT, SEG>(g, stream);
    }
    // block with weight groups: 256 x 192 ping-pong, folding in the reference's order
    else if constexpr (MODE == MODE_BLOCK && WG && !SEG) return launch_pingpong<256, 192, 2, 4, MODE, true, false, DT, false>(g, stream);
    else return launch_ring<128, 256, 4, 2, MODE, WG, BIASED, DT, false, SEG>(g, stream);
}

template <int DT, bool SEG>
static int dispatch_gemm(GemmArgs& g, const Variant& v, hipStream_t stream) {
    if (!offsets_fit(g)) return -2;
    if (v.mode == MODE_ROW) return launch_tiles<MODE_ROW, false, false, DT, SEG>(g, v.tile, stream);
    if (v.mode == MODE_EXACT && !v.wgroup) return launch_tiles<MODE_EXACT, false, false, DT, SEG>(g, v.tile, stream);
    if (v.mode == MODE_BLOCK && !v.wgroup) {
        if (v.biased) return launch_tiles<MODE_BLOCK, false, true, DT, SEG>(g, v.tile, stream);
        return launch_tiles<MODE_BLOCK, false, false, DT, SEG>(g, v.tile, stream);
    }
    if constexpr (!SEG) {
        if (v.mode == MODE_BLOCK) return launch_tiles<MODE_BLOCK, true, false, DT, false>(g, v.tile, stream);
        return launch_tiles<MODE_EXACT, true, false, DT, false>(g, v.tile, stream);
    }
    return -4;
}

thread_local GemmArgs g_gemm_extra{};  // row offsets / segments of the wrapping entry points

// Block scales (rows x cols, row-major; source rows start at in_first + counter[0] * in_step when counter is set)
// transposed to dst[c * rows + r]: the GEMM then reads a k-block's scales of 64 consecutive tokens or channels as 256
// contiguous bytes. Thread r takes row r, 16 columns at a time: the loads of a wave cover its 64 rows' bytes whole (16-byte
// pieces when the row pitch allows), each store writes 64 consecutive floats of one output row.
__global__ void __launch_bounds__(64) transpose_scales(const float* src, float* dst, int rows, int cols, const long long* counter,
                                                       long long in_first, long long in_step, float divisor) {
    const long long shift = counter ? in_first + *counter * in_step : 0;
    const int r = blockIdx.x * 64 + threadIdx.x;
    if (r >= rows) return;
    const float* row = src + (shift + r) * int64_t(cols);
    const bool vec = (cols % 4) == 0 && (reinterpret_cast<uintptr_t>(src) % 16) == 0;
    for (int c0 = 0; c0 < cols; c0 += 16) {
        float v[16];
        if (vec && c0 + 16 <= cols) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const v4f f = *reinterpret_cast<const v4f*>(row + c0 + 4 * q);
#pragma unroll
                for (int e = 0; e < 4; ++e) v[4 * q + e] = f[e];
            }
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) v[e] = c0 + e < cols ? row[c0 + e] : 0.0f;
        }
#pragma unroll
        for (int e = 0; e < 16; ++e)
            if (c0 + e < cols) dst[int64_t(c0 + e) * rows + r] = divisor == 1.0f ? v[e] : v[e] / divisor;
    }
}

// divisor: 254 for the exact+g weight scales (the kernel's fold takes sb / 254, correctly rounded), else 1
static int transpose(const float* src, float* dst, int rows, int cols, const GemmArgs& g, bool shifted, hipStream_t stream,
                     float divisor = 1.0f) {
    transpose_scales<<<(rows + 63) / 64, 64, 0, stream>>>(src, dst, rows, cols, shifted ? g.counter : nullptr, g.in_first, g.in_step, divisor);
    return int(hipGetLastError());
}

// workspace bytes of the transposed block scales: [sa_t (m x kblocks)][sb_t (n x kblocks)], each 256-byte aligned
static int64_t align256(int64_t v) { return (v + 255) / 256 * 256; }
static void scale_workspace(int m, int n, int k, const Variant& v, int64_t& sa_bytes, int64_t& sb_bytes) {
    const int64_t kb = (k + 127) / 128;
    sa_bytes = v.mode == MODE_BLOCK ? align256(int64_t(m) * kb * 4) : 0;
    sb_bytes = v.wgroup ? align256(int64_t(n) * kb * 4) : 0;
}

// The reference's tile estimate (K8:1554-1568) restated for this library's tiles: padded work of the waves of
// workgroups that run at once, divided by a relative mainloop efficiency.
static double estimate_tiles(int m, int n, int k, int sms, int bm, int bn, int per_cu, double efficiency) {
    const long long tm = (m + bm - 1) / bm, tn = (n + bn - 1) / bn, tiles = tm * tn;
    const long long slots = (long long)per_cu * sms, waves = (tiles + slots - 1) / slots;
    return double(waves) * double(bm) * double(bn) * double(k) / efficiency;
}

}  // namespace wq8

using namespace wq8;

WQ8_API void wq8_gemm_workspace(int m, int n, int k, int variant, int sms, int split, int64_t* sizes) {
    // whole tiles only: no stream-K counters; the slots hold the block modes' transposed scales
    (void)sms; (void)split;
    Variant v;
    int64_t sa_bytes = 0, sb_bytes = 0;
    if (variant_info(variant, v)) scale_workspace(m, n, k, v, sa_bytes, sb_bytes);
    sizes[0] = sa_bytes + sb_bytes;
    sizes[1] = 0;
}

WQ8_API int wq8_gemm_select(int m, int n, int k, int hilo, int sms) {
    if (hilo) return estimate_tiles(m, n, k, sms, 128, 256, 1, 1.0) <= estimate_tiles(m, n, k, sms, 32, 128, 2, 0.5) ? 1 : 7;
    return estimate_tiles(m, n, k, sms, 256, 256, 1, 1.0) <= estimate_tiles(m, n, k, sms, 64, 128, 2, 0.5) ? 0 : 6;
}

WQ8_API int wq8_gemm(const int8_t* a, const int8_t* a_lo, const float* sa, const int8_t* b, const float* sb, const void* bias, const void* residual,
                     const void* rscale, void* y, int m, int n, int k, int dtype, int variant, int sms, int split, int* workspace, int* counters,
                     hipStream_t stream) {
    (void)split; (void)counters;
    if (!m || !n) return 0;
    Variant v;
    if (!variant_info(variant, v)) return -3;
    if ((v.mode == MODE_EXACT) != (a_lo != nullptr)) return -2;
    if (m < 0 || n < 0 || k <= 0 || k % 16) return -2;
    GemmArgs g = g_gemm_extra;
    g.a = a; g.a_lo = a_lo; g.sa = sa; g.b = b; g.sb = sb; g.bias = bias; g.residual = residual; g.rscale = rscale; g.y = y;
    g.sums = nullptr;
    g.m = m; g.n = n; g.k = k; g.kblocks = (k + 127) / 128; g.sms = sms;
    const bool seg = g.seg_rows > 0;
    if (seg && v.wgroup) return -4;
    int64_t sa_bytes = 0, sb_bytes = 0;
    scale_workspace(m, n, k, v, sa_bytes, sb_bytes);
    if (sa_bytes + sb_bytes) {
        if (!workspace) return -2;  // sized by wq8_gemm_workspace
        if (!offsets_fit(g)) return -2;
        uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
        if (sa_bytes) {
            g.sa_t = reinterpret_cast<float*>(ws);
            const int rc = transpose(sa, reinterpret_cast<float*>(ws), m, g.kblocks, g, true, stream);
            if (rc) return rc;
        }
        if (sb_bytes) {
            g.sb_t = reinterpret_cast<float*>(ws + sa_bytes);
            const int rc = transpose(sb, reinterpret_cast<float*>(ws + sa_bytes), n, g.kblocks, g, false, stream,
                                     v.mode == MODE_EXACT ? 254.0f : 1.0f);
            if (rc) return rc;
        }
    }
    if (dtype == DT_F16) return seg ? dispatch_gemm<DT_F16, true>(g, v, stream) : dispatch_gemm<DT_F16, false>(g, v, stream);
    if (dtype == DT_BF16) return seg ? dispatch_gemm<DT_BF16, true>(g, v, stream) : dispatch_gemm<DT_BF16, false>(g, v, stream);
    return -1;
}

WQ8_API int wq8_gemm_at(const int8_t* a, const int8_t* a_lo, const float* sa, const int8_t* b, const float* sb, const void* bias, const void* residual,
                        const void* rscale, void* y, int m, int n, int k, int dtype, int variant, int sms, int split, int* workspace, int* counters,
                        const long long* counter, long long first, long long step, long long span, long long scale_step, long long in_first,
                        long long in_step, hipStream_t stream) {
    g_gemm_extra = GemmArgs{};
    g_gemm_extra.counter = counter; g_gemm_extra.first = first; g_gemm_extra.step = step; g_gemm_extra.span = span;
    g_gemm_extra.scale_step = scale_step; g_gemm_extra.in_first = in_first; g_gemm_extra.in_step = in_step;
    const int rc = wq8_gemm(a, a_lo, sa, b, sb, bias, residual, rscale, y, m, n, k, dtype, variant, sms, split, workspace, counters, stream);
    g_gemm_extra = GemmArgs{};
    return rc;
}

WQ8_API int wq8_gemm_segments(const int8_t* a, const int8_t* a_lo, const float* sa, const int8_t* const* bs, const float* const* sbs,
                              const void* const* biases, void* const* ys, int count, int rows, int m, int k, int dtype, int variant, int sms,
                              int split, int* workspace, int* counters, hipStream_t stream) {
    if (count < 1 || count > 4 || rows <= 0 || rows % 8) return -4;
    g_gemm_extra = GemmArgs{};
    g_gemm_extra.seg_rows = rows;
    for (int s = 0; s < count; ++s) {
        g_gemm_extra.seg_b[s] = bs[s]; g_gemm_extra.seg_sb[s] = sbs[s]; g_gemm_extra.seg_bias[s] = biases[s]; g_gemm_extra.seg_y[s] = ys[s];
    }
    const int rc = wq8_gemm(a, a_lo, sa, bs[0], sbs[0], nullptr, nullptr, nullptr, ys[0], m, count * rows, k, dtype, variant, sms, split, workspace,
                            counters, stream);
    g_gemm_extra = GemmArgs{};
    return rc;
}

// ---- allocation-free GEMM --------------------------------------------------------------------------------------------
// For callers that cannot allocate (code under graph capture, serving loops, harnesses that forbid hipMalloc): the
// workspace wq8_gemm takes from its caller lives in a file-scope device array instead. Each GPU the library runs on holds
// its own copy until the process ends; every call on a GPU shares it, so calls that overlap on one GPU race.
namespace wq8 {
constexpr int64_t NOALLOC_SCRATCH_BYTES = int64_t(32) << 20;  // WQ8_GEMM_NOALLOC_MAX_BYTES of include/wq8.h
constexpr int NOALLOC_MAX_DEVICES = 64;
__device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];
static std::mutex g_scratch_mutex;
static void* g_scratch_ptr[NOALLOC_MAX_DEVICES];

// Device address of the current device's copy of `scratch` (looked up once per device; the array's name is only a
// host-side stand-in). 0 on success.
static int scratch_address(void** out) {
    int device = 0;
    if (hipError_t e = hipGetDevice(&device)) return int(e);
    if (device < 0 || device >= NOALLOC_MAX_DEVICES) return -2;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[device]) {
        void* p = nullptr;
        if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) return int(e);
        g_scratch_ptr[device] = p;
    }
    *out = g_scratch_ptr[device];
    return 0;
}

__global__ void __launch_bounds__(256) zero_words(int* p, int words) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < words) p[i] = 0;
}
}  // namespace wq8

WQ8_API int wq8_gemm_noalloc(const int8_t* a, const int8_t* a_lo, const float* sa, const int8_t* b, const float* sb, const void* bias,
                             const void* residual, const void* rscale, void* y, int m, int n, int k, int dtype, int variant, int sms,
                             int split, hipStream_t stream) {
    if (!m || !n) return 0;
    int64_t sizes[2] = {0, 0};
    wq8_gemm_workspace(m, n, k, variant, sms, split, sizes);
    const int64_t slot_bytes = align256(sizes[0]);
    if (slot_bytes + sizes[1] > NOALLOC_SCRATCH_BYTES) return -5;
    void* base = nullptr;
    if (int rc = scratch_address(&base)) return rc;
    uint8_t* ws = static_cast<uint8_t*>(base);
    int* counters = nullptr;
    if (sizes[1]) {
        // split counters start at zero: cleared by a kernel (a memset node would be wrong in a replayed graph)
        counters = reinterpret_cast<int*>(ws + slot_bytes);
        const int words = int(sizes[1] / 4);
        zero_words<<<(words + 255) / 256, 256, 0, stream>>>(counters, words);
        if (hipError_t e = hipGetLastError()) return int(e);
    }
    return wq8_gemm(a, a_lo, sa, b, sb, bias, residual, rscale, y, m, n, k, dtype, variant, sms, split,
                    sizes[0] ? reinterpret_cast<int*>(ws) : nullptr, counters, stream);
}

// Test entry point (no counterpart in the reference): the exact INT32 sums of every 128-element K block,
// sums[(t * N + c) * ceil(K / 128) + kb], computed by the block-mode GEMM mainloop instead of being folded.
WQ8_API int wq8_debug_block_sums(const int8_t* a, const int8_t* b, int32_t* sums, int m, int n, int k, hipStream_t stream) {
    if (!m || !n) return 0;
    if (m < 0 || n < 0 || k <= 0 || k % 16) return -2;
    GemmArgs g{};
    g.a = a; g.b = b; g.sums = sums;
    g.m = m; g.n = n; g.k = k; g.kblocks = (k + 127) / 128;
    if (!offsets_fit(g)) return -2;
    return launch_ring<128, 256, 4, 2, MODE_ROW, false, false, DT_BF16, true, false>(g, stream);
}
