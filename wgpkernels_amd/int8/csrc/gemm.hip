// INT8 x INT8 GEMM on gfx950 matrix cores (v_mfma_i32_32x32x32_i8), all modes of the reference's gemm_s8
// (wgpkernels/int8/int8_gemm.cu, K8:528-986):
//   row     Y = float(A.B) * sa[r] * sb[c] + bias
//   exact   two activation operands hi / lo:   (float(hi.B) + float(lo.B) / 254) * sa[r] * sb[c] + bias
//   block   sa per token and 128-element K block: the exact INT32 sums of each block are scaled into FP32
//   +g      weight scales per channel and 128-element K block (block and exact modes)
// then Y = R + rscale * Y (optional residual, may alias Y), one rounding to BF16 / FP16.
//
// Design (gfx950, wave64):
// - One 256-thread workgroup (4 waves) per BM x BN output tile (BM tokens x BN channels), BK = 128: one k-tile is
//   exactly one scale block, so the block fold runs once per k-tile with no predication.
// - The weights are the MFMA "A" operand (32 channels) and the activations the "B" operand (32 tokens): a lane of the
//   32x32 accumulator holds one token and 16 channels, so a block fold needs one activation scale per lane and
//   32-token fragment.
// - Operands go global -> registers -> LDS (double buffered, 16-byte chunks XOR-swizzled by row so that the 32 rows of
//   a fragment read hit distinct banks); the next k-tile's global loads are in flight during the MFMAs.
// - Tiles map XCD-aware: consecutive workgroups land on different XCDs (round robin), so workgroup b is given the
//   virtual tile (b % 8) * (tiles / 8) + b / 8 and each XCD works through a contiguous band of a grouped raster,
//   sharing A and B panels in its own L2.
#include "wq8_common.h"
#include "wq8_abi.h"

namespace wq8 {

enum { MODE_ROW = 0, MODE_EXACT = 1, MODE_BLOCK = 2 };

struct GemmArgs {
    const int8_t* a;
    const int8_t* a_lo;
    const float* sa;
    const int8_t* b;
    const float* sb;
    const void* bias;
    const void* residual;
    const void* rscale;
    void* y;
    int32_t* sums;  // block-sum dump (test entry point) or null
    int m, n, k, kblocks, tiles_m, tiles_n;
    // row offsets of CUDA-graph-style loops (wq8_gemm_at): output / residual rows first + counter * step,
    // residual scales per span of rows, input rows in_first + counter * in_step
    const long long* counter;
    long long first, step, span, scale_step, in_first, in_step;
    // output segments (wq8_gemm_segments): channel c belongs to segment c / seg_rows
    int seg_rows;
    const int8_t* seg_b[4];
    const float* seg_sb[4];
    const void* seg_bias[4];
    void* seg_y[4];
};

template <int BM, int BN, int WAVES_N, int MODE, bool WG, int DT, bool SUMS, bool SEG>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) gemm_i8(GemmArgs g) {
    using raw = typename Elem<DT>::raw;
    constexpr bool HILO = MODE == MODE_EXACT;
    constexpr bool FOLD = MODE == MODE_BLOCK || WG;
    constexpr int WAVES_M = 4 / WAVES_N;
    constexpr int WN = BN / WAVES_N, WM = BM / WAVES_M;
    constexpr int FN = WN / 32, FM = WM / 32;
    constexpr int A_ROWS = BM * (HILO ? 2 : 1);
    constexpr int STAGE = (A_ROWS + BN) * 128;
    constexpr int A_PIECES = A_ROWS / 32, B_PIECES = BN / 32;  // 16-byte pieces per thread and k-tile
    constexpr int SCALES = FOLD ? (MODE == MODE_BLOCK ? BM : 0) + (WG ? BN : 0) : 1;
    static_assert(BM % 32 == 0 && BN % 32 == 0 && FN >= 1 && FM >= 1, "tile");
    static_assert(SCALES <= 256, "one thread per staged scale");
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * STAGE];
    __shared__ __attribute__((aligned(16))) float s_scale[2][SCALES];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wn = wave % WAVES_N, wm = wave / WAVES_N;
    const int m = g.m, n = g.n, k = g.k, kblocks = g.kblocks;

    // ---- tile of this workgroup: XCD-aware band of a grouped raster -------------------------------------------
    int tm, tn;
    {
        const int tiles = g.tiles_m * g.tiles_n, b = blockIdx.x;
        const int q = tiles / 8, r = tiles % 8, xcd = b % 8, idx = b / 8;
        const int v = xcd * q + (xcd < r ? xcd : r) + idx;
        constexpr int GROUP_M = 8;
        const int width = GROUP_M * g.tiles_n, first = (v / width) * GROUP_M;
        const int rows = g.tiles_m - first < GROUP_M ? g.tiles_m - first : GROUP_M;
        tm = first + (v % width) % rows;
        tn = (v % width) / rows;
    }
    const int m0 = tm * BM, n0 = tn * BN;
    const long long in_shift = g.counter && (g.in_first || g.in_step) ? g.in_first + __ldg(g.counter) * g.in_step : 0;
    const int8_t* a = g.a + in_shift * k;
    const int8_t* a_lo = HILO ? g.a_lo + in_shift * k : nullptr;
    const float* sa = g.sa + in_shift * (MODE == MODE_BLOCK ? kblocks : 1);

    // ---- per-thread copy sources: chunk tid % 8 of rows tid / 8 + 32 u (clamped: rows past M / N are never stored)
    const int chunk = tid & 7;
    const int8_t* a_src[A_PIECES];
    uint32_t a_dst[A_PIECES];
#pragma unroll
    for (int u = 0; u < A_PIECES; ++u) {
        const int row = (tid >> 3) + 32 * u;
        const int tok = m0 + (row % BM) < m ? m0 + (row % BM) : m - 1;
        a_src[u] = (HILO && row >= BM ? a_lo : a) + int64_t(tok) * k + chunk * 16;
        a_dst[u] = row * 128 + ((chunk ^ (row & 7)) << 4);
    }
    const int8_t* b_src[B_PIECES];
    uint32_t b_dst[B_PIECES];
#pragma unroll
    for (int u = 0; u < B_PIECES; ++u) {
        const int row = (tid >> 3) + 32 * u;
        const int ch = n0 + row < n ? n0 + row : n - 1;
        if constexpr (SEG) b_src[u] = g.seg_b[ch / g.seg_rows] + int64_t(ch % g.seg_rows) * k + chunk * 16;
        else b_src[u] = g.b + int64_t(ch) * k + chunk * 16;
        b_dst[u] = (A_ROWS + row) * 128 + ((chunk ^ (row & 7)) << 4);
    }

    const int k_tiles = (k + 127) / 128;
    u32x4 a_reg[A_PIECES], b_reg[B_PIECES];
    float s_reg = 0.0f;
    auto load_tile = [&](int kt) {
        const int k0 = kt * 128;
        const bool ok = k0 + chunk * 16 < k;
#pragma unroll
        for (int u = 0; u < A_PIECES; ++u) a_reg[u] = ok ? *reinterpret_cast<const u32x4*>(a_src[u] + k0) : u32x4{0, 0, 0, 0};
#pragma unroll
        for (int u = 0; u < B_PIECES; ++u) b_reg[u] = ok ? *reinterpret_cast<const u32x4*>(b_src[u] + k0) : u32x4{0, 0, 0, 0};
        if constexpr (FOLD) {
            int idx = tid;
            if (MODE == MODE_BLOCK) {
                if (idx < BM) {
                    const int tok = m0 + idx < m ? m0 + idx : m - 1;
                    s_reg = sa[int64_t(tok) * kblocks + kt];
                }
                idx -= BM;
            }
            if (WG && idx >= 0 && idx < BN) {
                const int ch = n0 + idx < n ? n0 + idx : n - 1;
                s_reg = g.sb[int64_t(ch) * kblocks + kt];
            }
        }
    };
    auto store_tile = [&](int st) {
        uint8_t* base = lds + st * STAGE;
#pragma unroll
        for (int u = 0; u < A_PIECES; ++u) *reinterpret_cast<u32x4*>(base + a_dst[u]) = a_reg[u];
#pragma unroll
        for (int u = 0; u < B_PIECES; ++u) *reinterpret_cast<u32x4*>(base + b_dst[u]) = b_reg[u];
        if constexpr (FOLD) {
            if (tid < SCALES) s_scale[st][tid] = s_reg;
        }
    };

    v16i acc[FN][FM];
    v16i acc_lo[HILO ? FN : 1][HILO ? FM : 1];
    v16f accf[FOLD ? FN : 1][FOLD ? FM : 1];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) {
            acc[i][j] = v16i{};
            if constexpr (HILO) acc_lo[i][j] = v16i{};
            if constexpr (FOLD) accf[i][j] = v16f{};
        }

    // fragment addresses: row (lane % 32) of a 32-row fragment, 16-byte chunk 2 ks + lane / 32, swizzled by row % 8
    const int frag_row = lane & 31;
    auto swz = [&](int ks) { return ((2 * ks + (lane >> 5)) ^ (lane & 7)) << 4; };

    load_tile(0);
    store_tile(0);
    __syncthreads();
    for (int kt = 0; kt < k_tiles; ++kt) {
        const int st = kt & 1;
        if (kt + 1 < k_tiles) load_tile(kt + 1);
        const uint8_t* as = lds + st * STAGE;
        const uint8_t* bs = as + A_ROWS * 128;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int sw = swz(ks);
            v4i bf[FN], af[FM], lf[HILO ? FM : 1];
#pragma unroll
            for (int i = 0; i < FN; ++i) bf[i] = *reinterpret_cast<const v4i*>(bs + (wn * WN + i * 32 + frag_row) * 128 + sw);
#pragma unroll
            for (int j = 0; j < FM; ++j) {
                af[j] = *reinterpret_cast<const v4i*>(as + (wm * WM + j * 32 + frag_row) * 128 + sw);
                if constexpr (HILO) lf[j] = *reinterpret_cast<const v4i*>(as + (BM + wm * WM + j * 32 + frag_row) * 128 + sw);
            }
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[i], af[j], acc[i][j], 0, 0, 0);
                    if constexpr (HILO) acc_lo[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[i], lf[j], acc_lo[i][j], 0, 0, 0);
                }
        }
        if constexpr (SUMS) {
            // exact INT32 block sums, dumped as sums[(t * N + c) * kblocks + kt]
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j) {
                    const int t = m0 + wm * WM + j * 32 + frag_row;
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int c = n0 + wn * WN + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                        if (t < m && c < n) g.sums[(int64_t(t) * n + c) * kblocks + kt] = acc[i][j][e];
                    }
                    acc[i][j] = v16i{};
                }
        } else if constexpr (FOLD) {
            const float* scales = s_scale[st];
#pragma unroll
            for (int j = 0; j < FM; ++j) {
                const float s_tok = MODE == MODE_BLOCK ? scales[wm * WM + j * 32 + frag_row] : 1.0f;
#pragma unroll
                for (int i = 0; i < FN; ++i) {
                    if constexpr (WG) {
                        const float* sbk = scales + (MODE == MODE_BLOCK ? BM : 0) + wn * WN + i * 32 + 4 * (lane >> 5);
#pragma unroll
                        for (int gi = 0; gi < 4; ++gi) {
                            const v4f s4 = *reinterpret_cast<const v4f*>(sbk + 8 * gi);
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const int x = 4 * gi + e;
                                if constexpr (MODE == MODE_BLOCK) {
                                    accf[i][j][x] = __builtin_fmaf(float(acc[i][j][x]), s_tok * s4[e], accf[i][j][x]);
                                } else {
                                    const float v = __builtin_fmaf(float(acc_lo[i][j][x]), 1.0f / 254.0f, float(acc[i][j][x]));
                                    accf[i][j][x] = __builtin_fmaf(v, s4[e], accf[i][j][x]);
                                }
                            }
                        }
                    } else {
#pragma unroll
                        for (int x = 0; x < 16; ++x) accf[i][j][x] = __builtin_fmaf(float(acc[i][j][x]), s_tok, accf[i][j][x]);
                    }
                    acc[i][j] = v16i{};
                    if constexpr (HILO) acc_lo[i][j] = v16i{};
                }
            }
        }
        if (kt + 1 < k_tiles) store_tile(st ^ 1);
        __syncthreads();
    }
    if constexpr (SUMS) return;

    // ---- epilogue: FP32 arithmetic of K8:810-863, one rounding --------------------------------------------------
    const long long shift = g.counter ? g.first + __ldg(g.counter) * g.step : 0;
    raw* y = static_cast<raw*>(g.y) + shift * n;
    const raw* residual = g.residual ? static_cast<const raw*>(g.residual) + shift * n : nullptr;
    const raw* bias = static_cast<const raw*>(g.bias);
#pragma unroll
    for (int j = 0; j < FM; ++j) {
        const int t = m0 + wm * WM + j * 32 + frag_row;
        if (t >= m) continue;
        const float row_scale = MODE == MODE_BLOCK ? 1.0f : sa[t];
        const raw* rs_row = g.rscale ? static_cast<const raw*>(g.rscale) + (g.span ? (shift + t) / g.span * g.scale_step : 0) : nullptr;
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int gi = 0; gi < 4; ++gi) {
                const int c0 = n0 + wn * WN + i * 32 + 8 * gi + 4 * (lane >> 5);
                if (c0 >= n) continue;
                float out[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int x = 4 * gi + e, c = c0 + e < n ? c0 + e : n - 1;
                    float v;
                    if constexpr (FOLD) v = accf[i][j][x];
                    else if constexpr (HILO) v = __builtin_fmaf(float(acc_lo[i][j][x]), 1.0f / 254.0f, float(acc[i][j][x]));
                    else v = float(acc[i][j][x]);
                    float col_scale, bv;
                    if constexpr (SEG) {
                        const int s = c / g.seg_rows, cc = c % g.seg_rows;
                        col_scale = g.seg_sb[s][cc];
                        bv = g.seg_bias[s] ? Elem<DT>::to_f(static_cast<const raw*>(g.seg_bias[s])[cc]) : 0.0f;
                    } else {
                        col_scale = WG ? 1.0f : g.sb[c];
                        bv = bias ? Elem<DT>::to_f(bias[c]) : 0.0f;
                    }
                    float o = __builtin_fmaf(v * row_scale, col_scale, bv);
                    if (residual) {
                        const float rs = rs_row ? Elem<DT>::to_f(rs_row[c]) : 1.0f;
                        o = __builtin_fmaf(o, rs, Elem<DT>::to_f(residual[int64_t(t) * n + c]));
                    }
                    out[e] = o;
                }
                if constexpr (SEG) {
                    const int s = c0 / g.seg_rows, cc = c0 % g.seg_rows;
                    raw* yp = static_cast<raw*>(g.seg_y[s]) + int64_t(t) * g.seg_rows + cc;
                    *reinterpret_cast<u32x2*>(yp) = u32x2{uint32_t(Elem<DT>::from_f(out[0])) | (uint32_t(Elem<DT>::from_f(out[1])) << 16),
                                                          uint32_t(Elem<DT>::from_f(out[2])) | (uint32_t(Elem<DT>::from_f(out[3])) << 16)};
                } else if (c0 + 3 < n && (n & 3) == 0) {
                    *reinterpret_cast<u32x2*>(y + int64_t(t) * n + c0) =
                        u32x2{uint32_t(Elem<DT>::from_f(out[0])) | (uint32_t(Elem<DT>::from_f(out[1])) << 16),
                              uint32_t(Elem<DT>::from_f(out[2])) | (uint32_t(Elem<DT>::from_f(out[3])) << 16)};
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (c0 + e < n) y[int64_t(t) * n + c0 + e] = Elem<DT>::from_f(out[e]);
                }
            }
    }
}

// ---- variants: the reference's variant ids keep their mode (K8:1417-1432); the tiles are this library's -------
struct Variant { int mode; bool wgroup; int bm, bn; };
static bool variant_info(int v, Variant& out) {
    switch (v) {
        case 0: case 2: out = {MODE_ROW, false, 128, 128}; return true;
        case 6: out = {MODE_ROW, false, 32, 128}; return true;
        case 1: out = {MODE_EXACT, false, 128, 128}; return true;
        case 7: out = {MODE_EXACT, false, 32, 128}; return true;
        case 10: out = {MODE_BLOCK, false, 128, 128}; return true;
        case 11: out = {MODE_BLOCK, false, 32, 128}; return true;
        case 12: out = {MODE_BLOCK, true, 128, 128}; return true;
        case 13: out = {MODE_BLOCK, true, 32, 128}; return true;
        case 14: out = {MODE_EXACT, true, 128, 128}; return true;
    }
    return false;
}

template <int BM, int BN, int WAVES_N, int MODE, bool WG, int DT, bool SUMS, bool SEG>
static int launch_gemm(GemmArgs& g, hipStream_t stream) {
    g.tiles_m = (g.m + BM - 1) / BM;
    g.tiles_n = (g.n + BN - 1) / BN;
    const int tiles = g.tiles_m * g.tiles_n;
    gemm_i8<BM, BN, WAVES_N, MODE, WG, DT, SUMS, SEG><<<tiles, 256, 0, stream>>>(g);
    return int(hipGetLastError());
}

template <int MODE, bool WG, int DT, bool SEG>
static int launch_tiles(GemmArgs& g, int bm, hipStream_t stream) {
    if (bm == 128) return launch_gemm<128, 128, 2, MODE, WG, DT, false, SEG>(g, stream);
    return launch_gemm<32, 128, 4, MODE, WG, DT, false, SEG>(g, stream);
}

template <int DT, bool SEG>
static int dispatch_gemm(GemmArgs& g, const Variant& v, hipStream_t stream) {
    if (v.mode == MODE_ROW) return launch_tiles<MODE_ROW, false, DT, SEG>(g, v.bm, stream);
    if (v.mode == MODE_EXACT && !v.wgroup) return launch_tiles<MODE_EXACT, false, DT, SEG>(g, v.bm, stream);
    if (v.mode == MODE_BLOCK && !v.wgroup) return launch_tiles<MODE_BLOCK, false, DT, SEG>(g, v.bm, stream);
    if constexpr (!SEG) {
        if (v.mode == MODE_BLOCK) return launch_tiles<MODE_BLOCK, true, DT, false>(g, v.bm, stream);
        return launch_tiles<MODE_EXACT, true, DT, false>(g, v.bm, stream);
    }
    return -4;
}

thread_local GemmArgs g_gemm_extra{};  // row offsets / segments of the wrapping entry points

// The reference's tile estimate (K8:1554-1568) restated for this library's two tile heights: padded work divided
// by the workgroups that run at once (two per CU).
static double estimate_tiles(int m, int n, int k, int sms, int bm, double efficiency) {
    const long long tm = (m + bm - 1) / bm, tn = (n + 127) / 128, tiles = tm * tn;
    const double slots = 2.0 * sms, waves = double((tiles + (long long)slots - 1) / (long long)slots);
    return waves * double(bm) * 128.0 * double(k) / efficiency;
}

}  // namespace wq8

using namespace wq8;

WQ8_API void wq8_gemm_workspace(int m, int n, int k, int variant, int sms, int split, int64_t* sizes) {
    // whole tiles only: no stream-K slots or counters
    (void)m; (void)n; (void)k; (void)variant; (void)sms; (void)split;
    sizes[0] = 0;
    sizes[1] = 0;
}

WQ8_API int wq8_gemm_select(int m, int n, int k, int hilo, int sms) {
    const double big = estimate_tiles(m, n, k, sms, 128, 1.0), small = estimate_tiles(m, n, k, sms, 32, 0.55);
    if (hilo) return big <= small ? 1 : 7;
    return big <= small ? 0 : 6;
}

WQ8_API int wq8_gemm(const int8_t* a, const int8_t* a_lo, const float* sa, const int8_t* b, const float* sb, const void* bias, const void* residual,
                     const void* rscale, void* y, int m, int n, int k, int dtype, int variant, int sms, int split, int* workspace, int* counters,
                     hipStream_t stream) {
    (void)sms; (void)split; (void)workspace; (void)counters;
    if (!m || !n) return 0;
    Variant v;
    if (!variant_info(variant, v)) return -3;
    if ((v.mode == MODE_EXACT) != (a_lo != nullptr)) return -2;
    if (m < 0 || n < 0 || k <= 0 || k % 16) return -2;
    GemmArgs g = g_gemm_extra;
    g.a = a; g.a_lo = a_lo; g.sa = sa; g.b = b; g.sb = sb; g.bias = bias; g.residual = residual; g.rscale = rscale; g.y = y;
    g.sums = nullptr;
    g.m = m; g.n = n; g.k = k; g.kblocks = (k + 127) / 128;
    const bool seg = g.seg_rows > 0;
    if (seg && v.wgroup) return -4;
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

// Test entry point (no counterpart in the reference): the exact INT32 sums of every 128-element K block,
// sums[(t * N + c) * ceil(K / 128) + kb], computed by the block-mode GEMM mainloop instead of being folded.
WQ8_API int wq8_debug_block_sums(const int8_t* a, const int8_t* b, int32_t* sums, int m, int n, int k, hipStream_t stream) {
    if (!m || !n) return 0;
    if (m < 0 || n < 0 || k <= 0 || k % 16) return -2;
    GemmArgs g{};
    g.a = a; g.b = b; g.sums = sums;
    g.m = m; g.n = n; g.k = k; g.kblocks = (k + 127) / 128;
    return launch_gemm<128, 128, 2, MODE_ROW, false, DT_BF16, true, false>(g, stream);
}
