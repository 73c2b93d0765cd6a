// Shared pieces of the INT8 GEMM kernels: arguments, the XCD-aware tile raster, LDS DMA primitives and the FP32
// epilogue (bias, scales, residual, one rounding). Reference arithmetic: wgpkernels/int8/int8_gemm.cu (K8) :773-863.
#pragma once
#include "wq8_common.h"
#include <type_traits>

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
    // block scales transposed to one row per 128-element k-block (launcher-filled workspace): sa_t[kb * m + t] (block
    // mode), sb_t[kb * n + c] (weight groups)
    const float* sa_t;
    const float* sb_t;
    int m, n, k, kblocks, tiles_m, tiles_n;
    int n_first;  // first channel of the launch's tiles (a launch may cover channels [n_first, n_first + tiles_n * BN))
    int sms;  // compute units (the C-ABI's sms argument), for the choice of tile by wave count
    // row offsets of CUDA-graph-style loops (wq8_gemm_at): output / residual rows first + counter * step,
    // residual scales per span of rows, input rows in_first + counter * in_step
    const long long* counter;
    long long first, step, span, scale_step, in_first, in_step;
    // split-K tail (wq8_gemm with split != 0): with pieces > 1, workgroups [0, dp_tiles) take whole tiles and the others
    // one of `pieces` ranges of 128-element k-blocks of the last tiles; partial sums go to split_slots, arrivals are
    // counted in split_counters (one per split tile: zero on entry, left zero)
    int dp_tiles, pieces;
    uint32_t* split_slots;
    int* split_counters;
    // deep split (defer = 1, few tiles): every tile is split, each piece stores its partial sums row-major in
    // split_slots[(piece * words + word) * m * n + t * n + c] and gemm_split_finish adds them and runs the epilogue
    int defer;
    // output segments (wq8_gemm_segments): channel c belongs to segment c / seg_rows
    int seg_rows;
    const int8_t* seg_b[4];
    const float* seg_sb[4];
    const void* seg_bias[4];
    void* seg_y[4];
};

template <int N> struct IntC { static constexpr int value = N; };

// The INT8 matrix-core instruction of an MF x MF output tile (A: MF rows of 16-byte k-chunks, lane l holding row
// l % MF; B likewise for the columns): v_mfma_i32_32x32x32_i8 (16 sums per lane, row 8 (x / 4) + 4 (lane / 32) + x % 4,
// column lane % 32) or v_mfma_i32_16x16x64_i8 (4 sums per lane, row 4 (lane / 16) + x, column lane % 16). Under the
// power limit the 16 x 16 x 64 form sustains more: 3546-3551 TOPS on random operands against 2566-2810 (and 4565-4711
// against 3857-4029 on zero operands) in the same back-to-back probe on the box.
template <int MF> struct MfmaI8;
template <> struct MfmaI8<32> {
    using acc = v16i;
    using accf = v16f;
    static WQ8_DEVICE v16i run(const v4i& a, const v4i& b, const v16i& c) { return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0); }
};
template <> struct MfmaI8<16> {
    using acc = v4i;
    using accf = v4f;
    static WQ8_DEVICE v4i run(const v4i& a, const v4i& b, const v4i& c) { return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0); }
};

// The work of workgroup blockIdx.x: a tile (tm, tn) and the k-blocks [kb0, kb1) it sums, with tail = -1 for a whole
// tile, or the index of a split tile and the piece of it.
// Whole tiles: consecutive workgroups are dispatched round robin over the 8 XCDs, so workgroup b gets the virtual tile
// (b % 8) * (whole / 8) + b / 8 (each XCD a contiguous band), then a grouped raster (GROUP_M token tiles sweep the
// channel tiles) keeps the band's activation and weight panels resident in that XCD's L2. Split tiles are the last
// virtual tiles, each taken by `pieces` consecutive workgroups, piece p summing k-blocks [p KB / pieces, (p + 1) KB /
// pieces).
struct Work { int tm, tn, kb0, kb1, tail, piece; };
WQ8_DEVICE Work work_of_block(const GemmArgs& g) {
    const int tiles = g.tiles_m * g.tiles_n, b = blockIdx.x;
    const int whole = g.pieces > 1 ? g.dp_tiles : tiles;
    Work w{0, 0, 0, g.kblocks, -1, 0};
    int v;
    if (b < whole) {
        const int q = whole / 8, r = whole % 8, xcd = b % 8, idx = b / 8;
        v = xcd * q + (xcd < r ? xcd : r) + idx;
    } else {
        const int s = b - whole;
        w.tail = s / g.pieces;
        w.piece = s - w.tail * g.pieces;
        v = whole + w.tail;
        w.kb0 = w.piece * g.kblocks / g.pieces;
        w.kb1 = (w.piece + 1) * g.kblocks / g.pieces;
    }
    constexpr int GROUP_M = 4;
    const int width = GROUP_M * g.tiles_n, first = (v / width) * GROUP_M;
    const int rows = g.tiles_m - first < GROUP_M ? g.tiles_m - first : GROUP_M;
    w.tm = first + (v % width) % rows;
    w.tn = (v % width) / rows;
    // uniform over the workgroup (integer divisions by kernel arguments run on the vector unit): kept in SGPRs, so that
    // the addressing derived from them stays scalar
    w.tm = __builtin_amdgcn_readfirstlane(w.tm);
    w.tn = __builtin_amdgcn_readfirstlane(w.tn);
    w.kb0 = __builtin_amdgcn_readfirstlane(w.kb0);
    w.kb1 = __builtin_amdgcn_readfirstlane(w.kb1);
    w.tail = __builtin_amdgcn_readfirstlane(w.tail);
    w.piece = __builtin_amdgcn_readfirstlane(w.piece);
    return w;
}

// ---- LDS DMA ------------------------------------------------------------------------------------------------------
// Copies of 16 (or 4) bytes per lane from global memory straight into LDS: lane l writes lds + l * size, lds uniform
// over the wave (it goes to M0). Issued as inline assembly so that the compiler's wait-count pass does not treat later
// LDS reads as possible aliases of the copies in flight (it would wait for all of them and serialize the ring); the
// kernels wait for their copies explicitly (wait_vmcnt).
WQ8_DEVICE uint32_t lds_addr(const void* p) { return __builtin_amdgcn_readfirstlane(uint32_t(reinterpret_cast<uintptr_t>(p))); }

WQ8_DEVICE void dma16(const void* src, void* dst) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" :: "v"(src), "s"(lds_addr(dst)) : "memory", "m0");
}
WQ8_DEVICE void dma4(const void* src, void* dst) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" :: "v"(src), "s"(lds_addr(dst)) : "memory", "m0");
}

// Raw buffer resource (128-bit descriptor in SGPRs) over `bytes` bytes at `base`: loads at offsets >= bytes return zeros,
// which pads partial tiles (rows past M / N, the K tail) for free.
typedef int sgpr4 __attribute__((ext_vector_type(4)));
WQ8_DEVICE sgpr4 buffer_rsrc(const void* base, uint32_t bytes) {
    const uint64_t p = reinterpret_cast<uint64_t>(base);
    sgpr4 r;
    r[0] = __builtin_amdgcn_readfirstlane(int(uint32_t(p)));
    r[1] = __builtin_amdgcn_readfirstlane(int(uint32_t(p >> 32) & 0xffffu));  // stride 0
    r[2] = __builtin_amdgcn_readfirstlane(int(bytes));
    r[3] = 0x00020000;  // raw 32-bit data format, no swizzle
    return r;
}
WQ8_DEVICE void bdma16(sgpr4 rsrc, uint32_t voffset, void* dst) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" :: "v"(voffset), "s"(rsrc), "s"(lds_addr(dst))
                 : "memory", "m0");
}
// the same for data read once (non-temporal: streamed past the caches)
WQ8_DEVICE void bdma16_nt(sgpr4 rsrc, uint32_t voffset, void* dst) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen nt lds" :: "v"(voffset), "s"(rsrc), "s"(lds_addr(dst))
                 : "memory", "m0");
}
WQ8_DEVICE void bdma4(sgpr4 rsrc, uint32_t voffset, void* dst) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dword %0, %1, 0 offen lds" :: "v"(voffset), "s"(rsrc), "s"(lds_addr(dst))
                 : "memory", "m0");
}

// s_waitcnt on one counter (gfx9 encoding: vmcnt[3:0] | expcnt << 4 | lgkmcnt << 8 | vmcnt[5:4] << 14)
template <int N> WQ8_DEVICE void wait_vmcnt() { __builtin_amdgcn_s_waitcnt((N & 15) | 0x70 | 0xF00 | ((N >> 4) << 14)); }
WQ8_DEVICE void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Split tiles: every piece stores its partial sums (NV words per thread, value(v): FP32 bits of the folded accumulators,
// or the INT32 sums) in a slot of its own, then counts its arrival on the tile's counter. split_arrive returns true in
// the last piece to arrive (which leaves the counter at zero) and false in the others (their workgroup is done). The
// last piece then reads every piece's word v back with split_sum, added in piece order (FP32: ((p0 + p1) + p2) + p3,
// the same order whichever piece arrives last; INT32: exact) while its epilogue runs: its own accumulators are dead by
// then, which keeps the mainloop's registers as they are. The partial sums are written and read at agent scope, through
// to the device's coherence point, so no L2 writeback or invalidation is needed: each thread's stores have completed
// (vmcnt 0) before the barrier that precedes the count, and the last piece's loads are issued after it has read it.
template <int NV, int THREADS, class Get>
WQ8_DEVICE bool split_arrive(const GemmArgs& g, const Work& w, Get value) {
    __shared__ int last;
    const int tid = threadIdx.x;
    uint32_t* own = g.split_slots + (int64_t(w.tail) * g.pieces + w.piece) * (int64_t(NV) * THREADS) + tid;
#pragma unroll
    for (int v = 0; v < NV; ++v) __hip_atomic_store(own + v * THREADS, value(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    wait_vmcnt<0>();
    __syncthreads();
    if (tid == 0) {
        last = __hip_atomic_fetch_add(g.split_counters + w.tail, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == g.pieces - 1;
        if (last) __hip_atomic_store(g.split_counters + w.tail, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    return last;
}
template <int NV, int THREADS, bool FP>
WQ8_DEVICE uint32_t split_sum(const GemmArgs& g, const Work& w, int v) {
    const uint32_t* slot = g.split_slots + int64_t(w.tail) * g.pieces * (int64_t(NV) * THREADS) + v * THREADS + threadIdx.x;
    uint32_t sum = __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int p = 1; p < 4; ++p) {
        if (p >= g.pieces) break;
        const uint32_t x = __hip_atomic_load(slot + int64_t(p) * NV * THREADS, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if constexpr (FP) sum = __builtin_bit_cast(uint32_t, __builtin_bit_cast(float, sum) + __builtin_bit_cast(float, x));
        else sum = uint32_t(int32_t(sum) + int32_t(x));
    }
    return sum;
}

// ---- epilogue -----------------------------------------------------------------------------------------------------
// Accumulator layout (the weights as the MFMA's operand A, MfmaI8<MF>): element x of a lane's MF x MF tile is token
// lane % MF and channel 8 (x / 4) + 4 (lane / 32) + x % 4 (MF 32) or 4 (lane / 16) + x (MF 16). value(i, j, x) gives the
// FP32 pre-scale value v of channel fragment i, token fragment j; the output is y = fmaf(v * row_scale, col_scale, bias),
// then y = fmaf(y, rscale, residual), rounded once (K8:836-863).
//
// The wave's WM x WN output block goes through its own LDS area (rows of WN values padded by 16 bytes): the residual is
// read into it with coalesced 16-byte loads, every lane combines its values there, and whole rows leave with coalesced
// 16-byte stores (a 32x32 accumulator tile alone would store 8-byte pieces of 32 different rows). `stage` must hold
// WM * (WN * 2 + 16) bytes for this wave and be free (the caller synchronizes with the mainloop).
template <int WN, int WM> constexpr int epilogue_stage_bytes() { return WM * (WN * 2 + 16); }

// Per-tile epilogue parameters, parked in LDS once the mainloop is done: FP32 weight scales, raw 16-bit bias and residual
// scales of the tile's BN channels, FP32 row scales of its BM tokens. Thread `tid` loads channel tid and token tid at
// the start of the tile (the loads' latency hides under the mainloop); channels and tokens past N / M hold zeros.
template <int DT, int MODE, bool WG, bool SEG, int BM, int BN> struct EpilogueParams {
    using raw = typename Elem<DT>::raw;
    static constexpr int BYTES = BN * 8 + BM * 4;
    float sb = 0.0f, sa = 0.0f;
    raw bias = raw(0), rs = raw(0);

    WQ8_DEVICE void load(const GemmArgs& g, int m0, int n0, const float* sa_rows, int tid) {
        const int c = n0 + tid, t = m0 + tid;
        if (tid < BN && c < g.n) {
            if constexpr (SEG) {
                const int s = c / g.seg_rows, cc = c - s * g.seg_rows;
                sb = g.seg_sb[s][cc];
                if (g.seg_bias[s]) bias = static_cast<const raw*>(g.seg_bias[s])[cc];
            } else {
                if constexpr (!WG) sb = g.sb[c];
                if (g.bias) bias = static_cast<const raw*>(g.bias)[c];
                if (g.rscale && !g.span) rs = static_cast<const raw*>(g.rscale)[c];
            }
        }
        if constexpr (MODE != MODE_BLOCK)
            if (tid < BM && t < g.m) sa = sa_rows[t];
    }
    WQ8_DEVICE void park(uint8_t* lds, int tid) const {
        if (tid < BN) {
            reinterpret_cast<float*>(lds)[tid] = sb;
            reinterpret_cast<raw*>(lds + BN * 4)[tid] = bias;
            reinterpret_cast<raw*>(lds + BN * 6)[tid] = rs;
        }
        if (tid < BM) reinterpret_cast<float*>(lds + BN * 8)[tid] = sa;
    }
};

// Deep split: a piece's pre-epilogue values of the wave's WM x WN block, word(i, j, x, h) for element x of fragment tile
// (i, j) (h: 0, or 1 for the lo sum of the exact mode), stored row-major as WORDS planes of m x n words per piece (16-byte
// stores of the lane's 4 consecutive channels where they lie inside N and N % 4 == 0). Element mapping as in
// gemm_epilogue.
template <int FN, int FM, int WN, int WM, int MF, int WORDS, class Word>
WQ8_DEVICE void defer_store(const GemmArgs& g, int m0, int n0, int wn, int wm, int piece, Word word) {
    const int lane = threadIdx.x & 63, frag_row = lane & (MF - 1);
    const int m = g.m, n = g.n;
    const int64_t plane = int64_t(m) * n;
    uint32_t* base = g.split_slots + int64_t(piece) * WORDS * plane;
    const int t_base = m0 + wm * WM, c_base = n0 + wn * WN;
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int gi = 0; gi < MF * MF / 256; ++gi) {
            const int c0 = c_base + i * MF + (MF == 32 ? 8 * gi + 4 * (lane >> 5) : 4 * (lane >> 4));
#pragma unroll
            for (int j = 0; j < FM; ++j) {
                const int t = t_base + j * MF + frag_row;
                if (t >= m || c0 >= n) continue;
#pragma unroll
                for (int h = 0; h < WORDS; ++h) {
                    u32x4 v;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = word(i, j, 4 * gi + e, h);
                    uint32_t* dst = base + h * plane + int64_t(t) * n + c0;
                    if (c0 + 4 <= n && n % 4 == 0) {
                        __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(dst));
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (c0 + e < n) dst[e] = v[e];
                    }
                }
            }
        }
}

// The deep split's second launch: one thread per 4 consecutive output elements (16-byte loads of the planes when n % 4
// == 0) adds the pieces' partial sums in piece order (FP32: ((p0 + p1) + p2) + ...; INT32: exact) and applies
// gemm_epilogue's arithmetic to the sum: value x row scale (token scale, except in block mode) x channel scale (none
// with weight groups) + bias, then x residual scale + residual, rounded once to the output type. FP: FP32 folds (block,
// exact+g); WORDS 2: the exact mode's hi and lo sums.
template <int DT, int MODE, bool WG, bool FP, int WORDS>
__global__ void __launch_bounds__(256) gemm_split_finish(GemmArgs g) {
    using raw = typename Elem<DT>::raw;
    constexpr int V = 4;
    const int m = g.m, n = g.n;
    const int64_t plane = int64_t(m) * n, e0 = (int64_t(blockIdx.x) * 256 + threadIdx.x) * V;
    if (e0 >= plane) return;
    const bool vec = (n % V) == 0;  // then e0 .. e0 + 3 lie in one row, 16-byte aligned in every plane
    const int pieces = g.pieces;
    // the 4 elements' words of plane q (piece p, word h: q = p * WORDS + h)
    auto load = [&](int q, uint32_t (&w)[V]) {
        const uint32_t* src = g.split_slots + int64_t(q) * plane + e0;
        if (vec) {
            const u32x4 x = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
#pragma unroll
            for (int j = 0; j < V; ++j) w[j] = x[j];
        } else {
#pragma unroll
            for (int j = 0; j < V; ++j) w[j] = e0 + j < plane ? __builtin_nontemporal_load(src + j) : 0u;
        }
    };
    float value[V];
    if constexpr (FP) {
        float v[V];
        for (int p0 = 0; p0 < pieces; p0 += 8) {
            uint32_t part[8][V];
#pragma unroll
            for (int q = 0; q < 8; ++q)
                if (p0 + q < pieces) load(p0 + q, part[q]);
#pragma unroll
            for (int q = 0; q < 8; ++q)
#pragma unroll
                for (int j = 0; j < V; ++j)
                    if (p0 + q < pieces) v[j] = p0 + q == 0 ? __builtin_bit_cast(float, part[q][j]) : v[j] + __builtin_bit_cast(float, part[q][j]);
        }
#pragma unroll
        for (int j = 0; j < V; ++j) value[j] = v[j];
    } else {
        int32_t s[WORDS][V] = {};
        for (int p0 = 0; p0 < pieces; p0 += 8) {
#pragma unroll
            for (int h = 0; h < WORDS; ++h) {
                uint32_t part[8][V];
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    if (p0 + q < pieces) load((p0 + q) * WORDS + h, part[q]);
#pragma unroll
                for (int q = 0; q < 8; ++q)
#pragma unroll
                    for (int j = 0; j < V; ++j)
                        if (p0 + q < pieces) s[h][j] += int32_t(part[q][j]);
            }
        }
#pragma unroll
        for (int j = 0; j < V; ++j) {
            if constexpr (WORDS == 2) value[j] = __builtin_fmaf(float(s[1][j]), 1.0f / 254.0f, float(s[0][j]));
            else value[j] = float(s[0][j]);
        }
    }
    const long long shift = g.counter ? g.first + __ldg(g.counter) * g.step : 0;
    const long long in_shift = g.counter && (g.in_first || g.in_step) ? g.in_first + __ldg(g.counter) * g.in_step : 0;
    // (32-bit division when the plane allows: the 64-bit one is a long software sequence)
    int t = plane < (int64_t(1) << 31) ? int(uint32_t(e0) / uint32_t(n)) : int(e0 / n), c = int(e0 - int64_t(t) * n);
    static_assert(sizeof(raw) == 2, "16-bit outputs");
    const bool vec_out = vec && (reinterpret_cast<uintptr_t>(g.y) & 7) == 0;
    // channel scales and bias of the 4 channels: one 16-byte and one 8-byte load when they lie in one row and aligned
    float cs4[V], bv4[V];
    const bool vec_sb = !WG && vec && (reinterpret_cast<uintptr_t>(g.sb) & 15) == 0;
    const bool vec_bias = g.bias && vec && (reinterpret_cast<uintptr_t>(g.bias) & 7) == 0;
    if (vec_sb) {
        const v4f x = *reinterpret_cast<const v4f*>(g.sb + c);
#pragma unroll
        for (int j = 0; j < V; ++j) cs4[j] = x[j];
    }
    if (vec_bias) {
        const u32x2 x = *reinterpret_cast<const u32x2*>(static_cast<const raw*>(g.bias) + c);
#pragma unroll
        for (int j = 0; j < V; ++j) bv4[j] = Elem<DT>::to_f(raw(x[j / 2] >> (16 * (j % 2))));
    }
    raw o16[V];
    int64_t out0 = 0;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        if (e0 + j >= plane) break;
        const float row_scale = MODE == MODE_BLOCK ? 1.0f : g.sa[in_shift + t];
        const float cs = WG ? 1.0f : vec_sb ? cs4[j] : g.sb[c];
        const float bv = vec_bias ? bv4[j] : g.bias ? Elem<DT>::to_f(static_cast<const raw*>(g.bias)[c]) : 0.0f;
        float o = __builtin_fmaf(value[j] * row_scale, cs, bv);
        const int64_t out = (shift + t) * int64_t(n) + c;
        if (j == 0) out0 = out;
        if (g.residual) {
            float rs = 1.0f;
            if (g.rscale && g.span) rs = Elem<DT>::to_f(static_cast<const raw*>(g.rscale)[(shift + t) / g.span * g.scale_step + c]);
            else if (g.rscale) rs = Elem<DT>::to_f(static_cast<const raw*>(g.rscale)[c]);
            o = __builtin_fmaf(o, rs, Elem<DT>::to_f(static_cast<const raw*>(g.residual)[out]));
        }
        o16[j] = Elem<DT>::from_f(o);
        if (!vec_out) static_cast<raw*>(g.y)[out] = o16[j];
        if (++c == n) {
            c = 0;
            ++t;
        }
    }
    if (vec_out)  // the 4 outputs of one row in one 8-byte store
        *reinterpret_cast<u32x2*>(static_cast<raw*>(g.y) + out0) =
            u32x2{uint32_t(o16[0]) | uint32_t(o16[1]) << 16, uint32_t(o16[2]) | uint32_t(o16[3]) << 16};
}

// params: the tile's EpilogueParams<..., BM, BN> in LDS
template <int DT, int MODE, bool WG, bool SEG, int BM, int BN, int FN, int FM, int WN, int WM, int MF = 32, class Value>
WQ8_DEVICE void gemm_epilogue(const GemmArgs& g, int m0, int n0, int wn, int wm, const uint8_t* __restrict__ params, uint8_t* __restrict__ stage,
                              Value value) {
    using raw = typename Elem<DT>::raw;
    static_assert(sizeof(raw) == 2, "16-bit outputs");
    constexpr int LD = WN * 2 + 16;          // staged row bytes
    constexpr int CHUNKS = WN / 8;           // 16-byte chunks per row
    constexpr int ROWS_PER_PASS = 64 / CHUNKS;  // lanes past ROWS_PER_PASS * CHUNKS idle when CHUNKS does not divide 64
    constexpr int PASSES = (WM + ROWS_PER_PASS - 1) / ROWS_PER_PASS;
    static_assert(CHUNKS <= 64, "epilogue lanes");
    const int lane = threadIdx.x & 63, frag_row = lane & (MF - 1);
    const int m = g.m, n = g.n;
    const long long shift = g.counter ? g.first + __ldg(g.counter) * g.step : 0;
    const int t_base = m0 + wm * WM, c_base = n0 + wn * WN;  // first token / channel of the wave's block
    const bool full_cols = c_base + WN <= n && (SEG ? (g.seg_rows % 8) == 0 : (n % 8) == 0);
    const float* p_sb = reinterpret_cast<const float*>(params) + wn * WN;
    const raw* p_bias = reinterpret_cast<const raw*>(params + BN * 4) + wn * WN;
    const raw* p_rs = reinterpret_cast<const raw*>(params + BN * 6) + wn * WN;
    const float* p_sa = reinterpret_cast<const float*>(params + BN * 8) + wm * WM;
    // output row pointer and its channel offset for a chunk of 8 channels starting at column c (SEG: per segment)
    auto out_ptr = [&](int t, int c) -> raw* {
        if constexpr (SEG) {
            const int s = c / g.seg_rows;
            return static_cast<raw*>(g.seg_y[s]) + int64_t(t) * g.seg_rows + (c - s * g.seg_rows);
        } else {
            return static_cast<raw*>(g.y) + (shift + t) * int64_t(n) + c;
        }
    };
    const raw* residual = static_cast<const raw*>(g.residual);
    // The uniform conditions (residual present, residual scales per span, whole 16-byte column chunks) are resolved once
    // here so that every unrolled loop below is straight-line code the scheduler can interleave freely.
    // 1. residual block -> LDS (coalesced)
    auto load_residual = [&](auto full_tag) {
        constexpr bool FULL = decltype(full_tag)::value;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int r = p * ROWS_PER_PASS + lane / CHUNKS, cc = (lane % CHUNKS) * 8;
            if (r >= WM || lane >= ROWS_PER_PASS * CHUNKS) continue;
            const int t = t_base + r, c = c_base + cc;
            u32x4 v = {0, 0, 0, 0};
            if (t < m) {
                const raw* src = residual + (shift + t) * int64_t(n) + c;
                if constexpr (FULL) {
                    v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));  // read once (+1.0-1.3% with a residual)
                } else {
                    raw e[8];
#pragma unroll
                    for (int q = 0; q < 8; ++q) e[q] = c + q < n ? src[q] : raw(0);
                    v = __builtin_bit_cast(u32x4, e);
                }
            }
            *reinterpret_cast<u32x4*>(stage + r * LD + cc * 2) = v;
        }
    };
    // 2. combine in registers, write back to LDS
    auto combine = [&](auto res_tag, auto span_tag) {
        constexpr bool RES = decltype(res_tag)::value, SPAN = decltype(span_tag)::value;
        const bool col_rs = RES && !SPAN && g.rscale;  // residual scales per channel
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int gi = 0; gi < MF * MF / 256; ++gi) {
                // local column of the lane's 4 channels of group gi (elements 4 gi .. 4 gi + 3)
                const int col = i * MF + (MF == 32 ? 8 * gi + 4 * (lane >> 5) : 4 * (lane >> 4));
                const int c0 = c_base + col;
                float cs[4], bv[4], rs[4];
                {
                    const v4f sb4 = *reinterpret_cast<const v4f*>(p_sb + col);
                    const u32x2 b4 = *reinterpret_cast<const u32x2*>(p_bias + col), r4 = *reinterpret_cast<const u32x2*>(p_rs + col);
                    const raw* bb = reinterpret_cast<const raw*>(&b4);
                    const raw* rr = reinterpret_cast<const raw*>(&r4);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        cs[e] = WG ? 1.0f : sb4[e];
                        bv[e] = Elem<DT>::to_f(bb[e]);
                        rs[e] = col_rs ? Elem<DT>::to_f(rr[e]) : 1.0f;
                    }
                }
#pragma unroll
                for (int j = 0; j < FM; ++j) {
                    const int r = j * MF + frag_row, t = t_base + r;
                    const float row_scale = MODE == MODE_BLOCK ? 1.0f : p_sa[r];
                    if constexpr (SPAN) {
                        // residual scales per span of output rows (row-offset entry point): read per token
                        const raw* rs_row = static_cast<const raw*>(g.rscale) + (shift + t) / g.span * g.scale_step;
#pragma unroll
                        for (int e = 0; e < 4; ++e) rs[e] = Elem<DT>::to_f(rs_row[c0 + e < n ? c0 + e : n - 1]);
                    }
                    raw* cell = reinterpret_cast<raw*>(stage + r * LD + col * 2);
                    raw res4[4];
                    if constexpr (RES) *reinterpret_cast<u32x2*>(res4) = *reinterpret_cast<const u32x2*>(cell);
                    raw o4[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float o = __builtin_fmaf(value(i, j, 4 * gi + e) * row_scale, cs[e], bv[e]);
                        if constexpr (RES) o = __builtin_fmaf(o, rs[e], Elem<DT>::to_f(res4[e]));
                        o4[e] = Elem<DT>::from_f(o);
                    }
                    *reinterpret_cast<u32x2*>(cell) = *reinterpret_cast<const u32x2*>(o4);
                }
            }
    };
    // 3. rows -> global (coalesced 16-byte stores)
    auto store_rows = [&](auto full_tag) {
        constexpr bool FULL = decltype(full_tag)::value;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int r = p * ROWS_PER_PASS + lane / CHUNKS, cc = (lane % CHUNKS) * 8;
            if (r >= WM || lane >= ROWS_PER_PASS * CHUNKS) continue;
            const int t = t_base + r, c = c_base + cc;
            if (t >= m || c >= n) continue;
            const u32x4 v = *reinterpret_cast<const u32x4*>(stage + r * LD + cc * 2);
            if constexpr (FULL) {
                // Y is written once and not read back by this kernel: streamed past L2 rather than left there to evict
                // the operands' lines (0.5% block, 0.8% exact, 1.4% row at the headline shape)
                __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(out_ptr(t, c)));
            } else {
                const raw* e = reinterpret_cast<const raw*>(&v);
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    if (c + q < n) *out_ptr(t, c + q) = e[q];
            }
        }
    };
    using T = std::true_type;
    using F = std::false_type;
    if (residual) {
        if (full_cols) load_residual(T{});
        else load_residual(F{});
        if (g.rscale && g.span) combine(T{}, T{});
        else combine(T{}, F{});
    } else {
        combine(F{}, F{});
    }
    if (full_cols) store_rows(T{});
    else store_rows(F{});
}

}  // namespace wq8
