// Few-token paths on gfx950 (unquantized activations, exact INT8 weights, FP32 accumulation):
//   lines (1-4 tokens)  VALU GEMV: each wave streams its weight rows, every lane loading 16 contiguous bytes per row
//                       (one 1 KiB line per row and load instruction), exact INT8 -> BF16 / FP16 weight pairs,
//                       v_dot2c_f32 products into FP32 accumulators, wave64 butterfly reduction. With K <= 16 KiB every
//                       load of a wave is issued before its first product and the activations are staged in LDS per
//                       workgroup (gemv_linesx); 3-4 tokens with K % 16 == 0 take the products on matrix cores instead
//                       (gemv_quads, v_mfma_f32_4x4x4, persistent workgroups); otherwise a looped kernel (gemv_lines).
//   small (<= 32)       matrix cores: weights and activations DMA'd to LDS, INT8 weights converted exactly to BF16 /
//                       FP16 in registers feed v_mfma_f32_16x16x32_{bf16,f16} (16 channels x 16 tokens x 32 k).
//                       Above 32 weight rows per CU, or for weights of 48 MiB or more, one workgroup per CU streams an
//                       equal share of 33-64 rows over K or a part of it (w8_rows); otherwise split-K across many
//                       workgroups (w8_small). FP32 partial slots of K splits are added in order by a second kernel
//                       (small_reduce).
// Reference: wgpkernels/int8/int8_gemm.cu (K8) :1039-1151 (w8a16_small), :1768-1810 (gemv_lines), :1684-1759 and
// :1833-1858 (launch / C ABI).
#include "gemm_common.h"
#include "wq8_abi.h"

namespace wq8 {

struct FewArgs {
    const void* x;
    int64_t ldx;
    const int8_t* w;
    const float* sw;
    const void* bias;
    const void* residual;
    const void* rscale;
    void* y;
    int m, n, k;
    float* slots;   // small: split partials
    int* counters;  // unused (the C ABI keeps the argument)
    int splits;
};

// Bytes of the activation rows the kernels read through a buffer descriptor: rows 0 .. m - 1 at pitch ldx, k values each
// (a one-row input's pitch can be anything, e.g. 1 for a transposed (K, 1) column), at least m * ldx as the row loops
// address them. Loads past it read zeros.
WQ8_DEVICE uint32_t x_span_bytes(const FewArgs& p) {
    const int64_t rows = int64_t(p.m - 1) * p.ldx + p.k, pitched = int64_t(p.m) * p.ldx;
    return uint32_t((rows > pitched ? rows : pitched) * 2);
}
static bool x_span_fits(const FewArgs& p) {
    const int64_t rows = int64_t(p.m - 1) * p.ldx + p.k, pitched = int64_t(p.m) * p.ldx;
    return (rows > pitched ? rows : pitched) * 2 < (int64_t(1) << 31);
}

// y = fmaf(acc, sw, bias), then fmaf(y, rscale, residual), one rounding (K8:1803-1806, K8:1146-1147)
template <int DT>
WQ8_DEVICE void store_out(const FewArgs& p, int t, int c, float acc) {
    using raw = typename Elem<DT>::raw;
    float v = __builtin_fmaf(acc, p.sw[c], p.bias ? Elem<DT>::to_f(static_cast<const raw*>(p.bias)[c]) : 0.0f);
    if (p.residual) {
        const float rs = p.rscale ? Elem<DT>::to_f(static_cast<const raw*>(p.rscale)[c]) : 1.0f;
        v = __builtin_fmaf(v, rs, Elem<DT>::to_f(static_cast<const raw*>(p.residual)[int64_t(t) * p.n + c]));
    }
    static_cast<raw*>(p.y)[int64_t(t) * p.n + c] = Elem<DT>::from_f(v);
}

// ---------------------------------------------------------------------------------------------------------------
// lines
// ---------------------------------------------------------------------------------------------------------------
// Pairs of 16-bit values against pairs of INT8 weights: the weight word's 4 bytes become 2 exact BF16 / FP16 pairs
// (sign-extending byte converts, then one pack per pair), and v_dot2c_f32_{bf16,f16} adds a pair's two exact products
// to an FP32 accumulator (1.5 VALU ops per weight for the conversion, 0.5 per weight and token for the products; the
// activations are used as loaded).
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
template <int DT> struct Dot2;
template <> struct Dot2<DT_BF16> {
    static WQ8_DEVICE uint32_t pack(float a, float b) {
        return __builtin_bit_cast(uint32_t, bf16x2{static_cast<__bf16>(a), static_cast<__bf16>(b)});
    }
    static WQ8_DEVICE float dot(uint32_t w, uint32_t x, float acc) {
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), __builtin_bit_cast(bf16x2, x), acc, false);
    }
};
template <> struct Dot2<DT_F16> {
    static WQ8_DEVICE uint32_t pack(float a, float b) {
        return __builtin_bit_cast(uint32_t, f16x2{static_cast<_Float16>(a), static_cast<_Float16>(b)});
    }
    static WQ8_DEVICE float dot(uint32_t w, uint32_t x, float acc) {
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), __builtin_bit_cast(f16x2, x), acc, false);
    }
};
// weight pairs (bytes 0-1, bytes 2-3) of one word (|w| <= 127: exact in BF16 and FP16)
template <int DT> WQ8_DEVICE void weight_pairs(uint32_t word, uint32_t& p01, uint32_t& p23) {
    p01 = Dot2<DT>::pack(float(int8_t(word)), float(int8_t(word >> 8)));
    p23 = Dot2<DT>::pack(float(int8_t(word >> 16)), float(int8_t(word >> 24)));
}

constexpr int LINE_CH = 4;  // weight rows per wave

template <int DT, int ROWS>
__global__ void __launch_bounds__(256) gemv_lines(FewArgs p) {
    using raw = typename Elem<DT>::raw;
    const int lane = threadIdx.x & 63;
    const int group = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int ch0 = group * LINE_CH;
    if (ch0 >= p.n) return;
    const int k = p.k, k16 = k & ~15;
    const raw* x = static_cast<const raw*>(p.x);
    const int8_t* wrow[LINE_CH];
#pragma unroll
    for (int c = 0; c < LINE_CH; ++c) wrow[c] = p.w + int64_t(ch0 + c < p.n ? ch0 + c : p.n - 1) * k;
    float acc[LINE_CH][ROWS][2];
#pragma unroll
    for (int c = 0; c < LINE_CH; ++c)
#pragma unroll
        for (int r = 0; r < ROWS; ++r) acc[c][r][0] = acc[c][r][1] = 0.0f;

#pragma unroll 2
    for (int kk = lane * 16; kk < k16; kk += 1024) {
        u32x4 wv[LINE_CH];
#pragma unroll
        for (int c = 0; c < LINE_CH; ++c) wv[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[c] + kk));
        if constexpr (DT == DT_F32) {
            float xf[ROWS][16];
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                load8<DT>(x + int64_t(r) * p.ldx + kk, xf[r], true);
                load8<DT>(x + int64_t(r) * p.ldx + kk + 8, xf[r] + 8, true);
            }
#pragma unroll
            for (int c = 0; c < LINE_CH; ++c)
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float wf = float(int8_t(wv[c][q] >> (8 * e)));
#pragma unroll
                        for (int r = 0; r < ROWS; ++r) acc[c][r][e & 1] = __builtin_fmaf(wf, xf[r][4 * q + e], acc[c][r][e & 1]);
                    }
        } else {
            u32x4 xv[ROWS][2];
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                xv[r][0] = *reinterpret_cast<const u32x4*>(x + int64_t(r) * p.ldx + kk);
                xv[r][1] = *reinterpret_cast<const u32x4*>(x + int64_t(r) * p.ldx + kk + 8);
            }
#pragma unroll
            for (int c = 0; c < LINE_CH; ++c)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    uint32_t p01, p23;
                    weight_pairs<DT>(wv[c][q], p01, p23);
#pragma unroll
                    for (int r = 0; r < ROWS; ++r) {
                        const u32x4& xq = xv[r][q >> 1];
                        acc[c][r][0] = Dot2<DT>::dot(p01, xq[2 * (q & 1)], acc[c][r][0]);
                        acc[c][r][1] = Dot2<DT>::dot(p23, xq[2 * (q & 1) + 1], acc[c][r][1]);
                    }
                }
        }
    }
    // K % 16 tail: 4-byte pieces (K is a multiple of 4)
    for (int kk = k16 + 4 * lane; kk < k; kk += 256) {
#pragma unroll
        for (int c = 0; c < LINE_CH; ++c) {
            const uint32_t word = *reinterpret_cast<const uint32_t*>(wrow[c] + kk);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float wf = float(int8_t(word >> (8 * e)));
#pragma unroll
                for (int r = 0; r < ROWS; ++r)
                    acc[c][r][e & 1] = __builtin_fmaf(wf, Elem<DT>::to_f(x[int64_t(r) * p.ldx + kk + e]), acc[c][r][e & 1]);
            }
        }
    }
#pragma unroll
    for (int c = 0; c < LINE_CH; ++c)
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            const float s = wave_sum(acc[c][r][0] + acc[c][r][1]);
            if (lane == 0 && ch0 + c < p.n) store_out<DT>(p, r, ch0 + c, s);
        }
}

// 1-4 tokens, 16-bit activations, K <= 16 KiB with MT * NIT <= LINEX_LINES: a wave takes CH weight rows and issues
// every load of them (NIT 1 KiB lines per row, 16-byte nontemporal loads) before its first product, so that the whole
// weight matrix is requested from HBM at once instead of a few lines per wave and round trip; the grid's many short
// waves keep every CU's loads in flight. Exact INT8 -> 16-bit weight pairs, v_dot2c products, wave64 butterfly. The
// activations of the MT tokens are staged once per workgroup in LDS (buffer_load ... lds): a wave holds only its weight
// lines, and the activation row is read from L2 once per workgroup rather than once per wave. Line it of token t is
// stored as two 1 KiB halves: half h holds, at 16 l, values 16 l + 8 h .. 16 l + 8 h + 7 of the line, so lane l's two
// 16-byte reads are contiguous across the wave.
constexpr int LINEX_LINES = 32;  // staged 2 KiB lines per workgroup (64 KiB of LDS)
template <int DT, int CH, int NIT, int MT, int WPG = 4>
__global__ void __launch_bounds__(64 * WPG) gemv_linesx(FewArgs p) {
    using raw = typename Elem<DT>::raw;
    static_assert(sizeof(raw) == 2, "16-bit activations");
    static_assert(MT * NIT <= LINEX_LINES, "staged lines");
    __shared__ __attribute__((aligned(1024))) uint8_t xs[MT * NIT * 2048];
    constexpr uint32_t OUT_OF_RANGE = 0x80000000u;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ch0 = (blockIdx.x * WPG + wave) * CH;  // waves past N still stage activations and meet the barrier
    const int k = p.k, k16 = k & ~15, n = p.n;
    const raw* x = static_cast<const raw*>(p.x);
    // activations -> LDS: copy q = (token, line, half), spread over the workgroup's WPG waves; zeros past the row
    const sgpr4 rx = buffer_rsrc(p.x, x_span_bytes(p));
#pragma unroll
    for (int q = wave; q < MT * NIT * 2; q += WPG) {
        const int t = q / (2 * NIT), it = (q / 2) % NIT, h = q % 2;
        const int kk = it * 1024 + lane * 16;
        bdma16(rx, t < p.m && kk < k16 ? (uint32_t(t) * uint32_t(p.ldx) + uint32_t(kk + 8 * h)) * 2u : OUT_OF_RANGE, xs + q * 1024);
    }
    const int8_t* wrow[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) wrow[c] = p.w + int64_t(ch0 + c < n ? ch0 + c : n - 1) * k;
    u32x4 wv[NIT][CH];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int kk = it * 1024 + lane * 16, kc = kk < k16 ? kk : 0;
#pragma unroll
        for (int c = 0; c < CH; ++c) wv[it][c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[c] + kc));
    }
    __builtin_amdgcn_sched_barrier(0);  // every load is in flight before the first product
    wait_vmcnt<NIT * CH>();  // the activation copies, issued first, have landed (loads complete in issue order)
    __syncthreads();         // ... for every wave of the workgroup
    float acc[CH][MT][2];
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[c][t][0] = acc[c][t][1] = 0.0f;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const bool valid = it * 1024 + lane * 16 < k16;
        u32x4 xv[MT][2];
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int h = 0; h < 2; ++h) xv[t][h] = *reinterpret_cast<const u32x4*>(xs + ((t * NIT + it) * 2 + h) * 1024 + lane * 16);
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint32_t p01, p23;
                weight_pairs<DT>(valid ? wv[it][c][q] : 0u, p01, p23);
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    acc[c][t][0] = Dot2<DT>::dot(p01, xv[t][q >> 1][2 * (q & 1)], acc[c][t][0]);
                    acc[c][t][1] = Dot2<DT>::dot(p23, xv[t][q >> 1][2 * (q & 1) + 1], acc[c][t][1]);
                }
            }
    }
    if (ch0 >= n) return;
    // K % 16 tail: 4-byte pieces (K is a multiple of 4)
    for (int kk = k16 + 4 * lane; kk < k; kk += 256) {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const uint32_t word = *reinterpret_cast<const uint32_t*>(wrow[c] + kk);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float wf = float(int8_t(word >> (8 * e)));
#pragma unroll
                for (int t = 0; t < MT; ++t)
                    if (t < p.m) acc[c][t][e & 1] = __builtin_fmaf(wf, Elem<DT>::to_f(x[int64_t(t) * p.ldx + kk + e]), acc[c][t][e & 1]);
            }
        }
    }
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const float s = wave_sum(acc[c][t][0] + acc[c][t][1]);
            if (lane == 0 && ch0 + c < n && t < p.m) store_out<DT>(p, t, ch0 + c, s);
        }
}

template <int DT, int CH, int NIT, int MT> static int launch_linesx(FewArgs& p, hipStream_t stream) {
    const int groups = (p.n + CH - 1) / CH;
    // 8 waves per workgroup (the staged activations shared by twice the rows) at N < 8192 for 2-4 tokens, and for one
    // token with rows up to 8 KiB: measured 10% faster at 3-4 tokens, K = N = 5120, 9% at 2 tokens, K = 13824, N = 5120
    // and 5% at one token, K = N = 5120; slower at N = 13824 and for one token at K = 13824
    if (p.n < 8192 && (MT >= 2 || NIT <= 8)) gemv_linesx<DT, CH, NIT, MT, 8><<<(groups + 7) / 8, 512, 0, stream>>>(p);
    else gemv_linesx<DT, CH, NIT, MT><<<(groups + 3) / 4, 256, 0, stream>>>(p);
    return int(hipGetLastError());
}

// two rows per wave when there are many rows and few lines (fewer, fuller waves), else one
template <int DT, int MT, int NIT = 1> static int dispatch_linesx(FewArgs& p, int nit, hipStream_t stream) {
    if constexpr (NIT > 16 || MT * NIT > LINEX_LINES) {
        return -2;
    } else {
        if (nit == NIT) return p.n >= 8192 && NIT <= 8 ? launch_linesx<DT, 2, NIT, MT>(p, stream) : launch_linesx<DT, 1, NIT, MT>(p, stream);
        return dispatch_linesx<DT, MT, NIT + 1>(p, nit, stream);
    }
}

// quads: 3-4 tokens on matrix cores. v_mfma_f32_4x4x4_{bf16,f16} computes 16 independent 4 x 4 products over 4 k each.
// A wave takes a quad of 4 weight rows; its 16-byte load puts row i, k = k0 + 16 b .. k0 + 16 b + 15 in lane 4 b + i (4
// rows x 256 contiguous bytes per load), whose 4 words become the A operands of 4 products (exact INT8 -> 16-bit
// conversion, 1.5 VALU ops per weight), and lane 4 b + j holds the matching activations of token j as B, so that block b
// accumulates row i x token j over its slices of k and the tokens cost no VALU (v_dot2c: 0.5 ops per weight and token).
// The workgroup's CG x S waves take CG quads and S consecutive ranges of NL chunks of 256 k. The workgroup is persistent:
// workgroup b of G takes quad groups b, b + G, ..., and the next group's weight loads are in flight while the current
// group's products run; the activations (4 tokens, zeros past M and K) are staged once, in LDS, in lane order (chunk c,
// half h: lane 4 b + j's 16 bytes are x[j][256 c + 16 b + 8 h ..]). The 16 block partials of a wave are added by two DPP
// rotations within each 16-lane row, then the 4 rows and the S ranges through LDS (two slots, alternating by group).
template <int DT> struct Mfma4;
template <> struct Mfma4<DT_BF16> {
    typedef short op __attribute__((ext_vector_type(4)));
    static WQ8_DEVICE v4f run(op a, op b, v4f c) { return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a, b, c, 0, 0, 0); }
};
template <> struct Mfma4<DT_F16> {
    typedef _Float16 op __attribute__((ext_vector_type(4)));
    static WQ8_DEVICE v4f run(op a, op b, v4f c) { return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 0, 0, 0); }
};

template <int DT, int NL, int CG, int S>
__global__ void __launch_bounds__(64 * CG * S) gemv_quads(FewArgs p, int groups) {
    using op = typename Mfma4<DT>::op;
    constexpr int W = CG * S;
    __shared__ __attribute__((aligned(1024))) uint8_t xs[S * NL * 2048];
    __shared__ float red[2][CG][S][4][16];
    constexpr uint32_t OUT_OF_RANGE = 0x80000000u;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int cg = wave % CG, s = wave / CG;
    const int k = p.k, n = p.n;
    const int b = lane >> 2, q4 = lane & 3;
    const sgpr4 rx = buffer_rsrc(p.x, x_span_bytes(p));
#pragma unroll
    for (int q = wave; q < S * NL * 2; q += W) {
        const int kk = (q >> 1) * 256 + 16 * b + 8 * (q & 1);
        bdma16(rx, q4 < p.m && kk < k ? (uint32_t(q4) * uint32_t(p.ldx) + uint32_t(kk)) * 2u : OUT_OF_RANGE, xs + q * 1024);
    }
    auto issue = [&](int g, u32x4 (&wv)[NL]) {
        const int row = (g * CG + cg) * 4 + q4;
        const int8_t* wrow = p.w + int64_t(row < n ? row : n - 1) * k;
#pragma unroll
        for (int l = 0; l < NL; ++l) {
            const int kk = (s * NL + l) * 256 + 16 * b;  // past K: any row bytes, against zero activations
            wv[l] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + (kk < k ? kk : 0)));
        }
    };
    // products of one group, block partials -> LDS slot, barrier, one thread per (row, token) adds and stores
    auto finish = [&](int g, int slot, const u32x4 (&wv)[NL]) {
        v4f acc[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[q] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int l = 0; l < NL; ++l) {
            const int c = s * NL + l;
            const u32x4 x0 = *reinterpret_cast<const u32x4*>(xs + (2 * c) * 1024 + lane * 16);
            const u32x4 x1 = *reinterpret_cast<const u32x4*>(xs + (2 * c + 1) * 1024 + lane * 16);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint32_t p01, p23;
                weight_pairs<DT>(wv[l][q], p01, p23);
                const u32x4& xh = q < 2 ? x0 : x1;
                acc[q] = Mfma4<DT>::run(__builtin_bit_cast(op, u32x2{p01, p23}), __builtin_bit_cast(op, u32x2{xh[2 * (q & 1)], xh[2 * (q & 1) + 1]}), acc[q]);
            }
        }
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = (acc[0][i] + acc[1][i]) + (acc[2][i] + acc[3][i]);
            v[i] += dpp_f<0x124>(v[i]);  // row_ror:4
            v[i] += dpp_f<0x128>(v[i]);  // row_ror:8
        }
        if ((lane & 15) < 4) {
#pragma unroll
            for (int i = 0; i < 4; ++i) red[slot][cg][s][lane >> 4][q4 * 4 + i] = v[i];
        }
        __syncthreads();
        if (threadIdx.x < CG * 16) {
            const int gg = threadIdx.x >> 4, o = threadIdx.x & 15, t = o >> 2, ch = (g * CG + gg) * 4 + (o & 3);
            float sum = 0.0f;
#pragma unroll
            for (int r = 0; r < S; ++r)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) sum += red[slot][gg][r][rr][o];
            if (ch < n && t < p.m) store_out<DT>(p, t, ch, sum);
        }
    };
    u32x4 wa[NL], wb[NL];
    const int G = gridDim.x;
    int g = blockIdx.x;
    issue(g, wa);
    bool first = true;
    for (;;) {
        // even step: products of wa while wb's loads fly
        if (g + G < groups) {
            issue(g + G, wb);
            wait_vmcnt<NL>();
        } else {
            wait_vmcnt<0>();
        }
        if (first) __syncthreads();  // the staged activations of every wave have landed
        first = false;
        finish(g, 0, wa);
        g += G;
        if (g >= groups) break;
        if (g + G < groups) {
            issue(g + G, wa);
            wait_vmcnt<NL>();
        } else {
            wait_vmcnt<0>();
        }
        finish(g, 1, wb);
        g += G;
        if (g >= groups) break;
    }
}

static int cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        cached[dev] = v;
    }
    return cached[dev];
}
// grid: as many workgroups as the CUs hold at once (at most 2 per CU, measured best), never more than the groups
template <int DT, int CG, int S, int NL = 1> static int launch_quads(FewArgs& p, int nl, hipStream_t stream) {
    if constexpr (NL > 8) {
        return -2;
    } else {
        if (nl != NL) return launch_quads<DT, CG, S, NL + 1>(p, nl, stream);
        static int per_cu = 0;
        if (!per_cu) {
            int v = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, gemv_quads<DT, NL, CG, S>, 64 * CG * S, 0) != hipSuccess || v < 1) v = 1;
            per_cu = v < 2 ? v : 2;
        }
        const int groups = ((p.n + 3) / 4 + CG - 1) / CG;
        const int grid = std::min(groups, cu_count() * per_cu);
        gemv_quads<DT, NL, CG, S><<<grid, 64 * CG * S, 0, stream>>>(p, groups);
        return int(hipGetLastError());
    }
}

template <int DT>
static int launch_lines(FewArgs& p, hipStream_t stream) {
    const int nit = ((p.k & ~15) + 1023) / 1024;
    if constexpr (DT != DT_F32) {
        // activations staged in LDS (32-bit activation offsets)
        if (nit >= 1 && nit <= 16 && x_span_fits(p)) {
            if (p.m == 1) return dispatch_linesx<DT, 1>(p, nit, stream);
            // 3-4 tokens on matrix cores: 2 row quads x 4 k ranges per workgroup up to 8 KiB rows, 1 x 8 beyond
            if (p.m >= 3 && p.k % 16 == 0) {
                const int chunks = (p.k + 255) / 256;
                if (chunks <= 32) return launch_quads<DT, 2, 4>(p, (chunks + 3) / 4, stream);
                return launch_quads<DT, 1, 8>(p, (chunks + 7) / 8, stream);
            }
            if (p.m == 2) return dispatch_linesx<DT, 2>(p, nit, stream);
            if (p.m <= 4 && nit <= LINEX_LINES / 4) return dispatch_linesx<DT, 4>(p, nit, stream);
        }
    }
    const int groups = (p.n + LINE_CH - 1) / LINE_CH, grid = (groups + 3) / 4;
    switch (p.m) {
        case 1: gemv_lines<DT, 1><<<grid, 256, 0, stream>>>(p); break;
        case 2: gemv_lines<DT, 2><<<grid, 256, 0, stream>>>(p); break;
        case 3: gemv_lines<DT, 3><<<grid, 256, 0, stream>>>(p); break;
        default: gemv_lines<DT, 4><<<grid, 256, 0, stream>>>(p); break;
    }
    return int(hipGetLastError());
}

// ---------------------------------------------------------------------------------------------------------------
// small
// ---------------------------------------------------------------------------------------------------------------
constexpr int SMALL_KSTEP = 64;
constexpr int SMALL_WAVES = 4;                 // waves per workgroup, one fragment of 16 channels each
constexpr int SMALL_CH = 16 * SMALL_WAVES;     // channels per workgroup

template <int DT> struct Mfma16;
template <> struct Mfma16<DT_BF16> {
    using frag = bf16x8;
    static WQ8_DEVICE v4f run(frag a, frag b, v4f c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
    static WQ8_DEVICE __bf16 cvt(float f) { return static_cast<__bf16>(f); }
};
template <> struct Mfma16<DT_F16> {
    using frag = f16x8;
    static WQ8_DEVICE v4f run(frag a, frag b, v4f c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
    static WQ8_DEVICE _Float16 cvt(float f) { return static_cast<_Float16>(f); }
};

// 8 INT8 weights (two 32-bit words) -> 8 exact BF16 / FP16 values
template <int DT>
WQ8_DEVICE typename Mfma16<DT>::frag weights8(uint32_t lo, uint32_t hi) {
    typename Mfma16<DT>::frag f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        f[e] = Mfma16<DT>::cvt(float(int8_t(lo >> (8 * e))));
        f[4 + e] = Mfma16<DT>::cvt(float(int8_t(hi >> (8 * e))));
    }
    return f;
}

// K elements per split (one LDS line of weights per channel)
constexpr int SMALL_LINE = 512;
static int small_splits(int k) { return (k + SMALL_LINE - 1) / SMALL_LINE; }

// Partial products of one split: workgroup (channel group, split) = 64 channels x MT tiles of 16 tokens over one line of
// SMALL_LINE k. Everything reaches LDS by buffer_load ... lds (no registers held while the loads fly, zeros past M, N and
// K from out-of-range offsets): the split's activations once per workgroup (one row of SMALL_LINE values per token,
// padded by 16 bytes), and per wave its 16 weight rows, each DMA instruction covering whole rows of the line (the
// HBM-friendly pattern: 512 contiguous bytes per row). The 16-byte chunks of weight row r are stored at slot
// chunk ^ (r % 16), so that a fragment read (16 rows, one chunk each) hits 16 distinct bank groups. Then per 64-k step
// a wave reads its weight fragment (16 rows x 64 bytes), converts each INT8 weight exactly to BF16 / FP16, and runs
// v_mfma_f32_16x16x32 against the activation fragments of each token tile, FP32 accumulation. k permutation shared by
// both operands: lane l of a step takes the 16 values at 16 (l / 16) of the step's 64, the first 8 for the step's first
// MFMA and the last 8 for its second. With one split the workgroup finishes the outputs; otherwise it writes FP32
// partials slots[split][token][channel] and small_reduce() adds them in split order. With XR < 16 staged token rows
// (M <= XR, MT = 1) the workgroup needs less LDS and more of them share a CU: the activation fragment rows past XR read
// row r % XR, which only feeds the products of tokens past M, never stored.
template <int DT, int MT, int XR>
__global__ void __launch_bounds__(64 * SMALL_WAVES) w8_small(FewArgs p) {
    using raw = typename Elem<DT>::raw;
    using M = Mfma16<DT>;
    constexpr int ROW_BYTES = SMALL_LINE;                     // one weight row of the line
    constexpr int ROWS_PER_DMA = 1024 / ROW_BYTES;            // rows per 1 KiB DMA instruction
    constexpr int XP = SMALL_LINE * 2 + 16;                   // staged activation row pitch in bytes
    constexpr int XDMA = SMALL_LINE * 2 / 1024;               // DMA instructions per activation row
    static_assert(ROW_BYTES % 256 == 0 && ROWS_PER_DMA >= 1, "line");
    static_assert(XR == 16 || (MT == 1 && XR < 16 && 16 % XR == 0), "staged token rows");
    constexpr int XROWS = XR == 16 ? MT * 16 : XR;
    __shared__ __attribute__((aligned(1024))) uint8_t wl[SMALL_WAVES][16 * ROW_BYTES];
    __shared__ __attribute__((aligned(1024))) uint8_t xl[XROWS * XP];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int k = p.k, n = p.n, m = p.m;
    const int ch_base = blockIdx.x * SMALL_CH, k0 = blockIdx.y * SMALL_LINE;
    constexpr uint32_t OUT_OF_RANGE = 0x80000000u;

    // activations: token rows t = wave, wave + 4, ...; lane i takes values 8 i .. 8 i + 7 of its 1 KiB piece
    const sgpr4 rx = buffer_rsrc(p.x, x_span_bytes(p));
#pragma unroll
    for (int q = wave; q < XROWS * XDMA; q += SMALL_WAVES) {
        const int t = q / XDMA, h = q % XDMA;
        const int kk = k0 + h * 512 + 8 * lane;
        bdma16(rx, t < m && kk < k ? (uint32_t(t) * uint32_t(p.ldx) + uint32_t(kk)) * 2u : OUT_OF_RANGE, xl + t * XP + h * 1024);
    }
    // weights: row r of this wave is channel ch_base + 16 wave + r; one instruction covers ROWS_PER_DMA rows
    const sgpr4 rw = buffer_rsrc(p.w, uint32_t(n) * uint32_t(k));
    constexpr int LANES_PER_ROW = 64 / ROWS_PER_DMA;
#pragma unroll
    for (int d = 0; d < 16 / ROWS_PER_DMA; ++d) {
        const int r = d * ROWS_PER_DMA + lane / LANES_PER_ROW, slot = lane % LANES_PER_ROW;
        const int chunk = slot ^ (r & 15);                    // logical chunk stored in this lane's slot
        const int c = ch_base + 16 * wave + r, kk = k0 + 16 * chunk;
        // M <= 4 (XR < 16): the weights, read once, stream past the caches (6-9% faster at N or K = 13824; with 16 or 32
        // staged token rows the same hint measured 1-4% slower)
        const uint32_t off = c < n && kk < k ? uint32_t(c) * uint32_t(k) + uint32_t(kk) : OUT_OF_RANGE;
        if constexpr (XR < 16) bdma16_nt(rw, off, wl[wave] + d * 1024);
        else bdma16(rw, off, wl[wave] + d * 1024);
    }
    wait_vmcnt<0>();
    __syncthreads();  // the activations are shared by the workgroup's waves

    v4f acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = v4f{0, 0, 0, 0};
    const int r = lane & 15, sub = lane >> 4;
#pragma unroll
    for (int s = 0; s < SMALL_LINE / SMALL_KSTEP; ++s) {
        const u32x4 w4 = *reinterpret_cast<const u32x4*>(wl[wave] + r * ROW_BYTES + 16 * ((4 * s + sub) ^ r));
        const typename M::frag wa = weights8<DT>(w4[0], w4[1]), wb = weights8<DT>(w4[2], w4[3]);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const uint8_t* xr = xl + (XR == 16 ? 16 * t + r : r % XR) * XP + (s * SMALL_KSTEP + 16 * sub) * 2;
            const typename M::frag xa = __builtin_bit_cast(typename M::frag, *reinterpret_cast<const u32x4*>(xr));
            const typename M::frag xb = __builtin_bit_cast(typename M::frag, *reinterpret_cast<const u32x4*>(xr + 16));
            acc[t] = M::run(wa, xa, acc[t]);
            acc[t] = M::run(wb, xb, acc[t]);
        }
    }
    // accumulator lane layout: token 16 t + lane % 16, channels 16 wave + 4 (lane / 16) + e
    const int c0 = ch_base + 16 * wave + 4 * sub;
    const int split = blockIdx.y;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const int tok = 16 * t + (lane & 15);
        if (tok >= m) continue;
        if (gridDim.y == 1) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (c0 + e < n) store_out<DT>(p, tok, c0 + e, acc[t][e]);
        } else {
            float* dst = p.slots + (int64_t(split) * m + tok) * n + c0;
            if (c0 + 4 <= n && n % 4 == 0) {
                *reinterpret_cast<v4f*>(dst) = acc[t];
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (c0 + e < n) dst[e] = acc[t][e];
            }
        }
    }
}

// y[t, c] = epilogue(sum over splits of slots[split][t][c]), the splits added in order; the partials are loaded 8 at a
// time (independent loads in flight, then the ordered adds)
template <int DT>
__global__ void __launch_bounds__(256) small_reduce(FewArgs p, int splits) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x, mn = int64_t(p.m) * p.n;
    if (i >= mn) return;
    float v = 0.0f;
    for (int s0 = 0; s0 < splits; s0 += 8) {
        float part[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) part[s] = s0 + s < splits ? __builtin_nontemporal_load(p.slots + int64_t(s0 + s) * mn + i) : 0.0f;
#pragma unroll
        for (int s = 0; s < 8; ++s)
            if (s0 + s < splits) v = s0 + s == 0 ? part[s] : v + part[s];
    }
    store_out<DT>(p, int(i / p.n), int(i % p.n), v);
}

// Row-balanced form of small: one workgroup per CU (whole rounds of them past 64 rows per CU), each taking an equal share
// of the channels (33-64 of them) over the whole of K, or, with fewer than 33 rows per CU, over an equal part of K (a few K splits, whose FP32 partials
// small_reduce adds in order). Every CU streams the same number of weight bytes. Waves w and w + 4 compute channels
// 16 w .. 16 w + 15 of the share, over alternate k-steps.
// The weights and the activations go through a ring of STAGES stages of 256 k-elements (64 weight rows of 256 bytes and
// 16 MT token rows of 512 bytes per stage, buffer_load ... lds, zeros past the share, M and the split's K); the 16-byte
// chunks of every staged row are stored at slot chunk ^ (row % 16), which keeps the fragment reads conflict free. A
// workgroup stages the activations of its K range whole, so shares of fewer than 33 rows would read more activation
// than weight bytes: the K split keeps the shares at 33-64 rows. The MFMAs, the k permutation and the exact INT8 ->
// BF16 / FP16 conversion are small's.
template <int DT, int MT, int WAVES>
__global__ void __launch_bounds__(64 * WAVES) w8_rows(FewArgs p, int groups, int splits, int split_chunks) {
    using M = Mfma16<DT>;
    using raw = typename Elem<DT>::raw;
    // WAVES = 8: two waves per 16-channel fragment, taking alternate k-steps (2 waves per SIMD, so that one converts and
    // multiplies while the other waits); their sums are added through LDS at the end
    constexpr int FRAGS = 4, PH = WAVES / FRAGS, CH = 256, XR = 16 * MT, RW = 16 * FRAGS;
    static_assert(WAVES == 4 || WAVES == 8, "one or two waves per fragment");
    constexpr int W_BYTES = RW * CH, X_ROW = 2 * CH, X_BYTES = XR * X_ROW, STAGE = W_BYTES + X_BYTES, STAGES = 4;
    constexpr int WPW = W_BYTES / 1024 / WAVES, XPW = X_BYTES / 1024 / WAVES, L = WPW + XPW;  // 1 KiB copies per wave, stage
    static_assert(W_BYTES % (1024 * WAVES) == 0 && X_BYTES % (1024 * WAVES) == 0, "copies spread evenly over the waves");
    constexpr int WCPR = CH / 16, XCPR = X_ROW / 16;  // 16-byte chunks per staged row (4 weight rows, 2 token rows per copy)
    constexpr uint32_t OUT_OF_RANGE = 0x80000000u;
    __shared__ __attribute__((aligned(1024))) uint8_t ring[STAGES * STAGE];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = p.n, k = p.k, m = p.m;
    // workgroup (row group, K split): row group gi takes channels [gi n / groups, (gi + 1) n / groups), split si the
    // chunks [si split_chunks, (si + 1) split_chunks) of K
    const int gi = int(blockIdx.x) % groups, si = int(blockIdx.x) / groups;
    const int ch0 = int(int64_t(gi) * n / groups), nch = int(int64_t(gi + 1) * n / groups) - ch0;
    const int c_first = si * split_chunks, c_all = (k + CH - 1) / CH;
    const int chunks = (c_all - c_first < split_chunks ? c_all - c_first : split_chunks);
    const int k_end = (c_first + chunks) * CH < k ? (c_first + chunks) * CH : k;  // this split's K range ends here
    const sgpr4 rw = buffer_rsrc(p.w, uint32_t(n) * uint32_t(k));
    const sgpr4 rx = buffer_rsrc(p.x, x_span_bytes(p));

    // this lane's source of each of its copies at k-chunk 0 and the k of its chunk (past K or past the share: zeros)
    uint32_t w_src[WPW], x_src[XPW];
    int w_kk[WPW], x_kk[XPW];
#pragma unroll
    for (int i = 0; i < WPW; ++i) {
        const int r = (wave + WAVES * i) * (1024 / CH) + lane / WCPR, chunk = (lane % WCPR) ^ (r & 15);
        w_kk[i] = r < nch ? 16 * chunk : 1 << 30;
        w_src[i] = uint32_t(ch0 + r) * uint32_t(k) + 16u * uint32_t(chunk);
    }
#pragma unroll
    for (int i = 0; i < XPW; ++i) {
        const int r = 2 * (wave + WAVES * i) + lane / XCPR, chunk = (lane % XCPR) ^ (r & 15);
        x_kk[i] = r < m ? 8 * chunk : 1 << 30;
        x_src[i] = (uint32_t(r) * uint32_t(p.ldx) + 8u * uint32_t(chunk)) * 2u;
    }
    auto issue = [&](int c) {
        uint8_t* st = ring + (c % STAGES) * STAGE;
        const int kc = (c_first + c) * CH;
#pragma unroll
        for (int i = 0; i < WPW; ++i)
            bdma16(rw, kc + w_kk[i] < k_end ? w_src[i] + uint32_t(kc) : OUT_OF_RANGE, st + (wave + WAVES * i) * 1024);
#pragma unroll
        for (int i = 0; i < XPW; ++i)
            bdma16(rx, kc + x_kk[i] < k_end ? x_src[i] + 2u * uint32_t(kc) : OUT_OF_RANGE, st + W_BYTES + (wave + WAVES * i) * 1024);
    };

    // the epilogue's operands of this lane (channels 16 f + 4 sub + e of the share, tokens 16 t + r), loaded before
    // the mainloop so that their latency hides under it: y = fmaf(acc, sw, bias), then fmaf(y, rscale, residual), one
    // rounding (store_out's arithmetic)
    const int r = lane & 15, sub = lane >> 4, f = wave % FRAGS, ph = wave / FRAGS;
    float e_sw[4], e_bias[4], e_rs[4], e_res[MT][4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int cl = 16 * f + 4 * sub + e, c = ch0 + (cl < nch ? cl : 0);
        e_sw[e] = p.sw[c];
        e_bias[e] = p.bias ? Elem<DT>::to_f(static_cast<const raw*>(p.bias)[c]) : 0.0f;
        e_rs[e] = p.rscale ? Elem<DT>::to_f(static_cast<const raw*>(p.rscale)[c]) : 1.0f;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int tok = 16 * t + r;
            e_res[t][e] = p.residual && tok < m ? Elem<DT>::to_f(static_cast<const raw*>(p.residual)[int64_t(tok) * n + c]) : 0.0f;
        }
    }

    v4f acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = v4f{0, 0, 0, 0};
    auto compute = [&](int c) {
        const uint8_t* ws = ring + (c % STAGES) * STAGE + (16 * f + r) * CH;
        const uint8_t* xs = ring + (c % STAGES) * STAGE + W_BYTES + r * X_ROW;
#pragma unroll
        for (int q = 0; q < CH / 64 / PH; ++q) {
            const int s = q * PH + ph;
            const u32x4 w4 = *reinterpret_cast<const u32x4*>(ws + 16 * ((4 * s + sub) ^ r));
            const typename M::frag wa = weights8<DT>(w4[0], w4[1]), wb = weights8<DT>(w4[2], w4[3]);
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const uint8_t* xr = xs + t * 16 * X_ROW;
                const auto xa = __builtin_bit_cast(typename M::frag, *reinterpret_cast<const u32x4*>(xr + 16 * ((8 * s + 2 * sub) ^ r)));
                const auto xb = __builtin_bit_cast(typename M::frag, *reinterpret_cast<const u32x4*>(xr + 16 * ((8 * s + 2 * sub + 1) ^ r)));
                acc[t] = M::run(wa, xa, acc[t]);
                acc[t] = M::run(wb, xb, acc[t]);
            }
        }
    };

#pragma unroll
    for (int c = 0; c < STAGES - 1; ++c) issue(c);
    for (int c = 0; c < chunks; ++c) {
        wait_vmcnt<(STAGES - 2) * L>();  // this wave's copies of chunk c have landed
        wait_lgkm0();                    // and its reads of chunk c - 1 are done
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();    // every wave's: chunk c is whole and chunk c - 1's stage is free
        issue(c + STAGES - 1);           // past the last chunk: zeros into a free stage (the same count every time)
        compute(c);
    }
    wait_vmcnt<0>();  // no copy in flight when the workgroup ends
    if constexpr (PH > 1) {
        // the second wave of each fragment hands its sums to the first through the (now idle) ring
        wait_lgkm0();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        v4f* red = reinterpret_cast<v4f*>(ring) + (f * MT) * 64 + lane;
        if (ph == 1) {
#pragma unroll
            for (int t = 0; t < MT; ++t) red[t * 64] = acc[t];
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        if (ph == 1) return;
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[t] += red[t * 64];
    }

    // accumulator lane layout: token 16 t + r, channel 16 f + 4 sub + e of the share
    if (splits > 1) {
        // FP32 partials slots[split][token][channel], added in split order by small_reduce
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int tok = 16 * t + r;
            if (tok >= m) continue;
            float* dst = p.slots + (int64_t(si) * m + tok) * n + ch0 + 16 * f + 4 * sub;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (16 * f + 4 * sub + e < nch) dst[e] = acc[t][e];
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const int tok = 16 * t + r;
        if (tok >= m) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int cl = 16 * f + 4 * sub + e;
            if (cl >= nch) continue;
            float v = __builtin_fmaf(acc[t][e], e_sw[e], e_bias[e]);
            if (p.residual) v = __builtin_fmaf(v, e_rs[e], e_res[t][e]);
            static_cast<raw*>(p.y)[int64_t(tok) * n + ch0 + cl] = Elem<DT>::from_f(v);
        }
    }
}

// Launch shape of the row-balanced form: row groups of 33-64 channels, groups x splits = one workgroup per CU (or whole
// rounds of them, past 64 rows per CU), each K split taking an equal number of 256-k chunks (K splits when there are fewer than 33 rows per CU: their FP32 partials
// are added by small_reduce); groups = 0 selects the split form of w8_small instead. K splits are taken only for
// weights of 48 MiB or more: at N = 5120 they measured 12-19% faster than the split form at K = 13824 (M = 16-32), mixed
// at K = 5120 (-3% to +7%) and 10-20% slower at N = 1536.
struct RowsPlan { int groups = 0, splits = 1, split_chunks = 0; };
static RowsPlan rows_plan(int m, int n, int k, int sms) {
    RowsPlan r;
    if (n <= 0 || k <= 0) return r;
    const int cus = sms > 0 ? sms : 256, chunks = (k + 255) / 256;
    int splits = int(int64_t(64) * cus / n);
    splits = splits < 1 ? 1 : splits > chunks ? chunks : splits;
    if (splits > 1 && int64_t(n) * k < (int64_t(48) << 20)) return r;
    int groups = cus / splits;
    // at most 64 rows a workgroup: past 64 rows per CU, whole rounds of one workgroup per CU. Each round waits for its
    // first chunks again: at M <= 16 two rounds measured slower than the split form (N = 20480, M = 4: 30.9 against 24.6
    // us) or equal, at M = 32 7-25% faster (N = 20480-27648)
    if (int64_t(n) > int64_t(64) * groups) {
        if (m <= 16) return r;
        groups = int((int64_t(n) + int64_t(64) * cus - 1) / (int64_t(64) * cus)) * cus;
    }
    if ((n + groups - 1) / groups <= 32) return r;
    r.groups = groups;
    r.splits = splits;
    r.split_chunks = (chunks + splits - 1) / splits;
    r.splits = (chunks + r.split_chunks - 1) / r.split_chunks;
    return r;
}

template <int DT>
static int launch_small(FewArgs& p, int sms, hipStream_t stream) {
    if (int64_t(p.n) * p.k >= (int64_t(1) << 31) || !x_span_fits(p)) return -2;  // 32-bit offsets
    const RowsPlan rp = rows_plan(p.m, p.n, p.k, sms);
    if (rp.groups) {
        if (rp.splits > 1 && !p.slots) return -2;
        const int grid = rp.groups * rp.splits;
        // 8 waves: 3-6% faster than 4 at K = 5120, N = 13824, M = 4-32
        if (p.m <= 16) w8_rows<DT, 1, 8><<<grid, 512, 0, stream>>>(p, rp.groups, rp.splits, rp.split_chunks);
        else w8_rows<DT, 2, 8><<<grid, 512, 0, stream>>>(p, rp.groups, rp.splits, rp.split_chunks);
        if (int rc = int(hipGetLastError())) return rc;
        if (rp.splits == 1) return 0;
        const int64_t outs = int64_t(p.m) * p.n;
        small_reduce<DT><<<int((outs + 255) / 256), 256, 0, stream>>>(p, rp.splits);
        return int(hipGetLastError());
    }
    const int splits = small_splits(p.k);
    if (splits > 1 && !p.slots) return -2;
    const dim3 grid((p.n + SMALL_CH - 1) / SMALL_CH, splits);
    if (p.m <= 4) w8_small<DT, 1, 4><<<grid, 64 * SMALL_WAVES, 0, stream>>>(p);
    else if (p.m <= 16) w8_small<DT, 1, 16><<<grid, 64 * SMALL_WAVES, 0, stream>>>(p);
    else w8_small<DT, 2, 16><<<grid, 64 * SMALL_WAVES, 0, stream>>>(p);
    if (int rc = int(hipGetLastError())) return rc;
    if (splits == 1) return 0;
    const int64_t outs = int64_t(p.m) * p.n;
    small_reduce<DT><<<int((outs + 255) / 256), 256, 0, stream>>>(p, splits);
    return int(hipGetLastError());
}

}  // namespace wq8

using namespace wq8;

WQ8_API void wq8_small_workspace(int m, int n, int k, int sms, int64_t* sizes) {
    // the FP32 partials of every K split (no counters: the splits are added by a second kernel): the split form's, or
    // the row-balanced form's when it splits K; none for a single split
    const RowsPlan rp = rows_plan(m, n, k > 0 ? k : 64, sms);
    const int splits = rp.groups ? rp.splits : small_splits(k > 0 ? k : 64);
    sizes[0] = splits > 1 ? int64_t(splits) * (m > 0 ? m : 0) * n * 4 : 0;
    sizes[1] = 0;
}

WQ8_API int wq8_small(const void* x, int64_t ldx, const int8_t* w, const float* sw, const void* bias, const void* residual, const void* rscale,
                      void* y, int m, int n, int k, int dtype, int sms, float* slots, int* counters, hipStream_t stream) {
    if (!m || !n) return 0;
    if (k % 64 || m > 32 || m < 0 || n < 0) return -2;
    FewArgs p{x, ldx, w, sw, bias, residual, rscale, y, m, n, k, slots, counters, 0};
    if (dtype == DT_F16) return launch_small<DT_F16>(p, sms, stream);
    if (dtype == DT_BF16) return launch_small<DT_BF16>(p, sms, stream);
    return -1;
}

WQ8_API int wq8_gemv_lines(const void* x, int64_t ldx, const int8_t* w, const float* sw, const void* bias, const void* residual, const void* rscale,
                           void* y, int m, int n, int k, int dtype, hipStream_t stream) {
    if (!m || !n) return 0;
    if (m > 4 || m < 0 || n < 0 || k % 4) return -2;
    FewArgs p{x, ldx, w, sw, bias, residual, rscale, y, m, n, k, nullptr, nullptr, 0};
    if (dtype == DT_F16) return launch_lines<DT_F16>(p, stream);
    if (dtype == DT_BF16) return launch_lines<DT_BF16>(p, stream);
    return -1;
}
