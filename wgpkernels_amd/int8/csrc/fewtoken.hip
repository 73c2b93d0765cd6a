// Few-token paths on gfx950 (unquantized activations, exact INT8 weights, FP32 accumulation):
//   lines (1-4 tokens)  VALU GEMV: each wave streams its weight rows, every lane loading 16 contiguous bytes per row
//                       (one 1 KiB line per row and load instruction), exact byte -> FP32 conversion (SDWA
//                       sign-extending converts), FP32 FMAs, wave64 butterfly reduction. One token with K <= 16 KiB:
//                       every load of a wave is issued before its first FMA (gemv_line1).
//   small (<= 32)       matrix cores: INT8 weights converted exactly to BF16 / FP16 in registers feed
//                       v_mfma_f32_16x16x32_{bf16,f16} (16 channels x 16 tokens x 32 k), split-K across workgroups
//                       with FP32 partial slots and a deterministic last-arriver reduction.
// Reference: wgpkernels/int8/int8_gemm.cu (K8) :1039-1151 (w8a16_small), :1768-1810 (gemv_lines), :1684-1759 and
// :1833-1858 (launch / C ABI).
#include "wq8_common.h"
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
    int* counters;  // small: per channel-group arrival counters (zero on entry, left zero)
    int splits;
};

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
        float xf[ROWS][16];
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            load8<DT>(x + int64_t(r) * p.ldx + kk, xf[r], true);
            load8<DT>(x + int64_t(r) * p.ldx + kk + 8, xf[r] + 8, true);
        }
#pragma unroll
        for (int c = 0; c < LINE_CH; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t word = wv[c][q];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float wf = float(int8_t(word >> (8 * e)));
#pragma unroll
                    for (int r = 0; r < ROWS; ++r) acc[c][r][e & 1] = __builtin_fmaf(wf, xf[r][4 * q + e], acc[c][r][e & 1]);
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

// One token, K <= 16 KiB, 16-bit activations: a wave takes CH weight rows and issues every load of them (NIT 1 KiB lines
// per row, plus the matching activation chunks) before its first FMA, so that the whole weight matrix is requested from
// HBM at once instead of a few lines per wave and round trip; the grid's many short waves keep every CU's loads in flight.
template <int DT, int CH, int NIT>
__global__ void __launch_bounds__(256) gemv_line1(FewArgs p) {
    using raw = typename Elem<DT>::raw;
    static_assert(sizeof(raw) == 2, "16-bit activations");
    const int lane = threadIdx.x & 63;
    const int ch0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * CH;
    if (ch0 >= p.n) return;
    const int k = p.k, k16 = k & ~15;
    const raw* x = static_cast<const raw*>(p.x);
    const int8_t* wrow[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) wrow[c] = p.w + int64_t(ch0 + c < p.n ? ch0 + c : p.n - 1) * k;
    u32x4 wv[NIT][CH], xv[NIT][2];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int kk = it * 1024 + lane * 16, kc = kk < k16 ? kk : 0;  // lanes past the row read its start, then drop it
#pragma unroll
        for (int c = 0; c < CH; ++c) wv[it][c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[c] + kc));
    }
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int kk = it * 1024 + lane * 16, kc = kk < k16 ? kk : 0;
        xv[it][0] = *reinterpret_cast<const u32x4*>(x + kc);
        xv[it][1] = *reinterpret_cast<const u32x4*>(x + kc + 8);
    }
    float acc[CH][2];
#pragma unroll
    for (int c = 0; c < CH; ++c) acc[c][0] = acc[c][1] = 0.0f;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const bool valid = it * 1024 + lane * 16 < k16;
        float xf[16];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t word = valid ? xv[it][h][j] : 0u;
                xf[8 * h + 2 * j] = Elem<DT>::to_f(uint16_t(word & 0xffffu));
                xf[8 * h + 2 * j + 1] = Elem<DT>::to_f(uint16_t(word >> 16));
            }
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t word = wv[it][c][q];
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[c][e & 1] = __builtin_fmaf(float(int8_t(word >> (8 * e))), xf[4 * q + e], acc[c][e & 1]);
            }
    }
    // K % 16 tail: 4-byte pieces (K is a multiple of 4)
    for (int kk = k16 + 4 * lane; kk < k; kk += 256) {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const uint32_t word = *reinterpret_cast<const uint32_t*>(wrow[c] + kk);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[c][e & 1] = __builtin_fmaf(float(int8_t(word >> (8 * e))), Elem<DT>::to_f(x[kk + e]), acc[c][e & 1]);
        }
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const float s = wave_sum(acc[c][0] + acc[c][1]);
        if (lane == 0 && ch0 + c < p.n) store_out<DT>(p, 0, ch0 + c, s);
    }
}

template <int DT, int CH, int NIT> static int launch_line1(FewArgs& p, hipStream_t stream) {
    const int groups = (p.n + CH - 1) / CH;
    gemv_line1<DT, CH, NIT><<<(groups + 3) / 4, 256, 0, stream>>>(p);
    return int(hipGetLastError());
}

// 1 KiB lines per row; two rows per wave when there are many rows and few lines (fewer, fuller waves), else one
template <int DT, int NIT = 1> static int dispatch_line1(FewArgs& p, int nit, hipStream_t stream) {
    if constexpr (NIT > 16) {
        return -2;
    } else {
        if (nit == NIT) return p.n >= 8192 && NIT <= 8 ? launch_line1<DT, 2, NIT>(p, stream) : launch_line1<DT, 1, NIT>(p, stream);
        return dispatch_line1<DT, NIT + 1>(p, nit, stream);
    }
}

template <int DT>
static int launch_lines(FewArgs& p, hipStream_t stream) {
    const int nit = ((p.k & ~15) + 1023) / 1024;
    if constexpr (DT != DT_F32)
        if (p.m == 1 && nit >= 1 && nit <= 16) return dispatch_line1<DT>(p, nit, stream);
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
constexpr int SMALL_CH = 64;   // channels per workgroup (4 fragments of 16)
constexpr int SMALL_KSTEP = 64;

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

// Workgroup: 64 channels (4 fragments of 16) x MT tiles of 16 tokens, a K range of whole 64-element steps split over
// the grid's y dimension; its 4 waves take interleaved 64-element steps of that range and meet in LDS.
template <int DT, int MT>
__global__ void __launch_bounds__(256) w8_small(FewArgs p) {
    using raw = typename Elem<DT>::raw;
    using M = Mfma16<DT>;
    __shared__ float part[4][MT * 16][SMALL_CH + 1];
    __shared__ int s_last;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int k = p.k, n = p.n, m = p.m;
    const int ch_base = blockIdx.x * SMALL_CH;
    const int steps = k / SMALL_KSTEP, splits = gridDim.y;
    const int s_begin = int((long long)blockIdx.y * steps / splits), s_end = int((long long)(blockIdx.y + 1) * steps / splits);
    const int sub = lane >> 4;  // 16-byte k piece of the step: elements 16 sub .. 16 sub + 15

    const int8_t* wp[4];
#pragma unroll
    for (int f = 0; f < 4; ++f) {
        const int ch = ch_base + 16 * f + (lane & 15);
        wp[f] = p.w + int64_t(ch < n ? ch : n - 1) * k + 16 * sub;
    }
    const raw* xp[MT];
    bool xok[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const int tok = 16 * t + (lane & 15);
        xok[t] = tok < m;
        xp[t] = static_cast<const raw*>(p.x) + int64_t(xok[t] ? tok : 0) * p.ldx + 16 * sub;
    }
    v4f acc[4][MT];
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[f][t] = v4f{0, 0, 0, 0};

    for (int s = s_begin + wave; s < s_end; s += 4) {
        const int k0 = s * SMALL_KSTEP;
        u32x4 wv[4];
#pragma unroll
        for (int f = 0; f < 4; ++f) wv[f] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wp[f] + k0));
        typename M::frag xa[MT], xb[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const u32x4 lo = xok[t] ? *reinterpret_cast<const u32x4*>(xp[t] + k0) : u32x4{0, 0, 0, 0};
            const u32x4 hi = xok[t] ? *reinterpret_cast<const u32x4*>(xp[t] + k0 + 8) : u32x4{0, 0, 0, 0};
            xa[t] = __builtin_bit_cast(typename M::frag, lo);
            xb[t] = __builtin_bit_cast(typename M::frag, hi);
        }
#pragma unroll
        for (int f = 0; f < 4; ++f) {
            const typename M::frag wa = weights8<DT>(wv[f][0], wv[f][1]), wb = weights8<DT>(wv[f][2], wv[f][3]);
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                acc[f][t] = M::run(wa, xa[t], acc[f][t]);
                acc[f][t] = M::run(wb, xb[t], acc[f][t]);
            }
        }
    }
    // accumulator lane layout: token 16 t + lane % 16, channels 16 f + 4 (lane / 16) + e
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) part[wave][16 * t + (lane & 15)][16 * f + 4 * (lane >> 4) + e] = acc[f][t][e];
    __syncthreads();
    constexpr int OUTS = MT * 16 * SMALL_CH;
    float* own = splits > 1 ? p.slots + (int64_t(blockIdx.x) * splits + blockIdx.y) * OUTS : nullptr;
    for (int i = tid; i < OUTS; i += 256) {
        const int tok = i / SMALL_CH, c = i % SMALL_CH;
        const float v = ((part[0][tok][c] + part[1][tok][c]) + part[2][tok][c]) + part[3][tok][c];
        part[0][tok][c] = v;
        if (own) __builtin_nontemporal_store(v, own + i);
    }
    if (splits > 1) {
        __threadfence();
        __syncthreads();
        if (tid == 0) s_last = atomicAdd(p.counters + blockIdx.x, 1) == splits - 1;
        __syncthreads();
        if (!s_last) return;
        __threadfence();
        const float* tile = p.slots + int64_t(blockIdx.x) * splits * OUTS;
        for (int i = tid; i < OUTS; i += 256) {
            float v = 0.0f;
            for (int sp = 0; sp < splits; ++sp) v += __builtin_nontemporal_load(tile + int64_t(sp) * OUTS + i);
            part[0][i / SMALL_CH][i % SMALL_CH] = v;
        }
        if (tid == 0) p.counters[blockIdx.x] = 0;
        __syncthreads();
    }
    for (int i = tid; i < OUTS; i += 256) {
        const int tok = i / SMALL_CH, c = ch_base + i % SMALL_CH;
        if (tok < m && c < n) store_out<DT>(p, tok, c, part[0][tok][i % SMALL_CH]);
    }
}

// K splits so that about two workgroups per CU stream weights, each with at least 8 steps of 64.
static int small_splits(int n, int k, int sms) {
    const int groups = (n + SMALL_CH - 1) / SMALL_CH, steps = k / SMALL_KSTEP;
    int splits = (2 * sms + groups - 1) / groups;
    const int most = steps / 8 > 1 ? steps / 8 : 1;
    return splits < most ? splits : most;
}

template <int DT>
static int launch_small(FewArgs& p, int sms, hipStream_t stream) {
    const dim3 grid((p.n + SMALL_CH - 1) / SMALL_CH, small_splits(p.n, p.k, sms));
    if (grid.y > 1 && (!p.slots || !p.counters)) return -2;
    if (p.m <= 16) w8_small<DT, 1><<<grid, 256, 0, stream>>>(p);
    else w8_small<DT, 2><<<grid, 256, 0, stream>>>(p);
    return int(hipGetLastError());
}

}  // namespace wq8

using namespace wq8;

WQ8_API void wq8_small_workspace(int m, int n, int k, int sms, int64_t* sizes) {
    const int groups = (n + SMALL_CH - 1) / SMALL_CH, splits = small_splits(n, k, sms), mt = m <= 16 ? 1 : 2;
    sizes[0] = splits > 1 ? int64_t(groups) * splits * mt * 16 * SMALL_CH * 4 : 0;
    sizes[1] = splits > 1 ? 4 * int64_t(groups) : 0;
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
