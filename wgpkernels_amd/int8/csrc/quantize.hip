// Activation preparation on gfx950: per-block INT8 (block path), per-row INT8 with an optional hi/lo split
// (row / exact paths), and the unquantized few-token prologue (transform_rows, rotate_groups).
//
// One 256-thread workgroup (4 waves of 64) per row. The row is cut into 8-element chunks; thread t takes chunks
// t, t + 256, ... (16-byte loads, consecutive threads on consecutive chunks: coalesced). Up to 2048 * CPW elements a
// thread keeps its chunks in registers (one read of the row); longer rows are read again per pass.
// Reference: wgpkernels/int8/int8_gemm.cu (K8) :253-485 (kernels), :1354-1414 and :1860-1977 (launch / C ABI).
#include "wq8_common.h"
#include "wq8_abi.h"

namespace wq8 {

enum { PREP_BLOCKS = 0, PREP_ROWS = 1, PREP_TRANSFORM = 2 };

struct PrepArgs {
    const void* x;          // input rows (ldx elements apart)
    int8_t* q;              // BLOCKS: q; ROWS: hi
    int8_t* lo;             // ROWS: optional lo
    float* scale;           // BLOCKS: (m, ceil(k/128)); ROWS: (m)
    void* out;              // TRANSFORM: (m, k) in x's dtype
    float* inv_rms;         // optional: 1 / RMS per row (RMSNorm only)
    const void* act_weight; // RMSNorm weight (k values) or null
    const long long* counter; long long first, step;  // row offset first + counter[0] * step of x (graph loops)
    int64_t ldx;
    int k, group, act;
    float eps;
};

// Sum over the 4 waves of a workgroup in the fixed order ((w0 + w1) + w2) + w3.
WQ8_DEVICE float block_sum4(float wave_value, float* lds4) {
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds4[wave] = wave_value;
    __syncthreads();
    return ((lds4[0] + lds4[1]) + lds4[2]) + lds4[3];
}

WQ8_DEVICE float block_max4(float wave_value, float* lds4) {
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds4[wave] = wave_value;
    __syncthreads();
    return fmaxf(fmaxf(lds4[0], lds4[1]), fmaxf(lds4[2], lds4[3]));
}

// Waves per SIMD asked of the register allocator: a thread caches 8 * CPW floats, and these budgets (64, 96, 128 VGPRs)
// keep the occupancy that the cache alone allows. FP16 rows of the block quantizer and of transform_rows need more
// registers to convert and would spill under them; there the budget only holds 4 waves at 6 chunks of the quantizer.
constexpr int prep_waves(int dt, int mode, int cpw) {
    return dt == DT_F16 && mode != PREP_ROWS ? (mode == PREP_BLOCKS && cpw == 6 ? 4 : 1) : cpw <= 4 ? 8 : cpw <= 7 ? 5 : 4;
}

template <int DT, int MODE, int CPW>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(prep_waves(DT, MODE, CPW)))) prep_rows(PrepArgs p) {
    using raw = typename Elem<DT>::raw;
    __shared__ float lds4[4];
    const int tid = threadIdx.x;
    const int k = p.k, chunks = k >> 3, act = p.act, group = p.group;
    const long long shift = p.counter ? p.first + __ldg(p.counter) * p.step : 0;
    const raw* row = static_cast<const raw*>(p.x) + (int64_t(blockIdx.x) + shift) * p.ldx;
    const raw* aw = static_cast<const raw*>(p.act_weight);
    const int64_t r = blockIdx.x;
    const int iters = CPW ? CPW : (chunks + 255) >> 8;

    // RMSNorm: sum of squares in the fixed tree (per thread: chunks in order, fmaf per element; wave butterfly;
    // ((w0 + w1) + w2) + w3).
    float cache[CPW ? CPW : 1][8];
    float inv_rms = 1.0f;
    if (CPW) {
#pragma unroll
        for (int i = 0; i < (CPW ? CPW : 1); ++i) {
            const int c = tid + 256 * i;
            load_act<DT>(row, k, 8 * c, cache[i], c < chunks, act == ACT_RMS ? ACT_NONE : act);
        }
    }
    if (act == ACT_RMS) {
        float ss = 0.0f;
        for (int i = 0; i < iters; ++i) {
            float v[8];
            const int c = tid + 256 * i;
            if (CPW) {
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = cache[CPW ? i : 0][j];
            } else {
                load8<DT>(row + 8 * c, v, c < chunks);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) ss = __builtin_fmaf(v[j], v[j], ss);
        }
        inv_rms = rms_inverse(block_sum4(wave_sum(ss), lds4), k, p.eps);
        if (p.inv_rms && tid == 0) p.inv_rms[r] = inv_rms;
    }
    // the prepared (op, RMSNorm, rotated) chunk i of this thread
    auto chunk = [&](int i, float* v) {
        const int c = tid + 256 * i;
        const bool valid = c < chunks;
        if (CPW) {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = cache[CPW ? i : 0][j];
        } else {
            load_act<DT>(row, k, 8 * c, v, valid, act == ACT_RMS ? ACT_NONE : act);
        }
        if (act == ACT_RMS) apply_rms<DT>(v, inv_rms, aw, 8 * c, valid);
        rotate_chunk(v, group);
    };
    const float norm = group_norm(group);

    if constexpr (MODE == PREP_BLOCKS) {
        // one FP32 scale per 128-element block = 16 consecutive lanes (one DPP row)
        const int kblocks = (k + 127) >> 7;
        for (int i = 0; i < iters; ++i) {
            // a wave whose chunks all lie past the row has nothing to store (its blocks are another wave's)
            if (256 * i + (tid & ~63) >= chunks) break;
            float v[8];
            chunk(i, v);
            const int c = tid + 256 * i;
            float amax = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) amax = fmaxf(amax, __builtin_fabsf(v[j]));
            amax = row16_max(amax);
            const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
            if (c < chunks) {
                if ((c & 15) == 0) p.scale[r * kblocks + (c >> 4)] = div127(amax * norm);
                int qv[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    // |v inv| <= 127: the code is the low byte. FP32 rows keep the conversion, whose NaN result is 0
                    // whatever the NaN's payload (a BF16 / FP16 input NaN has a zero low byte either way)
                    if constexpr (DT == DT_F32) qv[j] = rne_int(v[j] * inv);
                    else qv[j] = rne_low_byte(v[j] * inv);
                }
                *reinterpret_cast<u32x2*>(p.q + r * k + 8 * c) =
                    u32x2{pack_s8x4(qv[0], qv[1], qv[2], qv[3]), pack_s8x4(qv[4], qv[5], qv[6], qv[7])};
            }
        }
    } else if constexpr (MODE == PREP_ROWS) {
        float amax = 0.0f;
        for (int i = 0; i < iters; ++i) {
            float v[8];
            chunk(i, v);
            if (CPW) {
#pragma unroll
                for (int j = 0; j < 8; ++j) cache[CPW ? i : 0][j] = v[j];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) amax = fmaxf(amax, __builtin_fabsf(v[j]));
        }
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) amax = fmaxf(amax, xor_shfl(amax, d));
        amax = block_max4(amax, lds4);
        const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
        if (tid == 0) p.scale[r] = div127(amax * norm);
        for (int i = 0; i < iters; ++i) {
            float v[8];
            if (CPW) {
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = cache[CPW ? i : 0][j];
            } else {
                chunk(i, v);
            }
            const int c = tid + 256 * i;
            if (c >= chunks) continue;
            int hv[8], lv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float t = v[j] * inv;
                hv[j] = rne_int(t);
                lv[j] = rne_int((t - float(hv[j])) * 254.0f);
            }
            *reinterpret_cast<u32x2*>(p.q + r * k + 8 * c) =
                u32x2{pack_s8x4(hv[0], hv[1], hv[2], hv[3]), pack_s8x4(hv[4], hv[5], hv[6], hv[7])};
            if (p.lo)
                *reinterpret_cast<u32x2*>(p.lo + r * k + 8 * c) =
                    u32x2{pack_s8x4(lv[0], lv[1], lv[2], lv[3]), pack_s8x4(lv[4], lv[5], lv[6], lv[7])};
        }
    } else {
        raw* out = static_cast<raw*>(p.out) + r * k;
        for (int i = 0; i < iters; ++i) {
            // a wave whose chunks all lie past the row has nothing to store (its blocks are another wave's)
            if (256 * i + (tid & ~63) >= chunks) break;
            float v[8];
            chunk(i, v);
            const int c = tid + 256 * i;
            if (c >= chunks) continue;
            if constexpr (DT == DT_F32) {
#pragma unroll
                for (int j = 0; j < 8; ++j) out[8 * c + j] = v[j] * norm;
            } else {
                u32x4 packed;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    packed[j] = uint32_t(Elem<DT>::from_f(v[2 * j] * norm)) | (uint32_t(Elem<DT>::from_f(v[2 * j + 1] * norm)) << 16);
                *reinterpret_cast<u32x4*>(out + 8 * c) = packed;
            }
        }
    }
}

template <int DT, int MODE>
static int launch_prep(const PrepArgs& p, int m, hipStream_t stream) {
    const int chunks = p.k / 8;
    // chunks per thread: the smallest count that covers the row (K = 5120 -> 3, 13824 -> 7), so no thread evaluates the
    // activation on chunks past the row
    if (chunks <= 256) prep_rows<DT, MODE, 1><<<m, 256, 0, stream>>>(p);
    else if (chunks <= 512) prep_rows<DT, MODE, 2><<<m, 256, 0, stream>>>(p);
    else if (chunks <= 768) prep_rows<DT, MODE, 3><<<m, 256, 0, stream>>>(p);
    else if (chunks <= 1024) prep_rows<DT, MODE, 4><<<m, 256, 0, stream>>>(p);
    else if (chunks <= 1536) prep_rows<DT, MODE, 6><<<m, 256, 0, stream>>>(p);
    else if (chunks <= 1792) prep_rows<DT, MODE, 7><<<m, 256, 0, stream>>>(p);
    else if (chunks <= 2048) prep_rows<DT, MODE, 8><<<m, 256, 0, stream>>>(p);
    else prep_rows<DT, MODE, 0><<<m, 256, 0, stream>>>(p);
    return int(hipGetLastError());
}

template <int MODE>
static int dispatch_prep(const PrepArgs& p, int m, int dtype, hipStream_t stream) {
    if (dtype == DT_F16) return launch_prep<DT_F16, MODE>(p, m, stream);
    if (dtype == DT_BF16) return launch_prep<DT_BF16, MODE>(p, m, stream);
    if (dtype == DT_F32 && !p.act) return launch_prep<DT_F32, MODE>(p, m, stream);
    return -1;
}

// argument checks shared by the preparation entry points (before any launch)
static int check_prep(int m, int k, int dtype, int group, int act) {
    if (dtype < 0 || dtype > 2) return -1;
    if (group != 0 && group != 16 && group != 64 && group != 256) return -1;
    if (act < 0 || act > 3) return -1;
    if (dtype == DT_F32 && act) return -1;
    if (m < 0 || k <= 0 || k % 8 || (group && k % group)) return -2;
    return 0;
}

thread_local RowOffsetArgs g_prep_offset = {nullptr, 0, 0};

}  // namespace wq8

using namespace wq8;

WQ8_API int wq8_quantize(const void* x, int8_t* hi, int8_t* lo, float* scale, int m, int k, int64_t ldx, int dtype, int group, int act,
                         const void* act_weight, float eps, hipStream_t stream) {
    if (!m) return 0;
    if (int rc = check_prep(m, k, dtype, group, act)) return rc;
    PrepArgs p{x, hi, lo, scale, nullptr, nullptr, act_weight, g_prep_offset.counter, g_prep_offset.first, g_prep_offset.step,
               ldx, k, group, act, eps};
    return dispatch_prep<PREP_ROWS>(p, m, dtype, stream);
}

WQ8_API int wq8_quantize_blocks(const void* x, int8_t* q, float* scale, int m, int k, int64_t ldx, int dtype, int group, int act,
                                const void* act_weight, float eps, float* inv_rms, hipStream_t stream) {
    if (!m) return 0;
    if (int rc = check_prep(m, k, dtype, group, act)) return rc;
    // the reference's caller supplies inv_rms scratch for RMSNorm rows longer than 16384 (K8:1887-1890); kept as a
    // contract: this library fills it with the rows' 1 / RMS
    if (act == ACT_RMS && k > 16384 && !inv_rms) return -2;
    PrepArgs p{x, q, nullptr, scale, nullptr, inv_rms, act_weight, g_prep_offset.counter, g_prep_offset.first, g_prep_offset.step,
               ldx, k, group, act, eps};
    return dispatch_prep<PREP_BLOCKS>(p, m, dtype, stream);
}

WQ8_API int wq8_quantize_at(const void* x, int8_t* hi, int8_t* lo, float* scale, int m, int k, int64_t ldx, int dtype, int group, int act,
                            const void* act_weight, float eps, const long long* counter, long long first, long long step, hipStream_t stream) {
    g_prep_offset = {counter, first, step};
    const int rc = wq8_quantize(x, hi, lo, scale, m, k, ldx, dtype, group, act, act_weight, eps, stream);
    g_prep_offset = {nullptr, 0, 0};
    return rc;
}

WQ8_API int wq8_quantize_blocks_at(const void* x, int8_t* q, float* scale, int m, int k, int64_t ldx, int dtype, int group, int act,
                                   const void* act_weight, float eps, float* inv_rms, const long long* counter, long long first, long long step,
                                   hipStream_t stream) {
    g_prep_offset = {counter, first, step};
    const int rc = wq8_quantize_blocks(x, q, scale, m, k, ldx, dtype, group, act, act_weight, eps, inv_rms, stream);
    g_prep_offset = {nullptr, 0, 0};
    return rc;
}

WQ8_API int wq8_transform_rows(const void* x, void* out, int m, int k, int64_t ldx, int dtype, int group, int act, const void* act_weight,
                               float eps, hipStream_t stream) {
    if (!m) return 0;
    if (dtype != DT_F16 && dtype != DT_BF16) return -1;
    if (int rc = check_prep(m, k, dtype, group, act)) return rc;
    PrepArgs p{x, nullptr, nullptr, nullptr, out, nullptr, act_weight, nullptr, 0, 0, ldx, k, group, act, eps};
    return dispatch_prep<PREP_TRANSFORM>(p, m, dtype, stream);
}

WQ8_API int wq8_rotate_groups(const void* x, void* out, int m, int k, int64_t ldx, int dtype, int group, hipStream_t stream) {
    if (!m) return 0;
    if (dtype != DT_F16 && dtype != DT_BF16) return -1;
    if (group != 16 && group != 64 && group != 256) return -1;
    if (k <= 0 || k % group) return -2;
    PrepArgs p{x, nullptr, nullptr, nullptr, out, nullptr, nullptr, nullptr, 0, 0, ldx, k, group, ACT_NONE, 0.0f};
    return dispatch_prep<PREP_TRANSFORM>(p, m, dtype, stream);
}
