// Shared device code of the gfx950 INT8 linear library: element types, the input operations (RMSNorm,
// SwiGLU, GELU) with this build's exp / tanh, the ConvRot rotation and wave64 reductions.
//
// Floating-point rule of the whole library: it is compiled with -ffp-contract=off, so every multiply-add that
// is fused is an explicit fmaf; division and sqrt are IEEE correctly rounded
// (-fhip-fp32-correctly-rounded-divide-sqrt) and denormals are kept. The quantizers then give the same bits as a
// CPU running the same operation sequence.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define WQ8_DEVICE __device__ __forceinline__

namespace wq8 {

enum { ACT_NONE = 0, ACT_RMS = 1, ACT_SWIGLU = 2, ACT_GELU = 3 };
// dtype codes of the C-ABI (wgpkernels/int8/__init__.py:50 of the reference)
enum { DT_F16 = 0, DT_BF16 = 1, DT_F32 = 2 };

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// ---- element conversions (16-bit elements travel as raw uint16 bits) ---------------------------------------
template <int DT> struct Elem;
template <> struct Elem<DT_BF16> {
    using raw = uint16_t;
    static WQ8_DEVICE float to_f(uint16_t h) { return __builtin_bit_cast(float, uint32_t(h) << 16); }
    static WQ8_DEVICE uint16_t from_f(float f) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f)); }
};
template <> struct Elem<DT_F16> {
    using raw = uint16_t;
    static WQ8_DEVICE float to_f(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }
    // The FP32 value is pinned in a register first: otherwise the backend may fold a producing fmaf into v_fma_mix{lo,hi}_f16,
    // which rounds the fused result to FP16 once instead of to FP32 and then FP16, and so differs in the last place.
    static WQ8_DEVICE uint16_t from_f(float f) {
        asm("" : "+v"(f));
        return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
    }
};
template <> struct Elem<DT_F32> {
    using raw = float;
    static WQ8_DEVICE float to_f(float h) { return h; }
    static WQ8_DEVICE float from_f(float f) { return f; }
};

// 8 consecutive elements as FP32 (16-byte or 32-byte load); zeros when !valid.
template <int DT> WQ8_DEVICE void load8(const typename Elem<DT>::raw* p, float* v, bool valid) {
    if constexpr (DT == DT_F32) {
        v4f a = valid ? reinterpret_cast<const v4f*>(p)[0] : v4f{0, 0, 0, 0};
        v4f b = valid ? reinterpret_cast<const v4f*>(p)[1] : v4f{0, 0, 0, 0};
        for (int j = 0; j < 4; ++j) { v[j] = a[j]; v[j + 4] = b[j]; }
    } else {
        u32x4 raw = valid ? *reinterpret_cast<const u32x4*>(p) : u32x4{0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[2 * j] = Elem<DT>::to_f(uint16_t(raw[j] & 0xffffu));
            v[2 * j + 1] = Elem<DT>::to_f(uint16_t(raw[j] >> 16));
        }
    }
}

// ---- exp / logistic of this build ---------------------------------------------------------------------------
// exp_core(z) for z in [-87, 80]: t = z log2(e) + 1.5 2^23 in one FMA, so t holds n = rint(z log2 e) in its low
// mantissa bits and t - 1.5 2^23 = n exactly; r = z - n ln2 with ln2 split in two (Cody & Waite, |r| <= 0.347);
// exp(r) by Horner on a degree-6 polynomial fitted for least maximum relative error on |r| <= 0.347 (8e-9 with FP32
// coefficients); 2^n applied by adding n to p's exponent field, (bits(t) << 23) being n << 23 modulo 2^32 (one
// v_lshl_add_u32; the result is normal for every n in [-126, 116] that the clamp allows).
WQ8_DEVICE float exp_core(float z) {
    const float t = __builtin_fmaf(z, 0x1.715476p+0f, 0x1.8p23f);
    const float n = t - 0x1.8p23f;
    float r = __builtin_fmaf(-n, 0x1.62e4p-1f, z);
    r = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = 0x1.69d528p-10f;
    p = __builtin_fmaf(p, r, 0x1.126946p-7f);
    p = __builtin_fmaf(p, r, 0x1.55596cp-5f);
    p = __builtin_fmaf(p, r, 0x1.55544p-3f);
    p = __builtin_fmaf(p, r, 0x1.fffffcp-2f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, p) + (__builtin_bit_cast(uint32_t, t) << 23));
}

// 1 / d for d in [1, 2^116]: the integer seed 0x7EF311C3 - bits(d) (within 5.1 % of 1 / d) and three Newton steps
// e = 1 - d r, r = r + r e (two FMAs each): within 0.5006 ulp, no division. (v_rcp_f32 with one Newton step gives the
// correctly rounded quotient in 3 instructions, but its transcendental issue made the gelu quantizer slower.)
WQ8_DEVICE float recip(float d) {
    float r = __builtin_bit_cast(float, 0x7EF311C3u - __builtin_bit_cast(uint32_t, d));
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const float e = __builtin_fmaf(-d, r, 1.0f);
        r = __builtin_fmaf(r, e, r);
    }
    return r;
}

// logistic(s) = 1 / (1 + exp(-s)); exp's argument is clamped to [-87, 80]: below -87, 1 + exp rounds to 1; from -s >=
// 80 the result stays at 1 / (1 + e^80) < 2^-115, within 2^-115 of the true value (which is smaller still)
WQ8_DEVICE float logistic(float s) {
    // clamp to [-87, 80] in one v_med3_f32 (a NaN input gives a NaN result)
    const float e = exp_core(__builtin_amdgcn_fmed3f(-s, -87.0f, 80.0f));
    return recip(1.0f + e);
}

// GELU, tanh approximation, as x * logistic(2 sqrt(2/pi) (x + 0.044715 x^3)) (= 0.5 x (1 + tanh(...))), in FP32
// with the constants folded: the logistic's argument is x (c0 + c1 x^2), c0 = 2 sqrt(2/pi), c1 = 0.044715 c0
WQ8_DEVICE float wq_gelu(float x) {
    return x * logistic(x * __builtin_fmaf(x * x, 0x1.2444f2p-4f, 0x1.988454p+0f));
}

// SiLU(g) * u = g * logistic(g) * u
WQ8_DEVICE float wq_swiglu(float g, float u) { return g * logistic(g) * u; }

WQ8_DEVICE float rms_inverse(float ss, int k, float eps) { return 1.0f / __builtin_sqrtf(ss / float(k) + eps); }

WQ8_DEVICE float group_norm(int group) {
    return group == 256 ? 1.0f / 16 : group == 64 ? 1.0f / 8 : group == 16 ? 1.0f / 4 : 1.0f;
}

// x / 127 correctly rounded for x >= 0: q = x RN(1/127), then one remainder correction r = x - 127 q (exact by FMA),
// q + r RN(1/127); +inf passes through (its remainder is NaN). Equal to the IEEE quotient for every non-negative x up to
// +inf, denormals included (checked over all 2^31 - 2^23 + 1 such bit patterns; the oracle library's or_check_div127
// repeats the check over any range). Five ops against the ten of a general division.
WQ8_DEVICE float div127(float x) {
    constexpr float INV = 1.0f / 127.0f;
    const float q = x * INV;
    const float c = __builtin_fmaf(__builtin_fmaf(-q, 127.0f, x), INV, q);
    return __builtin_isinf(x) ? x : c;
}

// round to nearest even and convert (v_rndne_f32 + v_cvt_i32_f32; NaN gives 0)
WQ8_DEVICE int rne_int(float t) { return int(__builtin_rintf(t)); }

// rne_int(t) & 0xff for |t| < 2^22 in one add: t + 1.5 2^23 rounds t to the nearest even integer n and holds it in the
// low mantissa bits (0x4B400000 + n). A NaN t keeps its payload: 0 as rne_int's for NaNs made from BF16 / FP16 inputs
// (whose low 13 bits are 0) or by the arithmetic, but the payload's low byte for an FP32 input NaN (FP32 rows use
// rne_int).
WQ8_DEVICE int rne_low_byte(float t) { return int(__builtin_bit_cast(uint32_t, t + 0x1.8p23f)); }

// ---- cross-lane -------------------------------------------------------------------------------------------
WQ8_DEVICE float xor_shfl(float v, int mask) { return __shfl_xor(v, mask, 64); }

// Max over each row of 16 lanes with DPP (no LDS round trips): quad_perm [1,0,3,2] and [2,3,0,1] combine the lanes of a
// quad, row_half_mirror the two quads of each half row, row_mirror the two halves. Every lane of the row ends with the
// row's maximum (max is exact, so the order does not matter).
// The values are block maxima of |x| taken with fmaxf from +0, so never NaN and never negative: for them the unsigned
// order of the bit patterns is the float order, and the maximum runs as v_max_u32 with the DPP operand folded in (one
// instruction per step; a float max would add a canonicalizing v_max per step).
template <int CTRL> WQ8_DEVICE float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL> WQ8_DEVICE uint32_t dpp_u(uint32_t v) {
    return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), CTRL, 0xF, 0xF, true));
}
WQ8_DEVICE float row16_max(float amax) {
    uint32_t v = __builtin_bit_cast(uint32_t, amax);
    v = max(v, dpp_u<0xB1>(v));   // quad_perm [1,0,3,2]
    v = max(v, dpp_u<0x4E>(v));   // quad_perm [2,3,0,1]
    v = max(v, dpp_u<0x141>(v));  // row_half_mirror
    v = max(v, dpp_u<0x140>(v));  // row_mirror
    return __builtin_bit_cast(float, v);
}

// Butterfly sum over the 64 lanes (xor 32 .. 1): every lane ends with the same value (the RMS norm's pinned tree order).
WQ8_DEVICE float wave_sum(float v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += xor_shfl(v, d);
    return v;
}

// ---- ConvRot rotation of one 8-element chunk -------------------------------------------------------------
// A row is cut into 8-element chunks held one per lane, consecutive lanes holding consecutive chunks, so a
// group of 256 elements spans 32 lanes (aligned). In-group index e = 8 * (lane % 32) + j, base-4 digits
// d0 = j & 3, d1 = (j >> 2) | ((lane & 1) << 1), d2 = (lane >> 1) & 3, d3 = (lane >> 3) & 3.
// Stages along d0, d1, d2, d3 (up to the group): four values (a, b, c, d) along the digit give
// s = (a + b) + (c + d) and out[i] = s - 2 * in[3 - i]. Unnormalised (the 1/sqrt(group) goes to the scale).
WQ8_DEVICE void rotate_chunk(float* v, int group) {
    if (group < 16) return;
#pragma unroll
    for (int h = 0; h < 8; h += 4) {
        const float a = v[h], b = v[h + 1], c = v[h + 2], d = v[h + 3];
        const float s = (a + b) + (c + d);
        v[h] = s - 2.0f * d; v[h + 1] = s - 2.0f * c; v[h + 2] = s - 2.0f * b; v[h + 3] = s - 2.0f * a;
    }
    {
        float out[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float t = v[j] + v[j + 4];
            const float s = t + xor_shfl(t, 1);
            out[j] = s - 2.0f * xor_shfl(v[j + 4], 1);
            out[j + 4] = s - 2.0f * xor_shfl(v[j], 1);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = out[j];
    }
    if (group >= 64) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float a = v[j] + xor_shfl(v[j], 2);
            const float s = a + xor_shfl(a, 4);
            v[j] = s - 2.0f * xor_shfl(v[j], 6);
        }
    }
    if (group >= 256) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float a = v[j] + xor_shfl(v[j], 8);
            const float s = a + xor_shfl(a, 16);
            v[j] = s - 2.0f * xor_shfl(v[j], 24);
        }
    }
}

// op(x) (without the RMSNorm scaling) of the 8 elements at `col` of a row; SwiGLU rows hold [gate (k) | value (k)].
template <int DT> WQ8_DEVICE void load_act(const typename Elem<DT>::raw* row, int k, int col, float* v, bool valid, int act) {
    load8<DT>(row + col, v, valid);
    if (!valid) return;  // zeros (gelu(0) = swiglu(0, 0) = 0); whole waves past the row skip the activation
    if (act == ACT_SWIGLU) {
        float u[8];
        load8<DT>(row + k + col, u, valid);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = wq_swiglu(v[j], u[j]);
    } else if (act == ACT_GELU) {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = wq_gelu(v[j]);
    }
}

// v * inv * weight (weight optional)
template <int DT> WQ8_DEVICE void apply_rms(float* v, float inv, const typename Elem<DT>::raw* w, int col, bool valid) {
    float wv[8];
    if (w) load8<DT>(w + col, wv, valid);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = v[j] * inv * (w ? wv[j] : 1.0f);
}

WQ8_DEVICE uint32_t pack_s8x4(int a, int b, int c, int d) {
    return (uint32_t(a) & 0xffu) | ((uint32_t(b) & 0xffu) << 8) | ((uint32_t(c) & 0xffu) << 16) | (uint32_t(d) << 24);
}

}  // namespace wq8
