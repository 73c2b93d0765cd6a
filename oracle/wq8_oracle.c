/*
 * CPU oracle of the INT8 weight linear -- TEST INFRASTRUCTURE ONLY.
 *
 * This file is a plain-C restatement of the arithmetic of WGPKernels' INT8 path, used by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg as the checker. The product (the HIP library
 * under wgpkernels_amd/int8/csrc) never links, loads or calls it.
 *
 * Reference files followed (paths relative to the reference checkout):
 *   wgpkernels/int8/int8_gemm.cu  (cited as K8:<line>)
 *   wgpkernels/int8/__init__.py   (cited as I:<line>)
 *
 * Every floating-point step is written out operation by operation so that the GPU kernels, which perform
 * the same sequence, produce identical bits. Compile with -ffp-contract=off -fno-fast-math (oracle/Makefile).
 *
 * Where this build had to fix an order or a function that the reference leaves to CUDA:
 *   - GELU's tanh and SwiGLU's exp (K8:197-209) are this build's own: GELU is evaluated as
 *     x * logistic(2u) (equal to 0.5 x (1 + tanh u)), the logistic as 1 / (1 + exp(-s)) with exp by
 *     Cody-Waite range reduction and a degree-6 minimax polynomial and the reciprocal by Newton steps
 *     from an integer seed. They are pinned against libm double precision in tests/test_oracle.py.
 *   - the RMSNorm sum of squares uses a fixed 256-slot / wave64 tree (see ss_tree below), the order
 *     of the gfx950 kernels (the reference's is a 32-lane x 8-warp tree, K8:227-236).
 * Everything else restates the reference's order exactly.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ACT_NONE 0
#define ACT_RMS 1
#define ACT_SWIGLU 2
#define ACT_GELU 3

/* ------------------------------------------------------------------------------------------------ */
/* element conversions                                                                               */
/* ------------------------------------------------------------------------------------------------ */
static float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static float bf16_to_f(uint16_t h) { return bits_f((uint32_t)h << 16); }

/* round to nearest even, NaN kept quiet */
static uint16_t f_to_bf16(float f) {
    uint32_t u = f_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static float f16_to_f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1f, man = h & 0x3ffu;
    if (exp == 0) {
        /* zero or subnormal: man * 2^-24, exact in float */
        float v = (float)man * 5.9604644775390625e-8f;
        return sign ? -v : v;
    }
    if (exp == 31) return bits_f(sign | 0x7f800000u | (man << 13));
    return bits_f(sign | ((exp + 112u) << 23) | (man << 13));
}

/* IEEE binary16, round to nearest even, overflow to infinity */
static uint16_t f_to_f16(float f) {
    uint32_t u = f_bits(f), sign = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (a < 0x38800000u) {
        /* subnormal half: value / 2^-24 rounded to nearest even integer */
        float v = bits_f(a) * 16777216.0f; /* exact scaling by 2^24 */
        float r = nearbyintf(v);
        return (uint16_t)(sign | (uint32_t)r);
    }
    uint32_t e = (a >> 23) - 112u, m = a & 0x7fffffu;
    uint32_t half = (e << 10) | (m >> 13), rest = m & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (half & 1u))) half += 1;
    return (uint16_t)(sign | half);
}

static float load_elem(const void* p, int64_t i, int dtype) {
    if (dtype == 0) return f16_to_f(((const uint16_t*)p)[i]);
    if (dtype == 1) return bf16_to_f(((const uint16_t*)p)[i]);
    return ((const float*)p)[i];
}

static void store_elem(void* p, int64_t i, int dtype, float v) {
    if (dtype == 0) ((uint16_t*)p)[i] = f_to_f16(v);
    else if (dtype == 1) ((uint16_t*)p)[i] = f_to_bf16(v);
    else ((float*)p)[i] = v;
}

/* round to nearest even, as v_rndne_f32 + v_cvt_i32_f32; NaN -> 0 (the hardware conversion) */
static int rne_int(float t) {
    if (t != t) return 0;
    return (int)nearbyintf(t);
}

/* ------------------------------------------------------------------------------------------------ */
/* exp / logistic of this build (the same operation sequence runs in csrc/wq8_common.h)              */
/* ------------------------------------------------------------------------------------------------ */

/* exp(z) for z in [-87, 80]: t = fma(z, log2(e), 1.5*2^23) holds n = rint(z * log2(e)) (the exact product rounded
 * once) in its low mantissa bits; r = z - n*ln2 (Cody-Waite, two-part ln2, |r| <= 0.347); exp(r) by Horner on a
 * degree-6 polynomial of least maximum relative error on that range (8e-9 with these FP32 coefficients); scaled by
 * 2^n by adding n << 23 to p's bits (n in [-126, 116]: the result stays normal). */
float or_exp_core(float z) {
    const float t = fmaf(z, 0x1.715476p+0f, 0x1.8p23f);            /* log2(e), 1.5 * 2^23 */
    const float n = t - 0x1.8p23f;
    float r = fmaf(-n, 0x1.62e4p-1f, z);                           /* ln2 high part (14 bits: n*hi exact) */
    r = fmaf(-n, 0x1.7f7d1cp-20f, r);                              /* ln2 - high part */
    float p = 0x1.69d528p-10f;
    p = fmaf(p, r, 0x1.126946p-7f);
    p = fmaf(p, r, 0x1.55596cp-5f);
    p = fmaf(p, r, 0x1.55544p-3f);
    p = fmaf(p, r, 0x1.fffffcp-2f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return bits_f(f_bits(p) + (uint32_t)((int32_t)n * (1 << 23)));
}

/* 1/d for d in [1, 2^116]: integer seed 0x7EF311C3 - bits(d) (within 5.1 % of 1/d), then three Newton steps
 * e = 1 - d*r, r = r + r*e (fused); within 0.5006 ulp, no division. */
float or_recip(float d) {
    float r = bits_f(0x7EF311C3u - f_bits(d));
    for (int i = 0; i < 3; ++i) {
        const float e = fmaf(-d, r, 1.0f);
        r = fmaf(r, e, r);
    }
    return r;
}

/* logistic(s) = 1 / (1 + exp(-s)); the exponent is clamped to [-87, 80], so from -s >= 80 the result stays at
 * 1 / (1 + e^80) < 2^-115 */
float or_logistic(float s) {
    const float z = -s;
    const float e = or_exp_core(z > -87.0f ? (z < 80.0f ? z : 80.0f) : -87.0f);
    return or_recip(1.0f + e);
}

/* Checker of the GPU kernels' division by 127 (q = x RN(1/127); q + fma(-q, 127, x) RN(1/127); +inf kept) against the
 * IEEE quotient x / 127, over the bit patterns lo, lo + step, ... below hi: the number of patterns that differ. */
long long or_check_div127(uint32_t lo, uint32_t hi, uint32_t step) {
    const float inv = 1.0f / 127.0f;
    long long bad = 0;
    for (uint64_t u = lo; u < hi; u += step) {
        const float x = bits_f((uint32_t)u);
        const float q = x * inv;
        const float got = isinf(x) ? x : fmaf(fmaf(-q, 127.0f, x), inv, q);
        const float want = x / 127.0f;
        if (f_bits(got) != f_bits(want)) ++bad;
    }
    return bad;
}

/* GELU, tanh approximation (K8:197-200), as x * logistic(2*sqrt(2/pi)*(x + 0.044715 x^3)), which equals
 * 0.5 x (1 + tanh(sqrt(2/pi)(x + 0.044715 x^3))); the argument as x * (c0 + c1 x^2), c0 = 2 sqrt(2/pi) and
 * c1 = 0.044715 c0, each rounded to FP32 */
float or_gelu(float x) {
    return x * or_logistic(x * fmaf(x * x, 0x1.2444f2p-4f, 0x1.988454p+0f));
}

/* silu(g) * u = g * logistic(g) * u, K8:208 with this build's logistic */
float or_swiglu(float g, float u) { return g * or_logistic(g) * u; }

/* ------------------------------------------------------------------------------------------------ */
/* row helpers                                                                                       */
/* ------------------------------------------------------------------------------------------------ */
/* op(x) of one row without RMSNorm scaling: v[k] (swiglu reads [gate | value] of width 2k), K8:202-211 */
static void act_row(const void* x, int64_t row_off, int k, int dtype, int act, float* v) {
    for (int i = 0; i < k; ++i) {
        float g = load_elem(x, row_off + i, dtype);
        if (act == ACT_SWIGLU) g = or_swiglu(g, load_elem(x, row_off + k + i, dtype));
        else if (act == ACT_GELU) g = or_gelu(g);
        v[i] = g;
    }
}

/* Sum of squares of a row in the gfx950 kernels' fixed order: 256 slots, slot s takes the 8-element
 * chunks s, s+256, ... in order (fmaf per element); each 64-slot wave reduces with a butterfly
 * (xor 32, 16, 8, 4, 2, 1: every lane ends with the same sum); then ((w0 + w1) + w2) + w3. */
static float ss_tree(const float* v, int k) {
    float slot[256];
    const int chunks = k / 8;
    for (int s = 0; s < 256; ++s) {
        float ss = 0.0f;
        for (int c = s; c < chunks; c += 256)
            for (int j = 0; j < 8; ++j) ss = fmaf(v[8 * c + j], v[8 * c + j], ss);
        slot[s] = ss;
    }
    float wave[4];
    for (int w = 0; w < 4; ++w) {
        float l[64], n[64];
        for (int i = 0; i < 64; ++i) l[i] = slot[64 * w + i];
        for (int d = 32; d >= 1; d >>= 1) {
            for (int i = 0; i < 64; ++i) n[i] = l[i] + l[i ^ d];
            memcpy(l, n, sizeof(l));
        }
        wave[w] = l[0];
    }
    return ((wave[0] + wave[1]) + wave[2]) + wave[3];
}

/* 1 / sqrt(ss / K + eps), K8:225 */
static float rms_inverse(float ss, int k, float eps) { return 1.0f / sqrtf(ss / (float)k + eps); }

/* x * inv * weight, K8:216-222 */
static void apply_rms(float* v, int k, float inv, const void* w, int dtype) {
    for (int i = 0; i < k; ++i) v[i] = v[i] * inv * (w ? load_elem(w, i, dtype) : 1.0f);
}

/* ConvRot's unnormalised rotation of each group of `group` elements (16, 64, 256): radix-4 stages along
 * base-4 digits of the in-group index, least significant first (strides 1, 4, 16, 64); along a digit the
 * four values (a, b, c, d) give s = (a + b) + (c + d) and out[i] = s - 2 * in[3 - i] (H4 = J - 2*antidiag).
 * Equals v @ kron(H4, ..., H4) of I:579-584 times sqrt(group). K8:138-172, K8:1814-1831. */
static void rotate_row(float* v, int k, int group) {
    if (!group) return;
    float in[4];
    for (int stride = 1; stride < group; stride *= 4) {
        for (int base = 0; base < k; base += 4 * stride) {
            for (int off = 0; off < stride; ++off) {
                float* p = v + base + off;
                for (int i = 0; i < 4; ++i) in[i] = p[i * stride];
                const float s = (in[0] + in[1]) + (in[2] + in[3]);
                for (int i = 0; i < 4; ++i) p[i * stride] = s - 2.0f * in[3 - i];
            }
        }
    }
}

/* 1 / sqrt(group), folded into the stored scales: K8:297 */
static float group_norm(int group) {
    return group == 256 ? 1.0f / 16 : group == 64 ? 1.0f / 8 : group == 16 ? 1.0f / 4 : 1.0f;
}

/* op(x) then rotation (unnormalised) of row r into v */
static void prepare_row(const void* x, int r, int k, int64_t ldx, int dtype, int group, int act, const void* aw, float eps, float* v) {
    act_row(x, (int64_t)r * ldx, k, dtype, act == ACT_RMS ? ACT_NONE : act, v);
    if (act == ACT_RMS) apply_rms(v, k, rms_inverse(ss_tree(v, k), k, eps), aw, dtype);
    rotate_row(v, k, group);
}

static int check_common(int k, int dtype, int group, int act) {
    if (dtype < 0 || dtype > 2) return -1;
    if (group != 0 && group != 16 && group != 64 && group != 256) return -1;
    if (act < 0 || act > 3) return -1;
    if (dtype == 2 && act) return -1;
    if (k % 8 || (group && k % group)) return -2;
    return 0;
}

/* ------------------------------------------------------------------------------------------------ */
/* quantizers                                                                                        */
/* ------------------------------------------------------------------------------------------------ */
/* Per-block INT8: one FP32 scale per row and 128-element block of K; K8:392-424 (store_chunk_blocks):
 * amax = max |v| of the block, inv = amax > 0 ? 127 / amax : 0, scale = amax * norm / 127, q = rne(v * inv). */
int or_quantize_blocks(const void* x, int8_t* q, float* scale, int m, int k, int64_t ldx, int dtype, int group, int act,
                       const void* aw, float eps) {
    int rc = check_common(k, dtype, group, act);
    if (rc) return rc;
    const int kb = (k + 127) / 128;
    const float norm = group_norm(group);
    float* v = (float*)malloc(sizeof(float) * (size_t)k);
    for (int r = 0; r < m; ++r) {
        prepare_row(x, r, k, ldx, dtype, group, act, aw, eps, v);
        for (int b = 0; b < kb; ++b) {
            const int lo = b * 128, hi = lo + 128 < k ? lo + 128 : k;
            float amax = 0.0f;
            for (int i = lo; i < hi; ++i) amax = fmaxf(amax, fabsf(v[i]));
            const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
            scale[(int64_t)r * kb + b] = amax * norm / 127.0f;
            for (int i = lo; i < hi; ++i) q[(int64_t)r * k + i] = (int8_t)rne_int(v[i] * inv);
        }
    }
    free(v);
    return 0;
}

/* Row INT8 with optional hi/lo split: K8:269-327. scale = amax * norm / 127, t = v * (127 / amax),
 * hi = rne(t), lo = rne((t - hi) * 254). */
int or_quantize(const void* x, int8_t* hi, int8_t* lo, float* scale, int m, int k, int64_t ldx, int dtype, int group, int act,
                const void* aw, float eps) {
    int rc = check_common(k, dtype, group, act);
    if (rc) return rc;
    const float norm = group_norm(group);
    float* v = (float*)malloc(sizeof(float) * (size_t)k);
    for (int r = 0; r < m; ++r) {
        prepare_row(x, r, k, ldx, dtype, group, act, aw, eps, v);
        float amax = 0.0f;
        for (int i = 0; i < k; ++i) amax = fmaxf(amax, fabsf(v[i]));
        const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
        scale[r] = amax * norm / 127.0f;
        for (int i = 0; i < k; ++i) {
            const float t = v[i] * inv;
            const int h = rne_int(t);
            hi[(int64_t)r * k + i] = (int8_t)h;
            if (lo) lo[(int64_t)r * k + i] = (int8_t)rne_int((t - (float)h) * 254.0f);
        }
    }
    free(v);
    return 0;
}

/* Few-token prologue: rotate(op(x)) * norm rounded once to the input dtype; K8:453-485. */
int or_transform_rows(const void* x, void* out, int m, int k, int64_t ldx, int dtype, int group, int act, const void* aw, float eps) {
    int rc = check_common(k, dtype, group, act);
    if (rc) return rc;
    const float norm = group_norm(group);
    float* v = (float*)malloc(sizeof(float) * (size_t)k);
    for (int r = 0; r < m; ++r) {
        prepare_row(x, r, k, ldx, dtype, group, act, aw, eps, v);
        for (int i = 0; i < k; ++i) store_elem(out, (int64_t)r * k + i, dtype, v[i] * norm);
    }
    free(v);
    return 0;
}

/* ConvRot only, rounded once: K8:1814-1831. */
int or_rotate_groups(const void* x, void* out, int m, int k, int64_t ldx, int dtype, int group) {
    if (group != 16 && group != 64 && group != 256) return -1;
    return or_transform_rows(x, out, m, k, ldx, dtype, group, ACT_NONE, 0, 0.0f);
}

/* ------------------------------------------------------------------------------------------------ */
/* INT8 GEMM epilogue arithmetic: K8:773-863                                                         */
/* ------------------------------------------------------------------------------------------------ */
/* Exact INT32 sums of 128-element K blocks: sums[(r * n + c) * kb + b]. |sum| <= 128 * 127 * 128 < 2^22. */
void or_block_sums(const int8_t* a, const int8_t* b, int32_t* sums, int m, int n, int k) {
    const int kb = (k + 127) / 128;
    for (int r = 0; r < m; ++r)
        for (int c = 0; c < n; ++c)
            for (int blk = 0; blk < kb; ++blk) {
                int32_t s = 0;
                const int lo = blk * 128, hi = lo + 128 < k ? lo + 128 : k;
                for (int i = lo; i < hi; ++i) s += (int32_t)a[(int64_t)r * k + i] * (int32_t)b[(int64_t)c * k + i];
                sums[((int64_t)r * n + c) * kb + blk] = s;
            }
}

/*
 * Y = epilogue(A, B) in one of the reference's modes (mode 0 row, 1 exact (hi/lo), 2 block; wgroup: weight
 * scales sb of shape (N, ceil(K/128))):
 *   row:     v = float(acc);                                   y = fmaf(v * sa[r], sb[c], bias[c])
 *   exact:   v = fmaf(float(acc_lo), 1/254, float(acc_hi));    y = fmaf(v * sa[r], sb[c], bias[c])
 *   block:   f = sum_kb fmaf(float(S_kb), sa[r,kb], f);        y = fmaf(f * 1, sb[c], bias[c])
 *   block+g: f = sum_kb fmaf(float(S_kb), sa[r,kb] * sb[c,kb], f);  y = fmaf(f * 1, 1, bias[c])
 *   exact+g: f = sum_kb fmaf(fmaf(float(L_kb), 1/254, float(H_kb)), sb[c,kb], f);  y = fmaf(f * sa[r], 1, bias[c])
 *   exact+g, combined (mode 4; the gfx950 kernel's order, not the reference's): the block's two INT32 sums combine
 *            exactly, S = 254 H_kb + L_kb (|S| < 2^30), then f = sum_kb fmaf(float(S), sb[c,kb] / 254, f);
 *            y = fmaf(f * sa[r], 1, bias[c])
 *   block, biased (mode 3; the gfx950 wide kernel's single-FMA fold, not the reference's order):
 *            f = sum_kb fmaf(1.5*2^23 + S_kb, sa[r,kb], f); corr = sum_kb fmaf(1.5*2^23, sa[r,kb], corr);
 *            y = fmaf((f - corr) * 1, sb[c], bias[c])
 * then y = fmaf(y, rscale[c] or 1, residual[r,c]) and one rounding to the output dtype (0 f16, 1 bf16).
 * Block folds run in increasing block order, as the reference's non-split tiles do.
 *
 * pieces > 1: the split-K order of a tile split along K (the reference's stream-K pieces, K8:912-973, with this build's
 * piece boundaries): piece p folds blocks [p KB / pieces, (p + 1) KB / pieces) from zero in the mode's order (biased:
 * its own f - corr), and the pieces' values add in piece order, ((v0 + v1) + v2) + v3. Integer sums (row, exact) are
 * exact in any split, so pieces changes nothing there.
 */
int or_gemm_pieces(const int8_t* a, const int8_t* a_lo, const float* sa, const int8_t* b, const float* sb, const void* bias,
                   const void* residual, const void* rscale, void* y, int m, int n, int k, int dtype, int mode, int wgroup,
                   int pieces);

int or_gemm(const int8_t* a, const int8_t* a_lo, const float* sa, const int8_t* b, const float* sb, const void* bias,
            const void* residual, const void* rscale, void* y, int m, int n, int k, int dtype, int mode, int wgroup) {
    return or_gemm_pieces(a, a_lo, sa, b, sb, bias, residual, rscale, y, m, n, k, dtype, mode, wgroup, 1);
}

int or_gemm_pieces(const int8_t* a, const int8_t* a_lo, const float* sa, const int8_t* b, const float* sb, const void* bias,
                   const void* residual, const void* rscale, void* y, int m, int n, int k, int dtype, int mode, int wgroup,
                   int pieces) {
    if (dtype != 0 && dtype != 1) return -1;
    if (mode < 0 || mode > 4) return -2;
    if ((mode == 1 || mode == 4) != (a_lo != 0)) return -2;
    if (wgroup ? (mode == 0 || mode == 3) : mode == 4) return -2;
    const int biased = mode == 3, combined = mode == 4;
    if (biased) mode = 2;
    if (combined) mode = 1;
    const int kb = (k + 127) / 128;
    const int fold = mode == 2 || wgroup;
    if (pieces < 1 || (fold && pieces > kb)) return -2;
    if (!fold) pieces = 1;
    for (int r = 0; r < m; ++r) {
        const int8_t* ar = a + (int64_t)r * k;
        const int8_t* lr = a_lo ? a_lo + (int64_t)r * k : 0;
        for (int c = 0; c < n; ++c) {
            const int8_t* br = b + (int64_t)c * k;
            float v;
            if (fold) {
              for (int piece = 0; piece < pieces; ++piece) {
                float f = 0.0f, corr = 0.0f;
                for (int blk = piece * kb / pieces; blk < (piece + 1) * kb / pieces; ++blk) {
                    const int lo = blk * 128, hi = lo + 128 < k ? lo + 128 : k;
                    int32_t sh = 0, sl = 0;
                    for (int i = lo; i < hi; ++i) {
                        sh += (int32_t)ar[i] * (int32_t)br[i];
                        if (lr) sl += (int32_t)lr[i] * (int32_t)br[i];
                    }
                    if (biased) {
                        const float s = sa[(int64_t)r * kb + blk];
                        f = fmaf(12582912.0f + (float)sh, s, f); /* exact: |sh| < 2^22 */
                        corr = fmaf(12582912.0f, s, corr);
                    } else if (mode == 2) {
                        const float s = wgroup ? sa[(int64_t)r * kb + blk] * sb[(int64_t)c * kb + blk] : sa[(int64_t)r * kb + blk];
                        f = fmaf((float)sh, s, f);
                    } else if (combined) {
                        const int32_t sc = sh * 254 + sl; /* exact: |sh|, |sl| <= 128 * 127 * 127 */
                        f = fmaf((float)sc, sb[(int64_t)c * kb + blk] / 254.0f, f);
                    } else { /* exact+g */
                        const float hv = fmaf((float)sl, 1.0f / 254.0f, (float)sh);
                        f = fmaf(hv, sb[(int64_t)c * kb + blk], f);
                    }
                }
                const float part = biased ? f - corr : f;
                v = piece == 0 ? part : v + part;
              }
            } else {
                int32_t sh = 0, sl = 0;
                for (int i = 0; i < k; ++i) {
                    sh += (int32_t)ar[i] * (int32_t)br[i];
                    if (lr) sl += (int32_t)lr[i] * (int32_t)br[i];
                }
                v = mode == 1 ? fmaf((float)sl, 1.0f / 254.0f, (float)sh) : (float)sh;
            }
            const float row_scale = mode == 2 ? 1.0f : sa[r];
            const float col_scale = wgroup ? 1.0f : sb[c];
            const float bv = bias ? load_elem(bias, c, dtype) : 0.0f;
            float out = fmaf(v * row_scale, col_scale, bv);
            if (residual) {
                const float rs = rscale ? load_elem(rscale, c, dtype) : 1.0f;
                out = fmaf(out, rs, load_elem(residual, (int64_t)r * n + c, dtype));
            }
            store_elem(y, (int64_t)r * n + c, dtype, out);
        }
    }
    return 0;
}

/* FP64-accumulated reference of the few-token paths on already prepared (T-rounded) activations:
 * y = x @ (w * sw).T + bias, then residual; returned unrounded in FP32 (out_f) -- K8:1146-1147, K8:1803-1806. */
void or_linear_f64(const void* x, int64_t ldx, const int8_t* w, const float* sw, const void* bias, const void* residual,
                   const void* rscale, float* out_f, int m, int n, int k, int dtype) {
    for (int r = 0; r < m; ++r)
        for (int c = 0; c < n; ++c) {
            double s = 0.0;
            for (int i = 0; i < k; ++i) s += (double)load_elem(x, (int64_t)r * ldx + i, dtype) * (double)w[(int64_t)c * k + i];
            double v = s * (double)sw[c] + (bias ? (double)load_elem(bias, c, dtype) : 0.0);
            if (residual) v = v * (rscale ? (double)load_elem(rscale, c, dtype) : 1.0) + (double)load_elem(residual, (int64_t)r * n + c, dtype);
            out_f[(int64_t)r * n + c] = (float)v;
        }
}

/* conversions exposed for tests */
void or_to_dtype(const float* in, void* out, int64_t count, int dtype) {
    for (int64_t i = 0; i < count; ++i) store_elem(out, i, dtype, in[i]);
}
void or_from_dtype(const void* in, float* out, int64_t count, int dtype) {
    for (int64_t i = 0; i < count; ++i) out[i] = load_elem(in, i, dtype);
}
void or_exp_vec(const float* in, float* out, int64_t count) { for (int64_t i = 0; i < count; ++i) out[i] = or_exp_core(in[i]); }
void or_recip_vec(const float* in, float* out, int64_t count) { for (int64_t i = 0; i < count; ++i) out[i] = or_recip(in[i]); }
void or_logistic_vec(const float* in, float* out, int64_t count) { for (int64_t i = 0; i < count; ++i) out[i] = or_logistic(in[i]); }
void or_swiglu_vec(const float* g, const float* u, float* out, int64_t count) { for (int64_t i = 0; i < count; ++i) out[i] = or_swiglu(g[i], u[i]); }
void or_gelu_vec(const float* in, float* out, int64_t count) { for (int64_t i = 0; i < count; ++i) out[i] = or_gelu(in[i]); }
float or_ss_tree(const float* v, int k) { return ss_tree(v, k); }
void or_rotate_row(float* v, int k, int group) { rotate_row(v, k, group); }
