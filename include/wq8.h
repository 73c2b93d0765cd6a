/*
 * C-ABI of libwgp_int8.so, the gfx950 (MI355X) INT8 weight linear library.
 *
 * Drop-in for the reference library of the same name: every entry point below has the argument list, argument
 * meaning and return codes of the reference's wgpkernels/int8/int8_gemm.cu (cited as K8:<line>) as bound by its
 * ctypes layer wgpkernels/int8/__init__.py (cited as I:<line>), so that layer loads this library unchanged once
 * "gfx950" is in its HIP_ARCHS (I:47).
 *
 * Conventions (as the reference):
 *  - returns 0 on success, a HIP error code from the launch, or -1 (bad dtype / group / act), -2 (bad shape or
 *    operand combination), -3 (unknown variant), -4 (bad segments), -5 (workspace beyond the allocation-free
 *    entry point's array), -6 (allocation-free entry point first called on a device under graph capture);
 *    calls are asynchronous on `stream`;
 *  - dtype: 0 FP16, 1 BF16, 2 FP32 (activations only); group: 0, 16, 64 or 256 (ConvRot); act: 0 none,
 *    1 RMSNorm, 2 SwiGLU (rows hold [gate | value]), 3 GELU (tanh approximation);
 *  - every buffer belongs to the caller; y may alias residual.
 */
#ifndef WQ8_H
#define WQ8_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* wq8_stream_t; /* hipStream_t */

/* ABI version, 11. Replaces K8:1349; checked at I:69. */
int wq8_abi(void);

/* Feature bits; bit 0: per-(channel, 128-element K block) weight scales. Replaces K8:1352; read at I:71-72. */
int wq8_features(void);

/* Row INT8 of op(x) with optional hi/lo split: hi, lo (m, k) int8, scale (m) f32. Replaces K8:1404; bound at I:74. */
int wq8_quantize(const void* x, int8_t* hi, int8_t* lo, float* scale, int m, int k, int64_t ldx, int dtype, int group, int act,
                 const void* act_weight, float eps, wq8_stream_t stream);

/* Per-128-block INT8 of op(x): q (m, k) int8, scale (m, ceil(k/128)) f32; inv_rms: m floats, required for RMSNorm
 * with k > 16384. Replaces K8:1936; bound at I:75. */
int wq8_quantize_blocks(const void* x, int8_t* q, float* scale, int m, int k, int64_t ldx, int dtype, int group, int act,
                        const void* act_weight, float eps, float* inv_rms, wq8_stream_t stream);

/* wq8_quantize / wq8_quantize_blocks reading input rows first + counter[0] * step (counter: int64 on the GPU).
 * Replace K8:1396 and K8:1926 (not bound by I; called directly by graph-loop callers). */
int wq8_quantize_at(const void* x, int8_t* hi, int8_t* lo, float* scale, int m, int k, int64_t ldx, int dtype, int group, int act,
                    const void* act_weight, float eps, const long long* counter, long long first, long long step, wq8_stream_t stream);
int wq8_quantize_blocks_at(const void* x, int8_t* q, float* scale, int m, int k, int64_t ldx, int dtype, int group, int act,
                           const void* act_weight, float eps, float* inv_rms, const long long* counter, long long first, long long step,
                           wq8_stream_t stream);

/* rotate(op(x)) rounded once to x's dtype: out (m, k). Replaces K8:1971; bound at I:76. */
int wq8_transform_rows(const void* x, void* out, int m, int k, int64_t ldx, int dtype, int group, int act, const void* act_weight,
                       float eps, wq8_stream_t stream);

/* ConvRot rotation only (group 16, 64, 256), rounded once. Replaces K8:1871; bound at I:87. */
int wq8_rotate_groups(const void* x, void* out, int m, int k, int64_t ldx, int dtype, int group, wq8_stream_t stream);

/* Y (m, n) = epilogue(A (m, k) int8 [, A_lo], B (n, k) int8); variant ids keep the reference's modes: 0, 2, 6 row;
 * 1, 7 exact (a_lo required); 10, 11 block (sa (m, ceil(k/128))); 12, 13 block with weight scales sb (n, ceil(k/128));
 * 14 exact with such weight scales; 15 (no counterpart in the reference) the short block tile with 10's biased fold. k % 16 == 0. Replaces K8:1648; bound at I:79. */
int wq8_gemm(const int8_t* a, const int8_t* a_lo, const float* sa, const int8_t* b, const float* sb, const void* bias, const void* residual,
             const void* rscale, void* y, int m, int n, int k, int dtype, int variant, int sms, int split, int* workspace, int* counters,
             wq8_stream_t stream);

/* Workspace bytes {slots, counters} of a wq8_gemm call: slots = the block modes' transposed scales, then with split != 0
 * the split-K partial sums (per split tile, or whole m x n planes per piece for launches of few tiles); counters = one
 * int per tail-split tile (zero on entry, left zero). wq8_gemm returns -2 for a workspace that is not 16-byte aligned.
 * Replaces K8:1506; bound at I:80-81. */
void wq8_gemm_workspace(int m, int n, int k, int variant, int sms, int split, int64_t* sizes);

/* Untuned variant choice for the row (hilo 0) or exact (hilo 1) mode. Replaces K8:1564; bound at I:82. */
int wq8_gemm_select(int m, int n, int k, int hilo, int sms);

/* wq8_gemm writing output / residual rows first + counter[0] * step, residual scales per span of rows, input rows from
 * in_first + counter[0] * in_step. Replaces K8:1637 (not bound by I). */
int wq8_gemm_at(const int8_t* a, const int8_t* a_lo, const float* sa, const int8_t* b, const float* sb, const void* bias, const void* residual,
                const void* rscale, void* y, int m, int n, int k, int dtype, int variant, int sms, int split, int* workspace, int* counters,
                const long long* counter, long long first, long long step, long long span, long long scale_step, long long in_first,
                long long in_step, wq8_stream_t stream);

/* 1 to 4 linears of one prepared input in one launch: ys[s] (m, rows) = A @ (bs[s] * sbs[s]).T + biases[s]; rows % 8 == 0.
 * Replaces K8:1663; bound at I:88-89 (hasattr-gated). */
int wq8_gemm_segments(const int8_t* a, const int8_t* a_lo, const float* sa, const int8_t* const* bs, const float* const* sbs,
                      const void* const* biases, void* const* ys, int count, int rows, int m, int k, int dtype, int variant, int sms,
                      int split, int* workspace, int* counters, wq8_stream_t stream);

/* wq8_gemm for callers that cannot allocate (code under graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. The workspace and split counters wq8_gemm takes from its caller live in
 * a library-owned device array of WQ8_GEMM_NOALLOC_MAX_BYTES per GPU, held until the process ends; a call needing more
 * returns -5. It allocates nothing. Every call on a GPU shares that GPU's array: calls that overlap on one GPU (several
 * streams) race. Results equal wq8_gemm's bit for bit. The array's address is resolved by the first wq8_gemm_workspace
 * query on a device (outside capture); a first call on a device made under graph capture returns -6. */
#define WQ8_GEMM_NOALLOC_MAX_BYTES (32ll << 20)
int wq8_gemm_noalloc(const int8_t* a, const int8_t* a_lo, const float* sa, const int8_t* b, const float* sb, const void* bias,
                     const void* residual, const void* rscale, void* y, int m, int n, int k, int dtype, int variant, int sms, int split,
                     wq8_stream_t stream);

/* Few tokens (m <= 32, k % 64 == 0): unquantized activations, exact INT8 weights on BF16/FP16 matrix cores, split-K
 * with `slots` (f32 partials) sized by wq8_small_workspace; `counters` is accepted and unused (its size is 0). Replace K8:1752 / K8:1693;
 * bound at I:83-85. */
int wq8_small(const void* x, int64_t ldx, const int8_t* w, const float* sw, const void* bias, const void* residual, const void* rscale,
              void* y, int m, int n, int k, int dtype, int sms, float* slots, int* counters, wq8_stream_t stream);
void wq8_small_workspace(int m, int n, int k, int sms, int64_t* sizes);

/* One to four tokens (k % 4 == 0): FP32 GEMV streaming the weights. Replaces K8:1851; bound at I:86. */
int wq8_gemv_lines(const void* x, int64_t ldx, const int8_t* w, const float* sw, const void* bias, const void* residual, const void* rscale,
                   void* y, int m, int n, int k, int dtype, wq8_stream_t stream);

/* Cold-cache timing: reads `bytes` of a library-owned buffer on `stream` (nonzero if it cannot be allocated);
 * release frees it. Replace K8:1997-2016; bound at I:77-78. */
int wq8_l2_flush(int device, int64_t bytes, wq8_stream_t stream);
void wq8_l2_flush_release(void);

#ifdef __cplusplus
}
#endif
#endif
