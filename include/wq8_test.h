/*
 * C-ABI of libwgp_int8_test.so: entry points with no counterpart in the reference, built apart from the product
 * library (libwgp_int8.so exports only include/wq8.h). Used by the parity tests and by bench.py; same conventions.
 */
#ifndef WQ8_TEST_H
#define WQ8_TEST_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* wq8_stream_t; /* hipStream_t */

/* The exact INT32 sums of every 128-element K block, sums[(t * n + c) * ceil(k/128) + kb], from a GEMM mainloop that
 * computes them instead of folding them: kernel 0 the ring kernel's (row mode), kernel 1 the ping-pong kernel of the
 * long block tiles (the headline kernel's mainloop, biased chains). */
int wq8_debug_block_sums(const int8_t* a, const int8_t* b, int32_t* sums, int m, int n, int k, int kernel, wq8_stream_t stream);

/* The INT8 matrix-core rate probe. blocks workgroups of 4 waves each run iters rounds of 16 independent
 * v_mfma_i32_32x32x32_i8 (shape 0), or 32 of v_mfma_i32_16x16x64_i8 (shape 1, the same ops), on operand fragments
 * loaded once from `operands` (blocks * 2048 16-byte fragments); out holds blocks * 256 ints. Used by bench.py for the
 * in-run matrix-core ceiling. */
int wq8_debug_mfma_probe(const void* operands, int* out, int blocks, int iters, int shape, wq8_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif
