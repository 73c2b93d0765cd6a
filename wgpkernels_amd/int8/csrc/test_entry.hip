// Test library (libwgp_int8_test.so, not the product library): entry points with no counterpart in the reference, for
// the parity tests and bench.py. They share the product's kernels (headers) and take raw device pointers like its C ABI.
#include "gemm_launch.h"
#include "wq8_abi.h"

using namespace wq8;

namespace {

// Matrix-core rate probe: each wave loads 8 operand fragments (16 bytes per lane each) from `operands` and runs `iters`
// rounds of 16 independent v_mfma_i32_32x32x32_i8 on them, with no memory traffic in the loop. Zero operands against
// random ones show how much of the chip's INT8 rate the power limit leaves for real data.
__global__ void __launch_bounds__(256) mfma_probe(const v4i* __restrict__ operands, int* __restrict__ out, int iters) {
    const int lane = threadIdx.x & 63, wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    v4i a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a[i] = operands[(wave * 8 + i) * 64 + lane];
        b[i] = operands[(wave * 8 + 4 + i) * 64 + lane];
    }
    v16i acc[4][4] = {};
    for (int it = 0; it < iters; ++it)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) sum += acc[i][j][e];
    out[wave * 64 + lane] = sum;
}

// The same probe on v_mfma_i32_16x16x64_i8 (the same MACs per clock, a quarter of the accumulator registers per
// instruction): 16 independent accumulators over the same 8 fragments, 16 x 16 x 64 MACs per instruction.
__global__ void __launch_bounds__(256) mfma_probe16(const v4i* __restrict__ operands, int* __restrict__ out, int iters) {
    const int lane = threadIdx.x & 63, wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    v4i a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a[i] = operands[(wave * 8 + i) * 64 + lane];
        b[i] = operands[(wave * 8 + 4 + i) * 64 + lane];
    }
    v4i acc[4][4] = {};
    for (int it = 0; it < iters; ++it)
#pragma unroll
        for (int rep = 0; rep < 2; ++rep)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) sum += acc[i][j][e];
    out[wave * 64 + lane] = sum;
}

}  // namespace

// The exact INT32 sums of every 128-element K block, sums[(t * N + c) * ceil(K / 128) + kb], as a GEMM mainloop computes
// them instead of folding them: kernel 0 the ring kernel's (row mode, 128 x 256 tiles), kernel 1 the ping-pong kernel of
// the long block tiles (256 x 192, biased chains: each sum is read off its chain's start value).
WQ8_API int wq8_debug_block_sums(const int8_t* a, const int8_t* b, int32_t* sums, int m, int n, int k, int kernel, hipStream_t stream) {
    if (!m || !n) return 0;
    if (m < 0 || n < 0 || k <= 0 || k % 16 || (kernel != 0 && kernel != 1)) return -2;
    GemmArgs g{};
    g.a = a; g.b = b; g.sums = sums;
    g.m = m; g.n = n; g.k = k; g.kblocks = (k + 127) / 128;
    if (!offsets_fit(g)) return -2;
    if (kernel == 0) return launch_ring<128, 256, 4, 2, MODE_ROW, false, false, DT_BF16, true, false>(g, stream);
    // the block kernel reads scales (sa_t) and channel scales (sb) that its discarded folds use: any readable memory of
    // the right size (the sums buffer, m * n * kblocks words) serves
    g.sa_t = reinterpret_cast<const float*>(sums);
    g.sb = reinterpret_cast<const float*>(sums);
    g.tiles_m = (m + 255) / 256;
    g.tiles_n = (n + 191) / 192;
    gemm_pingpong<256, 192, 2, 4, MODE_BLOCK, false, true, DT_BF16, false, true, false, true, pp_mf<MODE_BLOCK>><<<g.tiles_m * g.tiles_n, 512, 0, stream>>>(g);
    return int(hipGetLastError());
}

// The matrix-core rate probe over `blocks` workgroups of 4 waves; operands holds blocks * 4 * 8 * 64 16-byte fragments,
// out blocks * 256 ints. Ops per call: blocks * 4 * iters * 16 * 65536 for either shape.
// shape 0: v_mfma_i32_32x32x32_i8, 1: v_mfma_i32_16x16x64_i8 (the same ops per call).
WQ8_API int wq8_debug_mfma_probe(const void* operands, int* out, int blocks, int iters, int shape, hipStream_t stream) {
    if (blocks <= 0 || iters <= 0 || (shape != 0 && shape != 1)) return -2;
    if (shape == 0) mfma_probe<<<blocks, 256, 0, stream>>>(static_cast<const v4i*>(operands), out, iters);
    else mfma_probe16<<<blocks, 256, 0, stream>>>(static_cast<const v4i*>(operands), out, iters);
    return int(hipGetLastError());
}
