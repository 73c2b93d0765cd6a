// Library identity and the cold-cache helper of the autotuner.
// Reference: wgpkernels/int8/int8_gemm.cu (K8) :1349-1352 (wq8_abi / wq8_features), :1984-2016 (L2 flush).
#include "wq8_common.h"
#include "wq8_abi.h"

// ABI version checked by the Python layer on load (I:69 of the reference): argument lists unchanged.
WQ8_API int wq8_abi() { return 11; }

// bit 0: per-(channel, 128-element K block) weight scales (variants 12-14)
WQ8_API int wq8_features() { return 1; }

namespace wq8 {
// Reads the whole buffer with ordinary (allocating) 16-byte loads, so that later launches find neither weights nor
// activations in L2 or in the Infinity Cache (MALL): the buffer must exceed their sum (4 MiB per XCD x 8 + 256 MiB on
// MI355X). Non-temporal loads would stream past the caches and leave what they hold in place.
__global__ void __launch_bounds__(256) cache_flush_read(const u32x4* __restrict__ p, int64_t n16, int* sink) {
    u32x4 acc = {0, 0, 0, 0};
    for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n16; i += int64_t(gridDim.x) * blockDim.x) acc ^= p[i];
    if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x5bd1e995u && sink) *sink = 1;  // keeps the loads; practically never stores
}
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

static void* g_flush = nullptr;
static int64_t g_flush_bytes = 0;
static int g_flush_device = -1;
}  // namespace wq8

using namespace wq8;

// Reads `bytes` of a library-owned buffer (allocated on first use on `device`, outside PyTorch's allocator) on
// `stream`; nonzero when the memory cannot be allocated.
WQ8_API int wq8_l2_flush(int device, int64_t bytes, hipStream_t stream) {
    if (g_flush_bytes < bytes || g_flush_device != device) {
        int previous = 0;
        (void)hipGetDevice(&previous);
        (void)hipSetDevice(device);
        if (g_flush) (void)hipFree(g_flush);
        g_flush = nullptr;
        g_flush_bytes = 0;
        g_flush_device = -1;
        if (hipMalloc(&g_flush, bytes + 16) != hipSuccess) {
            (void)hipGetLastError();
            g_flush = nullptr;
            (void)hipSetDevice(previous);
            return 1;
        }
        g_flush_bytes = bytes;
        g_flush_device = device;
        (void)hipSetDevice(previous);
    }
    cache_flush_read<<<4096, 256, 0, stream>>>(static_cast<const u32x4*>(g_flush), bytes / 16,
                                                reinterpret_cast<int*>(static_cast<char*>(g_flush) + (bytes & ~int64_t(3))));
    return int(hipGetLastError());
}

WQ8_API void wq8_l2_flush_release() {
    if (g_flush) {
        (void)hipDeviceSynchronize();
        (void)hipFree(g_flush);
    }
    g_flush = nullptr;
    g_flush_bytes = 0;
    g_flush_device = -1;
}

// Test entry point (no counterpart in the reference): the matrix-core rate probe over `blocks` workgroups of 4 waves;
// operands holds blocks * 4 * 8 * 64 16-byte fragments, out blocks * 256 ints. Ops per call: blocks * 4 * iters * 16 *
// 65536.
WQ8_API int wq8_debug_mfma_probe(const void* operands, int* out, int blocks, int iters, hipStream_t stream) {
    if (blocks <= 0 || iters <= 0) return -2;
    mfma_probe<<<blocks, 256, 0, stream>>>(static_cast<const v4i*>(operands), out, iters);
    return int(hipGetLastError());
}
