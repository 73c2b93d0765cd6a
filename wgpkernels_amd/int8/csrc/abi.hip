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
