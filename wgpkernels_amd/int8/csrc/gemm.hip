// INT8 x INT8 GEMM on gfx950 matrix cores (v_mfma_i32_16x16x64_i8 in the ping-pong kernels, v_mfma_i32_32x32x32_i8 in
// the ring kernels), all modes of the reference's gemm_s8 (wgpkernels/int8/int8_gemm.cu, K8:528-986):
//   row     Y = float(A.B) * sa[r] * sb[c] + bias
//   exact   two activation operands hi / lo:   (float(hi.B) + float(lo.B) / 254) * sa[r] * sb[c] + bias
//   block   sa per token and 128-element K block: the exact INT32 sums of each block are scaled into FP32
//   +g      weight scales per channel and 128-element K block (block and exact modes)
// then Y = R + rscale * Y (optional residual, may alias Y), one rounding to BF16 / FP16.
// Kernels: gemm_pingpong (gemm_pingpong.h) for the long tiles of every mode but block in the reference order, gemm_ring
// (gemm_ring.h) for those and the short tiles.
// Launch side: gemm_launch.h; per-dtype kernel instantiations: gemm_bf16.hip, gemm_f16.hip. C ABI below.
#include "gemm_launch.h"
#include "wq8_abi.h"
#include <mutex>

namespace wq8 {

thread_local GemmArgs g_gemm_extra{};  // row offsets / segments of the wrapping entry points

// Block scales (rows x cols, one column per 128-element k-block; row r of the source at src + (shift + r) * cols)
// transposed to dst[c * rows + r]: the GEMM then reads a k-block's scales of 64 consecutive tokens or channels as 256
// contiguous bytes. A 256-thread workgroup moves a 32 x 32 tile through LDS: coalesced row reads, coalesced column
// writes, and the whole grid in flight at once (one workgroup per 32 rows and 32 columns), so that a call with a few
// dozen rows costs a launch and one memory round trip rather than one thread's walk along its row.
__global__ void __launch_bounds__(256) transpose_scales(const float* src, float* dst, int rows, int cols, const long long* counter,
                                                        long long in_first, long long in_step, float divisor) {
    __shared__ float tile[32][33];
    const long long shift = counter ? in_first + *counter * in_step : 0;
    const int r0 = blockIdx.x * 32, c0 = blockIdx.y * 32, tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
#pragma unroll
    for (int j = 0; j < 32; j += 8) {
        const int r = r0 + ty + j, c = c0 + tx;
        if (r < rows && c < cols) {
            const float v = src[(shift + r) * int64_t(cols) + c];
            tile[ty + j][tx] = divisor == 1.0f ? v : v / divisor;
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 32; j += 8) {
        const int c = c0 + ty + j, r = r0 + tx;
        if (c < cols && r < rows) dst[int64_t(c) * rows + r] = tile[tx][ty + j];
    }
}

// divisor: 254 for the exact+g weight scales (the kernel's fold takes sb / 254, correctly rounded), else 1
static int transpose(const float* src, float* dst, int rows, int cols, const GemmArgs& g, bool shifted, hipStream_t stream,
                     float divisor = 1.0f) {
    transpose_scales<<<dim3((rows + 31) / 32, (cols + 31) / 32), 256, 0, stream>>>(src, dst, rows, cols, shifted ? g.counter : nullptr,
                                                                                  g.in_first, g.in_step, divisor);
    return int(hipGetLastError());
}

}  // namespace wq8

using namespace wq8;

namespace wq8 {
static int scratch_address(void** out, hipStream_t capturing = nullptr);
}

namespace wq8 {
// sizes[0]: workspace bytes ([transposed block scales][split slots]); sizes[1]: counter bytes (split tiles x 4)
static void gemm_workspace_sizes(int m, int n, int k, int variant, int sms, int split, int64_t* sizes) {
    sizes[0] = sizes[1] = 0;
    Variant v;
    if (!variant_info(variant, v) || m <= 0 || n <= 0 || k <= 0) return;
    int64_t sa_bytes = 0, sb_bytes = 0, slot_bytes = 0, counter_bytes = 0;
    scale_workspace(m, n, k, v, sa_bytes, sb_bytes);
    GemmArgs g{};
    g.m = m; g.n = n; g.k = k; g.kblocks = (k + 127) / 128; g.sms = sms;
    split_workspace(g, v, split, slot_bytes, counter_bytes);
    sizes[0] = sa_bytes + sb_bytes + slot_bytes;
    sizes[1] = counter_bytes;
}
}  // namespace wq8

// The workspace query. It also resolves, once per device, the address of wq8_gemm_noalloc's array on the current
// device: the Python layer makes this query on every GPU when it loads the library, so that no symbol lookup happens
// under graph capture.
WQ8_API void wq8_gemm_workspace(int m, int n, int k, int variant, int sms, int split, int64_t* sizes) {
    void* scratch_ptr = nullptr;
    (void)scratch_address(&scratch_ptr);  // no device (a CPU-only host): nothing to resolve
    gemm_workspace_sizes(m, n, k, variant, sms, split, sizes);
}

WQ8_API int wq8_gemm_select(int m, int n, int k, int hilo, int sms) {
    if (hilo) return estimate_tiles(m, n, k, sms, 128, 256, 1, 1.0) <= estimate_tiles(m, n, k, sms, 32, 128, 2, 0.5) ? 1 : 7;
    return estimate_tiles(m, n, k, sms, 256, 256, 1, 1.0) <= estimate_tiles(m, n, k, sms, 64, 128, 2, 0.5) ? 0 : 6;
}

WQ8_API int wq8_gemm(const int8_t* a, const int8_t* a_lo, const float* sa, const int8_t* b, const float* sb, const void* bias, const void* residual,
                     const void* rscale, void* y, int m, int n, int k, int dtype, int variant, int sms, int split, int* workspace, int* counters,
                     hipStream_t stream) {
    if (!m || !n) return 0;
    Variant v;
    if (!variant_info(variant, v)) return -3;
    if ((v.mode == MODE_EXACT) != (a_lo != nullptr)) return -2;
    if (m < 0 || n < 0 || k <= 0 || k % 16) return -2;
    GemmArgs g = g_gemm_extra;
    g.a = a; g.a_lo = a_lo; g.sa = sa; g.b = b; g.sb = sb; g.bias = bias; g.residual = residual; g.rscale = rscale; g.y = y;
    g.sums = nullptr;
    g.m = m; g.n = n; g.k = k; g.kblocks = (k + 127) / 128; g.sms = sms;
    const bool seg = g.seg_rows > 0;
    if (seg && v.wgroup) return -4;
    if (seg) split = 0;  // segments run whole tiles: their split kernels would spill registers in the mainloop
    int64_t sa_bytes = 0, sb_bytes = 0, slot_bytes = 0, counter_bytes = 0;
    scale_workspace(m, n, k, v, sa_bytes, sb_bytes);
    split_workspace(g, v, split, slot_bytes, counter_bytes);
    // the workspace holds FP32 scales and 16-byte stores of partial sums: 16-byte aligned (device allocations are 256)
    if ((sa_bytes + sb_bytes + slot_bytes) && (reinterpret_cast<uintptr_t>(workspace) & 15)) return -2;
    if (slot_bytes) {
        // split tiles: their partial sums after the scales, their counters in `counters` (zero on entry, left zero;
        // none for the deep split, whose pieces are added by a second launch)
        if (!workspace || (counter_bytes && !counters)) return -2;
        g.split_slots = reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(workspace) + sa_bytes + sb_bytes);
        g.split_counters = counters;
    } else {
        split = 0;
    }
    if (sa_bytes + sb_bytes) {
        if (!workspace) return -2;  // sized by wq8_gemm_workspace
        if (!offsets_fit(g)) return -2;
        uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
        if (sa_bytes) {
            g.sa_t = reinterpret_cast<float*>(ws);
            const int rc = transpose(sa, reinterpret_cast<float*>(ws), m, g.kblocks, g, true, stream);
            if (rc) return rc;
        }
        if (sb_bytes) {
            g.sb_t = reinterpret_cast<float*>(ws + sa_bytes);
            const int rc = transpose(sb, reinterpret_cast<float*>(ws + sa_bytes), n, g.kblocks, g, false, stream,
                                     v.mode == MODE_EXACT ? 254.0f : 1.0f);
            if (rc) return rc;
        }
    }
    if (dtype == DT_F16) return seg ? dispatch_gemm<DT_F16, true>(g, v, split, stream) : dispatch_gemm<DT_F16, false>(g, v, split, stream);
    if (dtype == DT_BF16) return seg ? dispatch_gemm<DT_BF16, true>(g, v, split, stream) : dispatch_gemm<DT_BF16, false>(g, v, split, stream);
    return -1;
}

WQ8_API int wq8_gemm_at(const int8_t* a, const int8_t* a_lo, const float* sa, const int8_t* b, const float* sb, const void* bias, const void* residual,
                        const void* rscale, void* y, int m, int n, int k, int dtype, int variant, int sms, int split, int* workspace, int* counters,
                        const long long* counter, long long first, long long step, long long span, long long scale_step, long long in_first,
                        long long in_step, hipStream_t stream) {
    g_gemm_extra = GemmArgs{};
    g_gemm_extra.counter = counter; g_gemm_extra.first = first; g_gemm_extra.step = step; g_gemm_extra.span = span;
    g_gemm_extra.scale_step = scale_step; g_gemm_extra.in_first = in_first; g_gemm_extra.in_step = in_step;
    const int rc = wq8_gemm(a, a_lo, sa, b, sb, bias, residual, rscale, y, m, n, k, dtype, variant, sms, split, workspace, counters, stream);
    g_gemm_extra = GemmArgs{};
    return rc;
}

WQ8_API int wq8_gemm_segments(const int8_t* a, const int8_t* a_lo, const float* sa, const int8_t* const* bs, const float* const* sbs,
                              const void* const* biases, void* const* ys, int count, int rows, int m, int k, int dtype, int variant, int sms,
                              int split, int* workspace, int* counters, hipStream_t stream) {
    if (count < 1 || count > 4 || rows <= 0 || rows % 8) return -4;
    g_gemm_extra = GemmArgs{};
    g_gemm_extra.seg_rows = rows;
    for (int s = 0; s < count; ++s) {
        g_gemm_extra.seg_b[s] = bs[s]; g_gemm_extra.seg_sb[s] = sbs[s]; g_gemm_extra.seg_bias[s] = biases[s]; g_gemm_extra.seg_y[s] = ys[s];
    }
    const int rc = wq8_gemm(a, a_lo, sa, bs[0], sbs[0], nullptr, nullptr, nullptr, ys[0], m, count * rows, k, dtype, variant, sms, split, workspace,
                            counters, stream);
    g_gemm_extra = GemmArgs{};
    return rc;
}

// ---- allocation-free GEMM --------------------------------------------------------------------------------------------
// For callers that cannot allocate (code under graph capture, serving loops, harnesses that forbid hipMalloc): the
// workspace wq8_gemm takes from its caller lives in a file-scope device array instead. Each GPU the library runs on holds
// its own copy until the process ends; every call on a GPU shares it, so calls that overlap on one GPU race.
namespace wq8 {
constexpr int64_t NOALLOC_SCRATCH_BYTES = int64_t(32) << 20;  // WQ8_GEMM_NOALLOC_MAX_BYTES of include/wq8.h
constexpr int NOALLOC_MAX_DEVICES = 64;
__device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];
static std::mutex g_scratch_mutex;
static void* g_scratch_ptr[NOALLOC_MAX_DEVICES];

// Device address of the current device's copy of `scratch` (looked up once per device; the array's name is only a
// host-side stand-in). 0 on success.
// With a capturing stream, an address not resolved yet is an error (-6): the lookup is not made under capture.
static int scratch_address(void** out, hipStream_t capturing) {
    int device = 0;
    if (hipError_t e = hipGetDevice(&device)) {
        (void)hipGetLastError();
        return int(e);
    }
    if (device < 0 || device >= NOALLOC_MAX_DEVICES) return -2;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[device]) {
        hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
        if (capturing && hipStreamIsCapturing(capturing, &status) == hipSuccess && status != hipStreamCaptureStatusNone) return -6;
        void* p = nullptr;
        if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) return int(e);
        g_scratch_ptr[device] = p;
    }
    *out = g_scratch_ptr[device];
    return 0;
}

__global__ void __launch_bounds__(256) zero_words(int* p, int words) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < words) p[i] = 0;
}
}  // namespace wq8

WQ8_API int wq8_gemm_noalloc(const int8_t* a, const int8_t* a_lo, const float* sa, const int8_t* b, const float* sb, const void* bias,
                             const void* residual, const void* rscale, void* y, int m, int n, int k, int dtype, int variant, int sms,
                             int split, hipStream_t stream) {
    if (!m || !n) return 0;
    int64_t sizes[2] = {0, 0};
    gemm_workspace_sizes(m, n, k, variant, sms, split, sizes);  // the query without the address lookup
    const int64_t slot_bytes = align256(sizes[0]);
    if (slot_bytes + sizes[1] > NOALLOC_SCRATCH_BYTES) return -5;
    void* base = nullptr;
    if (int rc = scratch_address(&base, stream)) return rc;
    uint8_t* ws = static_cast<uint8_t*>(base);
    int* counters = nullptr;
    if (sizes[1]) {
        // split counters start at zero: cleared by a kernel (a memset node would be wrong in a replayed graph)
        counters = reinterpret_cast<int*>(ws + slot_bytes);
        const int words = int(sizes[1] / 4);
        zero_words<<<(words + 255) / 256, 256, 0, stream>>>(counters, words);
        if (hipError_t e = hipGetLastError()) return int(e);
    }
    return wq8_gemm(a, a_lo, sa, b, sb, bias, residual, rscale, y, m, n, k, dtype, variant, sms, split,
                    sizes[0] ? reinterpret_cast<int*>(ws) : nullptr, counters, stream);
}
