// Internal declarations shared by the library's translation units (the public C-ABI is include/wq8.h).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define WQ8_API extern "C" __attribute__((visibility("default")))

namespace wq8 {
// Row offset read on the GPU for CUDA-graph-style loops: rows first + counter[0] * step.
struct RowOffsetArgs { const long long* counter; long long first, step; };
}  // namespace wq8
