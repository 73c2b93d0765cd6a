// The INT8 GEMM kernels with F16 outputs: the dispatch of gemm_launch.h instantiated for this dtype (its kernels
// compile here, in parallel with the other dtype's).
#include "gemm_launch.h"

namespace wq8 {
template int dispatch_gemm<DT_F16, false>(GemmArgs&, const Variant&, int, hipStream_t);
template int dispatch_gemm<DT_F16, true>(GemmArgs&, const Variant&, int, hipStream_t);
}  // namespace wq8
