// matmul_waves_nt.hip -- the gemm_waves_kernel instantiations behind the plain decode GEMM, weight stream with
// the non-temporal load policy (gemm_launch.h).
#include "gemm_launch.h"

namespace sandy_hip {
template void launch_waves_plain<true>(int, int, int, dim3, hipStream_t, const GemmArgs&);
} // namespace sandy_hip
