// matmul_norm.hip -- the gemm_waves_kernel instantiations behind the decode GEMM with the RMSNorm prologue
// (sandy_hip_matmul_rms), weight stream with the default load policy (gemm_launch.h).
#include "gemm_launch.h"

namespace sandy_hip {
template void launch_waves_norm<false>(int, int, int, dim3, hipStream_t, const GemmArgs&);
} // namespace sandy_hip
