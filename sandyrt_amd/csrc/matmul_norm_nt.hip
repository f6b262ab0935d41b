// matmul_norm_nt.hip -- the gemm_waves_kernel instantiations behind the decode GEMM with the RMSNorm prologue
// (sandy_hip_matmul_rms), weight stream with the non-temporal load policy (gemm_launch.h).
#include "gemm_launch.h"

namespace sandy_hip {
template void launch_waves_norm<true>(int, int, int, dim3, hipStream_t, const GemmArgs&);
} // namespace sandy_hip
