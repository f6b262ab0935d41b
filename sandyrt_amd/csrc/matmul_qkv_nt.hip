// matmul_qkv_nt.hip -- the gemm_waves_kernel instantiations behind the q/k/v decode GEMM with the RoPE + paged-
// append epilogue (sandy_hip_device_matmul_qkv), weight stream with the non-temporal load policy
// (gemm_launch.h).
#include "gemm_launch.h"

namespace sandy_hip {
template void launch_waves_qkv<true>(int, int, int, bool, dim3, hipStream_t, const GemmArgs&);
} // namespace sandy_hip
