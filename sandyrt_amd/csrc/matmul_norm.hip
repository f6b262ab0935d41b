// matmul_norm.hip -- the decode GEMM with the RMSNorm prologue
// (gemm_waves_kernel<..., NORM = true>, gemm.h): the instantiations behind
// sandy_hip_matmul_rms, dispatched by matmul.hip's host heuristic.  A
// translation unit of its own so it compiles in parallel with matmul.hip.
#include "gemm.h"

namespace sandy_hip {

void launch_waves_norm(int variant, int cps, int qdepth, dim3 grid, hipStream_t stream, const GemmArgs& g) {
#define NORM_RUN(RT_, CT_, OCC_, R_)                                                                            \
    case R_:                                                                                                    \
        if (qdepth >= 4 && R_ >= 4 && RT_ * CT_ <= 2)                                                           \
            hipLaunchKernelGGL((gemm_waves_kernel<RT_, CT_, 4, R_, 1, true>), grid, dim3(256), 0, stream, g);  \
        else                                                                                                    \
            hipLaunchKernelGGL((gemm_waves_kernel<RT_, CT_, 2, R_, OCC_, true>), grid, dim3(256), 0, stream, g); \
        break;
#define NORM_CPS(RT_, CT_, OCC_)                                                                          \
    switch (cps) {                                                                                        \
        NORM_RUN(RT_, CT_, OCC_, 2) NORM_RUN(RT_, CT_, OCC_, 3) NORM_RUN(RT_, CT_, OCC_, 4)              \
        NORM_RUN(RT_, CT_, OCC_, 5) NORM_RUN(RT_, CT_, OCC_, 6) NORM_RUN(RT_, CT_, OCC_, 8)              \
        NORM_RUN(RT_, CT_, OCC_, 10) NORM_RUN(RT_, CT_, OCC_, 12)                                        \
    }
    // variants as in matmul.hip: (RT, CT) = 0 (1, 1), 1 (2, 1), 3 (2, 2), 4 (1, 2), 5 (2, 4), 6 (1, 4)
    switch (variant) {
        case 0: NORM_CPS(1, 1, 4); break;
        case 1: NORM_CPS(2, 1, 4); break;
        case 3: NORM_CPS(2, 2, 2); break;
        case 4: NORM_CPS(1, 2, 4); break;
        case 5: NORM_CPS(2, 4, 2); break;
        default: NORM_CPS(1, 4, 2); break;
    }
#undef NORM_RUN
#undef NORM_CPS
}

} // namespace sandy_hip
