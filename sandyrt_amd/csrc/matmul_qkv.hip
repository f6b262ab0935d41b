// matmul_qkv.hip -- the decode q/k/v GEMM with the RoPE + paged-append
// epilogue (gemm_waves_kernel<..., ROPE = true>, gemm.h), with and without the
// RMSNorm prologue: the instantiations behind sandy_hip_device_matmul_qkv,
// dispatched by matmul.hip's host heuristic (16-row tiles of 16 or 32
// columns, every run length of the plain kernels -- the run length fixes how
// K is split over the waves, so the products match the plain GEMM's bit for
// bit -- and four chunks in flight from run length 4, which change no arithmetic).
#include "gemm.h"

namespace sandy_hip {

void launch_waves_qkv(int variant, int cps, int qdepth, bool norm, dim3 grid, hipStream_t stream, const GemmArgs& g) {
    (void)qdepth;
#define QKV_RUN(CT_, R_, N_)                                                                                    \
    case R_:                                                                                                    \
        if (R_ >= 4)                                                                                            \
            hipLaunchKernelGGL((gemm_waves_kernel<1, CT_, 4, R_, 1, N_, true>), grid, dim3(256), 0, stream, g); \
        else                                                                                                    \
            hipLaunchKernelGGL((gemm_waves_kernel<1, CT_, 2, R_, 4, N_, true>), grid, dim3(256), 0, stream, g); \
        break;
#define QKV_CPS(CT_, N_)                                                                                          \
    switch (cps) {                                                                                                \
        QKV_RUN(CT_, 2, N_) QKV_RUN(CT_, 3, N_) QKV_RUN(CT_, 4, N_) QKV_RUN(CT_, 5, N_) QKV_RUN(CT_, 6, N_)      \
        QKV_RUN(CT_, 8, N_) QKV_RUN(CT_, 10, N_) default: QKV_RUN(CT_, 12, N_)                                  \
    }
    if (norm) {
        if (variant == 0) QKV_CPS(1, true)
        else QKV_CPS(2, true)
    } else {
        if (variant == 0) QKV_CPS(1, false)
        else QKV_CPS(2, false)
    }
#undef QKV_RUN
#undef QKV_CPS
}

} // namespace sandy_hip
