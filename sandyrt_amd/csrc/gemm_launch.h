// gemm_launch.h -- the launchers of gemm_waves_kernel (gemm.h) for every tile
// variant and run length the host heuristic of matmul.hip picks.  Included by
// one translation unit per (form, NT) -- matmul_waves*.hip, matmul_norm*.hip,
// matmul_qkv*.hip -- each instantiating one of them, so the kernels compile
// in parallel.
#pragma once
#include "gemm.h"

namespace sandy_hip {

// (RT, CT) = 0 (1, 1), 1 (2, 1), 3 (2, 2), 4 (1, 2), 5 (2, 4), 6 (1, 4); four
// chunks in flight only for RT * CT <= 2 (register bound)
#define SANDY_WAVES_RUN(RT_, CT_, OCC_, R_, NORM_)                                                                  \
    case R_:                                                                                                        \
        if (qdepth >= 4 && R_ >= 4 && RT_ * CT_ <= 2)                                                               \
            hipLaunchKernelGGL((gemm_waves_kernel<RT_, CT_, 4, R_, 1, NORM_, false, NT>), grid, dim3(256), 0,      \
                               stream, g);                                                                          \
        else                                                                                                        \
            hipLaunchKernelGGL((gemm_waves_kernel<RT_, CT_, 2, R_, OCC_, NORM_, false, NT>), grid, dim3(256), 0,   \
                               stream, g);                                                                          \
        break;
#define SANDY_WAVES_CPS(RT_, CT_, OCC_, NORM_)                                                                  \
    switch (cps) {                                                                                              \
        SANDY_WAVES_RUN(RT_, CT_, OCC_, 2, NORM_) SANDY_WAVES_RUN(RT_, CT_, OCC_, 3, NORM_)                    \
        SANDY_WAVES_RUN(RT_, CT_, OCC_, 4, NORM_) SANDY_WAVES_RUN(RT_, CT_, OCC_, 5, NORM_)                    \
        SANDY_WAVES_RUN(RT_, CT_, OCC_, 6, NORM_) SANDY_WAVES_RUN(RT_, CT_, OCC_, 8, NORM_)                    \
        SANDY_WAVES_RUN(RT_, CT_, OCC_, 10, NORM_) SANDY_WAVES_RUN(RT_, CT_, OCC_, 12, NORM_)                  \
    }
#define SANDY_WAVES_VARIANTS(NORM_)                    \
    switch (variant) {                                 \
        case 0: SANDY_WAVES_CPS(1, 1, 4, NORM_); break; \
        case 1: SANDY_WAVES_CPS(2, 1, 4, NORM_); break; \
        case 3: SANDY_WAVES_CPS(2, 2, 2, NORM_); break; \
        case 4: SANDY_WAVES_CPS(1, 2, 4, NORM_); break; \
        case 5: SANDY_WAVES_CPS(2, 4, 2, NORM_); break; \
        default: SANDY_WAVES_CPS(1, 4, 2, NORM_); break; \
    }

template <bool NT>
void launch_waves_plain(int variant, int cps, int qdepth, dim3 grid, hipStream_t stream, const GemmArgs& g) {
    SANDY_WAVES_VARIANTS(false)
}

template <bool NT>
void launch_waves_norm(int variant, int cps, int qdepth, dim3 grid, hipStream_t stream, const GemmArgs& g) {
    SANDY_WAVES_VARIANTS(true)
}

// 16-row tiles of 16 or 32 columns (variant 0 or 4), every run length of the
// plain kernels -- the run length fixes how K is split over the waves, so the
// products match the plain GEMM's bit for bit -- and four chunks in flight
// from run length 4, which change no arithmetic
template <bool NT>
void launch_waves_qkv(int variant, int cps, int qdepth, bool norm, dim3 grid, hipStream_t stream, const GemmArgs& g) {
    (void)qdepth;
#define SANDY_QKV_RUN(CT_, R_, N_)                                                                                 \
    case R_:                                                                                                       \
        if (R_ >= 4)                                                                                               \
            hipLaunchKernelGGL((gemm_waves_kernel<1, CT_, 4, R_, 1, N_, true, NT>), grid, dim3(256), 0, stream, g); \
        else                                                                                                       \
            hipLaunchKernelGGL((gemm_waves_kernel<1, CT_, 2, R_, 4, N_, true, NT>), grid, dim3(256), 0, stream, g); \
        break;
#define SANDY_QKV_CPS(CT_, N_)                                                                                     \
    switch (cps) {                                                                                                 \
        SANDY_QKV_RUN(CT_, 2, N_) SANDY_QKV_RUN(CT_, 3, N_) SANDY_QKV_RUN(CT_, 4, N_) SANDY_QKV_RUN(CT_, 5, N_)    \
        SANDY_QKV_RUN(CT_, 6, N_) SANDY_QKV_RUN(CT_, 8, N_) SANDY_QKV_RUN(CT_, 10, N_)                             \
        default: SANDY_QKV_RUN(CT_, 12, N_)                                                                        \
    }
    if (norm) {
        if (variant == 0) SANDY_QKV_CPS(1, true)
        else SANDY_QKV_CPS(2, true)
    } else {
        if (variant == 0) SANDY_QKV_CPS(1, false)
        else SANDY_QKV_CPS(2, false)
    }
#undef SANDY_QKV_RUN
#undef SANDY_QKV_CPS
}

#undef SANDY_WAVES_VARIANTS
#undef SANDY_WAVES_CPS
#undef SANDY_WAVES_RUN

} // namespace sandy_hip
