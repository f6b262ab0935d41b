// norm.hip -- RMSNorm, LayerNorm and the residual-add + RMSNorm pair.
//
// Semantics follow the reference CPU math: src/core/TensorCalc.cpp:1953-2000
// (rms_norm_impl: double sum of squares, float inverse RMS, y = x * inv * w)
// and :2010-2077 (layer_norm: double mean and variance, float inverse std,
// y = (x - mean) * inv * w + b).  The reference CUDA kernels
// (CudaNormKernels.cu:146-206) use one 256-thread block per row with a shared
// memory tree and read x two or three times.
//
// gfx950 design: one wave64 per row; each lane owns 8-element chunks loaded
// with 128-bit loads and kept in registers, so x (and the residual) is read
// from HBM exactly once and the output written once.  Row statistics are
// accumulated in double like the reference (bf16 squares are exact in double,
// so the bf16 sum is order independent and the result bit-matches the CPU),
// reduced with wave butterflies; no LDS, no block barriers.  Rows wider than
// 4096 elements or not a multiple of 8 use a block-per-row two-pass kernel.
#include "common.h"

namespace sandy_hip {
namespace {

constexpr int kRowsPerBlock = 4;  // 4 waves, one row each

// FULL: cols == NCH * 512, so every lane owns exactly NCH chunks and no load
// is guarded (guards around the loads cost ~15% here by serialising them).
// All of a lane's loads are issued before any value is used.  NTL reads the
// streamed inputs non-temporally.
// Loads are issued before any is used, without guards: a chunk past the row
// end re-reads the row's last chunk (its values are not used), since a
// guarded load is sunk into its guard and waits there.  WPRE (few rows, a
// latency-bound launch) also requests the weights with the row; with many
// rows the weights are L2-resident and are read after the reduction, which
// keeps the register count down.
template <typename T, int NCH, bool RESID, bool HASW, bool FULL, bool WPRE>
__global__ __launch_bounds__(256) void rms_rows_kernel(
        const void* __restrict__ x, const void* __restrict__ resid, const void* __restrict__ w,
        void* __restrict__ sum_out, void* __restrict__ out, int64_t rows, int cols, float eps) {
    const int lane = threadIdx.x & 63;
    // a wave per row: WPRE launches one-wave workgroups, the others four
    const int64_t row = WPRE ? static_cast<int64_t>(blockIdx.x)
                             : static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int chunks = cols >> 3;
    const int64_t base = row * cols;
    typename Vec8<T>::raw xr[NCH], hr[NCH], wr[NCH];
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int c = lane + j * 64;
        const int cc = FULL || c < chunks ? c : chunks - 1;
        xr[j] = Vec8<T>::load_raw_nt(x, base + cc * 8);
        if constexpr (RESID) hr[j] = Vec8<T>::load_raw_nt(resid, base + cc * 8);
    }
    if constexpr (HASW && WPRE) {
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int c = lane + j * 64;
            wr[j] = Vec8<T>::load_raw(w, (FULL || c < chunks ? c : chunks - 1) * 8);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep them in flight with the row (not sunk to their use)
    }
    float v[NCH][8];
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int c = lane + j * 64;
        const bool in = FULL || c < chunks;
        Vec8<T>::unpack(xr[j], v[j]);
        if constexpr (RESID) {
            float h[8];
            Vec8<T>::unpack(hr[j], h);
#pragma unroll
            for (int i = 0; i < 8; i++) v[j][i] = Vec8<T>::round(__fadd_rn(v[j][i], h[i]));
            if (in) Vec8<T>::store(sum_out, base + c * 8, v[j]);
        }
#pragma unroll
        for (int i = 0; i < 8; i++) acc += in ? static_cast<double>(v[j][i]) * static_cast<double>(v[j][i]) : 0.0;
    }
    acc = wave_sum(acc);
    const float inv = 1.0f / sqrtf(static_cast<float>(acc / static_cast<double>(cols)) + eps);
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int c = lane + j * 64;
        if (FULL || c < chunks) {
            float y[8];
            float wv[8];
            if constexpr (HASW) {
                if constexpr (WPRE) Vec8<T>::unpack(wr[j], wv);
                else Vec8<T>::load(w, c * 8, wv);
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                y[i] = __fmul_rn(v[j][i], inv);
                if constexpr (HASW) y[i] = __fmul_rn(y[i], wv[i]);
            }
            Vec8<T>::store(out, base + c * 8, y);
        }
    }
}

template <typename T, int NCH>
__global__ __launch_bounds__(256) void layer_rows_kernel(
        const void* __restrict__ x, const void* __restrict__ w, const void* __restrict__ b,
        void* __restrict__ out, int64_t rows, int cols, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int chunks = cols >> 3;
    const int64_t base = row * cols;
    float v[NCH][8];
    double sum = 0.0;
    // row, weight and bias loads all issued first, unguarded (clamped chunk:
    // a guarded load waits behind its guard); used only for c < chunks
    typename Vec8<T>::raw xr[NCH], wr[NCH], br[NCH];
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int c = lane + j * 64;
        const int cc = c < chunks ? c : chunks - 1;
        xr[j] = Vec8<T>::load_raw(x, base + cc * 8);
        wr[j] = Vec8<T>::load_raw(w, cc * 8);
        br[j] = Vec8<T>::load_raw(b, cc * 8);
    }
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int c = lane + j * 64;
        Vec8<T>::unpack(xr[j], v[j]);
        if (c < chunks) {
#pragma unroll
            for (int i = 0; i < 8; i++) sum += static_cast<double>(v[j][i]);
        }
    }
    const double mean = wave_sum(sum) / static_cast<double>(cols);
    double var = 0.0;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int c = lane + j * 64;
        if (c < chunks) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const double d = static_cast<double>(v[j][i]) - mean;
                var += d * d;
            }
        }
    }
    var = wave_sum(var) / static_cast<double>(cols);
    const float inv = 1.0f / sqrtf(static_cast<float>(var) + eps);
    const float meanf = static_cast<float>(mean);
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int c = lane + j * 64;
        if (c < chunks) {
            float wv[8], bv[8], y[8];
            Vec8<T>::unpack(wr[j], wv);
            Vec8<T>::unpack(br[j], bv);
#pragma unroll
            for (int i = 0; i < 8; i++)
                y[i] = __fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(v[j][i], meanf), inv), wv[i]), bv[i]);
            Vec8<T>::store(out, base + c * 8, y);
        }
    }
}

// Generic row kernel: one 256-thread block per row, any width, scalar access.
// kind 0 = rms (w may be null), 1 = layer, 2 = add + rms.
template <typename T>
__global__ __launch_bounds__(256) void norm_generic_kernel(
        int kind, const void* __restrict__ x, const void* __restrict__ resid, const void* __restrict__ w,
        const void* __restrict__ b, void* __restrict__ sum_out, void* __restrict__ out, int64_t cols, float eps) {
    __shared__ double red[4];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * cols;
    const int tid = threadIdx.x;
    auto load_x = [&](int64_t c) -> float {
        float v = Vec8<T>::load1(x, base + c);
        if (kind == 2) v = Vec8<T>::round(__fadd_rn(v, Vec8<T>::load1(resid, base + c)));
        return v;
    };
    auto block_sum = [&](double v) -> double {
        v = wave_sum(v);
        __syncthreads();
        if ((tid & 63) == 0) red[tid >> 6] = v;
        __syncthreads();
        return red[0] + red[1] + red[2] + red[3];
    };
    if (kind == 2) {
        for (int64_t c = tid; c < cols; c += 256) Vec8<T>::store1(sum_out, base + c, load_x(c));
        __syncthreads();
    }
    const void* src = kind == 2 ? sum_out : x;
    if (kind == 1) {
        double s = 0.0;
        for (int64_t c = tid; c < cols; c += 256) s += static_cast<double>(Vec8<T>::load1(src, base + c));
        const double mean = block_sum(s) / static_cast<double>(cols);
        double q = 0.0;
        for (int64_t c = tid; c < cols; c += 256) {
            const double d = static_cast<double>(Vec8<T>::load1(src, base + c)) - mean;
            q += d * d;
        }
        const double var = block_sum(q) / static_cast<double>(cols);
        const float inv = 1.0f / sqrtf(static_cast<float>(var) + eps);
        const float meanf = static_cast<float>(mean);
        for (int64_t c = tid; c < cols; c += 256) {
            float y = __fmul_rn(__fsub_rn(Vec8<T>::load1(src, base + c), meanf), inv);
            y = __fadd_rn(__fmul_rn(y, Vec8<T>::load1(w, c)), Vec8<T>::load1(b, c));
            Vec8<T>::store1(out, base + c, y);
        }
        return;
    }
    double q = 0.0;
    for (int64_t c = tid; c < cols; c += 256) {
        const double v = static_cast<double>(Vec8<T>::load1(src, base + c));
        q += v * v;
    }
    const double total = block_sum(q);
    const float inv = 1.0f / sqrtf(static_cast<float>(total / static_cast<double>(cols)) + eps);
    for (int64_t c = tid; c < cols; c += 256) {
        float y = __fmul_rn(Vec8<T>::load1(src, base + c), inv);
        if (w) y = __fmul_rn(y, Vec8<T>::load1(w, c));
        Vec8<T>::store1(out, base + c, y);
    }
}

template <typename T, int NCH, bool RESID, bool HASW>
void launch_rms_n(bool full, dim3 grid, hipStream_t s, const void* x, const void* r, const void* w, void* so,
                  void* out, int64_t rows, int cols, float eps) {
    // weights with the row when the launch is a few waves (latency-bound);
    // then also one wave per workgroup, so the rows spread over as many CUs
    const bool wpre = rows <= 1024;
    const dim3 g = wpre ? dim3(static_cast<unsigned>(rows)) : grid;
    const dim3 blk = wpre ? dim3(64) : dim3(256);
#define RMS_LAUNCH(F, P) \
    hipLaunchKernelGGL((rms_rows_kernel<T, NCH, RESID, HASW, F, P>), g, blk, 0, s, x, r, w, so, out, rows, cols, eps)
    if (full) {
        if (wpre) RMS_LAUNCH(true, true);
        else RMS_LAUNCH(true, false);
    } else {
        if (wpre) RMS_LAUNCH(false, true);
        else RMS_LAUNCH(false, false);
    }
#undef RMS_LAUNCH
}

template <typename T, bool RESID, bool HASW>
void launch_rms(int nch, dim3 grid, hipStream_t s, const void* x, const void* r, const void* w, void* so,
                void* out, int64_t rows, int cols, float eps) {
    const bool full = cols == nch * 512;
    switch (nch) {
        case 1: launch_rms_n<T, 1, RESID, HASW>(full, grid, s, x, r, w, so, out, rows, cols, eps); break;
        case 2: launch_rms_n<T, 2, RESID, HASW>(full, grid, s, x, r, w, so, out, rows, cols, eps); break;
        case 4: launch_rms_n<T, 4, RESID, HASW>(full, grid, s, x, r, w, so, out, rows, cols, eps); break;
        default: launch_rms_n<T, 8, RESID, HASW>(full, grid, s, x, r, w, so, out, rows, cols, eps); break;
    }
}

template <typename T>
void launch_layer(int nch, dim3 grid, hipStream_t s, const void* x, const void* w, const void* b, void* out,
                  int64_t rows, int cols, float eps) {
    switch (nch) {
        case 1: hipLaunchKernelGGL((layer_rows_kernel<T, 1>), grid, dim3(256), 0, s, x, w, b, out, rows, cols, eps); break;
        case 2: hipLaunchKernelGGL((layer_rows_kernel<T, 2>), grid, dim3(256), 0, s, x, w, b, out, rows, cols, eps); break;
        case 4: hipLaunchKernelGGL((layer_rows_kernel<T, 4>), grid, dim3(256), 0, s, x, w, b, out, rows, cols, eps); break;
        default: hipLaunchKernelGGL((layer_rows_kernel<T, 8>), grid, dim3(256), 0, s, x, w, b, out, rows, cols, eps); break;
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// kind: 0 rms, 1 layer, 2 add+rms
int run_norm(int kind, const SandyTensor* x, const SandyTensor* resid, const SandyTensor* weight,
             const SandyTensor* bias, double epsilon, const SandyTensor* sum_out, const SandyTensor* out,
             hipStream_t stream, Err e) {
    const char* op = kind == 1 ? "layer_norm" : "rms_norm";
    if (!valid_rank(x) || !valid_rank(out)) return fail(e, SANDY_ERR_INVALID, "%s tensor rank out of range", op);
    if (!is_float(x->dtype)) return fail(e, SANDY_ERR_INVALID, "%s input unsupported dtype", op);
    if (x->rank < 1) return fail(e, SANDY_ERR_INVALID, "%s input must have rank >= 1", op);
    if (!same_shape(*x, *out)) return fail(e, SANDY_ERR_INVALID, "%s output shape mismatch", op);
    if (out->dtype != x->dtype) return fail(e, SANDY_ERR_INVALID, "%s output dtype mismatch", op);
    const int64_t cols = x->dims[x->rank - 1];
    if (weight) {
        if (weight->dtype != x->dtype) return fail(e, SANDY_ERR_INVALID, "%s operands must have same dtype", op);
        if (weight->rank != 1) return fail(e, SANDY_ERR_INVALID, "%s weight must have rank 1", op);
        if (weight->dims[0] != cols) return fail(e, SANDY_ERR_INVALID, "%s weight dimension mismatch", op);
    }
    if (kind == 1) {
        if (!weight || !bias) return fail(e, SANDY_ERR_INVALID, "layer_norm requires weight and bias");
        if (bias->dtype != x->dtype) return fail(e, SANDY_ERR_INVALID, "layer_norm operands must have same dtype");
        if (bias->rank != 1) return fail(e, SANDY_ERR_INVALID, "layer_norm bias must have rank 1");
        if (bias->dims[0] != cols) return fail(e, SANDY_ERR_INVALID, "layer_norm bias dimension mismatch");
    }
    if (kind == 2) {
        if (!resid || !sum_out) return fail(e, SANDY_ERR_INVALID, "add_rms_norm requires residual and sum output");
        if (!same_shape(*x, *resid) || !same_shape(*x, *sum_out))
            return fail(e, SANDY_ERR_INVALID, "add operands must have same shape");
        if (resid->dtype != x->dtype || sum_out->dtype != x->dtype)
            return fail(e, SANDY_ERR_INVALID, "add operands must have same dtype");
    }
    const SandyTensor* all[5] = {x, out, weight, bias, kind == 2 ? resid : nullptr};
    for (const SandyTensor* t : all)
        if (t && !contiguous(*t)) return fail(e, SANDY_ERR_UNSUPPORTED, "%s requires contiguous tensors", op);
    if (kind == 2 && !contiguous(*sum_out)) return fail(e, SANDY_ERR_UNSUPPORTED, "%s requires contiguous tensors", op);
    const int64_t total = numel(*x);
    if (total == 0 || cols == 0) return ok(e);
    const int64_t rows = total / cols;
    const float eps = static_cast<float>(epsilon);
    const bool bf = x->dtype == SANDY_BF16;

    const void* px = base_ptr(*x);
    void* po = base_ptr(*out);
    const void* pw = weight ? base_ptr(*weight) : nullptr;
    const void* pb = bias ? base_ptr(*bias) : nullptr;
    const void* pr = kind == 2 ? base_ptr(*resid) : nullptr;
    void* ps = kind == 2 ? base_ptr(*sum_out) : nullptr;

    bool fast = cols % 8 == 0 && cols <= 4096;
    for (const void* p : {px, static_cast<const void*>(po), pw, pb, pr, static_cast<const void*>(ps)})
        if (p && !aligned16(p)) fast = false;
    if (fast) {
        const int chunks = static_cast<int>(cols / 8);
        const int nch = chunks <= 64 ? 1 : chunks <= 128 ? 2 : chunks <= 256 ? 4 : 8;
        dim3 grid(static_cast<unsigned>((rows + kRowsPerBlock - 1) / kRowsPerBlock));
        const int c = static_cast<int>(cols);
        if (kind == 1) {
            if (bf) launch_layer<BF16>(nch, grid, stream, px, pw, pb, po, rows, c, eps);
            else launch_layer<F32>(nch, grid, stream, px, pw, pb, po, rows, c, eps);
        } else if (kind == 2) {
            if (bf) {
                if (pw) launch_rms<BF16, true, true>(nch, grid, stream, px, pr, pw, ps, po, rows, c, eps);
                else launch_rms<BF16, true, false>(nch, grid, stream, px, pr, pw, ps, po, rows, c, eps);
            } else {
                if (pw) launch_rms<F32, true, true>(nch, grid, stream, px, pr, pw, ps, po, rows, c, eps);
                else launch_rms<F32, true, false>(nch, grid, stream, px, pr, pw, ps, po, rows, c, eps);
            }
        } else {
            if (bf) {
                if (pw) launch_rms<BF16, false, true>(nch, grid, stream, px, nullptr, pw, nullptr, po, rows, c, eps);
                else launch_rms<BF16, false, false>(nch, grid, stream, px, nullptr, pw, nullptr, po, rows, c, eps);
            } else {
                if (pw) launch_rms<F32, false, true>(nch, grid, stream, px, nullptr, pw, nullptr, po, rows, c, eps);
                else launch_rms<F32, false, false>(nch, grid, stream, px, nullptr, pw, nullptr, po, rows, c, eps);
            }
        }
    } else {
        dim3 grid(static_cast<unsigned>(rows));
        if (bf)
            hipLaunchKernelGGL(norm_generic_kernel<BF16>, grid, dim3(256), 0, stream, kind, px, pr, pw, pb, ps, po, cols, eps);
        else
            hipLaunchKernelGGL(norm_generic_kernel<F32>, grid, dim3(256), 0, stream, kind, px, pr, pw, pb, ps, po, cols, eps);
    }
    SANDY_HIP_TRY(hipGetLastError(), e, op);
    return ok(e);
}

} // namespace
} // namespace sandy_hip

using namespace sandy_hip;

extern "C" int sandy_hip_norm(int32_t kind, const SandyTensor* x, const SandyTensor* weight,
                              const SandyTensor* bias, double epsilon, const SandyTensor* out,
                              void* stream, char* err, size_t err_cap) {
    Err e{err, err_cap};
    if (kind != 0 && kind != 1) return fail(e, SANDY_ERR_INVALID, "norm kind must be 0 (rms) or 1 (layer)");
    if (kind == 0 && bias) return fail(e, SANDY_ERR_INVALID, "rms_norm takes no bias");
    if (!x || !out) return fail(e, SANDY_ERR_INVALID, "norm requires input and output");
    return run_norm(kind, x, nullptr, weight, bias, epsilon, nullptr, out, static_cast<hipStream_t>(stream), e);
}

extern "C" int sandy_hip_add_rms_norm(const SandyTensor* x, const SandyTensor* residual,
                                      const SandyTensor* weight, double epsilon,
                                      const SandyTensor* sum_out, const SandyTensor* out,
                                      void* stream, char* err, size_t err_cap) {
    Err e{err, err_cap};
    if (!x || !out) return fail(e, SANDY_ERR_INVALID, "add_rms_norm requires input and output");
    return run_norm(2, x, residual, weight, nullptr, epsilon, sum_out, out, static_cast<hipStream_t>(stream), e);
}
