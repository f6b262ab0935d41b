// softmax.hip -- SoftmaxKernelOp, ReductionKernelOp (sum) and GatherKernelOp.
//
// softmax: src/core/TensorCalc.cpp:1337-1399 -- float max over the axis, an
// all -inf row gives zeros, double sum of float expf(x - max), float
// invSum = 1 / (float)sum, out = expf(x - max) * invSum.  Last-axis rows up to
// 2048 elements run one wave per row with the row in registers (one HBM read,
// one write); other shapes run one thread per (outer, inner) column.  The
// reference CUDA kernel handles the last axis only (CudaSoftmaxKernels.cu:
// 52-53) with a 256-thread block per row reading x three times.
//
// sum: TensorCalc.cpp:1401-1445 -- float accumulation in axis order; kept
// sequential per output element so the result equals the CPU's bit for bit.
//
// gather (embedding): TensorCalc.cpp:1520-1563 -- out[i, :] = table[ids[i], :],
// out-of-range ids set the sticky device error word.
#include "common.h"

namespace sandy_hip {
namespace {

template <typename T, int NCH>
__global__ __launch_bounds__(256) void softmax_rows_kernel(const void* __restrict__ x, void* __restrict__ out,
                                                           int64_t rows, int cols) {
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t base = row * cols;
    float v[NCH];
    float m = -INFINITY;
#pragma unroll
    // unguarded loads (clamped index) so that all are in flight at once; a
    // guarded load waits behind its guard
    for (int j = 0; j < NCH; j++) {
        const int c = lane + j * 64;
        v[j] = Vec8<T>::load1(x, base + (c < cols ? c : cols - 1));
    }
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        v[j] = lane + j * 64 < cols ? v[j] : -INFINITY;
        m = fmaxf(m, v[j]);
    }
    m = wave_max(m);
    if (isinf(m) && m < 0.0f) {
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int c = lane + j * 64;
            if (c < cols) Vec8<T>::store1(out, base + c, 0.0f);
        }
        return;
    }
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int c = lane + j * 64;
        if (c < cols) {
            v[j] = expf(__fsub_rn(v[j], m));
            s += static_cast<double>(v[j]);
        }
    }
    s = wave_sum(s);
    const float inv = 1.0f / static_cast<float>(s);
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int c = lane + j * 64;
        if (c < cols) Vec8<T>::store1(out, base + c, __fmul_rn(v[j], inv));
    }
}

template <typename T>
__global__ __launch_bounds__(256) void softmax_columns_kernel(const void* __restrict__ x, void* __restrict__ out,
                                                              int64_t outer, int64_t axis, int64_t inner) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= outer * inner) return;
    const int64_t o = t / inner, i = t % inner;
    const int64_t base = o * axis * inner + i;
    float m = -INFINITY;
    for (int64_t a = 0; a < axis; a++) m = fmaxf(m, Vec8<T>::load1(x, base + a * inner));
    if (isinf(m) && m < 0.0f) {
        for (int64_t a = 0; a < axis; a++) Vec8<T>::store1(out, base + a * inner, 0.0f);
        return;
    }
    double s = 0.0;
    for (int64_t a = 0; a < axis; a++) s += static_cast<double>(expf(__fsub_rn(Vec8<T>::load1(x, base + a * inner), m)));
    const float inv = 1.0f / static_cast<float>(s);
    for (int64_t a = 0; a < axis; a++)
        Vec8<T>::store1(out, base + a * inner, __fmul_rn(expf(__fsub_rn(Vec8<T>::load1(x, base + a * inner), m)), inv));
}

template <typename T>
__global__ __launch_bounds__(256) void sum_columns_kernel(const void* __restrict__ x, void* __restrict__ out,
                                                          int64_t outer, int64_t axis, int64_t inner) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= outer * inner) return;
    const int64_t o = t / inner, i = t % inner;
    const int64_t base = o * axis * inner + i;
    float acc = 0.0f;
    for (int64_t a = 0; a < axis; a++) acc = __fadd_rn(acc, Vec8<T>::load1(x, base + a * inner));
    Vec8<T>::store1(out, o * inner + i, acc);
}

__global__ __launch_bounds__(256) void gather_rows_kernel(const void* __restrict__ ids, int32_t ids_dt, int64_t n,
                                                          const void* __restrict__ table, int64_t vocab,
                                                          int64_t row_bytes, void* __restrict__ out, uint32_t* errw) {
    // one wave per id; 16-byte (or byte) copies of the row
    const int lane = threadIdx.x & 63;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (i >= n) return;
    const int64_t id = load_index(ids, ids_dt, i);
    if (id < 0 || id >= vocab) {
        if (lane == 0) atomicOr(errw, static_cast<uint32_t>(SANDY_DEVERR_GATHER_ID));
        return;
    }
    const char* src = static_cast<const char*>(table) + id * row_bytes;
    char* dst = static_cast<char*>(out) + i * row_bytes;
    if ((row_bytes & 15) == 0 && ((reinterpret_cast<uintptr_t>(table) | reinterpret_cast<uintptr_t>(out)) & 15) == 0) {
        for (int64_t b = lane * 16; b < row_bytes; b += 64 * 16)
            *reinterpret_cast<uint4*>(dst + b) = *reinterpret_cast<const uint4*>(src + b);
    } else {
        for (int64_t b = lane; b < row_bytes; b += 64) dst[b] = src[b];
    }
}

int split_axis(const SandyTensor& x, int64_t axis, int64_t& ax, int64_t& outer, int64_t& inner) {
    const int rank = x.rank;
    if (axis < -rank || axis >= rank) return -1;
    ax = axis < 0 ? axis + rank : axis;
    outer = 1;
    inner = 1;
    for (int i = 0; i < ax; i++) outer *= x.dims[i];
    for (int i = static_cast<int>(ax) + 1; i < rank; i++) inner *= x.dims[i];
    return 0;
}

} // namespace
} // namespace sandy_hip

using namespace sandy_hip;

extern "C" int sandy_hip_softmax(const SandyTensor* x, int64_t axis, const SandyTensor* out, void* stream_,
                                 char* err, size_t err_cap) {
    Err e{err, err_cap};
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (!valid_rank(x) || !valid_rank(out)) return fail(e, SANDY_ERR_INVALID, "softmax tensor rank out of range");
    if (!is_float(x->dtype)) return fail(e, SANDY_ERR_INVALID, "softmax input unsupported dtype");
    if (!same_shape(*x, *out)) return fail(e, SANDY_ERR_INVALID, "softmax output shape mismatch");
    if (out->dtype != x->dtype) return fail(e, SANDY_ERR_INVALID, "softmax output dtype mismatch");
    if (x->rank < 1) return fail(e, SANDY_ERR_INVALID, "softmax input must have rank >= 1");
    int64_t ax, outer, inner;
    if (split_axis(*x, axis, ax, outer, inner)) return fail(e, SANDY_ERR_INVALID, "softmax dim out of range");
    if (!contiguous(*x) || !contiguous(*out)) return fail(e, SANDY_ERR_UNSUPPORTED, "softmax requires contiguous tensors");
    if (numel(*x) == 0) return ok(e);
    const int64_t n = x->dims[ax];
    const void* px = base_ptr(*x);
    void* po = base_ptr(*out);
    const bool bf = x->dtype == SANDY_BF16;
    if (inner == 1 && n <= 2048) {
        dim3 grid(static_cast<unsigned>((outer + 3) / 4));
        const int c = static_cast<int>(n);
#define SM_LAUNCH(NCH)                                                                                          \
    if (bf) hipLaunchKernelGGL((softmax_rows_kernel<BF16, NCH>), grid, dim3(256), 0, stream, px, po, outer, c); \
    else hipLaunchKernelGGL((softmax_rows_kernel<F32, NCH>), grid, dim3(256), 0, stream, px, po, outer, c)
        if (n <= 64) { SM_LAUNCH(1); }
        else if (n <= 128) { SM_LAUNCH(2); }
        else if (n <= 256) { SM_LAUNCH(4); }
        else if (n <= 512) { SM_LAUNCH(8); }
        else if (n <= 1024) { SM_LAUNCH(16); }
        else { SM_LAUNCH(32); }
#undef SM_LAUNCH
    } else {
        const int64_t threads = outer * inner;
        dim3 grid(static_cast<unsigned>((threads + 255) / 256));
        if (bf) hipLaunchKernelGGL(softmax_columns_kernel<BF16>, grid, dim3(256), 0, stream, px, po, outer, n, inner);
        else hipLaunchKernelGGL(softmax_columns_kernel<F32>, grid, dim3(256), 0, stream, px, po, outer, n, inner);
    }
    SANDY_HIP_TRY(hipGetLastError(), e, "softmax launch");
    return ok(e);
}

extern "C" int sandy_hip_reduce_sum(const SandyTensor* x, int64_t axis, int32_t keep_dims, const SandyTensor* out,
                                    void* stream_, char* err, size_t err_cap) {
    Err e{err, err_cap};
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (!valid_rank(x) || !valid_rank(out)) return fail(e, SANDY_ERR_INVALID, "sum tensor rank out of range");
    if (!is_float(x->dtype)) return fail(e, SANDY_ERR_INVALID, "sum input unsupported dtype");
    if (x->rank < 1) return fail(e, SANDY_ERR_INVALID, "sum input must have rank >= 1");
    int64_t ax, outer, inner;
    if (split_axis(*x, axis, ax, outer, inner)) return fail(e, SANDY_ERR_INVALID, "sum dim out of range");
    // expected output shape
    int orank = keep_dims ? x->rank : x->rank - 1;
    if (out->rank != orank || out->dtype != x->dtype) return fail(e, SANDY_ERR_INVALID, "sum output shape mismatch");
    for (int i = 0, j = 0; i < x->rank; i++) {
        if (i == ax) {
            if (keep_dims && out->dims[j++] != 1) return fail(e, SANDY_ERR_INVALID, "sum output shape mismatch");
            continue;
        }
        if (out->dims[j++] != x->dims[i]) return fail(e, SANDY_ERR_INVALID, "sum output shape mismatch");
    }
    const int64_t n = x->dims[ax];
    if (n <= 0) return fail(e, SANDY_ERR_INVALID, "sum axis dimension must be static and positive");
    if (!contiguous(*x) || !contiguous(*out)) return fail(e, SANDY_ERR_UNSUPPORTED, "sum requires contiguous tensors");
    const int64_t threads = outer * inner;
    if (threads == 0) return ok(e);
    dim3 grid(static_cast<unsigned>((threads + 255) / 256));
    if (x->dtype == SANDY_BF16)
        hipLaunchKernelGGL(sum_columns_kernel<BF16>, grid, dim3(256), 0, stream, base_ptr(*x), base_ptr(*out), outer, n, inner);
    else
        hipLaunchKernelGGL(sum_columns_kernel<F32>, grid, dim3(256), 0, stream, base_ptr(*x), base_ptr(*out), outer, n, inner);
    SANDY_HIP_TRY(hipGetLastError(), e, "sum launch");
    return ok(e);
}

extern "C" int sandy_hip_gather(const SandyTensor* ids, const SandyTensor* table, const SandyTensor* out,
                                void* stream_, char* err, size_t err_cap) {
    Err e{err, err_cap};
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (!valid_rank(ids) || !valid_rank(table) || !valid_rank(out))
        return fail(e, SANDY_ERR_INVALID, "embedding tensor rank out of range");
    if (!is_index(ids->dtype)) return fail(e, SANDY_ERR_INVALID, "embedding ids must be i32 or i64");
    if (!is_float(table->dtype)) return fail(e, SANDY_ERR_INVALID, "embedding weight unsupported dtype");
    if (table->rank != 1 && table->rank != 2) return fail(e, SANDY_ERR_INVALID, "embedding weight must have rank 1 or rank 2");
    const int64_t vocab = table->dims[0];
    const int64_t hidden = table->rank == 2 ? table->dims[1] : 1;
    const int64_t n = numel(*ids);
    if (out->dtype != table->dtype || numel(*out) != n * hidden)
        return fail(e, SANDY_ERR_INVALID, "embedding output shape mismatch");
    if (!contiguous(*ids) || !contiguous(*table) || !contiguous(*out))
        return fail(e, SANDY_ERR_UNSUPPORTED, "embedding requires contiguous tensors");
    if (n == 0) return ok(e);
    int status = 0;
    uint32_t* errw = device_error_word(e, &status);
    if (status) return status;
    const int64_t row_bytes = hidden * static_cast<int64_t>(dtype_size(table->dtype));
    dim3 grid(static_cast<unsigned>((n + 3) / 4));
    hipLaunchKernelGGL(gather_rows_kernel, grid, dim3(256), 0, stream, base_ptr(*ids), ids->dtype, n, base_ptr(*table),
                       vocab, row_bytes, base_ptr(*out), errw);
    SANDY_HIP_TRY(hipGetLastError(), e, "embedding launch");
    return ok(e);
}
