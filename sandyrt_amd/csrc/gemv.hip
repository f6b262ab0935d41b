// gemv.hip -- fp32 decode rows through the reference's LayerNorm -> linear
// -> activation -> residual chain, one launch for the whole machine.
//
// The reference's GPT-2 program runs, per block, LayerNorm, the q/k/v
// linears, c_proj + residual add, LayerNorm, c_fc + GELU, c_proj + residual
// add as separate ops (src/models/gpt2_small.sandy.go; CPU arithmetic
// src/core/TensorCalc.cpp layer_norm 2010-2077, linear 722-773, the GELU of
// src/ir/BuiltinLowering.cpp:116-140, add 562-663).  A single-token decode
// step makes every one of them a few microseconds of launch and first-byte
// latency around very little work, and an in-order k loop per output column
// leaves the machine idle.  Here one launch does
//     out = [residual +] act(linear([LayerNorm](x), weight, bias))
// for up to four rows:
//   - every workgroup stages the rows of x in LDS, applying the LayerNorm
//     there when asked (double sums as the reference, then its float
//     operation order (x - mean) * inv_std * w + b);
//   - each wave owns RW output columns (rows of weight [N, K]) and reads them
//     as whole 1 KB runs of 64 lanes x 16 bytes, all of a lane's pieces
//     requested before the first is used; products accumulate in fp32 per
//     lane, then a wave butterfly sums the lanes in a fixed order;
//   - the epilogue adds the bias, applies the GELU node chain (the element-
//     wise group's operation order and tanh, so fusing does not change the
//     value given the same linear output) and the residual.
// The k order of the sums differs from the reference's sequential loop:
// results agree to fp32 rounding (well inside 1e-5 relative), not bit for
// bit; deterministic run to run.
#include "common.h"

namespace sandy_hip {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kGemvMaxRows = 4;
constexpr int kGemvMaxK = 8192;  // x rows staged in LDS: rows * K <= 16384 floats (64 KB)

struct GemvArgs {
    const float* x;          // [M, K]
    const float* ln_w;       // [K] or null (no LayerNorm)
    const float* ln_b;       // [K]
    float eps;
    const float* w;          // [N, K]
    const float* bias;       // [N] or null
    const float* resid;      // [M, N] or null
    float* out;              // [M, N]
    int32_t M, N, K;
};

// GELU node chain of ops.gelu_nodes (BuiltinLowering.cpp:116-140): (0.5 x) *
// (1 + tanh(0.7978845608028654 * (x + 0.044715 * (x * x * x)))), each
// product and sum rounded once, no contraction.
__device__ __forceinline__ float gelu_chain(float x) {
    const float h = __fmul_rn(0.5f, x);
    const float x3 = __fmul_rn(__fmul_rn(x, x), x);
    const float inner = __fadd_rn(x, __fmul_rn(0.044715f, x3));
    const float t = sandy_tanh(__fmul_rn(0.7978845608028654f, inner));
    return __fmul_rn(h, __fadd_rn(1.0f, t));
}

__device__ __forceinline__ double block_sum_d(double v, double* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

// M rows, RW weight rows per wave, PIECES 16-byte pieces per lane per row
// (K = 256 * PIECES; 0 = any K, looped).
template <int M, int RW, int PIECES, bool LN, int ACT, bool RES>
__global__ __launch_bounds__(256) void gemv_f32_kernel(GemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) float xs[];  // [M][K]
    __shared__ double red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = a.K;
    const int k4 = K >> 2;

    // weight pieces first: their latency covers the x staging and LayerNorm
    const int n0 = (static_cast<int>(blockIdx.x) * 4 + wave) * RW;
    constexpr int kP = PIECES > 0 ? PIECES : 1;
    v4f wv[RW][kP];
    if constexpr (PIECES > 0) {
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const int n = min(n0 + r, a.N - 1);
            const v4f* wr = reinterpret_cast<const v4f*>(a.w + static_cast<int64_t>(n) * K);
#pragma unroll
            for (int p = 0; p < PIECES; p++) wv[r][p] = __builtin_nontemporal_load(wr + lane + 64 * p);
        }
    }

    // x rows -> LDS (LayerNorm applied there)
    for (int m = 0; m < M; m++) {
        const v4f* xr = reinterpret_cast<const v4f*>(a.x + static_cast<int64_t>(m) * K);
        v4f* xd = reinterpret_cast<v4f*>(xs + m * K);
        for (int i = tid; i < k4; i += 256) xd[i] = xr[i];
    }
    if constexpr (LN) {
        __syncthreads();
        for (int m = 0; m < M; m++) {
            float* row = xs + m * K;
            double s = 0.0;
            for (int i = tid; i < K; i += 256) s += static_cast<double>(row[i]);
            const double mean = block_sum_d(s, red) / static_cast<double>(K);
            double v = 0.0;
            for (int i = tid; i < K; i += 256) {
                const double c = static_cast<double>(row[i]) - mean;
                v += c * c;
            }
            const double var = block_sum_d(v, red) / static_cast<double>(K);
            const float inv = 1.0f / sqrtf(static_cast<float>(var) + a.eps);
            const float meanf = static_cast<float>(mean);
            __syncthreads();  // every thread has read the row's raw values
            for (int i = tid; i < K; i += 256)
                row[i] = __fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(row[i], meanf), inv), a.ln_w[i]), a.ln_b[i]);
        }
    }
    __syncthreads();
    if (n0 >= a.N) return;

    float acc[RW][M];
#pragma unroll
    for (int r = 0; r < RW; r++)
#pragma unroll
        for (int m = 0; m < M; m++) acc[r][m] = 0.0f;
    auto dot = [&](int r, const v4f& w4, int piece) {
#pragma unroll
        for (int m = 0; m < M; m++) {
            const v4f x4 = *reinterpret_cast<const v4f*>(xs + m * K + 4 * piece);
            acc[r][m] = fmaf(w4.x, x4.x, acc[r][m]);
            acc[r][m] = fmaf(w4.y, x4.y, acc[r][m]);
            acc[r][m] = fmaf(w4.z, x4.z, acc[r][m]);
            acc[r][m] = fmaf(w4.w, x4.w, acc[r][m]);
        }
    };
    if constexpr (PIECES > 0) {
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int p = 0; p < PIECES; p++) dot(r, wv[r][p], lane + 64 * p);
    } else {
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const int n = min(n0 + r, a.N - 1);
            const v4f* wr = reinterpret_cast<const v4f*>(a.w + static_cast<int64_t>(n) * K);
            for (int p0 = lane; p0 < k4; p0 += 256) {
                v4f q[4];
#pragma unroll
                for (int u = 0; u < 4; u++) q[u] = p0 + 64 * u < k4 ? __builtin_nontemporal_load(wr + p0 + 64 * u) : v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int u = 0; u < 4; u++)
                    if (p0 + 64 * u < k4) dot(r, q[u], p0 + 64 * u);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RW; r++) {
        const int n = n0 + r;
#pragma unroll
        for (int m = 0; m < M; m++) {
            float v = acc[r][m];
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
            if (lane == 0 && n < a.N) {
                if (a.bias) v = __fadd_rn(v, a.bias[n]);
                if constexpr (ACT == 2) v = gelu_chain(v);
                if constexpr (RES) v = __fadd_rn(a.resid[static_cast<int64_t>(m) * a.N + n], v);
                a.out[static_cast<int64_t>(m) * a.N + n] = v;
            }
        }
    }
}

template <int M, int RW, int PIECES, bool LN, int ACT>
const void* pick_res(bool res) {
    return res ? reinterpret_cast<const void*>(&gemv_f32_kernel<M, RW, PIECES, LN, ACT, true>)
               : reinterpret_cast<const void*>(&gemv_f32_kernel<M, RW, PIECES, LN, ACT, false>);
}

template <int M, int RW, int PIECES>
const void* pick(bool ln, int act, bool res) {
    if (ln) return act == 2 ? pick_res<M, RW, PIECES, true, 2>(res) : pick_res<M, RW, PIECES, true, 0>(res);
    return act == 2 ? pick_res<M, RW, PIECES, false, 2>(res) : pick_res<M, RW, PIECES, false, 0>(res);
}

template <int M>
const void* pick_k(int pieces, bool ln, int act, bool res) {
    // K = 768 (3 pieces per lane, two columns per wave), K = 3072 (12 pieces,
    // one column per wave, 48 loads in flight per lane), else the looped form
    switch (pieces) {
        case 3: return pick<M, 2, 3>(ln, act, res);
        case 12: return pick<M, 1, 12>(ln, act, res);
        default: return pick<M, 1, 0>(ln, act, res);
    }
}

bool dense_f32(const SandyTensor* t) { return valid_rank(t) && t->dtype == SANDY_F32 && contiguous(*t); }

} // namespace
} // namespace sandy_hip

using namespace sandy_hip;

extern "C" int sandy_hip_decode_linear(const SandyTensor* x, const SandyTensor* ln_weight, const SandyTensor* ln_bias,
                                       double eps, const SandyTensor* weight, const SandyTensor* bias,
                                       int32_t activation, const SandyTensor* residual, const SandyTensor* out,
                                       void* stream_, char* err, size_t err_cap) {
    Err e{err, err_cap};
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (!dense_f32(x) || !dense_f32(weight) || !dense_f32(out) || x->rank < 1 || weight->rank != 2)
        return fail(e, SANDY_ERR_INVALID, "decode linear takes contiguous f32 x [..., k], weight [n, k] and out");
    const int64_t K = x->dims[x->rank - 1], N = weight->dims[0];
    const int64_t M = K > 0 ? numel(*x) / K : 0;
    if (weight->dims[1] != K) return fail(e, SANDY_ERR_INVALID, "linear input/weight feature mismatch");
    if (out->rank != x->rank || out->dims[out->rank - 1] != N || numel(*out) != M * N)
        return fail(e, SANDY_ERR_INVALID, "linear output shape mismatch");
    if (M < 1 || M > kGemvMaxRows) return fail(e, SANDY_ERR_UNSUPPORTED, "decode linear takes 1 to %d rows", kGemvMaxRows);
    if (K % 4 != 0 || K > kGemvMaxK || static_cast<int64_t>(M) * K > 16384)
        return fail(e, SANDY_ERR_UNSUPPORTED, "decode linear needs k a multiple of 4 and at most 16384 staged values (rows x k)");
    if ((ln_weight == nullptr) != (ln_bias == nullptr))
        return fail(e, SANDY_ERR_INVALID, "decode linear takes both LayerNorm weight and bias or neither");
    if (ln_weight && (!dense_f32(ln_weight) || !dense_f32(ln_bias) || numel(*ln_weight) != K || numel(*ln_bias) != K))
        return fail(e, SANDY_ERR_INVALID, "layer_norm weight and bias must be f32 [k]");
    if (bias && (!dense_f32(bias) || numel(*bias) != N)) return fail(e, SANDY_ERR_INVALID, "linear bias shape mismatch");
    if (residual && (!dense_f32(residual) || numel(*residual) != M * N))
        return fail(e, SANDY_ERR_INVALID, "decode linear residual must be f32 like out");
    if (activation != 0 && activation != 2) return fail(e, SANDY_ERR_INVALID, "decode linear activation must be 0 or 2 (gelu)");
    const uintptr_t al = reinterpret_cast<uintptr_t>(base_ptr(*x)) | reinterpret_cast<uintptr_t>(base_ptr(*weight));
    if (al & 15u) return fail(e, SANDY_ERR_UNSUPPORTED, "decode linear needs 16-byte aligned x and weight");
    {
        // every workgroup stages all of x while others already write out
        const uintptr_t xb = reinterpret_cast<uintptr_t>(base_ptr(*x)), ob = reinterpret_cast<uintptr_t>(base_ptr(*out));
        const uintptr_t xe = xb + static_cast<uintptr_t>(M * K) * sizeof(float), oe = ob + static_cast<uintptr_t>(M * N) * sizeof(float);
        if (M * N > 0 && xb < oe && ob < xe) return fail(e, SANDY_ERR_INVALID, "decode linear out must not alias x");
    }
    if (N == 0) return ok(e);
    const int pieces = K == 768 ? 3 : K == 3072 ? 12 : 0;
    const int rw = pieces == 3 ? 2 : 1;
    const int64_t blocks = (N + 4 * rw - 1) / (4 * rw);
    if (blocks > 0x7fffffff) return fail(e, SANDY_ERR_UNSUPPORTED, "decode linear shape exceeds the launch grid");
    const bool ln = ln_weight != nullptr, res = residual != nullptr;
    const void* fn = M == 1   ? pick_k<1>(pieces, ln, activation, res)
                     : M == 2 ? pick_k<2>(pieces, ln, activation, res)
                     : M == 3 ? pick_k<3>(pieces, ln, activation, res)
                              : pick_k<4>(pieces, ln, activation, res);
    GemvArgs a{};
    a.x = static_cast<const float*>(base_ptr(*x));
    a.ln_w = ln ? static_cast<const float*>(base_ptr(*ln_weight)) : nullptr;
    a.ln_b = ln ? static_cast<const float*>(base_ptr(*ln_bias)) : nullptr;
    a.eps = static_cast<float>(eps);
    a.w = static_cast<const float*>(base_ptr(*weight));
    a.bias = bias ? static_cast<const float*>(base_ptr(*bias)) : nullptr;
    a.resid = res ? static_cast<const float*>(base_ptr(*residual)) : nullptr;
    a.out = static_cast<float*>(base_ptr(*out));
    a.M = static_cast<int32_t>(M);
    a.N = static_cast<int32_t>(N);
    a.K = static_cast<int32_t>(K);
    void* args[] = {&a};
    SANDY_HIP_TRY(hipLaunchKernel(fn, dim3(static_cast<unsigned>(blocks)), dim3(256), args,
                                  static_cast<size_t>(M * K) * sizeof(float), stream),
                  e, "decode linear launch");
    return ok(e);
}
