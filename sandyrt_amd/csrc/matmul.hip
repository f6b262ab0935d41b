// matmul.hip -- dense matmul and linear (the projections and the lm-head).
//
// Semantics (src/core/TensorCalc.cpp):
//   matmul 804-919   for every batch of the broadcast batch shape
//                    (ShapeUtil.cpp:39-71; a smaller batch dim d serves
//                    batch/d consecutive output coordinates, TensorCalc.cpp:
//                    213-240), out[m, n] = sum over k in order of
//                    lhs[m, k] * rhs[k, n], either operand read transposed;
//                    float accumulation
//   linear 722-773   out[r, o] = bias[o] + sum over i in order of
//                    x[r, i] * w[o, i]
// Validation follows launch_cuda_matmul (src/device/cuda/
// CudaMatMulKernels.cu:78-141): same float dtype, contiguous views, rank >= 2,
// matching contracting dims and the exact output shape.
//
// The reference hands both to cuBLAS (cublasGemmEx, CudaMatMulKernels.cu:
// 173-216; its CUDA linear is not implemented, CudaDevice.cpp:536-537).
// Here there are three kernels:
//   - bf16 with the weight read row-major as [n, k] (transpose_rhs, the
//     layout of every projection and the lm-head) runs on
//     v_mfma_f32_16x16x32_bf16 with fp32 accumulation:
//       gemm_waves_kernel for decode-sized products (up to 64 rows): weight
//         streams, HBM-bound, K split over the waves of a workgroup and, when
//         the column tiles alone cannot fill the chip, over workgroups, with
//         the last-arriving workgroup of each output tile summing the fp32
//         partials in split order -- one launch, no second reduction pass;
//       gemm_lines_kernel for larger row counts: 64 x 256 tiles;
//   - gemm_simt_kernel: every other case (f32, either operand transposed,
//     unaligned shapes).  Register-tiled FMA-free float loops that keep the
//     reference's k order per output, so f32 results are bit-identical to the
//     CPU path.
#include "gemm.h"

#include <algorithm>
#include <cstdlib>

namespace sandy_hip {
namespace {

// decode GEMM workgroups resident at once (two per CU on the 256 CUs)
constexpr int64_t kWavesResident = 512;

// Prefill-sized products: workgroup = 16 * RT rows x 64 * CT columns of one
// batch; wave w owns columns n0 = (tile * 4 + w) * 16 * CT .. + 16 * CT.  Per
// chunk of 64 k the workgroup stages its activation rows once in LDS and
// each wave its own weight rows, both as whole 128-byte lines (8 rows x 128
// bytes per load instruction: on gfx950 that streams at about 5.0 TB/s
// against 3.2 TB/s for MFMA-layout half lines) into tiles whose 16-byte
// pieces are XOR-swizzled by (row / 2) % 8, so the 128-bit LDS writes and the
// MFMA-layout 128-bit reads are conflict-free.  Tiles are double buffered:
// chunk c + 1's loads are in flight while chunk c multiplies.  Loads go
// through buffer resources whose range checks return zero past the operand's
// last row; every offset is in the checked vector offset.
template <int RT, int CT, int OCC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(OCC))) void gemm_lines_kernel(GemmArgs g) {
    constexpr int kWTile = 16 * CT * 128;
    constexpr int kXTile = 16 * RT * 128;
    constexpr int kXPer = (16 * RT * 8 + 255) / 256;
    __shared__ __attribute__((aligned(16))) unsigned char lds[2 * kXTile + 4 * 2 * kWTile];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ct = static_cast<int>(blockIdx.x);
    const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 16 * RT;
    const int64_t bz = blockIdx.z;
    int64_t lo, ro;
    batch_offsets(g.bm, bz, lo, ro);
    const int64_t M = g.M, N = g.N, K = g.K;
    const int64_t n0 = (static_cast<int64_t>(ct) * 4 + wave) * 16 * CT;
    const bool wave_live = n0 < N;
    unsigned char* xt = lds;
    unsigned char* wt = lds + 2 * kXTile + wave * 2 * kWTile;
    auto swz = [](int row, int piece) { return row * 128 + ((piece ^ ((row >> 1) & 7)) << 4); };
    // chunk indices are 32-bit (K <= 2^21): their compares stay on the scalar unit
    const int ksteps = static_cast<int>(K / 32);
    const int chunks = (ksteps + 1) / 2;

    const int64_t wrows = wave_live ? min<int64_t>(16 * CT, N - n0) : 0;
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(g.w + ro + (wave_live ? n0 : 0) * K), 0, static_cast<int>(wrows * K * 2), 0x00020000);
    const int64_t xrows = min<int64_t>(16 * RT, M - r0);
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(g.a + lo + r0 * K), 0, static_cast<int>(xrows * K * 2), 0x00020000);
    // weight load i covers tile rows 8i .. 8i + 7 (lane: row 8i + lane/8, piece lane%8)
    const int wlane = static_cast<int>((lane >> 3) * K * 2 + (lane & 7) * 16);
    const int wstep = static_cast<int>(8 * K * 2);
    // tile row 8i + lane/8 swizzles by (4i + lane/16) % 8: one base for even i, one for odd i (+ i * 1024)
    const int wbase[2] = {swz(lane >> 3, lane & 7), swz(8 + (lane >> 3), lane & 7) - 1024};
    const bool w_hi = (lane & 7) >= 4;  // this lane's piece lies in the chunk's second k-step
    int xaddr[kXPer], xoff[kXPer];
    bool xlive[kXPer], x_hi[kXPer];
#pragma unroll
    for (int q = 0; q < kXPer; q++) {
        const int p = tid + 256 * q;
        xlive[q] = p < 16 * RT * 8;
        const int row = xlive[q] ? p >> 3 : 0;
        xaddr[q] = swz(row, p & 7);
        xoff[q] = static_cast<int>(row * K * 2 + (p & 7) * 16);
        x_hi[q] = (p & 7) >= 4;
    }
    int raddr[2][CT], aaddr[2][RT];
#pragma unroll
    for (int u = 0; u < 2; u++) {
#pragma unroll
        for (int c = 0; c < CT; c++) raddr[u][c] = swz(16 * c + (lane & 15), 4 * u + (lane >> 4));
#pragma unroll
        for (int t = 0; t < RT; t++) aaddr[u][t] = swz(16 * t + (lane & 15), 4 * u + (lane >> 4));
    }

    f32x4_t acc[RT][CT];
#pragma unroll
    for (int t = 0; t < RT; t++)
#pragma unroll
        for (int c = 0; c < CT; c++) acc[t][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    uint4 wv[2 * CT], xv[kXPer];
    // the k-tail mask is applied when the registers are written to LDS
    auto load = [&](int ch) {
        const int kb = ch * 128;
#pragma unroll
        for (int i = 0; i < 2 * CT; i++)
            wv[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wres, wlane + i * wstep + kb, 0, 0));
#pragma unroll
        for (int q = 0; q < kXPer; q++)
            xv[q] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xres, xoff[q] + kb, 0, 0));
    };
    auto store = [&](int buf, int ch) {
        const bool win = 2 * ch + (w_hi ? 1 : 0) < ksteps;
#pragma unroll
        for (int i = 0; i < 2 * CT; i++)
            *reinterpret_cast<uint4*>(wt + buf * kWTile + wbase[i & 1] + i * 1024) = win ? wv[i] : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < kXPer; q++)
            if (xlive[q])
                *reinterpret_cast<uint4*>(xt + buf * kXTile + xaddr[q]) =
                    2 * ch + (x_hi[q] ? 1 : 0) < ksteps ? xv[q] : make_uint4(0, 0, 0, 0);
    };
    auto mma = [&](int buf) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            uint4 av[RT];
#pragma unroll
            for (int t = 0; t < RT; t++) av[t] = *reinterpret_cast<const uint4*>(xt + buf * kXTile + aaddr[u][t]);
#pragma unroll
            for (int c = 0; c < CT; c++) {
                const uint4 bv = *reinterpret_cast<const uint4*>(wt + buf * kWTile + raddr[u][c]);
#pragma unroll
                for (int t = 0; t < RT; t++)
                    acc[t][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av[t]),
                                                                        __builtin_bit_cast(bf16x8_t, bv), acc[t][c],
                                                                        0, 0, 0);
            }
        }
    };
    load(0);
    store(0, 0);
    __syncthreads();
    for (int ch = 0; ch < chunks; ch++) {
        if (ch + 1 < chunks) load(ch + 1);
        if (wave_live) mma(ch & 1);
        if (ch + 1 < chunks) store((ch + 1) & 1, ch + 1);
        __syncthreads();
    }
    if (!wave_live) return;
    // acc[t][c][i]: row r0 + 16 t + 4 (lane / 16) + i, column n0 + 16 c + lane % 16
    const int64_t ob = bz * M * N;
#pragma unroll
    for (int c = 0; c < CT; c++) {
        const int64_t nc = n0 + 16 * c + (lane & 15);
        if (nc >= N) continue;
        const float bias = g.bias ? bf16_to_f32(g.bias[nc]) : 0.0f;
#pragma unroll
        for (int t = 0; t < RT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int64_t rr = r0 + 16 * t + 4 * (lane >> 4) + i;
                if (rr < M) g.out[ob + rr * N + nc] = f32_to_bf16(acc[t][c][i] + bias);  // 2-byte: L2 combines them
            }
    }
}

// Any dtype, either operand transposed: 64 x 64 output tile per workgroup,
// 4 x 4 outputs per thread, k staged 16 at a time through LDS.  Each output
// is acc = (bias or 0) then acc = acc + a * b over k in order (no FMA
// contraction), the reference's loop exactly.
template <typename T>
__global__ __launch_bounds__(256) void gemm_simt_kernel(const void* __restrict__ lhs, const void* __restrict__ rhs,
                                                        const void* __restrict__ bias, void* __restrict__ out,
                                                        int64_t M, int64_t N, int64_t K, int32_t tl, int32_t tr,
                                                        int64_t lrs, int64_t rrs, BatchMap bm) {
    constexpr int kT = 64, kK = 16;
    __shared__ float As[kK][kT + 4];
    __shared__ float Bs[kK][kT + 4];
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;
    const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kT, n0 = static_cast<int64_t>(blockIdx.x) * kT;
    const int64_t bz = blockIdx.z;
    int64_t lo, ro;
    batch_offsets(bm, bz, lo, ro);
    float acc[4][4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int64_t n = n0 + tx + 16 * j;
        const float b0 = bias && n < N ? Vec8<T>::load1(bias, n) : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i][j] = b0;
    }
    for (int64_t k0 = 0; k0 < K; k0 += kK) {
        // 1024 elements of each operand tile, 4 per thread; the fast index
        // follows the operand's contiguous dimension
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int e = tid + 256 * q;
            int mm, kk;
            if (tl) { mm = e & 63; kk = e >> 6; } else { kk = e & 15; mm = e >> 4; }
            const int64_t gm = m0 + mm, gk = k0 + kk;
            float v = 0.0f;
            if (gm < M && gk < K) v = Vec8<T>::load1(lhs, lo + (tl ? gk * lrs + gm : gm * lrs + gk));
            As[kk][mm] = v;
            int nn;
            if (tr) { kk = e & 15; nn = e >> 4; } else { nn = e & 63; kk = e >> 6; }
            const int64_t gn = n0 + nn, gk2 = k0 + kk;
            float w = 0.0f;
            if (gn < N && gk2 < K) w = Vec8<T>::load1(rhs, ro + (tr ? gn * rrs + gk2 : gk2 * rrs + gn));
            Bs[kk][nn] = w;
        }
        __syncthreads();
        const int kn = static_cast<int>(min<int64_t>(kK, K - k0));
        for (int kk = 0; kk < kn; kk++) {
            float av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) av[i] = As[kk][ty + 16 * i];
#pragma unroll
            for (int j = 0; j < 4; j++) bv[j] = Bs[kk][tx + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = __fadd_rn(acc[i][j], __fmul_rn(av[i], bv[j]));
        }
        __syncthreads();
    }
    const int64_t ob = bz * M * N;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int64_t m = m0 + ty + 16 * i;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int64_t n = n0 + tx + 16 * j;
            if (n < N) Vec8<T>::store1(out, ob + m * N + n, acc[i][j]);
        }
    }
}

// --------------------------------------------------------------------- host
struct Plan {
    int64_t M, N, K, batches;
    int64_t lrs, rrs;  // row strides (last dims) of lhs and rhs
    BatchMap bm;
};

// f32 products of a few rows against a weight read as [n, k] (linear, and
// matmul with transpose_rhs).  Each output column walks k in the reference's
// order (acc = bias, then acc + x * w rounded at each step, no contraction),
// so results stay bit-identical to the CPU path.  A wave owns 16 output
// columns: it loads their weight rows 32 k at a time as whole 128-byte lines
// (8 lanes per line, Q chunks in flight) into an LDS tile, and lanes 0..15
// then walk their row in order.  Per-lane row streams (64 distinct lines per
// load instruction) were bound by the CU's outstanding misses (59 us for
// 768 x 768); 16 columns per wave also spreads a 768-column output over 48
// CUs.  The activation rows are staged in LDS per block of k.
template <int MR, int Q>
__global__ __launch_bounds__(64) void gemv_seq_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                     const float* __restrict__ bias, float* __restrict__ out,
                                                     int64_t M, int64_t N, int64_t K, BatchMap bm) {
    constexpr int kCols = 16;  // output columns per wave
    constexpr int kXs = 8192;  // activation floats staged in LDS per block of k
    constexpr int kRow = 33;   // tile row stride in floats (conflict-free column walks)
    __shared__ float xs[kXs];
    __shared__ float tile[kCols * kRow];
    const int lane = threadIdx.x;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kCols;
    const int64_t n = n0 + lane;
    const int64_t bz = blockIdx.z;
    int64_t lo, ro;
    batch_offsets(bm, bz, lo, ro);
    const bool live = lane < kCols && n < N;
    const float* xr = x + lo;
    // this lane's two 16-byte pieces of each chunk: rows (lane / 8) and 8 + (lane / 8), piece lane % 8
    const int prow[2] = {lane >> 3, 8 + (lane >> 3)};
    const float* wrow[2];
#pragma unroll
    for (int i = 0; i < 2; i++) wrow[i] = w + ro + min<int64_t>(n0 + prow[i], N - 1) * K + (lane & 7) * 4;
    float acc[MR];
    const float b0 = bias && live ? bias[n] : 0.0f;
#pragma unroll
    for (int r = 0; r < MR; r++) acc[r] = b0;
    const int64_t kb_len = max<int64_t>(32, (kXs / M) & ~int64_t(31));
    float4 buf[Q][2];
    for (int64_t kb = 0; kb < K; kb += kb_len) {
        const int64_t len = min(kb_len, K - kb);
        __syncthreads();  // the previous block's reads of xs are done
        for (int64_t j = lane; j < M * len; j += 64) {
            const int64_t r = j / len, kk = j - r * len;
            xs[r * len + kk] = xr[r * K + kb + kk];
        }
        __syncthreads();
        const int64_t nch = len / 32;
        auto load = [&](int64_t c, int slot) {
#pragma unroll
            for (int i = 0; i < 2; i++) buf[slot][i] = *reinterpret_cast<const float4*>(wrow[i] + kb + c * 32);
        };
#pragma unroll
        for (int q = 0; q < Q; q++)
            if (q < nch) load(q, q);
        for (int64_t c0 = 0; c0 < nch; c0 += Q) {
#pragma unroll
            for (int q = 0; q < Q; q++) {
                const int64_t c = c0 + q;
                if (c >= nch) break;
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    float* t = tile + prow[i] * kRow + (lane & 7) * 4;
                    t[0] = buf[q][i].x;
                    t[1] = buf[q][i].y;
                    t[2] = buf[q][i].z;
                    t[3] = buf[q][i].w;
                }
                if (c + Q < nch) load(c + Q, q);
                __syncthreads();
                if (lane < kCols) {
                    // every LDS read is unconditional (rows past M read row M - 1), so the
                    // compiler issues them ahead of the in-order chain; only the
                    // accumulate is selected
                    const float* trow = tile + lane * kRow;
                    float wv[32];
#pragma unroll
                    for (int j = 0; j < 32; j++) wv[j] = trow[j];
#pragma unroll
                    for (int r = 0; r < MR; r++) {
                        const float* xc = xs + min<int64_t>(r, M - 1) * len + c * 32;
                        float xv[32];
#pragma unroll
                        for (int j = 0; j < 32; j++) xv[j] = xc[j];
                        float a_r = acc[r];
#pragma unroll
                        for (int j = 0; j < 32; j++) a_r = __fadd_rn(a_r, __fmul_rn(xv[j], wv[j]));
                        acc[r] = r < M ? a_r : acc[r];
                    }
                }
                __syncthreads();  // the tile is rewritten by the next chunk
            }
        }
        if (live)  // k tail past the 32-wide chunks, in order
            for (int64_t kk = nch * 32; kk < len; kk++) {
                const float wv = w[ro + n * K + kb + kk];
#pragma unroll
                for (int r = 0; r < MR; r++)
                    if (r < M) acc[r] = __fadd_rn(acc[r], __fmul_rn(xs[r * len + kk], wv));
            }
    }
    if (!live) return;
#pragma unroll
    for (int r = 0; r < MR; r++)
        if (r < M) out[(bz * M + r) * N + n] = acc[r];
}

// Fills the plan from operand shapes with the reference's rules; returns an
// error message or null.
const char* plan_matmul(const SandyTensor& l, const SandyTensor& r, const SandyTensor& o, bool tl, bool tr, Plan& p) {
    const int lr = l.rank, rr = r.rank;
    if (lr < 2) return "matmul lhs must have rank >= 2";
    if (rr < 2) return "matmul rhs must have rank >= 2";
    p.M = l.dims[lr - (tl ? 1 : 2)];
    const int64_t lk = l.dims[lr - (tl ? 2 : 1)];
    const int64_t rk = r.dims[rr - (tr ? 1 : 2)];
    p.N = r.dims[rr - (tr ? 2 : 1)];
    if (p.M < 0 || p.N < 0 || lk < 0 || rk < 0) return "matmul matrix dimensions must be static";
    if (lk != rk) return "matmul contracting dimension mismatch";
    p.K = lk;
    const int lb = lr - 2, rb = rr - 2;
    const int brank = std::max(lb, rb);
    if (o.rank != brank + 2) return "matmul output shape mismatch";
    BatchMap& m = p.bm;
    m.rank = brank;
    p.batches = 1;
    // contiguous strides of each operand's batch dims
    int64_t ls[SANDY_HIP_MAX_RANK], rs[SANDY_HIP_MAX_RANK];
    int64_t s = l.dims[lr - 1] * l.dims[lr - 2];
    for (int d = lb - 1; d >= 0; d--) { ls[d] = s; s *= l.dims[d]; }
    s = r.dims[rr - 1] * r.dims[rr - 2];
    for (int d = rb - 1; d >= 0; d--) { rs[d] = s; s *= r.dims[d]; }
    for (int i = 0; i < brank; i++) {
        const int li = lb - brank + i, ri = rb - brank + i;
        const int64_t a = li >= 0 ? l.dims[li] : 1, b = ri >= 0 ? r.dims[ri] : 1;
        int64_t d;
        if (a == b) d = a;
        else if (a == 1) d = b;
        else if (b == 1) d = a;
        else if (a > b && a % b == 0) d = a;
        else if (b > a && b % a == 0) d = b;
        else return "cannot broadcast matmul batch shapes";
        m.dims[i] = d;
        m.l_stride[i] = (li >= 0 && a != 1) ? ls[li] : 0;
        m.l_div[i] = (li >= 0 && a != 1) ? d / a : 1;
        m.r_stride[i] = (ri >= 0 && b != 1) ? rs[ri] : 0;
        m.r_div[i] = (ri >= 0 && b != 1) ? d / b : 1;
        if (o.dims[i] != d) return "matmul output shape mismatch";
        p.batches *= d;
    }
    if (o.dims[brank] != p.M || o.dims[brank + 1] != p.N) return "matmul output shape mismatch";
    p.lrs = l.dims[lr - 1];
    p.rrs = r.dims[rr - 1];
    return nullptr;
}

// The decode GEMM's fused forms: a residual-add epilogue with row sums of
// squares, and an RMSNorm prologue from such sums.
struct Fusion {
    const uint16_t* resid = nullptr;
    double* rsq_out = nullptr;
    int64_t rsq_parts = 0;
    const double* rsq_in = nullptr;
    int64_t rsq_in_parts = 0;
    const uint16_t* norm_w = nullptr;
    float eps = 0.0f;
    const QkvRope* qr = nullptr;  // q/k/v RoPE + paged-append epilogue
    bool dry = false;             // every check and workspace, no launch
};

int launch(const Plan& p, const SandyTensor& l, const SandyTensor& r, const SandyTensor* bias, const SandyTensor& o,
           bool tl, bool tr, hipStream_t stream, Err e, const char* what, int glu = 0, const Fusion* fz = nullptr) {
    if (p.batches == 0 || p.M == 0 || p.N == 0) return ok(e);
    if (p.batches > 65535) return fail(e, SANDY_ERR_UNSUPPORTED, "%s batch count exceeds 65535", what);
    const void* pl = base_ptr(l);
    const void* pr = base_ptr(r);
    const void* pb = bias ? base_ptr(*bias) : nullptr;
    void* po = base_ptr(o);
    const bool aligned = ((reinterpret_cast<uintptr_t>(pl) | reinterpret_cast<uintptr_t>(pr)) & 15) == 0;
    const bool lines = l.dtype == SANDY_BF16 && !tl && tr && p.K % 32 == 0 && p.K > 0 && aligned &&
                       p.K <= (int64_t{1} << 21) && env_int("SANDY_GEMM_SIMT", 0) == 0;
    const bool waves = lines && env_int("SANDY_GEMM_WAVES", p.M <= 64 ? 1 : 0) != 0;
    if ((glu || fz) && !waves)
        return fail(e, SANDY_ERR_UNSUPPORTED, "%s needs bf16 operands, k a multiple of 32 and at most 64 rows", what);
    if (fz && p.batches != 1) return fail(e, SANDY_ERR_UNSUPPORTED, "%s takes one [m, k] matrix", what);
    const bool norm = fz && fz->norm_w;
    // f32, few rows, weight rows contiguous: the exact-order GEMV
    const bool gemv = l.dtype == SANDY_F32 && !tl && tr && p.M <= 8 && p.K % 4 == 0 && aligned &&
                      p.lrs == p.K && p.rrs == p.K && env_int("SANDY_GEMM_SIMT", 0) == 0;
    if (gemv) {
        const int64_t blocks = (p.N + 15) / 16;
        if (blocks > 0x7fffffff) return fail(e, SANDY_ERR_UNSUPPORTED, "%s shape exceeds the launch grid", what);
        const dim3 grid(static_cast<unsigned>(blocks), 1, static_cast<unsigned>(p.batches));
        const float* x = static_cast<const float*>(pl);
        const float* w = static_cast<const float*>(pr);
        const float* b = static_cast<const float*>(pb);
        float* y = static_cast<float*>(po);
        if (p.M == 1) hipLaunchKernelGGL((gemv_seq_kernel<1, 8>), grid, dim3(64), 0, stream, x, w, b, y, p.M, p.N, p.K, p.bm);
        else if (p.M <= 2) hipLaunchKernelGGL((gemv_seq_kernel<2, 8>), grid, dim3(64), 0, stream, x, w, b, y, p.M, p.N, p.K, p.bm);
        else if (p.M <= 4) hipLaunchKernelGGL((gemv_seq_kernel<4, 8>), grid, dim3(64), 0, stream, x, w, b, y, p.M, p.N, p.K, p.bm);
        else hipLaunchKernelGGL((gemv_seq_kernel<8, 8>), grid, dim3(64), 0, stream, x, w, b, y, p.M, p.N, p.K, p.bm);
    } else if (waves) {
        GemmArgs g{};
        g.a = static_cast<const uint16_t*>(pl);
        g.w = static_cast<const uint16_t*>(pr);
        g.bias = static_cast<const uint16_t*>(pb);
        g.out = static_cast<uint16_t*>(po);
        g.M = p.M;
        g.N = p.N;
        g.K = p.K;
        g.bm = p.bm;
        g.glu = glu;
        if (fz) {
            g.resid = fz->resid;
            g.rsq_out = fz->rsq_out;
            g.rsq_parts = fz->rsq_parts;
            g.rsq_in = fz->rsq_in;
            g.rsq_in_parts = fz->rsq_in_parts;
            g.norm_w = fz->norm_w;
            g.eps = fz->eps;
            if (fz->qr) g.qr = *fz->qr;
        }
        // tile: 16 * RT rows x 16 * CT columns, variants (RT, CT) = 0 (1, 1),
        // 1 (2, 1), 3 (2, 2), 4 (1, 2), 5 (2, 4), 6 (1, 4) -- the ones the
        // heuristic below picks (2 is unused); SANDY_GEMM_TILE / SANDY_GEMM_CPS
        // select one of them and a run length for the tests that cover every
        // instantiated form
        static const int kRT[] = {1, 2, 2, 2, 1, 2, 1};
        static const int kCT[] = {1, 1, 1, 2, 2, 4, 4};
        const int64_t chunks = (p.K / 32 + 1) / 2;
        int variant = env_int("SANDY_GEMM_TILE", -1);
        int cps = env_int("SANDY_GEMM_CPS", 0);
        // K: at most 32 chunks (2048 k) per workgroup, split evenly; the
        // per-wave run is rounded up to a built run length
        int64_t ksplits = (chunks + 31) / 32;
        // chunks in flight per wave (4 only for RT * CT <= 2, register bound)
        int qdepth = 2;
        if (variant < 0 || variant > 6 || variant == 2) {
            // Measured on decode shapes with the weights streamed from HBM
            // (rotated over >= 1 GiB of copies):
            //   <= 16 rows: 16 x 16 tiles, 16 x 32 from N >= 16384 (lm-head);
            //   <= 32 rows: 16-row tiles (the second row tile re-reads the
            //     weights from cache), 32 columns from N K >= 5M; 17..32 rows
            //     of N K >= 16M without the norm prologue: one 32-row tile
            //     (weights streamed once);
            //   weights past 64 MB at 32 rows, and 33..64 rows: 32-row tiles,
            //     the widest column tile giving >= 120 workgroups;
            //   4 chunks in flight per wave for weights under 8M elements
            //   (o projection at 32 rows 8.3 -> 6.1 us, q/k/v at one row
            //   7.4 -> 5.5 us), 2 for the larger ones;
            //   up to 32 rows with K past 2048: up to 48 chunks per
            //   workgroup and 4 in flight (down projection, 5632 x 2048: two
            //   K splits of runs of 12 against three of 8; 32 rows
            //   12.8 -> 11.6 us, one row 9.2 -> 8.7 us).
            const bool big = p.N * p.K * 2 > (int64_t(64) << 20);
            int64_t rt = 1, ct = 1;
            if (p.M <= 16 && !big) {
                ct = p.N >= 16384 ? 2 : 1;
                qdepth = 4;
                if (chunks > 32) ksplits = (chunks + 47) / 48;
            } else if (p.M <= 32 && !big && !norm && p.M > 16 && p.N * p.K >= 16 * (int64_t(1) << 20) && chunks <= 32) {
                // 17..32 rows of a wide projection (gate/up, 2048 x 11264): one
                // 32-row tile, so the weights stream once, non-temporal, with four
                // chunks in flight (15.2 -> 14.2 us; two 16-row tiles re-read
                // them from L2 and must keep them cached).  Not with the RMSNorm
                // prologue, whose work grows with the rows of a tile (gated
                // gate/up 17.0 -> 18.2 us)
                rt = 2;
                qdepth = 4;
            } else if (p.M <= 32 && !big) {
                ct = p.N * p.K >= 5 * (int64_t(1) << 20) ? 2 : 1;
                qdepth = p.N * p.K < 8 * (int64_t(1) << 20) ? 4 : 2;
                if (chunks > 32) {
                    ksplits = (chunks + 47) / 48;
                    qdepth = 4;
                }
            } else {
                rt = p.M <= 16 ? 1 : 2;
                const int64_t rows = (p.M + 16 * rt - 1) / (16 * rt) * p.batches;
                for (int c : {4, 2}) {
                    if ((p.N + 16 * c - 1) / (16 * c) * rows * ksplits >= 120) {
                        ct = c;
                        break;
                    }
                }
            }
            static const int kPick[2][3] = {{0, 4, 6}, {1, 3, 5}};  // [RT 1/2][CT 1/2/4]
            variant = kPick[rt == 1 ? 0 : 1][ct == 1 ? 0 : ct == 2 ? 1 : 2];
        }
        qdepth = env_int("SANDY_GEMM_Q", qdepth);
        // the q/k/v epilogue kernels: 16-row tiles of 16 or 32 columns
        const bool qkv = fz && fz->qr;
        if (qkv) variant = kCT[variant] == 1 ? 0 : 4;
        const int RT = kRT[variant], CT = kCT[variant];
        const int64_t row_tiles = (p.M + 16 * RT - 1) / (16 * RT);
        const int64_t col_tiles = (p.N + 16 * CT - 1) / (16 * CT);
        if (row_tiles > 65535 || col_tiles > (1 << 24))
            return fail(e, SANDY_ERR_UNSUPPORTED, "%s shape exceeds the launch grid", what);
        const int64_t tiles = row_tiles * col_tiles * p.batches;
        if (cps <= 0) cps = static_cast<int>(((chunks + ksplits - 1) / ksplits + 3) / 4);
        // built run lengths: per-split chunks are at most 48 (cps <= 12)
        static const int kRuns[] = {2, 3, 4, 5, 6, 8, 10, 12};
        int run = 12;
        for (int r : kRuns) {
            if (r >= cps) {
                run = r;
                break;
            }
        }
        cps = run;
        const int64_t splits = (chunks + 4 * cps - 1) / (4 * cps);
        g.col_tiles = static_cast<int32_t>(col_tiles);
        g.row_tiles = static_cast<int32_t>(row_tiles);
        g.splits = static_cast<int32_t>(splits);
        g.split_chunks = 4 * cps;
        if (col_tiles * splits > 0x7fffffff) return fail(e, SANDY_ERR_UNSUPPORTED, "%s shape exceeds the launch grid", what);
        if (splits > 1) {
            int status = 0;
            const size_t part = static_cast<size_t>(tiles * splits) * RT * CT * 64 * 4 * sizeof(float);
            g.part = static_cast<float*>(device_workspace(4, part, stream, e, &status));
            if (status) return status;
            g.counters = static_cast<uint32_t*>(device_counters(1, static_cast<size_t>(tiles) * sizeof(uint32_t), stream, e, &status));
            if (status) return status;
        }
        const dim3 grid(static_cast<unsigned>(col_tiles * splits), static_cast<unsigned>(row_tiles),
                        static_cast<unsigned>(p.batches));
        // the weight stream non-temporal where nothing re-reads it from L2 later:
        // one row tile, or every workgroup resident at once (the row tiles of a
        // column tile run together); measured at 1 row: q/k/v 5.2 -> 4.6 us,
        // o 5.1 -> 4.5, gate/up 10.4 -> 9.3, down 8.5 -> 7.8; at 32 rows the
        // 704-workgroup gate/up re-reads its weights after 352 other workgroups
        // (15.3 -> 16.5 us non-temporal) and keeps the default policy
        // (batched products may share one rhs across the batch: only a single
        // matrix counts as read once when the grid is not resident at once)
        const bool nt = (row_tiles == 1 && p.batches == 1) || col_tiles * splits * row_tiles * p.batches <= kWavesResident;
        if (qkv) {
            int status = 0;
            g.qr.arrivals = static_cast<uint32_t*>(
                device_counters(3, static_cast<size_t>(row_tiles) * sizeof(uint32_t), stream, e, &status));
            if (status) return status;
            // column tiles holding a k or v column, times the K splits
            const int64_t q_cols = static_cast<int64_t>(g.qr.hq) * g.qr.d;
            g.qr.kv_arrivals = static_cast<int32_t>((col_tiles - std::min<int64_t>(col_tiles, q_cols / (16 * CT))) * splits);
            if (fz->dry) return ok(e);
            if (nt) launch_waves_qkv<true>(variant, cps, qdepth, norm, grid, stream, g);
            else launch_waves_qkv<false>(variant, cps, qdepth, norm, grid, stream, g);
        } else if (norm) {
            if (nt) launch_waves_norm<true>(variant, cps, qdepth, grid, stream, g);
            else launch_waves_norm<false>(variant, cps, qdepth, grid, stream, g);
        } else {
            if (nt) launch_waves_plain<true>(variant, cps, qdepth, grid, stream, g);
            else launch_waves_plain<false>(variant, cps, qdepth, grid, stream, g);
        }
        SANDY_HIP_TRY(hipGetLastError(), e, what);
        return ok(e);
    } else if (lines) {
        // 64 x 256 tiles for prefill-sized products (the K loop is rolled and
        // the grid never splits K)
        GemmArgs g{};
        g.a = static_cast<const uint16_t*>(pl);
        g.w = static_cast<const uint16_t*>(pr);
        g.bias = static_cast<const uint16_t*>(pb);
        g.out = static_cast<uint16_t*>(po);
        g.M = p.M;
        g.N = p.N;
        g.K = p.K;
        g.bm = p.bm;
        const int64_t row_tiles = (p.M + 63) / 64;
        const int64_t col_tiles = (p.N + 255) / 256;
        if (row_tiles > 65535 || col_tiles > 0x7fffffff)
            return fail(e, SANDY_ERR_UNSUPPORTED, "%s shape exceeds the launch grid", what);
        g.col_tiles = static_cast<int32_t>(col_tiles);
        g.row_tiles = static_cast<int32_t>(row_tiles);
        g.splits = 1;
        g.split_chunks = static_cast<int32_t>((p.K / 32 + 1) / 2);
        const dim3 grid(static_cast<unsigned>(col_tiles), static_cast<unsigned>(row_tiles),
                        static_cast<unsigned>(p.batches));
        hipLaunchKernelGGL((gemm_lines_kernel<4, 4, 2>), grid, dim3(256), 0, stream, g);
    } else {
        const int64_t gy = (p.M + 63) / 64, gx = (p.N + 63) / 64;
        if (gy > 65535 || gx > 0x7fffffff) return fail(e, SANDY_ERR_UNSUPPORTED, "%s shape exceeds the launch grid", what);
        const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy), static_cast<unsigned>(p.batches));
        if (l.dtype == SANDY_BF16)
            hipLaunchKernelGGL(gemm_simt_kernel<BF16>, grid, dim3(256), 0, stream, pl, pr, pb, po, p.M, p.N, p.K,
                               static_cast<int32_t>(tl), static_cast<int32_t>(tr), p.lrs, p.rrs, p.bm);
        else
            hipLaunchKernelGGL(gemm_simt_kernel<F32>, grid, dim3(256), 0, stream, pl, pr, pb, po, p.M, p.N, p.K,
                               static_cast<int32_t>(tl), static_cast<int32_t>(tr), p.lrs, p.rrs, p.bm);
    }
    SANDY_HIP_TRY(hipGetLastError(), e, what);
    return ok(e);
}

} // namespace
} // namespace sandy_hip

using namespace sandy_hip;

extern "C" int sandy_hip_matmul(const SandyTensor* lhs, const SandyTensor* rhs, int32_t transpose_lhs,
                                int32_t transpose_rhs, const SandyTensor* out, void* stream_, char* err,
                                size_t err_cap) {
    Err e{err, err_cap};
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (!valid_rank(lhs) || !valid_rank(rhs) || !valid_rank(out))
        return fail(e, SANDY_ERR_INVALID, "matmul requires lhs, rhs and out");
    if (lhs->dtype != rhs->dtype || lhs->dtype != out->dtype)
        return fail(e, SANDY_ERR_INVALID, "matmul operands must have same dtype");
    if (!is_float(lhs->dtype)) return fail(e, SANDY_ERR_INVALID, "matmul unsupported dtype");
    if (!contiguous(*lhs) || !contiguous(*rhs) || !contiguous(*out))
        return fail(e, SANDY_ERR_UNSUPPORTED, "matmul requires contiguous tensor views");
    Plan p{};
    if (const char* msg = plan_matmul(*lhs, *rhs, *out, transpose_lhs != 0, transpose_rhs != 0, p))
        return fail(e, SANDY_ERR_INVALID, "%s", msg);
    return launch(p, *lhs, *rhs, nullptr, *out, transpose_lhs != 0, transpose_rhs != 0, stream, e, "matmul");
}

extern "C" int sandy_hip_matmul_glu(const SandyTensor* lhs, const SandyTensor* rhs, int32_t activation,
                                    const SandyTensor* out, void* stream_, char* err, size_t err_cap) {
    Err e{err, err_cap};
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (!valid_rank(lhs) || !valid_rank(rhs) || !valid_rank(out))
        return fail(e, SANDY_ERR_INVALID, "matmul requires lhs, rhs and out");
    if (activation != 1 && activation != 2) return fail(e, SANDY_ERR_INVALID, "gated matmul activation must be 1 (silu) or 2 (gelu)");
    if (lhs->dtype != rhs->dtype || lhs->dtype != out->dtype)
        return fail(e, SANDY_ERR_INVALID, "matmul operands must have same dtype");
    if (!contiguous(*lhs) || !contiguous(*rhs) || !contiguous(*out))
        return fail(e, SANDY_ERR_UNSUPPORTED, "matmul requires contiguous tensor views");
    if (rhs->rank != 2 || rhs->dims[0] % 2 != 0)
        return fail(e, SANDY_ERR_INVALID, "gated matmul weight must be [2 * ffn, k] with gate and up rows interleaved");
    // plan the product against the full [.., M, 2 ffn] output; the epilogue writes half of it
    SandyTensor full = *out;
    if (full.rank < 1 || full.dims[full.rank - 1] * 2 != rhs->dims[0])
        return fail(e, SANDY_ERR_INVALID, "matmul output shape mismatch");
    full.dims[full.rank - 1] = rhs->dims[0];
    Plan p{};
    if (const char* msg = plan_matmul(*lhs, *rhs, full, false, true, p)) return fail(e, SANDY_ERR_INVALID, "%s", msg);
    return launch(p, *lhs, *rhs, nullptr, *out, false, true, stream, e, "gated matmul", activation);
}

// Shared checks of the fused decode GEMMs: bf16, lhs [m, k], rhs [n, k]
// (transposed weight), row statistics of ceil(cols / 16) float64 partials.
static int check_fused(const SandyTensor* lhs, const SandyTensor* rhs, const SandyTensor* out, Err e, const char* what) {
    if (!valid_rank(lhs) || !valid_rank(rhs) || !valid_rank(out))
        return fail(e, SANDY_ERR_INVALID, "%s requires lhs, rhs and out", what);
    if (lhs->dtype != SANDY_BF16 || rhs->dtype != SANDY_BF16 || out->dtype != SANDY_BF16)
        return fail(e, SANDY_ERR_UNSUPPORTED, "%s takes bf16 operands", what);
    if (lhs->rank != 2 || rhs->rank != 2 || out->rank != 2)
        return fail(e, SANDY_ERR_INVALID, "%s expects lhs [m, k], rhs [n, k] and out [m, n]", what);
    if (!contiguous(*lhs) || !contiguous(*rhs) || !contiguous(*out))
        return fail(e, SANDY_ERR_UNSUPPORTED, "%s requires contiguous tensor views", what);
    return SANDY_OK;
}

static bool stats_ok(const SandyRowStats* st, int64_t rows, int64_t cols) {
    return st && st->sumsq && st->rows == rows && st->parts == (cols + 15) / 16 &&
           (reinterpret_cast<uintptr_t>(st->sumsq) & 7u) == 0;
}

extern "C" int sandy_hip_matmul_residual(const SandyTensor* lhs, const SandyTensor* rhs, const SandyTensor* residual,
                                         const SandyTensor* out, const SandyRowStats* out_stats, void* stream_,
                                         char* err, size_t err_cap) {
    Err e{err, err_cap};
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    const char* what = "residual matmul";
    if (int st = check_fused(lhs, rhs, out, e, what)) return st;
    if (!valid_rank(residual) || residual->dtype != SANDY_BF16 || !same_shape(*residual, *out) || !contiguous(*residual))
        return fail(e, SANDY_ERR_INVALID, "%s residual must be a contiguous bf16 tensor shaped like out", what);
    if (base_ptr(*out) == base_ptr(*lhs)) return fail(e, SANDY_ERR_INVALID, "%s out must not alias lhs", what);
    Plan p{};
    if (const char* msg = plan_matmul(*lhs, *rhs, *out, false, true, p)) return fail(e, SANDY_ERR_INVALID, "%s", msg);
    if (out_stats && !stats_ok(out_stats, p.M, p.N))
        return fail(e, SANDY_ERR_INVALID, "%s row statistics must be [m, ceil(n / 16)] float64", what);
    Fusion fz;
    fz.resid = static_cast<const uint16_t*>(base_ptr(*residual));
    fz.rsq_out = out_stats ? out_stats->sumsq : nullptr;
    fz.rsq_parts = out_stats ? out_stats->parts : 0;
    return launch(p, *lhs, *rhs, nullptr, *out, false, true, stream, e, what, 0, &fz);
}

extern "C" int sandy_hip_matmul_rms(const SandyTensor* lhs, const SandyRowStats* lhs_stats,
                                    const SandyTensor* norm_weight, double eps, const SandyTensor* rhs,
                                    int32_t activation, const SandyTensor* out, void* stream_, char* err,
                                    size_t err_cap) {
    Err e{err, err_cap};
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    const char* what = "rms matmul";
    if (int st = check_fused(lhs, rhs, out, e, what)) return st;
    if (activation < 0 || activation > 2) return fail(e, SANDY_ERR_INVALID, "gated matmul activation must be 1 (silu) or 2 (gelu)");
    const int64_t K = lhs->dims[1];
    if (!valid_rank(norm_weight) || norm_weight->dtype != SANDY_BF16 || numel(*norm_weight) != K ||
        !contiguous(*norm_weight) || (reinterpret_cast<uintptr_t>(base_ptr(*norm_weight)) & 15u) != 0)
        return fail(e, SANDY_ERR_INVALID, "%s norm weight must be a 16-byte aligned bf16 [k] vector", what);
    if (!stats_ok(lhs_stats, lhs->dims[0], K))
        return fail(e, SANDY_ERR_INVALID, "%s row statistics must be [m, ceil(k / 16)] float64", what);
    SandyTensor full = *out;
    if (activation) {
        if (rhs->dims[0] % 2 != 0 || out->dims[1] * 2 != rhs->dims[0])
            return fail(e, SANDY_ERR_INVALID, "gated matmul weight must be [2 * ffn, k] with gate and up rows interleaved");
        full.dims[1] = rhs->dims[0];
    }
    Plan p{};
    if (const char* msg = plan_matmul(*lhs, *rhs, full, false, true, p)) return fail(e, SANDY_ERR_INVALID, "%s", msg);
    Fusion fz;
    fz.rsq_in = lhs_stats->sumsq;
    fz.rsq_in_parts = lhs_stats->parts;
    fz.norm_w = static_cast<const uint16_t*>(base_ptr(*norm_weight));
    fz.eps = static_cast<float>(eps);
    return launch(p, *lhs, *rhs, nullptr, *out, false, true, stream, e, what, activation, &fz);
}

namespace sandy_hip {
int matmul_qkv(const SandyTensor* lhs, const SandyRowStats* lhs_stats, const SandyTensor* norm_weight, double eps,
               const SandyTensor* rhs, const QkvRope& qr, hipStream_t stream, Err e, bool dry) {
    const char* what = "qkv matmul";
    if (!valid_rank(lhs) || !valid_rank(rhs)) return fail(e, SANDY_ERR_INVALID, "%s requires lhs and rhs", what);
    if (lhs->dtype != SANDY_BF16 || rhs->dtype != SANDY_BF16) return fail(e, SANDY_ERR_UNSUPPORTED, "%s takes bf16 operands", what);
    if (lhs->rank != 2 || rhs->rank != 2 || !contiguous(*lhs) || !contiguous(*rhs))
        return fail(e, SANDY_ERR_INVALID, "%s expects contiguous lhs [m, k] and rhs [n, k]", what);
    const int64_t M = lhs->dims[0], K = lhs->dims[1];
    if (M > kQkvMaxRows) return fail(e, SANDY_ERR_UNSUPPORTED, "%s takes at most %d rows", what, kQkvMaxRows);
    if (rhs->dims[0] != static_cast<int64_t>(qr.hq + 2 * qr.hkv) * qr.d || rhs->dims[1] != K)
        return fail(e, SANDY_ERR_INVALID, "%s weight must be [(q_heads + 2 kv_heads) head_dim, k]", what);
    const bool norm = lhs_stats || norm_weight;
    if (norm) {
        if (!valid_rank(norm_weight) || norm_weight->dtype != SANDY_BF16 || numel(*norm_weight) != K ||
            !contiguous(*norm_weight) || (reinterpret_cast<uintptr_t>(base_ptr(*norm_weight)) & 15u) != 0)
            return fail(e, SANDY_ERR_INVALID, "%s norm weight must be a 16-byte aligned bf16 [k] vector", what);
        if (!stats_ok(lhs_stats, M, K))
            return fail(e, SANDY_ERR_INVALID, "%s row statistics must be [m, ceil(k / 16)] float64", what);
    }
    // the product is planned against an [m, n] output the epilogue never writes
    SandyTensor full{};
    full.dtype = SANDY_BF16;
    full.rank = 2;
    full.dims[0] = M;
    full.dims[1] = rhs->dims[0];
    full.strides[0] = rhs->dims[0];
    full.strides[1] = 1;
    Plan p{};
    if (const char* msg = plan_matmul(*lhs, *rhs, full, false, true, p)) return fail(e, SANDY_ERR_INVALID, "%s", msg);
    Fusion fz;
    if (norm) {
        fz.rsq_in = lhs_stats->sumsq;
        fz.rsq_in_parts = lhs_stats->parts;
        fz.norm_w = static_cast<const uint16_t*>(base_ptr(*norm_weight));
        fz.eps = static_cast<float>(eps);
    }
    fz.qr = &qr;
    fz.dry = dry;
    return launch(p, *lhs, *rhs, nullptr, full, false, true, stream, e, what, 0, &fz);
}
} // namespace sandy_hip

extern "C" int sandy_hip_linear(const SandyTensor* x, const SandyTensor* weight, const SandyTensor* bias,
                                const SandyTensor* out, void* stream_, char* err, size_t err_cap) {
    Err e{err, err_cap};
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (!valid_rank(x) || !valid_rank(weight) || !valid_rank(bias) || !valid_rank(out))
        return fail(e, SANDY_ERR_INVALID, "linear requires input, weight, bias and out");
    if (!is_float(x->dtype)) return fail(e, SANDY_ERR_INVALID, "linear input unsupported dtype");
    if (weight->dtype != x->dtype || bias->dtype != x->dtype || out->dtype != x->dtype)
        return fail(e, SANDY_ERR_INVALID, "linear operands must have same dtype");
    if (x->rank < 1 || weight->rank != 2 || bias->rank != 1)
        return fail(e, SANDY_ERR_INVALID, "linear expects input [..., in], weight [out, in], bias [out]");
    const int64_t in_f = x->dims[x->rank - 1], out_f = weight->dims[0];
    if (weight->dims[1] != in_f) return fail(e, SANDY_ERR_INVALID, "linear input/weight feature mismatch");
    if (bias->dims[0] != out_f) return fail(e, SANDY_ERR_INVALID, "linear bias shape mismatch");
    if (out->rank != x->rank || out->dims[x->rank - 1] != out_f)
        return fail(e, SANDY_ERR_INVALID, "linear output shape mismatch");
    for (int i = 0; i + 1 < x->rank; i++)
        if (out->dims[i] != x->dims[i]) return fail(e, SANDY_ERR_INVALID, "linear output shape mismatch");
    if (!contiguous(*x) || !contiguous(*weight) || !contiguous(*bias) || !contiguous(*out))
        return fail(e, SANDY_ERR_UNSUPPORTED, "linear requires contiguous tensor views");
    // rows of x flattened: [rows, in] times weight^T
    SandyTensor x2 = *x, o2 = *out;
    int64_t rows = 1;
    for (int i = 0; i + 1 < x->rank; i++) rows *= x->dims[i];
    x2.rank = 2;
    x2.dims[0] = rows;
    x2.dims[1] = in_f;
    x2.strides[0] = in_f;
    x2.strides[1] = 1;
    o2.rank = 2;
    o2.dims[0] = rows;
    o2.dims[1] = out_f;
    o2.strides[0] = out_f;
    o2.strides[1] = 1;
    Plan p{};
    if (const char* msg = plan_matmul(x2, *weight, o2, false, true, p)) return fail(e, SANDY_ERR_INVALID, "%s", msg);
    return launch(p, x2, *weight, bias, o2, false, true, stream, e, "linear");
}
