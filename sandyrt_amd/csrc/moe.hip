// moe.hip -- MoE routing and expert execution: top-k, stable permute
// (moe_gather), grouped expert GEMM on MFMA (moe_matmul) and the weighted
// combine (moe_scatter_sum).
//
// Semantics (src/core/TensorCalc.cpp):
//   topk 1447-1518          k largest by (value desc, index asc)
//   moe_gather 1565-1667    packed rows ordered expert, then token, then slot;
//                           expert_offsets[e] = first row of expert e
//   moe_matmul 1669-1743    rows [off[e], off[e+1]) times W[e]^T (or W[e])
//   moe_scatter_sum 1745-1811  out[token] accumulated in packed-row order, the
//                           accumulator rounded to the output dtype after
//                           every add
//
// The reference CUDA path (CudaGatherKernels.cu:283-649,
// CudaMoeScatterSumKernels.cu:152-405, CudaMatMulKernels.cu:294-616) assigns
// rows with atomics (nondeterministic order within an expert), round-trips
// counts and offsets through the host with stream syncs, combines with fp32
// atomics and hands the grouped GEMM to cuBLAS.  Here:
//   - the permute is a device-side stable counting sort: one workgroup per
//     (expert, share of its rows) ranks that expert's routes by ballots and
//     copies its rows in the same launch (one workgroup per batch ranks
//     longer route lists), so rows come out in exactly the CPU order and no
//     host round trip is needed;
//   - the combine is a gather-reduce: one wave per (token, 512 columns)
//     finds its rows with ballots in row order and accumulates with the
//     reference's per-add rounding -- bit-identical to the CPU, no atomics;
//   - the grouped GEMM streams each expert's weights once through
//     v_mfma_f32_16x16x32_bf16 tiles (rows of the expert as the M dimension),
//     HBM-bound like the reference's cuBLAS grouped GEMM.
#include "common.h"

#include <algorithm>
#include <type_traits>
#include <cstdlib>

namespace sandy_hip {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- top-k
__device__ __forceinline__ bool better(float v, int64_t i, float bv, int64_t bi) {
    return v != bv ? v > bv : i < bi;
}

// One wave per row (last axis, <= 64 * NV elements); k rounds of a wave
// argmax under (value desc, index asc).
template <typename T, int NV>
__global__ __launch_bounds__(256) void topk_rows_kernel(const void* __restrict__ x, void* __restrict__ values,
                                                        void* __restrict__ indices, int32_t idx_dt, int64_t rows,
                                                        int axis, int k) {
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    float v[NV];
    bool taken[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int c = lane + 64 * j;
        v[j] = c < axis ? Vec8<T>::load1(x, row * axis + c) : 0.0f;
        taken[j] = c >= axis;
    }
    for (int r = 0; r < k; r++) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        bool have = false;
#pragma unroll
        for (int j = 0; j < NV; j++) {
            const int c = lane + 64 * j;
            if (!taken[j] && (!have || better(v[j], c, bv, bi))) {
                bv = v[j];
                bi = c;
                have = true;
            }
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const float ov = __shfl_xor(bv, m, 64);
            const int oi = __shfl_xor(bi, m, 64);
            const bool oh = __shfl_xor(static_cast<int>(have), m, 64) != 0;
            if (oh && (!have || better(ov, oi, bv, bi))) {
                bv = ov;
                bi = oi;
                have = true;
            }
        }
        // bi is now the same in every lane: its owner marks it taken
#pragma unroll
        for (int j = 0; j < NV; j++)
            if (lane + 64 * j == bi) taken[j] = true;
        if (lane == 0) {
            Vec8<T>::store1(values, row * k + r, bv);
            store_index(indices, idx_dt, row * k + r, bi);
        }
    }
}

// Small rows (<= 256), one row per workgroup: the row is staged in LDS, and
// wave w counts, for every element, the better elements in the w-th quarter
// of the row; the four partial ranks are summed through LDS and the
// elements with rank < k written straight to their slot.  A quarter of the
// compares per lane of a one-wave-per-row form, whose 2 * 128 compares per
// lane were most of a [512, 128] launch (6.6 -> 3.6 us).
__device__ __forceinline__ bool better32(float v, int i, float bv, int bi) { return v != bv ? v > bv : i < bi; }

template <typename T, int NV>
__global__ __launch_bounds__(256) void topk_rank4_kernel(const void* __restrict__ x, void* __restrict__ values,
                                                         void* __restrict__ indices, int32_t idx_dt, int64_t rows,
                                                         int axis, int k) {
    __shared__ __attribute__((aligned(16))) float row_v[64 * NV];
    __shared__ int part[4][64 * NV];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t row = blockIdx.x;
    // one element per thread (clamped, unguarded load), pads past the row -inf
    if (tid < 64 * NV) {
        const float v = Vec8<T>::load1(x, row * axis + (tid < axis ? tid : axis - 1));
        row_v[tid] = tid < axis ? v : -INFINITY;
    }
    __syncthreads();
    float v[NV];
    int rank[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) {
        v[j] = row_v[lane + 64 * j];
        rank[j] = 0;
    }
    // this wave's quarter: 16 * NV elements, read as 128-bit LDS pieces
    const float4* rv4 = reinterpret_cast<const float4*>(row_v + wave * 16 * NV);
    const int base = wave * 16 * NV;
#pragma unroll
    for (int s4 = 0; s4 < 4 * NV; s4++) {
        const float4 o4 = rv4[s4];
        const float o[4] = {o4.x, o4.y, o4.z, o4.w};
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int j = 0; j < NV; j++) rank[j] += better32(o[q], base + 4 * s4 + q, v[j], lane + 64 * j) ? 1 : 0;
    }
#pragma unroll
    for (int j = 0; j < NV; j++) part[wave][lane + 64 * j] = rank[j];
    __syncthreads();
    if (tid < axis) {
        const int r = part[0][tid] + part[1][tid] + part[2][tid] + part[3][tid];
        if (r < k) {
            Vec8<T>::store1(values, row * k + r, row_v[tid]);
            store_index(indices, idx_dt, row * k + r, tid);
        }
    }
}

// Any axis: one thread per (outer, inner) column, selection over the axis.
template <typename T>
__global__ __launch_bounds__(256) void topk_columns_kernel(const void* __restrict__ x, void* __restrict__ values,
                                                           void* __restrict__ indices, int32_t idx_dt, int64_t outer,
                                                           int64_t axis, int64_t inner, int64_t k) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= outer * inner) return;
    const int64_t o = t / inner, in = t % inner;
    const int64_t base = o * axis * inner + in;
    float pv = INFINITY;
    int64_t pi = -1;  // previous pick: next pick must come strictly after it in the order
    for (int64_t r = 0; r < k; r++) {
        float bv = 0.0f;
        int64_t bi = -1;
        for (int64_t a = 0; a < axis; a++) {
            const float v = Vec8<T>::load1(x, base + a * inner);
            const bool after_prev = pi < 0 || better(pv, pi, v, a);
            if (after_prev && (bi < 0 || better(v, a, bv, bi))) {
                bv = v;
                bi = a;
            }
        }
        const int64_t oi = o * k * inner + r * inner + in;
        Vec8<T>::store1(values, oi, bv);
        store_index(indices, idx_dt, oi, bi);
        pv = bv;
        pi = bi;
    }
}

// Long rows (inner == 1, axis > 1024, k <= 16): greedy token selection over a
// vocabulary is the case that matters.  Phase 1: workgroup (chunk of 4096,
// row) keeps its 16 elements per thread in registers (loads coalesced per
// step) and runs k rounds of a block argmax, each round taking the best item
// strictly after the previous pick in (value desc, index asc) order;
// phase 2: one workgroup per row merges the chunks' candidates the same way.
constexpr int kWideChunk = 4096;
constexpr int kWideMaxK = 16;

__device__ __forceinline__ void take_if_better(float& v, int64_t& i, float ov, int64_t oi) {
    if (oi >= 0 && (i < 0 || better(ov, oi, v, i))) {
        v = ov;
        i = oi;
    }
}

// Best (value, index) over the workgroup's 256 threads (index < 0: none);
// every thread returns the result.
__device__ __forceinline__ void block_best(float& v, int64_t& i, float* sv, int64_t* si) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o, 64);
        const uint32_t lo = __shfl_xor(static_cast<uint32_t>(i), o, 64);
        const uint32_t hi = __shfl_xor(static_cast<uint32_t>(static_cast<uint64_t>(i) >> 32), o, 64);
        take_if_better(v, i, ov, static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo));
    }
    if (lane == 0) {
        sv[wave] = v;
        si[wave] = i;
    }
    __syncthreads();
    v = sv[0];
    i = si[0];
#pragma unroll
    for (int w = 1; w < 4; w++) take_if_better(v, i, sv[w], si[w]);
    __syncthreads();
}

// VEC: 8-element (16- or 32-byte) loads, thread t covering elements
// 8t .. 8t + 7 and 2048 + 8t .. of its chunk; else 16 strided scalar loads.
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void topk_wide_chunks_kernel(const void* __restrict__ x, int64_t n, int64_t chunks,
                                                               int k, float* __restrict__ cv, int64_t* __restrict__ ci) {
    __shared__ float sv[4];
    __shared__ int64_t si[4];
    const int64_t c = blockIdx.x, row = blockIdx.y;
    float v[16];
    int64_t id[16];
    if constexpr (VEC) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int64_t i0 = c * kWideChunk + 2048 * h + 8 * threadIdx.x;
            float part[8];
            Vec8<T>::load(x, row * n + (i0 < n ? i0 : 0), part);  // n % 8 == 0: a vector is all in or all out
#pragma unroll
            for (int q = 0; q < 8; q++) {
                v[8 * h + q] = part[q];
                id[8 * h + q] = i0 + q;
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < 16; j++) {
            id[j] = c * kWideChunk + threadIdx.x + 256 * j;
            v[j] = Vec8<T>::load1(x, row * n + (id[j] < n ? id[j] : 0));
        }
    }
    float pv = 0.0f;
    int64_t pi = -1;
    bool done = false;
    float* ov = cv + (row * chunks + c) * k;
    int64_t* oi = ci + (row * chunks + c) * k;
    for (int r = 0; r < k; r++) {
        float bv = 0.0f;
        int64_t bi = -1;
        if (!done) {
#pragma unroll
            for (int j = 0; j < 16; j++)
                if (id[j] < n && (pi < 0 || better(pv, pi, v[j], id[j]))) take_if_better(bv, bi, v[j], id[j]);
        }
        block_best(bv, bi, sv, si);
        if (threadIdx.x == 0) {
            ov[r] = bv;
            oi[r] = bi;
        }
        done = bi < 0;  // the chunk has fewer than k items: the rest stay empty
        pv = bv;
        pi = bi;
    }
}

template <typename T>
__global__ __launch_bounds__(256) void topk_wide_merge_kernel(const float* __restrict__ cv, const int64_t* __restrict__ ci,
                                                              int64_t chunks, int k, void* __restrict__ values,
                                                              void* __restrict__ indices, int32_t idx_dt) {
    __shared__ float sv[4];
    __shared__ int64_t si[4];
    const int64_t row = blockIdx.x;
    const int64_t m = chunks * k;
    const float* rv = cv + row * m;
    const int64_t* ri = ci + row * m;
    float pv = 0.0f;
    int64_t pi = -1;
    for (int r = 0; r < k; r++) {
        float bv = 0.0f;
        int64_t bi = -1;
        for (int64_t j = threadIdx.x; j < m; j += 256) {
            const int64_t idx = ri[j];
            if (idx >= 0 && (pi < 0 || better(pv, pi, rv[j], idx))) take_if_better(bv, bi, rv[j], idx);
        }
        block_best(bv, bi, sv, si);
        if (threadIdx.x == 0) {
            Vec8<T>::store1(values, row * k + r, bv);
            store_index(indices, idx_dt, row * k + r, bi);
        }
        pv = bv;
        pi = bi;
    }
}

// Greedy selection (k == 1) over long rows in one pass.  (value desc, index
// asc) is the unsigned order of the 64-bit key  ord(value) << 32 | ~index,
// where ord maps the float's bits to an order-preserving u32 (-0 taken as +0,
// the reference compares them equal; NaN mapped to 0, below every number).
// Workgroup (chunk, row) reduces its U * 2048 elements to one key, merges it
// into the row's slot with a 64-bit atomic max, and the last workgroup of the
// row to arrive (a counter) takes the slot (resetting it and the
// counter to zero for the next call), re-reads the winning element so the
// value is stored bit for bit, and writes value and index.
__device__ __forceinline__ uint32_t order_key(float v) {
    uint32_t u = __float_as_uint(v);
    if ((u << 1) == 0) u = 0;                 // -0 -> +0
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0u;  // NaN: lowest
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// one row's key and counter, alone on a 256-byte span: rows' atomics then
// land in different memory channels instead of queueing on one line
constexpr int kArgmaxSlotWords = 32;

__device__ __forceinline__ uint64_t key_max(uint64_t a, uint64_t b) { return a > b ? a : b; }

template <typename T, int U, bool VEC>
__global__ __launch_bounds__(256) void argmax_wide_kernel(const void* __restrict__ x, int64_t n, int chunks,
                                                          uint64_t* __restrict__ slots, void* __restrict__ values,
                                                          void* __restrict__ indices, int32_t idx_dt) {
    constexpr int kChunk = U * 2048;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t row = blockIdx.y;
    const int64_t c0 = static_cast<int64_t>(blockIdx.x) * kChunk;
    const int64_t rbase = row * n;
    uint32_t best_ord = 0, best_idx = 0xffffffffu;
    bool any = false;
    if constexpr (VEC) {
        typename Vec8<T>::raw raw[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t i0 = c0 + 2048 * u + 8 * tid;
            // non-temporal (each element is read once): Gemma [64, 262144] 11.8 -> 11.5 us
            raw[u] = Vec8<T>::load_raw_nt(x, rbase + (i0 < n ? i0 : 0));  // n % 8 == 0: a vector is all in or all out
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t i0 = c0 + 2048 * u + 8 * tid;
            if (i0 >= n) break;
            float v[8];
            Vec8<T>::unpack(raw[u], v);
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const uint32_t o = order_key(v[q]);
                if (!any || o > best_ord) {  // indices increase: strict > keeps the first of equals
                    best_ord = o;
                    best_idx = static_cast<uint32_t>(i0 + q);
                    any = true;
                }
            }
        }
    } else {
        float v[8 * U];
#pragma unroll
        for (int j = 0; j < 8 * U; j++) {
            const int64_t i = c0 + tid + 256 * j;
            v[j] = Vec8<T>::load1(x, rbase + (i < n ? i : 0));
        }
#pragma unroll
        for (int j = 0; j < 8 * U; j++) {
            const int64_t i = c0 + tid + 256 * j;
            if (i >= n) break;
            const uint32_t o = order_key(v[j]);
            if (!any || o > best_ord) {
                best_ord = o;
                best_idx = static_cast<uint32_t>(i);
                any = true;
            }
        }
    }
    // a thread with no element keeps key 0, which any element's key beats
    // or equals (ties at 0 are NaN-only rows, where ~index still orders)
    uint64_t key = any ? (static_cast<uint64_t>(best_ord) << 32) | static_cast<uint32_t>(~best_idx) : 0;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint32_t lo = __shfl_xor(static_cast<uint32_t>(key), o, 64);
        const uint32_t hi = __shfl_xor(static_cast<uint32_t>(key >> 32), o, 64);
        key = key_max(key, (static_cast<uint64_t>(hi) << 32) | lo);
    }
    __shared__ uint64_t wk[4];
    if (lane == 0) wk[wave] = key;
    __syncthreads();
    if (tid != 0) return;
    key = key_max(key_max(wk[0], wk[1]), key_max(wk[2], wk[3]));
    uint64_t* slot = slots + kArgmaxSlotWords * row;
    uint64_t* ctr = slot + 1;
    // device-scope atomics resolve past the XCD's L2; waiting for the max to
    // return before counting orders the two without an acquire/release pair
    // (which would write back and invalidate the L2 in every workgroup)
    const uint64_t before = __hip_atomic_fetch_max(slot, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const uint64_t prev = __hip_atomic_fetch_add(ctr, uint64_t{1} + 0 * before, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev != static_cast<uint64_t>(chunks - 1)) return;
    __hip_atomic_store(ctr, uint64_t{0}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t win = __hip_atomic_exchange(slot, uint64_t{0}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int64_t idx = static_cast<int64_t>(~static_cast<uint32_t>(win));
    Vec8<T>::store1(values, row, Vec8<T>::load1(x, rbase + idx));
    store_index(indices, idx_dt, row, idx);
}

// ---------------------------------------------------------------- moe_gather
constexpr int kRouteThreads = 1024;
constexpr int kRouteWaves = kRouteThreads / 64;
constexpr int kRouteStage = 4096;  // routes whose ids and weights are staged in LDS

// Exclusive scan of the per-expert counts held in cursor[] -> expert offsets
// (written out) and starting cursors: each wave-0 pass scans a 64-expert
// segment with shuffles, segments chained serially.
__device__ __forceinline__ void scan_expert_counts(int32_t* cursor, int64_t experts, void* offsets, int32_t off_dt,
                                                   int b, int tid, int lane, int wave) {
    __shared__ int32_t seg_total;
    if (tid == 0) seg_total = 0;
    __syncthreads();
    for (int64_t s0 = 0; s0 < experts; s0 += 64) {
        if (wave == 0) {
            const int64_t ex = s0 + lane;
            const int32_t c = ex < experts ? cursor[ex] : 0;
            int32_t incl = c;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int32_t up = __shfl_up(incl, d, 64);
                if (lane >= d) incl += up;
            }
            const int32_t base = seg_total;
            if (ex < experts) {
                cursor[ex] = base + incl - c;
                store_index(offsets, off_dt, static_cast<int64_t>(b) * (experts + 1) + ex, base + incl - c);
            }
            const int32_t tot = __shfl(incl, 63, 64);
            if (lane == 0) seg_total = base + tot;
        }
        __syncthreads();
    }
    if (tid == 0) store_index(offsets, off_dt, static_cast<int64_t>(b) * (experts + 1) + experts, seg_total);
}

// Routes beyond the fused dispatch's limit: one workgroup per batch.
// dest[r] receives the packed row of route r (token-major route order
// r = token * top_k + slot); rows of one expert are in route order.  Pass 1
// counts routes per expert; pass 2 walks the routes in order, 1024 at a time:
// inside a wave, lanes routed to the same expert are ranked by ballot; waves
// are ordered through LDS prefix sums; a per-expert cursor carries across
// chunks.
__global__ __launch_bounds__(kRouteThreads) void moe_route_kernel(
        const void* __restrict__ ids, int32_t ids_dt, const void* __restrict__ w, int32_t w_dt, int64_t seq,
        int64_t top_k, int64_t experts, void* __restrict__ packed_w, void* __restrict__ token_ids, int32_t tok_dt,
        void* __restrict__ offsets, int32_t off_dt, int32_t* __restrict__ dest, uint32_t* errw) {
    extern __shared__ __attribute__((aligned(16))) int32_t lds[];
    int32_t* cursor = lds;                      // [E]
    int32_t* wcount = lds + experts;            // [kRouteWaves][E]
    int32_t* sid = wcount + kRouteWaves * experts;          // staged ids  [kRouteStage]
    float* sw = reinterpret_cast<float*>(sid + kRouteStage);  // staged weights [kRouteStage]
    const int b = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t routes = seq * top_k;
    const int64_t rb = static_cast<int64_t>(b) * routes;
    const bool staged = routes <= kRouteStage;
    for (int64_t e = tid; e < experts; e += kRouteThreads) cursor[e] = 0;
    if (staged) {  // all loads independent: one memory round trip
        for (int64_t r = tid; r < routes; r += kRouteThreads) {
            int64_t e = load_index(ids, ids_dt, rb + r);
            if (e < 0 || e >= experts) {
                atomicOr(errw, static_cast<uint32_t>(SANDY_DEVERR_EXPERT_ID));
                e = -1;
            }
            sid[r] = static_cast<int32_t>(e);
            sw[r] = load_any(w, w_dt, rb + r);
        }
    }
    __syncthreads();
    for (int64_t r = tid; r < routes; r += kRouteThreads) {
        int64_t e;
        if (staged) e = sid[r];
        else {
            e = load_index(ids, ids_dt, rb + r);
            if (e < 0 || e >= experts) {
                atomicOr(errw, static_cast<uint32_t>(SANDY_DEVERR_EXPERT_ID));
                e = -1;
            }
        }
        if (e >= 0) atomicAdd(&cursor[e], 1);
    }
    __syncthreads();
    scan_expert_counts(cursor, experts, offsets, off_dt, b, tid, lane, wave);
    __syncthreads();
    for (int64_t c0 = 0; c0 < routes; c0 += kRouteThreads) {
        const int64_t r = c0 + tid;
        int64_t e = -1;
        if (r < routes) e = staged ? sid[r] : load_index(ids, ids_dt, rb + r);
        if (e >= experts) e = -1;
        for (int64_t i = lane; i < experts; i += 64) wcount[wave * experts + i] = 0;
        __syncthreads();
        // rank among equal experts inside the wave
        int rank = 0;
        uint64_t pending = __ballot(e >= 0);
        while (pending) {
            const int leader = __ffsll(static_cast<long long>(pending)) - 1;
            const int64_t le = __builtin_amdgcn_readlane(static_cast<int>(e), leader);
            const uint64_t same = __ballot(e == le);
            if (e == le) rank = __popcll(same & ((1ull << lane) - 1ull));
            if (lane == leader) wcount[wave * experts + le] = __popcll(same);
            pending &= ~same;
        }
        __syncthreads();
        // per expert: prefix over the waves, then advance the cursor
        for (int64_t x = tid; x < experts; x += kRouteThreads) {
            int32_t run = cursor[x];
            for (int wv = 0; wv < kRouteWaves; wv++) {
                const int32_t c = wcount[wv * experts + x];
                wcount[wv * experts + x] = run;
                run += c;
            }
            cursor[x] = run;
        }
        __syncthreads();
        if (e >= 0) {
            const int32_t row = wcount[wave * experts + e] + rank;
            dest[rb + r] = row;
            const int64_t mb = static_cast<int64_t>(b) * routes;
            store_any(packed_w, w_dt, mb + row, staged ? sw[r] : load_any(w, w_dt, rb + r));
            store_index(token_ids, tok_dt, mb + row, r / top_k);
        } else if (r < routes) {
            dest[rb + r] = -1;
        }
        __syncthreads();
    }
}

// packed_x[dest[r]] = x[token(r)]: one wave per route, 16-byte copies.
__global__ __launch_bounds__(256) void moe_copy_rows_kernel(const char* __restrict__ x, char* __restrict__ packed,
                                                            const int32_t* __restrict__ dest, int64_t batch,
                                                            int64_t seq, int64_t top_k, int64_t row_bytes,
                                                            int aligned) {
    const int lane = threadIdx.x & 63;
    const int64_t gr = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);  // global route
    const int64_t routes = seq * top_k;
    if (gr >= batch * routes) return;
    const int64_t b = gr / routes, r = gr % routes;
    const int32_t row = dest[gr];
    if (row < 0) return;
    const char* src = x + (b * seq + r / top_k) * row_bytes;
    char* dst = packed + (b * routes + row) * row_bytes;
    if (aligned) {
        typedef unsigned u32x4_nt __attribute__((ext_vector_type(4)));
        for (int64_t o = lane * 16; o < row_bytes; o += 64 * 16)
            __builtin_nontemporal_store(*reinterpret_cast<const u32x4_nt*>(src + o), reinterpret_cast<u32x4_nt*>(dst + o));
    } else {
        for (int64_t o = lane; o < row_bytes; o += 64) dst[o] = src[o];
    }
}

// Fused permute for up to kDispatchRoutes routes per batch: workgroup =
// (expert e, share c of C, batch).  Every workgroup reads all route ids
// (coalesced, L2-resident after the first) and derives, with no atomics and
// no other workgroup:
//   - e's offset: the number of valid routes to lower experts;
//   - e's routes in route order (= token, then slot: the reference's order
//     within an expert), ranked by per-(chunk, wave) ballot counts and one
//     exclusive scan in LDS;
// then writes token id and weight of, and copies x into, the rows q of e
// with q % C == c (one wave per row).  Share 0 writes e's offset (the last
// expert also the total).
constexpr int kDispatchRoutes = 8192;

// CH chunks of 256 routes per thread in registers (16 up to 4096 routes, 32
// up to 8192): all their loads are in flight at once, so registers, and with
// them occupancy, scale with CH
template <int CH>
__global__ __launch_bounds__(256) void moe_dispatch_kernel(
        const void* __restrict__ ids, int32_t ids_dt, const void* __restrict__ w, int32_t w_dt, int64_t seq,
        int64_t top_k, int64_t experts, int shares, const char* __restrict__ x, char* __restrict__ packed,
        int64_t row_bytes, int aligned, void* __restrict__ packed_w, void* __restrict__ token_ids, int32_t tok_dt,
        void* __restrict__ offsets, int32_t off_dt, uint32_t* errw) {
    __shared__ int32_t list[CH * 256];
    __shared__ int32_t cnt[CH * 4];
    __shared__ int32_t below_sum, total;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t e = blockIdx.x / shares;
    const int c = static_cast<int>(blockIdx.x % shares);
    const int64_t b = blockIdx.y;
    const int64_t routes = seq * top_k;
    const int64_t rb = b * routes;
    const int J = static_cast<int>((routes + 255) / 256);
    if (tid == 0) below_sum = 0;
    // every load issued before any is used (one dtype branch, clamped
    // indices): a guarded load per route would wait for each in turn
    int64_t raw[CH];
    if (ids_dt == SANDY_I64) {
        const int64_t* p = static_cast<const int64_t*>(ids) + rb;
#pragma unroll
        for (int j = 0; j < CH; j++) {
            const int64_t r = tid + 256 * j;
            raw[j] = p[r < routes ? r : 0];
        }
    } else {
        const int32_t* p = static_cast<const int32_t*>(ids) + rb;
#pragma unroll
        for (int j = 0; j < CH; j++) {
            const int64_t r = tid + 256 * j;
            raw[j] = p[r < routes ? r : 0];
        }
    }
    int32_t v[CH];
#pragma unroll
    for (int j = 0; j < CH; j++) {
        const int64_t r = tid + 256 * j;
        v[j] = r >= routes ? -1 : (raw[j] >= 0 && raw[j] < experts ? static_cast<int32_t>(raw[j]) : -2);
    }
    int below = 0;
    bool bad = false;
#pragma unroll
    for (int j = 0; j < CH; j++) {
        if (j >= J) break;
        below += v[j] >= 0 && v[j] < e;
        bad |= v[j] == -2;
        const uint64_t m = __ballot(v[j] == e);
        if (lane == 0) cnt[j * 4 + wave] = __popcll(m);
    }
    if (bad && e == 0 && c == 0) atomicOr(errw, static_cast<uint32_t>(SANDY_DEVERR_EXPERT_ID));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) below += __shfl_xor(below, o, 64);
    __syncthreads();
    if (lane == 0) atomicAdd(&below_sum, below);
    if (wave == 0) {  // exclusive scan of the J * 4 (chunk, wave) counts, two per lane
        const int n = J * 4;
        const int a0 = 2 * lane < n ? cnt[2 * lane] : 0;
        const int a1 = 2 * lane + 1 < n ? cnt[2 * lane + 1] : 0;
        int incl = a0 + a1;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int up = __shfl_up(incl, d, 64);
            if (lane >= d) incl += up;
        }
        const int excl = incl - a0 - a1;
        if (2 * lane < n) cnt[2 * lane] = excl;
        if (2 * lane + 1 < n) cnt[2 * lane + 1] = excl + a0;
        if (lane == 63) total = incl;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < CH; j++) {
        if (j >= J) break;
        const uint64_t m = __ballot(v[j] == e);
        if (v[j] == e) list[cnt[j * 4 + wave] + __popcll(m & ((1ull << lane) - 1ull))] = tid + 256 * j;
    }
    __syncthreads();
    const int n = total;
    const int64_t base = below_sum;
    if (c == 0 && tid == 0) {
        store_index(offsets, off_dt, b * (experts + 1) + e, base);
        if (e == experts - 1) store_index(offsets, off_dt, b * (experts + 1) + experts, base + n);
    }
    // one wave per row of this share
    for (int q = c + shares * wave; q < n; q += shares * 4) {
        const int64_t r = list[q];
        const int64_t row = base + q;
        const int64_t t = r / top_k;
        // the weight's load is issued here, its store after the row's loads
        const float wr = load_any(w, w_dt, rb + r);
        const char* src = x + (b * seq + t) * row_bytes;
        char* dst = packed + (rb + row) * row_bytes;
        if (aligned) {
            typedef unsigned u32x4_nt __attribute__((ext_vector_type(4)));
            constexpr int kU = 8;  // 8 KiB of the row in flight per wave
            for (int64_t o0 = lane * 16; o0 < row_bytes; o0 += 64 * 16 * kU) {
                u32x4_nt tmp[kU];
#pragma unroll
                for (int u = 0; u < kU; u++) {
                    const int64_t o = o0 + u * 64 * 16;
                    if (o < row_bytes) tmp[u] = *reinterpret_cast<const u32x4_nt*>(src + o);
                }
#pragma unroll
                for (int u = 0; u < kU; u++) {
                    const int64_t o = o0 + u * 64 * 16;
                    if (o < row_bytes) __builtin_nontemporal_store(tmp[u], reinterpret_cast<u32x4_nt*>(dst + o));
                }
            }
        } else {
            for (int64_t o = lane; o < row_bytes; o += 64) dst[o] = src[o];
        }
        if (lane == 0) {
            store_any(packed_w, w_dt, rb + row, wr);
            store_index(token_ids, tok_dt, rb + row, t);
        }
    }
}

// Token-major form of the same permute (the default up to 8192 routes):
// workgroup = (TPW consecutive tokens, batch).  Every workgroup reads the
// batch's route ids once and builds in LDS the per-expert count of all valid
// routes and of those before its first route; an exclusive scan of the
// counts gives the expert offsets.  Its own routes (TPW * k <= 64) are ranked
// by one wave against the earlier ones of the same expert, so route r lands
// on row offset[e] + (routes of e before r) -- the reference's expert-major,
// then token, then slot order.  Each token's row is then read once and
// written to the rows of its k routes: x is read from HBM once, where the
// expert-major form reads each row from every XCD that holds one of its
// experts (1.5x the algorithmic bytes at config 5).
//
// Nothing loaded is consumed before every load is issued: ids are compiled
// for their width (I64), the routing weight is copied as raw bits (packed
// weights share its dtype), and the copy is compiled for the route count
// per token (TK; 0 = any, destination rows read 8 at a time), so each
// piece's stores issue back to back instead of one LDS round trip apart.
template <int CH, int TK, bool I64>
__global__ __launch_bounds__(256) void moe_dispatch_tokens_kernel(
        const void* __restrict__ ids, const void* __restrict__ w, int32_t w_dt, int64_t seq,
        int64_t top_k_arg, int64_t experts, int tpw, const char* __restrict__ x, char* __restrict__ packed,
        int64_t row_bytes, void* __restrict__ packed_w, void* __restrict__ token_ids, int32_t tok_dt,
        void* __restrict__ offsets, int32_t off_dt, uint32_t* errw) {
    // 32-bit route and expert arithmetic: the launch keeps routes <= 8192
    // and 2 * experts + 64 <= 16384
    const int top_k = TK > 0 ? TK : static_cast<int>(top_k_arg);
    const int E = static_cast<int>(experts);
    extern __shared__ int32_t sh[];
    int32_t* total = sh;           // [experts] valid routes (low 16 bits) and those before r0 (high 16 bits)
    int32_t* before = sh + E;      // [experts] first row of the expert's routes from r0 on
    int32_t* dest = sh + 2 * E;    // [64] rows of this workgroup's routes (-1: invalid id)
    const int tid = threadIdx.x, lane = tid & 63;
    const int64_t b = blockIdx.y;
    const int routes = static_cast<int>(seq) * top_k;
    const int64_t rb = b * routes;
    const int t0 = static_cast<int>(blockIdx.x) * tpw;
    const int t1 = min(static_cast<int>(seq), t0 + tpw);
    const int r0 = t0 * top_k, r1 = t1 * top_k;
    for (int i = tid; i < E; i += 256) total[i] = 0;
    // lane i of wave 0: the id and routing weight of route r0 + i, requested
    // with the rest (their addresses do not depend on the ranking)
    const int rmine = min(r0 + lane, max(r1, r0 + 1) - 1);
    typedef typename std::conditional<I64, uint64_t, uint32_t>::type id_t;  // unsigned: one range test
    const id_t* idp = static_cast<const id_t*>(ids) + rb;
    const bool wbf = w_dt == SANDY_BF16;
    id_t mine_id = 0;
    uint32_t mine_w = 0;  // raw bits of the routing weight
    if (tid < 64) {
        mine_id = idp[rmine];
        mine_w = wbf ? static_cast<uint32_t>(static_cast<const uint16_t*>(w)[rb + rmine])
                     : static_cast<const uint32_t*>(w)[rb + rmine];
    }
    id_t raw[CH];  // every id requested before any is used (clamped)
#pragma unroll
    for (int j = 0; j < CH; j++) {
        const int r = tid + 256 * j;
        raw[j] = idp[r < routes ? r : 0];
    }
    // the first batch of this workgroup's row pieces, requested with the ids
    // (they do not depend on the ranking); used after it
    typedef unsigned u32x4_nt __attribute__((ext_vector_type(4)));
    const int P = static_cast<int>(row_bytes >> 4);
    const int items = (t1 - t0) * P;
    const char* xw = x + (b * seq + t0) * row_bytes;  // this workgroup's first token row
    constexpr int kU = 8;
    u32x4_nt tmp[kU];
#pragma unroll
    for (int u = 0; u < kU; u++) {
        const int it = min(tid + 256 * u, items - 1);
        const int tl = it / P, pc = it - tl * P;
        tmp[u] = *reinterpret_cast<const u32x4_nt*>(xw + tl * row_bytes + pc * 16);
    }
    // the ids are first used here, after every load above is issued (the
    // compiler would otherwise hoist their range tests up to their loads and
    // wait there, ahead of the row pieces)
#pragma unroll
    for (int j = 0; j < CH; j++) asm volatile("" : "+v"(raw[j]));
    __syncthreads();
    bool bad = false;
    // every id is tested whatever its route (no early exit): a use only past
    // a branch would let the compiler move that id's load behind the barrier
#pragma unroll
    for (int j = 0; j < CH; j++) {
        const int r = tid + 256 * j;
        const bool in = r < routes;
        const bool ok = raw[j] < static_cast<id_t>(E);  // negative ids wrap past E
        const int e = static_cast<int>(raw[j]);
        bad = bad || (in && !ok);
        if (in && ok) atomicAdd(&total[e], r < r0 ? 0x10001 : 1);  // both counts in one atomic (routes < 2^16)
    }

    if (bad && blockIdx.x == 0) atomicOr(errw, static_cast<uint32_t>(SANDY_DEVERR_EXPERT_ID));
    __syncthreads();
    if (tid < 64) {
        // exclusive scan of the expert totals into `before` (+= offset), 64 lanes x (experts / 64) each
        const int per = (E + 63) >> 6;
        const int ex0 = lane * per;
        int run = 0;
        for (int q = 0; q < per; q++) run += ex0 + q < E ? total[ex0 + q] & 0xffff : 0;
        int incl = run;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int up = __shfl_up(incl, d, 64);
            if (lane >= d) incl += up;
        }
        int acc = incl - run;
        const int64_t ob = b * (experts + 1);
        for (int q = 0; q < per; q++) {
            const int ex = ex0 + q;
            if (ex < E) {
                const int tc = total[ex];
                if (blockIdx.x == 0) store_index(offsets, off_dt, ob + ex, acc);
                before[ex] = acc + (tc >> 16);
                acc += tc & 0xffff;
            }
        }
        if (blockIdx.x == 0 && lane == 63) store_index(offsets, off_dt, ob + E, incl);
        // rank this workgroup's routes (lane i: route r0 + i) against the earlier ones of their expert
        const int r = r0 + lane;
        const int er = r < r1 && mine_id < static_cast<id_t>(E) ? static_cast<int>(mine_id) : -1;
        // over this workgroup's routes only (TPW * k of them, uniform)
        const int nr = r1 - r0;
        int earlier = 0;
        for (int j = 0; j < nr; j++) {
            const int ej = __builtin_amdgcn_readlane(er, j);
            earlier += j < lane && ej == er;
        }
        if (r < r1) {
            const int row = er >= 0 ? before[er] + earlier : -1;
            dest[lane] = row;
            if (row >= 0) {
                if (wbf)
                    static_cast<uint16_t*>(packed_w)[rb + row] = static_cast<uint16_t>(mine_w);
                else
                    static_cast<uint32_t*>(packed_w)[rb + row] = mine_w;
                store_index(token_ids, tok_dt, rb + row, r / top_k);
            }
        }
    }
    __syncthreads();
    // copy: each token's row read once (16-byte pieces), written to its k rows
    for (int i0 = 0; i0 < items; i0 += 256 * kU) {
        if (i0 > 0) {
#pragma unroll
            for (int u = 0; u < kU; u++) {
                const int it = min(i0 + tid + 256 * u, items - 1);
                const int tl = it / P, pc = it - tl * P;
                tmp[u] = *reinterpret_cast<const u32x4_nt*>(xw + tl * row_bytes + pc * 16);
            }
        }
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const int it = i0 + tid + 256 * u;
            if (it >= items) break;
            const int tl = it / P, pc = it - tl * P;
            constexpr int kS = TK > 0 ? TK : 8;  // destination rows read per group
            for (int s0 = 0; s0 < top_k; s0 += kS) {
                int rows[kS];
#pragma unroll
                for (int s = 0; s < kS; s++) rows[s] = TK > 0 || s0 + s < top_k ? dest[tl * top_k + s0 + s] : -1;
#pragma unroll
                for (int s = 0; s < kS; s++)
                    if (rows[s] >= 0)
                        __builtin_nontemporal_store(tmp[u],
                                                    reinterpret_cast<u32x4_nt*>(packed + (rb + rows[s]) * row_bytes + pc * 16));
            }
        }
    }
}

template <int CH, int TK>
const void* dispatch_tokens_for(bool i64) {
    return i64 ? reinterpret_cast<const void*>(&moe_dispatch_tokens_kernel<CH, TK, true>)
               : reinterpret_cast<const void*>(&moe_dispatch_tokens_kernel<CH, TK, false>);
}

template <int CH>
const void* dispatch_tokens_ch(int64_t top_k, bool i64) {
    return top_k == 8   ? dispatch_tokens_for<CH, 8>(i64)
           : top_k == 4 ? dispatch_tokens_for<CH, 4>(i64)
           : top_k == 2 ? dispatch_tokens_for<CH, 2>(i64)
                        : dispatch_tokens_for<CH, 0>(i64);
}

// ---------------------------------------------------------------- moe_scatter_sum
// Workgroup = (batch, 4 tokens, 512-column chunk); wave = one token.  The
// workgroup reads the batch's token ids once (16 loads per thread in flight)
// and each thread tests its own ids against the workgroup's 4 tokens: a hit
// is appended to its token's list with an LDS atomic, and each wave then puts
// its list (the token's k rows) back in row order by ranking.  No wave scans
// the whole id list.  The rows are processed 8 at a time: the 8 rows' loads
// are issued together and accumulated in row order with the reference's two
// roundings (product, then sum rounded to the output dtype) -- bit-identical
// to the CPU, no atomics on the output.  A token with more than kCombineHits
// rows falls back to collecting them in row order with ballots.
__device__ __forceinline__ float elem_to_f32(uint16_t b) { return bf16_to_f32(b); }
__device__ __forceinline__ float elem_to_f32(float f) { return f; }

constexpr int kCombineHits = 128;  // per-wave hit list

template <typename T>
__global__ __launch_bounds__(256) void moe_combine_kernel(const void* __restrict__ packed,
                                                          const void* __restrict__ pw,
                                                          const void* __restrict__ tok, int32_t tok_dt,
                                                          void* __restrict__ out, int64_t batch, int64_t rows,
                                                          int64_t hidden, int64_t seq, uint32_t* errw) {
    __shared__ int32_t hit[4][kCombineHits];
    __shared__ int32_t hits_n[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t chunks = (hidden + 511) / 512;
    const int64_t tgroups = (seq + 3) / 4;
    const int64_t ch = blockIdx.x % chunks;
    const int64_t tg = (blockIdx.x / chunks) % tgroups;
    const int64_t b = blockIdx.x / (chunks * tgroups);
    const int64_t t = tg * 4 + wave;
    const int64_t mb = b * rows;
    if (threadIdx.x < 4) hits_n[threadIdx.x] = 0;
    __syncthreads();
    {
        // 16 loads per thread in flight at once, then the tests
        constexpr int kBatch = 16;
        const int64_t tbase = tg * 4;
        const bool flag = blockIdx.x % (chunks * tgroups) == 0;  // one workgroup per batch raises the flag
        for (int64_t r0 = threadIdx.x; r0 < rows; r0 += 256 * kBatch) {
            int64_t v[kBatch];
            // one dtype branch around the whole batch: a per-load select made
            // the compiler wait for every load in turn
            if (tok_dt == SANDY_I64) {
#pragma unroll
                for (int u = 0; u < kBatch; u++) {
                    const int64_t r = r0 + 256 * u;
                    v[u] = static_cast<const int64_t*>(tok)[mb + (r < rows ? r : 0)];
                }
            } else {
#pragma unroll
                for (int u = 0; u < kBatch; u++) {
                    const int64_t r = r0 + 256 * u;
                    v[u] = static_cast<const int32_t*>(tok)[mb + (r < rows ? r : 0)];
                }
            }
#pragma unroll
            for (int u = 0; u < kBatch; u++) {
                const int64_t r = r0 + 256 * u;
                if (r >= rows) break;
                const bool valid = v[u] >= 0 && v[u] < seq;
                if (!valid && flag) atomicOr(errw, static_cast<uint32_t>(SANDY_DEVERR_TOKEN_ID));
                const uint64_t d = static_cast<uint64_t>(v[u] - tbase);
                if (valid && d < 4) {
                    const int slot = atomicAdd(&hits_n[d], 1);
                    if (slot < kCombineHits) hit[d][slot] = static_cast<int32_t>(r);
                }
            }
        }
    }
    __syncthreads();
    if (t >= seq) return;
    const int64_t c0 = ch * 512 + lane * 8;
    const bool vec = (hidden & 7) == 0;
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = 0.0f;
    // accumulate the n collected rows of hit[wave], 8 loads in flight at a time
    // every load of a group of 8 rows is issued before any is used: rows
    // past n repeat row g and columns past the end repeat column 0 (their
    // values are not accumulated), so no load sits behind a branch
    auto accumulate = [&](int n) {
        const int64_t cc = c0 < hidden ? c0 : 0;
        for (int g = 0; g < n; g += 8) {
            using E = typename Vec8<T>::elem;
            int64_t row[8];
#pragma unroll
            for (int u = 0; u < 8; u++) row[u] = hit[wave][g + u < n ? g + u : g];
            if (vec) {
                // raw row pieces first, then the raw weights, converted only
                // when used (a conversion is a use: it would wait for the load)
                typename Vec8<T>::raw pr[8];
                E we[8];
#pragma unroll
                for (int u = 0; u < 8; u++) pr[u] = Vec8<T>::load_raw(packed, (mb + row[u]) * hidden + cc);
#pragma unroll
                for (int u = 0; u < 8; u++) we[u] = static_cast<const E*>(pw)[mb + row[u]];
                // computed for every u and kept by a select: a branch around
                // the uses lets the compiler sink each load into it
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const bool live = g + u < n && c0 < hidden;
                    float pv[8];
                    Vec8<T>::unpack(pr[u], pv);
                    const float wv = elem_to_f32(we[u]);
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        const float nv = Vec8<T>::round(__fadd_rn(acc[i], __fmul_rn(wv, pv[i])));
                        acc[i] = live ? nv : acc[i];
                    }
                }
            } else {
                float wv[8];
#pragma unroll
                for (int u = 0; u < 8; u++) wv[u] = Vec8<T>::load1(pw, mb + row[u]);
                float pv[8][8];
#pragma unroll
                for (int u = 0; u < 8; u++)
#pragma unroll
                    for (int i = 0; i < 8; i++)
                        pv[u][i] = Vec8<T>::load1(packed, (mb + row[u]) * hidden + (c0 + i < hidden ? c0 + i : 0));
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    if (g + u >= n) break;
#pragma unroll
                    for (int i = 0; i < 8; i++) acc[i] = Vec8<T>::round(__fadd_rn(acc[i], __fmul_rn(wv[u], pv[u][i])));
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
    };
    int64_t r0 = 0;
    const int n_hits = hits_n[wave];
    if (n_hits <= kCombineHits) {
        // the list holds the token's rows in arrival order: rank each (rows
        // are distinct) and write it back at its rank
        const int e0 = lane < n_hits ? hit[wave][lane] : 0;
        const int e1 = lane + 64 < n_hits ? hit[wave][lane + 64] : 0;
        int k0 = 0, k1 = 0;
        for (int j = 0; j < n_hits; j++) {
            const int ej = hit[wave][j];  // same address in every lane: one broadcast read
            k0 += ej < e0;
            k1 += ej < e1;
        }
        __builtin_amdgcn_wave_barrier();
        if (lane < n_hits) hit[wave][k0] = e0;
        if (lane + 64 < n_hits) hit[wave][k1] = e1;
        __builtin_amdgcn_wave_barrier();
        accumulate(n_hits);
        r0 = rows;
    }
    while (r0 < rows) {
        // collect up to kCombineHits rows of token t, in row order
        int n = 0;
        for (; r0 < rows && n + 64 <= kCombineHits; r0 += 64) {
            const int64_t r = r0 + lane;
            int64_t tr = -1;
            if (r < rows) tr = load_index(tok, tok_dt, mb + r);  // invalid ids were flagged above
            const uint64_t hits = __ballot(tr == t);
            if (tr == t) hit[wave][n + __popcll(hits & ((1ull << lane) - 1ull))] = static_cast<int32_t>(r);
            n += __popcll(hits);
        }
        __builtin_amdgcn_wave_barrier();
        accumulate(n);
        __builtin_amdgcn_wave_barrier();
    }
    if (c0 < hidden) {
        const int64_t dst = (b * seq + t) * hidden + c0;
        if (vec) {
            Vec8<T>::store(out, dst, acc);
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (c0 + i < hidden) Vec8<T>::store1(out, dst + i, acc[i]);
        }
    }
}

// ---------------------------------------------------------------- moe_matmul
// Grouped GEMM, bf16, transpose_rhs: out[row, n] = sum_k x[row, k] W[e, n, k].
// Workgroup = (expert, 64 * CT output columns); wave w owns 16 * CT columns
// and up to 16 * RT rows of the expert per pass (A = x rows, B = W rows on
// v_mfma_f32_16x16x32_bf16); the weight slice is streamed from HBM once per
// pass.  Both operands are read as whole 128-byte lines: loading MFMA
// operands straight into registers touches 16 rows x 64 bytes per
// instruction; on gfx950 that pattern streams at about 3.2 TB/s against
// 5.0 TB/s for 8 rows x 128 bytes.  Per chunk of 64 k:
//   - the workgroup loads the expert's 16 * RT activation rows once (every
//     wave multiplies them) into a shared LDS tile;
//   - each wave loads its 16 * CT weight rows into a private LDS tile;
// both as full lines (8 rows x 128 bytes per instruction) into tiles whose
// 16-byte pieces are XOR-swizzled by (row / 2) % 8, so 128-bit writes and
// the MFMA-layout 128-bit reads are conflict-free; the k order inside a
// chunk is unchanged.  Tiles are double buffered: chunk c + 1's loads are in
// flight while chunk c multiplies, then land in the other buffer before the
// workgroup barrier.  Two waves fit per SIMD at RT = CT = 4.
template <int RT, int CT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void moe_gemm_lines_kernel(
        const uint16_t* __restrict__ x, const void* __restrict__ offs, int32_t off_dt, const uint16_t* __restrict__ w,
        uint16_t* __restrict__ out, int64_t rows, int64_t K, int64_t M, int64_t experts, int64_t batch,
        uint32_t* errw) {
    constexpr int kWTile = 16 * CT * 128;  // one wave's weight rows x 128 bytes
    constexpr int kXTile = 16 * RT * 128;  // the workgroup's activation rows x 128 bytes
    constexpr int kXPer = (16 * RT * 8 + 255) / 256;  // 16-byte activation pieces per thread
    __shared__ __attribute__((aligned(16))) unsigned char lds[2 * kXTile + 4 * 2 * kWTile];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t e = blockIdx.x % experts;
    const int64_t b = blockIdx.x / experts;
    const int64_t n0 = (static_cast<int64_t>(blockIdx.y) * 4 + wave) * 16 * CT;
    const int64_t ob = b * (experts + 1);
    const int64_t begin = load_index(offs, off_dt, ob + e);
    const int64_t end = load_index(offs, off_dt, ob + e + 1);
    if (begin < 0 || end < begin || end > rows) {
        if (tid == 0 && blockIdx.y == 0) atomicOr(errw, static_cast<uint32_t>(SANDY_DEVERR_OFFSETS));
        return;
    }
    if (end == begin || static_cast<int64_t>(blockIdx.y) * 64 * CT >= M) return;  // workgroup-uniform exits only
    const bool wave_live = n0 < M;
    unsigned char* xt = lds;                           // [2][kXTile]
    unsigned char* wt = lds + 2 * kXTile + wave * 2 * kWTile;  // [2][kWTile]
    auto swz = [](int row, int piece) { return row * 128 + ((piece ^ ((row >> 1) & 7)) << 4); };
    const int64_t xb = b * rows * K, yb = b * rows * M;
    const int64_t ksteps = K / 32;
    const int64_t chunks = (ksteps + 1) / 2;  // 64 k per chunk
    // Buffer resources: one scalar base, a 32-bit lane offset and a scalar
    // offset per load; pieces past the range read as zero.
    const int64_t wrows = wave_live ? min<int64_t>(16 * CT, M - n0) : 0;
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(w + (e * M + (wave_live ? n0 : 0)) * K), 0, static_cast<int>(wrows * K * 2), 0x00020000);
    // weight instruction i covers tile rows 8i .. 8i + 7 (lane: row 8i + lane/8, piece lane%8)
    const int wlane = static_cast<int>((lane >> 3) * K * 2 + (lane & 7) * 16);
    const int wstep = static_cast<int>(8 * K * 2);
    // tile row 8i + lane/8 swizzles by (4i + lane/16) % 8: one base for even i, one for odd i (+ i * 1024)
    const int wbase[2] = {swz(lane >> 3, lane & 7), swz(8 + (lane >> 3), lane & 7) - 1024};
    const bool w_hi = (lane & 7) >= 4;  // this lane's weight piece lies in the chunk's second k-step
    // activation piece q of this thread: tile row p / 8, piece p % 8 with p = tid + 256 q
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

    for (int64_t r0 = begin; r0 < end; r0 += 16 * RT) {
        const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(x + xb + r0 * K), 0, static_cast<int>(min<int64_t>(end - r0, 16 * RT) * K * 2),
            0x00020000);
        f32x4_t acc[RT][CT];
#pragma unroll
        for (int t = 0; t < RT; t++)
#pragma unroll
            for (int c = 0; c < CT; c++) acc[t][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        uint4 wv[2 * CT], xv[kXPer];
        auto load = [&](int64_t ch) {
            const bool win = 2 * ch + (w_hi ? 1 : 0) < ksteps;
#pragma unroll
            for (int i = 0; i < 2 * CT; i++) {
                // non-temporal: each expert weight line is read by exactly one
                // workgroup (gate 97.5 -> 92.7 us, down 106.6 -> 98.4 at config 5)
                const uint4 v = __builtin_bit_cast(
                    uint4, __builtin_amdgcn_raw_buffer_load_b128(wres, wlane, static_cast<int>(i * wstep + ch * 128), 2));
                wv[i] = win ? v : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int q = 0; q < kXPer; q++) {
                const uint4 v = __builtin_bit_cast(
                    uint4, __builtin_amdgcn_raw_buffer_load_b128(xres, xoff[q], static_cast<int>(ch * 128), 0));
                xv[q] = 2 * ch + (x_hi[q] ? 1 : 0) < ksteps ? v : make_uint4(0, 0, 0, 0);
            }
        };
        auto store = [&](int buf) {
#pragma unroll
            for (int i = 0; i < 2 * CT; i++)
                *reinterpret_cast<uint4*>(wt + buf * kWTile + wbase[i & 1] + i * 1024) = wv[i];
#pragma unroll
            for (int q = 0; q < kXPer; q++)
                if (xlive[q]) *reinterpret_cast<uint4*>(xt + buf * kXTile + xaddr[q]) = xv[q];
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
                                                                            __builtin_bit_cast(bf16x8_t, bv),
                                                                            acc[t][c], 0, 0, 0);
                }
            }
        };
        // chunk ch multiplies out of buffer ch % 2 while chunk ch + 1's loads are in flight
        load(0);
        store(0);
        __syncthreads();
        for (int64_t ch = 0; ch < chunks; ch++) {
            if (ch + 1 < chunks) load(ch + 1);
            if (wave_live) mma(static_cast<int>(ch & 1));
            if (ch + 1 < chunks) store(static_cast<int>((ch + 1) & 1));
            __syncthreads();
        }
        if (wave_live) {
            // acc[t][c][i]: row r0 + 16 t + 4 (lane/16) + i, column n0 + 16 c + lane%16
#pragma unroll
            for (int t = 0; t < RT; t++)
#pragma unroll
                for (int c = 0; c < CT; c++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int64_t rr = r0 + 16 * t + 4 * (lane >> 4) + i;
                        const int64_t nc = n0 + 16 * c + (lane & 15);
                        if (rr < end && nc < M) out[yb + rr * M + nc] = f32_to_bf16(acc[t][c][i]);  // 2-byte: L2 combines them
                    }
        }
    }
}

// Any dtype / layout: one thread per (row, column), float accumulation in k
// order like the reference.
template <typename T>
__global__ __launch_bounds__(256) void moe_gemm_generic_kernel(const void* __restrict__ x,
                                                               const void* __restrict__ offs, int32_t off_dt,
                                                               const void* __restrict__ w, void* __restrict__ out,
                                                               int64_t rows, int64_t K, int64_t M, int64_t experts,
                                                               int64_t batch, int32_t transpose_rhs, uint32_t* errw) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= batch * rows * M) return;
    const int64_t o = t % M, r = (t / M) % rows, b = t / (M * rows);
    const int64_t ob = b * (experts + 1);
    // expert of row r: last e with off[e] <= r < off[e + 1]
    int64_t e = -1;
    int64_t lo = 0, hi = experts;  // binary search on the monotone offsets
    while (lo < hi) {
        const int64_t mid = (lo + hi) / 2;
        if (load_index(offs, off_dt, ob + mid + 1) <= r) lo = mid + 1;
        else hi = mid;
    }
    if (lo < experts && load_index(offs, off_dt, ob + lo) <= r && r < load_index(offs, off_dt, ob + lo + 1)) e = lo;
    if (e < 0) return;  // row outside every expert range: the reference leaves it untouched
    float acc = 0.0f;
    for (int64_t k = 0; k < K; k++) {
        const float xv = Vec8<T>::load1(x, (b * rows + r) * K + k);
        const int64_t wi = transpose_rhs ? (e * M + o) * K + k : (e * K + k) * M + o;
        acc = __fadd_rn(acc, __fmul_rn(xv, Vec8<T>::load1(w, wi)));
    }
    Vec8<T>::store1(out, (b * rows + r) * M + o, acc);
}

// One thread per (batch, expert): offsets must be non-negative, monotone and
// within the row count.
__global__ void validate_offsets_kernel(const void* __restrict__ offs, int32_t off_dt, int64_t experts, int64_t rows,
                                        int64_t batch, uint32_t* errw) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= batch * experts) return;
    const int64_t b = t / experts, e = t % experts;
    const int64_t lo = load_index(offs, off_dt, b * (experts + 1) + e);
    const int64_t hi = load_index(offs, off_dt, b * (experts + 1) + e + 1);
    if (lo < 0 || hi < lo || hi > rows) atomicOr(errw, static_cast<uint32_t>(SANDY_DEVERR_OFFSETS));
}

} // namespace
} // namespace sandy_hip

using namespace sandy_hip;

extern "C" int sandy_hip_topk(const SandyTensor* x, int64_t k, int64_t axis, const SandyTensor* values,
                              const SandyTensor* indices, void* stream_, char* err, size_t err_cap) {
    Err e{err, err_cap};
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (!valid_rank(x) || !valid_rank(values) || !valid_rank(indices)) return fail(e, SANDY_ERR_INVALID, "topk tensor rank out of range");
    if (!is_float(x->dtype)) return fail(e, SANDY_ERR_INVALID, "topk input unsupported dtype");
    const int rank = x->rank;
    if (rank < 1) return fail(e, SANDY_ERR_INVALID, "topk input must have rank >= 1");
    if (axis < -rank || axis >= rank) return fail(e, SANDY_ERR_INVALID, "topk dim out of range");
    if (axis < 0) axis += rank;
    if (k <= 0) return fail(e, SANDY_ERR_INVALID, "topk k must be > 0");
    const int64_t n = x->dims[axis];
    if (n <= 0 || k > n) return fail(e, SANDY_ERR_INVALID, "topk invalid k or axis dimension");
    bool shape_ok = values->rank == rank && indices->rank == rank && values->dtype == x->dtype;
    for (int i = 0; shape_ok && i < rank; i++) {
        const int64_t want = i == axis ? k : x->dims[i];
        shape_ok = values->dims[i] == want && indices->dims[i] == want;
    }
    if (!shape_ok || values->dtype != x->dtype) return fail(e, SANDY_ERR_INVALID, "topk values output shape mismatch");
    if (!is_index(indices->dtype)) return fail(e, SANDY_ERR_INVALID, "topk indices output shape or dtype mismatch");
    if (!contiguous(*x) || !contiguous(*values) || !contiguous(*indices))
        return fail(e, SANDY_ERR_UNSUPPORTED, "topk requires contiguous tensors");
    int64_t outer = 1, inner = 1;
    for (int i = 0; i < axis; i++) outer *= x->dims[i];
    for (int i = static_cast<int>(axis) + 1; i < rank; i++) inner *= x->dims[i];
    if (outer * inner == 0) return ok(e);
    const bool bf = x->dtype == SANDY_BF16;
    const void* px = base_ptr(*x);
    void* pv = base_ptr(*values);
    void* pi = base_ptr(*indices);
    if (inner == 1 && n <= 1024) {
        dim3 grid(static_cast<unsigned>((outer + 3) / 4));
        const int ax = static_cast<int>(n), kk = static_cast<int>(k);
#define TOPK_LAUNCH(NV)                                                                                                 \
    if (bf) hipLaunchKernelGGL((topk_rows_kernel<BF16, NV>), grid, dim3(256), 0, stream, px, pv, pi, indices->dtype, outer, ax, kk); \
    else hipLaunchKernelGGL((topk_rows_kernel<F32, NV>), grid, dim3(256), 0, stream, px, pv, pi, indices->dtype, outer, ax, kk)
#define TOPK_RANK4(NV)                                                                                                  \
    if (bf) hipLaunchKernelGGL((topk_rank4_kernel<BF16, NV>), dim3(static_cast<unsigned>(outer)), dim3(256), 0, stream, px, pv, pi, indices->dtype, outer, ax, kk); \
    else hipLaunchKernelGGL((topk_rank4_kernel<F32, NV>), dim3(static_cast<unsigned>(outer)), dim3(256), 0, stream, px, pv, pi, indices->dtype, outer, ax, kk)
        if (n <= 64) { TOPK_RANK4(1); }
        else if (n <= 128) { TOPK_RANK4(2); }
        else if (n <= 256) { TOPK_RANK4(4); }
        else if (n <= 512) { TOPK_LAUNCH(8); }
        else { TOPK_LAUNCH(16); }
#undef TOPK_LAUNCH
#undef TOPK_RANK4
    } else if (inner == 1 && k == 1 && outer <= 65535 && n < (int64_t{1} << 31)) {
        // workgroup chunk of U * 2048 elements: the largest U in {2, 4, 8}
        // that still gives at least 2048 workgroups
        static const int forced = [] {
            const char* v = std::getenv("SANDY_ARGMAX_U");
            return v ? std::atoi(v) : 0;
        }();
        int u = 8;
        while (u > 2 && outer * ((n + u * 2048 - 1) / (u * 2048)) < 2048) u >>= 1;
        if (forced == 2 || forced == 4 || forced == 8) u = forced;
        const int64_t chunks = (n + u * 2048 - 1) / (u * 2048);
        int status = 0;
        uint64_t* slots = static_cast<uint64_t*>(
            device_counters(2, static_cast<size_t>(outer) * kArgmaxSlotWords * sizeof(uint64_t), stream, e, &status));
        if (status) return status;
        dim3 g1(static_cast<unsigned>(chunks), static_cast<unsigned>(outer));
        const bool vec = n % 8 == 0 && (reinterpret_cast<uintptr_t>(px) & 31) == 0;
        const int ch = static_cast<int>(chunks);
        const int32_t idt = indices->dtype;
#define ARGMAX_LAUNCH(T, UU)                                                                                           \
    if (vec) hipLaunchKernelGGL((argmax_wide_kernel<T, UU, true>), g1, dim3(256), 0, stream, px, n, ch, slots, pv, pi, idt); \
    else hipLaunchKernelGGL((argmax_wide_kernel<T, UU, false>), g1, dim3(256), 0, stream, px, n, ch, slots, pv, pi, idt)
#define ARGMAX_U(T) \
    if (u == 2) { ARGMAX_LAUNCH(T, 2); } else if (u == 4) { ARGMAX_LAUNCH(T, 4); } else { ARGMAX_LAUNCH(T, 8); }
        if (bf) { ARGMAX_U(BF16); } else { ARGMAX_U(F32); }
#undef ARGMAX_U
#undef ARGMAX_LAUNCH
    } else if (inner == 1 && k <= kWideMaxK && outer <= 65535) {
        const int64_t chunks = (n + kWideChunk - 1) / kWideChunk;
        int status = 0;
        char* ws = static_cast<char*>(
            device_workspace(3, static_cast<size_t>(outer * chunks * k) * (sizeof(float) + sizeof(int64_t)), stream, e,
                             &status));
        if (status) return status;
        int64_t* ci = reinterpret_cast<int64_t*>(ws);
        float* cv = reinterpret_cast<float*>(ci + outer * chunks * k);
        const int kk = static_cast<int>(k);
        dim3 g1(static_cast<unsigned>(chunks), static_cast<unsigned>(outer));
        const bool vec = n % 8 == 0 && (reinterpret_cast<uintptr_t>(px) & 31) == 0;
        if (bf) {
            if (vec) hipLaunchKernelGGL((topk_wide_chunks_kernel<BF16, true>), g1, dim3(256), 0, stream, px, n, chunks, kk, cv, ci);
            else hipLaunchKernelGGL((topk_wide_chunks_kernel<BF16, false>), g1, dim3(256), 0, stream, px, n, chunks, kk, cv, ci);
            hipLaunchKernelGGL(topk_wide_merge_kernel<BF16>, dim3(static_cast<unsigned>(outer)), dim3(256), 0, stream, cv, ci,
                               chunks, kk, pv, pi, indices->dtype);
        } else {
            if (vec) hipLaunchKernelGGL((topk_wide_chunks_kernel<F32, true>), g1, dim3(256), 0, stream, px, n, chunks, kk, cv, ci);
            else hipLaunchKernelGGL((topk_wide_chunks_kernel<F32, false>), g1, dim3(256), 0, stream, px, n, chunks, kk, cv, ci);
            hipLaunchKernelGGL(topk_wide_merge_kernel<F32>, dim3(static_cast<unsigned>(outer)), dim3(256), 0, stream, cv, ci,
                               chunks, kk, pv, pi, indices->dtype);
        }
    } else {
        const int64_t threads = outer * inner;
        dim3 grid(static_cast<unsigned>((threads + 255) / 256));
        if (bf) hipLaunchKernelGGL(topk_columns_kernel<BF16>, grid, dim3(256), 0, stream, px, pv, pi, indices->dtype, outer, n, inner, k);
        else hipLaunchKernelGGL(topk_columns_kernel<F32>, grid, dim3(256), 0, stream, px, pv, pi, indices->dtype, outer, n, inner, k);
    }
    SANDY_HIP_TRY(hipGetLastError(), e, "topk launch");
    return ok(e);
}

extern "C" int sandy_hip_moe_gather(const SandyTensor* x, const SandyTensor* topk_ids, const SandyTensor* topk_weights,
                                    int64_t num_experts, int64_t top_k, const SandyTensor* packed_x,
                                    const SandyTensor* packed_weights, const SandyTensor* token_ids,
                                    const SandyTensor* expert_offsets, void* stream_, char* err, size_t err_cap) {
    Err e{err, err_cap};
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    const SandyTensor* all[] = {x, topk_ids, topk_weights, packed_x, packed_weights, token_ids, expert_offsets};
    for (const SandyTensor* t : all)
        if (!valid_rank(t)) return fail(e, SANDY_ERR_INVALID, "moe_gather requires every tensor");
    if (!is_float(x->dtype)) return fail(e, SANDY_ERR_INVALID, "moe_gather x unsupported dtype");
    if (!is_float(topk_weights->dtype)) return fail(e, SANDY_ERR_INVALID, "moe_gather topk_weights unsupported dtype");
    if (!is_index(topk_ids->dtype)) return fail(e, SANDY_ERR_INVALID, "moe_gather topk_ids must be i32 or i64");
    if (!is_index(token_ids->dtype)) return fail(e, SANDY_ERR_INVALID, "moe_gather token_ids must be i32 or i64");
    if (!is_index(expert_offsets->dtype)) return fail(e, SANDY_ERR_INVALID, "moe_gather expert_offsets must be i32 or i64");
    const int xr = x->rank;
    if ((xr != 2 && xr != 3) || topk_ids->rank != xr || topk_weights->rank != xr)
        return fail(e, SANDY_ERR_INVALID, "moe_gather inputs must have rank 2 or rank 3");
    if (num_experts <= 0 || top_k <= 0) return fail(e, SANDY_ERR_INVALID, "moe_gather num_experts and top_k must be positive");
    const int64_t batch = xr == 3 ? x->dims[0] : 1;
    const int64_t seq = x->dims[xr - 2], hidden = x->dims[xr - 1];
    for (int i = 0; i < xr - 1; i++)
        if (x->dims[i] != topk_ids->dims[i] || x->dims[i] != topk_weights->dims[i])
            return fail(e, SANDY_ERR_INVALID, "moe_gather leading dimension mismatch");
    if (topk_ids->dims[xr - 1] != top_k || topk_weights->dims[xr - 1] != top_k)
        return fail(e, SANDY_ERR_INVALID, "moe_gather top_k dimension mismatch");
    const int64_t routes = seq * top_k;
    if (numel(*packed_x) != batch * routes * hidden || packed_x->dtype != x->dtype ||
        packed_x->dims[packed_x->rank - 1] != hidden)
        return fail(e, SANDY_ERR_INVALID, "moe_gather packed_x output shape mismatch");
    if (numel(*packed_weights) != batch * routes || packed_weights->dtype != topk_weights->dtype)
        return fail(e, SANDY_ERR_INVALID, "moe_gather packed_weights output shape mismatch");
    if (numel(*token_ids) != batch * routes || numel(*expert_offsets) != batch * (num_experts + 1))
        return fail(e, SANDY_ERR_INVALID, "moe_gather metadata output shape mismatch");
    for (const SandyTensor* t : all)
        if (!contiguous(*t)) return fail(e, SANDY_ERR_UNSUPPORTED, "moe_gather requires contiguous tensors");
    const size_t lds = static_cast<size_t>(num_experts) * (1 + kRouteWaves) * sizeof(int32_t) + 2 * kRouteStage * 4;
    if (lds > 64 * 1024) return fail(e, SANDY_ERR_UNSUPPORTED, "moe_gather supports up to %d experts", (64 * 1024 / 4 - 2 * kRouteStage) / (1 + kRouteWaves));
    if (batch == 0) return ok(e);
    int status = 0;
    uint32_t* errw = device_error_word(e, &status);
    if (status) return status;
    const int64_t row_bytes = hidden * static_cast<int64_t>(dtype_size(x->dtype));
    const int aligned = (row_bytes % 16 == 0) &&
                        ((reinterpret_cast<uintptr_t>(base_ptr(*x)) | reinterpret_cast<uintptr_t>(base_ptr(*packed_x))) & 15) == 0;
    if (routes <= kDispatchRoutes && batch <= 65535 && aligned && top_k <= 64 && 2 * num_experts + 64 <= 16384 &&
        env_int("SANDY_MOE_ROUTE_GENERAL", 0) == 0) {
        // token-major: about 256 workgroups of ceil(seq / 256) tokens (at most 64 routes each)
        const int64_t tpw = std::max<int64_t>(1, std::min<int64_t>(64 / top_k, (seq + 255) / 256));
        const int64_t wgs = (seq + tpw - 1) / tpw;
        if (wgs > 0x7fffffff) return fail(e, SANDY_ERR_UNSUPPORTED, "moe_gather too many tokens");
        const size_t shb = static_cast<size_t>(2 * num_experts + 64) * sizeof(int32_t);
        dim3 grid(static_cast<unsigned>(wgs), static_cast<unsigned>(batch));
        const bool i64 = topk_ids->dtype == SANDY_I64;
        const void* kern = routes <= 4096 ? dispatch_tokens_ch<16>(top_k, i64) : dispatch_tokens_ch<32>(top_k, i64);
        const void* ids_p = base_ptr(*topk_ids);
        const void* w_p = base_ptr(*topk_weights);
        int32_t w_dt = topk_weights->dtype, tok_dt = token_ids->dtype, off_dt = expert_offsets->dtype;
        int64_t seq_a = seq, topk_a = top_k, experts_a = num_experts;
        int tpw_a = static_cast<int>(tpw);
        const char* x_p = static_cast<const char*>(base_ptr(*x));
        char* px_p = static_cast<char*>(base_ptr(*packed_x));
        int64_t rb_a = row_bytes;
        void* pw_p = base_ptr(*packed_weights);
        void* tok_p = base_ptr(*token_ids);
        void* off_p = base_ptr(*expert_offsets);
        void* args[] = {&ids_p, &w_p, &w_dt, &seq_a, &topk_a, &experts_a, &tpw_a, &x_p, &px_p,
                        &rb_a, &pw_p, &tok_p, &tok_dt, &off_p, &off_dt, &errw};
        SANDY_HIP_TRY(hipLaunchKernel(kern, grid, dim3(256), args, shb, stream), e, "moe_gather launch");
        return ok(e);
    }
    if (routes <= kDispatchRoutes && batch <= 65535 && env_int("SANDY_MOE_ROUTE_GENERAL", 0) == 0) {
        // about 512 workgroups, each expert's rows shared by up to 8: every
        // workgroup re-reads the route ids, so more workgroups cost more
        // than their extra copy bandwidth gains (config 5: 8 -> 11.6 us,
        // 4 -> 11.3, 2 -> 14.0, 16 -> 16.7)
        const int64_t shares = std::max<int64_t>(1, std::min<int64_t>(8, 512 / std::max<int64_t>(1, num_experts * batch)));
        if (num_experts * shares > 0x7fffffff) return fail(e, SANDY_ERR_UNSUPPORTED, "moe_gather too many experts");
        dim3 grid(static_cast<unsigned>(num_experts * shares), static_cast<unsigned>(batch));
        hipLaunchKernelGGL(routes <= 4096 ? moe_dispatch_kernel<16> : moe_dispatch_kernel<32>, grid, dim3(256), 0, stream, base_ptr(*topk_ids), topk_ids->dtype,
                           base_ptr(*topk_weights), topk_weights->dtype, seq, top_k, num_experts,
                           static_cast<int>(shares), static_cast<const char*>(base_ptr(*x)),
                           static_cast<char*>(base_ptr(*packed_x)), row_bytes, aligned, base_ptr(*packed_weights),
                           base_ptr(*token_ids), token_ids->dtype, base_ptr(*expert_offsets), expert_offsets->dtype,
                           errw);
        SANDY_HIP_TRY(hipGetLastError(), e, "moe_gather launch");
        return ok(e);
    }
    int32_t* dest = static_cast<int32_t*>(device_workspace(2, static_cast<size_t>(batch * routes) * sizeof(int32_t), stream, e, &status));
    if (status) return status;
    hipLaunchKernelGGL(moe_route_kernel, dim3(static_cast<unsigned>(batch)), dim3(kRouteThreads), lds, stream,
                       base_ptr(*topk_ids), topk_ids->dtype, base_ptr(*topk_weights), topk_weights->dtype, seq, top_k,
                       num_experts, base_ptr(*packed_weights), base_ptr(*token_ids), token_ids->dtype,
                       base_ptr(*expert_offsets), expert_offsets->dtype, dest, errw);
    if (routes > 0 && hidden > 0) {
        const int64_t waves = batch * routes;
        hipLaunchKernelGGL(moe_copy_rows_kernel, dim3(static_cast<unsigned>((waves + 3) / 4)), dim3(256), 0, stream,
                           static_cast<const char*>(base_ptr(*x)), static_cast<char*>(base_ptr(*packed_x)), dest, batch,
                           seq, top_k, row_bytes, aligned);
    }
    SANDY_HIP_TRY(hipGetLastError(), e, "moe_gather launch");
    return ok(e);
}

namespace sandy_hip {
namespace {
// Column tile (16 * CT columns a wave, 64 * CT a workgroup) of the 64-row
// grouped-GEMM kernel: the one whose workgroups fill whole rounds of the
// resident slots best (two workgroups a CU), counting the padded columns of
// the last tile; ties go to the wider tile (fewer activation re-reads).
// Config 5: gate and up (704 columns, 128 experts) take 192-column tiles,
// 512 workgroups, one full round (gate 91.4 -> 86.1 us, up 85.2 -> 81.0);
// down (2816 columns) keeps 256 (98.0 us against 100.6-101.0 at 192).
int moe_column_tile(int64_t M, int64_t groups) {
    static const int slots = [] {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        return 2 * cus;
    }();
    int best = 4;
    double best_eff = -1.0;
    for (int ct = 4; ct >= 2; ct--) {
        const int64_t tiles = (M + 64 * ct - 1) / (64 * ct);
        const int64_t wgs = tiles * groups;
        const int64_t rounds = (wgs + slots - 1) / slots;
        const double eff = static_cast<double>(M) / static_cast<double>(tiles * 64 * ct) *
                           static_cast<double>(wgs) / static_cast<double>(rounds * slots);
        if (eff > best_eff + 1e-9) {
            best_eff = eff;
            best = ct;
        }
    }
    return best;
}
} // namespace
} // namespace sandy_hip

extern "C" int sandy_hip_moe_matmul(const SandyTensor* x, const SandyTensor* expert_offsets, const SandyTensor* weight,
                                    int32_t transpose_rhs, const SandyTensor* out, void* stream_, char* err,
                                    size_t err_cap) {
    Err e{err, err_cap};
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (!valid_rank(x) || !valid_rank(expert_offsets) || !valid_rank(weight) || !valid_rank(out))
        return fail(e, SANDY_ERR_INVALID, "moe_matmul requires every tensor");
    if (!is_float(x->dtype) || !is_float(weight->dtype)) return fail(e, SANDY_ERR_INVALID, "moe_matmul x unsupported dtype");
    if (x->dtype != weight->dtype) return fail(e, SANDY_ERR_INVALID, "moe_matmul x and weight must have same dtype");
    if (!is_index(expert_offsets->dtype)) return fail(e, SANDY_ERR_INVALID, "moe_matmul expert_offsets must be i32 or i64");
    const int xr = x->rank;
    if ((xr != 2 && xr != 3) || expert_offsets->rank != xr - 1 || weight->rank != 3)
        return fail(e, SANDY_ERR_INVALID, "moe_matmul expects ranks [N,K], [E+1], [E,M,K] or [B,N,K], [B,E+1], [E,M,K]");
    const int64_t batch = xr == 3 ? x->dims[0] : 1;
    const int64_t rows = x->dims[xr - 2], K = x->dims[xr - 1], experts = weight->dims[0];
    const int64_t M = transpose_rhs ? weight->dims[1] : weight->dims[2];
    const int64_t rk = transpose_rhs ? weight->dims[2] : weight->dims[1];
    if (batch <= 0 || rows < 0 || K <= 0 || experts <= 0 || M <= 0)
        return fail(e, SANDY_ERR_INVALID, "moe_matmul expects static positive dimensions");
    if (rk != K) return fail(e, SANDY_ERR_INVALID, "moe_matmul contracting dimension mismatch");
    if (expert_offsets->dims[xr - 2] != experts + 1) return fail(e, SANDY_ERR_INVALID, "moe_matmul expert_offsets shape mismatch");
    if (xr == 3 && expert_offsets->dims[0] != batch) return fail(e, SANDY_ERR_INVALID, "moe_matmul batch dimension mismatch");
    if (out->rank != xr || out->dtype != x->dtype || out->dims[xr - 1] != M || out->dims[xr - 2] != rows)
        return fail(e, SANDY_ERR_INVALID, "moe_matmul output shape mismatch");
    if (!contiguous(*x) || !contiguous(*expert_offsets) || !contiguous(*weight) || !contiguous(*out))
        return fail(e, SANDY_ERR_UNSUPPORTED, "moe_matmul requires contiguous tensors");
    if (rows == 0) return ok(e);
    int status = 0;
    uint32_t* errw = device_error_word(e, &status);
    if (status) return status;
    const bool aligned = ((reinterpret_cast<uintptr_t>(base_ptr(*x)) | reinterpret_cast<uintptr_t>(base_ptr(*weight))) & 15) == 0;
    if (x->dtype == SANDY_BF16 && transpose_rhs && K % 32 == 0 && aligned) {
        // every workgroup checks the offsets of its own expert
        const int64_t avg = rows / experts;
        const auto* px = static_cast<const uint16_t*>(base_ptr(*x));
        const auto* pw = static_cast<const uint16_t*>(base_ptr(*weight));
        auto* po = static_cast<uint16_t*>(base_ptr(*out));
        const void* po_ = base_ptr(*expert_offsets);
        // tile: 16 rows x 32 columns per wave for decode-sized batches, otherwise
        // 64 rows x the column tile of moe_column_tile
        const int col_tile = avg <= 16 ? 2 : moe_column_tile(M, batch * experts);
        const int variant = env_int("SANDY_MOE_GEMM", avg <= 16 ? 0 : col_tile == 3 ? 5 : col_tile == 2 ? 2 : 1);
        auto grid_for = [&](int ct) {
            return dim3(static_cast<unsigned>(batch * experts), static_cast<unsigned>((M + 64 * ct - 1) / (64 * ct)));
        };
#define LINES_LAUNCH(RT, CT)                                                                                        \
    hipLaunchKernelGGL((moe_gemm_lines_kernel<RT, CT>), grid_for(CT), dim3(256), 0, stream, px, po_,               \
                       expert_offsets->dtype, pw, po, rows, K, M, experts, batch, errw)
        switch (variant) {
            case 0: LINES_LAUNCH(1, 2); break;
            case 2: LINES_LAUNCH(4, 2); break;
            case 3: LINES_LAUNCH(2, 4); break;
            case 4: LINES_LAUNCH(2, 2); break;
            case 5: LINES_LAUNCH(4, 3); break;
            default: LINES_LAUNCH(4, 4); break;
        }
#undef LINES_LAUNCH
    } else {
        hipLaunchKernelGGL(validate_offsets_kernel, dim3(static_cast<unsigned>((batch * experts + 255) / 256)), dim3(256), 0, stream,
                           base_ptr(*expert_offsets), expert_offsets->dtype, experts, rows, batch, errw);
        const int64_t threads = batch * rows * M;
        dim3 grid(static_cast<unsigned>((threads + 255) / 256));
        if (x->dtype == SANDY_BF16)
            hipLaunchKernelGGL(moe_gemm_generic_kernel<BF16>, grid, dim3(256), 0, stream, base_ptr(*x), base_ptr(*expert_offsets),
                               expert_offsets->dtype, base_ptr(*weight), base_ptr(*out), rows, K, M, experts, batch, transpose_rhs, errw);
        else
            hipLaunchKernelGGL(moe_gemm_generic_kernel<F32>, grid, dim3(256), 0, stream, base_ptr(*x), base_ptr(*expert_offsets),
                               expert_offsets->dtype, base_ptr(*weight), base_ptr(*out), rows, K, M, experts, batch, transpose_rhs, errw);
    }
    SANDY_HIP_TRY(hipGetLastError(), e, "moe_matmul launch");
    return ok(e);
}

extern "C" int sandy_hip_moe_scatter_sum(const SandyTensor* packed_out, const SandyTensor* packed_weights,
                                         const SandyTensor* token_ids, const SandyTensor* out, void* stream_, char* err,
                                         size_t err_cap) {
    Err e{err, err_cap};
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (!valid_rank(packed_out) || !valid_rank(packed_weights) || !valid_rank(token_ids) || !valid_rank(out))
        return fail(e, SANDY_ERR_INVALID, "moe_scatter_sum requires every tensor");
    if (!is_float(packed_out->dtype)) return fail(e, SANDY_ERR_INVALID, "moe_scatter_sum packed_out unsupported dtype");
    if (!is_index(token_ids->dtype)) return fail(e, SANDY_ERR_INVALID, "moe_scatter_sum token_ids must be i32 or i64");
    const int pr = packed_out->rank, orr = out->rank;
    if ((pr != 2 && pr != 3) || packed_weights->rank != pr - 1 || token_ids->rank != pr - 1 || (orr != 2 && orr != 3) || pr != orr)
        return fail(e, SANDY_ERR_INVALID, "moe_scatter_sum expects ranks [N,H], [N], [N], [T,H] or [B,N,H], [B,N], [B,N], [B,T,H]");
    if (packed_out->dtype != packed_weights->dtype || packed_out->dtype != out->dtype)
        return fail(e, SANDY_ERR_INVALID, "moe_scatter_sum dtype mismatch");
    const int64_t rows = packed_out->dims[pr - 2], hidden = packed_out->dims[pr - 1];
    const int64_t batch = orr == 3 ? out->dims[0] : 1;
    const int64_t seq = out->dims[orr - 2];
    if ((pr == 3 && (packed_out->dims[0] != batch || packed_weights->dims[0] != batch || token_ids->dims[0] != batch)) ||
        packed_weights->dims[pr - 2] != rows || token_ids->dims[pr - 2] != rows || out->dims[orr - 1] != hidden)
        return fail(e, SANDY_ERR_INVALID, "moe_scatter_sum shape mismatch");
    if (!contiguous(*packed_out) || !contiguous(*packed_weights) || !contiguous(*token_ids) || !contiguous(*out))
        return fail(e, SANDY_ERR_UNSUPPORTED, "moe_scatter_sum requires contiguous tensors");
    if (batch * seq * hidden == 0) return ok(e);
    int status = 0;
    uint32_t* errw = device_error_word(e, &status);
    if (status) return status;
    const int64_t blocks = batch * ((seq + 3) / 4) * ((hidden + 511) / 512);
    dim3 grid(static_cast<unsigned>(blocks));
    const bool aligned = ((reinterpret_cast<uintptr_t>(base_ptr(*packed_out)) | reinterpret_cast<uintptr_t>(base_ptr(*out))) & 15) == 0;
    if (!aligned && hidden % 8 == 0) return fail(e, SANDY_ERR_UNSUPPORTED, "moe_scatter_sum needs 16-byte aligned rows");
    if (packed_out->dtype == SANDY_BF16)
        hipLaunchKernelGGL(moe_combine_kernel<BF16>, grid, dim3(256), 0, stream, base_ptr(*packed_out), base_ptr(*packed_weights),
                           base_ptr(*token_ids), token_ids->dtype, base_ptr(*out), batch, rows, hidden, seq, errw);
    else
        hipLaunchKernelGGL(moe_combine_kernel<F32>, grid, dim3(256), 0, stream, base_ptr(*packed_out), base_ptr(*packed_weights),
                           base_ptr(*token_ids), token_ids->dtype, base_ptr(*out), batch, rows, hidden, seq, errw);
    SANDY_HIP_TRY(hipGetLastError(), e, "moe_scatter_sum launch");
    return ok(e);
}
